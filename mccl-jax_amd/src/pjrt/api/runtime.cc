// Completions, the watcher thread, storage blocks and the small helpers the
// slot implementations share (see plugin.h for the model).
#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <thread>

#include "pjrt/api/plugin.h"

namespace mi::pjrt {

// ------------------------------------------------------------------ Completion
std::shared_ptr<Completion> Completion::Done(std::string error) {
  std::shared_ptr<Completion> c(new Completion());
  c->error_ = std::move(error);
  return c;
}

std::shared_ptr<Completion> Completion::AfterGpu(int ordinal, Lane lane, hipEvent_t ev,
                                                 std::function<std::string()> host_step) {
  std::shared_ptr<Completion> c(new Completion());
  c->state_ = State::kGpu;
  c->ev_ = ev;
  c->ordinal_ = ordinal;
  c->lane_ = lane;
  c->host_step_ = std::move(host_step);
  return c;
}

Completion::~Completion() {
  if (ev_) (void)hipEventDestroy(ev_);
}

void Completion::Settle(std::string gpu_error) {
  std::function<std::string()> step;
  {
    std::lock_guard<std::mutex> lk(mu_);
    if (state_ != State::kGpu) return;  // another thread settles it
    state_ = State::kSettling;
    step.swap(host_step_);
  }
  std::string err = std::move(gpu_error);
  if (step) {
    std::string e2 = step();  // runs even after a GPU error: it releases staging
    if (err.empty()) err = std::move(e2);
  }
  std::vector<Callback> cbs;
  {
    std::lock_guard<std::mutex> lk(mu_);
    state_ = State::kReady;
    error_ = err;
    cbs.swap(waiting_);
  }
  cv_.notify_all();
  for (auto& cb : cbs) cb(err);
}

bool Completion::Test() {
  hipEvent_t ev;
  {
    std::lock_guard<std::mutex> lk(mu_);
    if (state_ != State::kGpu) return state_ == State::kReady;
    ev = ev_;
  }
  hipError_t r = hipEventQuery(ev);
  if (r == hipErrorNotReady) return false;
  Settle(r == hipSuccess ? "" : std::string("device execution failed: ") + hipGetErrorString(r));
  std::lock_guard<std::mutex> lk(mu_);
  return state_ == State::kReady;
}

std::string Completion::Wait() {
  hipEvent_t ev = nullptr;
  int ordinal = 0;
  {
    std::lock_guard<std::mutex> lk(mu_);
    if (state_ == State::kGpu) {
      ev = ev_;
      ordinal = ordinal_;
    }
  }
  if (ev) {
    (void)exec::UseDevice(ordinal, nullptr);
    hipError_t r = hipEventSynchronize(ev);
    Settle(r == hipSuccess ? "" : std::string("device execution failed: ") + hipGetErrorString(r));
  }
  std::unique_lock<std::mutex> lk(mu_);
  cv_.wait(lk, [&] { return state_ == State::kReady; });
  return error_;
}

void Completion::Then(Callback cb) {
  {
    std::lock_guard<std::mutex> lk(mu_);
    if (state_ != State::kReady) {
      waiting_.push_back(std::move(cb));
      cb = nullptr;
    }
  }
  if (cb) {
    cb(error());
    return;
  }
  // not complete yet: the watcher drives it (registering twice is harmless)
  Watch(shared_from_this());
}

std::string Completion::error() {
  std::lock_guard<std::mutex> lk(mu_);
  return state_ == State::kReady ? error_ : std::string();
}

hipEvent_t Completion::PendingEvent(Lane* lane) {
  std::lock_guard<std::mutex> lk(mu_);
  if (state_ != State::kGpu) return nullptr;
  if (lane) *lane = lane_;
  return ev_;
}

// ------------------------------------------------------------------ watcher
namespace {

class Watcher {
 public:
  static Watcher& Get() {
    static Watcher* w = new Watcher();  // never destroyed: its thread may outlive statics
    return *w;
  }
  void Add(const std::shared_ptr<Completion>& c) {
    {
      std::lock_guard<std::mutex> lk(mu_);
      if (stopping_) return;
      pending_.push_back(c);
      if (!started_) {
        started_ = true;
        std::atexit([] { Watcher::Get().Stop(); });
        std::thread([this] { Loop(); }).detach();
      }
    }
    cv_.notify_one();
  }
  void Stop() {
    {
      std::lock_guard<std::mutex> lk(mu_);
      stopping_ = true;
    }
    cv_.notify_all();
  }

 private:
  void Loop() {
    auto nap = std::chrono::microseconds(20);
    for (;;) {
      std::vector<std::shared_ptr<Completion>> batch;
      {
        std::unique_lock<std::mutex> lk(mu_);
        cv_.wait(lk, [&] { return stopping_ || !pending_.empty(); });
        if (stopping_) return;  // no HIP calls while the process tears down
        batch.swap(pending_);
      }
      std::vector<std::shared_ptr<Completion>> still;
      for (auto& c : batch)
        if (!c->Test()) still.push_back(std::move(c));
      const bool progressed = still.size() < batch.size();
      {
        std::lock_guard<std::mutex> lk(mu_);
        for (auto& c : still) pending_.push_back(std::move(c));
      }
      if (!still.empty()) {
        nap = progressed ? std::chrono::microseconds(20) : std::min(nap * 2, std::chrono::microseconds(1000));
        std::this_thread::sleep_for(nap);
      }
    }
  }

  std::mutex mu_;
  std::condition_variable cv_;
  std::vector<std::shared_ptr<Completion>> pending_;
  bool started_ = false;
  bool stopping_ = false;
};

}  // namespace

void Watch(const std::shared_ptr<Completion>& c) {
  if (c && !c->Test()) Watcher::Get().Add(c);
}

// ------------------------------------------------------------------ Block
Block::~Block() {
  if (on_release) {
    on_release();
    return;
  }
  if (!ptr) return;
  switch (where) {
    case Placement::kPinnedHost:
      if (pending_write) (void)pending_write->Wait();  // no DMA may still target it
      (void)hipHostFree(ptr);
      break;
    case Placement::kHbm:
      if (ctx) {
        // the pool reuses memory in compute-stream order: order the compute
        // stream after a transfer-stream write still in flight
        (void)OrderComputeAfter(pending_write, ctx, nullptr);
        ctx->Free(ptr);
      }
      break;
    case Placement::kForeign:
      break;
  }
}

// ------------------------------------------------------------------ NamedValues
PJRT_NamedValue& NamedValues::Add(const char* name, PJRT_NamedValue_Type t) {
  strings_.emplace_back(name);
  PJRT_NamedValue v{};
  v.struct_size = sizeof(PJRT_NamedValue);
  v.name = strings_.back().c_str();
  v.name_size = strings_.back().size();
  v.type = t;
  v.value_size = 1;
  values_.push_back(v);
  return values_.back();
}
void NamedValues::Str(const char* name, std::string s) {
  PJRT_NamedValue& v = Add(name, PJRT_NamedValue_kString);
  strings_.push_back(std::move(s));
  v.string_value = strings_.back().c_str();
  v.value_size = strings_.back().size();
}
void NamedValues::Int(const char* name, int64_t x) { Add(name, PJRT_NamedValue_kInt64).int64_value = x; }
void NamedValues::Ints(const char* name, std::vector<int64_t> xs) {
  PJRT_NamedValue& v = Add(name, PJRT_NamedValue_kInt64List);
  lists_.push_back(std::move(xs));
  v.int64_array_value = lists_.back().data();
  v.value_size = lists_.back().size();
}
void NamedValues::Bool(const char* name, bool b) { Add(name, PJRT_NamedValue_kBool).bool_value = b; }

// ------------------------------------------------------------------ helpers
PJRT_Error* Fail(PJRT_Error_Code code, std::string text) { return new PJRT_Error{code, std::move(text)}; }

size_t ElementBytes(PJRT_Buffer_Type t) {
  switch (t) {
    case PJRT_Buffer_Type_PRED: case PJRT_Buffer_Type_S8: case PJRT_Buffer_Type_U8:
      return 1;
    case PJRT_Buffer_Type_S16: case PJRT_Buffer_Type_U16: case PJRT_Buffer_Type_F16: case PJRT_Buffer_Type_BF16:
      return 2;
    case PJRT_Buffer_Type_S32: case PJRT_Buffer_Type_U32: case PJRT_Buffer_Type_F32:
      return 4;
    case PJRT_Buffer_Type_S64: case PJRT_Buffer_Type_U64: case PJRT_Buffer_Type_F64:
      return 8;
    default:
      return 0;  // complex, fp8, sub-byte and token types are not carried
  }
}

exec::DeviceContext* ContextOf(PJRT_Device* d, std::string* error) {
  if (!d || d->hip_ordinal < 0) {
    if (error) *error = "no HIP device is available to this client";
    return nullptr;
  }
  return exec::DeviceContext::Get(d->hip_ordinal, error);
}

bool OrderComputeAfter(const std::shared_ptr<Completion>& c, exec::DeviceContext* ctx, std::string* error) {
  if (!c || !ctx) return true;
  Lane lane = Lane::kHost;
  hipEvent_t ev = c->PendingEvent(&lane);
  if (!ev || lane == Lane::kCompute) return true;  // done, or already in compute-stream order
  if (lane == Lane::kHost) {  // a host-side step: only a wait orders it
    std::string e = c->Wait();
    if (!e.empty() && error) *error = e;
    return e.empty();
  }
  hipError_t r = hipStreamWaitEvent(ctx->stream(), ev, 0);
  if (r != hipSuccess) {
    if (error) *error = std::string("hipStreamWaitEvent: ") + hipGetErrorString(r);
    return false;
  }
  return true;
}

std::string Fingerprint(const char* p, size_t n) {
  // 64-bit FNV-1a of the program bytes, as 16 hex digits
  uint64_t h = 0xcbf29ce484222325ull;
  for (size_t i = 0; i < n; ++i) {
    h ^= static_cast<unsigned char>(p[i]);
    h *= 0x100000001b3ull;
  }
  char buf[24];
  snprintf(buf, sizeof(buf), "%016llx", static_cast<unsigned long long>(h));
  return buf;
}

const std::string& PlatformVersion() {
  static const std::string v = [] {
    int rt = 0;
    if (hipRuntimeGetVersion(&rt) != hipSuccess) {
      (void)hipGetLastError();
      rt = 0;
    }
    char buf[96];
    snprintf(buf, sizeof(buf), "mi355x-pjrt 0.2 (PJRT %d.%d, HIP %d.%d)", MI_PJRT_API_MAJOR, MI_PJRT_API_MINOR,
             rt / 10000000, (rt / 100000) % 100);
    return std::string(buf);
  }();
  return v;
}

std::vector<exec::GpuProps> VisibleGpus() {
  std::vector<exec::GpuProps> out;
  const int n = exec::DeviceContext::DeviceCount();
  for (int k = 0; k < n; ++k) {
    exec::GpuProps p;
    if (!exec::DeviceContext::Probe(k, &p, nullptr)) break;
    out.push_back(std::move(p));
  }
  return out;
}

void Describe(PJRT_DeviceDescription* d, int id, int process, const exec::GpuProps& gpu) {
  d->global_id = id;
  d->process = process;
  d->gpu = gpu;
  const std::string arch = gpu.arch.empty() ? std::string("none") : gpu.arch.substr(0, gpu.arch.find(':'));
  d->label = std::string(kDeviceKind) + "#" + std::to_string(id) + " (" + arch + ")";
  d->detail = "mi355x gpu " + std::to_string(id) + ": " + (gpu.name.empty() ? "no HIP device" : gpu.name) +
              ", " + std::to_string(gpu.compute_units) + " CUs, " + std::to_string(gpu.hbm_bytes >> 30) +
              " GiB HBM, pci " + (gpu.pci_bus_id.empty() ? "-" : gpu.pci_bus_id);
  d->attrs.Str("gfx_arch", arch);
  d->attrs.Int("compute_units", gpu.compute_units);
  d->attrs.Int("hbm_bytes", gpu.hbm_bytes);
  d->attrs.Str("pci_bus_id", gpu.pci_bus_id);
}

}  // namespace mi::pjrt

void ResultTable::Fill(const mi::jam::Program& p) {
  static const char kHbmKind[] = "device";
  for (const auto& t : p.outputs) {
    types.push_back(PJRT_Buffer_Type(int(t.dtype)));  // jam::DType values are PJRT_Buffer_Type values
    ranks.push_back(t.dims.size());
    dims.insert(dims.end(), t.dims.begin(), t.dims.end());
    kinds.push_back(kHbmKind);
    kind_lengths.push_back(sizeof(kHbmKind) - 1);
  }
}
