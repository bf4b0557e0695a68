#include "execution/device.h"

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <memory>

namespace mi::exec {

namespace {
std::mutex g_mu;
std::vector<std::unique_ptr<DeviceContext>>& Contexts() {
  static auto* v = new std::vector<std::unique_ptr<DeviceContext>>();
  return *v;
}
std::string HipMsg(const char* what, hipError_t e) {
  return std::string(what) + ": " + hipGetErrorString(e);
}
}  // namespace

bool UseDevice(int ordinal, std::string* error) {
  hipError_t e = hipSetDevice(ordinal);
  if (e != hipSuccess) {
    if (error) *error = HipMsg("hipSetDevice", e);
    return false;
  }
  return true;
}

int DeviceContext::DeviceCount() {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n;
}

DeviceContext* DeviceContext::Get(int ordinal, std::string* error) {
  std::lock_guard<std::mutex> lk(g_mu);
  auto& v = Contexts();
  if (ordinal < 0) {
    if (error) *error = "negative device ordinal";
    return nullptr;
  }
  if (size_t(ordinal) < v.size() && v[ordinal]) return v[ordinal].get();
  const int n = DeviceCount();
  if (ordinal >= n) {
    if (error) *error = "no HIP device " + std::to_string(ordinal) + " (found " + std::to_string(n) + ")";
    return nullptr;
  }
  std::unique_ptr<DeviceContext> ctx(new DeviceContext(ordinal));
  if (!ctx->Init(error)) return nullptr;
  if (v.size() <= size_t(ordinal)) v.resize(ordinal + 1);
  v[ordinal] = std::move(ctx);
  return v[ordinal].get();
}

bool DeviceContext::Probe(int ordinal, GpuProps* out, std::string* error) {
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, ordinal);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    if (error) *error = HipMsg("hipGetDeviceProperties", e);
    return false;
  }
  out->arch = prop.gcnArchName;
  out->name = prop.name;
  out->compute_units = prop.multiProcessorCount;
  out->hbm_bytes = int64_t(prop.totalGlobalMem);
  out->clock_khz = prop.clockRate;
  char bus[32];
  snprintf(bus, sizeof(bus), "%04x:%02x:%02x.0", unsigned(prop.pciDomainID), unsigned(prop.pciBusID),
           unsigned(prop.pciDeviceID));
  out->pci_bus_id = bus;
  return true;
}

bool DeviceContext::Init(std::string* error) {
  if (!UseDevice(ordinal_, error)) return false;
  if (!Probe(ordinal_, &props_, error)) return false;
  stats_.bytes_limit = props_.hbm_bytes;
  // default priority, non-blocking with respect to the legacy null stream
  hipError_t e = hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&upload_, hipStreamNonBlocking);
  if (e != hipSuccess) {
    if (error) *error = HipMsg("hipStreamCreate", e);
    return false;
  }
  return true;
}

size_t DeviceContext::SizeClass(size_t bytes) {
  if (bytes <= (size_t(1) << 20)) return (bytes + 255) & ~size_t(255);
  // above 1 MiB: round up to 1/8 of the enclosing power of two
  size_t p = size_t(1) << (63 - __builtin_clzll(bytes));
  size_t step = p / 8;
  return (bytes + step - 1) / step * step;
}

hipEvent_t DeviceContext::TakeEventLocked() {
  if (!idle_events_.empty()) {
    hipEvent_t ev = idle_events_.back();
    idle_events_.pop_back();
    return ev;
  }
  hipEvent_t ev = nullptr;
  if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  return ev;
}

void DeviceContext::DropEventLocked(hipEvent_t ev) {
  if (!ev) return;
  // one event marks every block of a flush: the last holder releases it
  auto r = event_refs_.find(ev);
  if (r != event_refs_.end() && --r->second > 0) return;
  if (r != event_refs_.end()) event_refs_.erase(r);
  // an event no stream can still be waiting on is recycled; a pending one is
  // destroyed (HIP releases it once the recorded work has passed)
  if (hipEventQuery(ev) == hipSuccess && idle_events_.size() < 256)
    idle_events_.push_back(ev);
  else
    (void)hipEventDestroy(ev);
}

void DeviceContext::FlushFreedLocked() {
  if (freed_.empty()) return;
  // every use of these blocks is queued on the compute stream (uploads into
  // them were ordered before their readers): one event after all of it,
  // recorded now, serves every block freed since the last flush (one
  // marker in the stream instead of one per block; later than each Free,
  // so never too early)
  hipEvent_t ev = TakeEventLocked();
  if (ev && hipEventRecord(ev, stream_) != hipSuccess) {
    (void)hipGetLastError();
    (void)hipEventDestroy(ev);
    ev = nullptr;
  }
  if (!ev) {  // no event: wait here rather than risk a transfer-stream race
    (void)hipStreamSynchronize(stream_);
  } else {
    event_refs_[ev] = int(freed_.size());
  }
  for (const Freed& f : freed_) free_.emplace(f.cls, Slot{f.p, ev});
  freed_.clear();
}

void* DeviceContext::Alloc(size_t bytes, std::string* error) {
  if (bytes == 0) return nullptr;
  const size_t cls = SizeClass(bytes);
  {
    std::lock_guard<std::mutex> lk(mu_);
    FlushFreedLocked();
    auto it = free_.find(cls);
    if (it != free_.end()) {
      Slot slot = it->second;
      free_.erase(it);
      if (slot.reuse_after && hipEventQuery(slot.reuse_after) == hipSuccess) {
        DropEventLocked(slot.reuse_after);
        slot.reuse_after = nullptr;
      }
      live_[slot.p] = Live{cls, slot.reuse_after};
      stats_.bytes_in_use += int64_t(cls);
      stats_.peak_bytes_in_use = std::max(stats_.peak_bytes_in_use, stats_.bytes_in_use);
      ++stats_.num_allocs;
      return slot.p;
    }
  }
  (void)UseDevice(ordinal_, nullptr);
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, cls);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    Trim();  // give cached blocks back and retry once
    e = hipMalloc(&p, cls);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      if (error) *error = "hipMalloc(" + std::to_string(cls) + " bytes) failed: " + hipGetErrorString(e);
      return nullptr;
    }
  }
  std::lock_guard<std::mutex> lk(mu_);
  live_[p] = Live{cls, nullptr};
  stats_.bytes_in_use += int64_t(cls);
  stats_.bytes_reserved += int64_t(cls);
  stats_.peak_bytes_in_use = std::max(stats_.peak_bytes_in_use, stats_.bytes_in_use);
  stats_.largest_alloc = std::max(stats_.largest_alloc, int64_t(cls));
  ++stats_.num_allocs;
  return p;
}

void DeviceContext::Free(void* p) {
  if (!p) return;
  (void)UseDevice(ordinal_, nullptr);
  std::lock_guard<std::mutex> lk(mu_);
  auto it = live_.find(p);
  if (it == live_.end()) return;  // not ours: ignore
  // cached once the next Alloc (or Trim) records the event that marks the
  // end of its queued uses (FlushFreedLocked)
  DropEventLocked(it->second.reuse_after);
  stats_.bytes_in_use -= int64_t(it->second.cls);
  freed_.push_back(Freed{p, it->second.cls});
  live_.erase(it);
}

bool DeviceContext::OrderUploadInto(void* dst, std::string* error) {
  std::lock_guard<std::mutex> lk(mu_);
  auto it = live_.upper_bound(dst);
  if (it == live_.begin()) return true;  // not a pool block: nothing to order
  --it;
  if (static_cast<char*>(dst) >= static_cast<char*>(it->first) + it->second.cls) return true;
  hipEvent_t ev = it->second.reuse_after;
  if (!ev) return true;
  if (hipEventQuery(ev) == hipSuccess) {
    DropEventLocked(ev);
    it->second.reuse_after = nullptr;
    return true;
  }
  hipError_t e = hipStreamWaitEvent(upload_, ev, 0);
  if (e != hipSuccess) {
    if (error) *error = HipMsg("hipStreamWaitEvent", e);
    return false;
  }
  return true;
}

void DeviceContext::Trim() {
  std::vector<void*> release;
  std::vector<hipEvent_t> events;
  {
    std::lock_guard<std::mutex> lk(mu_);
    FlushFreedLocked();
    for (auto& kv : free_) {
      release.push_back(kv.second.p);
      // a shared event is destroyed once, by its last holder
      if (kv.second.reuse_after) {
        auto r = event_refs_.find(kv.second.reuse_after);
        if (r != event_refs_.end() && --r->second > 0) continue;
        if (r != event_refs_.end()) event_refs_.erase(r);
        events.push_back(kv.second.reuse_after);
      }
    }
    for (auto& kv : free_) stats_.bytes_reserved -= int64_t(kv.first);
    free_.clear();
  }
  if (release.empty()) return;
  (void)UseDevice(ordinal_, nullptr);
  (void)hipStreamSynchronize(upload_);
  (void)hipStreamSynchronize(stream_);
  for (hipEvent_t ev : events) (void)hipEventDestroy(ev);
  for (void* p : release) (void)hipFree(p);
}

MemoryStats DeviceContext::Stats() {
  std::lock_guard<std::mutex> lk(mu_);
  return stats_;
}

namespace {
constexpr size_t kStagePiece = size_t(8) << 20;       // upload staging granule
constexpr size_t kPinnedCacheBytes = size_t(512) << 20;  // cached idle pinned chunks
constexpr size_t kPinnedBusyBytes = size_t(1) << 30;   // in-flight staging before waiting
}  // namespace

void DeviceContext::ReapPinnedLocked() {
  // busy chunks retire in stream order: stop at the first still in flight
  while (!pin_busy_.empty()) {
    Busy& b = pin_busy_.front();
    hipError_t q = hipEventQuery(b.until);
    if (q == hipErrorNotReady) break;
    (void)hipEventDestroy(b.until);
    const size_t cls = pin_size_[b.p];
    if (pin_cached_ + cls <= kPinnedCacheBytes) {
      pin_free_.emplace(cls, b.p);
      pin_cached_ += cls;
    } else {
      pin_size_.erase(b.p);
      (void)hipHostFree(b.p);
    }
    pin_busy_.pop_front();
  }
}

void* DeviceContext::TakePinned(size_t bytes, std::string* error) {
  const size_t cls = SizeClass(bytes ? bytes : 1);
  std::lock_guard<std::mutex> lk(pin_mu_);
  ReapPinnedLocked();
  auto it = pin_free_.find(cls);
  if (it != pin_free_.end()) {
    void* p = it->second;
    pin_free_.erase(it);
    pin_cached_ -= cls;
    return p;
  }
  size_t busy = 0;
  for (const Busy& b : pin_busy_) busy += pin_size_[b.p];
  while (busy > kPinnedBusyBytes && !pin_busy_.empty()) {  // bound the staging in flight
    (void)hipEventSynchronize(pin_busy_.front().until);
    busy -= pin_size_[pin_busy_.front().p];
    ReapPinnedLocked();
  }
  void* p = nullptr;
  hipError_t e = hipHostMalloc(&p, cls, hipHostMallocDefault);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    if (error) *error = HipMsg("hipHostMalloc", e);
    return nullptr;
  }
  pin_size_[p] = cls;
  return p;
}

void DeviceContext::ReturnPinned(void* p, hipEvent_t busy_until) {
  if (!p) return;
  std::lock_guard<std::mutex> lk(pin_mu_);
  if (busy_until) {
    pin_busy_.push_back({p, busy_until});
    return;
  }
  const size_t cls = pin_size_[p];
  if (pin_cached_ + cls <= kPinnedCacheBytes) {
    pin_free_.emplace(cls, p);
    pin_cached_ += cls;
  } else {
    pin_size_.erase(p);
    (void)hipHostFree(p);
  }
}

hipEvent_t DeviceContext::Upload(void* dst, const void* src, size_t bytes, std::string* error) {
  if (!UseDevice(ordinal_, error)) return nullptr;
  std::lock_guard<std::mutex> lk(upload_mu_);
  if (!OrderUploadInto(dst, error)) return nullptr;
  for (size_t off = 0; off < bytes;) {
    const size_t n = std::min(kStagePiece, bytes - off);
    void* chunk = TakePinned(n, error);
    if (!chunk) return nullptr;
    memcpy(chunk, static_cast<const char*>(src) + off, n);
    hipEvent_t ev = nullptr;
    hipError_t e = hipMemcpyAsync(static_cast<char*>(dst) + off, chunk, n, hipMemcpyHostToDevice, upload_);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventRecord(ev, upload_);
    if (e != hipSuccess) {
      if (error) *error = HipMsg("host-to-device copy", e);
      (void)hipStreamSynchronize(upload_);
      if (ev) (void)hipEventDestroy(ev);
      ReturnPinned(chunk, nullptr);
      return nullptr;
    }
    ReturnPinned(chunk, ev);  // the staging pool owns `ev` from here
    off += n;
  }
  hipEvent_t done = nullptr;
  hipError_t e = hipEventCreateWithFlags(&done, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventRecord(done, upload_);
  if (e != hipSuccess) {
    if (error) *error = HipMsg("hipEventRecord", e);
    if (done) (void)hipEventDestroy(done);
    return nullptr;
  }
  return done;
}

bool DeviceContext::UploadForCompute(void* dst, const void* src, size_t bytes, std::string* error) {
  if (bytes == 0) return true;
  hipEvent_t done = Upload(dst, src, bytes, error);
  if (!done) return false;
  hipError_t e = hipStreamWaitEvent(stream_, done, 0);
  (void)hipEventDestroy(done);  // the wait keeps what it needs
  if (e != hipSuccess) {
    if (error) *error = HipMsg("hipStreamWaitEvent", e);
    return false;
  }
  return true;
}

bool DeviceContext::CopyToHostAsync(void* dst, const void* src, size_t bytes, std::string* error) {
  if (bytes == 0) return true;
  (void)UseDevice(ordinal_, nullptr);
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, stream_);
  if (e != hipSuccess) {
    if (error) *error = HipMsg("device-to-host copy", e);
    return false;
  }
  return true;
}

bool DeviceContext::CopyDeviceToDevice(void* dst, const void* src, size_t bytes, std::string* error) {
  if (bytes == 0) return true;
  (void)UseDevice(ordinal_, nullptr);
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, stream_);
  if (e != hipSuccess) {
    if (error) *error = HipMsg("device-to-device copy", e);
    return false;
  }
  return true;
}

bool DeviceContext::Synchronize(std::string* error) {
  (void)UseDevice(ordinal_, nullptr);
  hipError_t e = hipStreamSynchronize(stream_);
  if (e != hipSuccess) {
    if (error) *error = HipMsg("hipStreamSynchronize", e);
    return false;
  }
  return true;
}

}  // namespace mi::exec
