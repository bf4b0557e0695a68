#include "execution/device.h"

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

bool DeviceContext::Init(std::string* error) {
  if (!UseDevice(ordinal_, error)) return false;
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, ordinal_);
  if (e != hipSuccess) {
    if (error) *error = HipMsg("hipGetDeviceProperties", e);
    return false;
  }
  name_ = prop.gcnArchName;
  cus_ = prop.multiProcessorCount;
  stats_.bytes_limit = int64_t(prop.totalGlobalMem);
  // default priority, non-blocking with respect to the legacy null stream
  e = hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking);
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

void* DeviceContext::Alloc(size_t bytes, std::string* error) {
  if (bytes == 0) return nullptr;
  const size_t cls = SizeClass(bytes);
  {
    std::lock_guard<std::mutex> lk(mu_);
    auto it = free_.find(cls);
    if (it != free_.end()) {
      void* p = it->second;
      free_.erase(it);
      live_[p] = cls;
      stats_.bytes_in_use += int64_t(cls);
      stats_.peak_bytes_in_use = std::max(stats_.peak_bytes_in_use, stats_.bytes_in_use);
      ++stats_.num_allocs;
      return p;
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
  live_[p] = cls;
  stats_.bytes_in_use += int64_t(cls);
  stats_.bytes_reserved += int64_t(cls);
  stats_.peak_bytes_in_use = std::max(stats_.peak_bytes_in_use, stats_.bytes_in_use);
  stats_.largest_alloc = std::max(stats_.largest_alloc, int64_t(cls));
  ++stats_.num_allocs;
  return p;
}

void DeviceContext::Free(void* p) {
  if (!p) return;
  std::lock_guard<std::mutex> lk(mu_);
  auto it = live_.find(p);
  if (it == live_.end()) return;  // not ours: ignore
  stats_.bytes_in_use -= int64_t(it->second);
  free_.emplace(it->second, p);
  live_.erase(it);
}

void DeviceContext::Trim() {
  std::vector<void*> release;
  {
    std::lock_guard<std::mutex> lk(mu_);
    for (auto& kv : free_) {
      release.push_back(kv.second);
      stats_.bytes_reserved -= int64_t(kv.first);
    }
    free_.clear();
  }
  if (release.empty()) return;
  (void)UseDevice(ordinal_, nullptr);
  (void)hipStreamSynchronize(stream_);
  for (void* p : release) (void)hipFree(p);
}

MemoryStats DeviceContext::Stats() {
  std::lock_guard<std::mutex> lk(mu_);
  return stats_;
}

bool DeviceContext::CopyToDevice(void* dst, const void* src, size_t bytes, std::string* error) {
  if (bytes == 0) return true;
  (void)UseDevice(ordinal_, nullptr);
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream_);
  if (e == hipSuccess) e = hipStreamSynchronize(stream_);
  if (e != hipSuccess) {
    if (error) *error = HipMsg("host-to-device copy", e);
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
