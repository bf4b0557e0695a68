// HIP device context: one stream and one HBM caching allocator per GPU.
//
// Replaces src/execution/metal_buffer.{h,mm} (shared-storage MTLBuffer
// allocation, metal_buffer.mm:13-29) and the size-exact BufferPool of
// src/jam/jam_run.mm:74-112.  Differences by design:
//  - memory is device HBM (hipMalloc), not CPU-visible unified memory;
//  - every launch and copy of the plugin goes to the context's single
//    stream, so a block returned to the pool can be handed out again at once:
//    any later use is ordered after the earlier use on that stream;
//  - blocks are rounded to size classes (256 B granularity below 1 MiB,
//    then 1/8-power-of-two steps) so near-equal sizes share free lists;
//  - hipFree is only called on trim (allocation failure) or process exit.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <map>
#include <mutex>
#include <string>
#include <vector>

namespace mi::exec {

struct MemoryStats {
  int64_t bytes_in_use = 0;
  int64_t peak_bytes_in_use = 0;
  int64_t num_allocs = 0;
  int64_t largest_alloc = 0;
  int64_t bytes_reserved = 0;  // held by the pool, in use or cached
  int64_t bytes_limit = 0;     // total device memory
};

class DeviceContext {
 public:
  // Returns the context of HIP device `ordinal`, creating it on first use;
  // nullptr (and *error) when the device cannot be opened.
  static DeviceContext* Get(int ordinal, std::string* error);
  static int DeviceCount();

  int ordinal() const { return ordinal_; }
  hipStream_t stream() const { return stream_; }
  const std::string& name() const { return name_; }
  int compute_units() const { return cus_; }

  // Stream-ordered allocation (see file comment).  Alloc(0) returns nullptr.
  void* Alloc(size_t bytes, std::string* error);
  void Free(void* p);
  MemoryStats Stats();
  void Trim();  // release every cached block back to HIP

  // Host <-> device copies on the context stream.
  bool CopyToDevice(void* dst, const void* src, size_t bytes, std::string* error);  // blocks until done
  bool CopyToHostAsync(void* dst, const void* src, size_t bytes, std::string* error);
  bool CopyDeviceToDevice(void* dst, const void* src, size_t bytes, std::string* error);
  bool Synchronize(std::string* error);

 private:
  explicit DeviceContext(int ordinal) : ordinal_(ordinal) {}
  bool Init(std::string* error);
  static size_t SizeClass(size_t bytes);

  int ordinal_;
  hipStream_t stream_ = nullptr;
  std::string name_;
  int cus_ = 0;
  std::mutex mu_;
  std::multimap<size_t, void*> free_;   // size class -> cached block
  std::map<void*, size_t> live_;        // block -> size class
  MemoryStats stats_;
};

// Sets the calling thread's current HIP device.
bool UseDevice(int ordinal, std::string* error);

}  // namespace mi::exec
