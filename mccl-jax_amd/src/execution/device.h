// HIP device context: the streams, the HBM caching allocator and the pinned
// staging memory of one GPU.
//
// Replaces src/execution/metal_buffer.{h,mm} (shared-storage MTLBuffer
// allocation, metal_buffer.mm:13-29) and the size-exact BufferPool of
// src/jam/jam_run.mm:74-112.  Differences by design:
//  - memory is device HBM (hipMalloc), not CPU-visible unified memory;
//  - kernels, device-to-device and device-to-host copies go to the compute
//    stream, so a block returned to the pool can be handed out again at once:
//    any later compute-stream use is ordered after the earlier use.  The
//    next Alloc after a run of Frees records one event on the compute stream
//    for all of those blocks (a step dropping hundreds of outputs adds one
//    marker to the stream, not hundreds); a DMA on the transfer stream into
//    a reused block first waits for that event (OrderUploadInto), so an
//    upload never overwrites memory a queued kernel still reads;
//  - host-to-device uploads go to a second (transfer) stream, so they never
//    wait for kernels already queued.  Data is first copied into pinned
//    staging chunks on the calling thread, then DMA'd; the caller gets the
//    hipEvent that marks the end of the DMA and makes whichever stream reads
//    the data wait for it (hipStreamWaitEvent);
//  - blocks are rounded to size classes (256 B granularity below 1 MiB,
//    then 1/8-power-of-two steps) so near-equal sizes share free lists;
//  - hipFree is only called on trim (allocation failure) or process exit.
// Both streams have the default priority.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <deque>
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

// What hipGetDeviceProperties reports about a GPU, kept for descriptions.
struct GpuProps {
  std::string arch;         // gcnArchName, e.g. "gfx950:sramecc+:xnack-"
  std::string name;         // marketing name
  std::string pci_bus_id;   // "0000:05:00.0"
  int compute_units = 0;
  int64_t hbm_bytes = 0;
  int clock_khz = 0;
};

class DeviceContext {
 public:
  // Returns the context of HIP device `ordinal`, creating it on first use;
  // nullptr (and *error) when the device cannot be opened.
  static DeviceContext* Get(int ordinal, std::string* error);
  static int DeviceCount();
  // Properties of device `ordinal` without opening a context (no streams).
  static bool Probe(int ordinal, GpuProps* out, std::string* error);

  int ordinal() const { return ordinal_; }
  hipStream_t stream() const { return stream_; }            // compute stream
  hipStream_t transfer_stream() const { return upload_; }   // host-to-device stream
  const GpuProps& props() const { return props_; }
  const std::string& name() const { return props_.arch; }
  int compute_units() const { return props_.compute_units; }

  // Stream-ordered allocation (see file comment).  Alloc(0) returns nullptr.
  void* Alloc(size_t bytes, std::string* error);
  void Free(void* p);
  MemoryStats Stats();
  void Trim();  // release every cached block back to HIP

  // Makes the transfer stream wait until the compute-stream work queued
  // before the last Free of the block holding `dst` has passed (no-op for a
  // fresh block or one whose freeing work is already done).
  bool OrderUploadInto(void* dst, std::string* error);

  // Host -> HBM without waiting for the compute stream (see file comment).
  // Returns an event recorded on the transfer stream after the last byte
  // landed (the caller destroys it), or nullptr and *error.  The host source
  // may be reused as soon as this returns.
  hipEvent_t Upload(void* dst, const void* src, size_t bytes, std::string* error);
  // Upload, then order the compute stream after it (no host wait).
  bool UploadForCompute(void* dst, const void* src, size_t bytes, std::string* error);

  // Pinned host chunks for staging.  ReturnPinned(p, ev) puts p back once
  // the GPU has passed `ev` (nullptr: at once).
  void* TakePinned(size_t bytes, std::string* error);
  void ReturnPinned(void* p, hipEvent_t busy_until);

  bool CopyToHostAsync(void* dst, const void* src, size_t bytes, std::string* error);
  bool CopyDeviceToDevice(void* dst, const void* src, size_t bytes, std::string* error);
  bool Synchronize(std::string* error);

 private:
  explicit DeviceContext(int ordinal) : ordinal_(ordinal) {}
  bool Init(std::string* error);
  static size_t SizeClass(size_t bytes);
  void ReapPinnedLocked();

  int ordinal_;
  hipStream_t stream_ = nullptr;
  hipStream_t upload_ = nullptr;
  GpuProps props_;
  std::mutex mu_;
  // A block's `reuse_after` is an event recorded on the compute stream when
  // it was last freed (nullptr once that work is known done).
  struct Slot {
    void* p;
    hipEvent_t reuse_after;
  };
  struct Live {
    size_t cls;
    hipEvent_t reuse_after;
  };
  struct Freed {
    void* p;
    size_t cls;
  };
  hipEvent_t TakeEventLocked();
  void DropEventLocked(hipEvent_t ev);  // ev may still be pending; one holder's release
  void FlushFreedLocked();              // freed_ -> free_ behind one new event
  std::multimap<size_t, Slot> free_;    // size class -> cached block
  std::map<void*, Live> live_;          // block -> size class, reuse event
  std::vector<Freed> freed_;            // freed since the last flush (not yet reusable)
  std::map<hipEvent_t, int> event_refs_;  // blocks holding each shared event
  std::vector<hipEvent_t> idle_events_;
  MemoryStats stats_;

  // pinned staging
  std::mutex pin_mu_;
  std::mutex upload_mu_;  // one upload at a time keeps chunk order simple
  std::multimap<size_t, void*> pin_free_;
  std::map<void*, size_t> pin_size_;
  struct Busy {
    void* p;
    hipEvent_t until;
  };
  std::deque<Busy> pin_busy_;
  size_t pin_cached_ = 0;
};

// Sets the calling thread's current HIP device.
bool UseDevice(int ordinal, std::string* error);

}  // namespace mi::exec
