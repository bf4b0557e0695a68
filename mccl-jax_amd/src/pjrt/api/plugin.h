// Object model of the MI355X PJRT plugin (PJRT C API v0.55).
//
// The C API hands out opaque handles (PJRT_Client, PJRT_Device, ...); this
// header gives them their definitions for this plugin, and declares one
// function per slot of PJRT_Api in namespace mi::pjrt::slot, named after
// the slot (slot::Client_Create fills PJRT_Api::PJRT_Client_Create).  The
// table itself is built from the slot list in pjrt_abi.h (plugin_table.cc),
// so a slot without a definition is a link error, not a null pointer.
//
// Model, MI355X-first:
//  * A client owns one PJRT_Device per visible HIP device, each built from
//    hipGetDeviceProperties (architecture, CUs, HBM size, PCI location) and
//    carrying its two memory spaces inline: HBM (kind "device", the default)
//    and pinned host memory (kind "pinned_host").  Memory ids are the device
//    index for HBM and device count + index for pinned host.
//  * A buffer is a shape plus a shared Block (the bytes, wherever they live)
//    plus a Completion that says when the bytes are defined.  Blocks are
//    shared so that a donated input hands its memory to an output and so
//    that in-flight work keeps memory alive.
//  * Every asynchronous result is a Completion: a hipEvent on one of the
//    device's two streams (compute, transfer) with an optional host step run
//    once after it (e.g. the copy out of pinned staging).  One watcher
//    thread per process drives completions that have callbacks or host steps.
#pragma once

#include <hip/hip_runtime_api.h>

#include <condition_variable>
#include <cstddef>
#include <cstdint>
#include <deque>
#include <functional>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "execution/device.h"
#include "jam/program.h"
#include "pjrt/api/pjrt_abi.h"

namespace mi::pjrt {

inline constexpr const char kPlatformName[] = "mi355x";  // not rocm/cuda: JAX emits no GPU custom_calls
inline constexpr const char kDeviceKind[] = "MI355X";

// ------------------------------------------------------------------ completions
enum class Lane : uint8_t { kHost, kCompute, kTransfer };

class Completion : public std::enable_shared_from_this<Completion> {
 public:
  using Callback = std::function<void(const std::string& error)>;

  // Already complete (error empty: success).
  static std::shared_ptr<Completion> Done(std::string error = "");
  // Complete once the GPU has passed `ev` (recorded on `lane` of device
  // `ordinal`; ownership of the event passes here) and `host_step`, if any,
  // has run on the host.  A non-empty string from host_step is the error.
  static std::shared_ptr<Completion> AfterGpu(int ordinal, Lane lane, hipEvent_t ev,
                                              std::function<std::string()> host_step = {});
  ~Completion();

  bool Test();          // non-blocking; true once complete
  std::string Wait();   // blocks; returns the error ("" on success)
  void Then(Callback cb);  // runs cb at once if complete, else from the watcher thread
  std::string error();  // "" while pending or on success

  // For hipStreamWaitEvent: the event while the GPU part may still be
  // pending on `lane`, nullptr once it is known to be done.
  hipEvent_t PendingEvent(Lane* lane);

 private:
  Completion() = default;
  void Settle(std::string gpu_error);

  enum class State : uint8_t { kGpu, kSettling, kReady };
  std::mutex mu_;
  std::condition_variable cv_;
  State state_ = State::kReady;
  std::string error_;
  hipEvent_t ev_ = nullptr;
  int ordinal_ = 0;
  Lane lane_ = Lane::kHost;
  std::function<std::string()> host_step_;
  std::vector<Callback> waiting_;
};

// Hands a completion to the process's watcher thread, which settles it (runs
// its host step and callbacks) soon after the GPU passes its event.
void Watch(const std::shared_ptr<Completion>& c);

// ------------------------------------------------------------------ storage
enum class Placement : uint8_t { kHbm, kPinnedHost, kForeign };

struct Block {
  void* ptr = nullptr;
  size_t bytes = 0;
  Placement where = Placement::kHbm;
  exec::DeviceContext* ctx = nullptr;  // owning device (HBM and foreign views)
  // a GPU write into this block that may still be in flight on a stream
  // other than the compute stream (an upload, or a download into pinned
  // host memory); the memory is only reused or freed after it
  std::shared_ptr<Completion> pending_write;
  std::function<void()> on_release;    // foreign views: the owner's delete callback
  ~Block();
};

// Owns the strings and lists behind a PJRT_NamedValue array.
class NamedValues {
 public:
  void Str(const char* name, std::string v);
  void Int(const char* name, int64_t v);
  void Ints(const char* name, std::vector<int64_t> v);
  void Bool(const char* name, bool v);
  const PJRT_NamedValue* data() const { return values_.empty() ? nullptr : values_.data(); }
  size_t size() const { return values_.size(); }

 private:
  PJRT_NamedValue& Add(const char* name, PJRT_NamedValue_Type t);
  std::deque<std::string> strings_;
  std::deque<std::vector<int64_t>> lists_;
  std::vector<PJRT_NamedValue> values_;
};

// ------------------------------------------------------------------ helpers
PJRT_Error* Fail(PJRT_Error_Code code, std::string text);
size_t ElementBytes(PJRT_Buffer_Type t);
exec::DeviceContext* ContextOf(PJRT_Device* d, std::string* error);
// The args struct the caller passed must reach at least `need` bytes.
inline bool Fits(size_t struct_size, size_t need) { return struct_size >= need; }
#define MI_NEED(args, Type, member)                                                            \
  do {                                                                                         \
    if ((args) == nullptr ||                                                                   \
        !::mi::pjrt::Fits((args)->struct_size, offsetof(Type, member) + sizeof((args)->member))) \
      return ::mi::pjrt::Fail(PJRT_Error_Code_INVALID_ARGUMENT, #Type ": struct_size too small"); \
  } while (0)

// Orders the compute stream of `ctx` after the pending transfer-stream write
// of `c`, if any.  No host wait.
bool OrderComputeAfter(const std::shared_ptr<Completion>& c, exec::DeviceContext* ctx, std::string* error);

std::string Fingerprint(const char* p, size_t n);
// Builds the platform version string: "mi355x-pjrt <v> (PJRT 0.55, HIP <runtime version>)".
const std::string& PlatformVersion();
// Enumerates the visible GPUs (empty when none).
std::vector<exec::GpuProps> VisibleGpus();
void Describe(PJRT_DeviceDescription* d, int id, int process, const exec::GpuProps& gpu);

}  // namespace mi::pjrt

// ------------------------------------------------------------------ handle types
struct PJRT_Error {
  PJRT_Error_Code code = PJRT_Error_Code_UNKNOWN;
  std::string text;
};

struct PJRT_Event {
  std::shared_ptr<mi::pjrt::Completion> done;
};

struct PJRT_DeviceDescription {
  int global_id = 0;
  int process = 0;
  mi::exec::GpuProps gpu;
  std::string label;   // ToString
  std::string detail;  // DebugString
  mi::pjrt::NamedValues attrs;
};

struct PJRT_Memory {
  mi::pjrt::Placement space = mi::pjrt::Placement::kHbm;
  int id = 0;
  PJRT_Device* owner[1] = {nullptr};
  std::string label;   // ToString
  std::string detail;  // DebugString
  const char* kind() const { return space == mi::pjrt::Placement::kPinnedHost ? "pinned_host" : "device"; }
  int kind_id() const { return space == mi::pjrt::Placement::kPinnedHost ? 1 : 0; }
};

struct PJRT_Device {
  PJRT_DeviceDescription desc;
  PJRT_Client* client = nullptr;
  int hip_ordinal = -1;  // -1: placeholder device of a client that sees no GPU
  PJRT_Memory hbm;
  PJRT_Memory host;
  PJRT_Memory* spaces[2] = {&hbm, &host};  // points into itself: never copied or moved
  PJRT_Device() = default;
  PJRT_Device(const PJRT_Device&) = delete;
  PJRT_Device& operator=(const PJRT_Device&) = delete;
};

struct PJRT_TopologyDescription {
  std::deque<PJRT_DeviceDescription> own;  // standalone topologies only
  std::vector<PJRT_DeviceDescription*> list;
  mi::pjrt::NamedValues attrs;
};

struct PJRT_Client {
  int process_index = 0;
  std::deque<PJRT_Device> gpus;             // stable addresses
  std::vector<PJRT_Device*> device_list;
  std::vector<PJRT_Memory*> memory_list;
  PJRT_TopologyDescription topology;        // views onto gpus[i].desc
};

struct PJRT_Buffer {
  PJRT_Client* client = nullptr;
  PJRT_Device* device = nullptr;
  PJRT_Memory* memory = nullptr;
  PJRT_Buffer_Type type = PJRT_Buffer_Type_INVALID;
  std::vector<int64_t> dims;
  std::vector<int64_t> minor_to_major;  // row-major: rank-1 ... 0
  size_t bytes = 0;
  std::shared_ptr<mi::pjrt::Block> block;
  std::shared_ptr<mi::pjrt::Completion> defined;  // null: the bytes are ready
  int pins = 0;  // external references (IncreaseExternalReferenceCount)
  // kDeletedPinned: deleted by the owner while external references hold the
  // memory; the block goes when the last reference does
  enum class Life : uint8_t { kLive, kDeletedPinned, kDeleted } life = Life::kLive;
  bool usable() const { return life == Life::kLive && block != nullptr; }
};

// What an executable hands out about its results, in the flat arrays the
// PJRT getters return.
struct ResultTable {
  std::vector<PJRT_Buffer_Type> types;
  std::vector<size_t> ranks;
  std::vector<int64_t> dims;
  std::vector<const char*> kinds;
  std::vector<size_t> kind_lengths;
  void Fill(const mi::jam::Program& p);
};

struct PJRT_Executable {
  std::shared_ptr<mi::jam::Program> program;
  std::shared_ptr<const std::string> source;  // the StableHLO it was compiled from
  std::string fingerprint;
  ResultTable results;
};

struct PJRT_LoadedExecutable {
  PJRT_Client* client = nullptr;
  std::shared_ptr<mi::jam::Program> program;  // null once deleted
  std::shared_ptr<const std::string> source;
  std::string fingerprint;
  std::vector<PJRT_Device*> devices;
};

struct PJRT_ExecuteContext {};

struct PJRT_SerializedExecutable {
  std::string bytes;
};

// ------------------------------------------------------------------ slots
namespace mi::pjrt::slot {
#define MI_DECLARE_SLOT(Name) PJRT_Error* Name(PJRT_##Name##_Args* args);
#define MI_DECLARE_VOID_SLOT(Name) void Name(PJRT_##Name##_Args* args);
MI_PJRT_SLOTS(MI_DECLARE_SLOT, MI_DECLARE_VOID_SLOT)
#undef MI_DECLARE_SLOT
#undef MI_DECLARE_VOID_SLOT
}  // namespace mi::pjrt::slot
