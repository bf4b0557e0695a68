// PJRT C API (v0.55) plugin for one or more MI355X GPUs of one process.
//
// Object model and error surface follow the reference plugin
// (src/pjrt/api/pjrt_c_api.cc): Client / Device / Memory / Topology /
// Event / Buffer / Executable objects, errors allocated here and freed by
// the caller, borrowed strings that live as long as their object, and
// UNIMPLEMENTED "<name> is not implemented in mi355x-pjrt" for the slots
// without an implementation (pjrt_c_api.cc:124-127, 832-872).
// What changes on MI355X:
//  * buffers live in HBM (DeviceContext caching pool), not unified memory;
//  * BufferFromHostBuffer copies host->HBM before returning (the host
//    buffer may be reused at once); ToHostBuffer and Execute are
//    asynchronous: they queue work on the device stream and hand back a
//    PJRT_Event backed by a hipEvent;
//  * compile lowers StableHLO text into a jam launch plan over the mk_*
//    kernels (no MPSGraph);
//  * platform name "mi355x" (not "rocm"/"cuda", so JAX emits no GPU
//    custom_calls); multi-process execution (num_nodes > 1) is rejected:
//    collectives are outside this build.
#include <hip/hip_runtime_api.h>

#include <atomic>
#include <condition_variable>
#include <cstddef>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <memory>
#include <mutex>
#include <set>
#include <string>
#include <thread>
#include <utility>
#include <vector>

#include "execution/device.h"
#include "jam/program.h"
#include "jam/run.h"
#include "pjrt/api/pjrt_abi.h"

using mi::exec::DeviceContext;

// ------------------------------------------------------------------ objects
struct PJRT_Error {
  PJRT_Error_Code code = PJRT_Error_Code_UNKNOWN;
  std::string message;
};

struct PJRT_DeviceDescription {
  int id = 0;
  int process_index = 0;
  std::string kind = "MI355X";
  std::string debug_string;
  std::string to_string;
  std::vector<PJRT_NamedValue> attrs;
  std::vector<int64_t> coords;
  std::string arch;
};

struct PJRT_Memory {
  int id = 0;
  std::string kind;
  int kind_id = 0;
  std::string debug_string;
  std::string to_string;
  std::vector<PJRT_Device*> devices;
};

struct PJRT_Device {
  PJRT_DeviceDescription description;
  PJRT_Client* client = nullptr;
  int local_hardware_id = 0;  // HIP ordinal, -1 when no GPU is present
  bool addressable = true;
  std::vector<PJRT_Memory*> memories;
  PJRT_Memory* default_memory = nullptr;
};

struct PJRT_TopologyDescription {
  std::string platform_name = "mi355x";
  std::string platform_version = "mi355x-pjrt 0.1.0 (PJRT 0.55)";
  std::vector<std::unique_ptr<PJRT_DeviceDescription>> owned;
  std::vector<PJRT_DeviceDescription*> descriptions;
};

struct PJRT_Client {
  std::string platform_name = "mi355x";
  std::string platform_version = "mi355x-pjrt 0.1.0 (PJRT 0.55)";
  int process_index = 0;
  std::vector<std::unique_ptr<PJRT_Device>> owned_devices;
  std::vector<PJRT_Device*> devices;
  std::vector<PJRT_Device*> addressable_devices;
  std::vector<std::unique_ptr<PJRT_Memory>> owned_memories;
  std::vector<PJRT_Memory*> memories;
  std::unique_ptr<PJRT_TopologyDescription> topology;
};

// Completion state shared by events and the buffers whose data they guard.
struct EventState {
  std::mutex mu;
  std::condition_variable cv;
  bool ready = false;
  std::string error;  // empty = success
  hipEvent_t ev = nullptr;
  int ordinal = 0;
  std::vector<std::pair<PJRT_Event_OnReadyCallback, void*>> callbacks;
  bool waiter = false;

  ~EventState() {
    if (ev) (void)hipEventDestroy(ev);
  }
  // block until the GPU work is done; returns the error (empty = ok)
  std::string Wait() {
    hipEvent_t e;
    {
      std::lock_guard<std::mutex> lk(mu);
      if (ready) return error;
      e = ev;
    }
    std::string err;
    if (e) {
      (void)mi::exec::UseDevice(ordinal, nullptr);
      hipError_t r = hipEventSynchronize(e);
      if (r != hipSuccess) err = std::string("device execution failed: ") + hipGetErrorString(r);
    }
    Complete(err);
    std::lock_guard<std::mutex> lk(mu);
    return error;
  }
  bool Poll() {
    hipEvent_t e;
    {
      std::lock_guard<std::mutex> lk(mu);
      if (ready) return true;
      e = ev;
    }
    if (!e) return false;
    hipError_t r = hipEventQuery(e);
    if (r == hipErrorNotReady) return false;
    Complete(r == hipSuccess ? "" : std::string("device execution failed: ") + hipGetErrorString(r));
    return true;
  }
  void Complete(const std::string& err) {
    std::vector<std::pair<PJRT_Event_OnReadyCallback, void*>> cbs;
    {
      std::lock_guard<std::mutex> lk(mu);
      if (ready) return;
      ready = true;
      error = err;
      cbs.swap(callbacks);
    }
    cv.notify_all();
    for (auto& cb : cbs)
      cb.first(err.empty() ? nullptr : new PJRT_Error{PJRT_Error_Code_INTERNAL, err}, cb.second);
  }
};

struct PJRT_Event {
  std::shared_ptr<EventState> st;
};

struct PJRT_ExecuteContext {};

// Device or pinned-host storage of a buffer.
struct Storage {
  void* data = nullptr;
  size_t nbytes = 0;
  bool host = false;          // pinned host memory (hipHostMalloc)
  DeviceContext* dev = nullptr;
  ~Storage() {
    if (!data) return;
    if (host) (void)hipHostFree(data);
    else if (dev) dev->Free(data);
  }
};

struct PJRT_Buffer {
  PJRT_Client* client = nullptr;
  PJRT_Device* device = nullptr;
  PJRT_Memory* memory = nullptr;
  PJRT_Buffer_Type type = PJRT_Buffer_Type_INVALID;
  std::vector<int64_t> dims;
  size_t nbytes = 0;
  std::shared_ptr<Storage> storage;
  std::shared_ptr<EventState> ready;  // null = ready
  int external_refs = 0;
  bool delete_requested = false;
  bool deleted = false;
};

struct PJRT_Executable {
  std::shared_ptr<mi::jam::Program> program;
  std::string name;
  std::string fingerprint;
  std::vector<PJRT_Buffer_Type> out_types;
  std::vector<int64_t> out_dims_flat;
  std::vector<size_t> out_dim_sizes;
  std::vector<std::string> out_mem_kinds;
  std::vector<const char*> out_mem_kind_ptrs;
  std::vector<size_t> out_mem_kind_sizes;
};

struct PJRT_LoadedExecutable {
  PJRT_Client* client = nullptr;
  std::shared_ptr<mi::jam::Program> program;
  std::string fingerprint;
  std::vector<PJRT_Device*> devices;
  bool deleted = false;
};

namespace {

PJRT_Error* Err(PJRT_Error_Code c, std::string m) { return new PJRT_Error{c, std::move(m)}; }
PJRT_Error* Unimplemented(const char* name) {
  return Err(PJRT_Error_Code_UNIMPLEMENTED, std::string(name) + " is not implemented in mi355x-pjrt");
}

// callers pass the size of the struct they were compiled against; anything
// smaller than the fields this plugin reads is rejected
#define MI_CHECK_ARGS(ArgsT, a, last)                                                             \
  do {                                                                                            \
    if ((a) == nullptr || (a)->struct_size < offsetof(ArgsT, last) + sizeof(((ArgsT*)0)->last))   \
      return Err(PJRT_Error_Code_INVALID_ARGUMENT, #ArgsT ": struct_size too small");             \
  } while (0)

size_t ByteWidth(PJRT_Buffer_Type t) {
  switch (t) {
    case PJRT_Buffer_Type_PRED: case PJRT_Buffer_Type_S8: case PJRT_Buffer_Type_U8: return 1;
    case PJRT_Buffer_Type_S16: case PJRT_Buffer_Type_U16: case PJRT_Buffer_Type_F16:
    case PJRT_Buffer_Type_BF16: return 2;
    case PJRT_Buffer_Type_S32: case PJRT_Buffer_Type_U32: case PJRT_Buffer_Type_F32: return 4;
    case PJRT_Buffer_Type_S64: case PJRT_Buffer_Type_U64: case PJRT_Buffer_Type_F64: return 8;
    default: return 0;
  }
}

DeviceContext* Ctx(PJRT_Device* d, std::string* err) {
  if (!d || d->local_hardware_id < 0) {
    if (err) *err = "no HIP device is available to this client";
    return nullptr;
  }
  return DeviceContext::Get(d->local_hardware_id, err);
}

PJRT_Event* ReadyEvent() {
  auto* e = new PJRT_Event{std::make_shared<EventState>()};
  e->st->ready = true;
  return e;
}

// hipEvent recorded on the device stream after everything queued so far
std::shared_ptr<EventState> RecordEvent(DeviceContext* dev, std::string* err) {
  auto st = std::make_shared<EventState>();
  st->ordinal = dev->ordinal();
  (void)mi::exec::UseDevice(dev->ordinal(), nullptr);
  hipError_t r = hipEventCreateWithFlags(&st->ev, hipEventDisableTiming);
  if (r == hipSuccess) r = hipEventRecord(st->ev, dev->stream());
  if (r != hipSuccess) {
    if (err) *err = std::string("hipEventRecord: ") + hipGetErrorString(r);
    return nullptr;
  }
  return st;
}

std::string Fnv(const char* p, size_t n) {
  uint64_t h = 1469598103934665603ull;
  for (size_t i = 0; i < n; ++i) h = (h ^ uint8_t(p[i])) * 1099511628211ull;
  char buf[32];
  snprintf(buf, sizeof(buf), "%016llx", (unsigned long long)h);
  return buf;
}

PJRT_Client* CreateClient(int node_id) {
  auto client = std::make_unique<PJRT_Client>();
  client->process_index = node_id;
  const int n_gpu = DeviceContext::DeviceCount();
  const int n = n_gpu > 0 ? n_gpu : 1;  // one placeholder device when no GPU is visible
  for (int k = 0; k < n; ++k) {
    const std::string ks = std::to_string(k);
    auto dev = std::make_unique<PJRT_Device>();
    dev->client = client.get();
    dev->local_hardware_id = n_gpu > 0 ? k : -1;
    dev->description.id = k;
    dev->description.process_index = node_id;
    dev->description.to_string = "MI355X(id=" + ks + ")";
    dev->description.debug_string = "mi355x:" + ks;
    PJRT_Device* d = dev.get();
    auto hbm = std::make_unique<PJRT_Memory>();
    hbm->id = 2 * k;
    hbm->kind = "device";
    hbm->kind_id = 0;
    hbm->debug_string = "hbm:" + ks;
    hbm->to_string = "HbmMemory(id=" + ks + ")";
    hbm->devices.push_back(d);
    auto host = std::make_unique<PJRT_Memory>();
    host->id = 2 * k + 1;
    host->kind = "pinned_host";
    host->kind_id = 1;
    host->debug_string = "pinned_host:" + ks;
    host->to_string = "PinnedHostMemory(id=" + ks + ")";
    host->devices.push_back(d);
    d->memories = {hbm.get(), host.get()};
    d->default_memory = hbm.get();
    client->memories.push_back(hbm.get());
    client->memories.push_back(host.get());
    client->addressable_devices.push_back(d);
    client->devices.push_back(d);
    client->owned_memories.push_back(std::move(hbm));
    client->owned_memories.push_back(std::move(host));
    client->owned_devices.push_back(std::move(dev));
  }
  auto topo = std::make_unique<PJRT_TopologyDescription>();
  for (PJRT_Device* d : client->devices) topo->descriptions.push_back(&d->description);
  client->topology = std::move(topo);
  return client.release();
}

// ------------------------------------------------------------------ errors / events / plugin
void ErrorDestroy(PJRT_Error_Destroy_Args* a) {
  if (a) delete a->error;
}
void ErrorMessage(PJRT_Error_Message_Args* a) {
  a->message = a->error->message.c_str();
  a->message_size = a->error->message.size();
}
PJRT_Error* ErrorGetCode(PJRT_Error_GetCode_Args* a) {
  a->code = a->error->code;
  return nullptr;
}

PJRT_Error* EventDestroy(PJRT_Event_Destroy_Args* a) {
  delete a->event;
  return nullptr;
}
PJRT_Error* EventIsReady(PJRT_Event_IsReady_Args* a) {
  MI_CHECK_ARGS(PJRT_Event_IsReady_Args, a, is_ready);
  a->is_ready = a->event->st->Poll();
  return nullptr;
}
PJRT_Error* EventError(PJRT_Event_Error_Args* a) {
  std::lock_guard<std::mutex> lk(a->event->st->mu);
  const std::string& e = a->event->st->error;
  return e.empty() ? nullptr : Err(PJRT_Error_Code_INTERNAL, e);
}
PJRT_Error* EventAwait(PJRT_Event_Await_Args* a) {
  std::string e = a->event->st->Wait();
  return e.empty() ? nullptr : Err(PJRT_Error_Code_INTERNAL, e);
}
PJRT_Error* EventOnReady(PJRT_Event_OnReady_Args* a) {
  MI_CHECK_ARGS(PJRT_Event_OnReady_Args, a, user_arg);
  std::shared_ptr<EventState> st = a->event->st;
  std::unique_lock<std::mutex> lk(st->mu);
  if (st->ready) {
    std::string e = st->error;
    lk.unlock();
    a->callback(e.empty() ? nullptr : Err(PJRT_Error_Code_INTERNAL, e), a->user_arg);
    return nullptr;
  }
  st->callbacks.emplace_back(a->callback, a->user_arg);
  if (!st->waiter) {
    st->waiter = true;
    lk.unlock();
    std::thread([st]() { st->Wait(); }).detach();
  }
  return nullptr;
}

PJRT_Error* PluginInitialize(PJRT_Plugin_Initialize_Args*) { return nullptr; }
PJRT_Error* PluginAttributes(PJRT_Plugin_Attributes_Args* a) {
  a->attributes = nullptr;
  a->num_attributes = 0;
  return nullptr;
}

// ------------------------------------------------------------------ client
PJRT_Error* ClientCreate(PJRT_Client_Create_Args* a) {
  MI_CHECK_ARGS(PJRT_Client_Create_Args, a, client);
  int node_id = 0, num_nodes = 1;
  for (size_t i = 0; i < a->num_options; ++i) {
    const PJRT_NamedValue& nv = a->create_options[i];
    const std::string name(nv.name, nv.name_size);
    if (nv.type == PJRT_NamedValue_kInt64) {
      if (name == "node_id") node_id = int(nv.int64_value);
      else if (name == "num_nodes") num_nodes = int(nv.int64_value);
    }
  }
  if (num_nodes > 1)
    return Err(PJRT_Error_Code_UNIMPLEMENTED,
               "mi355x-pjrt runs one process on one node: num_nodes > 1 needs the collective "
               "path, which this build does not include");
  a->client = CreateClient(node_id < 0 ? 0 : node_id);
  return nullptr;
}
PJRT_Error* ClientDestroy(PJRT_Client_Destroy_Args* a) {
  delete a->client;
  return nullptr;
}
PJRT_Error* ClientPlatformName(PJRT_Client_PlatformName_Args* a) {
  a->platform_name = a->client->platform_name.c_str();
  a->platform_name_size = a->client->platform_name.size();
  return nullptr;
}
PJRT_Error* ClientPlatformVersion(PJRT_Client_PlatformVersion_Args* a) {
  a->platform_version = a->client->platform_version.c_str();
  a->platform_version_size = a->client->platform_version.size();
  return nullptr;
}
PJRT_Error* ClientProcessIndex(PJRT_Client_ProcessIndex_Args* a) {
  a->process_index = a->client->process_index;
  return nullptr;
}
PJRT_Error* ClientDevices(PJRT_Client_Devices_Args* a) {
  a->devices = a->client->devices.data();
  a->num_devices = a->client->devices.size();
  return nullptr;
}
PJRT_Error* ClientAddressableDevices(PJRT_Client_AddressableDevices_Args* a) {
  a->addressable_devices = a->client->addressable_devices.data();
  a->num_addressable_devices = a->client->addressable_devices.size();
  return nullptr;
}
PJRT_Error* ClientAddressableMemories(PJRT_Client_AddressableMemories_Args* a) {
  a->addressable_memories = a->client->memories.data();
  a->num_addressable_memories = a->client->memories.size();
  return nullptr;
}
PJRT_Error* ClientLookupDevice(PJRT_Client_LookupDevice_Args* a) {
  for (PJRT_Device* d : a->client->devices)
    if (d->description.id == a->id) {
      a->device = d;
      return nullptr;
    }
  return Err(PJRT_Error_Code_INVALID_ARGUMENT, "no device with id " + std::to_string(a->id));
}
PJRT_Error* ClientLookupAddressableDevice(PJRT_Client_LookupAddressableDevice_Args* a) {
  for (PJRT_Device* d : a->client->addressable_devices)
    if (d->local_hardware_id == a->local_hardware_id) {
      a->addressable_device = d;
      return nullptr;
    }
  return Err(PJRT_Error_Code_INVALID_ARGUMENT,
             "no addressable device with local hardware id " + std::to_string(a->local_hardware_id));
}
PJRT_Error* ClientDefaultDeviceAssignment(PJRT_Client_DefaultDeviceAssignment_Args* a) {
  const size_t n = size_t(a->num_replicas) * size_t(a->num_partitions);
  const size_t nd = a->client->devices.size();
  for (size_t i = 0; i < n && i < a->default_assignment_size; ++i) a->default_assignment[i] = int(i % nd);
  return nullptr;
}
PJRT_Error* ClientTopologyDescription(PJRT_Client_TopologyDescription_Args* a) {
  a->topology = a->client->topology.get();
  return nullptr;
}

// ------------------------------------------------------------------ devices / memories
PJRT_Error* DeviceGetDescription(PJRT_Device_GetDescription_Args* a) {
  a->device_description = &a->device->description;
  return nullptr;
}
PJRT_Error* DeviceIsAddressable(PJRT_Device_IsAddressable_Args* a) {
  a->is_addressable = a->device->addressable;
  return nullptr;
}
PJRT_Error* DeviceLocalHardwareId(PJRT_Device_LocalHardwareId_Args* a) {
  a->local_hardware_id = a->device->local_hardware_id;
  return nullptr;
}
PJRT_Error* DeviceAddressableMemories(PJRT_Device_AddressableMemories_Args* a) {
  a->memories = a->device->memories.data();
  a->num_memories = a->device->memories.size();
  return nullptr;
}
PJRT_Error* DeviceDefaultMemory(PJRT_Device_DefaultMemory_Args* a) {
  a->memory = a->device->default_memory;
  return nullptr;
}
PJRT_Error* DeviceMemoryStats(PJRT_Device_MemoryStats_Args* a) {
  MI_CHECK_ARGS(PJRT_Device_MemoryStats_Args, a, peak_pool_bytes_is_set);
  std::string err;
  DeviceContext* dev = Ctx(a->device, &err);
  if (!dev) return Err(PJRT_Error_Code_UNAVAILABLE, err);
  mi::exec::MemoryStats s = dev->Stats();
  a->bytes_in_use = s.bytes_in_use;
  a->peak_bytes_in_use = s.peak_bytes_in_use;
  a->peak_bytes_in_use_is_set = true;
  a->num_allocs = s.num_allocs;
  a->num_allocs_is_set = true;
  a->largest_alloc_size = s.largest_alloc;
  a->largest_alloc_size_is_set = true;
  a->bytes_limit = s.bytes_limit;
  a->bytes_limit_is_set = true;
  a->bytes_reserved = s.bytes_reserved;
  a->bytes_reserved_is_set = true;
  a->peak_bytes_reserved_is_set = false;
  a->bytes_reservable_limit_is_set = false;
  a->largest_free_block_bytes_is_set = false;
  a->pool_bytes = s.bytes_reserved;
  a->pool_bytes_is_set = true;
  a->peak_pool_bytes_is_set = false;
  return nullptr;
}

PJRT_Error* DescId(PJRT_DeviceDescription_Id_Args* a) {
  a->id = a->device_description->id;
  return nullptr;
}
PJRT_Error* DescProcessIndex(PJRT_DeviceDescription_ProcessIndex_Args* a) {
  a->process_index = a->device_description->process_index;
  return nullptr;
}
PJRT_Error* DescAttributes(PJRT_DeviceDescription_Attributes_Args* a) {
  a->num_attributes = 0;
  a->attributes = nullptr;
  return nullptr;
}
PJRT_Error* DescKind(PJRT_DeviceDescription_Kind_Args* a) {
  a->device_kind = a->device_description->kind.c_str();
  a->device_kind_size = a->device_description->kind.size();
  return nullptr;
}
PJRT_Error* DescDebugString(PJRT_DeviceDescription_DebugString_Args* a) {
  a->debug_string = a->device_description->debug_string.c_str();
  a->debug_string_size = a->device_description->debug_string.size();
  return nullptr;
}
PJRT_Error* DescToString(PJRT_DeviceDescription_ToString_Args* a) {
  a->to_string = a->device_description->to_string.c_str();
  a->to_string_size = a->device_description->to_string.size();
  return nullptr;
}

PJRT_Error* MemoryId(PJRT_Memory_Id_Args* a) {
  a->id = a->memory->id;
  return nullptr;
}
PJRT_Error* MemoryKind(PJRT_Memory_Kind_Args* a) {
  a->kind = a->memory->kind.c_str();
  a->kind_size = a->memory->kind.size();
  return nullptr;
}
PJRT_Error* MemoryKindId(PJRT_Memory_Kind_Id_Args* a) {
  a->kind_id = a->memory->kind_id;
  return nullptr;
}
PJRT_Error* MemoryDebugString(PJRT_Memory_DebugString_Args* a) {
  a->debug_string = a->memory->debug_string.c_str();
  a->debug_string_size = a->memory->debug_string.size();
  return nullptr;
}
PJRT_Error* MemoryToString(PJRT_Memory_ToString_Args* a) {
  a->to_string = a->memory->to_string.c_str();
  a->to_string_size = a->memory->to_string.size();
  return nullptr;
}
PJRT_Error* MemoryAddressableByDevices(PJRT_Memory_AddressableByDevices_Args* a) {
  a->devices = a->memory->devices.data();
  a->num_devices = a->memory->devices.size();
  return nullptr;
}

// ------------------------------------------------------------------ topology / execute context
PJRT_Error* TopologyCreate(PJRT_TopologyDescription_Create_Args* a) {
  auto* t = new PJRT_TopologyDescription();
  const int n = std::max(1, DeviceContext::DeviceCount());
  for (int k = 0; k < n; ++k) {
    auto d = std::make_unique<PJRT_DeviceDescription>();
    d->id = k;
    d->to_string = "MI355X(id=" + std::to_string(k) + ")";
    d->debug_string = "mi355x:" + std::to_string(k);
    t->descriptions.push_back(d.get());
    t->owned.push_back(std::move(d));
  }
  a->topology = t;
  return nullptr;
}
PJRT_Error* TopologyDestroy(PJRT_TopologyDescription_Destroy_Args* a) {
  delete a->topology;
  return nullptr;
}
PJRT_Error* TopologyPlatformName(PJRT_TopologyDescription_PlatformName_Args* a) {
  a->platform_name = a->topology->platform_name.c_str();
  a->platform_name_size = a->topology->platform_name.size();
  return nullptr;
}
PJRT_Error* TopologyPlatformVersion(PJRT_TopologyDescription_PlatformVersion_Args* a) {
  a->platform_version = a->topology->platform_version.c_str();
  a->platform_version_size = a->topology->platform_version.size();
  return nullptr;
}
PJRT_Error* TopologyGetDeviceDescriptions(PJRT_TopologyDescription_GetDeviceDescriptions_Args* a) {
  a->descriptions = a->topology->descriptions.data();
  a->num_descriptions = a->topology->descriptions.size();
  return nullptr;
}
PJRT_Error* TopologyAttributes(PJRT_TopologyDescription_Attributes_Args* a) {
  a->attributes = nullptr;
  a->num_attributes = 0;
  return nullptr;
}
PJRT_Error* ExecuteContextCreate(PJRT_ExecuteContext_Create_Args* a) {
  a->context = new PJRT_ExecuteContext();
  return nullptr;
}
PJRT_Error* ExecuteContextDestroy(PJRT_ExecuteContext_Destroy_Args* a) {
  delete a->context;
  return nullptr;
}

// ------------------------------------------------------------------ buffers
PJRT_Buffer* NewBuffer(PJRT_Client* client, PJRT_Device* dev, PJRT_Memory* mem, PJRT_Buffer_Type type,
                       std::vector<int64_t> dims, std::shared_ptr<Storage> storage) {
  auto* b = new PJRT_Buffer();
  b->client = client;
  b->device = dev;
  b->memory = mem;
  b->type = type;
  b->dims = std::move(dims);
  b->nbytes = storage->nbytes;
  b->storage = std::move(storage);
  return b;
}

std::shared_ptr<Storage> AllocStorage(PJRT_Device* dev, bool host, size_t nbytes, std::string* err) {
  auto s = std::make_shared<Storage>();
  s->nbytes = nbytes;
  s->host = host;
  if (nbytes == 0) return s;
  if (host) {
    if (hipHostMalloc(&s->data, nbytes, hipHostMallocDefault) != hipSuccess) {
      (void)hipGetLastError();
      *err = "hipHostMalloc failed";
      s->data = nullptr;
      return nullptr;
    }
    return s;
  }
  s->dev = Ctx(dev, err);
  if (!s->dev) return nullptr;
  s->data = s->dev->Alloc(nbytes, err);
  if (!s->data) return nullptr;
  return s;
}

PJRT_Error* ClientBufferFromHostBuffer(PJRT_Client_BufferFromHostBuffer_Args* a) {
  MI_CHECK_ARGS(PJRT_Client_BufferFromHostBuffer_Args, a, buffer);
  const size_t width = ByteWidth(a->type);
  if (width == 0) return Err(PJRT_Error_Code_UNIMPLEMENTED, "BufferFromHostBuffer: unsupported element type");
  if (a->device_layout != nullptr)
    return Err(PJRT_Error_Code_UNIMPLEMENTED, "BufferFromHostBuffer: custom device layouts are not supported");
  size_t count = 1;
  for (size_t i = 0; i < a->num_dims; ++i) {
    if (a->dims[i] < 0) return Err(PJRT_Error_Code_INVALID_ARGUMENT, "BufferFromHostBuffer: negative dimension");
    count *= size_t(a->dims[i]);
  }
  const size_t nbytes = count * width;
  PJRT_Device* device = a->device;
  PJRT_Memory* memory = a->memory;
  if (!device && memory && !memory->devices.empty()) device = memory->devices.front();
  if (!device) device = a->client->addressable_devices.front();
  if (!memory) memory = device->default_memory;
  const bool host = memory->kind == "pinned_host";
  // gather a strided host array into dense row-major order first
  const char* src = static_cast<const char*>(a->data);
  std::vector<char> packed;
  if (a->byte_strides && a->num_byte_strides == a->num_dims && count > 0) {
    bool dense = true;
    int64_t expect = int64_t(width);
    for (int d = int(a->num_dims) - 1; d >= 0; --d) {
      if (a->dims[d] != 1 && a->byte_strides[d] != expect) dense = false;
      expect *= a->dims[d];
    }
    if (!dense) {
      packed.resize(nbytes);
      std::vector<int64_t> idx(a->num_dims, 0);
      for (size_t e = 0; e < count; ++e) {
        int64_t off = 0;
        for (size_t d = 0; d < a->num_dims; ++d) off += idx[d] * a->byte_strides[d];
        memcpy(&packed[e * width], src + off, width);
        for (int d = int(a->num_dims) - 1; d >= 0; --d) {
          if (++idx[d] < a->dims[d]) break;
          idx[d] = 0;
        }
      }
      src = packed.data();
    }
  }
  std::string err;
  auto storage = AllocStorage(device, host, nbytes, &err);
  if (!storage) return Err(PJRT_Error_Code_RESOURCE_EXHAUSTED, "BufferFromHostBuffer: " + err);
  if (nbytes) {
    if (host) {
      memcpy(storage->data, src, nbytes);
    } else if (!storage->dev->CopyToDevice(storage->data, src, nbytes, &err)) {
      return Err(PJRT_Error_Code_INTERNAL, "BufferFromHostBuffer: " + err);
    }
  }
  a->buffer = NewBuffer(a->client, device, memory, a->type,
                        std::vector<int64_t>(a->dims, a->dims + a->num_dims), std::move(storage));
  a->done_with_host_buffer = ReadyEvent();  // the copy finished before returning
  return nullptr;
}

PJRT_Error* BufferToHostBuffer(PJRT_Buffer_ToHostBuffer_Args* a) {
  MI_CHECK_ARGS(PJRT_Buffer_ToHostBuffer_Args, a, event);
  PJRT_Buffer* b = a->src;
  if (b->deleted) return Err(PJRT_Error_Code_INVALID_ARGUMENT, "ToHostBuffer: buffer was deleted");
  if (a->host_layout != nullptr)
    return Err(PJRT_Error_Code_UNIMPLEMENTED, "ToHostBuffer: host layouts are not supported");
  if (a->dst == nullptr) {
    a->dst_size = b->nbytes;
    a->event = ReadyEvent();
    return nullptr;
  }
  if (a->dst_size < b->nbytes) return Err(PJRT_Error_Code_INVALID_ARGUMENT, "ToHostBuffer: dst_size too small");
  Storage* s = b->storage.get();
  if (b->nbytes == 0) {
    a->event = ReadyEvent();
    return nullptr;
  }
  if (s->host) {
    memcpy(a->dst, s->data, b->nbytes);
    a->event = ReadyEvent();
    return nullptr;
  }
  std::string err;
  if (!s->dev->CopyToHostAsync(a->dst, s->data, b->nbytes, &err))
    return Err(PJRT_Error_Code_INTERNAL, "ToHostBuffer: " + err);
  auto st = RecordEvent(s->dev, &err);
  if (!st) return Err(PJRT_Error_Code_INTERNAL, "ToHostBuffer: " + err);
  a->event = new PJRT_Event{st};
  return nullptr;
}

PJRT_Buffer* CopyBuffer(PJRT_Buffer* src, PJRT_Device* dev, PJRT_Memory* mem, std::string* err) {
  const bool host = mem->kind == "pinned_host";
  auto storage = AllocStorage(dev, host, src->nbytes, err);
  if (!storage) return nullptr;
  Storage* s = src->storage.get();
  if (src->nbytes) {
    hipMemcpyKind kind = s->host ? (host ? hipMemcpyHostToHost : hipMemcpyHostToDevice)
                                 : (host ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice);
    DeviceContext* ctx = s->dev ? s->dev : storage->dev;
    hipStream_t stream = ctx ? ctx->stream() : nullptr;
    if (ctx) (void)mi::exec::UseDevice(ctx->ordinal(), nullptr);
    hipError_t e = hipMemcpyAsync(storage->data, s->data, src->nbytes, kind, stream);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    if (e != hipSuccess) {
      *err = std::string("copy failed: ") + hipGetErrorString(e);
      return nullptr;
    }
  }
  return NewBuffer(src->client, dev, mem, src->type, src->dims, std::move(storage));
}

PJRT_Error* BufferCopyToMemory(PJRT_Buffer_CopyToMemory_Args* a) {
  if (a->buffer->deleted) return Err(PJRT_Error_Code_INVALID_ARGUMENT, "CopyToMemory: deleted buffer");
  PJRT_Memory* mem = a->dst_memory;
  if (!mem) return Err(PJRT_Error_Code_INVALID_ARGUMENT, "CopyToMemory: null memory");
  PJRT_Device* dev = mem->devices.empty() ? a->buffer->device : mem->devices.front();
  std::string err;
  a->dst_buffer = CopyBuffer(a->buffer, dev, mem, &err);
  return a->dst_buffer ? nullptr : Err(PJRT_Error_Code_RESOURCE_EXHAUSTED, "CopyToMemory: " + err);
}
PJRT_Error* BufferCopyToDevice(PJRT_Buffer_CopyToDevice_Args* a) {
  if (a->buffer->deleted) return Err(PJRT_Error_Code_INVALID_ARGUMENT, "CopyToDevice: deleted buffer");
  PJRT_Device* dev = a->dst_device;
  if (!dev) return Err(PJRT_Error_Code_INVALID_ARGUMENT, "CopyToDevice: null device");
  std::string err;
  a->dst_buffer = CopyBuffer(a->buffer, dev, dev->default_memory, &err);
  return a->dst_buffer ? nullptr : Err(PJRT_Error_Code_RESOURCE_EXHAUSTED, "CopyToDevice: " + err);
}

PJRT_Error* BufferDestroy(PJRT_Buffer_Destroy_Args* a) {
  delete a->buffer;  // storage is released with the last reference
  return nullptr;
}
PJRT_Error* BufferDelete(PJRT_Buffer_Delete_Args* a) {
  PJRT_Buffer* b = a->buffer;
  b->deleted = true;
  if (b->external_refs == 0) b->storage.reset();
  else b->delete_requested = true;
  return nullptr;
}
PJRT_Error* BufferIsDeleted(PJRT_Buffer_IsDeleted_Args* a) {
  a->is_deleted = a->buffer->deleted;
  return nullptr;
}
PJRT_Error* BufferElementType(PJRT_Buffer_ElementType_Args* a) {
  a->type = a->buffer->type;
  return nullptr;
}
PJRT_Error* BufferDimensions(PJRT_Buffer_Dimensions_Args* a) {
  a->dims = a->buffer->dims.data();
  a->num_dims = a->buffer->dims.size();
  return nullptr;
}
PJRT_Error* BufferUnpaddedDimensions(PJRT_Buffer_UnpaddedDimensions_Args* a) {
  a->unpadded_dims = a->buffer->dims.data();
  a->num_dims = a->buffer->dims.size();
  return nullptr;
}
PJRT_Error* BufferDynamicDimensionIndices(PJRT_Buffer_DynamicDimensionIndices_Args* a) {
  a->dynamic_dim_indices = nullptr;
  a->num_dynamic_dims = 0;
  return nullptr;
}
PJRT_Error* BufferOnDeviceSizeInBytes(PJRT_Buffer_OnDeviceSizeInBytes_Args* a) {
  a->on_device_size_in_bytes = a->buffer->nbytes;
  return nullptr;
}
PJRT_Error* BufferDevice(PJRT_Buffer_Device_Args* a) {
  a->device = a->buffer->device;
  return nullptr;
}
PJRT_Error* BufferMemory(PJRT_Buffer_Memory_Args* a) {
  a->memory = a->buffer->memory;
  return nullptr;
}
PJRT_Error* BufferIsOnCpu(PJRT_Buffer_IsOnCpu_Args* a) {
  a->is_on_cpu = a->buffer->storage && a->buffer->storage->host;
  return nullptr;
}
PJRT_Error* BufferReadyEvent(PJRT_Buffer_ReadyEvent_Args* a) {
  if (a->buffer->ready) a->event = new PJRT_Event{a->buffer->ready};
  else a->event = ReadyEvent();
  return nullptr;
}
PJRT_Error* BufferUnsafePointer(PJRT_Buffer_UnsafePointer_Args* a) {
  a->buffer_pointer = reinterpret_cast<uintptr_t>(a->buffer->storage ? a->buffer->storage->data : nullptr);
  return nullptr;
}
PJRT_Error* BufferOpaqueDeviceMemoryDataPointer(PJRT_Buffer_OpaqueDeviceMemoryDataPointer_Args* a) {
  a->device_memory_ptr = a->buffer->storage ? a->buffer->storage->data : nullptr;
  return nullptr;
}
PJRT_Error* BufferIncreaseExternalReferenceCount(PJRT_Buffer_IncreaseExternalReferenceCount_Args* a) {
  ++a->buffer->external_refs;
  return nullptr;
}
PJRT_Error* BufferDecreaseExternalReferenceCount(PJRT_Buffer_DecreaseExternalReferenceCount_Args* a) {
  PJRT_Buffer* b = a->buffer;
  if (b->external_refs > 0) --b->external_refs;
  if (b->external_refs == 0 && b->delete_requested) b->storage.reset();
  return nullptr;
}

// ------------------------------------------------------------------ compile / executables
PJRT_Buffer_Type ToPjrt(mi::jam::DType d) { return PJRT_Buffer_Type(int(d)); }

void CacheOutputs(PJRT_Executable* e) {
  for (const auto& t : e->program->outputs) {
    e->out_types.push_back(ToPjrt(t.dtype));
    e->out_dim_sizes.push_back(t.dims.size());
    for (int64_t d : t.dims) e->out_dims_flat.push_back(d);
    e->out_mem_kinds.push_back("device");
  }
  for (const auto& k : e->out_mem_kinds) {
    e->out_mem_kind_ptrs.push_back(k.c_str());
    e->out_mem_kind_sizes.push_back(k.size());
  }
}

PJRT_Error* ClientCompile(PJRT_Client_Compile_Args* a) {
  MI_CHECK_ARGS(PJRT_Client_Compile_Args, a, executable);
  const PJRT_Program* p = a->program;
  if (!p || !p->code) return Err(PJRT_Error_Code_INVALID_ARGUMENT, "jam compile: null program");
  const std::string format(p->format ? p->format : "", p->format ? p->format_size : 0);
  if (!format.empty() && format != "mlir")
    return Err(PJRT_Error_Code_INVALID_ARGUMENT, "jam compile: unsupported program format '" + format + "'");
  if (const char* dump = std::getenv("JAM_DUMP_ARTIFACT")) {  // pjrt_c_api.cc:684-686
    if (FILE* f = std::fopen(dump, "wb")) {
      std::fwrite(p->code, 1, p->code_size, f);
      std::fclose(f);
    }
  }
  mi::jam::CompileResult r = mi::jam::Compile(p->code, p->code_size, mi::jam::OptionsFromEnv());
  if (!r.program) return Err(PJRT_Error_Code_INVALID_ARGUMENT, "jam compile: " + r.error);
  if (std::getenv("JAM_DUMP_PLAN")) std::fputs(r.program->Dump().c_str(), stderr);
  auto le = std::make_unique<PJRT_LoadedExecutable>();
  le->client = a->client;
  le->program = r.program;
  le->fingerprint = Fnv(p->code, p->code_size);
  le->devices = {a->client->addressable_devices.front()};
  a->executable = le.release();
  return nullptr;
}

PJRT_Error* LoadedGetExecutable(PJRT_LoadedExecutable_GetExecutable_Args* a) {
  if (!a->loaded_executable->program)
    return Err(PJRT_Error_Code_INVALID_ARGUMENT, "GetExecutable: executable was deleted");
  auto* e = new PJRT_Executable();
  e->program = a->loaded_executable->program;
  e->name = e->program->name;
  e->fingerprint = a->loaded_executable->fingerprint;
  CacheOutputs(e);
  a->executable = e;
  return nullptr;
}
PJRT_Error* ExecutableDestroy(PJRT_Executable_Destroy_Args* a) {
  delete a->executable;
  return nullptr;
}
PJRT_Error* ExecutableName(PJRT_Executable_Name_Args* a) {
  a->executable_name = a->executable->name.c_str();
  a->executable_name_size = a->executable->name.size();
  return nullptr;
}
PJRT_Error* ExecutableNumReplicas(PJRT_Executable_NumReplicas_Args* a) {
  a->num_replicas = 1;
  return nullptr;
}
PJRT_Error* ExecutableNumPartitions(PJRT_Executable_NumPartitions_Args* a) {
  a->num_partitions = 1;
  return nullptr;
}
PJRT_Error* ExecutableNumOutputs(PJRT_Executable_NumOutputs_Args* a) {
  a->num_outputs = a->executable->program->outputs.size();
  return nullptr;
}
PJRT_Error* ExecutableSizeOfGeneratedCode(PJRT_Executable_SizeOfGeneratedCodeInBytes_Args* a) {
  a->size_in_bytes = int64_t(a->executable->program->steps.size() * sizeof(mi::jam::Step));
  return nullptr;
}
PJRT_Error* ExecutableFingerprint(PJRT_Executable_Fingerprint_Args* a) {
  a->executable_fingerprint = a->executable->fingerprint.c_str();
  a->executable_fingerprint_size = a->executable->fingerprint.size();
  return nullptr;
}
PJRT_Error* LoadedFingerprint(PJRT_LoadedExecutable_Fingerprint_Args* a) {
  a->executable_fingerprint = a->executable->fingerprint.c_str();
  a->executable_fingerprint_size = a->executable->fingerprint.size();
  return nullptr;
}
// The "optimized program" of a jam executable is its launch plan, as text
// (format "jam-plan"); two-call protocol: code == nullptr asks for the size.
PJRT_Error* ExecutableOptimizedProgram(PJRT_Executable_OptimizedProgram_Args* a) {
  MI_CHECK_ARGS(PJRT_Executable_OptimizedProgram_Args, a, program);
  static const char kFormat[] = "jam-plan";
  PJRT_Program* p = a->program;
  if (!p) return Err(PJRT_Error_Code_INVALID_ARGUMENT, "OptimizedProgram: null program");
  const std::string text = a->executable->program->Dump();
  p->format = kFormat;
  p->format_size = sizeof(kFormat) - 1;
  if (p->code == nullptr) {
    p->code_size = text.size();
    return nullptr;
  }
  if (p->code_size < text.size())
    return Err(PJRT_Error_Code_INVALID_ARGUMENT, "OptimizedProgram: code buffer too small");
  memcpy(p->code, text.data(), text.size());
  p->code_size = text.size();
  return nullptr;
}
PJRT_Error* ExecutableGetCostAnalysis(PJRT_Executable_GetCostAnalysis_Args* a) {
  a->num_properties = 0;
  a->properties = nullptr;
  return nullptr;
}
PJRT_Error* ExecutableOutputElementTypes(PJRT_Executable_OutputElementTypes_Args* a) {
  a->output_types = a->executable->out_types.data();
  a->num_output_types = a->executable->out_types.size();
  return nullptr;
}
PJRT_Error* ExecutableOutputDimensions(PJRT_Executable_OutputDimensions_Args* a) {
  PJRT_Executable* e = a->executable;
  a->num_outputs = e->out_dim_sizes.size();
  a->dims = e->out_dims_flat.data();
  a->dim_sizes = e->out_dim_sizes.data();
  return nullptr;
}
PJRT_Error* ExecutableOutputMemoryKinds(PJRT_Executable_OutputMemoryKinds_Args* a) {
  PJRT_Executable* e = a->executable;
  a->num_outputs = e->out_mem_kind_ptrs.size();
  a->memory_kinds = e->out_mem_kind_ptrs.data();
  a->memory_kind_sizes = e->out_mem_kind_sizes.data();
  return nullptr;
}
PJRT_Error* ExecutableGetCompiledMemoryStats(PJRT_Executable_GetCompiledMemoryStats_Args* a) {
  const auto& p = *a->executable->program;
  int64_t in = 0, out = 0;
  for (const auto& t : p.inputs) in += int64_t(t.bytes());
  for (const auto& t : p.outputs) out += int64_t(t.bytes());
  a->generated_code_size_in_bytes = 0;
  a->argument_size_in_bytes = in;
  a->output_size_in_bytes = out;
  a->alias_size_in_bytes = 0;
  a->temp_size_in_bytes = int64_t(p.arena_bytes);
  a->host_generated_code_size_in_bytes = 0;
  a->host_argument_size_in_bytes = 0;
  a->host_output_size_in_bytes = 0;
  a->host_alias_size_in_bytes = 0;
  a->host_temp_size_in_bytes = 0;
  return nullptr;
}
PJRT_Error* LoadedDestroy(PJRT_LoadedExecutable_Destroy_Args* a) {
  delete a->executable;
  return nullptr;
}
PJRT_Error* LoadedDelete(PJRT_LoadedExecutable_Delete_Args* a) {
  a->executable->deleted = true;
  a->executable->program.reset();
  return nullptr;
}
PJRT_Error* LoadedIsDeleted(PJRT_LoadedExecutable_IsDeleted_Args* a) {
  a->is_deleted = a->executable->deleted;
  return nullptr;
}
PJRT_Error* LoadedAddressableDevices(PJRT_LoadedExecutable_AddressableDevices_Args* a) {
  a->addressable_devices = a->executable->devices.data();
  a->num_addressable_devices = a->executable->devices.size();
  return nullptr;
}

PJRT_Error* LoadedExecute(PJRT_LoadedExecutable_Execute_Args* a) {
  MI_CHECK_ARGS(PJRT_LoadedExecutable_Execute_Args, a, execute_device);
  PJRT_LoadedExecutable* le = a->executable;
  std::shared_ptr<mi::jam::Program> prog = le->program;
  if (!prog) return Err(PJRT_Error_Code_INVALID_ARGUMENT, "Execute: deleted executable");  // pjrt_c_api.cc:755
  if (a->num_args != prog->inputs.size())
    return Err(PJRT_Error_Code_INVALID_ARGUMENT, "Execute: expected " + std::to_string(prog->inputs.size()) +
                                                     " arguments, got " + std::to_string(a->num_args));
  for (size_t d = 0; d < a->num_devices; ++d) {
    PJRT_Device* dev = a->execute_device;
    if (!dev) {
      dev = a->num_devices == 1 ? le->devices.front()
                                : le->client->addressable_devices[d % le->client->addressable_devices.size()];
    }
    std::string err;
    DeviceContext* ctx = Ctx(dev, &err);
    if (!ctx) return Err(PJRT_Error_Code_UNAVAILABLE, "Execute: " + err);
    std::vector<mi::jam::RunInput> ins;
    ins.reserve(a->num_args);
    std::vector<std::shared_ptr<Storage>> keep;  // inputs stay alive until launches are queued
    // Donation: an input the program may overwrite with an output
    // (prog->input_alias) gives that output its memory, unless the caller
    // lists it in non_donatable_input_indices, or its storage is shared
    // (external references, another buffer, or passed twice).
    std::vector<void*> preset(prog->outputs.size(), nullptr);
    std::vector<std::pair<size_t, int>> donated;  // (argument, output)
    {
      std::set<int64_t> keep_args;
      const PJRT_ExecuteOptions* opt = a->options;
      const size_t need = offsetof(PJRT_ExecuteOptions, num_non_donatable_input_indices) + sizeof(size_t);
      if (opt && opt->struct_size < need)
        return Err(PJRT_Error_Code_INVALID_ARGUMENT, "Execute: PJRT_ExecuteOptions struct_size too small");
      if (opt && opt->non_donatable_input_indices)
        for (size_t k = 0; k < opt->num_non_donatable_input_indices; ++k)
          keep_args.insert(opt->non_donatable_input_indices[k]);
      for (size_t i = 0; i < a->num_args && i < prog->input_alias.size(); ++i) {
        const int o = prog->input_alias[i];
        PJRT_Buffer* b = a->argument_lists[d][i];
        if (o < 0 || keep_args.count(int64_t(i)) || !b || b->deleted || !b->storage || b->storage->host ||
            b->storage->dev != ctx || b->external_refs != 0 || b->storage.use_count() != 1)
          continue;
        bool twice = false;
        for (size_t j = 0; j < a->num_args; ++j)
          if (j != i && a->argument_lists[d][j] == b) twice = true;
        if (twice) continue;
        preset[size_t(o)] = b->storage->data;
        donated.emplace_back(i, o);
      }
    }
    for (size_t i = 0; i < a->num_args; ++i) {
      PJRT_Buffer* b = a->argument_lists[d][i];
      if (!b || b->deleted || !b->storage)
        return Err(PJRT_Error_Code_INVALID_ARGUMENT, "Execute: argument " + std::to_string(i) + " was deleted");
      if (b->storage->host)
        return Err(PJRT_Error_Code_INVALID_ARGUMENT,
                   "Execute: argument " + std::to_string(i) + " is in pinned_host memory; copy it to the device first");
      if (b->storage->dev != ctx)
        return Err(PJRT_Error_Code_INVALID_ARGUMENT, "Execute: argument " + std::to_string(i) + " lives on another device");
      ins.push_back({b->storage->data, b->nbytes});
      keep.push_back(b->storage);
    }
    std::vector<mi::jam::RunOutput> outs;
    err = mi::jam::Run(*prog, *ctx, ins, outs, &preset);
    if (!err.empty()) return Err(PJRT_Error_Code_INTERNAL, err);
    std::shared_ptr<EventState> done = RecordEvent(ctx, &err);
    if (!done) return Err(PJRT_Error_Code_INTERNAL, "Execute: " + err);
    // donated inputs hand their storage to the output and are deleted
    std::vector<std::shared_ptr<Storage>> from_input(outs.size());
    for (const auto& [arg, o] : donated) {
      PJRT_Buffer* b = a->argument_lists[d][arg];
      keep.clear();  // drop the extra references taken above
      from_input[size_t(o)] = std::move(b->storage);
      b->deleted = true;
    }
    for (size_t i = 0; i < outs.size(); ++i) {
      std::shared_ptr<Storage> s = from_input[i] ? from_input[i] : std::make_shared<Storage>();
      s->data = outs[i].data;
      s->nbytes = outs[i].nbytes;
      s->dev = ctx;
      PJRT_Buffer* ob = NewBuffer(le->client, dev, dev->default_memory, ToPjrt(outs[i].type.dtype),
                                  outs[i].type.dims, std::move(s));
      ob->ready = done;
      a->output_lists[d][i] = ob;
    }
    if (a->device_complete_events) a->device_complete_events[d] = new PJRT_Event{done};
  }
  return nullptr;
}

// ------------------------------------------------------------------ unimplemented slots
#define MI_UNIMPLEMENTED(X)                                                              \
  X(Executable_Serialize) X(Executable_DeserializeAndLoad)                                \
  X(Buffer_GetMemoryLayout) X(CopyToDeviceStream_Destroy) X(CopyToDeviceStream_AddChunk)  \
  X(CopyToDeviceStream_TotalBytes) X(CopyToDeviceStream_GranuleSize)                      \
  X(CopyToDeviceStream_CurrentBytes) X(TopologyDescription_Serialize) X(Compile)          \
  X(Client_CreateViewOfDeviceBuffer)

#define MI_DEFINE_STUB(name) \
  PJRT_Error* name##_Stub(PJRT_##name##_Args*) { return Unimplemented("PJRT_" #name); }
MI_UNIMPLEMENTED(MI_DEFINE_STUB)
#undef MI_DEFINE_STUB

}  // namespace

extern "C" __attribute__((visibility("default"))) const PJRT_Api* GetPjrtApi() {
  static PJRT_Api api = [] {
    PJRT_Api a;
    memset(&a, 0, sizeof(a));
    a.struct_size = sizeof(PJRT_Api);
    a.pjrt_api_version.struct_size = sizeof(PJRT_Api_Version);
    a.pjrt_api_version.major_version = MI_PJRT_API_MAJOR;
    a.pjrt_api_version.minor_version = MI_PJRT_API_MINOR;

    a.PJRT_Error_Destroy = ErrorDestroy;
    a.PJRT_Error_Message = ErrorMessage;
    a.PJRT_Error_GetCode = ErrorGetCode;
    a.PJRT_Plugin_Initialize = PluginInitialize;
    a.PJRT_Plugin_Attributes = PluginAttributes;
    a.PJRT_Event_Destroy = EventDestroy;
    a.PJRT_Event_IsReady = EventIsReady;
    a.PJRT_Event_Error = EventError;
    a.PJRT_Event_Await = EventAwait;
    a.PJRT_Event_OnReady = EventOnReady;

    a.PJRT_Client_Create = ClientCreate;
    a.PJRT_Client_Destroy = ClientDestroy;
    a.PJRT_Client_PlatformName = ClientPlatformName;
    a.PJRT_Client_ProcessIndex = ClientProcessIndex;
    a.PJRT_Client_PlatformVersion = ClientPlatformVersion;
    a.PJRT_Client_Devices = ClientDevices;
    a.PJRT_Client_AddressableDevices = ClientAddressableDevices;
    a.PJRT_Client_LookupDevice = ClientLookupDevice;
    a.PJRT_Client_LookupAddressableDevice = ClientLookupAddressableDevice;
    a.PJRT_Client_AddressableMemories = ClientAddressableMemories;
    a.PJRT_Client_Compile = ClientCompile;
    a.PJRT_Client_DefaultDeviceAssignment = ClientDefaultDeviceAssignment;
    a.PJRT_Client_BufferFromHostBuffer = ClientBufferFromHostBuffer;
    a.PJRT_Client_TopologyDescription = ClientTopologyDescription;

    a.PJRT_DeviceDescription_Id = DescId;
    a.PJRT_DeviceDescription_ProcessIndex = DescProcessIndex;
    a.PJRT_DeviceDescription_Attributes = DescAttributes;
    a.PJRT_DeviceDescription_Kind = DescKind;
    a.PJRT_DeviceDescription_DebugString = DescDebugString;
    a.PJRT_DeviceDescription_ToString = DescToString;

    a.PJRT_Device_GetDescription = DeviceGetDescription;
    a.PJRT_Device_IsAddressable = DeviceIsAddressable;
    a.PJRT_Device_LocalHardwareId = DeviceLocalHardwareId;
    a.PJRT_Device_AddressableMemories = DeviceAddressableMemories;
    a.PJRT_Device_DefaultMemory = DeviceDefaultMemory;
    a.PJRT_Device_MemoryStats = DeviceMemoryStats;

    a.PJRT_Memory_Id = MemoryId;
    a.PJRT_Memory_Kind = MemoryKind;
    a.PJRT_Memory_Kind_Id = MemoryKindId;
    a.PJRT_Memory_DebugString = MemoryDebugString;
    a.PJRT_Memory_ToString = MemoryToString;
    a.PJRT_Memory_AddressableByDevices = MemoryAddressableByDevices;

    a.PJRT_Executable_Destroy = ExecutableDestroy;
    a.PJRT_Executable_Name = ExecutableName;
    a.PJRT_Executable_NumReplicas = ExecutableNumReplicas;
    a.PJRT_Executable_NumPartitions = ExecutableNumPartitions;
    a.PJRT_Executable_NumOutputs = ExecutableNumOutputs;
    a.PJRT_Executable_SizeOfGeneratedCodeInBytes = ExecutableSizeOfGeneratedCode;
    a.PJRT_Executable_GetCostAnalysis = ExecutableGetCostAnalysis;
    a.PJRT_Executable_OptimizedProgram = ExecutableOptimizedProgram;
    a.PJRT_Executable_OutputMemoryKinds = ExecutableOutputMemoryKinds;
    a.PJRT_Executable_OutputElementTypes = ExecutableOutputElementTypes;
    a.PJRT_Executable_OutputDimensions = ExecutableOutputDimensions;
    a.PJRT_Executable_Fingerprint = ExecutableFingerprint;
    a.PJRT_Executable_GetCompiledMemoryStats = ExecutableGetCompiledMemoryStats;

    a.PJRT_LoadedExecutable_Destroy = LoadedDestroy;
    a.PJRT_LoadedExecutable_GetExecutable = LoadedGetExecutable;
    a.PJRT_LoadedExecutable_AddressableDevices = LoadedAddressableDevices;
    a.PJRT_LoadedExecutable_Delete = LoadedDelete;
    a.PJRT_LoadedExecutable_IsDeleted = LoadedIsDeleted;
    a.PJRT_LoadedExecutable_Execute = LoadedExecute;
    a.PJRT_LoadedExecutable_Fingerprint = LoadedFingerprint;

    a.PJRT_Buffer_Destroy = BufferDestroy;
    a.PJRT_Buffer_ElementType = BufferElementType;
    a.PJRT_Buffer_Dimensions = BufferDimensions;
    a.PJRT_Buffer_UnpaddedDimensions = BufferUnpaddedDimensions;
    a.PJRT_Buffer_DynamicDimensionIndices = BufferDynamicDimensionIndices;
    a.PJRT_Buffer_OnDeviceSizeInBytes = BufferOnDeviceSizeInBytes;
    a.PJRT_Buffer_Device = BufferDevice;
    a.PJRT_Buffer_Memory = BufferMemory;
    a.PJRT_Buffer_Delete = BufferDelete;
    a.PJRT_Buffer_IsDeleted = BufferIsDeleted;
    a.PJRT_Buffer_CopyToDevice = BufferCopyToDevice;
    a.PJRT_Buffer_CopyToMemory = BufferCopyToMemory;
    a.PJRT_Buffer_ToHostBuffer = BufferToHostBuffer;
    a.PJRT_Buffer_IsOnCpu = BufferIsOnCpu;
    a.PJRT_Buffer_ReadyEvent = BufferReadyEvent;
    a.PJRT_Buffer_UnsafePointer = BufferUnsafePointer;
    a.PJRT_Buffer_IncreaseExternalReferenceCount = BufferIncreaseExternalReferenceCount;
    a.PJRT_Buffer_DecreaseExternalReferenceCount = BufferDecreaseExternalReferenceCount;
    a.PJRT_Buffer_OpaqueDeviceMemoryDataPointer = BufferOpaqueDeviceMemoryDataPointer;

    a.PJRT_TopologyDescription_Create = TopologyCreate;
    a.PJRT_TopologyDescription_Destroy = TopologyDestroy;
    a.PJRT_TopologyDescription_PlatformName = TopologyPlatformName;
    a.PJRT_TopologyDescription_PlatformVersion = TopologyPlatformVersion;
    a.PJRT_TopologyDescription_GetDeviceDescriptions = TopologyGetDeviceDescriptions;
    a.PJRT_TopologyDescription_Attributes = TopologyAttributes;

    a.PJRT_ExecuteContext_Create = ExecuteContextCreate;
    a.PJRT_ExecuteContext_Destroy = ExecuteContextDestroy;

#define MI_BIND_STUB(name) a.PJRT_##name = name##_Stub;
    MI_UNIMPLEMENTED(MI_BIND_STUB)
#undef MI_BIND_STUB
    return a;
  }();
  return &api;
}
