// Slots for errors, events, the plugin itself, clients, devices, memories,
// topologies and execute contexts.
//
// Reference counterparts: src/pjrt/api/pjrt_c_api.cc:185-451 (same PJRT
// contract: errors owned by the caller, borrowed strings that live as long
// as their object; "device"/"pinned_host" memory kinds).  The client here
// is built from the HIP devices this process sees.
#include <cstring>

#include "pjrt/api/plugin.h"

namespace mi::pjrt {
namespace {

// PJRT_Client_Create options this plugin understands (jax.distributed
// passes node_id / num_nodes as int64).
struct CreateOptions {
  int64_t node_id = 0;
  int64_t num_nodes = 1;
  std::string unknown;  // names of options that were ignored (for messages)

  static CreateOptions Read(const PJRT_NamedValue* v, size_t n) {
    CreateOptions o;
    for (size_t i = 0; i < n; ++i) {
      const std::string key(v[i].name, v[i].name_size);
      int64_t* slot = key == "node_id" ? &o.node_id : key == "num_nodes" ? &o.num_nodes : nullptr;
      if (slot && v[i].type == PJRT_NamedValue_kInt64) *slot = v[i].int64_value;
      else o.unknown += (o.unknown.empty() ? "" : ",") + key;
    }
    return o;
  }
};

PJRT_Client* BuildClient(int process) {
  auto* c = new PJRT_Client();
  c->process_index = process;
  std::vector<exec::GpuProps> gpus = VisibleGpus();
  const bool none = gpus.empty();
  if (none) gpus.emplace_back();  // one placeholder device: compile still works without a GPU
  const int n = int(gpus.size());
  for (int k = 0; k < n; ++k) {
    PJRT_Device& d = c->gpus.emplace_back();
    d.client = c;
    d.hip_ordinal = none ? -1 : k;
    Describe(&d.desc, k, process, gpus[k]);
    d.hbm.space = Placement::kHbm;
    d.hbm.id = k;
    d.host.space = Placement::kPinnedHost;
    d.host.id = n + k;
    for (PJRT_Memory* m : d.spaces) {
      m->owner[0] = &d;
      m->label = d.desc.label + "/" + m->kind();
      m->detail = std::string(m->kind()) + " memory " + std::to_string(m->id) + " of " + d.desc.label;
    }
    c->device_list.push_back(&d);
    c->topology.list.push_back(&d.desc);
  }
  for (PJRT_Device& d : c->gpus) c->memory_list.push_back(&d.hbm);
  for (PJRT_Device& d : c->gpus) c->memory_list.push_back(&d.host);
  return c;
}

}  // namespace

namespace slot {

// ------------------------------------------------------------------ errors
void Error_Destroy(PJRT_Error_Destroy_Args* a) {
  if (a) delete a->error;
}
void Error_Message(PJRT_Error_Message_Args* a) {
  a->message = a->error->text.c_str();
  a->message_size = a->error->text.size();
}
PJRT_Error* Error_GetCode(PJRT_Error_GetCode_Args* a) {
  a->code = a->error->code;
  return nullptr;
}

// ------------------------------------------------------------------ plugin
PJRT_Error* Plugin_Initialize(PJRT_Plugin_Initialize_Args*) { return nullptr; }

// Version attributes a PJRT client reads to choose what it serializes:
// the StableHLO/VHLO versions this plugin accepts (the text reader takes any
// StableHLO 1.x module; 1.0.0 is the first VHLO version with a compatibility
// guarantee) and the XLA plugin-interface version.
PJRT_Error* Plugin_Attributes(PJRT_Plugin_Attributes_Args* a) {
  MI_NEED(a, PJRT_Plugin_Attributes_Args, num_attributes);
  static const NamedValues* attrs = [] {
    auto* v = new NamedValues();
    v->Int("xla_version", 2);
    v->Ints("stablehlo_current_version", {1, 0, 0});
    v->Ints("stablehlo_minimum_version", {1, 0, 0});
    v->Bool("supports_cross_host_transfers", false);
    return v;
  }();
  a->attributes = attrs->data();
  a->num_attributes = attrs->size();
  return nullptr;
}

// ------------------------------------------------------------------ events
PJRT_Error* Event_Destroy(PJRT_Event_Destroy_Args* a) {
  delete a->event;
  return nullptr;
}
PJRT_Error* Event_IsReady(PJRT_Event_IsReady_Args* a) {
  MI_NEED(a, PJRT_Event_IsReady_Args, is_ready);
  a->is_ready = a->event->done->Test();
  return nullptr;
}
PJRT_Error* Event_Error(PJRT_Event_Error_Args* a) {
  std::string e = a->event->done->error();
  return e.empty() ? nullptr : Fail(PJRT_Error_Code_INTERNAL, e);
}
PJRT_Error* Event_Await(PJRT_Event_Await_Args* a) {
  std::string e = a->event->done->Wait();
  return e.empty() ? nullptr : Fail(PJRT_Error_Code_INTERNAL, e);
}
PJRT_Error* Event_OnReady(PJRT_Event_OnReady_Args* a) {
  MI_NEED(a, PJRT_Event_OnReady_Args, user_arg);
  PJRT_Event_OnReadyCallback fn = a->callback;
  void* user = a->user_arg;
  a->event->done->Then([fn, user](const std::string& e) {
    fn(e.empty() ? nullptr : Fail(PJRT_Error_Code_INTERNAL, e), user);  // the callee owns the error
  });
  return nullptr;
}

// ------------------------------------------------------------------ client
PJRT_Error* Client_Create(PJRT_Client_Create_Args* a) {
  MI_NEED(a, PJRT_Client_Create_Args, client);
  const CreateOptions o = CreateOptions::Read(a->create_options, a->num_options);
  if (o.num_nodes > 1)
    return Fail(PJRT_Error_Code_UNIMPLEMENTED,
                "mi355x-pjrt drives the GPUs of one process: num_nodes = " + std::to_string(o.num_nodes) +
                    " needs a collective runtime, which this build leaves out");
  a->client = BuildClient(int(o.node_id > 0 ? o.node_id : 0));
  return nullptr;
}
PJRT_Error* Client_Destroy(PJRT_Client_Destroy_Args* a) {
  delete a->client;
  return nullptr;
}
PJRT_Error* Client_PlatformName(PJRT_Client_PlatformName_Args* a) {
  a->platform_name = kPlatformName;
  a->platform_name_size = sizeof(kPlatformName) - 1;
  return nullptr;
}
PJRT_Error* Client_PlatformVersion(PJRT_Client_PlatformVersion_Args* a) {
  a->platform_version = PlatformVersion().c_str();
  a->platform_version_size = PlatformVersion().size();
  return nullptr;
}
PJRT_Error* Client_ProcessIndex(PJRT_Client_ProcessIndex_Args* a) {
  a->process_index = a->client->process_index;
  return nullptr;
}
PJRT_Error* Client_Devices(PJRT_Client_Devices_Args* a) {
  a->devices = a->client->device_list.data();
  a->num_devices = a->client->device_list.size();
  return nullptr;
}
PJRT_Error* Client_AddressableDevices(PJRT_Client_AddressableDevices_Args* a) {
  // one process drives every GPU it sees: all devices are addressable
  a->addressable_devices = a->client->device_list.data();
  a->num_addressable_devices = a->client->device_list.size();
  return nullptr;
}
PJRT_Error* Client_AddressableMemories(PJRT_Client_AddressableMemories_Args* a) {
  a->addressable_memories = a->client->memory_list.data();
  a->num_addressable_memories = a->client->memory_list.size();
  return nullptr;
}
PJRT_Error* Client_LookupDevice(PJRT_Client_LookupDevice_Args* a) {
  PJRT_Client* c = a->client;
  if (a->id < 0 || size_t(a->id) >= c->gpus.size())
    return Fail(PJRT_Error_Code_INVALID_ARGUMENT, "LookupDevice: no device with id " + std::to_string(a->id));
  a->device = &c->gpus[size_t(a->id)];
  return nullptr;
}
PJRT_Error* Client_LookupAddressableDevice(PJRT_Client_LookupAddressableDevice_Args* a) {
  for (PJRT_Device& d : a->client->gpus)
    if (d.hip_ordinal == a->local_hardware_id) {
      a->addressable_device = &d;
      return nullptr;
    }
  return Fail(PJRT_Error_Code_INVALID_ARGUMENT,
              "LookupAddressableDevice: no device with local hardware id " + std::to_string(a->local_hardware_id));
}
PJRT_Error* Client_DefaultDeviceAssignment(PJRT_Client_DefaultDeviceAssignment_Args* a) {
  const size_t want = size_t(a->num_replicas) * size_t(a->num_partitions);
  if (want > a->default_assignment_size)
    return Fail(PJRT_Error_Code_INVALID_ARGUMENT, "DefaultDeviceAssignment: output array too small");
  const size_t n = a->client->gpus.size();
  // replica-major: replica r, partition p -> device (r * partitions + p) mod n
  for (size_t k = 0; k < want; ++k) a->default_assignment[k] = int(k % n);
  return nullptr;
}
PJRT_Error* Client_TopologyDescription(PJRT_Client_TopologyDescription_Args* a) {
  a->topology = &a->client->topology;
  return nullptr;
}

// ------------------------------------------------------------------ device descriptions
PJRT_Error* DeviceDescription_Id(PJRT_DeviceDescription_Id_Args* a) {
  a->id = a->device_description->global_id;
  return nullptr;
}
PJRT_Error* DeviceDescription_ProcessIndex(PJRT_DeviceDescription_ProcessIndex_Args* a) {
  a->process_index = a->device_description->process;
  return nullptr;
}
PJRT_Error* DeviceDescription_Attributes(PJRT_DeviceDescription_Attributes_Args* a) {
  a->attributes = a->device_description->attrs.data();
  a->num_attributes = a->device_description->attrs.size();
  return nullptr;
}
PJRT_Error* DeviceDescription_Kind(PJRT_DeviceDescription_Kind_Args* a) {
  a->device_kind = kDeviceKind;
  a->device_kind_size = sizeof(kDeviceKind) - 1;
  return nullptr;
}
PJRT_Error* DeviceDescription_DebugString(PJRT_DeviceDescription_DebugString_Args* a) {
  a->debug_string = a->device_description->detail.c_str();
  a->debug_string_size = a->device_description->detail.size();
  return nullptr;
}
PJRT_Error* DeviceDescription_ToString(PJRT_DeviceDescription_ToString_Args* a) {
  a->to_string = a->device_description->label.c_str();
  a->to_string_size = a->device_description->label.size();
  return nullptr;
}

// ------------------------------------------------------------------ devices
PJRT_Error* Device_GetDescription(PJRT_Device_GetDescription_Args* a) {
  a->device_description = &a->device->desc;
  return nullptr;
}
PJRT_Error* Device_IsAddressable(PJRT_Device_IsAddressable_Args* a) {
  a->is_addressable = true;
  return nullptr;
}
PJRT_Error* Device_LocalHardwareId(PJRT_Device_LocalHardwareId_Args* a) {
  a->local_hardware_id = a->device->hip_ordinal;
  return nullptr;
}
PJRT_Error* Device_AddressableMemories(PJRT_Device_AddressableMemories_Args* a) {
  a->memories = a->device->spaces;
  a->num_memories = 2;
  return nullptr;
}
PJRT_Error* Device_DefaultMemory(PJRT_Device_DefaultMemory_Args* a) {
  a->memory = &a->device->hbm;
  return nullptr;
}
PJRT_Error* Device_MemoryStats(PJRT_Device_MemoryStats_Args* a) {
  MI_NEED(a, PJRT_Device_MemoryStats_Args, peak_pool_bytes_is_set);
  std::string err;
  exec::DeviceContext* ctx = ContextOf(a->device, &err);
  if (!ctx) return Fail(PJRT_Error_Code_UNAVAILABLE, "MemoryStats: " + err);
  const exec::MemoryStats s = ctx->Stats();
  // clear every output, then report what the HBM pool tracks
  a->peak_bytes_reserved_is_set = a->bytes_reservable_limit_is_set = a->largest_free_block_bytes_is_set = false;
  a->peak_pool_bytes_is_set = false;
  a->bytes_in_use = s.bytes_in_use;
  a->peak_bytes_in_use = s.peak_bytes_in_use;
  a->num_allocs = s.num_allocs;
  a->largest_alloc_size = s.largest_alloc;
  a->bytes_limit = s.bytes_limit;
  a->bytes_reserved = s.bytes_reserved;
  a->pool_bytes = s.bytes_reserved;
  a->peak_bytes_in_use_is_set = a->num_allocs_is_set = a->largest_alloc_size_is_set = true;
  a->bytes_limit_is_set = a->bytes_reserved_is_set = a->pool_bytes_is_set = true;
  return nullptr;
}

// ------------------------------------------------------------------ memories
PJRT_Error* Memory_Id(PJRT_Memory_Id_Args* a) {
  a->id = a->memory->id;
  return nullptr;
}
PJRT_Error* Memory_Kind(PJRT_Memory_Kind_Args* a) {
  a->kind = a->memory->kind();
  a->kind_size = strlen(a->kind);
  return nullptr;
}
PJRT_Error* Memory_Kind_Id(PJRT_Memory_Kind_Id_Args* a) {
  a->kind_id = a->memory->kind_id();
  return nullptr;
}
PJRT_Error* Memory_DebugString(PJRT_Memory_DebugString_Args* a) {
  a->debug_string = a->memory->detail.c_str();
  a->debug_string_size = a->memory->detail.size();
  return nullptr;
}
PJRT_Error* Memory_ToString(PJRT_Memory_ToString_Args* a) {
  a->to_string = a->memory->label.c_str();
  a->to_string_size = a->memory->label.size();
  return nullptr;
}
PJRT_Error* Memory_AddressableByDevices(PJRT_Memory_AddressableByDevices_Args* a) {
  a->devices = a->memory->owner;
  a->num_devices = 1;
  return nullptr;
}

// ------------------------------------------------------------------ topology
PJRT_Error* TopologyDescription_Create(PJRT_TopologyDescription_Create_Args* a) {
  auto* t = new PJRT_TopologyDescription();
  std::vector<exec::GpuProps> gpus = VisibleGpus();
  if (gpus.empty()) gpus.emplace_back();
  for (size_t k = 0; k < gpus.size(); ++k) {
    PJRT_DeviceDescription& d = t->own.emplace_back();
    Describe(&d, int(k), 0, gpus[k]);
    t->list.push_back(&d);
  }
  a->topology = t;
  return nullptr;
}
PJRT_Error* TopologyDescription_Destroy(PJRT_TopologyDescription_Destroy_Args* a) {
  // a client's own topology is a member of the client, not a separate object
  if (!a->topology->own.empty()) delete a->topology;
  return nullptr;
}
PJRT_Error* TopologyDescription_PlatformName(PJRT_TopologyDescription_PlatformName_Args* a) {
  a->platform_name = kPlatformName;
  a->platform_name_size = sizeof(kPlatformName) - 1;
  return nullptr;
}
PJRT_Error* TopologyDescription_PlatformVersion(PJRT_TopologyDescription_PlatformVersion_Args* a) {
  a->platform_version = PlatformVersion().c_str();
  a->platform_version_size = PlatformVersion().size();
  return nullptr;
}
PJRT_Error* TopologyDescription_GetDeviceDescriptions(PJRT_TopologyDescription_GetDeviceDescriptions_Args* a) {
  a->descriptions = a->topology->list.data();
  a->num_descriptions = a->topology->list.size();
  return nullptr;
}
PJRT_Error* TopologyDescription_Attributes(PJRT_TopologyDescription_Attributes_Args* a) {
  a->attributes = a->topology->attrs.data();
  a->num_attributes = a->topology->attrs.size();
  return nullptr;
}

// ------------------------------------------------------------------ execute context
PJRT_Error* ExecuteContext_Create(PJRT_ExecuteContext_Create_Args* a) {
  a->context = new PJRT_ExecuteContext();
  return nullptr;
}
PJRT_Error* ExecuteContext_Destroy(PJRT_ExecuteContext_Destroy_Args* a) {
  delete a->context;
  return nullptr;
}

}  // namespace slot
}  // namespace mi::pjrt
