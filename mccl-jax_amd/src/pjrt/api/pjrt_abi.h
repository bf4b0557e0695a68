// ABI of the PJRT C API, version 0.55, as consumed by jaxlib.
//
// The layouts below must be byte-identical to the PJRT C API header of XLA
// commit 76da730179313b3bebad6dea6861768421b7358c (the version the reference
// pins, third_party/xla/pjrt/c/PROVENANCE.md:6-8): the member order and types
// of every argument struct, the enumerator values, and the order of the 100
// function slots of PJRT_Api.  Only the structs this plugin reads or writes
// are spelled out; the argument structs of functions it answers with
// UNIMPLEMENTED stay incomplete types.  Every argument struct starts with
// {size_t struct_size; PJRT_Extension_Base* extension_start;}.
#pragma once

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MI_PJRT_API_MAJOR 0
#define MI_PJRT_API_MINOR 55

typedef enum {
  PJRT_Extension_Type_Gpu_Custom_Call = 0,
  PJRT_Extension_Type_Profiler,
  PJRT_Extension_Type_Custom_Partitioner,
  PJRT_Extension_Type_Stream,
  PJRT_Extension_Type_Layouts,
  PJRT_Extension_Type_FFI,
} PJRT_Extension_Type;

typedef struct PJRT_Extension_Base {
  size_t struct_size;
  PJRT_Extension_Type type;
  struct PJRT_Extension_Base* next;
} PJRT_Extension_Base;

#define MI_ARGS_HEAD           \
  size_t struct_size;          \
  PJRT_Extension_Base* extension_start;
#define MI_ARGS(Name, ...) \
  typedef struct Name {    \
    MI_ARGS_HEAD           \
    __VA_ARGS__            \
  } Name;

typedef struct PJRT_Api_Version {
  MI_ARGS_HEAD
  int major_version;
  int minor_version;
} PJRT_Api_Version;

// ---- opaque handles (defined by the implementation)
typedef struct PJRT_Error PJRT_Error;
typedef struct PJRT_Event PJRT_Event;
typedef struct PJRT_Client PJRT_Client;
typedef struct PJRT_Device PJRT_Device;
typedef struct PJRT_Memory PJRT_Memory;
typedef struct PJRT_DeviceDescription PJRT_DeviceDescription;
typedef struct PJRT_TopologyDescription PJRT_TopologyDescription;
typedef struct PJRT_Executable PJRT_Executable;
typedef struct PJRT_LoadedExecutable PJRT_LoadedExecutable;
typedef struct PJRT_Buffer PJRT_Buffer;
typedef struct PJRT_ExecuteContext PJRT_ExecuteContext;
typedef struct PJRT_CopyToDeviceStream PJRT_CopyToDeviceStream;

// ---- enums (values fixed by the ABI)
typedef enum {
  PJRT_Error_Code_CANCELLED = 1,
  PJRT_Error_Code_UNKNOWN = 2,
  PJRT_Error_Code_INVALID_ARGUMENT = 3,
  PJRT_Error_Code_DEADLINE_EXCEEDED = 4,
  PJRT_Error_Code_NOT_FOUND = 5,
  PJRT_Error_Code_ALREADY_EXISTS = 6,
  PJRT_Error_Code_PERMISSION_DENIED = 7,
  PJRT_Error_Code_RESOURCE_EXHAUSTED = 8,
  PJRT_Error_Code_FAILED_PRECONDITION = 9,
  PJRT_Error_Code_ABORTED = 10,
  PJRT_Error_Code_OUT_OF_RANGE = 11,
  PJRT_Error_Code_UNIMPLEMENTED = 12,
  PJRT_Error_Code_INTERNAL = 13,
  PJRT_Error_Code_UNAVAILABLE = 14,
  PJRT_Error_Code_DATA_LOSS = 15,
  PJRT_Error_Code_UNAUTHENTICATED = 16
} PJRT_Error_Code;

typedef enum {
  PJRT_NamedValue_kString = 0,
  PJRT_NamedValue_kInt64,
  PJRT_NamedValue_kInt64List,
  PJRT_NamedValue_kFloat,
  PJRT_NamedValue_kBool,
} PJRT_NamedValue_Type;

typedef enum {
  PJRT_Buffer_Type_INVALID,
  PJRT_Buffer_Type_PRED,
  PJRT_Buffer_Type_S8,
  PJRT_Buffer_Type_S16,
  PJRT_Buffer_Type_S32,
  PJRT_Buffer_Type_S64,
  PJRT_Buffer_Type_U8,
  PJRT_Buffer_Type_U16,
  PJRT_Buffer_Type_U32,
  PJRT_Buffer_Type_U64,
  PJRT_Buffer_Type_F16,
  PJRT_Buffer_Type_F32,
  PJRT_Buffer_Type_F64,
  PJRT_Buffer_Type_BF16,
  PJRT_Buffer_Type_C64,
  PJRT_Buffer_Type_C128,
  PJRT_Buffer_Type_F8E5M2,
  PJRT_Buffer_Type_F8E4M3FN,
  PJRT_Buffer_Type_F8E4M3B11FNUZ,
  PJRT_Buffer_Type_F8E5M2FNUZ,
  PJRT_Buffer_Type_F8E4M3FNUZ,
  PJRT_Buffer_Type_S4,
  PJRT_Buffer_Type_U4,
  PJRT_Buffer_Type_TOKEN,
  PJRT_Buffer_Type_S2,
  PJRT_Buffer_Type_U2,
  PJRT_Buffer_Type_F8E4M3,
  PJRT_Buffer_Type_F8E3M4,
} PJRT_Buffer_Type;

typedef enum {
  PJRT_HostBufferSemantics_kImmutableOnlyDuringCall,
  PJRT_HostBufferSemantics_kImmutableUntilTransferCompletes,
  PJRT_HostBufferSemantics_kImmutableZeroCopy,
  PJRT_HostBufferSemantics_kMutableZeroCopy,
} PJRT_HostBufferSemantics;

typedef enum {
  PJRT_Buffer_MemoryLayout_Type_Tiled = 0,
  PJRT_Buffer_MemoryLayout_Type_Strides,
} PJRT_Buffer_MemoryLayout_Type;

// ---- value structs
typedef struct PJRT_NamedValue {
  MI_ARGS_HEAD
  const char* name;
  size_t name_size;
  PJRT_NamedValue_Type type;
  union {
    const char* string_value;
    int64_t int64_value;
    const int64_t* int64_array_value;
    float float_value;
    bool bool_value;
  };
  size_t value_size;
} PJRT_NamedValue;

typedef struct PJRT_Program {
  MI_ARGS_HEAD
  char* code;
  size_t code_size;
  const char* format;
  size_t format_size;
} PJRT_Program;

typedef struct PJRT_Buffer_MemoryLayout_Tiled {
  MI_ARGS_HEAD
  const int64_t* minor_to_major;
  size_t minor_to_major_size;
  const int64_t* tile_dims;
  const size_t* tile_dim_sizes;
  size_t num_tiles;
} PJRT_Buffer_MemoryLayout_Tiled;

typedef struct PJRT_Buffer_MemoryLayout_Strides {
  MI_ARGS_HEAD
  const int64_t* byte_strides;
  size_t num_byte_strides;
} PJRT_Buffer_MemoryLayout_Strides;

typedef struct PJRT_Buffer_MemoryLayout {
  MI_ARGS_HEAD
  union {
    PJRT_Buffer_MemoryLayout_Tiled tiled;
    PJRT_Buffer_MemoryLayout_Strides strides;
  };
  PJRT_Buffer_MemoryLayout_Type type;
} PJRT_Buffer_MemoryLayout;

typedef struct PJRT_ExecuteOptions {
  MI_ARGS_HEAD
  void** send_callbacks;
  void** recv_callbacks;
  size_t num_send_ops;
  size_t num_recv_ops;
  int launch_id;
  const int64_t* non_donatable_input_indices;
  size_t num_non_donatable_input_indices;
} PJRT_ExecuteOptions;

typedef void (*PJRT_Event_OnReadyCallback)(PJRT_Error* error, void* user_arg);

// ---- argument structs of the implemented functions
MI_ARGS(PJRT_Error_Destroy_Args, PJRT_Error* error;)
MI_ARGS(PJRT_Error_Message_Args, const PJRT_Error* error; const char* message; size_t message_size;)
MI_ARGS(PJRT_Error_GetCode_Args, const PJRT_Error* error; PJRT_Error_Code code;)
MI_ARGS(PJRT_Plugin_Initialize_Args, )
MI_ARGS(PJRT_Plugin_Attributes_Args, const PJRT_NamedValue* attributes; size_t num_attributes;)

MI_ARGS(PJRT_Event_Destroy_Args, PJRT_Event* event;)
MI_ARGS(PJRT_Event_IsReady_Args, PJRT_Event* event; bool is_ready;)
MI_ARGS(PJRT_Event_Error_Args, PJRT_Event* event;)
MI_ARGS(PJRT_Event_Await_Args, PJRT_Event* event;)
MI_ARGS(PJRT_Event_OnReady_Args, PJRT_Event* event; PJRT_Event_OnReadyCallback callback; void* user_arg;)

MI_ARGS(PJRT_Client_Create_Args, const PJRT_NamedValue* create_options; size_t num_options;
        void* kv_get_callback; void* kv_get_user_arg; void* kv_put_callback;
        void* kv_put_user_arg; PJRT_Client* client;)
MI_ARGS(PJRT_Client_Destroy_Args, PJRT_Client* client;)
MI_ARGS(PJRT_Client_PlatformName_Args, PJRT_Client* client; const char* platform_name; size_t platform_name_size;)
MI_ARGS(PJRT_Client_ProcessIndex_Args, PJRT_Client* client; int process_index;)
MI_ARGS(PJRT_Client_PlatformVersion_Args, PJRT_Client* client; const char* platform_version; size_t platform_version_size;)
MI_ARGS(PJRT_Client_TopologyDescription_Args, PJRT_Client* client; PJRT_TopologyDescription* topology;)
MI_ARGS(PJRT_Client_Devices_Args, PJRT_Client* client; PJRT_Device* const* devices; size_t num_devices;)
MI_ARGS(PJRT_Client_AddressableDevices_Args, PJRT_Client* client; PJRT_Device* const* addressable_devices; size_t num_addressable_devices;)
MI_ARGS(PJRT_Client_LookupDevice_Args, PJRT_Client* client; int id; PJRT_Device* device;)
MI_ARGS(PJRT_Client_LookupAddressableDevice_Args, PJRT_Client* client; int local_hardware_id; PJRT_Device* addressable_device;)
MI_ARGS(PJRT_Client_AddressableMemories_Args, PJRT_Client* client; PJRT_Memory* const* addressable_memories; size_t num_addressable_memories;)
MI_ARGS(PJRT_Client_Compile_Args, PJRT_Client* client; const PJRT_Program* program;
        const char* compile_options; size_t compile_options_size; PJRT_LoadedExecutable* executable;)
MI_ARGS(PJRT_Client_DefaultDeviceAssignment_Args, PJRT_Client* client; int num_replicas;
        int num_partitions; size_t default_assignment_size; int* default_assignment;)
MI_ARGS(PJRT_Client_BufferFromHostBuffer_Args, PJRT_Client* client; const void* data;
        PJRT_Buffer_Type type; const int64_t* dims; size_t num_dims; const int64_t* byte_strides;
        size_t num_byte_strides; PJRT_HostBufferSemantics host_buffer_semantics;
        PJRT_Device* device; PJRT_Memory* memory; PJRT_Buffer_MemoryLayout* device_layout;
        PJRT_Event* done_with_host_buffer; PJRT_Buffer* buffer;)

MI_ARGS(PJRT_DeviceDescription_Id_Args, PJRT_DeviceDescription* device_description; int id;)
MI_ARGS(PJRT_DeviceDescription_ProcessIndex_Args, PJRT_DeviceDescription* device_description; int process_index;)
MI_ARGS(PJRT_DeviceDescription_Attributes_Args, PJRT_DeviceDescription* device_description;
        size_t num_attributes; const PJRT_NamedValue* attributes;)
MI_ARGS(PJRT_DeviceDescription_Kind_Args, PJRT_DeviceDescription* device_description; const char* device_kind; size_t device_kind_size;)
MI_ARGS(PJRT_DeviceDescription_DebugString_Args, PJRT_DeviceDescription* device_description; const char* debug_string; size_t debug_string_size;)
MI_ARGS(PJRT_DeviceDescription_ToString_Args, PJRT_DeviceDescription* device_description; const char* to_string; size_t to_string_size;)

MI_ARGS(PJRT_Device_GetDescription_Args, PJRT_Device* device; PJRT_DeviceDescription* device_description;)
MI_ARGS(PJRT_Device_IsAddressable_Args, PJRT_Device* device; bool is_addressable;)
MI_ARGS(PJRT_Device_LocalHardwareId_Args, PJRT_Device* device; int local_hardware_id;)
MI_ARGS(PJRT_Device_AddressableMemories_Args, PJRT_Device* device; PJRT_Memory* const* memories; size_t num_memories;)
MI_ARGS(PJRT_Device_DefaultMemory_Args, PJRT_Device* device; PJRT_Memory* memory;)
MI_ARGS(PJRT_Device_MemoryStats_Args, PJRT_Device* device; int64_t bytes_in_use;
        int64_t peak_bytes_in_use; bool peak_bytes_in_use_is_set;
        int64_t num_allocs; bool num_allocs_is_set;
        int64_t largest_alloc_size; bool largest_alloc_size_is_set;
        int64_t bytes_limit; bool bytes_limit_is_set;
        int64_t bytes_reserved; bool bytes_reserved_is_set;
        int64_t peak_bytes_reserved; bool peak_bytes_reserved_is_set;
        int64_t bytes_reservable_limit; bool bytes_reservable_limit_is_set;
        int64_t largest_free_block_bytes; bool largest_free_block_bytes_is_set;
        int64_t pool_bytes; bool pool_bytes_is_set;
        int64_t peak_pool_bytes; bool peak_pool_bytes_is_set;)

MI_ARGS(PJRT_Memory_Id_Args, PJRT_Memory* memory; int id;)
MI_ARGS(PJRT_Memory_Kind_Args, PJRT_Memory* memory; const char* kind; size_t kind_size;)
MI_ARGS(PJRT_Memory_Kind_Id_Args, PJRT_Memory* memory; int kind_id;)
MI_ARGS(PJRT_Memory_DebugString_Args, PJRT_Memory* memory; const char* debug_string; size_t debug_string_size;)
MI_ARGS(PJRT_Memory_ToString_Args, PJRT_Memory* memory; const char* to_string; size_t to_string_size;)
MI_ARGS(PJRT_Memory_AddressableByDevices_Args, PJRT_Memory* memory; PJRT_Device* const* devices; size_t num_devices;)

MI_ARGS(PJRT_ExecuteContext_Create_Args, PJRT_ExecuteContext* context;)
MI_ARGS(PJRT_ExecuteContext_Destroy_Args, PJRT_ExecuteContext* context;)

MI_ARGS(PJRT_Executable_Destroy_Args, PJRT_Executable* executable;)
MI_ARGS(PJRT_LoadedExecutable_Destroy_Args, PJRT_LoadedExecutable* executable;)
MI_ARGS(PJRT_LoadedExecutable_GetExecutable_Args, PJRT_LoadedExecutable* loaded_executable; PJRT_Executable* executable;)
MI_ARGS(PJRT_Executable_Name_Args, PJRT_Executable* executable; const char* executable_name; size_t executable_name_size;)
MI_ARGS(PJRT_Executable_NumReplicas_Args, PJRT_Executable* executable; size_t num_replicas;)
MI_ARGS(PJRT_Executable_NumPartitions_Args, PJRT_Executable* executable; size_t num_partitions;)
MI_ARGS(PJRT_LoadedExecutable_AddressableDevices_Args, PJRT_LoadedExecutable* executable;
        PJRT_Device* const* addressable_devices; size_t num_addressable_devices;)
MI_ARGS(PJRT_LoadedExecutable_Delete_Args, PJRT_LoadedExecutable* executable;)
MI_ARGS(PJRT_LoadedExecutable_IsDeleted_Args, PJRT_LoadedExecutable* executable; bool is_deleted;)
MI_ARGS(PJRT_LoadedExecutable_Execute_Args, PJRT_LoadedExecutable* executable;
        PJRT_ExecuteOptions* options; PJRT_Buffer* const* const* argument_lists;
        size_t num_devices; size_t num_args; PJRT_Buffer** const* output_lists;
        PJRT_Event** device_complete_events; PJRT_Device* execute_device;)
MI_ARGS(PJRT_Executable_NumOutputs_Args, PJRT_Executable* executable; size_t num_outputs;)
MI_ARGS(PJRT_Executable_OptimizedProgram_Args, PJRT_Executable* executable; PJRT_Program* program;)
MI_ARGS(PJRT_Executable_SizeOfGeneratedCodeInBytes_Args, PJRT_Executable* executable; int64_t size_in_bytes;)
MI_ARGS(PJRT_Executable_Fingerprint_Args, PJRT_Executable* executable; const char* executable_fingerprint; size_t executable_fingerprint_size;)
MI_ARGS(PJRT_LoadedExecutable_Fingerprint_Args, PJRT_LoadedExecutable* executable; const char* executable_fingerprint; size_t executable_fingerprint_size;)
MI_ARGS(PJRT_Executable_GetCostAnalysis_Args, PJRT_Executable* executable; size_t num_properties; const PJRT_NamedValue* properties;)
MI_ARGS(PJRT_Executable_OutputElementTypes_Args, PJRT_Executable* executable; PJRT_Buffer_Type* output_types; size_t num_output_types;)
MI_ARGS(PJRT_Executable_OutputDimensions_Args, PJRT_Executable* executable; size_t num_outputs; const int64_t* dims; const size_t* dim_sizes;)
MI_ARGS(PJRT_Executable_OutputMemoryKinds_Args, PJRT_Executable* executable; size_t num_outputs;
        const char* const* memory_kinds; const size_t* memory_kind_sizes;)
MI_ARGS(PJRT_Executable_GetCompiledMemoryStats_Args, PJRT_Executable* executable;
        int64_t generated_code_size_in_bytes; int64_t argument_size_in_bytes;
        int64_t output_size_in_bytes; int64_t alias_size_in_bytes; int64_t temp_size_in_bytes;
        int64_t host_generated_code_size_in_bytes; int64_t host_argument_size_in_bytes;
        int64_t host_output_size_in_bytes; int64_t host_alias_size_in_bytes;
        int64_t host_temp_size_in_bytes;)

MI_ARGS(PJRT_Buffer_Destroy_Args, PJRT_Buffer* buffer;)
MI_ARGS(PJRT_Buffer_ElementType_Args, PJRT_Buffer* buffer; PJRT_Buffer_Type type;)
MI_ARGS(PJRT_Buffer_Dimensions_Args, PJRT_Buffer* buffer; const int64_t* dims; size_t num_dims;)
MI_ARGS(PJRT_Buffer_UnpaddedDimensions_Args, PJRT_Buffer* buffer; const int64_t* unpadded_dims; size_t num_dims;)
MI_ARGS(PJRT_Buffer_DynamicDimensionIndices_Args, PJRT_Buffer* buffer; const size_t* dynamic_dim_indices; size_t num_dynamic_dims;)
MI_ARGS(PJRT_Buffer_GetMemoryLayout_Args, PJRT_Buffer* buffer; PJRT_Buffer_MemoryLayout layout;)
MI_ARGS(PJRT_Buffer_ToHostBuffer_Args, PJRT_Buffer* src; PJRT_Buffer_MemoryLayout* host_layout;
        void* dst; size_t dst_size; PJRT_Event* event;)
MI_ARGS(PJRT_Buffer_OnDeviceSizeInBytes_Args, PJRT_Buffer* buffer; size_t on_device_size_in_bytes;)
MI_ARGS(PJRT_Buffer_Delete_Args, PJRT_Buffer* buffer;)
MI_ARGS(PJRT_Buffer_IsDeleted_Args, PJRT_Buffer* buffer; bool is_deleted;)
MI_ARGS(PJRT_Buffer_CopyToDevice_Args, PJRT_Buffer* buffer; PJRT_Device* dst_device; PJRT_Buffer* dst_buffer;)
MI_ARGS(PJRT_Buffer_CopyToMemory_Args, PJRT_Buffer* buffer; PJRT_Memory* dst_memory; PJRT_Buffer* dst_buffer;)
MI_ARGS(PJRT_Buffer_IsOnCpu_Args, PJRT_Buffer* buffer; bool is_on_cpu;)
MI_ARGS(PJRT_Buffer_Device_Args, PJRT_Buffer* buffer; PJRT_Device* device;)
MI_ARGS(PJRT_Buffer_Memory_Args, PJRT_Buffer* buffer; PJRT_Memory* memory;)
MI_ARGS(PJRT_Buffer_ReadyEvent_Args, PJRT_Buffer* buffer; PJRT_Event* event;)
MI_ARGS(PJRT_Buffer_UnsafePointer_Args, PJRT_Buffer* buffer; uintptr_t buffer_pointer;)
MI_ARGS(PJRT_Buffer_IncreaseExternalReferenceCount_Args, PJRT_Buffer* buffer;)
MI_ARGS(PJRT_Buffer_DecreaseExternalReferenceCount_Args, PJRT_Buffer* buffer;)
MI_ARGS(PJRT_Buffer_OpaqueDeviceMemoryDataPointer_Args, PJRT_Buffer* buffer; void* device_memory_ptr;)
MI_ARGS(PJRT_Client_CreateViewOfDeviceBuffer_Args, PJRT_Client* client; void* device_buffer_ptr;
        const int64_t* dims; size_t num_dims; PJRT_Buffer_Type element_type;
        PJRT_Buffer_MemoryLayout* layout; PJRT_Device* device;
        void (*on_delete_callback)(void* device_buffer_ptr, void* user_arg);
        void* on_delete_callback_arg; intptr_t stream; PJRT_Buffer* buffer;)

MI_ARGS(PJRT_TopologyDescription_Create_Args, const char* topology_name; size_t topology_name_size;
        const PJRT_NamedValue* create_options; size_t num_options; PJRT_TopologyDescription* topology;)
MI_ARGS(PJRT_TopologyDescription_Destroy_Args, PJRT_TopologyDescription* topology;)
MI_ARGS(PJRT_TopologyDescription_PlatformVersion_Args, PJRT_TopologyDescription* topology;
        const char* platform_version; size_t platform_version_size;)
MI_ARGS(PJRT_TopologyDescription_PlatformName_Args, PJRT_TopologyDescription* topology;
        const char* platform_name; size_t platform_name_size;)
MI_ARGS(PJRT_TopologyDescription_GetDeviceDescriptions_Args, PJRT_TopologyDescription* topology;
        PJRT_DeviceDescription* const* descriptions; size_t num_descriptions;)
MI_ARGS(PJRT_TopologyDescription_Attributes_Args, PJRT_TopologyDescription* topology;
        const PJRT_NamedValue* attributes; size_t num_attributes;)

typedef struct PJRT_SerializedExecutable PJRT_SerializedExecutable;
MI_ARGS(PJRT_Executable_Serialize_Args, const PJRT_Executable* executable;
        const char* serialized_bytes; size_t serialized_bytes_size;
        PJRT_SerializedExecutable* serialized_executable;
        void (*serialized_executable_deleter)(PJRT_SerializedExecutable* exec);)
MI_ARGS(PJRT_Executable_DeserializeAndLoad_Args, PJRT_Client* client; const char* serialized_executable;
        size_t serialized_executable_size; PJRT_LoadedExecutable* loaded_executable;)
MI_ARGS(PJRT_Compile_Args, const PJRT_TopologyDescription* topology; const PJRT_Program* program;
        const char* compile_options; size_t compile_options_size; PJRT_Client* client;
        PJRT_Executable* executable;)

// ---- argument structs of functions answered with UNIMPLEMENTED (layout unused)
typedef struct PJRT_CopyToDeviceStream_Destroy_Args PJRT_CopyToDeviceStream_Destroy_Args;
typedef struct PJRT_CopyToDeviceStream_AddChunk_Args PJRT_CopyToDeviceStream_AddChunk_Args;
typedef struct PJRT_CopyToDeviceStream_TotalBytes_Args PJRT_CopyToDeviceStream_TotalBytes_Args;
typedef struct PJRT_CopyToDeviceStream_GranuleSize_Args PJRT_CopyToDeviceStream_GranuleSize_Args;
typedef struct PJRT_CopyToDeviceStream_CurrentBytes_Args PJRT_CopyToDeviceStream_CurrentBytes_Args;
typedef struct PJRT_TopologyDescription_Serialize_Args PJRT_TopologyDescription_Serialize_Args;

// ---- the function table.  MI_PJRT_SLOTS lists the 100 slots in ABI order;
// V marks the two slots whose functions return void.
#define MI_PJRT_SLOTS(F, V)                                                                         \
  V(Error_Destroy) V(Error_Message) F(Error_GetCode) F(Plugin_Initialize) F(Plugin_Attributes)     \
  F(Event_Destroy) F(Event_IsReady) F(Event_Error) F(Event_Await) F(Event_OnReady)                 \
  F(Client_Create) F(Client_Destroy) F(Client_PlatformName) F(Client_ProcessIndex)                 \
  F(Client_PlatformVersion) F(Client_Devices) F(Client_AddressableDevices) F(Client_LookupDevice)  \
  F(Client_LookupAddressableDevice) F(Client_AddressableMemories) F(Client_Compile)                \
  F(Client_DefaultDeviceAssignment) F(Client_BufferFromHostBuffer)                                \
  F(DeviceDescription_Id) F(DeviceDescription_ProcessIndex) F(DeviceDescription_Attributes)        \
  F(DeviceDescription_Kind) F(DeviceDescription_DebugString) F(DeviceDescription_ToString)         \
  F(Device_GetDescription) F(Device_IsAddressable) F(Device_LocalHardwareId)                       \
  F(Device_AddressableMemories) F(Device_DefaultMemory) F(Device_MemoryStats)                      \
  F(Memory_Id) F(Memory_Kind) F(Memory_DebugString) F(Memory_ToString)                             \
  F(Memory_AddressableByDevices)                                                                   \
  F(Executable_Destroy) F(Executable_Name) F(Executable_NumReplicas) F(Executable_NumPartitions)   \
  F(Executable_NumOutputs) F(Executable_SizeOfGeneratedCodeInBytes) F(Executable_GetCostAnalysis)  \
  F(Executable_OutputMemoryKinds) F(Executable_OptimizedProgram) F(Executable_Serialize)           \
  F(LoadedExecutable_Destroy) F(LoadedExecutable_GetExecutable)                                    \
  F(LoadedExecutable_AddressableDevices) F(LoadedExecutable_Delete) F(LoadedExecutable_IsDeleted)  \
  F(LoadedExecutable_Execute) F(Executable_DeserializeAndLoad) F(LoadedExecutable_Fingerprint)     \
  F(Buffer_Destroy) F(Buffer_ElementType) F(Buffer_Dimensions) F(Buffer_UnpaddedDimensions)        \
  F(Buffer_DynamicDimensionIndices) F(Buffer_GetMemoryLayout) F(Buffer_OnDeviceSizeInBytes)        \
  F(Buffer_Device) F(Buffer_Memory) F(Buffer_Delete) F(Buffer_IsDeleted) F(Buffer_CopyToDevice)    \
  F(Buffer_ToHostBuffer) F(Buffer_IsOnCpu) F(Buffer_ReadyEvent) F(Buffer_UnsafePointer)            \
  F(Buffer_IncreaseExternalReferenceCount) F(Buffer_DecreaseExternalReferenceCount)                \
  F(Buffer_OpaqueDeviceMemoryDataPointer)                                                          \
  F(CopyToDeviceStream_Destroy) F(CopyToDeviceStream_AddChunk) F(CopyToDeviceStream_TotalBytes)    \
  F(CopyToDeviceStream_GranuleSize) F(CopyToDeviceStream_CurrentBytes)                             \
  F(TopologyDescription_Create) F(TopologyDescription_Destroy) F(TopologyDescription_PlatformName)  \
  F(TopologyDescription_PlatformVersion) F(TopologyDescription_GetDeviceDescriptions)              \
  F(TopologyDescription_Serialize) F(TopologyDescription_Attributes)                               \
  F(Compile) F(Executable_OutputElementTypes) F(Executable_OutputDimensions)                       \
  F(Buffer_CopyToMemory) F(Client_CreateViewOfDeviceBuffer) F(Executable_Fingerprint)              \
  F(Client_TopologyDescription) F(Executable_GetCompiledMemoryStats) F(Memory_Kind_Id)             \
  F(ExecuteContext_Create) F(ExecuteContext_Destroy)

#define MI_SLOT_FN(Name) PJRT_Error* (*PJRT_##Name)(struct PJRT_##Name##_Args*);
#define MI_SLOT_VOID(Name) void (*PJRT_##Name)(struct PJRT_##Name##_Args*);

struct PJRT_Api {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Api_Version pjrt_api_version;
  MI_PJRT_SLOTS(MI_SLOT_FN, MI_SLOT_VOID)
};
typedef struct PJRT_Api PJRT_Api;

#undef MI_SLOT_FN
#undef MI_SLOT_VOID

#ifdef __cplusplus
}  // extern "C"
#endif
