"""ctypes driver of libpjrt_mi355x.so through the PJRT C API (v0.55).

This is what jaxlib does when it loads the plugin, reduced to the calls a
test or a benchmark needs: create a client, upload numpy arrays, compile
StableHLO text, execute, read results back.  It mirrors the reference's C++
harness src/pjrt/pjrt_e2e.cc (load artifact -> BufferFromHostBuffer ->
Compile -> Execute -> ToHostBuffer, pjrt_e2e.cc:60-181) and adds bf16.

Every struct below mirrors the layout of the corresponding PJRT argument
struct: {size_t struct_size; void* extension_start; ...fields}.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

from . import PJRT_LIBRARY

_c = ctypes
_P = _c.c_void_p
_SZ = _c.c_size_t

# The 100 function slots of PJRT_Api, in ABI order.
SLOTS = """Error_Destroy Error_Message Error_GetCode Plugin_Initialize Plugin_Attributes
Event_Destroy Event_IsReady Event_Error Event_Await Event_OnReady
Client_Create Client_Destroy Client_PlatformName Client_ProcessIndex Client_PlatformVersion
Client_Devices Client_AddressableDevices Client_LookupDevice Client_LookupAddressableDevice
Client_AddressableMemories Client_Compile Client_DefaultDeviceAssignment Client_BufferFromHostBuffer
DeviceDescription_Id DeviceDescription_ProcessIndex DeviceDescription_Attributes DeviceDescription_Kind
DeviceDescription_DebugString DeviceDescription_ToString
Device_GetDescription Device_IsAddressable Device_LocalHardwareId Device_AddressableMemories
Device_DefaultMemory Device_MemoryStats
Memory_Id Memory_Kind Memory_DebugString Memory_ToString Memory_AddressableByDevices
Executable_Destroy Executable_Name Executable_NumReplicas Executable_NumPartitions Executable_NumOutputs
Executable_SizeOfGeneratedCodeInBytes Executable_GetCostAnalysis Executable_OutputMemoryKinds
Executable_OptimizedProgram Executable_Serialize
LoadedExecutable_Destroy LoadedExecutable_GetExecutable LoadedExecutable_AddressableDevices
LoadedExecutable_Delete LoadedExecutable_IsDeleted LoadedExecutable_Execute
Executable_DeserializeAndLoad LoadedExecutable_Fingerprint
Buffer_Destroy Buffer_ElementType Buffer_Dimensions Buffer_UnpaddedDimensions
Buffer_DynamicDimensionIndices Buffer_GetMemoryLayout Buffer_OnDeviceSizeInBytes Buffer_Device
Buffer_Memory Buffer_Delete Buffer_IsDeleted Buffer_CopyToDevice Buffer_ToHostBuffer Buffer_IsOnCpu
Buffer_ReadyEvent Buffer_UnsafePointer Buffer_IncreaseExternalReferenceCount
Buffer_DecreaseExternalReferenceCount Buffer_OpaqueDeviceMemoryDataPointer
CopyToDeviceStream_Destroy CopyToDeviceStream_AddChunk CopyToDeviceStream_TotalBytes
CopyToDeviceStream_GranuleSize CopyToDeviceStream_CurrentBytes
TopologyDescription_Create TopologyDescription_Destroy TopologyDescription_PlatformName
TopologyDescription_PlatformVersion TopologyDescription_GetDeviceDescriptions
TopologyDescription_Serialize TopologyDescription_Attributes
Compile Executable_OutputElementTypes Executable_OutputDimensions Buffer_CopyToMemory
Client_CreateViewOfDeviceBuffer Executable_Fingerprint Client_TopologyDescription
Executable_GetCompiledMemoryStats Memory_Kind_Id ExecuteContext_Create ExecuteContext_Destroy""".split()
assert len(SLOTS) == 100

# PJRT_Buffer_Type codes
PRED, S8, S16, S32, S64, U8, U16, U32, U64, F16, F32, F64, BF16 = range(1, 14)
_NP_TO_PJRT = {np.dtype(np.bool_): PRED, np.dtype(np.int8): S8, np.dtype(np.int16): S16,
               np.dtype(np.int32): S32, np.dtype(np.int64): S64, np.dtype(np.uint8): U8,
               np.dtype(np.uint16): U16, np.dtype(np.uint32): U32, np.dtype(np.uint64): U64,
               np.dtype(np.float16): F16, np.dtype(np.float32): F32, np.dtype(np.float64): F64}
_PJRT_TO_NP = {v: k for k, v in _NP_TO_PJRT.items()}
_PJRT_TO_NP[BF16] = np.dtype(np.uint16)  # bf16 travels as raw bits

ERROR_CODES = {1: "CANCELLED", 2: "UNKNOWN", 3: "INVALID_ARGUMENT", 4: "DEADLINE_EXCEEDED",
               5: "NOT_FOUND", 6: "ALREADY_EXISTS", 7: "PERMISSION_DENIED", 8: "RESOURCE_EXHAUSTED",
               9: "FAILED_PRECONDITION", 10: "ABORTED", 11: "OUT_OF_RANGE", 12: "UNIMPLEMENTED",
               13: "INTERNAL", 14: "UNAVAILABLE", 15: "DATA_LOSS", 16: "UNAUTHENTICATED"}


def _args(name, fields):
    return type(name, (_c.Structure,), {"_fields_": [("struct_size", _SZ), ("extension_start", _P)] + fields})


class NamedValue(_c.Structure):
    _fields_ = [("struct_size", _SZ), ("extension_start", _P), ("name", _c.c_char_p), ("name_size", _SZ),
                ("type", _c.c_int), ("value", _c.c_int64), ("value_size", _SZ)]


class ExecuteOptions(_c.Structure):
    _fields_ = [("struct_size", _SZ), ("extension_start", _P), ("send_callbacks", _P), ("recv_callbacks", _P),
                ("num_send_ops", _SZ), ("num_recv_ops", _SZ), ("launch_id", _c.c_int),
                ("non_donatable_input_indices", _P), ("num_non_donatable_input_indices", _SZ)]


class Program(_c.Structure):
    _fields_ = [("struct_size", _SZ), ("extension_start", _P), ("code", _P), ("code_size", _SZ),
                ("format", _c.c_char_p), ("format_size", _SZ)]


A = {
    "Error_Destroy": _args("ErrorDestroy", [("error", _P)]),
    "Error_Message": _args("ErrorMessage", [("error", _P), ("message", _P), ("message_size", _SZ)]),
    "Error_GetCode": _args("ErrorGetCode", [("error", _P), ("code", _c.c_int)]),
    "Plugin_Initialize": _args("PluginInitialize", []),
    "Event_Destroy": _args("EventDestroy", [("event", _P)]),
    "Event_Await": _args("EventAwait", [("event", _P)]),
    "Event_IsReady": _args("EventIsReady", [("event", _P), ("is_ready", _c.c_bool)]),
    "Client_Create": _args("ClientCreate", [("create_options", _P), ("num_options", _SZ),
                                             ("kv_get_callback", _P), ("kv_get_user_arg", _P),
                                             ("kv_put_callback", _P), ("kv_put_user_arg", _P),
                                             ("client", _P)]),
    "Client_Destroy": _args("ClientDestroy", [("client", _P)]),
    "Client_PlatformName": _args("ClientPlatformName", [("client", _P), ("platform_name", _P),
                                                        ("platform_name_size", _SZ)]),
    "Client_PlatformVersion": _args("ClientPlatformVersion", [("client", _P), ("platform_version", _P),
                                                              ("platform_version_size", _SZ)]),
    "Client_AddressableDevices": _args("ClientAddressableDevices", [("client", _P), ("devices", _P),
                                                                    ("num_devices", _SZ)]),
    "Client_Compile": _args("ClientCompile", [("client", _P), ("program", _c.POINTER(Program)),
                                              ("compile_options", _P), ("compile_options_size", _SZ),
                                              ("executable", _P)]),
    "Client_BufferFromHostBuffer": _args("ClientBufferFromHostBuffer", [
        ("client", _P), ("data", _P), ("type", _c.c_int), ("dims", _P), ("num_dims", _SZ),
        ("byte_strides", _P), ("num_byte_strides", _SZ), ("host_buffer_semantics", _c.c_int),
        ("device", _P), ("memory", _P), ("device_layout", _P), ("done_with_host_buffer", _P),
        ("buffer", _P)]),
    "Device_GetDescription": _args("DeviceGetDescription", [("device", _P), ("device_description", _P)]),
    "DeviceDescription_Kind": _args("DescKind", [("device_description", _P), ("device_kind", _P),
                                                 ("device_kind_size", _SZ)]),
    "Buffer_Destroy": _args("BufferDestroy", [("buffer", _P)]),
    "Buffer_Delete": _args("BufferDelete", [("buffer", _P)]),
    "Buffer_ElementType": _args("BufferElementType", [("buffer", _P), ("type", _c.c_int)]),
    "Buffer_Dimensions": _args("BufferDimensions", [("buffer", _P), ("dims", _P), ("num_dims", _SZ)]),
    "Buffer_ToHostBuffer": _args("BufferToHostBuffer", [("src", _P), ("host_layout", _P), ("dst", _P),
                                                        ("dst_size", _SZ), ("event", _P)]),
    "Buffer_ReadyEvent": _args("BufferReadyEvent", [("buffer", _P), ("event", _P)]),
    "Buffer_IsDeleted": _args("BufferIsDeleted", [("buffer", _P), ("is_deleted", _c.c_bool)]),
    "Buffer_UnsafePointer": _args("BufferUnsafePointer", [("buffer", _P), ("buffer_pointer", _c.c_size_t)]),
    "LoadedExecutable_Destroy": _args("LoadedDestroy", [("executable", _P)]),
    "LoadedExecutable_Delete": _args("LoadedDelete", [("executable", _P)]),
    "LoadedExecutable_GetExecutable": _args("LoadedGetExecutable", [("loaded_executable", _P),
                                                                    ("executable", _P)]),
    "LoadedExecutable_Execute": _args("LoadedExecute", [
        ("executable", _P), ("options", _P), ("argument_lists", _P), ("num_devices", _SZ),
        ("num_args", _SZ), ("output_lists", _P), ("device_complete_events", _P),
        ("execute_device", _P)]),
    "Executable_Destroy": _args("ExecutableDestroy", [("executable", _P)]),
    "Executable_NumOutputs": _args("ExecutableNumOutputs", [("executable", _P), ("num_outputs", _SZ)]),
    "Executable_OptimizedProgram": _args("ExecutableOptimizedProgram", [("executable", _P),
                                                                        ("program", _c.POINTER(Program))]),
    "Executable_OutputElementTypes": _args("ExecutableOutputElementTypes", [
        ("executable", _P), ("output_types", _P), ("num_output_types", _SZ)]),
    "Executable_OutputDimensions": _args("ExecutableOutputDimensions", [
        ("executable", _P), ("num_outputs", _SZ), ("dims", _P), ("dim_sizes", _P)]),
    "Plugin_Attributes": _args("PluginAttributes", [("attributes", _P), ("num_attributes", _SZ)]),
    "DeviceDescription_Attributes": _args("DescAttributes", [("device_description", _P),
                                                             ("num_attributes", _SZ), ("attributes", _P)]),
    "DeviceDescription_ToString": _args("DescToString", [("device_description", _P), ("to_string", _P),
                                                         ("to_string_size", _SZ)]),
    "Executable_Serialize": _args("ExecutableSerialize", [
        ("executable", _P), ("serialized_bytes", _P), ("serialized_bytes_size", _SZ),
        ("serialized_executable", _P), ("serialized_executable_deleter", _c.CFUNCTYPE(None, _P))]),
    "Executable_DeserializeAndLoad": _args("ExecutableDeserializeAndLoad", [
        ("client", _P), ("serialized_executable", _P), ("serialized_executable_size", _SZ),
        ("loaded_executable", _P)]),
    "Event_OnReady": _args("EventOnReady", [("event", _P), ("callback", _P), ("user_arg", _P)]),
}


def named_values(ptr, n) -> dict:
    """Decode a PJRT_NamedValue array into {name: value}."""
    out = {}
    for i in range(n):
        v = NamedValue.from_address(ptr + i * _c.sizeof(NamedValue))
        name = _c.string_at(v.name, v.name_size).decode()
        if v.type == 0:  # kString
            out[name] = _c.string_at(v.value, v.value_size).decode()
        elif v.type == 1:  # kInt64
            out[name] = int(v.value)
        elif v.type == 2:  # kInt64List
            out[name] = list((_c.c_int64 * v.value_size).from_address(v.value)) if v.value_size else []
        elif v.type == 4:  # kBool
            out[name] = bool(v.value & 0xFF)
        else:
            out[name] = v.value
    return out


class PjrtError(RuntimeError):
    def __init__(self, code, message):
        super().__init__(f"{ERROR_CODES.get(code, code)}: {message}")
        self.code = ERROR_CODES.get(code, code)
        self.message = message


class Plugin:
    """dlopen the plugin and resolve its PJRT_Api table."""

    def __init__(self, path: str = PJRT_LIBRARY):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built; run __graft_entry__.build()")
        self.lib = _c.CDLL(path)
        self.lib.GetPjrtApi.restype = _P
        self.api = self.lib.GetPjrtApi()
        if not self.api:
            raise RuntimeError("GetPjrtApi returned NULL")
        hdr = (_c.c_size_t * 2).from_address(self.api)
        self.struct_size = hdr[0]
        ver = (_c.c_int * 2).from_address(self.api + 16 + 16)
        self.version = (ver[0], ver[1])
        self._fns = {}
        self.call("Plugin_Initialize")

    def slot(self, name: str) -> int:
        """raw function pointer of a slot (0 when the slot is empty)."""
        return _c.c_void_p.from_address(self.api + 40 + 8 * SLOTS.index(name)).value or 0

    def _fn(self, name):
        f = self._fns.get(name)
        if f is None:
            ptr = self.slot(name)
            restype = None if name in ("Error_Destroy", "Error_Message") else _P
            f = _c.CFUNCTYPE(restype, _P)(ptr)
            self._fns[name] = f
        return f

    def call(self, name, **kw):
        a = A[name]()
        a.struct_size = _c.sizeof(a)
        for k, v in kw.items():
            setattr(a, k, v)
        err = self._fn(name)(_c.addressof(a))
        if err:
            raise self._error(err)
        return a

    def _error(self, err) -> PjrtError:
        m = A["Error_Message"]()
        m.struct_size = _c.sizeof(m)
        m.error = err
        self._fn("Error_Message")(_c.addressof(m))
        msg = _c.string_at(m.message, m.message_size).decode()
        g = A["Error_GetCode"]()
        g.struct_size = _c.sizeof(g)
        g.error = err
        self._fn("Error_GetCode")(_c.addressof(g))
        code = g.code
        d = A["Error_Destroy"]()
        d.struct_size = _c.sizeof(d)
        d.error = err
        self._fn("Error_Destroy")(_c.addressof(d))
        return PjrtError(code, msg)

    def event_ready(self, ev) -> bool:
        return bool(self.call("Event_IsReady", event=ev).is_ready)

    def on_ready(self, ev, fn):
        """Register fn(error_or_None) with PJRT_Event_OnReady; returns the
        ctypes callback, which the caller keeps alive until it has fired."""
        proto = _c.CFUNCTYPE(None, _P, _P)

        def trampoline(err, _user):
            fn(self._error(err) if err else None)

        cb = proto(trampoline)
        self.call("Event_OnReady", event=ev, callback=_c.cast(cb, _P), user_arg=None)
        return cb

    def await_event(self, ev):
        if not ev:
            return
        try:
            self.call("Event_Await", event=ev)
        finally:
            self.call("Event_Destroy", event=ev)

    def attributes(self) -> dict:
        a = self.call("Plugin_Attributes")
        return named_values(a.attributes, a.num_attributes)

    def client(self, options: dict | None = None) -> "Client":
        opts = options or {}
        arr = (NamedValue * max(len(opts), 1))()
        keep = []
        for i, (k, v) in enumerate(opts.items()):
            kb = k.encode()
            keep.append(kb)
            arr[i].struct_size = _c.sizeof(NamedValue)
            arr[i].name = kb
            arr[i].name_size = len(kb)
            arr[i].type = 1  # kInt64
            arr[i].value = int(v)
            arr[i].value_size = 1
        a = self.call("Client_Create", create_options=_c.addressof(arr) if opts else None, num_options=len(opts))
        return Client(self, a.client)


class Client:
    def __init__(self, plugin: Plugin, handle):
        self.p = plugin
        self.h = handle

    def close(self):
        if self.h:
            self.p.call("Client_Destroy", client=self.h)
            self.h = None

    def _str(self, slot, field):
        a = self.p.call(slot, client=self.h)
        return _c.string_at(getattr(a, field), getattr(a, field + "_size")).decode()

    @property
    def platform_name(self) -> str:
        return self._str("Client_PlatformName", "platform_name")

    @property
    def platform_version(self) -> str:
        return self._str("Client_PlatformVersion", "platform_version")

    def devices(self):
        a = self.p.call("Client_AddressableDevices", client=self.h)
        return [_c.c_void_p.from_address(a.devices + 8 * i).value for i in range(a.num_devices)]

    def device_kind(self, dev) -> str:
        d = self.p.call("Device_GetDescription", device=dev)
        k = self.p.call("DeviceDescription_Kind", device_description=d.device_description)
        return _c.string_at(k.device_kind, k.device_kind_size).decode()

    def device_attributes(self, dev) -> dict:
        d = self.p.call("Device_GetDescription", device=dev)
        a = self.p.call("DeviceDescription_Attributes", device_description=d.device_description)
        return named_values(a.attributes, a.num_attributes)

    def device_string(self, dev) -> str:
        d = self.p.call("Device_GetDescription", device=dev)
        t = self.p.call("DeviceDescription_ToString", device_description=d.device_description)
        return _c.string_at(t.to_string, t.to_string_size).decode()

    def deserialize(self, blob: bytes) -> "Executable":
        """PJRT_Executable_DeserializeAndLoad of bytes from Executable.serialize()."""
        buf = _c.create_string_buffer(blob, len(blob))
        a = self.p.call("Executable_DeserializeAndLoad", client=self.h, serialized_executable=_c.addressof(buf),
                        serialized_executable_size=len(blob))
        return Executable(self, a.loaded_executable)

    def compile(self, text: str | bytes) -> "Executable":
        code = text.encode() if isinstance(text, str) else bytes(text)
        buf = _c.create_string_buffer(code, len(code))
        prog = Program()
        prog.struct_size = _c.sizeof(Program)
        prog.code = _c.addressof(buf)
        prog.code_size = len(code)
        prog.format = b"mlir"
        prog.format_size = 4
        a = self.p.call("Client_Compile", client=self.h, program=_c.pointer(prog))
        return Executable(self, a.executable)

    def put(self, array: np.ndarray, dtype_code: int | None = None) -> "Buffer":
        """Upload a numpy array (bf16: pass uint16 bits and dtype_code=BF16)."""
        arr = np.ascontiguousarray(array)
        code = dtype_code if dtype_code is not None else _NP_TO_PJRT[arr.dtype]
        dims = (_c.c_int64 * max(arr.ndim, 1))(*arr.shape)
        a = self.p.call("Client_BufferFromHostBuffer", client=self.h, data=arr.ctypes.data, type=code,
                        dims=_c.addressof(dims), num_dims=arr.ndim, byte_strides=None, num_byte_strides=0,
                        host_buffer_semantics=0, device=None, memory=None, device_layout=None)
        self.p.await_event(a.done_with_host_buffer)
        return Buffer(self, a.buffer)


class Buffer:
    def __init__(self, client: Client, handle):
        self.c = client
        self.h = handle

    @property
    def type(self) -> int:
        return self.c.p.call("Buffer_ElementType", buffer=self.h).type

    @property
    def shape(self):
        a = self.c.p.call("Buffer_Dimensions", buffer=self.h)
        return tuple((_c.c_int64 * a.num_dims).from_address(a.dims)) if a.num_dims else ()

    def ready(self):
        a = self.c.p.call("Buffer_ReadyEvent", buffer=self.h)
        self.c.p.await_event(a.event)

    def to_numpy_async(self):
        """Start PJRT_Buffer_ToHostBuffer; returns (array, event).  The array
        holds the data once the event is ready."""
        dt = _PJRT_TO_NP[self.type]
        out = np.empty(self.shape, dtype=dt)
        a = self.c.p.call("Buffer_ToHostBuffer", src=self.h, host_layout=None, dst=out.ctypes.data,
                          dst_size=out.nbytes)
        return out, a.event

    def to_numpy(self) -> np.ndarray:
        out, ev = self.to_numpy_async()
        self.c.p.await_event(ev)
        return out

    def ready_event(self):
        return self.c.p.call("Buffer_ReadyEvent", buffer=self.h).event

    def delete(self):
        self.c.p.call("Buffer_Delete", buffer=self.h)

    @property
    def is_deleted(self) -> bool:
        return bool(self.c.p.call("Buffer_IsDeleted", buffer=self.h).is_deleted)

    @property
    def device_pointer(self) -> int:
        return int(self.c.p.call("Buffer_UnsafePointer", buffer=self.h).buffer_pointer)

    def destroy(self):
        if self.h:
            self.c.p.call("Buffer_Destroy", buffer=self.h)
            self.h = None


class Executable:
    def __init__(self, client: Client, handle):
        self.c = client
        self.h = handle
        e = client.p.call("LoadedExecutable_GetExecutable", loaded_executable=handle)
        self.e = e.executable

    @property
    def num_outputs(self) -> int:
        return self.c.p.call("Executable_NumOutputs", executable=self.e).num_outputs

    def output_types(self):
        a = self.c.p.call("Executable_OutputElementTypes", executable=self.e)
        return list((_c.c_int * a.num_output_types).from_address(a.output_types)) if a.num_output_types else []

    def output_shapes(self):
        a = self.c.p.call("Executable_OutputDimensions", executable=self.e)
        sizes = list((_c.c_size_t * a.num_outputs).from_address(a.dim_sizes)) if a.num_outputs else []
        total = sum(sizes)
        flat = list((_c.c_int64 * total).from_address(a.dims)) if total else []
        out, k = [], 0
        for s in sizes:
            out.append(tuple(flat[k:k + s]))
            k += s
        return out

    def plan(self) -> str:
        """The compiled launch plan (PJRT_Executable_OptimizedProgram, format jam-plan)."""
        prog = Program()
        prog.struct_size = _c.sizeof(Program)
        prog.code = None
        self.c.p.call("Executable_OptimizedProgram", executable=self.e, program=_c.pointer(prog))
        buf = _c.create_string_buffer(prog.code_size)
        prog.code = _c.addressof(buf)
        self.c.p.call("Executable_OptimizedProgram", executable=self.e, program=_c.pointer(prog))
        return buf.raw[:prog.code_size].decode()

    def execute(self, args, wait=True, non_donatable=None):
        """Run on one device; inputs the program aliases to outputs are
        donated unless listed in non_donatable.  wait=True awaits the
        completion event, False drops it, "event" returns (outputs, event)."""
        n = self.num_outputs
        opts = None
        if non_donatable is not None:
            idx = (_c.c_int64 * max(len(non_donatable), 1))(*non_donatable)
            o = ExecuteOptions()
            o.struct_size = _c.sizeof(ExecuteOptions)
            o.non_donatable_input_indices = _c.addressof(idx)
            o.num_non_donatable_input_indices = len(non_donatable)
            opts = _c.addressof(o)
        arg_arr = (_c.c_void_p * max(len(args), 1))(*[b.h for b in args])
        arg_lists = (_c.c_void_p * 1)(_c.addressof(arg_arr))
        out_arr = (_c.c_void_p * max(n, 1))()
        out_lists = (_c.c_void_p * 1)(_c.addressof(out_arr))
        events = (_c.c_void_p * 1)()
        self.c.p.call("LoadedExecutable_Execute", executable=self.h, options=opts,
                      argument_lists=_c.addressof(arg_lists), num_devices=1, num_args=len(args),
                      output_lists=_c.addressof(out_lists), device_complete_events=_c.addressof(events),
                      execute_device=None)
        outs = [Buffer(self.c, out_arr[i]) for i in range(n)]
        if wait == "event":
            return outs, events[0]
        if wait:
            self.c.p.await_event(events[0])
        else:
            self.c.p.call("Event_Destroy", event=events[0])
        return outs

    def serialize(self) -> bytes:
        a = self.c.p.call("Executable_Serialize", executable=self.e)
        blob = _c.string_at(a.serialized_bytes, a.serialized_bytes_size)
        a.serialized_executable_deleter(a.serialized_executable)
        return blob

    def delete(self):
        self.c.p.call("LoadedExecutable_Delete", executable=self.h)

    def destroy(self):
        if self.e:
            self.c.p.call("Executable_Destroy", executable=self.e)
            self.e = None
        if self.h:
            self.c.p.call("LoadedExecutable_Destroy", executable=self.h)
            self.h = None
