// Buffer slots: host transfers, device copies, views and buffer queries.
//
// Reference counterparts: pjrt_c_api.cc:453-627 (BufferFromHostBuffer,
// ToHostBuffer, CopyToDevice/CopyToMemory, Delete/Destroy, external
// references).  There every transfer is a synchronous memcpy into unified
// memory; here:
//  * uploads are staged through pinned memory and DMA'd on the device's
//    transfer stream, so they never wait for queued kernels; the buffer's
//    `defined` completion is that DMA, and whoever reads the buffer on the
//    compute stream first makes the stream wait for it (no host wait);
//  * downloads are DMA'd on the compute stream (after the kernels that
//    produce the data) into pinned staging, and the watcher thread copies
//    them to the caller's memory, after which the event completes;
//  * strided host arrays are gathered into row-major order; device layouts
//    other than dense row-major are refused with a named error.
#include <cstring>

#include "pjrt/api/plugin.h"

namespace mi::pjrt {
namespace {

std::vector<int64_t> RowMajor(size_t rank) {
  std::vector<int64_t> m(rank);
  for (size_t i = 0; i < rank; ++i) m[i] = int64_t(rank - 1 - i);
  return m;
}

// true if `layout` (may be null) describes dense row-major storage
bool IsRowMajor(const PJRT_Buffer_MemoryLayout* layout, const int64_t* dims, size_t rank, size_t width) {
  if (!layout) return true;
  if (layout->type == PJRT_Buffer_MemoryLayout_Type_Tiled) {
    const auto& t = layout->tiled;
    if (t.num_tiles != 0 || t.minor_to_major_size != rank) return false;
    for (size_t i = 0; i < rank; ++i)
      if (t.minor_to_major[i] != int64_t(rank - 1 - i)) return false;
    return true;
  }
  const auto& s = layout->strides;
  if (s.num_byte_strides != rank) return false;
  int64_t want = int64_t(width);
  for (size_t i = rank; i-- > 0;) {
    if (dims[i] != 1 && s.byte_strides[i] != want) return false;
    want *= dims[i];
  }
  return true;
}

// Gathers a host array with byte strides into row-major order; returns
// nullptr (and leaves `out` empty) when it is already dense.
const char* PackStrided(const char* src, const int64_t* dims, const int64_t* strides, size_t rank, size_t width,
                        size_t count, std::vector<char>* out) {
  int64_t want = int64_t(width);
  bool dense = true;
  for (size_t i = rank; i-- > 0;) {
    if (dims[i] != 1 && strides[i] != want) dense = false;
    want *= dims[i];
  }
  if (dense || count == 0) return nullptr;
  out->resize(count * width);
  std::vector<int64_t> at(rank, 0);
  int64_t off = 0;
  for (size_t e = 0; e < count; ++e) {
    memcpy(out->data() + e * width, src + off, width);
    for (size_t i = rank; i-- > 0;) {  // odometer over the index, innermost first
      off += strides[i];
      if (++at[i] < dims[i]) break;
      off -= strides[i] * dims[i];
      at[i] = 0;
    }
  }
  return out->data();
}

std::shared_ptr<Block> NewBlock(PJRT_Memory* mem, size_t bytes, std::string* error) {
  auto b = std::make_shared<Block>();
  b->bytes = bytes;
  b->where = mem->space;
  if (mem->space == Placement::kPinnedHost) {
    if (bytes && hipHostMalloc(&b->ptr, bytes, hipHostMallocDefault) != hipSuccess) {
      (void)hipGetLastError();
      b->ptr = nullptr;
      *error = "hipHostMalloc of " + std::to_string(bytes) + " bytes failed";
      return nullptr;
    }
    return b;
  }
  b->ctx = ContextOf(mem->owner[0], error);
  if (!b->ctx) return nullptr;
  if (bytes) {
    b->ptr = b->ctx->Alloc(bytes, error);
    if (!b->ptr) return nullptr;
  }
  return b;
}

PJRT_Buffer* Wrap(PJRT_Device* dev, PJRT_Memory* mem, PJRT_Buffer_Type type, std::vector<int64_t> dims,
                  std::shared_ptr<Block> block, std::shared_ptr<Completion> defined) {
  auto* b = new PJRT_Buffer();
  b->client = dev->client;
  b->device = dev;
  b->memory = mem;
  b->type = type;
  b->minor_to_major = RowMajor(dims.size());
  b->dims = std::move(dims);
  b->bytes = block->bytes;
  b->block = std::move(block);
  b->defined = std::move(defined);
  return b;
}

std::shared_ptr<Completion> RecordOn(exec::DeviceContext* ctx, hipStream_t s, Lane lane,
                                     std::function<std::string()> host_step, std::string* error) {
  hipEvent_t ev = nullptr;
  hipError_t r = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
  if (r == hipSuccess) r = hipEventRecord(ev, s);
  if (r != hipSuccess) {
    if (ev) (void)hipEventDestroy(ev);
    *error = std::string("hipEventRecord: ") + hipGetErrorString(r);
    return nullptr;
  }
  return Completion::AfterGpu(ctx->ordinal(), lane, ev, std::move(host_step));
}

// Copies a buffer into a fresh block in `mem`.
PJRT_Error* CopyInto(PJRT_Buffer* src, PJRT_Memory* mem, PJRT_Buffer** out, const char* what) {
  if (!src->usable()) return Fail(PJRT_Error_Code_INVALID_ARGUMENT, std::string(what) + ": buffer was deleted");
  std::string err;
  std::shared_ptr<Block> dst = NewBlock(mem, src->bytes, &err);
  if (!dst) return Fail(PJRT_Error_Code_RESOURCE_EXHAUSTED, std::string(what) + ": " + err);
  std::shared_ptr<Block> from = src->block;
  std::shared_ptr<Completion> defined;
  const bool src_host = from->where == Placement::kPinnedHost;
  const bool dst_host = dst->where == Placement::kPinnedHost;
  if (src->bytes == 0) {
    // nothing to move
  } else if (src_host && dst_host) {
    if (src->defined) err = src->defined->Wait();
    if (err.empty()) memcpy(dst->ptr, from->ptr, src->bytes);
  } else if (src_host) {
    // pinned host -> HBM: DMA on the destination's transfer stream; the
    // source block is held until the DMA is done
    if (src->defined) err = src->defined->Wait();
    exec::DeviceContext* ctx = dst->ctx;
    if (err.empty() && exec::UseDevice(ctx->ordinal(), &err) && ctx->OrderUploadInto(dst->ptr, &err)) {
      hipError_t r = hipMemcpyAsync(dst->ptr, from->ptr, src->bytes, hipMemcpyHostToDevice, ctx->transfer_stream());
      if (r != hipSuccess) err = std::string("hipMemcpyAsync: ") + hipGetErrorString(r);
      else defined = RecordOn(ctx, ctx->transfer_stream(), Lane::kTransfer, [from] { return std::string(); }, &err);
      dst->pending_write = defined;
      Watch(defined);  // drops the hold on the source once the DMA is done
    }
  } else {
    // HBM source: ordered on its device's compute stream
    exec::DeviceContext* ctx = from->ctx;
    if (exec::UseDevice(ctx->ordinal(), &err) && OrderComputeAfter(src->defined, ctx, &err)) {
      hipError_t r = hipMemcpyAsync(dst->ptr, from->ptr, src->bytes, hipMemcpyDefault, ctx->stream());
      if (r != hipSuccess) err = std::string("hipMemcpyAsync: ") + hipGetErrorString(r);
      else defined = RecordOn(ctx, ctx->stream(), Lane::kCompute, {}, &err);
      if (dst_host) dst->pending_write = defined;
      // another GPU's compute stream is not ordered by this one: settle here
      if (defined && !dst_host && dst->ctx != ctx) {
        err = defined->Wait();
        defined = nullptr;
      }
    }
  }
  if (!err.empty()) return Fail(PJRT_Error_Code_INTERNAL, std::string(what) + ": " + err);
  PJRT_Device* dev = mem->owner[0];
  *out = Wrap(dev, mem, src->type, src->dims, std::move(dst), std::move(defined));
  return nullptr;
}

}  // namespace

namespace slot {

PJRT_Error* Client_BufferFromHostBuffer(PJRT_Client_BufferFromHostBuffer_Args* a) {
  MI_NEED(a, PJRT_Client_BufferFromHostBuffer_Args, buffer);
  const size_t width = ElementBytes(a->type);
  if (width == 0)
    return Fail(PJRT_Error_Code_UNIMPLEMENTED,
                "BufferFromHostBuffer: element type " + std::to_string(int(a->type)) + " is not carried");
  size_t count = 1;
  for (size_t i = 0; i < a->num_dims; ++i) {
    if (a->dims[i] < 0) return Fail(PJRT_Error_Code_INVALID_ARGUMENT, "BufferFromHostBuffer: negative dimension");
    count *= size_t(a->dims[i]);
  }
  if (!IsRowMajor(a->device_layout, a->dims, a->num_dims, width))
    return Fail(PJRT_Error_Code_UNIMPLEMENTED,
                "BufferFromHostBuffer: only dense row-major device layouts are supported");
  // placement: an explicit memory wins; else the device's HBM; else device 0
  PJRT_Memory* mem = a->memory;
  PJRT_Device* dev = mem ? mem->owner[0] : a->device;
  if (!dev) dev = a->client->device_list.front();
  if (!mem) mem = &dev->hbm;
  if (a->device && a->device != dev)
    return Fail(PJRT_Error_Code_INVALID_ARGUMENT, "BufferFromHostBuffer: memory does not belong to device");

  std::vector<char> packed;
  const char* src = static_cast<const char*>(a->data);
  if (a->byte_strides && a->num_byte_strides == a->num_dims)
    if (const char* p = PackStrided(src, a->dims, a->byte_strides, a->num_dims, width, count, &packed)) src = p;

  std::string err;
  const size_t bytes = count * width;
  std::shared_ptr<Block> block = NewBlock(mem, bytes, &err);
  if (!block) return Fail(PJRT_Error_Code_RESOURCE_EXHAUSTED, "BufferFromHostBuffer: " + err);
  std::shared_ptr<Completion> defined;
  if (bytes && block->where == Placement::kPinnedHost) {
    memcpy(block->ptr, src, bytes);
  } else if (bytes) {
    hipEvent_t ev = block->ctx->Upload(block->ptr, src, bytes, &err);
    if (!ev) return Fail(PJRT_Error_Code_INTERNAL, "BufferFromHostBuffer: " + err);
    defined = Completion::AfterGpu(block->ctx->ordinal(), Lane::kTransfer, ev);
    block->pending_write = defined;
  }
  a->buffer = Wrap(dev, mem, a->type, std::vector<int64_t>(a->dims, a->dims + a->num_dims), std::move(block),
                   std::move(defined));
  // every byte was read into pinned staging before returning
  a->done_with_host_buffer = new PJRT_Event{Completion::Done()};
  return nullptr;
}

PJRT_Error* Buffer_ToHostBuffer(PJRT_Buffer_ToHostBuffer_Args* a) {
  MI_NEED(a, PJRT_Buffer_ToHostBuffer_Args, event);
  PJRT_Buffer* b = a->src;
  if (!b->usable()) return Fail(PJRT_Error_Code_INVALID_ARGUMENT, "ToHostBuffer: buffer was deleted");
  if (!IsRowMajor(a->host_layout, b->dims.data(), b->dims.size(), ElementBytes(b->type)))
    return Fail(PJRT_Error_Code_UNIMPLEMENTED, "ToHostBuffer: only dense row-major host layouts are supported");
  if (a->dst == nullptr) {  // size query
    a->dst_size = b->bytes;
    a->event = new PJRT_Event{Completion::Done()};
    return nullptr;
  }
  if (a->dst_size < b->bytes)
    return Fail(PJRT_Error_Code_INVALID_ARGUMENT, "ToHostBuffer: dst_size " + std::to_string(a->dst_size) +
                                                      " < " + std::to_string(b->bytes) + " bytes");
  Block* blk = b->block.get();
  if (b->bytes == 0) {
    a->event = new PJRT_Event{Completion::Done()};
    return nullptr;
  }
  if (blk->where == Placement::kPinnedHost) {
    std::string e = b->defined ? b->defined->Wait() : "";
    if (e.empty()) memcpy(a->dst, blk->ptr, b->bytes);
    a->event = new PJRT_Event{Completion::Done(e)};
    return nullptr;
  }
  exec::DeviceContext* ctx = blk->ctx;
  std::string err;
  if (!exec::UseDevice(ctx->ordinal(), &err) || !OrderComputeAfter(b->defined, ctx, &err))
    return Fail(PJRT_Error_Code_INTERNAL, "ToHostBuffer: " + err);
  void* stage = ctx->TakePinned(b->bytes, &err);
  if (!stage) return Fail(PJRT_Error_Code_RESOURCE_EXHAUSTED, "ToHostBuffer: " + err);
  hipError_t r = hipMemcpyAsync(stage, blk->ptr, b->bytes, hipMemcpyDeviceToHost, ctx->stream());
  if (r != hipSuccess) {
    ctx->ReturnPinned(stage, nullptr);
    return Fail(PJRT_Error_Code_INTERNAL, std::string("ToHostBuffer: hipMemcpyAsync: ") + hipGetErrorString(r));
  }
  void* dst = a->dst;
  const size_t n = b->bytes;
  std::shared_ptr<Completion> done = RecordOn(ctx, ctx->stream(), Lane::kCompute, [ctx, stage, dst, n] {
    memcpy(dst, stage, n);
    ctx->ReturnPinned(stage, nullptr);
    return std::string();
  }, &err);
  if (!done) {
    (void)hipStreamSynchronize(ctx->stream());
    ctx->ReturnPinned(stage, nullptr);
    return Fail(PJRT_Error_Code_INTERNAL, "ToHostBuffer: " + err);
  }
  Watch(done);  // the caller's memory is filled even if nobody waits
  a->event = new PJRT_Event{std::move(done)};
  return nullptr;
}

PJRT_Error* Buffer_CopyToMemory(PJRT_Buffer_CopyToMemory_Args* a) {
  if (!a->dst_memory) return Fail(PJRT_Error_Code_INVALID_ARGUMENT, "CopyToMemory: null memory");
  return CopyInto(a->buffer, a->dst_memory, &a->dst_buffer, "CopyToMemory");
}
PJRT_Error* Buffer_CopyToDevice(PJRT_Buffer_CopyToDevice_Args* a) {
  if (!a->dst_device) return Fail(PJRT_Error_Code_INVALID_ARGUMENT, "CopyToDevice: null device");
  return CopyInto(a->buffer, &a->dst_device->hbm, &a->dst_buffer, "CopyToDevice");
}

PJRT_Error* Client_CreateViewOfDeviceBuffer(PJRT_Client_CreateViewOfDeviceBuffer_Args* a) {
  MI_NEED(a, PJRT_Client_CreateViewOfDeviceBuffer_Args, buffer);
  const size_t width = ElementBytes(a->element_type);
  if (width == 0) return Fail(PJRT_Error_Code_UNIMPLEMENTED, "CreateViewOfDeviceBuffer: element type not carried");
  if (!IsRowMajor(a->layout, a->dims, a->num_dims, width))
    return Fail(PJRT_Error_Code_UNIMPLEMENTED, "CreateViewOfDeviceBuffer: only dense row-major layouts");
  PJRT_Device* dev = a->device ? a->device : a->client->device_list.front();
  std::string err;
  exec::DeviceContext* ctx = ContextOf(dev, &err);
  if (!ctx) return Fail(PJRT_Error_Code_UNAVAILABLE, "CreateViewOfDeviceBuffer: " + err);
  size_t count = 1;
  for (size_t i = 0; i < a->num_dims; ++i) count *= size_t(a->dims[i] < 0 ? 0 : a->dims[i]);
  auto block = std::make_shared<Block>();
  block->ptr = a->device_buffer_ptr;
  block->bytes = count * width;
  block->where = Placement::kForeign;
  block->ctx = ctx;
  auto cb = a->on_delete_callback;
  void* cb_arg = a->on_delete_callback_arg;
  void* ptr = a->device_buffer_ptr;
  block->on_release = [ctx, cb, cb_arg, ptr] {
    // hand the memory back only after work queued on it has finished
    (void)ctx->Synchronize(nullptr);
    if (cb) cb(ptr, cb_arg);
  };
  std::shared_ptr<Completion> defined;
  if (a->stream) {  // the data is ready once the caller's stream passes this point
    defined = RecordOn(ctx, reinterpret_cast<hipStream_t>(a->stream), Lane::kTransfer, {}, &err);
    if (!defined) return Fail(PJRT_Error_Code_INTERNAL, "CreateViewOfDeviceBuffer: " + err);
  }
  a->buffer = Wrap(dev, &dev->hbm, a->element_type, std::vector<int64_t>(a->dims, a->dims + a->num_dims),
                   std::move(block), std::move(defined));
  return nullptr;
}

PJRT_Error* Buffer_Destroy(PJRT_Buffer_Destroy_Args* a) {
  delete a->buffer;  // the block goes with its last holder
  return nullptr;
}
PJRT_Error* Buffer_Delete(PJRT_Buffer_Delete_Args* a) {
  PJRT_Buffer* b = a->buffer;
  if (b->life != PJRT_Buffer::Life::kLive) return nullptr;
  if (b->pins > 0) {
    b->life = PJRT_Buffer::Life::kDeletedPinned;
  } else {
    b->life = PJRT_Buffer::Life::kDeleted;
    b->block.reset();
  }
  return nullptr;
}
PJRT_Error* Buffer_IsDeleted(PJRT_Buffer_IsDeleted_Args* a) {
  a->is_deleted = a->buffer->life != PJRT_Buffer::Life::kLive;
  return nullptr;
}
PJRT_Error* Buffer_IncreaseExternalReferenceCount(PJRT_Buffer_IncreaseExternalReferenceCount_Args* a) {
  if (a->buffer->life != PJRT_Buffer::Life::kLive)
    return Fail(PJRT_Error_Code_INVALID_ARGUMENT, "IncreaseExternalReferenceCount: buffer was deleted");
  ++a->buffer->pins;
  return nullptr;
}
PJRT_Error* Buffer_DecreaseExternalReferenceCount(PJRT_Buffer_DecreaseExternalReferenceCount_Args* a) {
  PJRT_Buffer* b = a->buffer;
  if (b->pins == 0)
    return Fail(PJRT_Error_Code_FAILED_PRECONDITION, "DecreaseExternalReferenceCount: no external reference held");
  if (--b->pins == 0 && b->life == PJRT_Buffer::Life::kDeletedPinned) {
    b->life = PJRT_Buffer::Life::kDeleted;
    b->block.reset();
  }
  return nullptr;
}
PJRT_Error* Buffer_ElementType(PJRT_Buffer_ElementType_Args* a) {
  a->type = a->buffer->type;
  return nullptr;
}
PJRT_Error* Buffer_Dimensions(PJRT_Buffer_Dimensions_Args* a) {
  a->dims = a->buffer->dims.data();
  a->num_dims = a->buffer->dims.size();
  return nullptr;
}
PJRT_Error* Buffer_UnpaddedDimensions(PJRT_Buffer_UnpaddedDimensions_Args* a) {
  a->unpadded_dims = a->buffer->dims.data();  // no padding: dense storage
  a->num_dims = a->buffer->dims.size();
  return nullptr;
}
PJRT_Error* Buffer_DynamicDimensionIndices(PJRT_Buffer_DynamicDimensionIndices_Args* a) {
  a->dynamic_dim_indices = nullptr;  // static shapes only
  a->num_dynamic_dims = 0;
  return nullptr;
}
PJRT_Error* Buffer_GetMemoryLayout(PJRT_Buffer_GetMemoryLayout_Args* a) {
  PJRT_Buffer* b = a->buffer;
  PJRT_Buffer_MemoryLayout& l = a->layout;
  memset(&l, 0, sizeof(l));
  l.struct_size = sizeof(PJRT_Buffer_MemoryLayout);
  l.type = PJRT_Buffer_MemoryLayout_Type_Tiled;
  l.tiled.struct_size = sizeof(PJRT_Buffer_MemoryLayout_Tiled);
  l.tiled.minor_to_major = b->minor_to_major.data();
  l.tiled.minor_to_major_size = b->minor_to_major.size();
  l.tiled.num_tiles = 0;
  return nullptr;
}
PJRT_Error* Buffer_OnDeviceSizeInBytes(PJRT_Buffer_OnDeviceSizeInBytes_Args* a) {
  a->on_device_size_in_bytes = a->buffer->bytes;
  return nullptr;
}
PJRT_Error* Buffer_Device(PJRT_Buffer_Device_Args* a) {
  a->device = a->buffer->device;
  return nullptr;
}
PJRT_Error* Buffer_Memory(PJRT_Buffer_Memory_Args* a) {
  a->memory = a->buffer->memory;
  return nullptr;
}
PJRT_Error* Buffer_IsOnCpu(PJRT_Buffer_IsOnCpu_Args* a) {
  a->is_on_cpu = a->buffer->memory->space == Placement::kPinnedHost;
  return nullptr;
}
PJRT_Error* Buffer_ReadyEvent(PJRT_Buffer_ReadyEvent_Args* a) {
  const auto& d = a->buffer->defined;
  a->event = new PJRT_Event{d ? d : Completion::Done()};
  return nullptr;
}
PJRT_Error* Buffer_UnsafePointer(PJRT_Buffer_UnsafePointer_Args* a) {
  const auto& blk = a->buffer->block;
  a->buffer_pointer = reinterpret_cast<uintptr_t>(blk ? blk->ptr : nullptr);
  return nullptr;
}
PJRT_Error* Buffer_OpaqueDeviceMemoryDataPointer(PJRT_Buffer_OpaqueDeviceMemoryDataPointer_Args* a) {
  const auto& blk = a->buffer->block;
  a->device_memory_ptr = blk ? blk->ptr : nullptr;
  return nullptr;
}

}  // namespace slot
}  // namespace mi::pjrt
