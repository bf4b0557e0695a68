// Compile, executables and Execute.
//
// Reference counterparts: ClientCompile (pjrt_c_api.cc:681-697: program
// bytes -> jam::Compile, errors as INVALID_ARGUMENT "jam compile: ..."),
// the executable getters (699-751) and LoadedExecute (753-829: per-device
// argument and output lists, completion events).  Execute here queues the
// launch plan on the device's compute stream and returns; inputs still
// being uploaded are waited for on the GPU (hipStreamWaitEvent), and an
// input the plan may overwrite can be donated to an output.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <set>

#include "jam/run.h"
#include "pjrt/api/plugin.h"

namespace mi::pjrt {
namespace {

// Serialized executables: this magic, then the program bytes they were
// compiled from, StableHLO text or a portable artifact (recompiled on load;
// compilation is deterministic).
constexpr char kSerialMagic[] = "mi355x-jam/1\n";

struct Compiled {
  std::shared_ptr<jam::Program> program;
  std::shared_ptr<const std::string> source;
  std::string fingerprint;
};

PJRT_Error* CompileText(const char* code, size_t size, Compiled* out) {
  if (const char* path = std::getenv("MI355X_SAVE_PROGRAM")) {  // keep what the client sent
    if (FILE* f = std::fopen(path, "wb")) {
      std::fwrite(code, 1, size, f);
      std::fclose(f);
    }
  }
  jam::CompileResult r = jam::Compile(code, size, jam::OptionsFromEnv());
  if (!r.program) return Fail(PJRT_Error_Code_INVALID_ARGUMENT, "jam compile: " + r.error);
  if (std::getenv("MI355X_PRINT_PLAN")) std::fputs(r.program->Dump().c_str(), stderr);
  out->program = std::move(r.program);
  out->source = std::make_shared<const std::string>(code, size);
  out->fingerprint = Fingerprint(code, size);
  return nullptr;
}

PJRT_Error* ReadProgram(const PJRT_Program* p, const char** code, size_t* size) {
  if (!p || !p->code) return Fail(PJRT_Error_Code_INVALID_ARGUMENT, "jam compile: null program");
  const std::string format(p->format ? p->format : "", p->format ? p->format_size : 0);
  if (!format.empty() && format != "mlir")
    return Fail(PJRT_Error_Code_INVALID_ARGUMENT, "jam compile: unsupported program format '" + format + "'");
  *code = p->code;
  *size = p->code_size;
  return nullptr;
}

PJRT_LoadedExecutable* Load(PJRT_Client* client, Compiled c) {
  auto* le = new PJRT_LoadedExecutable();
  le->client = client;
  le->program = std::move(c.program);
  le->source = std::move(c.source);
  le->fingerprint = std::move(c.fingerprint);
  le->devices = {client->device_list.front()};
  return le;
}

PJRT_Executable* Unloaded(std::shared_ptr<jam::Program> p, std::shared_ptr<const std::string> src, std::string fp) {
  auto* e = new PJRT_Executable();
  e->program = std::move(p);
  e->source = std::move(src);
  e->fingerprint = std::move(fp);
  e->results.Fill(*e->program);
  return e;
}

// Which outputs take over the memory of which arguments, per the plan's
// aliases (Program::input_alias) and the caller's refusals.
std::vector<int> PlanDonations(const jam::Program& prog, PJRT_Buffer* const* args, size_t n,
                               const std::set<int64_t>& refused, exec::DeviceContext* ctx) {
  std::vector<int> taker_of(n, -1);  // per argument: the output that takes its memory
  for (size_t i = 0; i < n && i < prog.input_alias.size(); ++i) {
    const int out = prog.input_alias[i];
    if (out < 0 || refused.count(int64_t(i))) continue;
    PJRT_Buffer* b = args[i];
    if (!b->usable() || b->pins != 0 || b->block->where != Placement::kHbm || b->block->ctx != ctx) continue;
    if (b->block.use_count() != 1) continue;  // memory shared with in-flight work or another buffer
    bool twice = false;
    for (size_t j = 0; j < n; ++j) twice |= (j != i && args[j] == b);
    if (!twice) taker_of[i] = out;
  }
  return taker_of;
}

PJRT_Error* RunOnDevice(PJRT_LoadedExecutable* le, const jam::Program& prog_c, PJRT_Device* dev,
                        PJRT_Buffer* const* args, size_t n_args, const std::set<int64_t>& refused,
                        PJRT_Buffer** outputs, PJRT_Event** complete) {
  jam::Program& prog = const_cast<jam::Program&>(prog_c);
  std::string err;
  exec::DeviceContext* ctx = ContextOf(dev, &err);
  if (!ctx) return Fail(PJRT_Error_Code_UNAVAILABLE, "Execute: " + err);
  std::vector<jam::RunInput> ins;
  std::vector<std::shared_ptr<Block>> hold;  // keeps argument memory alive while launches are queued
  for (size_t i = 0; i < n_args; ++i) {
    PJRT_Buffer* b = args[i];
    const std::string which = "Execute: argument " + std::to_string(i);
    if (!b || !b->usable()) return Fail(PJRT_Error_Code_INVALID_ARGUMENT, which + " was deleted");
    if (b->block->where == Placement::kPinnedHost)
      return Fail(PJRT_Error_Code_INVALID_ARGUMENT, which + " is in pinned_host memory; copy it to the device first");
    if (b->block->ctx != ctx) return Fail(PJRT_Error_Code_INVALID_ARGUMENT, which + " lives on another device");
    if (b->bytes != prog.inputs[i].bytes())
      return Fail(PJRT_Error_Code_INVALID_ARGUMENT, which + " size mismatch: " + std::to_string(b->bytes) +
                                                       " bytes given, the program expects " +
                                                       std::to_string(prog.inputs[i].bytes()));
  }
  const std::vector<int> taker_of = PlanDonations(prog, args, n_args, refused, ctx);
  std::vector<void*> preset(prog.outputs.size(), nullptr);
  for (size_t i = 0; i < n_args; ++i)
    if (taker_of[i] >= 0) preset[size_t(taker_of[i])] = args[i]->block->ptr;
  for (size_t i = 0; i < n_args; ++i) {
    if (!OrderComputeAfter(args[i]->defined, ctx, &err)) return Fail(PJRT_Error_Code_INTERNAL, "Execute: " + err);
    ins.push_back({args[i]->block->ptr, args[i]->bytes});
    hold.push_back(args[i]->block);
  }
  std::vector<jam::RunOutput> outs;
  err = jam::Run(prog, *ctx, ins, outs, &preset);
  if (!err.empty()) return Fail(PJRT_Error_Code_INTERNAL, err);
  hipEvent_t ev = nullptr;
  hipError_t r = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
  if (r == hipSuccess) r = hipEventRecord(ev, ctx->stream());
  if (r != hipSuccess) {
    if (ev) (void)hipEventDestroy(ev);
    (void)ctx->Synchronize(nullptr);
    for (auto& o : outs)
      if (o.data) ctx->Free(o.data);
    return Fail(PJRT_Error_Code_INTERNAL, std::string("Execute: hipEventRecord: ") + hipGetErrorString(r));
  }
  std::shared_ptr<Completion> done = Completion::AfterGpu(ctx->ordinal(), Lane::kCompute, ev);
  hold.clear();
  // outputs; a donated argument's block moves to its output and the
  // argument is deleted
  std::vector<std::shared_ptr<Block>> taken(outs.size());
  for (size_t i = 0; i < n_args; ++i) {
    if (taker_of[i] < 0) continue;
    taken[size_t(taker_of[i])] = std::move(args[i]->block);
    args[i]->life = PJRT_Buffer::Life::kDeleted;
    args[i]->defined = nullptr;
  }
  for (size_t k = 0; k < outs.size(); ++k) {
    std::shared_ptr<Block> blk = taken[k];
    if (!blk) {
      blk = std::make_shared<Block>();
      blk->ptr = outs[k].data;
      blk->bytes = outs[k].nbytes;
      blk->where = Placement::kHbm;
      blk->ctx = ctx;
    }
    auto* ob = new PJRT_Buffer();
    ob->client = le->client;
    ob->device = dev;
    ob->memory = &dev->hbm;
    ob->type = PJRT_Buffer_Type(int(outs[k].type.dtype));
    ob->dims = outs[k].type.dims;
    ob->minor_to_major.resize(ob->dims.size());
    for (size_t d = 0; d < ob->dims.size(); ++d) ob->minor_to_major[d] = int64_t(ob->dims.size() - 1 - d);
    ob->bytes = outs[k].nbytes;
    ob->block = std::move(blk);
    ob->defined = done;
    outputs[k] = ob;
  }
  if (complete) *complete = new PJRT_Event{done};
  return nullptr;
}

}  // namespace

namespace slot {

PJRT_Error* Client_Compile(PJRT_Client_Compile_Args* a) {
  MI_NEED(a, PJRT_Client_Compile_Args, executable);
  const char* code = nullptr;
  size_t size = 0;
  if (PJRT_Error* e = ReadProgram(a->program, &code, &size)) return e;
  Compiled c;
  if (PJRT_Error* e = CompileText(code, size, &c)) return e;
  a->executable = Load(a->client, std::move(c));
  return nullptr;
}

// Ahead-of-time compile against a topology: the same launch plan, not yet
// bound to a client.
PJRT_Error* Compile(PJRT_Compile_Args* a) {
  MI_NEED(a, PJRT_Compile_Args, executable);
  const char* code = nullptr;
  size_t size = 0;
  if (PJRT_Error* e = ReadProgram(a->program, &code, &size)) return e;
  Compiled c;
  if (PJRT_Error* e = CompileText(code, size, &c)) return e;
  a->executable = Unloaded(std::move(c.program), std::move(c.source), std::move(c.fingerprint));
  return nullptr;
}

PJRT_Error* Executable_Serialize(PJRT_Executable_Serialize_Args* a) {
  MI_NEED(a, PJRT_Executable_Serialize_Args, serialized_executable_deleter);
  const PJRT_Executable* e = a->executable;
  auto* s = new PJRT_SerializedExecutable();
  s->bytes = std::string(kSerialMagic) + *e->source;
  a->serialized_bytes = s->bytes.data();
  a->serialized_bytes_size = s->bytes.size();
  a->serialized_executable = s;
  a->serialized_executable_deleter = [](PJRT_SerializedExecutable* p) { delete p; };
  return nullptr;
}

PJRT_Error* Executable_DeserializeAndLoad(PJRT_Executable_DeserializeAndLoad_Args* a) {
  MI_NEED(a, PJRT_Executable_DeserializeAndLoad_Args, loaded_executable);
  const size_t m = sizeof(kSerialMagic) - 1;
  if (!a->serialized_executable || a->serialized_executable_size < m ||
      memcmp(a->serialized_executable, kSerialMagic, m) != 0)
    return Fail(PJRT_Error_Code_INVALID_ARGUMENT, "DeserializeAndLoad: not an executable serialized by mi355x-pjrt");
  Compiled c;
  if (PJRT_Error* e = CompileText(a->serialized_executable + m, a->serialized_executable_size - m, &c)) return e;
  a->loaded_executable = Load(a->client, std::move(c));
  return nullptr;
}

PJRT_Error* LoadedExecutable_GetExecutable(PJRT_LoadedExecutable_GetExecutable_Args* a) {
  PJRT_LoadedExecutable* le = a->loaded_executable;
  if (!le->program) return Fail(PJRT_Error_Code_INVALID_ARGUMENT, "GetExecutable: executable was deleted");
  a->executable = Unloaded(le->program, le->source, le->fingerprint);
  return nullptr;
}
PJRT_Error* Executable_Destroy(PJRT_Executable_Destroy_Args* a) {
  delete a->executable;
  return nullptr;
}
PJRT_Error* Executable_Name(PJRT_Executable_Name_Args* a) {
  const std::string& n = a->executable->program->name;
  a->executable_name = n.c_str();
  a->executable_name_size = n.size();
  return nullptr;
}
PJRT_Error* Executable_NumReplicas(PJRT_Executable_NumReplicas_Args* a) {
  a->num_replicas = 1;
  return nullptr;
}
PJRT_Error* Executable_NumPartitions(PJRT_Executable_NumPartitions_Args* a) {
  a->num_partitions = 1;
  return nullptr;
}
PJRT_Error* Executable_NumOutputs(PJRT_Executable_NumOutputs_Args* a) {
  a->num_outputs = a->executable->results.types.size();
  return nullptr;
}
PJRT_Error* Executable_SizeOfGeneratedCodeInBytes(PJRT_Executable_SizeOfGeneratedCodeInBytes_Args* a) {
  // the "code" of a launch plan is its step list plus its constant pool
  const jam::Program& p = *a->executable->program;
  int64_t n = int64_t(p.steps.size() * sizeof(jam::Step));
  for (const auto& c : p.consts) n += int64_t(c.bytes.size());
  a->size_in_bytes = n;
  return nullptr;
}
PJRT_Error* Executable_Fingerprint(PJRT_Executable_Fingerprint_Args* a) {
  a->executable_fingerprint = a->executable->fingerprint.c_str();
  a->executable_fingerprint_size = a->executable->fingerprint.size();
  return nullptr;
}
PJRT_Error* LoadedExecutable_Fingerprint(PJRT_LoadedExecutable_Fingerprint_Args* a) {
  a->executable_fingerprint = a->executable->fingerprint.c_str();
  a->executable_fingerprint_size = a->executable->fingerprint.size();
  return nullptr;
}
// The optimized program of a jam executable is its launch plan, as text
// (format "jam-plan"); code == nullptr asks for the size first.
PJRT_Error* Executable_OptimizedProgram(PJRT_Executable_OptimizedProgram_Args* a) {
  MI_NEED(a, PJRT_Executable_OptimizedProgram_Args, program);
  static const char kFormat[] = "jam-plan";
  PJRT_Program* p = a->program;
  if (!p) return Fail(PJRT_Error_Code_INVALID_ARGUMENT, "OptimizedProgram: null program");
  const std::string plan = a->executable->program->Dump();
  p->format = kFormat;
  p->format_size = sizeof(kFormat) - 1;
  if (p->code != nullptr) {
    if (p->code_size < plan.size())
      return Fail(PJRT_Error_Code_INVALID_ARGUMENT, "OptimizedProgram: code buffer too small");
    memcpy(p->code, plan.data(), plan.size());
  }
  p->code_size = plan.size();
  return nullptr;
}
PJRT_Error* Executable_GetCostAnalysis(PJRT_Executable_GetCostAnalysis_Args* a) {
  a->num_properties = 0;
  a->properties = nullptr;
  return nullptr;
}
PJRT_Error* Executable_OutputElementTypes(PJRT_Executable_OutputElementTypes_Args* a) {
  ResultTable& r = a->executable->results;
  a->output_types = r.types.data();
  a->num_output_types = r.types.size();
  return nullptr;
}
PJRT_Error* Executable_OutputDimensions(PJRT_Executable_OutputDimensions_Args* a) {
  const ResultTable& r = a->executable->results;
  a->num_outputs = r.ranks.size();
  a->dims = r.dims.data();
  a->dim_sizes = r.ranks.data();
  return nullptr;
}
PJRT_Error* Executable_OutputMemoryKinds(PJRT_Executable_OutputMemoryKinds_Args* a) {
  const ResultTable& r = a->executable->results;
  a->num_outputs = r.kinds.size();
  a->memory_kinds = r.kinds.data();
  a->memory_kind_sizes = r.kind_lengths.data();
  return nullptr;
}
PJRT_Error* Executable_GetCompiledMemoryStats(PJRT_Executable_GetCompiledMemoryStats_Args* a) {
  const jam::Program& p = *a->executable->program;
  int64_t in = 0, out = 0, alias = 0;
  for (const auto& t : p.inputs) in += int64_t(t.bytes());
  for (const auto& t : p.outputs) out += int64_t(t.bytes());
  for (size_t i = 0; i < p.input_alias.size(); ++i)
    if (p.input_alias[i] >= 0) alias += int64_t(p.inputs[i].bytes());
  a->generated_code_size_in_bytes = 0;
  a->argument_size_in_bytes = in;
  a->output_size_in_bytes = out;
  a->alias_size_in_bytes = alias;
  a->temp_size_in_bytes = int64_t(p.arena_bytes);
  a->host_generated_code_size_in_bytes = a->host_argument_size_in_bytes = a->host_output_size_in_bytes = 0;
  a->host_alias_size_in_bytes = a->host_temp_size_in_bytes = 0;
  return nullptr;
}

PJRT_Error* LoadedExecutable_Destroy(PJRT_LoadedExecutable_Destroy_Args* a) {
  delete a->executable;
  return nullptr;
}
PJRT_Error* LoadedExecutable_Delete(PJRT_LoadedExecutable_Delete_Args* a) {
  a->executable->program.reset();
  return nullptr;
}
PJRT_Error* LoadedExecutable_IsDeleted(PJRT_LoadedExecutable_IsDeleted_Args* a) {
  a->is_deleted = a->executable->program == nullptr;
  return nullptr;
}
PJRT_Error* LoadedExecutable_AddressableDevices(PJRT_LoadedExecutable_AddressableDevices_Args* a) {
  a->addressable_devices = a->executable->devices.data();
  a->num_addressable_devices = a->executable->devices.size();
  return nullptr;
}

PJRT_Error* LoadedExecutable_Execute(PJRT_LoadedExecutable_Execute_Args* a) {
  MI_NEED(a, PJRT_LoadedExecutable_Execute_Args, execute_device);
  PJRT_LoadedExecutable* le = a->executable;
  std::shared_ptr<jam::Program> prog = le->program;  // stays alive for this call
  if (!prog) return Fail(PJRT_Error_Code_INVALID_ARGUMENT, "Execute: executable was deleted");
  if (a->num_args != prog->inputs.size())
    return Fail(PJRT_Error_Code_INVALID_ARGUMENT, "Execute: the program takes " +
                                                     std::to_string(prog->inputs.size()) + " arguments, got " +
                                                     std::to_string(a->num_args));
  std::set<int64_t> refused;
  if (const PJRT_ExecuteOptions* o = a->options) {
    if (!Fits(o->struct_size, offsetof(PJRT_ExecuteOptions, num_non_donatable_input_indices) + sizeof(size_t)))
      return Fail(PJRT_Error_Code_INVALID_ARGUMENT, "Execute: PJRT_ExecuteOptions struct_size too small");
    for (size_t k = 0; o->non_donatable_input_indices && k < o->num_non_donatable_input_indices; ++k)
      refused.insert(o->non_donatable_input_indices[k]);
  }
  const std::vector<PJRT_Device*>& all = le->client->device_list;
  for (size_t d = 0; d < a->num_devices; ++d) {
    PJRT_Device* dev = a->execute_device ? a->execute_device
                       : a->num_devices == 1 ? le->devices.front()
                                             : all[d % all.size()];
    PJRT_Event** complete = a->device_complete_events ? &a->device_complete_events[d] : nullptr;
    if (PJRT_Error* e = RunOnDevice(le, *prog, dev, a->argument_lists[d], a->num_args, refused,
                                    a->output_lists[d], complete))
      return e;
  }
  return nullptr;
}

}  // namespace slot
}  // namespace mi::pjrt
