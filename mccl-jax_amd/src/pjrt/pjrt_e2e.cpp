// pjrt_e2e: drive libpjrt_mi355x.so through the PJRT C API only.
//
// Counterpart of the reference harness src/pjrt/pjrt_e2e.cc (usage 61-63,
// compile 114-129, execute 147-161, readback 163-177): load the plugin with
// dlopen + GetPjrtApi, compile a StableHLO text module, upload raw input
// files, execute, write outN.bin.  Adds the bf16 typecode the reference
// lacks (pjrt_e2e.cc:22-33).
//
// usage: pjrt_e2e <plugin.so> <module.mlir> [--compile-only]
//                 [<type>:<d0>x<d1>...:<file.bin> ...] [--out DIR]
// types: f32 f16 bf16 i32 i8 u8 i16 u16 u32 pred
#include <dlfcn.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <sstream>
#include <string>
#include <vector>

#include "pjrt/api/pjrt_abi.h"

namespace {

const PJRT_Api* api = nullptr;

template <typename T>
T Args() {
  T a;
  memset(&a, 0, sizeof(a));
  a.struct_size = sizeof(T);
  return a;
}

bool Check(PJRT_Error* e, const char* what) {
  if (!e) return true;
  auto m = Args<PJRT_Error_Message_Args>();
  m.error = e;
  api->PJRT_Error_Message(&m);
  auto c = Args<PJRT_Error_GetCode_Args>();
  c.error = e;
  api->PJRT_Error_GetCode(&c);
  fprintf(stderr, "%s failed (code %d): %.*s\n", what, int(c.code), int(m.message_size), m.message);
  auto d = Args<PJRT_Error_Destroy_Args>();
  d.error = e;
  api->PJRT_Error_Destroy(&d);
  return false;
}

void Await(PJRT_Event* ev) {
  if (!ev) return;
  auto a = Args<PJRT_Event_Await_Args>();
  a.event = ev;
  Check(api->PJRT_Event_Await(&a), "Event_Await");
  auto d = Args<PJRT_Event_Destroy_Args>();
  d.event = ev;
  api->PJRT_Event_Destroy(&d);
}

PJRT_Buffer_Type TypeOf(const std::string& s, size_t* width) {
  struct T {
    const char* n;
    PJRT_Buffer_Type t;
    size_t w;
  } table[] = {{"f32", PJRT_Buffer_Type_F32, 4}, {"f16", PJRT_Buffer_Type_F16, 2},
               {"bf16", PJRT_Buffer_Type_BF16, 2}, {"i32", PJRT_Buffer_Type_S32, 4},
               {"i8", PJRT_Buffer_Type_S8, 1}, {"u8", PJRT_Buffer_Type_U8, 1},
               {"i16", PJRT_Buffer_Type_S16, 2}, {"u16", PJRT_Buffer_Type_U16, 2},
               {"u32", PJRT_Buffer_Type_U32, 4}, {"pred", PJRT_Buffer_Type_PRED, 1}};
  for (auto& t : table)
    if (s == t.n) {
      *width = t.w;
      return t.t;
    }
  *width = 0;
  return PJRT_Buffer_Type_INVALID;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 3) {
    fprintf(stderr, "usage: %s <plugin.so> <module.mlir> [--compile-only] [type:dims:file.bin ...] [--out DIR]\n", argv[0]);
    return 2;
  }
  void* h = dlopen(argv[1], RTLD_NOW | RTLD_LOCAL);
  if (!h) {
    fprintf(stderr, "dlopen: %s\n", dlerror());
    return 1;
  }
  auto get = reinterpret_cast<const PJRT_Api* (*)()>(dlsym(h, "GetPjrtApi"));
  if (!get || !(api = get())) {
    fprintf(stderr, "GetPjrtApi not found\n");
    return 1;
  }
  printf("PJRT API %d.%d, struct_size %zu\n", api->pjrt_api_version.major_version,
         api->pjrt_api_version.minor_version, api->struct_size);
  auto init = Args<PJRT_Plugin_Initialize_Args>();
  if (!Check(api->PJRT_Plugin_Initialize(&init), "Plugin_Initialize")) return 1;

  std::ifstream mf(argv[2], std::ios::binary);
  std::stringstream ss;
  ss << mf.rdbuf();
  std::string code = ss.str();
  bool compile_only = false;
  std::string out_dir = ".";
  std::vector<std::string> specs;
  for (int i = 3; i < argc; ++i) {
    std::string s = argv[i];
    if (s == "--compile-only") compile_only = true;
    else if (s == "--out" && i + 1 < argc) out_dir = argv[++i];
    else specs.push_back(s);
  }

  auto cc = Args<PJRT_Client_Create_Args>();
  if (!Check(api->PJRT_Client_Create(&cc), "Client_Create")) return 1;
  PJRT_Client* client = cc.client;
  auto pn = Args<PJRT_Client_PlatformName_Args>();
  pn.client = client;
  api->PJRT_Client_PlatformName(&pn);
  printf("platform %.*s\n", int(pn.platform_name_size), pn.platform_name);

  PJRT_Program prog;
  memset(&prog, 0, sizeof(prog));
  prog.struct_size = sizeof(prog);
  prog.code = code.data();
  prog.code_size = code.size();
  prog.format = "mlir";
  prog.format_size = 4;
  auto comp = Args<PJRT_Client_Compile_Args>();
  comp.client = client;
  comp.program = &prog;
  if (!Check(api->PJRT_Client_Compile(&comp), "Client_Compile")) return 1;
  PJRT_LoadedExecutable* exe = comp.executable;
  auto ge = Args<PJRT_LoadedExecutable_GetExecutable_Args>();
  ge.loaded_executable = exe;
  api->PJRT_LoadedExecutable_GetExecutable(&ge);
  auto no = Args<PJRT_Executable_NumOutputs_Args>();
  no.executable = ge.executable;
  api->PJRT_Executable_NumOutputs(&no);
  printf("compiled: %zu outputs\n", no.num_outputs);
  if (compile_only) return 0;

  std::vector<PJRT_Buffer*> args;
  std::vector<std::vector<char>> hosts;
  for (const std::string& s : specs) {
    size_t c1 = s.find(':'), c2 = s.rfind(':');
    size_t w;
    PJRT_Buffer_Type t = TypeOf(s.substr(0, c1), &w);
    std::vector<int64_t> dims;
    std::stringstream ds(s.substr(c1 + 1, c2 - c1 - 1));
    std::string tok;
    size_t n = 1;
    while (std::getline(ds, tok, 'x'))
      if (!tok.empty()) {
        dims.push_back(atoll(tok.c_str()));
        n *= size_t(dims.back());
      }
    std::ifstream f(s.substr(c2 + 1), std::ios::binary);
    hosts.emplace_back(n * w);
    f.read(hosts.back().data(), std::streamsize(n * w));
    auto b = Args<PJRT_Client_BufferFromHostBuffer_Args>();
    b.client = client;
    b.data = hosts.back().data();
    b.type = t;
    b.dims = dims.data();
    b.num_dims = dims.size();
    if (!Check(api->PJRT_Client_BufferFromHostBuffer(&b), "BufferFromHostBuffer")) return 1;
    Await(b.done_with_host_buffer);
    args.push_back(b.buffer);
  }
  std::vector<PJRT_Buffer*> outs(no.num_outputs);
  PJRT_Buffer* const* arg_list = args.data();
  PJRT_Buffer** out_list = outs.data();
  PJRT_Event* done = nullptr;
  auto ex = Args<PJRT_LoadedExecutable_Execute_Args>();
  ex.executable = exe;
  ex.argument_lists = &arg_list;
  ex.num_devices = 1;
  ex.num_args = args.size();
  ex.output_lists = &out_list;
  ex.device_complete_events = &done;
  if (!Check(api->PJRT_LoadedExecutable_Execute(&ex), "Execute")) return 1;
  Await(done);
  for (size_t i = 0; i < outs.size(); ++i) {
    auto q = Args<PJRT_Buffer_ToHostBuffer_Args>();
    q.src = outs[i];
    if (!Check(api->PJRT_Buffer_ToHostBuffer(&q), "ToHostBuffer(size)")) return 1;
    Await(q.event);
    std::vector<char> host(q.dst_size);
    q.dst = host.data();
    q.event = nullptr;
    if (!Check(api->PJRT_Buffer_ToHostBuffer(&q), "ToHostBuffer")) return 1;
    Await(q.event);
    std::string path = out_dir + "/out" + std::to_string(i) + ".bin";
    std::ofstream of(path, std::ios::binary);
    of.write(host.data(), std::streamsize(host.size()));
    printf("wrote %s (%zu bytes)\n", path.c_str(), host.size());
  }
  return 0;
}
