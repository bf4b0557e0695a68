// jam launch plan: what Compile produces and Run executes.
//
// The reference compiles a module into one MPSGraph (or graph segments plus
// collective steps) and runs it synchronously (program_impl.h:14-51,
// jam_run.mm:361-419).  jam instead produces a flat list of kernel launches
// over the C-ABI of include/mk_kernels.h.  Every buffer a launch touches is a
// BufRef resolved at run time: a program input, a program output, a slice
// of the per-run arena (temporaries, liveness-packed at compile time) or a
// constant uploaded once per device.
#pragma once

#include <cstdint>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "jam/ew_jit.h"
#include "jam/ir.h"

namespace mi::jam {

enum class Space : uint8_t { kInput, kOutput, kArena, kConst, kNone };

struct BufRef {
  Space space = Space::kNone;
  int index = 0;        // input / output / const index (unused for arena)
  int64_t offset = 0;   // byte offset (arena: absolute offset in the arena)
};

enum class StepKind : uint8_t {
  kGemm, kSdpa, kRowReduce, kArgmax, kLayerNorm, kGelu, kEw, kGather, kScatterAdd,
  kIota, kCopyStrided, kSoftmax, kConvert, kFill, kCopy, kSdpaBwd, kGemmBlas, kSoftmaxXent, kColSum,
  kGemmSplitK, kEwReduce, kLayerNormBwd,
};

const char* StepName(StepKind k);

struct Step {
  StepKind kind;
  std::vector<BufRef> bufs;    // kernel-specific order (documented in run.cc)
  std::vector<int64_t> i;      // integer parameters
  std::vector<float> f;        // float parameters
  std::vector<int32_t> prog;   // ew program (4 ints per instruction)
  std::vector<int64_t> strides;  // ew per-input strides (6 per input) / copy strides
  std::vector<int32_t> types;  // ew per-input dtypes
  std::string note;            // provenance for dumps / errors
  int jit = -1;                // ew: index of its generated kernel in Program::ew_jit (-1: interpreter)
  int batch = 1;               // ew: independent instances of one program; bufs holds each one's in turn
};

struct ConstBlob {
  TensorType type;
  std::vector<uint8_t> bytes;
};

class Program {
 public:
  std::vector<TensorType> inputs;
  std::vector<TensorType> outputs;
  std::vector<Step> steps;
  std::vector<ConstBlob> consts;
  size_t arena_bytes = 0;
  // Donation: per input, the output whose launches may write straight into
  // this input's memory when the caller donates it (-1: none).  Set only
  // where the plan allows it: no launch reads the input after the output's
  // first writer, which reads it (if at all) element for element in the
  // same layout.
  std::vector<int> input_alias;
  std::vector<std::string> alias_notes;  // why a requested alias was or was not taken (dumps)
  std::vector<std::string> patterns;   // fused patterns recognised (for tests / dumps)
  std::string name = "jam.main";
  // generated kernels of the ew steps (null when disabled)
  std::shared_ptr<EwJit> ew_jit;

  std::string Dump() const;

  // device copies of `consts`, uploaded lazily once per device ordinal
  std::vector<void*>* DeviceConsts(int ordinal);
  ~Program();

 private:
  std::mutex mu_;
  std::vector<std::vector<void*>> dev_consts_;
};

struct CompileOptions {
  bool fuse_sdpa = true;        // env JAM_NO_SDPA disables
  bool fuse_argmax = true;
  bool fuse_gemm_epilogue = true;
  bool fuse_layernorm = true;
  bool fuse_gelu = true;
  bool fuse_elementwise = true;
  bool fuse_xent = true;        // env JAM_NO_XENT disables
  bool ew_jit = true;           // env JAM_NO_EW_JIT disables (ew steps run the interpreter)
  bool ew_jit_eager = false;    // env JAM_EW_JIT_EAGER: compile the generated kernels in Compile
  bool ew_jit_strict = false;   // env JAM_EW_JIT_STRICT: no interpreter fallback (EwJit::strict)
  bool ew_batch = true;         // env JAM_NO_EW_BATCH disables batching independent ew steps
};

struct CompileResult {
  std::shared_ptr<Program> program;
  std::string error;
};

// Compile StableHLO (MLIR text) into a launch plan.  Mirrors
// jam::Compile(bytes, size, num_processes) of the reference (jam.cc:8-24).
CompileResult Compile(const char* code, size_t size, const CompileOptions& opts = CompileOptions());
CompileOptions OptionsFromEnv();

}  // namespace mi::jam
