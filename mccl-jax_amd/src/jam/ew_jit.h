// Compiled elementwise steps.
//
// An "ew" step carries a small register program (include/mk_kernels.h,
// mk_ew_program_multi) that the generic kernel decodes instruction by
// instruction at run time.  Its shape, strides, dtypes and constants are
// all known when the module is lowered, so jam also writes each such step
// out as HIP source with everything fixed: the program becomes straight-line
// fp32 code, the index decomposition divides by constants, broadcast inputs
// are read once per thread.  The sources of one module are compiled together
// with hiprtc for gfx950 (the kernel library's code-generation flags; the
// program's own operations are never contracted into fused multiply-adds,
// so each rounds on its own, as in the interpreter) the first time the
// module runs, and loaded once per device.
// The generated code evaluates the same fp32 expressions in the same order as
// the interpreter, so both give the same bits; a step whose kernel could not
// be built or whose buffers miss the assumed alignment runs the interpreter.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

namespace mi::jam {

struct Step;

constexpr int kEwJitBlock = 256;    // threads per block of every generated kernel
constexpr int kEwJitMaxBatch = 32;  // instances of one batched launch

// One generated kernel.
struct EwKernel {
  std::string name;       // entry: "ew_" + 16 hex digits of the code's hash [+ "_x<batch>"]
  std::string base;       // name of the single-instance entry
  std::string helpers;    // the program and one block's work as __device__ functions
  std::string source;     // helpers and the extern "C" __global__ entry
  uint32_t blocks = 0;    // grid of one instance (kEwJitBlock threads per block); 0: nothing to do
  int n_in = 0, n_out = 0;
  // 0: elementwise; 1: reduction of the program's value over trailing dims
  // (one launch); 2: sum over leading dims (this entry writes partial sums
  // of `chunks` row chunks, then `final_name` on `final_blocks` blocks adds them)
  int kind = 0;
  std::string final_name;
  uint32_t final_blocks = 0;
  int64_t chunks = 0;
  // 0: the entry takes the step's pointers; k >= 2: it takes a struct of k
  // instances' pointers (inputs p[k][t], outputs q[k][o]) and a grid of
  // instances x blocks, block b running block b % blocks of instance
  // b / blocks — independent steps of one shape in one launch
  int batch = 0;
  // per step buffer (inputs then outputs): byte alignment its resolved
  // pointer must have for the vector accesses the kernel makes (1: any)
  std::vector<uint8_t> align;
};

// Writes the kernel of ew step `s`; false with `why` when the step's encoding
// is outside what the generator handles (the step keeps the interpreter).
bool GenerateEwKernel(const Step& s, EwKernel* k, std::string* why);
// The kernel(s) of an ew reduce step (an ew program's value reduced without
// being stored).
bool GenerateEwReduceKernel(const Step& s, EwKernel* k, std::string* why);
// Workspace bytes of a sum over leading dims (rows summed, cols kept, inner
// the iteration space's innermost dim).
int64_t EwReduceWorkspaceBytes(int64_t rows, int64_t cols, int64_t inner);
// The batched entry (`batch` instances) of a single-instance kernel.
bool BatchEwKernel(const EwKernel& single, int batch, EwKernel* k);

// The generated kernels of one launch plan.  Identical kernels (same name)
// are kept once.  Compiled on first use; the code object is shared by every
// plan with the same set of kernels in this process and loaded once per
// device for the life of the process.
class EwJit {
 public:
  int Add(EwKernel k);  // returns the kernel's index
  size_t size() const { return kernels_.size(); }
  const EwKernel& kernel(int k) const { return kernels_[size_t(k)]; }

  // Compiles (once) without touching a device.  False when hiprtc failed;
  // error() says why.
  bool Build();
  // hipFunction_t handles, two per kernel (entry, final entry or null), on
  // the device `ordinal` (which must be current); compiles and loads on
  // first call.  Null on failure.
  void* const* Functions(int ordinal);
  std::string error() const;
  double compile_seconds() const { return compile_seconds_; }

  // Strict (env JAM_EW_JIT_STRICT, for tests): a step that would fall back
  // to the interpreter (kernels unavailable, a misaligned pointer) is an
  // error instead.
  bool strict = false;

  struct Code;  // a compiled code object and its per-device modules (shared)

 private:
  std::vector<EwKernel> kernels_;
  std::map<std::string, int> by_name_;
  mutable std::mutex mu_;
  bool built_ = false;
  std::string error_;
  double compile_seconds_ = 0;
  std::shared_ptr<Code> code_;
  std::vector<std::vector<void*>> fns_;  // per device ordinal
};

}  // namespace mi::jam
