#include "jam/ew_jit.h"

#include <hip/hip_runtime_api.h>
#include <dlfcn.h>
#include <hip/hiprtc.h>

#include <algorithm>
#include <array>
#include <chrono>
#include <cinttypes>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <sstream>
#include <type_traits>
#include <unordered_map>

#include "jam/program.h"
#include "mk_kernels.h"

namespace mi::jam {
namespace {

constexpr int kMaxRank = 6;
constexpr int kMaxRegs = 32;  // the interpreter's register file; programs are checked against it
constexpr int kMaxInputs = 8;
constexpr int kMaxOutputs = 4;
constexpr int kLanes = 4;     // consecutive elements per thread when the innermost dim allows

// Helpers every generated kernel uses.  The conversions are the kernel
// library's (mk_common.h): bf16 widening by shift, narrowing by the hardware
// RNE conversion of __bf16, f16 through _Float16; max / min propagate NaN.
// The f16 conversions pass their fp32 side through an empty asm so that the
// compiler cannot fold them with a neighbouring multiply into a mixed-
// precision FMA with a +0 addend (v_fma_mix), which turns a -0 product into
// +0; the interpreter converts separately, and so must these kernels.
const char kPreamble[] = R"(typedef float mkj_f4 __attribute__((ext_vector_type(4)));
typedef unsigned int mkj_u2 __attribute__((ext_vector_type(2)));
static __device__ __forceinline__ float mkj_f(int i) { return __builtin_bit_cast(float, i); }
static __device__ __forceinline__ float mkj_fu(unsigned u) { return __builtin_bit_cast(float, u); }
static __device__ __forceinline__ int mkj_i(float f) { return __builtin_bit_cast(int, f); }
static __device__ __forceinline__ float mkj_bf2f(unsigned short h) { return mkj_fu(unsigned(h) << 16); }
static __device__ __forceinline__ unsigned short mkj_f2bf(float f) { return __builtin_bit_cast(unsigned short, static_cast<__bf16>(f)); }
static __device__ __forceinline__ float mkj_h2f(unsigned short h) { float f = float(__builtin_bit_cast(_Float16, h)); asm("" : "+v"(f)); return f; }
static __device__ __forceinline__ unsigned short mkj_f2h(float f) { asm("" : "+v"(f)); return __builtin_bit_cast(unsigned short, static_cast<_Float16>(f)); }
static __device__ __forceinline__ float mkj_sign(float x) { return x > 0.f ? 1.f : (x < 0.f ? -1.f : x); }
static __device__ __forceinline__ float mkj_max(float x, float y) { return (x != x || y != y) ? __builtin_nanf("") : fmaxf(x, y); }
static __device__ __forceinline__ float mkj_min(float x, float y) { return (x != x || y != y) ? __builtin_nanf("") : fminf(x, y); }
static __device__ __forceinline__ int mkj_smax(int x, int y) { return x > y ? x : y; }
static __device__ __forceinline__ int mkj_smin(int x, int y) { return x < y ? x : y; }
)";

// Scalar load of element `o` of `p` into the register convention of the
// interpreter: float types widen to fp32, integer types hold their int32 bit
// pattern (64-bit truncated), predicates 0 / 1.
bool LoadExpr(int t, const std::string& p, const std::string& o, std::string* e) {
  auto at = [&](const char* ty) { return "((const " + std::string(ty) + "*)" + p + ")[" + o + "]"; };
  switch (t) {
    case MK_F32: *e = at("float"); return true;
    case MK_BF16: *e = "mkj_bf2f(" + at("unsigned short") + ")"; return true;
    case MK_F16: *e = "mkj_h2f(" + at("unsigned short") + ")"; return true;
    case MK_F64: *e = "float(" + at("double") + ")"; return true;
    case MK_PRED: *e = "(" + at("unsigned char") + " ? 1.f : 0.f)"; return true;
    case MK_S8: *e = "mkj_f(int(" + at("signed char") + "))"; return true;
    case MK_U8: *e = "mkj_f(int(" + at("unsigned char") + "))"; return true;
    case MK_S16: *e = "mkj_f(int(" + at("short") + "))"; return true;
    case MK_U16: *e = "mkj_f(int(" + at("unsigned short") + "))"; return true;
    case MK_S32: case MK_U32: *e = "mkj_f(" + at("int") + ")"; return true;
    case MK_S64: case MK_U64: *e = "mkj_f(int(" + at("long long") + "))"; return true;
    default: return false;
  }
}

// Store of fp32 register value `v` as element `o` of `q` (the interpreter's
// ew_store).
bool StoreStmt(int t, const std::string& q, const std::string& o, const std::string& v, std::string* s) {
  auto at = [&](const char* ty) { return "((" + std::string(ty) + "*)" + q + ")[" + o + "] = "; };
  switch (t) {
    case MK_F32: *s = at("float") + v + ";"; return true;
    case MK_BF16: *s = at("unsigned short") + "mkj_f2bf(" + v + ");"; return true;
    case MK_F16: *s = at("unsigned short") + "mkj_f2h(" + v + ");"; return true;
    case MK_F64: *s = at("double") + "double(" + v + ");"; return true;
    case MK_PRED: *s = at("unsigned char") + "(" + v + " != 0.f);"; return true;
    case MK_S8: case MK_U8: *s = at("unsigned char") + "(unsigned char)mkj_i(" + v + ");"; return true;
    case MK_S16: case MK_U16: *s = at("unsigned short") + "(unsigned short)mkj_i(" + v + ");"; return true;
    case MK_S32: case MK_U32: *s = at("int") + "mkj_i(" + v + ");"; return true;
    case MK_S64: *s = at("long long") + "(long long)mkj_i(" + v + ");"; return true;
    case MK_U64: *s = at("unsigned long long") + "(unsigned long long)(unsigned)mkj_i(" + v + ");"; return true;
    default: return false;
  }
}

std::string FloatLit(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  char b[32];
  snprintf(b, sizeof b, "mkj_fu(0x%08xu)", u);
  return b;
}

// The fp32 expression of one instruction (the interpreter's ew_run case for
// its opcode) over operand names a, b, c.  Integer arithmetic wraps through
// unsigned, which is what the interpreter's int32 operations compile to.
bool InstrExpr(int op, const std::string& a, const std::string& b, const std::string& c, std::string* e) {
  auto cmp = [&](const char* rel) { return "(" + a + " " + rel + " " + b + " ? 1.f : 0.f)"; };
  auto icmp = [&](const char* rel) { return "(mkj_i(" + a + ") " + rel + " mkj_i(" + b + ") ? 1.f : 0.f)"; };
  auto iop = [&](const char* o) {
    return "mkj_f(int(unsigned(mkj_i(" + a + ")) " + o + " unsigned(mkj_i(" + b + "))))";
  };
  switch (op) {
    case MK_EW_ADD: *e = "(" + a + " + " + b + ")"; return true;
    case MK_EW_SUB: *e = "(" + a + " - " + b + ")"; return true;
    case MK_EW_MUL: *e = "(" + a + " * " + b + ")"; return true;
    case MK_EW_DIV: *e = "(" + a + " / " + b + ")"; return true;
    case MK_EW_MAX: *e = "mkj_max(" + a + ", " + b + ")"; return true;
    case MK_EW_MIN: *e = "mkj_min(" + a + ", " + b + ")"; return true;
    case MK_EW_POW: *e = "powf(" + a + ", " + b + ")"; return true;
    case MK_EW_NEG: *e = "(-" + a + ")"; return true;
    case MK_EW_EXP: *e = "expf(" + a + ")"; return true;
    case MK_EW_LOG: *e = "logf(" + a + ")"; return true;
    case MK_EW_TANH: *e = "tanhf(" + a + ")"; return true;
    case MK_EW_SQRT: *e = "sqrtf(" + a + ")"; return true;
    case MK_EW_RSQRT: *e = "(1.f / sqrtf(" + a + "))"; return true;
    case MK_EW_ABS: *e = "fabsf(" + a + ")"; return true;
    case MK_EW_LOGISTIC: *e = "(1.f / (1.f + expf(-" + a + ")))"; return true;
    case MK_EW_CMP_EQ: *e = cmp("=="); return true;
    case MK_EW_CMP_NE: *e = cmp("!="); return true;
    case MK_EW_CMP_LT: *e = cmp("<"); return true;
    case MK_EW_CMP_LE: *e = cmp("<="); return true;
    case MK_EW_CMP_GT: *e = cmp(">"); return true;
    case MK_EW_CMP_GE: *e = cmp(">="); return true;
    case MK_EW_SELECT: *e = "(" + a + " != 0.f ? " + b + " : " + c + ")"; return true;
    case MK_EW_CLAMP: *e = "fminf(fmaxf(" + a + ", " + b + "), " + c + ")"; return true;
    case MK_EW_ROUND_BF16: *e = "mkj_bf2f(mkj_f2bf(" + a + "))"; return true;
    case MK_EW_ROUND_F16: *e = "mkj_h2f(mkj_f2h(" + a + "))"; return true;
    case MK_EW_FLOOR: *e = "floorf(" + a + ")"; return true;
    case MK_EW_CEIL: *e = "ceilf(" + a + ")"; return true;
    case MK_EW_SIGN: *e = "mkj_sign(" + a + ")"; return true;
    case MK_EW_AND: *e = "((" + a + " != 0.f && " + b + " != 0.f) ? 1.f : 0.f)"; return true;
    case MK_EW_OR: *e = "((" + a + " != 0.f || " + b + " != 0.f) ? 1.f : 0.f)"; return true;
    case MK_EW_NOT: *e = "(" + a + " == 0.f ? 1.f : 0.f)"; return true;
    case MK_EW_MOV: *e = a; return true;
    case MK_EW_CMP_LT_S32: *e = icmp("<"); return true;
    case MK_EW_CMP_GE_S32: *e = icmp(">="); return true;
    case MK_EW_ADD_S32: *e = iop("+"); return true;
    case MK_EW_SUB_S32: *e = iop("-"); return true;
    case MK_EW_MUL_S32: *e = iop("*"); return true;
    case MK_EW_S32_TO_F32: *e = "float(mkj_i(" + a + "))"; return true;
    case MK_EW_F32_TO_S32: *e = "mkj_f(int(" + a + "))"; return true;
    case MK_EW_ERF: *e = "erff(" + a + ")"; return true;
    case MK_EW_CMP_EQ_S32: *e = icmp("=="); return true;
    case MK_EW_CMP_NE_S32: *e = icmp("!="); return true;
    case MK_EW_CMP_LE_S32: *e = icmp("<="); return true;
    case MK_EW_CMP_GT_S32: *e = icmp(">"); return true;
    case MK_EW_MAX_S32: *e = "mkj_f(mkj_smax(mkj_i(" + a + "), mkj_i(" + b + ")))"; return true;
    case MK_EW_MIN_S32: *e = "mkj_f(mkj_smin(mkj_i(" + a + "), mkj_i(" + b + ")))"; return true;
    case MK_EW_NEG_S32: *e = "mkj_f(int(0u - unsigned(mkj_i(" + a + "))))"; return true;
    case MK_EW_AND_B32: *e = "mkj_f(mkj_i(" + a + ") & mkj_i(" + b + "))"; return true;
    case MK_EW_OR_B32: *e = "mkj_f(mkj_i(" + a + ") | mkj_i(" + b + "))"; return true;
    case MK_EW_XOR_B32: *e = "mkj_f(mkj_i(" + a + ") ^ mkj_i(" + b + "))"; return true;
    case MK_EW_PRED_TO_S32: *e = "mkj_f(" + a + " != 0.f ? 1 : 0)"; return true;
    case MK_EW_S32_TO_PRED: *e = "(mkj_i(" + a + ") != 0 ? 1.f : 0.f)"; return true;
    case MK_EW_U32_TO_F32: *e = "float(unsigned(mkj_i(" + a + ")))"; return true;
    default: return false;
  }
}

uint64_t Fnv1a(const std::string& s) {
  uint64_t h = 1469598103934665603ull;
  for (unsigned char c : s) {
    h ^= c;
    h *= 1099511628211ull;
  }
  return h;
}

void ReplaceAll(std::string& s, const std::string& from, const std::string& to) {
  for (size_t p = s.find(from); p != std::string::npos; p = s.find(from, p + to.size())) s.replace(p, from.size(), to);
}

}  // namespace

namespace {

// The iteration space of a program and how each input is read in it (the
// interpreter's modes; size-1 dims never contribute).
enum Mode { kScalarIn, kDenseIn, kStridedIn };
struct IterSpace {
  int rank = 0;
  int64_t dims[kMaxRank] = {};
  int64_t n = 1;
  int n_in = 0;
  std::vector<Mode> mode;
  std::vector<std::array<int64_t, kMaxRank>> st;
  std::vector<int> types;
  bool narrow = true;  // every index and offset fits 32 bits
};

bool Analyze(int rank, const int64_t* dims, int n_in, const std::vector<int64_t>& strides,
             const std::vector<int32_t>& types, IterSpace* sp, std::string* why) {
  if (rank < 0 || rank > kMaxRank) return (*why = "rank", false);
  if (n_in < 0 || n_in > kMaxInputs) return (*why = "operand count", false);
  if (strides.size() != size_t(kMaxRank * n_in) || types.size() != size_t(n_in))
    return (*why = "malformed step", false);
  sp->rank = rank;
  sp->n = 1;
  for (int d = 0; d < rank; ++d) {
    if (dims[d] < 0) return (*why = "negative dim", false);
    sp->dims[d] = dims[d];
    sp->n *= dims[d];
  }
  sp->n_in = n_in;
  sp->narrow = rank >= 1 && sp->n < (int64_t(1) << 31);
  sp->mode.assign(size_t(n_in), kScalarIn);
  sp->st.assign(size_t(n_in), {});
  sp->types.assign(types.begin(), types.end());
  for (int t = 0; t < n_in; ++t) {
    int64_t expect = 1, hi = 0;
    bool dense = true, scalar = true;
    for (int d = rank - 1; d >= 0; --d) {
      const int64_t v = dims[d] == 1 ? 0 : strides[size_t(t * kMaxRank + d)];
      sp->st[size_t(t)][size_t(d)] = v;
      if (dims[d] != 1 && v != expect) dense = false;
      if (dims[d] != 1 && v != 0) scalar = false;
      if (v < 0) sp->narrow = false;
      hi += (dims[d] - 1) * v;
      expect *= dims[d];
    }
    if (hi >= (int64_t(1) << 31) - kLanes) sp->narrow = false;
    sp->mode[size_t(t)] = scalar ? kScalarIn : (dense ? kDenseIn : kStridedIn);
    std::string probe;
    if (!LoadExpr(types[size_t(t)], "p", "0", &probe)) return (*why = "input dtype", false);
  }
  return true;
}

// The program as a straight-line __device__ function of one element's
// inputs x0.. writing the registers `out_regs` to y[0..].
bool BodyFn(const std::vector<int32_t>& prog, const std::vector<float>& consts, int n_in,
            const std::vector<int>& out_regs, std::ostringstream& src, std::string* why) {
  if (prog.size() % 4 != 0) return (*why = "malformed program", false);
  std::string reg[kMaxRegs];
  for (int r = 0; r < kMaxRegs; ++r) reg[r] = r < n_in ? "x" + std::to_string(r) : "0.f";
  src << "static __device__ __forceinline__ void @K@_body(";
  for (int t = 0; t < n_in; ++t) src << "float x" << t << ", ";
  src << "float* y) {\n#pragma clang fp contract(off)\n";
  for (size_t p = 0; p < prog.size() / 4; ++p) {
    const int op = prog[4 * p], dst = prog[4 * p + 1], a = prog[4 * p + 2], b = prog[4 * p + 3];
    if (dst < 0 || dst >= kMaxRegs) return (*why = "destination register", false);
    std::string e;
    if (op == MK_EW_CONST) {
      if (a < 0 || size_t(a) >= consts.size()) return (*why = "constant index", false);
      e = FloatLit(consts[size_t(a)]);
    } else {
      const int rb = b & 0xffff, rc = (b >> 16) & 0xffff;
      if (a < 0 || a >= kMaxRegs || rb >= kMaxRegs || rc >= kMaxRegs) return (*why = "source register", false);
      if (!InstrExpr(op, reg[a], reg[rb], reg[rc], &e)) return (*why = "opcode " + std::to_string(op), false);
    }
    src << "  const float v" << p << " = " << e << ";\n";
    reg[dst] = "v" + std::to_string(p);
  }
  for (size_t o = 0; o < out_regs.size(); ++o) {
    if (out_regs[o] < 0 || out_regs[o] >= kMaxRegs) return (*why = "output register", false);
    src << "  y[" << o << "] = " << reg[out_regs[o]] << ";\n";
  }
  src << "}\n";
  return true;
}

// Index decomposition of the linear element index `i0` (lanes consecutive
// elements per thread: the innermost dim is a multiple of lanes) and the
// loads of every input; x[t][l] names input t's fp32 value in lane l.  Vector
// loads (4 consecutive f32 / bf16 elements, unit inner stride, the other
// strides multiples of 4) record the byte alignment the input's pointer
// needs in align[t].
void EmitLoads(const IterSpace& sp, int lanes, const std::string& i0, const std::string& ind,
               std::ostringstream& src, std::vector<std::array<std::string, kLanes>>* x,
               std::vector<uint8_t>* align) {
  const std::string IT = sp.narrow ? "unsigned" : "long long";
  const std::string U = sp.narrow ? "u" : "ll";
  const int rank = sp.rank;
  // multi-dim index: only as far out as some strided input needs
  int lo = rank;
  for (int t = 0; t < sp.n_in; ++t)
    if (sp.mode[size_t(t)] == kStridedIn)
      for (int d = 0; d < rank; ++d)
        if (sp.st[size_t(t)][size_t(d)] != 0) lo = std::min(lo, d);
  if (lo < rank) {
    src << ind << IT << " r_ = " << i0 << ";\n";
    for (int d = rank - 1; d >= lo; --d) {
      if (d == 0) {
        src << ind << "const " << IT << " d0 = r_;\n";
      } else {
        src << ind << "const " << IT << " d" << d << " = r_ % " << sp.dims[d] << U << ";\n";
        if (d > lo) src << ind << "r_ /= " << sp.dims[d] << U << ";\n";
      }
    }
  }
  x->assign(size_t(sp.n_in), {});
  for (int t = 0; t < sp.n_in; ++t) {
    const int ty = sp.types[size_t(t)];
    const std::string p = "p" + std::to_string(t), tn = std::to_string(t);
    std::string off, e;
    int64_t step = 0;
    if (sp.mode[size_t(t)] == kScalarIn) {
      LoadExpr(ty, p, "0", &e);
      src << ind << "const float x" << tn << " = " << e << ";\n";
      for (int l = 0; l < lanes; ++l) (*x)[size_t(t)][size_t(l)] = "x" + tn;
      continue;
    }
    if (sp.mode[size_t(t)] == kDenseIn) {
      off = i0;
      step = 1;
    } else {
      std::string sum;
      for (int d = lo; d < rank; ++d) {
        const int64_t v = sp.st[size_t(t)][size_t(d)];
        if (v == 0) continue;
        sum += (sum.empty() ? "" : " + ") + std::string("d") + std::to_string(d) +
               (v == 1 ? "" : " * " + std::to_string(v) + U);
      }
      src << ind << "const " << IT << " o" << tn << " = " << sum << ";\n";
      off = "o" + tn;
      step = sp.st[size_t(t)][size_t(rank - 1)];
    }
    bool vec = lanes == kLanes && step == 1 && (ty == MK_F32 || ty == MK_BF16);
    for (int d = 0; vec && d + 1 < rank; ++d)
      if (sp.st[size_t(t)][size_t(d)] % kLanes != 0) vec = false;
    if (vec && ty == MK_F32) {
      src << ind << "const mkj_f4 w" << tn << " = *(const mkj_f4*)((const float*)" << p << " + " << off << ");\n";
      for (int l = 0; l < lanes; ++l) (*x)[size_t(t)][size_t(l)] = "w" + tn + "[" + std::to_string(l) + "]";
      (*align)[size_t(t)] = 16;
    } else if (vec) {
      src << ind << "const mkj_u2 w" << tn << " = *(const mkj_u2*)((const unsigned short*)" << p << " + " << off
          << ");\n";
      for (int l = 0; l < lanes; ++l) {
        src << ind << "const float x" << tn << "_" << l << " = mkj_bf2f((unsigned short)(w" << tn << "[" << l / 2
            << "]" << (l % 2 ? " >> 16" : "") << "));\n";
        (*x)[size_t(t)][size_t(l)] = "x" + tn + "_" + std::to_string(l);
      }
      (*align)[size_t(t)] = 8;
    } else if (step == 0 || lanes == 1) {
      LoadExpr(ty, p, off, &e);
      src << ind << "const float x" << tn << " = " << e << ";\n";
      for (int l = 0; l < lanes; ++l) (*x)[size_t(t)][size_t(l)] = "x" + tn;
    } else {
      for (int l = 0; l < lanes; ++l) {
        const std::string ol = l == 0 ? off : "(" + off + " + " + std::to_string(int64_t(l) * step) + U + ")";
        LoadExpr(ty, p, ol, &e);
        src << ind << "const float x" << tn << "_" << l << " = " << e << ";\n";
        (*x)[size_t(t)][size_t(l)] = "x" + tn + "_" + std::to_string(l);
      }
    }
  }
}

// Names the kernel by its text's hash and fills the entry fields.
void Finish(std::string helpers, std::string entry, EwKernel* k) {
  char name[32];
  snprintf(name, sizeof name, "ew_%016" PRIx64, Fnv1a(helpers + entry));
  ReplaceAll(helpers, "@K@", name);
  ReplaceAll(entry, "@K@", name);
  k->name = name;
  k->base = name;
  k->helpers = std::move(helpers);
  k->source = k->helpers + entry;
}

// fp32 value rounded to the type a materialized value would have
std::string RoundTo(int type, const std::string& v) {
  if (type == MK_BF16) return "mkj_bf2f(mkj_f2bf(" + v + "))";
  if (type == MK_F16) return "mkj_h2f(mkj_f2h(" + v + "))";
  return v;
}

// Row chunks of a sum over leading dims: enough blocks (tiles x chunks)
// to fill the chip, at most 512 chunks, every chunk non-empty.
int64_t ReduceChunks(int64_t rows, int64_t tiles) {
  int64_t chunks = std::max<int64_t>(1, std::min<int64_t>({rows, (1024 + tiles - 1) / tiles, int64_t(512)}));
  const int64_t rpc = (rows + chunks - 1) / chunks;
  return (rows + rpc - 1) / rpc;
}

std::string Combine(int rop, const std::string& a, const std::string& b) {
  switch (rop) {
    case 0: return "(" + a + " + " + b + ")";
    case 1: return "fmaxf(" + a + ", " + b + ")";
    case 2: return "fminf(" + a + ", " + b + ")";
    default: return "(" + a + " * " + b + ")";
  }
}

}  // namespace

// Step encoding (lower.cc EmitEwGroup): bufs = inputs then outputs; i = rank,
// dims[6], n_inputs, (out_reg, out_type) per output; prog 4 ints per
// instruction; strides 6 per input; types per input; f = constants.
bool GenerateEwKernel(const Step& s, EwKernel* k, std::string* why) {
  if (s.kind == StepKind::kEwReduce) return GenerateEwReduceKernel(s, k, why);
  if (s.kind != StepKind::kEw || s.i.size() < 8) return (*why = "not an ew step", false);
  const int rank = int(s.i[0]);
  const int n_in = int(s.i[7]);
  const int n_out = int(s.bufs.size()) - n_in;
  if (n_out < 1 || n_out > kMaxOutputs || s.i.size() != size_t(8 + 2 * n_out)) return (*why = "operand count", false);
  IterSpace sp;
  if (rank < 0 || rank > kMaxRank || !Analyze(rank, &s.i[1], n_in, s.strides, s.types, &sp, why)) return false;
  k->align.assign(s.bufs.size(), 1);
  if (sp.n == 0) {
    k->blocks = 0;
    k->name.clear();
    k->source.clear();
    return true;
  }
  std::vector<int> out_reg(static_cast<size_t>(n_out)), out_type(static_cast<size_t>(n_out));
  for (int o = 0; o < n_out; ++o) {
    out_reg[size_t(o)] = int(s.i[8 + 2 * size_t(o)]);
    out_type[size_t(o)] = int(s.i[9 + 2 * size_t(o)]);
    std::string probe;
    if (!StoreStmt(out_type[size_t(o)], "q", "0", "v", &probe)) return (*why = "output dtype", false);
  }
  const int lanes = rank >= 1 && sp.dims[rank - 1] % kLanes == 0 ? kLanes : 1;
  const int64_t blocks = (sp.n / lanes + kEwJitBlock - 1) / kEwJitBlock;
  if (blocks >= (int64_t(1) << 31)) return (*why = "grid too large", false);
  const std::string U = sp.narrow ? "u" : "ll";

  std::ostringstream src;
  src << "#ifndef @K@_DEF\n#define @K@_DEF\n";
  if (!BodyFn(s.prog, s.f, n_in, out_reg, src, why)) return false;
  // one block's work (block blk of the step's grid)
  std::string params;
  for (int t = 0; t < n_in; ++t) params += "const void* p" + std::to_string(t) + ", ";
  for (int o = 0; o < n_out; ++o) params += "void* q" + std::to_string(o) + (o + 1 < n_out ? ", " : "");
  src << "static __device__ __forceinline__ void @K@_run(unsigned blk, " << params << ") {\n";
  if (sp.narrow)
    src << "  const unsigned i0 = (blk * " << kEwJitBlock << "u + threadIdx.x) * " << lanes << "u;\n";
  else
    src << "  const long long i0 = ((long long)blk * " << kEwJitBlock << " + threadIdx.x) * " << lanes << ";\n";
  src << "  if (i0 >= " << sp.n << U << ") return;\n";
  std::vector<std::array<std::string, kLanes>> x;
  EmitLoads(sp, lanes, "i0", "  ", src, &x, &k->align);
  for (int l = 0; l < lanes; ++l) {
    src << "  float y" << l << "[" << n_out << "];\n  @K@_body(";
    for (int t = 0; t < n_in; ++t) src << x[size_t(t)][size_t(l)] << ", ";
    src << "y" << l << ");\n";
  }
  for (int o = 0; o < n_out; ++o) {
    const int ty = out_type[size_t(o)];
    const std::string q = "q" + std::to_string(o);
    auto y = [&](int l) { return "y" + std::to_string(l) + "[" + std::to_string(o) + "]"; };
    if (lanes == kLanes && ty == MK_F32) {
      src << "  *(mkj_f4*)((float*)" << q << " + i0) = mkj_f4{" << y(0) << ", " << y(1) << ", " << y(2) << ", "
          << y(3) << "};\n";
      k->align[size_t(n_in + o)] = 16;
    } else if (lanes == kLanes && ty == MK_BF16) {
      src << "  *(mkj_u2*)((unsigned short*)" << q << " + i0) = mkj_u2{unsigned(mkj_f2bf(" << y(0)
          << ")) | (unsigned(mkj_f2bf(" << y(1) << ")) << 16), unsigned(mkj_f2bf(" << y(2)
          << ")) | (unsigned(mkj_f2bf(" << y(3) << ")) << 16)};\n";
      k->align[size_t(n_in + o)] = 8;
    } else {
      for (int l = 0; l < lanes; ++l) {
        std::string stmt;
        StoreStmt(ty, q, l == 0 ? "i0" : "i0 + " + std::to_string(l), y(l), &stmt);
        src << "  " << stmt << "\n";
      }
    }
  }
  src << "}\n#endif\n";
  std::string args;
  for (int t = 0; t < n_in; ++t) args += ", p" + std::to_string(t);
  for (int o = 0; o < n_out; ++o) args += ", q" + std::to_string(o);
  const std::string entry = "extern \"C\" __global__ void __launch_bounds__(" + std::to_string(kEwJitBlock) +
                            ") @K@(" + params + ") { @K@_run(blockIdx.x" + args + "); }\n";
  Finish(src.str(), entry, k);
  k->kind = 0;
  k->blocks = uint32_t(blocks);
  k->n_in = n_in;
  k->n_out = n_out;
  k->batch = 0;
  return true;
}

// Reduction of an ew program's value (lower.cc LowerReduce): bufs = inputs,
// out, tmp, ws; i = rank, dims[6] (the iteration space), n_inputs, out_reg,
// val_type, out_type, rop, rows, cols, mode, init bits.  Mode 0 reduces the
// trailing dims (rows = kept elements, cols = reduced per row), one wave per
// row; mode 1 sums the leading dims (rows = reduced, cols = kept), partial
// sums of row chunks into ws, then a second kernel adds the chunks.  The
// value is rounded to val_type before it is combined, as the materialized
// value would be.  i[16] set: the value is also stored, densely in the
// iteration order, into a fourth buffer (the value's own, or its bf16 copy;
// the lowering only asks for it when that order is the value's layout).
bool GenerateEwReduceKernel(const Step& s, EwKernel* k, std::string* why) {
  if (s.kind != StepKind::kEwReduce || s.i.size() != 17) return (*why = "not an ew reduce step", false);
  // i[16]: the value is also stored, densely in iteration order, into the
  // step's fourth buffer: 1 in val_type, 2 rounded to bf16 (its readers'
  // narrow copy)
  const bool store = s.i[16] != 0;
  const int rank = int(s.i[0]), n_in = int(s.i[7]), out_reg = int(s.i[8]), val_type = int(s.i[9]),
            out_type = int(s.i[10]), rop = int(s.i[11]), mode = int(s.i[14]);
  const int64_t rows = s.i[12], cols = s.i[13];
  const int store_type = s.i[16] == 2 ? MK_BF16 : val_type;
  uint32_t init_bits = uint32_t(s.i[15]);
  float init;
  memcpy(&init, &init_bits, 4);
  if (s.bufs.size() != size_t(n_in + (store ? 4 : 3))) return (*why = "malformed ew reduce step", false);
  IterSpace sp;
  if (rank < 1 || rank > kMaxRank || !Analyze(rank, &s.i[1], n_in, s.strides, s.types, &sp, why)) return false;
  if (rows * cols != sp.n || rows <= 0 || cols <= 0) return (*why = "empty or inconsistent reduction", false);
  if (rop < 0 || rop > 3 || (mode == 1 && (rop != 0 || out_type != MK_F32))) return (*why = "reduction kind", false);
  if (val_type != MK_F32 && val_type != MK_BF16 && val_type != MK_F16) return (*why = "value type", false);
  std::string probe;
  if (!StoreStmt(out_type, "q", "0", "v", &probe)) return (*why = "output dtype", false);
  k->align.assign(s.bufs.size(), 1);
  const int lanes = sp.dims[rank - 1] % kLanes == 0 && cols % kLanes == 0 ? kLanes : 1;
  const std::string IT = sp.narrow ? "unsigned" : "long long";
  const std::string U = sp.narrow ? "u" : "ll";
  static const char* kIdentity[] = {"0.f", "-__builtin_inff()", "__builtin_inff()", "1.f"};

  std::ostringstream src;
  src << "#ifndef @K@_DEF\n#define @K@_DEF\n";
  if (!BodyFn(s.prog, s.f, n_in, {out_reg}, src, why)) return false;
  src << "#endif\n";
  std::string params;
  for (int t = 0; t < n_in; ++t) params += "const void* p" + std::to_string(t) + ", ";
  const std::string sparam = store ? ", void* qs" : "";
  std::ostringstream e;
  // per element: loads, the program, rounding, combine into the lane's acc
  // (and the stored copy of the value)
  auto element = [&](const std::string& i0, const std::string& ind, const std::string& acc, bool per_lane) {
    std::vector<std::array<std::string, kLanes>> x;
    e << ind << "{\n";
    EmitLoads(sp, lanes, i0, ind + "  ", e, &x, &k->align);
    for (int l = 0; l < lanes; ++l) {
      e << ind << "  float y" << l << "[1];\n" << ind << "  @K@_body(";
      for (int t = 0; t < n_in; ++t) e << x[size_t(t)][size_t(l)] << ", ";
      e << "y" << l << ");\n";
      const std::string v = RoundTo(val_type, "y" + std::to_string(l) + "[0]");
      const std::string a = per_lane ? acc + "[" + std::to_string(l) + "]" : acc;
      e << ind << "  { const float v = " << v << ";";
      if (rop == 1 || rop == 2) e << " nan_ |= v != v;";
      e << " " << a << " = " << Combine(rop, a, "v") << "; }\n";
    }
    if (store) {
      auto y = [&](int l) { return "y" + std::to_string(l) + "[0]"; };
      if (lanes == kLanes && store_type == MK_F32) {
        e << ind << "  *(mkj_f4*)((float*)qs + " << i0 << ") = mkj_f4{" << y(0) << ", " << y(1) << ", " << y(2)
          << ", " << y(3) << "};\n";
        k->align[size_t(n_in + 3)] = 16;
      } else if (lanes == kLanes && store_type == MK_BF16) {
        e << ind << "  *(mkj_u2*)((unsigned short*)qs + " << i0 << ") = mkj_u2{unsigned(mkj_f2bf(" << y(0)
          << ")) | (unsigned(mkj_f2bf(" << y(1) << ")) << 16), unsigned(mkj_f2bf(" << y(2)
          << ")) | (unsigned(mkj_f2bf(" << y(3) << ")) << 16)};\n";
        k->align[size_t(n_in + 3)] = 8;
      } else {
        for (int l = 0; l < lanes; ++l) {
          std::string stmt;
          StoreStmt(store_type, "qs", l == 0 ? i0 : i0 + " + " + std::to_string(l), y(l), &stmt);
          e << ind << "  " << stmt << "\n";
        }
      }
    }
    e << ind << "}\n";
  };
  if (mode == 0) {
    // one wave per row, lanes x 64 columns per iteration
    e << "extern \"C\" __global__ void __launch_bounds__(" << kEwJitBlock << ") @K@(" << params << "void* q0" << sparam
      << ") {\n";
    e << "#pragma clang fp contract(off)\n  const unsigned lane = threadIdx.x & 63u;\n";
    e << "  const " << IT << " row = (" << IT << ")blockIdx.x * " << kEwJitBlock / 64 << " + (threadIdx.x >> 6);\n";
    e << "  if (row >= " << rows << U << ") return;\n";
    e << "  float acc = " << kIdentity[rop] << ";\n  bool nan_ = false;\n";
    e << "  for (" << IT << " c = lane * " << lanes << U << "; c < " << cols << U << "; c += " << 64 * lanes << U
      << ") {\n";
    e << "    const " << IT << " i0 = row * " << cols << U << " + c;\n";
    element("i0", "    ", "acc", false);
    e << "  }\n";
    for (int m = 32; m >= 1; m /= 2) e << "  acc = " << Combine(rop, "acc", "__shfl_xor(acc, " + std::to_string(m) + ")") << ";\n";
    e << "  const bool any_nan = __any(nan_);\n  (void)any_nan;\n";
    e << "  if (lane == 0) {\n    float r = " << Combine(rop, "acc", FloatLit(init)) << ";\n";
    if (rop == 1 || rop == 2) e << "    if (any_nan || " << (init != init ? "true" : "false") << ") r = __builtin_nanf(\"\");\n";
    std::string stmt;
    StoreStmt(out_type, "q0", "row", "r", &stmt);
    e << "    " << stmt << "\n  }\n}\n";
    k->blocks = uint32_t((rows + kEwJitBlock / 64 - 1) / (kEwJitBlock / 64));
    k->kind = 1;
    k->chunks = 0;
  } else {
    // column tiles of 64 x lanes columns; row chunks; 4 waves per block
    // take every 4th row of the chunk; partial sums to ws[chunk][col]
    const int64_t tile_cols = 64 * lanes;
    const int64_t tiles = (cols + tile_cols - 1) / tile_cols;
    const int64_t chunks = ReduceChunks(rows, tiles);
    const int64_t rpc = (rows + chunks - 1) / chunks;
    if (tiles * chunks >= (int64_t(1) << 31)) return (*why = "grid too large", false);
    e << "extern \"C\" __global__ void __launch_bounds__(" << kEwJitBlock << ") @K@(" << params << "float* ws" << sparam
      << ") {\n";
    e << "#pragma clang fp contract(off)\n  const unsigned lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;\n";
    e << "  const unsigned tile = blockIdx.x % " << tiles << "u, chunk = blockIdx.x / " << tiles << "u;\n";
    e << "  const " << IT << " c = (" << IT << ")tile * " << tile_cols << U << " + lane * " << lanes << U << ";\n";
    e << "  float acc[" << lanes << "] = {};\n  bool nan_ = false;\n  (void)nan_;\n";
    e << "  if (c < " << cols << U << ") {\n";
    e << "    const " << IT << " r1 = (" << IT << ")(chunk + 1) * " << rpc << U << " < " << rows << U << " ? (" << IT
      << ")(chunk + 1) * " << rpc << U << " : " << rows << U << ";\n";
    e << "    for (" << IT << " r = (" << IT << ")chunk * " << rpc << U << " + wave; r < r1; r += 4) {\n";
    e << "      const " << IT << " i0 = r * " << cols << U << " + c;\n";
    element("i0", "      ", "acc", true);
    e << "    }\n  }\n";
    e << "  __shared__ float red_[4][" << tile_cols << "];\n";
    for (int l = 0; l < lanes; ++l) e << "  red_[wave][lane * " << lanes << " + " << l << "] = acc[" << l << "];\n";
    e << "  __syncthreads();\n";
    e << "  if (wave == 0 && c < " << cols << U << ") {\n";
    for (int l = 0; l < lanes; ++l)
      e << "    ws[(" << IT << ")chunk * " << cols << U << " + c + " << l << "] = ((red_[0][lane * " << lanes << " + "
        << l << "] + red_[1][lane * " << lanes << " + " << l << "]) + red_[2][lane * " << lanes << " + " << l
        << "]) + red_[3][lane * " << lanes << " + " << l << "];\n";
    e << "  }\n}\n";
    // the chunks' partial sums: 16 columns per block, 16 threads per
    // column adding chunks g, g + 16, ..., then their 16 totals in order
    e << "extern \"C\" __global__ void __launch_bounds__(" << kEwJitBlock << ") @K@_final(const float* ws, void* q0) {\n";
    e << "#pragma clang fp contract(off)\n";
    e << "  const unsigned t = threadIdx.x & 15u, g = threadIdx.x >> 4;\n";
    e << "  const " << IT << " c = (" << IT << ")blockIdx.x * 16" << U << " + t;\n";
    e << "  float s = 0.f;\n";
    e << "  if (c < " << cols << U << ") {\n#pragma unroll 4\n";
    e << "    for (" << IT << " j = g; j < " << chunks << U << "; j += 16) s += ws[j * " << cols << U << " + c];\n  }\n";
    e << "  __shared__ float part_[16][16];\n  part_[g][t] = s;\n  __syncthreads();\n";
    e << "  if (g != 0 || c >= " << cols << U << ") return;\n";
    e << "  s = part_[0][t];\n  for (int k = 1; k < 16; ++k) s += part_[k][t];\n";
    e << "  s = s + " << FloatLit(init) << ";\n";
    std::string stmt;
    StoreStmt(out_type, "q0", "c", "s", &stmt);
    e << "  " << stmt << "\n}\n";
    k->blocks = uint32_t(tiles * chunks);
    k->final_blocks = uint32_t((cols + 15) / 16);
    k->kind = 2;
    k->chunks = chunks;
  }
  Finish(src.str(), e.str(), k);
  if (k->kind == 2) k->final_name = k->name + "_final";
  k->n_in = n_in;
  k->n_out = 1;
  k->batch = 0;
  return true;
}

int64_t EwReduceWorkspaceBytes(int64_t rows, int64_t cols, int64_t inner) {
  const int lanes = inner % kLanes == 0 && cols % kLanes == 0 ? kLanes : 1;
  const int64_t tile_cols = 64 * lanes;
  return ReduceChunks(rows, (cols + tile_cols - 1) / tile_cols) * cols * 4;
}

bool BatchEwKernel(const EwKernel& single, int batch, EwKernel* k) {
  if (single.kind != 0 || single.batch != 0 || batch < 2 || batch > kEwJitMaxBatch) return false;
  if (int64_t(single.blocks) * batch >= (int64_t(1) << 31)) return false;
  *k = single;
  k->batch = batch;
  k->name = single.base + "_x" + std::to_string(batch);
  const int pi = std::max(single.n_in, 1);
  std::ostringstream e;
  // the instances' pointers by value: p[k][t] inputs, q[k][o] outputs
  e << "struct " << k->name << "_args { const void* p[" << batch << "][" << pi << "]; void* q[" << batch << "]["
    << single.n_out << "]; };\n";
  e << "extern \"C\" __global__ void __launch_bounds__(" << kEwJitBlock << ") " << k->name << "(const " << k->name
    << "_args a) {\n  const unsigned k = blockIdx.x / " << single.blocks << "u, blk = blockIdx.x - k * "
    << single.blocks << "u;\n  " << single.base << "_run(blk";
  for (int t = 0; t < single.n_in; ++t) e << ", a.p[k][" << t << "]";
  for (int o = 0; o < single.n_out; ++o) e << ", a.q[k][" << o << "]";
  e << ");\n}\n";
  k->source = single.helpers + e.str();
  return true;
}

// ------------------------------------------------------------------ compile / load
struct EwJit::Code {
  std::vector<char> bin;
  std::string error;
  double seconds = 0;
  std::mutex mu;
  std::vector<hipModule_t> modules;  // per device ordinal (null: not loaded)
};

namespace {

// The runtime compiler, loaded from the ROCm installation ($ROCM_PATH, else
// /opt/rocm) into a link namespace of its own: a process may already hold
// another ROCm's hiprtc / comgr under the same sonames (PyTorch wheels bundle
// theirs), and the generated kernels must come from the compiler that built
// the kernel library, whose math routines they share bit for bit.  When that
// fails, the hiprtc the process resolves by name is used.
struct Rtc {
  decltype(&hiprtcCreateProgram) create = nullptr;
  decltype(&hiprtcCompileProgram) compile = nullptr;
  decltype(&hiprtcGetProgramLogSize) log_size = nullptr;
  decltype(&hiprtcGetProgramLog) log = nullptr;
  decltype(&hiprtcGetCodeSize) code_size = nullptr;
  decltype(&hiprtcGetCode) code = nullptr;
  decltype(&hiprtcDestroyProgram) destroy = nullptr;
  decltype(&hiprtcGetErrorString) error_string = nullptr;
  std::string where, error;
};

const Rtc& LoadRtc() {
  static const Rtc rtc = [] {
    Rtc r;
    const char* root = getenv("ROCM_PATH");
    const std::string path = std::string(root && *root ? root : "/opt/rocm") + "/lib/libhiprtc.so";
    void* h = dlmopen(LM_ID_NEWLM, path.c_str(), RTLD_NOW | RTLD_LOCAL);
    r.where = path + " (own namespace)";
    if (!h) {
      r.error = dlerror();
      h = dlopen("libhiprtc.so", RTLD_NOW | RTLD_LOCAL);
      r.where = "libhiprtc.so";
    }
    if (!h) {
      r.error = "cannot load hiprtc (" + r.error + "; " + dlerror() + ")";
      return r;
    }
    bool ok = true;
    auto sym = [&](auto& fn, const char* name) {
      fn = reinterpret_cast<std::remove_reference_t<decltype(fn)>>(dlsym(h, name));
      ok = ok && fn != nullptr;
    };
    sym(r.create, "hiprtcCreateProgram");
    sym(r.compile, "hiprtcCompileProgram");
    sym(r.log_size, "hiprtcGetProgramLogSize");
    sym(r.log, "hiprtcGetProgramLog");
    sym(r.code_size, "hiprtcGetCodeSize");
    sym(r.code, "hiprtcGetCode");
    sym(r.destroy, "hiprtcDestroyProgram");
    sym(r.error_string, "hiprtcGetErrorString");
    if (!ok) r.error = r.where + ": missing hiprtc symbols";
    else r.error.clear();
    return r;
  }();
  return rtc;
}

// code objects by full source, for the life of the process
std::mutex g_codes_mu;
std::unordered_map<std::string, std::shared_ptr<EwJit::Code>>& Codes() {
  static auto* m = new std::unordered_map<std::string, std::shared_ptr<EwJit::Code>>();
  return *m;
}

}  // namespace

int EwJit::Add(EwKernel k) {
  auto it = by_name_.find(k.name);
  if (it != by_name_.end()) return it->second;
  const int idx = int(kernels_.size());
  by_name_[k.name] = idx;
  kernels_.push_back(std::move(k));
  return idx;
}

std::string EwJit::error() const {
  std::lock_guard<std::mutex> lk(mu_);
  return error_;
}

bool EwJit::Build() {
  std::lock_guard<std::mutex> lk(mu_);
  if (built_) return error_.empty();
  built_ = true;
  std::string source = kPreamble;
  for (const EwKernel& k : kernels_) source += k.source;
  if (const char* path = getenv("JAM_EW_JIT_SOURCE")) {  // debugging: the generated source
    if (FILE* fp = fopen(path, "w")) {
      fwrite(source.data(), 1, source.size(), fp);
      fclose(fp);
    }
  }
  std::shared_ptr<Code> code;
  {
    std::lock_guard<std::mutex> g(g_codes_mu);
    auto& m = Codes();
    auto it = m.find(source);
    if (it != m.end()) code = it->second;
    else {
      code = std::make_shared<Code>();
      m[source] = code;
    }
  }
  // one compile per distinct source; a concurrent Build of the same source
  // waits on the code's mutex
  std::lock_guard<std::mutex> cl(code->mu);
  if (code->bin.empty() && code->error.empty()) {
    const auto t0 = std::chrono::steady_clock::now();
    const Rtc& rtc = LoadRtc();
    hiprtcProgram p = nullptr;
    hiprtcResult r = HIPRTC_SUCCESS;
    if (!rtc.error.empty()) {
      code->error = rtc.error;
    } else if ((r = rtc.create(&p, source.c_str(), "jam_ew.hip", 0, nullptr, nullptr)) != HIPRTC_SUCCESS) {
      code->error = std::string("hiprtcCreateProgram: ") + rtc.error_string(r);
    } else {
      // the kernel library's code generation: gfx950, -O3, no packed fp32
      // ops, hipcc's default contraction mode (the math library's inlined
      // code then compiles as in the interpreter; the generated program's
      // own operations are kept apart by the pragma in each body)
      const char* opts[] = {"--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=fast-honor-pragmas",
                            "-fhip-fp32-correctly-rounded-divide-sqrt", "-fno-gpu-flush-denormals-to-zero",
                            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
      r = rtc.compile(p, int(sizeof opts / sizeof opts[0]), opts);
      if (r != HIPRTC_SUCCESS) {
        size_t ls = 0;
        rtc.log_size(p, &ls);
        std::string log(ls, '\0');
        if (ls) rtc.log(p, &log[0]);
        if (log.size() > 2000) log.resize(2000);
        code->error = std::string("hiprtcCompileProgram (") + rtc.where + "): " + rtc.error_string(r) + ": " + log;
      } else {
        size_t cs = 0;
        rtc.code_size(p, &cs);
        code->bin.resize(cs);
        if (cs) rtc.code(p, code->bin.data());
        if (code->bin.empty()) code->error = "hiprtc: empty code object";
      }
      rtc.destroy(&p);
    }
    code->seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
  }
  if (const char* path = getenv("JAM_EW_JIT_CODE")) {  // debugging: the code object
    if (FILE* fp = fopen(path, "wb")) {
      fwrite(code->bin.data(), 1, code->bin.size(), fp);
      fclose(fp);
    }
  }
  code_ = code;
  compile_seconds_ = code->seconds;
  error_ = code->error;
  return error_.empty();
}

void* const* EwJit::Functions(int ordinal) {
  if (ordinal < 0 || !Build()) return nullptr;
  std::lock_guard<std::mutex> lk(mu_);
  if (!error_.empty()) return nullptr;  // a failed load is not retried
  if (fns_.size() <= size_t(ordinal)) fns_.resize(size_t(ordinal) + 1);
  std::vector<void*>& f = fns_[size_t(ordinal)];
  if (f.size() == 2 * kernels_.size()) return f.data();
  hipModule_t mod = nullptr;
  {
    std::lock_guard<std::mutex> cl(code_->mu);
    if (code_->modules.size() <= size_t(ordinal)) code_->modules.resize(size_t(ordinal) + 1, nullptr);
    if (!code_->modules[size_t(ordinal)]) {
      hipError_t e = hipModuleLoadData(&code_->modules[size_t(ordinal)], code_->bin.data());
      if (e != hipSuccess) {
        code_->modules[size_t(ordinal)] = nullptr;
        error_ = std::string("hipModuleLoadData: ") + hipGetErrorString(e);
        return nullptr;
      }
    }
    mod = code_->modules[size_t(ordinal)];
  }
  std::vector<void*> out;
  for (const EwKernel& k : kernels_) {
    for (const std::string* name : {&k.name, &k.final_name}) {
      hipFunction_t fn = nullptr;
      if (!name->empty()) {
        hipError_t e = hipModuleGetFunction(&fn, mod, name->c_str());
        if (e != hipSuccess) {
          error_ = "hipModuleGetFunction(" + *name + "): " + hipGetErrorString(e);
          return nullptr;
        }
      }
      out.push_back(reinterpret_cast<void*>(fn));
    }
  }
  f = std::move(out);
  return f.data();
}

}  // namespace mi::jam
