// jam lowering: StableHLO IR -> launch plan over the mk_* C-ABI.
//
// Mirrors the role of the reference's Lower/WalkBlock (src/jam/lower.mm:
// 208-314, 460-566): inline func.call (245-268), bind @main arguments
// (477-487), dispatch every op, fail with "jam: unhandled op '<name>'" for
// anything without a lowering (308-310).  Where the reference emits one
// MPSGraph node per op, jam emits kernel launches:
//   * layout ops (reshape, broadcast_in_dim, transpose, slice) become strided
//     views and cost nothing until a consumer needs dense memory;
//   * chains of elementwise ops (incl. convert, compare, select, clamp) are
//     kept as expressions and compiled into ONE mk_ew_program launch each,
//     with per-op bf16/f16 rounding where the StableHLO result type is
//     bf16/f16 (what XLA:CPU computes);
//   * pattern matchers replace whole subgraphs by a fused kernel: causal /
//     full scaled-dot-product attention (QKᵀ -> scale -> mask -> softmax ->
//     PV, cf. TrySoftmax elementwise.mm:71-89), arg-max/min reduces
//     (DetectArgReduce reduce.mm:29-43), dot_general + bias (+ ReLU), and
//     attention together with the backward jax.grad emits for it (the
//     flash forward with lse, then the flash backward);
//   * temporaries live in one arena per run, packed by liveness.
#include <algorithm>
#include <array>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <map>
#include <random>
#include <set>
#include <sstream>
#include <unordered_map>

#include "jam/ir.h"
#include "jam/bytecode.h"
#include "jam/vhlo.h"
#include "jam/program.h"
#include "mk_kernels.h"

namespace mi::jam {

const char* StepName(StepKind k) {
  switch (k) {
    case StepKind::kGemm: return "gemm";
    case StepKind::kSdpa: return "sdpa";
    case StepKind::kRowReduce: return "row_reduce";
    case StepKind::kArgmax: return "argmax";
    case StepKind::kLayerNorm: return "layernorm";
    case StepKind::kGelu: return "gelu";
    case StepKind::kEw: return "ew";
    case StepKind::kGather: return "gather";
    case StepKind::kScatterAdd: return "scatter_add";
    case StepKind::kIota: return "iota";
    case StepKind::kCopyStrided: return "copy_strided";
    case StepKind::kSoftmax: return "softmax";
    case StepKind::kConvert: return "convert";
    case StepKind::kFill: return "fill";
    case StepKind::kCopy: return "copy";
    case StepKind::kSdpaBwd: return "sdpa_bwd";
    case StepKind::kGemmBlas: return "gemm_blas";
    case StepKind::kSoftmaxXent: return "softmax_xent";
    case StepKind::kColSum: return "col_sum";
    case StepKind::kLayerNormBwd: return "layernorm_bwd";
    case StepKind::kGemmSplitK: return "gemm_splitk";
    case StepKind::kEwReduce: return "ew_reduce";
  }
  return "?";
}

std::string Program::Dump() const {
  std::ostringstream os;
  os << "program " << name << ": " << inputs.size() << " inputs, " << outputs.size()
     << " outputs, " << steps.size() << " steps, arena " << arena_bytes << " B, " << consts.size()
     << " consts\n";
  for (const auto& p : patterns) os << "  pattern " << p << "\n";
  for (const auto& a : alias_notes) os << "  alias " << a << "\n";
  if (ew_jit) {
    int n = 0;
    for (const Step& st : steps) n += st.jit >= 0;
    os << "  ew_jit " << ew_jit->size() << " kernels for " << n << " steps\n";
  }
  for (size_t i = 0; i < steps.size(); ++i) {
    os << "  [" << i << "] " << StepName(steps[i].kind);
    if (!steps[i].note.empty()) os << " (" << steps[i].note << ")";
    // the generated kernel that runs the step (its name in profiles)
    if (ew_jit && steps[i].jit >= 0) os << " -> " << ew_jit->kernel(steps[i].jit).name;
    if (getenv("JAM_DUMP_BUFFERS")) {  // debugging: where each step's buffers live
      static const char* kSpace[] = {"in", "out", "arena", "const", "none"};
      for (const BufRef& b : steps[i].bufs) os << " " << kSpace[int(b.space)] << b.index << "@" << b.offset;
    }
    os << "\n";
  }
  return os.str();
}

CompileOptions OptionsFromEnv() {
  CompileOptions o;
  o.fuse_sdpa = getenv("JAM_NO_SDPA") == nullptr;
  o.fuse_argmax = getenv("JAM_NO_ARGMAX") == nullptr;
  o.fuse_gemm_epilogue = getenv("JAM_NO_GEMM_EPILOGUE") == nullptr;
  o.fuse_layernorm = getenv("JAM_NO_LAYERNORM") == nullptr;
  o.fuse_gelu = getenv("JAM_NO_GELU") == nullptr;
  o.fuse_elementwise = getenv("JAM_NO_EW_FUSION") == nullptr;
  o.fuse_xent = getenv("JAM_NO_XENT") == nullptr;
  o.ew_jit = getenv("JAM_NO_EW_JIT") == nullptr;
  o.ew_jit_eager = getenv("JAM_EW_JIT_EAGER") != nullptr;
  o.ew_jit_strict = getenv("JAM_EW_JIT_STRICT") != nullptr;
  o.ew_batch = getenv("JAM_NO_EW_BATCH") == nullptr;
  return o;
}

namespace {

// ------------------------------------------------------------------ constants
uint16_t F32ToBf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}
float Bf16ToF32(uint16_t h) {
  uint32_t u = uint32_t(h) << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}
// IEEE half, round to nearest even, with subnormals (the reference's
// FloatToHalf, structural.mm:22-31, truncates and flushes; XLA rounds).
uint16_t F32ToF16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return uint16_t(sign | 0x7e00u);
  if (ax >= 0x477ff000u) return uint16_t(sign | 0x7c00u);  // rounds to >= 65520 -> inf
  if (ax < 0x33000001u) return uint16_t(sign);             // < 2^-25 (+) -> 0
  int e = int(ax >> 23) - 127;
  uint32_t m = (ax & 0x7fffffu) | 0x800000u;
  int shift = e >= -14 ? 13 : 13 + (-14 - e);
  uint32_t hm = m >> shift;
  uint32_t rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
  if (rem > half || (rem == half && (hm & 1u))) ++hm;
  uint32_t h = e >= -14 ? (uint32_t(e + 15) << 10) + (hm - 0x400u) : hm;
  if (e >= -14 && hm >= 0x800u) h = (uint32_t(e + 16) << 10);  // mantissa overflow
  return uint16_t(sign | h);
}
float F16ToF32(uint16_t h) {
  const uint32_t s = (h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  uint32_t u;
  if (e == 0) {
    if (m == 0) u = s;
    else {
      float v = std::ldexp(float(m), -24);
      memcpy(&u, &v, 4);
      u |= s;
    }
  } else if (e == 31) {
    u = s | 0x7f800000u | (m << 13);
  } else {
    u = s | ((e + 112) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

double HexToValue(uint64_t bits, DType d) {
  switch (d) {
    case DType::kF32: {
      uint32_t u = uint32_t(bits);
      float f;
      memcpy(&f, &u, 4);
      return f;
    }
    case DType::kF64: {
      double v;
      memcpy(&v, &bits, 8);
      return v;
    }
    case DType::kBF16: return Bf16ToF32(uint16_t(bits));
    case DType::kF16: return F16ToF32(uint16_t(bits));
    default: return double(int64_t(bits));
  }
}

// Parse the body of dense<...> for a tensor type.  Fills fvals / ivals.
bool ParseDense(Attr& a, const TensorType& t, std::string& err) {
  std::string s = a.s;
  const int64_t n = t.numel();
  const bool fl = IsFloat(t.dtype);
  a.fvals.clear();
  a.ivals.clear();
  auto trim = [](std::string x) {
    size_t b = x.find_first_not_of(" \n\t"), e = x.find_last_not_of(" \n\t");
    return b == std::string::npos ? std::string() : x.substr(b, e - b + 1);
  };
  s = trim(s);
  if (s.size() >= 3 && s[0] == '"' && s[1] == '0' && (s[2] == 'x' || s[2] == 'X')) {
    // raw little-endian element bytes
    std::string hex = s.substr(3, s.size() - 4);
    std::vector<uint8_t> bytes;
    for (size_t i = 0; i + 1 < hex.size(); i += 2) bytes.push_back(uint8_t(strtoul(hex.substr(i, 2).c_str(), nullptr, 16)));
    const int w = DTypeBytes(t.dtype);
    if (w == 0 || bytes.size() % size_t(w) != 0) {
      err = "jam: malformed dense hex constant";
      return false;
    }
    const size_t cnt = bytes.size() / size_t(w);
    for (size_t i = 0; i < cnt; ++i) {
      uint64_t bits = 0;
      memcpy(&bits, &bytes[i * w], w);
      if (fl) a.fvals.push_back(HexToValue(bits, t.dtype));
      else if (IsSigned(t.dtype)) {
        int64_t v = int64_t(bits << (64 - 8 * w)) >> (64 - 8 * w);
        a.ivals.push_back(v);
      } else {
        a.ivals.push_back(int64_t(bits));
      }
    }
  } else {
    std::string tok;
    auto flush = [&]() {
      if (tok.empty()) return;
      if (tok == "true" || tok == "false") {
        a.ivals.push_back(tok == "true");
        a.fvals.push_back(tok == "true");
      } else if (tok.size() > 2 && tok[0] == '0' && (tok[1] == 'x' || tok[1] == 'X')) {
        uint64_t bits = strtoull(tok.c_str(), nullptr, 16);
        if (fl) a.fvals.push_back(HexToValue(bits, t.dtype));
        else a.ivals.push_back(int64_t(bits));
      } else if (tok == "inf" || tok == "+inf") {
        a.fvals.push_back(INFINITY);
      } else if (tok == "-inf") {
        a.fvals.push_back(-INFINITY);
      } else if (tok == "nan") {
        a.fvals.push_back(NAN);
      } else {
        if (fl) a.fvals.push_back(strtod(tok.c_str(), nullptr));
        else a.ivals.push_back(strtoll(tok.c_str(), nullptr, 10));
      }
      tok.clear();
    };
    for (char c : s) {
      if (c == '[' || c == ']' || c == ',' || c == ' ' || c == '\n' || c == '(' || c == ')') flush();
      else tok.push_back(c);
    }
    flush();
  }
  const size_t cnt = fl ? a.fvals.size() : a.ivals.size();
  if (cnt == 1 && n != 1) a.splat = true;
  else if (int64_t(cnt) != n) {
    err = "jam: dense constant has " + std::to_string(cnt) + " values for " + t.str();
    return false;
  } else {
    a.splat = (n == 1);
  }
  if (fl && a.ivals.empty()) for (double v : a.fvals) a.ivals.push_back(int64_t(v));
  if (!fl && a.fvals.empty()) for (int64_t v : a.ivals) a.fvals.push_back(double(v));
  return true;
}

// A decimal literal is read as a double and rounded ONCE to the element
// type (nearest, ties to even), as MLIR's APFloat conversion does; rounding
// through float first could round twice.  p = significand bits, emin = the
// smallest normal exponent (bf16: 8, -126; f16: 11, -14).  The result is
// exactly representable as a float.
double RoundToFormat(double v, int p, int emin) {
  if (!std::isfinite(v) || v == 0) return v;
  int e;
  std::frexp(v, &e);
  const double q = std::ldexp(1.0, std::max(e - 1, emin) - (p - 1));
  return std::nearbyint(v / q) * q;
}
uint16_t F64ToBf16(double v) { return F32ToBf16(float(RoundToFormat(v, 8, -126))); }
uint16_t F64ToF16(double v) { return F32ToF16(float(RoundToFormat(v, 11, -14))); }

void EncodeElement(double v, int64_t iv, DType d, uint8_t* out) {
  switch (d) {
    case DType::kF32: { float f = float(v); memcpy(out, &f, 4); break; }
    case DType::kF64: memcpy(out, &v, 8); break;
    case DType::kBF16: { uint16_t h = F64ToBf16(v); memcpy(out, &h, 2); break; }
    case DType::kF16: { uint16_t h = F64ToF16(v); memcpy(out, &h, 2); break; }
    case DType::kPred: out[0] = iv != 0; break;
    default: memcpy(out, &iv, size_t(DTypeBytes(d))); break;
  }
}

// value of a scalar of type d as it lives in the ew register file (32 bits)
uint32_t RegisterBits(double v, int64_t iv, DType d) {
  float f;
  if (IsFloat(d)) {
    if (d == DType::kBF16) f = Bf16ToF32(F64ToBf16(v));
    else if (d == DType::kF16) f = F16ToF32(F64ToF16(v));
    else f = float(v);
  } else if (d == DType::kPred) {
    f = iv != 0 ? 1.f : 0.f;
  } else {
    int32_t i = int32_t(iv);
    memcpy(&f, &i, 4);
  }
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

// ------------------------------------------------------------------ views
struct View {
  BufRef buf;                     // base buffer (offset in bytes)
  DType dtype = DType::kInvalid;
  std::vector<int64_t> dims;
  std::vector<int64_t> strides;   // elements
  int64_t offset = 0;             // elements, added to buf.offset

  int rank() const { return int(dims.size()); }
  int64_t numel() const {
    int64_t n = 1;
    for (int64_t d : dims) n *= d;
    return n;
  }
  bool dense() const {
    int64_t e = 1;
    for (int d = rank() - 1; d >= 0; --d) {
      if (dims[d] != 1 && strides[d] != e) return false;
      e *= dims[d];
    }
    return true;
  }
  BufRef at() const {
    BufRef r = buf;
    r.offset += offset * DTypeBytes(dtype);
    return r;
  }
};

std::vector<int64_t> DenseStrides(const std::vector<int64_t>& dims) {
  std::vector<int64_t> s(dims.size());
  int64_t e = 1;
  for (int d = int(dims.size()) - 1; d >= 0; --d) {
    s[d] = e;
    e *= dims[d];
  }
  return s;
}

// ------------------------------------------------------------------ lowering state
struct ValState {
  enum Kind { kUnset, kView, kEw, kScalar } kind = kUnset;
  View view;
  double fval = 0;      // kScalar
  int64_t ival = 0;
  int op = -1;          // kEw: index of the producing op
};

struct Fused {
  enum Kind { kSdpa, kArgmax, kGemmEpi, kLayerNorm, kGelu, kSdpaBwd, kXent, kLayerNormBwd } kind;
  std::vector<int> deps;  // value ids the fused step reads
  // sdpa (train: also lse and the bf16 O for the backward step)
  int q = -1, k = -1, v = -1;
  float scale = 1.f;
  bool causal = false;
  bool train = false;
  // sdpa_bwd: dO (bf16), the forward's anchor, the three gradients
  int dout = -1, fwd = -1, dq = -1, dk = -1, dv = -1;
  // softmax cross-entropy: logits (x), labels, per-row loss and dlogits values;
  // when every reader of an f32 dlogits converts it to bf16, those converts'
  // results (written by the fused step instead)
  int labels = -1, dlogits = -1;
  std::vector<int> dlogits_bf16;
  // argmax
  int x = -1;
  bool is_min = false;
  int red_op = -1;
  // gemm epilogue (gelu_out: a bf16 GELU of the result the epilogue also writes)
  int dot = -1, bias = -1;
  bool relu = false;
  int gelu_out = -1;
  // layernorm (in_dtype: x, gamma and beta; out_dtype: the result)
  int gamma = -1, beta = -1;
  float eps = 0;
  DType out_dtype = DType::kInvalid;
  DType in_dtype = DType::kInvalid;
  int add_a = -1, add_b = -1;  // x = add_a + add_b computed and stored by the LayerNorm step
  // layernorm backward (x, gamma, dout = dy): the residual cotangent added to
  // dx, and the dgamma / dbeta / bias-gradient values it also writes (-1: none)
  int dres = -1, dgamma = -1, dbeta = -1, colsum = -1;
  std::vector<int> dx_bf16;  // converts of dx to bf16 whose results it writes too
};

class Lowerer {
 public:
  Lowerer(Module& m, const CompileOptions& o) : m_(m), opts_(o) {}

  std::shared_ptr<Program> Run(std::string& err) {
    prog_ = std::make_shared<Program>();
    try {
      const Func* main = m_.find("main");
      if (!main) {
        for (const auto& f : m_.funcs)
          if (f.is_public) main = &f;
      }
      if (!main) throw std::string("jam: module has no @main function");  // lower.mm:464-466
      prog_->name = "jam." + (m_.name.empty() ? std::string("main") : m_.name);
      // flatten: inline calls
      std::unordered_map<int, int> remap;
      for (int a : main->args) {
        prog_->inputs.push_back(m_.types[a]);
        ops_.reserve(64);
      }
      Inline(*main, main->args, outputs_, 0);
      for (int o : outputs_) prog_->outputs.push_back(m_.types[o]);
      state_.assign(m_.types.size(), ValState());
      for (size_t i = 0; i < main->args.size(); ++i) {
        ValState& s = state_[main->args[i]];
        s.kind = ValState::kView;
        s.view.buf = BufRef{Space::kInput, int(i), 0};
        s.view.dtype = m_.types[main->args[i]].dtype;
        s.view.dims = m_.types[main->args[i]].dims;
        s.view.strides = DenseStrides(s.view.dims);
      }
      Analyze();
      Reachable();
      MatchPatterns();
      Liveness();
      Walk();
      PackArena();
      Aliases(*main);
      return prog_;
    } catch (const std::string& e) {
      err = e;
      return nullptr;
    }
  }

 private:
  // -------------------------------------------------------------- donation
  // Buffer indices a step writes (the rest it reads), per the encodings in
  // run.cc.
  static std::vector<size_t> WrittenBufs(const Step& s) {
    switch (s.kind) {
      case StepKind::kGemm: return s.bufs.size() > 4 ? std::vector<size_t>{2, 4} : std::vector<size_t>{2};
      case StepKind::kSdpa: return s.bufs.size() > 4 ? std::vector<size_t>{3, 4} : std::vector<size_t>{3};
      case StepKind::kSdpaBwd: return {6, 7, 8, 9};
      case StepKind::kGemmBlas: return {2};
      case StepKind::kSoftmaxXent: return {2, 3};
      case StepKind::kColSum: return {1, 2};
      case StepKind::kGemmSplitK: return {2, 3};
      case StepKind::kRowReduce: return {1};
      case StepKind::kArgmax: return {1, 2};
      case StepKind::kLayerNorm: return s.bufs.size() > 4 ? std::vector<size_t>{3, 5} : std::vector<size_t>{3};
      case StepKind::kLayerNormBwd: return s.bufs.size() > 9 ? std::vector<size_t>{4, 5, 6, 7, 8, 9}
                                                             : std::vector<size_t>{4, 5, 6, 7, 8};
      case StepKind::kGelu: return {1};
      case StepKind::kEw: {
        std::vector<size_t> w;
        for (size_t k = size_t(s.i[7]); k < s.bufs.size(); ++k) w.push_back(k);
        return w;
      }
      case StepKind::kEwReduce: {
        const size_t L = size_t(s.i[7]);
        if (s.bufs.size() > L + 3) return {L, L + 1, L + 2, L + 3};
        return {L, L + 1, L + 2};
      }
      case StepKind::kGather: return {2};
      case StepKind::kScatterAdd: return {3, 4};
      case StepKind::kIota: return {0};
      case StepKind::kCopyStrided: return {1};
      case StepKind::kSoftmax: return {1};
      case StepKind::kConvert: return {1};
      case StepKind::kFill: return {0};
      case StepKind::kCopy: return {1};
    }
    return {};
  }

  // Can output `o` be computed straight into input `in`'s memory?
  bool InPlaceSafe(int in, int o, std::string& why) const {
    const auto& steps = prog_->steps;
    auto is_in = [&](const BufRef& b) { return b.space == Space::kInput && b.index == in; };
    auto is_out = [&](const BufRef& b) { return b.space == Space::kOutput && b.index == o; };
    int first = -1;
    for (size_t k = 0; k < steps.size() && first < 0; ++k)
      for (size_t w : WrittenBufs(steps[k]))
        if (w < steps[k].bufs.size() && is_out(steps[k].bufs[w])) first = int(k);
    if (first < 0) {
      why = "output never written";
      return false;
    }
    for (size_t k = size_t(first) + 1; k < steps.size(); ++k)
      for (const BufRef& b : steps[k].bufs)
        if (is_in(b)) {
          why = "input read after the output is first written (step " + std::to_string(k) + ")";
          return false;
        }
    const Step& s = steps[size_t(first)];
    const std::vector<size_t> wr = WrittenBufs(s);
    std::vector<size_t> reads;
    for (size_t j = 0; j < s.bufs.size(); ++j)
      if (is_in(s.bufs[j]) && std::find(wr.begin(), wr.end(), j) == wr.end()) reads.push_back(j);
    if (reads.empty()) return true;
    // the writer reads the input too: only element-for-element in place
    size_t wo = wr.front();
    for (size_t w : wr)
      if (is_out(s.bufs[w])) wo = w;
    const BufRef& out = s.bufs[wo];
    for (size_t j : reads)
      if (s.bufs[j].offset != 0 || out.offset != 0) {
        why = "writer reads the input at an offset";
        return false;
      }
    switch (s.kind) {
      case StepKind::kGelu:
        return true;
      case StepKind::kConvert:
        if (DTypeBytes(DType(s.i[0])) == DTypeBytes(DType(s.i[1]))) return true;
        why = "convert changes the element width";
        return false;
      case StepKind::kEw: {
        const int rank = int(s.i[0]);
        std::vector<int64_t> dims(s.i.begin() + 1, s.i.begin() + 1 + rank);
        const std::vector<int64_t> dense = DenseStrides(dims);
        // output k of the step: its type is i[9] for k = 0, else i[11 + 2 (k - 1)]
        const size_t k_out = wo - size_t(s.i[7]);
        const int out_type = int(k_out == 0 ? s.i[9] : s.i[11 + 2 * (k_out - 1)]);
        for (size_t j : reads) {
          if (DTypeBytes(DType(s.types[j])) != DTypeBytes(DType(out_type))) {
            why = "elementwise input and output widths differ";
            return false;
          }
          for (int d = 0; d < rank; ++d)
            if (dims[size_t(d)] > 1 && s.strides[j * 6 + size_t(d)] != dense[size_t(d)]) {
              why = "elementwise input read in another layout (broadcast / transpose)";
              return false;
            }
        }
        return true;
      }
      default:
        why = std::string("writer is ") + StepName(s.kind) + ", not element-for-element";
        return false;
    }
  }

  void Aliases(const Func& main) {
    const size_t n_in = prog_->inputs.size(), n_out = prog_->outputs.size();
    prog_->input_alias.assign(n_in, -1);
    std::vector<bool> claimed(n_out, false);
    auto consider = [&](size_t i, int o, const char* how) {
      std::string why;
      if (o < 0 || size_t(o) >= n_out) {
        why = "no such output";
      } else if (claimed[size_t(o)]) {
        why = "output already aliased";
      } else if (prog_->inputs[i].bytes() != prog_->outputs[size_t(o)].bytes()) {
        why = "sizes differ";
      } else if (InPlaceSafe(int(i), o, why)) {
        prog_->input_alias[i] = o;
        claimed[size_t(o)] = true;
        prog_->alias_notes.push_back("input " + std::to_string(i) + " -> output " + std::to_string(o) +
                                     " in place (" + how + ")");
        return;
      }
      prog_->alias_notes.push_back("input " + std::to_string(i) + " -> output " + std::to_string(o) +
                                   " not in place (" + how + "): " + why);
    };
    for (size_t i = 0; i < n_in && i < main.arg_alias.size(); ++i)
      if (main.arg_alias[i] >= 0) consider(i, main.arg_alias[i], "tf.aliasing_output");
    // donors without an explicit output: the first unclaimed output of the same type
    for (size_t i = 0; i < n_in && i < main.arg_donor.size(); ++i) {
      if (!main.arg_donor[i] || prog_->input_alias[i] >= 0 || main.arg_alias[i] >= 0) continue;
      int match = -1;
      for (size_t o = 0; o < n_out && match < 0; ++o)
        if (!claimed[o] && prog_->outputs[o] == prog_->inputs[i]) match = int(o);
      if (match >= 0) consider(i, match, "jax.buffer_donor");
      else prog_->alias_notes.push_back("input " + std::to_string(i) + " donated: no output of its type");
    }
  }

  // -------------------------------------------------------------- inlining
  // Appends the ops of `f` (with args bound to `actuals`) to ops_, renaming
  // values; returns the values `f` returns in `results`.
  void Inline(const Func& f, const std::vector<int>& actuals, std::vector<int>& results, int depth) {
    if (depth > 32) throw std::string("jam: call depth exceeds 32 (recursive call?)");
    std::unordered_map<int, int> ren;
    for (size_t i = 0; i < f.args.size(); ++i) ren[f.args[i]] = actuals[i];
    auto R = [&](int v) {
      auto it = ren.find(v);
      return it == ren.end() ? v : it->second;
    };
    for (const Op& op0 : f.body.ops) {
      if (op0.name == "return") {
        results.clear();
        for (int v : op0.operands) results.push_back(R(v));
        return;
      }
      if (op0.name == "func.call") {
        const Attr* callee = op0.attr("callee");
        const Func* g = callee ? m_.find(callee->s) : nullptr;
        if (!g) throw std::string("jam: call to unknown function @" + (callee ? callee->s : "?"));
        std::vector<int> acts, rets;
        for (int v : op0.operands) acts.push_back(R(v));
        Inline(*g, acts, rets, depth + 1);
        if (rets.size() != op0.results.size()) throw std::string("jam: call result count mismatch");
        for (size_t i = 0; i < rets.size(); ++i) ren[op0.results[i]] = rets[i];
        continue;
      }
      if (op0.name == "stablehlo.optimization_barrier") {
        for (size_t i = 0; i < op0.results.size(); ++i) ren[op0.results[i]] = R(op0.operands[i]);
        continue;
      }
      Op op = op0;
      for (int& v : op.operands) v = R(v);
      // fresh result ids when a function is inlined more than once
      if (inlined_once_.count(&f)) {
        for (int& r : op.results) {
          int nv = m_.new_value(m_.types[r]);
          ren[r] = nv;
          r = nv;
        }
      }
      ops_.push_back(op);
    }
    inlined_once_.insert(&f);
  }

  // -------------------------------------------------------------- analysis
  void Analyze() {
    producer_.assign(m_.types.size(), -1);
    uses_.assign(m_.types.size(), 0);
    users_.assign(m_.types.size(), {});
    for (size_t i = 0; i < ops_.size(); ++i) {
      for (int r : ops_[i].results) producer_[r] = int(i);
      for (int v : ops_[i].operands) {
        ++uses_[v];
        users_[v].push_back(int(i));
      }
    }
    for (int o : outputs_) ++uses_[o];
  }
  const Op* prod(int v) const { return v >= 0 && producer_[v] >= 0 ? &ops_[producer_[v]] : nullptr; }

  // ops whose results reach a program output (before any fusion): the
  // backward of a jitted step carries transposes nothing reads (the
  // cotangent of a constant), which must not count as uses
  void Reachable() {
    reach_.assign(ops_.size(), false);
    std::vector<int> stack(outputs_.begin(), outputs_.end());
    std::vector<bool> seen(m_.types.size(), false);
    while (!stack.empty()) {
      const int v = stack.back();
      stack.pop_back();
      if (v < 0 || seen[v]) continue;
      seen[v] = true;
      const int pr = producer_[v];
      if (pr < 0 || reach_[pr]) continue;
      reach_[pr] = true;
      for (int o : ops_[pr].operands) stack.push_back(o);
      for (const auto& reg : ops_[pr].regions)
        for (const auto& blk : reg->blocks)
          for (const Op& inner : blk.ops)
            for (int o : inner.operands) stack.push_back(o);
    }
  }
  // reachable users of v
  std::vector<int> live_users(int v) const {
    std::vector<int> r;
    for (int u : users_[v])
      if (reach_[u]) r.push_back(u);
    return r;
  }
  bool is(int v, const char* name) const {
    const Op* p = prod(v);
    return p && p->name == name;
  }
  int through_converts(int v, std::vector<int>* path = nullptr) const {
    while (is(v, "stablehlo.convert") || is(v, "stablehlo.reshape")) {
      if (path) path->push_back(producer_[v]);
      v = prod(v)->operands[0];
    }
    return v;
  }
  // scalar value of a splat constant (possibly broadcast / reshaped / converted)
  bool scalar_of(int v, double* out) const {
    for (;;) {
      const Op* p = prod(v);
      if (!p) return false;
      if (p->name == "stablehlo.broadcast_in_dim" || p->name == "stablehlo.reshape" ||
          p->name == "stablehlo.convert" || p->name == "stablehlo.broadcast") {
        v = p->operands[0];
        continue;
      }
      if (p->name != "stablehlo.constant") return false;
      const Attr* a = ParsedConst(v);
      if (!a || (!a->splat && m_.types[v].numel() != 1)) return false;
      const DType d = m_.types[v].dtype;
      double x = a->fvals.empty() ? double(a->ivals[0]) : a->fvals[0];
      if (d == DType::kBF16) x = Bf16ToF32(F64ToBf16(x));
      else if (d == DType::kF16) x = F16ToF32(F64ToF16(x));
      else if (d == DType::kF32) x = float(x);
      *out = x;
      return true;
    }
  }
  std::vector<int64_t> attr_ints(const Op& op, std::initializer_list<const char*> names) const {
    for (const char* n : names)
      if (const Attr* a = op.attr(n)) return a->ints();
    return {};
  }
  struct DotDims {
    std::vector<int64_t> lb, rb, lc, rc;
  };
  DotDims dot_dims(const Op& op) const {
    DotDims d;
    if (const Attr* dn = op.attr("dot_dimension_numbers")) {
      if (const Attr* x = dn->get("lhs_batching_dimensions")) d.lb = x->ints();
      if (const Attr* x = dn->get("rhs_batching_dimensions")) d.rb = x->ints();
      if (const Attr* x = dn->get("lhs_contracting_dimensions")) d.lc = x->ints();
      if (const Attr* x = dn->get("rhs_contracting_dimensions")) d.rc = x->ints();
      return d;
    }
    if (const Attr* b = op.attr("batching_dims")) {
      d.lb = b->list.at(0).ints();
      d.rb = b->list.at(1).ints();
    }
    if (const Attr* c = op.attr("contracting_dims")) {
      d.lc = c->list.at(0).ints();
      d.rc = c->list.at(1).ints();
    }
    return d;
  }
  std::vector<int64_t> reduce_dims(const Op& op) const { return attr_ints(op, {"dimensions"}); }
  std::string reduce_body_op(const Op& op) const {
    if (op.regions.empty() || op.regions[0]->blocks.empty()) return "";
    for (const Op& b : op.regions[0]->blocks[0].ops)
      if (b.name != "return") return b.name;
    return "";
  }

  // -------------------------------------------------------------- pattern matching
  void MatchPatterns() {
    for (size_t i = 0; i < ops_.size(); ++i) {
      const Op& op = ops_[i];
      if (op.name == "stablehlo.dot_general" && opts_.fuse_sdpa) TryMatchSdpa(int(i));
      if (op.name == "stablehlo.reduce" && op.operands.size() == 4 && op.results.size() == 2 &&
          opts_.fuse_argmax)
        TryMatchArgmax(int(i));
    }
    if (opts_.fuse_xent)
      for (size_t i = 0; i < ops_.size(); ++i)
        if (ops_[i].name == "stablehlo.subtract" && !fused_.count(int(i))) TryMatchXent(int(i));
    if (opts_.fuse_gemm_epilogue)
      for (size_t i = 0; i < ops_.size(); ++i)
        if (ops_[i].name == "stablehlo.add" && !fused_.count(int(i)) && !absorbed_.count(int(i)))
          TryMatchGemmEpilogue(int(i));
    if (opts_.fuse_gemm_epilogue && opts_.fuse_gelu)
      for (size_t i = 0; i < ops_.size(); ++i)
        if (ops_[i].name == "stablehlo.convert" && !fused_.count(int(i)) && !absorbed_.count(int(i)))
          TryMatchGemmGelu(int(i));
    if (opts_.fuse_gelu)
      for (size_t i = 0; i < ops_.size(); ++i)
        if (ops_[i].name == "stablehlo.multiply" && !fused_.count(int(i))) TryMatchGelu(int(i));
    if (opts_.fuse_layernorm) {
      auto candidate = [&](size_t i) {
        return !fused_.count(int(i)) && !absorbed_.count(int(i)) &&
               (ops_[i].name == "stablehlo.add" || ops_[i].name == "stablehlo.multiply" ||
                ops_[i].name == "stablehlo.convert");
      };
      for (size_t i = ops_.size(); i-- > 0;)
        if (candidate(i)) TryMatchLayerNormTrain(int(i));
      for (size_t i = ops_.size(); i-- > 0;)
        if (candidate(i)) TryMatchLayerNorm(int(i));
    }
  }

  // ---- small structural-matching helpers
  bool IsConstNear(int v, double c, double rtol = 1e-6) const {
    double x;
    return scalar_of(v, &x) && std::fabs(x - c) <= rtol * std::max(1.0, std::fabs(c));
  }
  // commutative binary op `name` at v: f(a, b) for either operand order
  template <typename F>
  bool Comm(int v, const char* name, F f) const {
    const Op* p = prod(v);
    if (!p || p->name != name || p->operands.size() != 2) return false;
    return f(p->operands[0], p->operands[1]) || f(p->operands[1], p->operands[0]);
  }
  template <typename F>
  bool NonComm(int v, const char* name, F f) const {
    const Op* p = prod(v);
    if (!p || p->name != name || p->operands.size() != 2) return false;
    return f(p->operands[0], p->operands[1]);
  }
  // v = broadcast/reshape chain of a 1-D vector [n] onto the last dim of a
  // rank-r result; returns the vector (looking through one convert) or -1
  int VectorOnLastDim(int v, int64_t n, std::set<int>* ops) const {
    const TensorType& ot = m_.types[v];
    int b = v;
    std::vector<const Op*> chain;
    while ((is(b, "stablehlo.broadcast_in_dim") || is(b, "stablehlo.reshape")) && m_.types[b].rank() != 1) {
      chain.push_back(prod(b));
      b = prod(b)->operands[0];
    }
    if (chain.empty() || m_.types[b].rank() != 1 || m_.types[b].dims[0] != n) return -1;
    int pos = 0;
    for (auto it = chain.rbegin(); it != chain.rend(); ++it) {
      const Op* p = *it;
      const auto& rd = m_.types[p->results[0]].dims;
      if (p->name == "stablehlo.broadcast_in_dim") {
        const auto dd = attr_ints(*p, {"dims", "broadcast_dimensions"});
        if (pos >= int(dd.size())) return -1;
        pos = int(dd[pos]);
      } else {
        int found = -1, nonunit = 0;
        for (size_t k = 0; k < rd.size(); ++k)
          if (rd[k] != 1) {
            ++nonunit;
            found = int(k);
          }
        if (nonunit != 1 || rd[found] != n) return -1;
        pos = found;
      }
    }
    if (pos != ot.rank() - 1) return -1;
    if (ops)
      for (const Op* p : chain) ops->insert(int(p - ops_.data()));
    if (is(b, "stablehlo.convert")) {
      if (ops) ops->insert(producer_[b]);
      b = prod(b)->operands[0];
    }
    return b;
  }
  // v = broadcast chain of a row statistic: reduce_add over the last dim of
  // `x_full` (rank r) kept as [rows..., 1] and broadcast back; returns the
  // reduce input or -1.  scale: divide by n / multiply by 1/n folded in.
  int RowMeanOf(int v, int64_t n, std::set<int>& ops) const {
    int b = v;
    while (is(b, "stablehlo.broadcast_in_dim") || is(b, "stablehlo.reshape")) {
      ops.insert(producer_[b]);
      b = prod(b)->operands[0];
    }
    // mean = sum / n  or  sum * (1/n)
    int sum = -1;
    if (NonComm(b, "stablehlo.divide", [&](int a, int c) {
          if (!IsConstNear(c, double(n))) return false;
          sum = a;
          return true;
        }) ||
        Comm(b, "stablehlo.multiply", [&](int a, int c) {
          if (!IsConstNear(c, 1.0 / double(n), 1e-6)) return false;
          sum = a;
          return true;
        })) {
      ops.insert(producer_[b]);
    } else {
      return -1;
    }
    while (is(sum, "stablehlo.broadcast_in_dim") || is(sum, "stablehlo.reshape")) {
      ops.insert(producer_[sum]);
      sum = prod(sum)->operands[0];
    }
    const Op* r = prod(sum);
    if (!r || r->name != "stablehlo.reduce" || r->operands.size() != 2 || reduce_body_op(*r) != "stablehlo.add")
      return -1;
    double init;
    if (!scalar_of(r->operands[1], &init) || init != 0.0) return -1;
    const int in = r->operands[0];
    const auto dims = reduce_dims(*r);
    if (dims.size() != 1 || dims[0] != m_.types[in].rank() - 1 || m_.types[in].dims.back() != n) return -1;
    ops.insert(producer_[sum]);
    return in;
  }

  // all uses of `v` are by ops in `set` (and v is not a program output)
  bool uses_within(int v, const std::set<int>& set) const {
    for (int o : outputs_)
      if (o == v) return false;
    for (int u : users_[v])
      if (!set.count(u)) return false;
    return true;
  }

  // ---- the attention mask, proven rather than sampled
  //
  // A mask sub-expression is read symbolically over its own index axes:
  //   * an integer affine form c0 + Σ c[k]·idx[k] (iota, integer-valued splat
  //     constants, add/subtract/negate, multiply by a constant, and converts
  //     that are exact over the value's range),
  //   * a predicate: a boolean formula (and/or/not/xor) over half-planes
  //     `affine >= 0` (from compare of two affine forms, select between
  //     constant booleans, constant booleans),
  //   * a dense constant read through an index map (broadcast / transpose /
  //     unit reshape), optionally compared with a splat constant.
  // Layout ops remap the axes.  Anything else makes the mask "unknown" and
  // the attention stays on the generic path.
  struct MaskAff {
    int64_t c0 = 0;
    std::vector<int64_t> c;  // one coefficient per axis of the value
  };
  struct MaskNode {
    enum Kind { kLeaf, kConst, kAnd, kOr, kXor, kNot } kind = kConst;
    MaskAff aff;   // kLeaf: aff >= 0
    bool val = false;
    int a = -1, b = -1;
  };
  struct MaskSym {
    enum Kind { kNone, kAff, kPred, kTable } kind = kNone;
    MaskAff aff;
    std::vector<MaskNode> nodes;
    int root = -1;
    // kTable: element at idx = table[toff + Σ tstride[k]·idx[k]], then the
    // converts in `conv`, then (if cmp set) compared with cmp_val
    const Attr* table = nullptr;
    DType table_dtype = DType::kInvalid;
    std::vector<int64_t> tstride;
    int64_t toff = 0;
    std::vector<DType> conv;
    std::string cmp;
    double cmp_val = 0;
  };

  const Attr* ParsedConst(int v) const {
    const int pi = v >= 0 ? producer_[v] : -1;
    if (pi < 0 || ops_[pi].name != "stablehlo.constant") return nullptr;
    auto it = const_cache_.find(pi);
    if (it != const_cache_.end()) return it->second.get();
    auto a = std::make_shared<Attr>(*ops_[pi].attr("value"));
    std::string err;
    if (!ParseDense(*a, m_.types[v], err)) a.reset();
    return (const_cache_[pi] = a).get();
  }

  static int64_t AffBound(const MaskAff& f, const std::vector<int64_t>& dims) {
    // max |value| over the index box (saturating)
    double m = std::fabs(double(f.c0));
    for (size_t k = 0; k < f.c.size(); ++k) m += std::fabs(double(f.c[k])) * double(std::max<int64_t>(dims[k] - 1, 0));
    return m > 9e18 ? INT64_MAX : int64_t(m);
  }
  static bool ExactIn(int64_t bound, DType d) {
    switch (d) {
      case DType::kBF16: return bound <= (int64_t(1) << 8);
      case DType::kF16: return bound <= (int64_t(1) << 11);
      case DType::kF32: return bound <= (int64_t(1) << 24);
      case DType::kF64: return bound <= (int64_t(1) << 53);
      case DType::kI8: case DType::kU8: return bound < (int64_t(1) << 7);
      case DType::kI16: case DType::kU16: return bound < (int64_t(1) << 15);
      case DType::kI32: case DType::kU32: return bound < (int64_t(1) << 31);
      case DType::kI64: case DType::kU64: return bound < INT64_MAX;
      default: return false;
    }
  }
  static double ConvertScalar(double x, DType d) {
    switch (d) {
      case DType::kPred: return x != 0 ? 1.0 : 0.0;
      case DType::kBF16: return std::isnan(x) ? x : Bf16ToF32(F64ToBf16(x));
      case DType::kF16: return std::isnan(x) ? x : F16ToF32(F64ToF16(x));
      case DType::kF32: return double(float(x));
      case DType::kF64: return x;
      default: return std::isfinite(x) ? std::trunc(x) : 0.0;  // float -> int truncates
    }
  }
  static bool CompareDir(const std::string& dir, double a, double b, bool* ok) {
    *ok = true;
    if (dir == "GE") return a >= b;
    if (dir == "GT") return a > b;
    if (dir == "LE") return a <= b;
    if (dir == "LT") return a < b;
    if (dir == "EQ") return a == b;
    if (dir == "NE") return a != b;
    *ok = false;
    return false;
  }
  static std::string CompareDirOf(const Op& p) {
    if (const Attr* x = p.attr("comparison_direction")) return x->s;
    if (const Attr* x = p.attr("enum0")) return x->s;
    return "";
  }

  // Remap the axes of a symbolic value: new axis k takes the old axis
  // from[k] (-1: a new axis the value does not depend on); old axes of size
  // 1 that are dropped read index 0.
  static void RemapAff(MaskAff& f, const std::vector<int>& from) {
    std::vector<int64_t> c(from.size(), 0);
    for (size_t k = 0; k < from.size(); ++k)
      if (from[k] >= 0) c[k] = f.c[size_t(from[k])];
    f.c = std::move(c);
  }
  static void RemapSym(MaskSym& s, const std::vector<int>& from) {
    if (s.kind == MaskSym::kAff) RemapAff(s.aff, from);
    if (s.kind == MaskSym::kPred)
      for (auto& n : s.nodes)
        if (n.kind == MaskNode::kLeaf) RemapAff(n.aff, from);
    if (s.kind == MaskSym::kTable) {
      std::vector<int64_t> st(from.size(), 0);
      for (size_t k = 0; k < from.size(); ++k)
        if (from[k] >= 0) st[k] = s.tstride[size_t(from[k])];
      s.tstride = std::move(st);
    }
  }
  static MaskSym PredConst(bool v) {
    MaskSym s;
    s.kind = MaskSym::kPred;
    MaskNode n;
    n.kind = MaskNode::kConst;
    n.val = v;
    s.nodes.push_back(n);
    s.root = 0;
    return s;
  }
  static MaskSym PredCombine(MaskNode::Kind k, const MaskSym& x, const MaskSym* y) {
    MaskSym s;
    s.kind = MaskSym::kPred;
    s.nodes = x.nodes;
    const int ra = x.root;
    int rb = -1;
    if (y) {
      const int off = int(s.nodes.size());
      for (MaskNode n : y->nodes) {
        if (n.a >= 0) n.a += off;
        if (n.b >= 0) n.b += off;
        s.nodes.push_back(n);
      }
      rb = y->root + off;
    }
    MaskNode n;
    n.kind = k;
    n.a = ra;
    n.b = rb;
    s.nodes.push_back(n);
    s.root = int(s.nodes.size()) - 1;
    return s;
  }

  MaskSym MaskSymOf(int v, int depth = 0) const {
    MaskSym none;
    if (depth > 64) return none;
    const Op* p = prod(v);
    if (!p) return none;
    const TensorType& t = m_.types[v];
    const int r = t.rank();
    const std::string& n = p->name;
    auto sub = [&](int w) { return MaskSymOf(w, depth + 1); };
    if (n == "stablehlo.iota") {
      const auto dd = attr_ints(*p, {"dim", "iota_dimension"});
      const int64_t d = dd.empty() ? 0 : dd[0];
      if (d < 0 || d >= r || !ExactIn(t.dims[size_t(d)] - 1, t.dtype)) return none;
      MaskSym s;
      s.kind = MaskSym::kAff;
      s.aff.c.assign(size_t(r), 0);
      s.aff.c[size_t(d)] = 1;
      return s;
    }
    if (n == "stablehlo.constant") {
      const Attr* a = ParsedConst(v);
      if (!a) return none;
      if (a->splat || t.numel() == 1) {
        if (t.dtype == DType::kPred) return PredConst(a->ivals.at(0) != 0);
        const double x = a->fvals.empty() ? double(a->ivals.at(0)) : a->fvals.at(0);
        if (!(std::fabs(x) < 9e15) || x != std::trunc(x)) return none;
        MaskSym s;
        s.kind = MaskSym::kAff;
        s.aff.c0 = int64_t(x);
        s.aff.c.assign(size_t(r), 0);
        return s;
      }
      MaskSym s;
      s.kind = MaskSym::kTable;
      s.table = a;
      s.table_dtype = t.dtype;
      s.tstride = DenseStrides(t.dims);
      for (int k = 0; k < r; ++k)
        if (t.dims[size_t(k)] == 1) s.tstride[size_t(k)] = 0;
      return s;
    }
    if (n == "stablehlo.broadcast_in_dim") {
      const auto dims = attr_ints(*p, {"dims", "broadcast_dimensions"});
      const auto& id = m_.types[p->operands[0]].dims;
      if (dims.size() != id.size()) return none;
      MaskSym s = sub(p->operands[0]);
      if (s.kind == MaskSym::kNone) return none;
      std::vector<int> from(size_t(r), -1);
      for (size_t k = 0; k < id.size(); ++k) {
        if (dims[k] < 0 || dims[k] >= r) return none;
        if (id[k] != 1) from[size_t(dims[k])] = int(k);
      }
      RemapSym(s, from);
      return s;
    }
    if (n == "stablehlo.transpose") {
      const auto perm = attr_ints(*p, {"dims", "permutation"});
      if (int(perm.size()) != r) return none;
      MaskSym s = sub(p->operands[0]);
      if (s.kind == MaskSym::kNone) return none;
      std::vector<int> from(static_cast<size_t>(r));
      for (int k = 0; k < r; ++k) from[size_t(k)] = int(perm[size_t(k)]);
      RemapSym(s, from);
      return s;
    }
    if (n == "stablehlo.reshape") {
      // only insertion / removal of unit axes
      const auto& id = m_.types[p->operands[0]].dims;
      std::vector<int> in_nu, out_nu;
      for (size_t k = 0; k < id.size(); ++k)
        if (id[k] != 1) in_nu.push_back(int(k));
      for (int k = 0; k < r; ++k)
        if (t.dims[size_t(k)] != 1) out_nu.push_back(k);
      if (in_nu.size() != out_nu.size()) return none;
      std::vector<int> from(size_t(r), -1);
      for (size_t k = 0; k < in_nu.size(); ++k) {
        if (id[size_t(in_nu[k])] != t.dims[size_t(out_nu[k])]) return none;
        from[size_t(out_nu[k])] = in_nu[k];
      }
      MaskSym s = sub(p->operands[0]);
      if (s.kind == MaskSym::kNone) return none;
      RemapSym(s, from);
      return s;
    }
    if (n == "stablehlo.convert") {
      const int w = p->operands[0];
      MaskSym s = sub(w);
      const DType to = t.dtype;
      if (s.kind == MaskSym::kAff) {
        if (to == DType::kPred || !ExactIn(AffBound(s.aff, t.dims), to)) return none;
        return s;
      }
      if (s.kind == MaskSym::kPred) return to == DType::kPred ? s : none;
      if (s.kind == MaskSym::kTable && s.cmp.empty()) {
        s.conv.push_back(to);
        return s;
      }
      return none;
    }
    if (n == "stablehlo.negate") {
      MaskSym s = sub(p->operands[0]);
      if (s.kind != MaskSym::kAff || IsUnsigned(t.dtype)) return none;
      s.aff.c0 = -s.aff.c0;
      for (auto& c : s.aff.c) c = -c;
      return s;
    }
    if (n == "stablehlo.not") {
      MaskSym s = sub(p->operands[0]);
      if (s.kind == MaskSym::kPred) return PredCombine(MaskNode::kNot, s, nullptr);
      return none;
    }
    if ((n == "stablehlo.and" || n == "stablehlo.or" || n == "stablehlo.xor") && p->operands.size() == 2) {
      if (t.dtype != DType::kPred) return none;
      MaskSym a = sub(p->operands[0]), b = sub(p->operands[1]);
      if (a.kind != MaskSym::kPred || b.kind != MaskSym::kPred) return none;
      return PredCombine(n == "stablehlo.and" ? MaskNode::kAnd : n == "stablehlo.or" ? MaskNode::kOr : MaskNode::kXor,
                         a, &b);
    }
    if ((n == "stablehlo.add" || n == "stablehlo.subtract" || n == "stablehlo.multiply") && p->operands.size() == 2) {
      if (t.dtype == DType::kPred) return none;
      MaskSym a = sub(p->operands[0]), b = sub(p->operands[1]);
      if (a.kind != MaskSym::kAff || b.kind != MaskSym::kAff) return none;
      MaskSym s;
      s.kind = MaskSym::kAff;
      s.aff.c.assign(size_t(r), 0);
      if (n == "stablehlo.multiply") {
        const bool a_const = std::all_of(a.aff.c.begin(), a.aff.c.end(), [](int64_t c) { return c == 0; });
        const bool b_const = std::all_of(b.aff.c.begin(), b.aff.c.end(), [](int64_t c) { return c == 0; });
        if (!a_const && !b_const) return none;
        const MaskAff& f = a_const ? b.aff : a.aff;
        const int64_t m = a_const ? a.aff.c0 : b.aff.c0;
        if (std::llabs(m) > (int64_t(1) << 20)) return none;
        s.aff.c0 = f.c0 * m;
        for (size_t k = 0; k < f.c.size(); ++k) s.aff.c[k] = f.c[k] * m;
      } else {
        const int64_t sg = n == "stablehlo.add" ? 1 : -1;
        s.aff.c0 = a.aff.c0 + sg * b.aff.c0;
        for (size_t k = 0; k < s.aff.c.size(); ++k) s.aff.c[k] = a.aff.c[k] + sg * b.aff.c[k];
      }
      // every intermediate value must be exact in the op's own type
      if (!ExactIn(AffBound(s.aff, t.dims), t.dtype)) return none;
      if (IsUnsigned(t.dtype)) return none;  // wrap-around is not affine
      return s;
    }
    if (n == "stablehlo.compare" && p->operands.size() == 2) {
      const std::string dir = CompareDirOf(*p);
      MaskSym a = sub(p->operands[0]), b = sub(p->operands[1]);
      if (a.kind == MaskSym::kAff && b.kind == MaskSym::kAff) {
        // d = a - b; integer-valued, so GT d >= 1, LT -d >= 1
        MaskAff d;
        d.c.assign(size_t(r), 0);
        d.c0 = a.aff.c0 - b.aff.c0;
        for (size_t k = 0; k < d.c.size(); ++k) d.c[k] = a.aff.c[k] - b.aff.c[k];
        auto leaf = [&](MaskAff f) {
          MaskSym s;
          s.kind = MaskSym::kPred;
          MaskNode x;
          x.kind = MaskNode::kLeaf;
          x.aff = std::move(f);
          s.nodes.push_back(x);
          s.root = 0;
          return s;
        };
        MaskAff neg = d;
        neg.c0 = -neg.c0;
        for (auto& c : neg.c) c = -c;
        if (dir == "GE") return leaf(d);
        if (dir == "LE") return leaf(neg);
        if (dir == "GT") { d.c0 -= 1; return leaf(d); }
        if (dir == "LT") { neg.c0 -= 1; return leaf(neg); }
        if (dir == "EQ" || dir == "NE") {
          // d == 0  <=>  d >= 0 and -d >= 0
          MaskSym ge = leaf(d), le = leaf(neg);
          MaskSym eq = PredCombine(MaskNode::kAnd, ge, &le);
          return dir == "EQ" ? eq : PredCombine(MaskNode::kNot, eq, nullptr);
        }
        return none;
      }
      // table OP splat constant (either side)
      double c = 0;
      bool ok = false;
      if (a.kind == MaskSym::kTable && a.cmp.empty() && scalar_of(p->operands[1], &c)) {
        CompareDir(dir, 0, 0, &ok);
        if (!ok) return none;
        a.cmp = dir;
        a.cmp_val = c;
        return a;
      }
      if (b.kind == MaskSym::kTable && b.cmp.empty() && scalar_of(p->operands[0], &c)) {
        static const std::map<std::string, std::string> flip = {{"GE", "LE"}, {"LE", "GE"}, {"GT", "LT"},
                                                                  {"LT", "GT"}, {"EQ", "EQ"}, {"NE", "NE"}};
        auto it = flip.find(dir);
        if (it == flip.end()) return none;
        b.cmp = it->second;
        b.cmp_val = c;
        return b;
      }
      return none;
    }
    if (n == "stablehlo.select" && p->operands.size() == 3 && t.dtype == DType::kPred) {
      // select(p, true, false) = p ; select(p, false, true) = not p
      MaskSym c = sub(p->operands[0]);
      MaskSym x = sub(p->operands[1]), y = sub(p->operands[2]);
      auto const_of = [](const MaskSym& s, bool* v) {
        if (s.kind != MaskSym::kPred || s.nodes.size() != 1 || s.nodes[0].kind != MaskNode::kConst) return false;
        *v = s.nodes[0].val;
        return true;
      };
      bool xv, yv;
      if (c.kind != MaskSym::kPred || !const_of(x, &xv) || !const_of(y, &yv)) return none;
      if (xv == yv) return PredConst(xv);
      return xv ? c : PredCombine(MaskNode::kNot, c, nullptr);
    }
    return none;
  }

  // Visible keys of row i under a predicate formula, as sorted disjoint
  // half-open intervals [lo, hi) within [0, Sk).  Only axes 2 (query) and 3
  // (key) may carry coefficients; the caller checks that.
  using Ivals = std::vector<std::pair<int64_t, int64_t>>;
  static Ivals IvUnion(const Ivals& a, const Ivals& b) {
    Ivals all = a;
    all.insert(all.end(), b.begin(), b.end());
    std::sort(all.begin(), all.end());
    Ivals out;
    for (auto& iv : all) {
      if (iv.first >= iv.second) continue;
      if (!out.empty() && iv.first <= out.back().second) out.back().second = std::max(out.back().second, iv.second);
      else out.push_back(iv);
    }
    return out;
  }
  static Ivals IvComplement(const Ivals& a, int64_t Sk) {
    Ivals out;
    int64_t at = 0;
    for (auto& iv : a) {
      if (iv.first > at) out.push_back({at, iv.first});
      at = std::max(at, iv.second);
    }
    if (at < Sk) out.push_back({at, Sk});
    return out;
  }
  static Ivals IvIntersect(const Ivals& a, const Ivals& b, int64_t Sk) {
    return IvComplement(IvUnion(IvComplement(a, Sk), IvComplement(b, Sk)), Sk);
  }
  static int64_t FloorDiv(int64_t a, int64_t b) {
    int64_t q = a / b;
    if ((a % b != 0) && ((a < 0) != (b < 0))) --q;
    return q;
  }
  static Ivals RowVisible(const std::vector<MaskNode>& nodes, int at, int64_t i, int64_t Sk) {
    const MaskNode& n = nodes[size_t(at)];
    switch (n.kind) {
      case MaskNode::kConst: return n.val ? Ivals{{0, Sk}} : Ivals{};
      case MaskNode::kLeaf: {
        // c0 + ci*i + cj*j >= 0
        const int64_t ci = n.aff.c.size() > 2 ? n.aff.c[2] : 0, cj = n.aff.c.size() > 3 ? n.aff.c[3] : 0;
        const int64_t base = n.aff.c0 + ci * i;
        if (cj == 0) return base >= 0 ? Ivals{{0, Sk}} : Ivals{};
        if (cj > 0) {  // j >= ceil(-base / cj)
          const int64_t lo = -FloorDiv(base, cj);
          return IvUnion({{std::max<int64_t>(lo, 0), Sk}}, {});
        }
        const int64_t hi = FloorDiv(base, -cj);  // j <= floor(base / -cj)
        return IvUnion({{0, std::min<int64_t>(hi + 1, Sk)}}, {});
      }
      case MaskNode::kNot: return IvComplement(RowVisible(nodes, n.a, i, Sk), Sk);
      case MaskNode::kAnd: return IvIntersect(RowVisible(nodes, n.a, i, Sk), RowVisible(nodes, n.b, i, Sk), Sk);
      case MaskNode::kOr: return IvUnion(RowVisible(nodes, n.a, i, Sk), RowVisible(nodes, n.b, i, Sk));
      case MaskNode::kXor: {
        const Ivals x = RowVisible(nodes, n.a, i, Sk), y = RowVisible(nodes, n.b, i, Sk);
        return IvUnion(IvIntersect(x, IvComplement(y, Sk), Sk), IvIntersect(IvComplement(x, Sk), y, Sk));
      }
    }
    return {};
  }

  // 1 = causal (key j visible iff j <= i), 0 = all visible, -1 = anything
  // else.  Exact: every query row (and every (b, h) a dense table varies
  // over) is checked, never a sample.
  int ClassifyMask(int mask, int64_t B, int64_t H, int64_t Sq, int64_t Sk) const {
    const TensorType& mt = m_.types[mask];
    if (mt.rank() != 4 || mt.dims != std::vector<int64_t>{B, H, Sq, Sk}) return -1;
    MaskSym s = MaskSymOf(mask);
    bool causal = true, all = true;
    if (s.kind == MaskSym::kPred) {
      for (const auto& n : s.nodes)
        if (n.kind == MaskNode::kLeaf && ((B > 1 && n.aff.c[0] != 0) || (H > 1 && n.aff.c[1] != 0))) return -1;
      for (int64_t i = 0; i < Sq && (causal || all); ++i) {
        const Ivals v = RowVisible(s.nodes, s.root, i, Sk);
        const Ivals full{{0, Sk}};
        const Ivals tri{{0, std::min(i + 1, Sk)}};
        all &= v == full;
        causal &= v == tri;
      }
    } else if (s.kind == MaskSym::kTable) {
      const Attr& a = *s.table;
      const bool fl = IsFloat(s.table_dtype);
      const int64_t nb = s.tstride[0] ? B : 1, nh = s.tstride[1] ? H : 1;
      for (int64_t b = 0; b < nb; ++b)
        for (int64_t h = 0; h < nh; ++h)
          for (int64_t i = 0; i < Sq && (causal || all); ++i)
            for (int64_t j = 0; j < Sk; ++j) {
              const int64_t e = s.toff + b * s.tstride[0] + h * s.tstride[1] + i * s.tstride[2] + j * s.tstride[3];
              double x = fl ? a.fvals.at(size_t(e)) : double(a.ivals.at(size_t(e)));
              for (DType d : s.conv) x = ConvertScalar(x, d);
              bool vis = x != 0;
              if (!s.cmp.empty()) {
                bool ok;
                vis = CompareDir(s.cmp, x, s.cmp_val, &ok);
              }
              all &= vis;
              causal &= vis == (j <= i);
            }
    } else {
      return -1;
    }
    if (all) return 0;
    return causal ? 1 : -1;
  }

  bool is_reduce_over_last(int v, const char* body, int rank) const {
    const Op* p = prod(v);
    if (!p || p->name != "stablehlo.reduce" || p->operands.size() != 2) return false;
    const auto dims = reduce_dims(*p);
    return dims.size() == 1 && dims[0] == rank - 1 && reduce_body_op(*p) == body;
  }

  // softmax(S) along the last axis, as jax.nn.softmax lowers it:
  //   M = reduce_max(S)            [optionally max(M, -inf) for `initial`]
  //   E = exp(S - broadcast(M))
  //   P = E / broadcast(reduce_sum(E))   [sum possibly on an f32 convert of E]
  // returns S (the softmax input) and records the matched ops.
  int MatchSoftmax(int P, std::set<int>& ops) const {
    std::vector<int> path;
    const Op* div = prod(P);
    if (!div || div->name != "stablehlo.divide") return -1;
    ops.insert(producer_[P]);
    const int rank = m_.types[P].rank();
    int E = div->operands[0];
    int Z = div->operands[1];
    // Z = broadcast(reshape?(convert?(reduce_sum(convert?(E)))))
    int z = Z;
    while (is(z, "stablehlo.broadcast_in_dim") || is(z, "stablehlo.reshape") || is(z, "stablehlo.convert")) {
      ops.insert(producer_[z]);
      z = prod(z)->operands[0];
    }
    if (!is_reduce_over_last(z, "stablehlo.add", rank)) return -1;
    ops.insert(producer_[z]);
    std::vector<int> p2;
    int e_in_sum = through_converts(prod(z)->operands[0], &p2);
    for (int o : p2) ops.insert(o);
    int e_main = through_converts(E, &path);
    for (int o : path) ops.insert(o);
    if (e_in_sum != e_main) return -1;
    const Op* ex = prod(e_main);
    if (!ex || ex->name != "stablehlo.exponential") return -1;
    ops.insert(producer_[e_main]);
    const Op* sub = prod(ex->operands[0]);
    if (!sub || sub->name != "stablehlo.subtract") return -1;
    ops.insert(producer_[ex->operands[0]]);
    const int S = sub->operands[0];
    int m = sub->operands[1];
    while (is(m, "stablehlo.broadcast_in_dim") || is(m, "stablehlo.reshape") || is(m, "stablehlo.convert") ||
           is(m, "stablehlo.maximum")) {
      ops.insert(producer_[m]);
      const Op* q = prod(m);
      if (q->name == "stablehlo.maximum") {
        double c;
        // max(M, -inf) (jnp.max `initial`): keep the non-constant side
        if (scalar_of(q->operands[0], &c)) m = q->operands[1];
        else if (scalar_of(q->operands[1], &c)) m = q->operands[0];
        else return -1;
        if (!(c < -1e30)) return -1;
        continue;
      }
      m = q->operands[0];
    }
    if (!is_reduce_over_last(m, "stablehlo.maximum", rank)) return -1;
    ops.insert(producer_[m]);
    std::vector<int> p3;
    if (through_converts(prod(m)->operands[0], &p3) != through_converts(S)) return -1;
    for (int o : p3) ops.insert(o);
    return S;
  }

  // The attention forward anchored at the P·V product: Q·Kᵀ (bf16
  // operands), scale, optional mask select, softmax, P·V.
  struct SdpaFwdMatch {
    std::set<int> ops;  // matched ops, anchor included
    int q = -1, k = -1, v = -1;
    int pr = -1;        // the softmax output (the divide)
    int mask = -1;
    float scale = 1.f;
    bool causal = false;
  };
  bool MatchSdpaFwd(int anchor, SdpaFwdMatch& r) {
    const Op& d2 = ops_[anchor];
    const int P = d2.operands[0], V = d2.operands[1];
    const TensorType& pt = m_.types[P];
    const TensorType& vt = m_.types[V];
    if (pt.rank() != 4 || vt.rank() != 4) return false;
    DotDims dd = dot_dims(d2);
    if (dd.lb != std::vector<int64_t>{0, 1} || dd.rb != std::vector<int64_t>{0, 1} ||
        dd.lc != std::vector<int64_t>{3} || dd.rc != std::vector<int64_t>{2})
      return false;
    std::set<int>& ops = r.ops;
    ops.insert(anchor);
    std::vector<int> path;
    const int Pin = through_converts(P, &path);
    for (int o : path) ops.insert(o);
    int S = MatchSoftmax(Pin, ops);
    if (S < 0) return false;
    r.pr = Pin;
    // mask: select(mask, scores, -inf)
    int mask = -1;
    int sc = S;
    if (is(sc, "stablehlo.select")) {
      const Op* sel = prod(sc);
      double c;
      if (!scalar_of(sel->operands[2], &c) || !(c < -1e30)) return false;
      mask = sel->operands[0];
      ops.insert(producer_[sc]);
      sc = sel->operands[1];
    }
    path.clear();
    sc = through_converts(sc, &path);
    for (int o : path) ops.insert(o);
    // scale: multiply / divide by a splat constant (either side for multiply)
    float scale = 1.f;
    if (is(sc, "stablehlo.multiply") || is(sc, "stablehlo.divide")) {
      const Op* s = prod(sc);
      double c;
      if (s->name == "stablehlo.multiply" && scalar_of(s->operands[1], &c)) {
        scale = float(c);
        ops.insert(producer_[sc]);
        sc = s->operands[0];
      } else if (s->name == "stablehlo.multiply" && scalar_of(s->operands[0], &c)) {
        scale = float(c);
        ops.insert(producer_[sc]);
        sc = s->operands[1];
      } else if (s->name == "stablehlo.divide" && scalar_of(s->operands[1], &c)) {
        scale = float(1.0 / c);
        ops.insert(producer_[sc]);
        sc = s->operands[0];
      }
    }
    path.clear();
    sc = through_converts(sc, &path);
    for (int o : path) ops.insert(o);
    const Op* d1 = prod(sc);
    if (!d1 || d1->name != "stablehlo.dot_general") return false;
    DotDims e = dot_dims(*d1);
    if (e.lb != std::vector<int64_t>{0, 1} || e.rb != std::vector<int64_t>{0, 1} ||
        e.lc != std::vector<int64_t>{3} || e.rc != std::vector<int64_t>{3})
      return false;
    ops.insert(producer_[sc]);
    const int Q = d1->operands[0], K = d1->operands[1];
    const TensorType& qt = m_.types[Q];
    const TensorType& kt = m_.types[K];
    if (qt.dtype != DType::kBF16 || kt.dtype != DType::kBF16 || vt.dtype != DType::kBF16) return false;
    const int64_t D = qt.dims[3];
    if ((D != 64 && D != 128) || vt.dims[3] != D) return false;
    bool causal = false;
    if (mask >= 0) {
      const int cls = ClassifyMask(mask, qt.dims[0], qt.dims[1], qt.dims[2], kt.dims[2]);
      if (cls < 0) return false;
      causal = cls == 1;
    }
    r.q = Q;
    r.k = K;
    r.v = V;
    r.mask = mask;
    r.scale = scale;
    r.causal = causal;
    return true;
  }

  void TryMatchSdpa(int anchor) {
    SdpaFwdMatch r;
    if (!MatchSdpaFwd(anchor, r)) return;
    const Op& d2 = ops_[anchor];
    bool inside = m_.types[d2.results[0]].dtype == DType::kBF16;
    // every intermediate result must stay inside the pattern
    for (int o : r.ops)
      for (int res : ops_[o].results)
        if (o != anchor && !uses_within(res, r.ops)) inside = false;
    if (!inside) {
      TryMatchSdpaTrain(anchor, r);
      return;
    }
    Fused f;
    f.kind = Fused::kSdpa;
    f.q = r.q;
    f.k = r.k;
    f.v = r.v;
    f.scale = r.scale;
    f.causal = r.causal;
    f.deps = {r.q, r.k, r.v};
    fused_[anchor] = f;
    prog_->patterns.push_back(std::string("sdpa(") + (r.causal ? "causal" : "full") + ", scale=" +
                              std::to_string(r.scale) + ")");
  }

  // The attention forward together with the backward jax.grad emits for it
  // (jax.nn.softmax's rule dS = P (dP - sum(P dP)) over the last axis):
  //   dVᵀ = dot(dO, P) over the queries, dV = transpose(dVᵀ)
  //   dP  = dot(dO, V) over D
  //   G   = dP * P,  dS = G - P * bcast(sum(G))
  //   [select(mask, dS, 0)] * scale -> bf16 -> dQ = dot(., K), dK = dot(., Q)
  // The forward becomes mk_sdpa_fwd with lse (and its bf16 O kept), the
  // backward one mk_sdpa_bwd step anchored at the first of its products;
  // nothing S x S is formed.  Users that do not reach an output (transposes
  // toward constants) are ignored.
  void TryMatchSdpaTrain(int anchor, const SdpaFwdMatch& r) {
    const Op& d2 = ops_[anchor];
    const int Pbf = d2.operands[0], Vb = d2.operands[1];
    const TensorType& qt = m_.types[r.q];
    const TensorType& kt = m_.types[r.k];
    const int64_t B = qt.dims[0], H = qt.dims[1], Sq = qt.dims[2], Sk = kt.dims[2], D = qt.dims[3];
    auto dims_are = [&](int v, std::vector<int64_t> d) { return m_.types[v].dims == d; };
    auto find_user = [&](int v, const char* name, auto pred) -> int {
      for (int u : live_users(v))
        if (ops_[u].name == name && pred(ops_[u])) return u;
      return -1;
    };
    auto dot_is = [&](const Op& o, std::vector<int64_t> lc, std::vector<int64_t> rc) {
      DotDims dd = dot_dims(o);
      return dd.lb == std::vector<int64_t>{0, 1} && dd.rb == std::vector<int64_t>{0, 1} && dd.lc == lc && dd.rc == rc;
    };
    auto other = [](const Op& o, int v) { return o.operands[0] == v ? o.operands[1] : o.operands[0]; };
    std::set<int> bw;
    // dVᵀ = dot(dO, P) contracting the query dims, then the transpose to dV
    int dvt = -1, dO = -1;
    for (int u : live_users(Pbf)) {
      const Op& o = ops_[u];
      if (u != anchor && o.name == "stablehlo.dot_general" && o.operands.size() == 2 && o.operands[1] == Pbf &&
          dot_is(o, {2}, {2})) {
        dvt = u;
        dO = o.operands[0];
      }
    }
    if (dvt < 0 || m_.types[dO].dtype != DType::kBF16 || !dims_are(dO, {B, H, Sq, D})) return;
    bw.insert(dvt);
    const int dvt_v = ops_[dvt].results[0];
    const auto dvt_users = live_users(dvt_v);
    if (dvt_users.size() != 1 || ops_[dvt_users[0]].name != "stablehlo.transpose") return;
    if (attr_ints(ops_[dvt_users[0]], {"permutation", "dims"}) != std::vector<int64_t>{0, 1, 3, 2}) return;
    bw.insert(dvt_users[0]);
    const int dv = ops_[dvt_users[0]].results[0];
    // dP = dot(dO, V) over D
    const int dpd = find_user(dO, "stablehlo.dot_general", [&](const Op& o) {
      return o.operands.size() == 2 && o.operands[0] == dO && o.operands[1] == Vb && dot_is(o, {3}, {3});
    });
    if (dpd < 0) return;
    bw.insert(dpd);
    const int dP = ops_[dpd].results[0];
    // G = dP * P
    const int gm = find_user(dP, "stablehlo.multiply", [&](const Op& o) { return other(o, dP) == r.pr; });
    if (gm < 0) return;
    bw.insert(gm);
    const int G = ops_[gm].results[0];
    // t = sum(G) over the keys, P * bcast(t), dS = G - that
    int tsum = -1;
    for (int u : live_users(G))
      if (ops_[u].name == "stablehlo.reduce" && is_reduce_over_last(ops_[u].results[0], "stablehlo.add", 4)) tsum = u;
    if (tsum < 0) return;
    bw.insert(tsum);
    // the row sums [B,H,Sq] must come back along the keys: follow where each
    // of their three axes lands through the broadcasts, and reshapes that
    // only add or drop trailing unit dims, and require it to be {0,1,2}
    int tb = ops_[tsum].results[0];
    std::vector<int64_t> at = {0, 1, 2};
    while (true) {
      const auto us = live_users(tb);
      if (us.size() != 1) return;
      const Op& o = ops_[us[0]];
      if (o.name == "stablehlo.broadcast_in_dim") {
        const auto bd = attr_ints(o, {"dims", "broadcast_dimensions"});
        if (bd.size() != size_t(m_.types[tb].rank())) return;
        for (auto& a : at) a = bd[size_t(a)];
      } else if (o.name == "stablehlo.reshape") {
        const auto& from = m_.types[tb].dims;
        const auto& to = m_.types[o.results[0]].dims;
        const size_t common = std::min(from.size(), to.size());
        if (common < 3) return;
        for (size_t i = 0; i < common; ++i)
          if (from[i] != to[i]) return;
        for (size_t i = common; i < from.size(); ++i)
          if (from[i] != 1) return;
        for (size_t i = common; i < to.size(); ++i)
          if (to[i] != 1) return;
        for (auto a : at)
          if (size_t(a) >= common) return;
      } else {
        break;
      }
      bw.insert(us[0]);
      tb = o.results[0];
      if (dims_are(tb, {B, H, Sq, Sk})) break;
    }
    if (!dims_are(tb, {B, H, Sq, Sk}) || at != std::vector<int64_t>{0, 1, 2}) return;
    const int pm = find_user(tb, "stablehlo.multiply", [&](const Op& o) { return other(o, tb) == r.pr; });
    if (pm < 0) return;
    bw.insert(pm);
    const int PT = ops_[pm].results[0];
    const int dsub = find_user(G, "stablehlo.subtract", [&](const Op& o) {
      return o.operands[0] == G && o.operands[1] == PT;
    });
    if (dsub < 0) return;
    bw.insert(dsub);
    int dS = ops_[dsub].results[0];
    // select(mask, dS, 0) where the forward was masked
    if (r.mask >= 0) {
      const int sel = find_user(dS, "stablehlo.select", [&](const Op& o) {
        double c;
        return o.operands[1] == dS && scalar_of(o.operands[2], &c) && c == 0.0 &&
               (o.operands[0] == r.mask ||
                ClassifyMask(o.operands[0], B, H, Sq, Sk) == (r.causal ? 1 : 0));
      });
      if (sel < 0) return;
      bw.insert(sel);
      dS = ops_[sel].results[0];
    }
    // times the scale (splat constant, either side)
    const int sm = find_user(dS, "stablehlo.multiply", [&](const Op& o) {
      double c;
      return scalar_of(other(o, dS), &c) && float(c) == r.scale;
    });
    if (sm < 0) return;
    bw.insert(sm);
    const int dSs = ops_[sm].results[0];
    // bf16, then dQ = dot(dS, K) over the keys and dK = dot(dS, Q) over the queries
    const auto cu = live_users(dSs);
    if (cu.size() != 1 || ops_[cu[0]].name != "stablehlo.convert") return;
    bw.insert(cu[0]);
    const int dSb = ops_[cu[0]].results[0];
    if (m_.types[dSb].dtype != DType::kBF16) return;
    const int dqd = find_user(dSb, "stablehlo.dot_general", [&](const Op& o) {
      return o.operands.size() == 2 && o.operands[0] == dSb && o.operands[1] == r.k && dot_is(o, {3}, {2});
    });
    const int dkd = find_user(dSb, "stablehlo.dot_general", [&](const Op& o) {
      return o.operands.size() == 2 && o.operands[0] == dSb && o.operands[1] == r.q && dot_is(o, {2}, {2});
    });
    if (dqd < 0 || dkd < 0) return;
    bw.insert(dqd);
    bw.insert(dkd);
    const int dq = ops_[dqd].results[0], dk = ops_[dkd].results[0];
    if (!dims_are(dq, {B, H, Sq, D}) || !dims_are(dk, {B, H, Sk, D}) || !dims_are(dv, {B, H, Sk, D})) return;
    // everything else stays inside forward + backward
    std::set<int> all = r.ops;
    all.insert(bw.begin(), bw.end());
    const std::set<int> outs = {d2.results[0], dq, dk, dv};
    for (int o : all)
      for (int res : ops_[o].results) {
        if (outs.count(res)) continue;
        for (int oo : outputs_)
          if (oo == res) return;
        for (int u : live_users(res))
          if (!all.count(u)) return;
      }
    // the backward runs at its first product, after the forward
    const int banchor = std::min(dvt, dpd);
    if (banchor <= anchor || fused_.count(banchor)) return;
    Fused f;
    f.kind = Fused::kSdpa;
    f.train = true;
    f.q = r.q;
    f.k = r.k;
    f.v = r.v;
    f.scale = r.scale;
    f.causal = r.causal;
    f.deps = {r.q, r.k, r.v};
    fused_[anchor] = f;
    Fused b;
    b.kind = Fused::kSdpaBwd;
    b.q = r.q;
    b.k = r.k;
    b.v = r.v;
    b.dout = dO;
    b.fwd = anchor;
    b.dq = dq;
    b.dk = dk;
    b.dv = dv;
    b.scale = r.scale;
    b.causal = r.causal;
    b.deps = {r.q, r.k, r.v, dO, d2.results[0]};
    fused_[banchor] = b;
    for (int o : all)
      if (o != anchor && o != banchor) absorbed_.insert(o);
    prog_->patterns.push_back(std::string("sdpa_train(") + (r.causal ? "causal" : "full") + ", scale=" +
                              std::to_string(r.scale) + ")");
  }

  // value of a scalar expression of splat constants (multiply, divide,
  // negate, add, subtract; broadcasts and reshapes looked through)
  bool const_eval(int v, double* out, int depth = 0) const {
    if (scalar_of(v, out)) return true;
    const Op* p = prod(v);
    if (!p || depth > 8 || m_.types[v].numel() != 1) return false;
    if (p->name == "stablehlo.broadcast_in_dim" || p->name == "stablehlo.reshape")
      return const_eval(p->operands[0], out, depth + 1);
    if (p->name == "stablehlo.negate") {
      if (!const_eval(p->operands[0], out, depth + 1)) return false;
      *out = -*out;
      return true;
    }
    double a, b;
    if (p->operands.size() != 2 || !const_eval(p->operands[0], &a, depth + 1) ||
        !const_eval(p->operands[1], &b, depth + 1))
      return false;
    if (p->name == "stablehlo.multiply") *out = a * b;
    else if (p->name == "stablehlo.divide") *out = a / b;
    else if (p->name == "stablehlo.add") *out = a + b;
    else if (p->name == "stablehlo.subtract") *out = a - b;
    else return false;
    if (m_.types[v].dtype == DType::kF32) *out = float(*out);
    return true;
  }

  // Softmax cross-entropy with integer labels over the rows of fp32 / bf16
  // logits X [T, V], with the gradient jax.grad emits for its mean:
  //   M = max(X) (behind stop_gradient), E = exp(X - M), Z = sum(E)
  //   loss_rows = (log Z + M) - sum(select(X's column == label, X, 0))
  //   dX = select(onehot, bcast(-g), 0) + bcast(g / Z) * E
  // with g = bcast(c) the per-row cotangent of a constant c (1/T for the
  // mean).  Anchored at the loss_rows subtract: one mk_softmax_xent launch
  // writes loss_rows and dX (which no other op computes then).  A label
  // outside [0, V) drops the target term there, as the module's select does.
  void TryMatchXent(int anchor) {
    const Op& dsub = ops_[anchor];
    const int LSE = dsub.operands[0], PK = dsub.operands[1];
    if (m_.types[LSE].rank() != 1) return;
    const int64_t T = m_.types[LSE].dims[0];
    std::set<int> ops = {anchor};
    auto row_bcast_of = [&](int v, int* src) {  // broadcast_in_dim [T] -> [T, V] along dim 0
      const Op* b = prod(v);
      if (!b || b->name != "stablehlo.broadcast_in_dim" || attr_ints(*b, {"dims", "broadcast_dimensions"}) != std::vector<int64_t>{0})
        return false;
      *src = b->operands[0];
      return m_.types[*src].rank() == 1;
    };
    // lse = log(Z) + M
    const Op* ad = prod(LSE);
    if (!ad || ad->name != "stablehlo.add") return;
    ops.insert(producer_[LSE]);
    int LG = ad->operands[0], M = ad->operands[1];
    if (!is(LG, "stablehlo.log")) std::swap(LG, M);
    if (!is(LG, "stablehlo.log")) return;
    ops.insert(producer_[LG]);
    const int Z = prod(LG)->operands[0];
    if (!is_reduce_over_last(Z, "stablehlo.add", 2)) return;
    ops.insert(producer_[Z]);
    const int E = prod(Z)->operands[0];
    if (!is(E, "stablehlo.exponential")) return;
    ops.insert(producer_[E]);
    const int SH = prod(E)->operands[0];
    if (!is(SH, "stablehlo.subtract")) return;
    ops.insert(producer_[SH]);
    const int X = prod(SH)->operands[0];
    int Msrc = -1;
    if (!row_bcast_of(prod(SH)->operands[1], &Msrc) || Msrc != M) return;
    ops.insert(producer_[prod(SH)->operands[1]]);
    if (!is_reduce_over_last(M, "stablehlo.maximum", 2) || prod(M)->operands[0] != X) return;
    ops.insert(producer_[M]);
    const TensorType& xt = m_.types[X];
    if (xt.rank() != 2 || xt.dims[0] != T || (xt.dtype != DType::kF32 && xt.dtype != DType::kBF16)) return;
    const int64_t V = xt.dims[1];
    // picked = sum(select(onehot, X, 0)); onehot = compare EQ (iota over dim 1, bcast(labels))
    if (!is_reduce_over_last(PK, "stablehlo.add", 2)) return;
    ops.insert(producer_[PK]);
    const int SEL = prod(PK)->operands[0];
    if (!is(SEL, "stablehlo.select")) return;
    const Op* sel = prod(SEL);
    double z;
    if (sel->operands[1] != X || !scalar_of(sel->operands[2], &z) || z != 0.0) return;
    ops.insert(producer_[SEL]);
    const int OH = sel->operands[0];
    const Op* cmp = prod(OH);
    if (!cmp || cmp->name != "stablehlo.compare") return;
    {
      std::string d;
      if (const Attr* x = cmp->attr("comparison_direction")) d = x->s;
      else if (const Attr* x = cmp->attr("enum0")) d = x->s;
      if (d != "EQ") return;
    }
    int IO = cmp->operands[0], LB = cmp->operands[1];
    if (!is(IO, "stablehlo.iota")) std::swap(IO, LB);
    if (!is(IO, "stablehlo.iota") || attr_ints(*prod(IO), {"dim", "iota_dimension"}) != std::vector<int64_t>{1}) return;
    int lab = -1;
    if (!row_bcast_of(LB, &lab)) return;
    while (is(lab, "stablehlo.convert")) lab = prod(lab)->operands[0];
    const DType lt = m_.types[lab].dtype;
    if (m_.types[lab].rank() != 1 || (lt != DType::kI32 && lt != DType::kI64)) return;
    ops.insert(producer_[OH]);
    ops.insert(producer_[LB]);
    ops.insert(producer_[IO]);
    // the gradient: add(select(onehot, bcast(-g), 0), mul(bcast(g / Z), E))
    int dX = -1, gscale_v = -1;
    for (int u : live_users(OH)) {
      if (u == producer_[SEL] || ops_[u].name != "stablehlo.select") continue;
      const Op& s2 = ops_[u];
      double zz;
      int negsrc = -1;
      if (s2.operands[0] != OH || !scalar_of(s2.operands[2], &zz) || zz != 0.0 || !row_bcast_of(s2.operands[1], &negsrc) ||
          !is(negsrc, "stablehlo.negate"))
        continue;
      const int g = prod(negsrc)->operands[0];
      const auto us = live_users(s2.results[0]);
      if (us.size() != 1 || ops_[us[0]].name != "stablehlo.add") continue;
      const Op& a2 = ops_[us[0]];
      const int other_t = a2.operands[0] == s2.results[0] ? a2.operands[1] : a2.operands[0];
      const Op* m2 = prod(other_t);
      if (!m2 || m2->name != "stablehlo.multiply") continue;
      int bsrc = -1;
      const int mb = m2->operands[0] == E ? m2->operands[1] : m2->operands[0];
      if ((m2->operands[0] != E && m2->operands[1] != E) || !row_bcast_of(mb, &bsrc) || !is(bsrc, "stablehlo.divide"))
        continue;
      const Op* dv = prod(bsrc);
      if (dv->operands[0] != g || dv->operands[1] != Z) continue;
      ops.insert(u);
      ops.insert(producer_[s2.operands[1]]);
      ops.insert(producer_[negsrc]);
      ops.insert(us[0]);
      ops.insert(producer_[other_t]);
      ops.insert(producer_[mb]);
      ops.insert(producer_[bsrc]);
      dX = a2.results[0];
      gscale_v = g;
    }
    if (dX < 0) return;
    // g: the row broadcast of a constant
    const Op* gb = prod(gscale_v);
    if (!gb || gb->name != "stablehlo.broadcast_in_dim") return;
    double gscale;
    if (!const_eval(gb->operands[0], &gscale)) return;
    ops.insert(producer_[gscale_v]);
    // every other result stays inside
    for (int o : ops)
      for (int res : ops_[o].results) {
        if (res == dsub.results[0] || res == dX) continue;
        for (int oo : outputs_)
          if (oo == res) return;
        for (int u : live_users(res))
          if (!ops.count(u)) return;
      }
    if (m_.types[dX].dtype != xt.dtype || m_.types[dsub.results[0]].dtype != DType::kF32) return;
    Fused f;
    f.kind = Fused::kXent;
    f.x = X;
    f.labels = lab;
    f.dlogits = dX;
    f.scale = float(gscale);
    f.deps = {X, lab};
    // f32 logits whose gradient is only read through converts to bf16 (the
    // operands of the two products of the vocabulary projection's backward):
    // the kernel writes the bf16 gradient, and neither the f32 gradient nor
    // the conversion pass exists
    if (xt.dtype == DType::kF32 && std::count(outputs_.begin(), outputs_.end(), dX) == 0) {
      const auto us = live_users(dX);
      bool all_bf16 = !us.empty();
      for (int u : us)
        all_bf16 = all_bf16 && ops_[u].name == "stablehlo.convert" &&
                   m_.types[ops_[u].results[0]].dtype == DType::kBF16;
      if (all_bf16)
        for (int u : us) {
          f.dlogits_bf16.push_back(ops_[u].results[0]);
          ops.insert(u);
        }
    }
    fused_[anchor] = f;
    for (int o : ops)
      if (o != anchor) absorbed_.insert(o);
    // rows padded to 8 elements (16 bytes of bf16, 32 of f32): the logits
    // when a product writes them (through reshapes: its result's last dim is
    // the vocabulary), and the gradient the kernel writes
    if (V % 8 != 0) {
      const int64_t pitch = (V + 7) / 8 * 8;
      auto not_output = [&](int v) { return std::count(outputs_.begin(), outputs_.end(), v) == 0; };
      int src = X;
      while (is(src, "stablehlo.reshape") && m_.types[prod(src)->operands[0]].dims.back() == V)
        src = prod(src)->operands[0];
      if ((is(src, "stablehlo.dot_general") || is(src, "stablehlo.dot")) && not_output(src) &&
          m_.types[src].dims.back() == V)
        pad_rows_[src] = pitch;
      if (f.dlogits_bf16.empty()) {
        if (not_output(dX)) pad_rows_[dX] = pitch;
      } else {
        bool ok = true;
        for (int c : f.dlogits_bf16) ok = ok && not_output(c);
        if (ok)
          for (int c : f.dlogits_bf16) pad_rows_[c] = pitch;
      }
    }
    prog_->patterns.push_back("softmax_xent(" + std::to_string(T) + "x" + std::to_string(V) + ", grad_scale=" +
                              std::to_string(gscale) + ")");
  }

  void TryMatchArgmax(int anchor) {
    const Op& r = ops_[anchor];
    const auto dims = reduce_dims(r);
    if (dims.size() != 1) return;
    // direction from the first compare in the body (reduce.mm:29-43)
    int dir = 0;
    if (!r.regions.empty())
      for (const Op& b : r.regions[0]->blocks[0].ops)
        if (b.name == "stablehlo.compare") {
          std::string d;
          if (const Attr* x = b.attr("comparison_direction")) d = x->s;
          else if (const Attr* x = b.attr("enum0")) d = x->s;
          dir = d == "GT" ? 1 : d == "LT" ? -1 : 0;
          break;
        }
    if (dir == 0) return;
    // second operand must be an iota along the reduced dimension
    int ix = r.operands[1];
    int dim_in_iota = int(dims[0]);
    while (is(ix, "stablehlo.broadcast_in_dim")) {
      const Op* b = prod(ix);
      const auto bd = attr_ints(*b, {"dims", "broadcast_dimensions"});
      auto it = std::find(bd.begin(), bd.end(), int64_t(dim_in_iota));
      if (it == bd.end()) return;
      dim_in_iota = int(it - bd.begin());
      ix = b->operands[0];
    }
    if (!is(ix, "stablehlo.iota")) return;
    const auto idim = attr_ints(*prod(ix), {"dim", "iota_dimension"});
    if (idim.empty() || idim[0] != dim_in_iota) return;
    const DType xt = m_.types[r.operands[0]].dtype;
    if (xt != DType::kBF16 && xt != DType::kF32 && xt != DType::kF16) return;
    const DType it_ = m_.types[r.results[1]].dtype;
    if (it_ != DType::kI32 && it_ != DType::kI64) return;
    Fused f;
    f.kind = Fused::kArgmax;
    f.x = r.operands[0];
    f.is_min = dir < 0;
    f.deps = {f.x};
    fused_[anchor] = f;
    prog_->patterns.push_back(dir > 0 ? "argmax" : "argmin");
  }

  // add(dot_general(a, b), broadcast_in_dim(bias, dims=[last])) [-> max(., 0)]
  void TryMatchGemmEpilogue(int add_idx) {
    const Op& add = ops_[add_idx];
    for (int side = 0; side < 2; ++side) {
      const int d = add.operands[side], bb = add.operands[1 - side];
      const Op* dot = prod(d);
      if (!dot || dot->name != "stablehlo.dot_general" || uses_[d] != 1 || fused_.count(producer_[d])) continue;
      const TensorType& ot = m_.types[add.results[0]];
      if (ot.rank() != 2) continue;
      // bias: a chain of broadcast_in_dim / reshape from a 1-D [N] vector
      // that places the vector on the last output dim
      int b = bb;
      std::vector<const Op*> chain;
      while ((is(b, "stablehlo.broadcast_in_dim") || is(b, "stablehlo.reshape")) && m_.types[b].rank() >= 1 &&
             !(m_.types[b].rank() == 1)) {
        chain.push_back(prod(b));
        b = prod(b)->operands[0];
      }
      bool ok = !chain.empty() && m_.types[b].rank() == 1 && m_.types[b].dims[0] == ot.dims[1];
      int pos = 0;  // position of the vector's dim, innermost op outwards
      for (auto it = chain.rbegin(); ok && it != chain.rend(); ++it) {
        const Op* p = *it;
        const auto& rd = m_.types[p->results[0]].dims;
        if (p->name == "stablehlo.broadcast_in_dim") {
          const auto dd = attr_ints(*p, {"dims", "broadcast_dimensions"});
          ok = pos < int(dd.size());
          if (ok) pos = int(dd[pos]);
        } else {  // reshape that only adds / removes unit dims
          int found = -1, nonunit = 0;
          for (size_t k = 0; k < rd.size(); ++k)
            if (rd[k] != 1) {
              ++nonunit;
              found = int(k);
            }
          ok = nonunit == 1 && rd[found] == ot.dims[1];
          pos = found;
        }
      }
      ok = ok && pos == ot.rank() - 1;
      if (!ok || m_.types[b].dtype != ot.dtype) continue;
      Fused f;
      f.kind = Fused::kGemmEpi;
      f.dot = producer_[d];
      f.bias = b;
      int anchor = add_idx;
      // max(add, 0) -> relu
      if (uses_[add.results[0]] == 1 && users_[add.results[0]].size() == 1) {
        const int u = users_[add.results[0]][0];
        const Op& mx = ops_[u];
        if (mx.name == "stablehlo.maximum") {
          const int other = mx.operands[0] == add.results[0] ? mx.operands[1] : mx.operands[0];
          double c;
          if (scalar_of(other, &c) && c == 0.0) {
            f.relu = true;
            anchor = u;
          }
        }
      }
      f.deps = {dot->operands[0], dot->operands[1], b};
      fused_[anchor] = f;
      absorbed_.insert(f.dot);
      if (anchor != add_idx) absorbed_.insert(add_idx);
      prog_->patterns.push_back(f.relu ? "gemm+bias+relu" : "gemm+bias");
      return;
    }
  }

  // gelu_tanh(X) = X * (0.5 * (1 + tanh(c * (X + 0.044715 * X^3)))) as
  // jax.nn.gelu(approximate=True) lowers it (X^3 = X * (X * X)); either order
  // of every commutative op.  X is f32 (optionally convert(bf16)); a
  // convert-to-bf16 consumer is folded in so the kernel rounds once.
  // x when v = gelu_tanh(x) = 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))
  // in either association of the 0.5 factor, x * (0.5 (1 + t)) (jax.nn.gelu)
  // or (0.5 x) (1 + t), with x^3 = x (x x); else -1
  int GeluInput(int v) const {
    auto tanh_input = [&](int t) {
      int xr = -1;
      if (!is(t, "stablehlo.tanh")) return -1;
      Comm(prod(t)->operands[0], "stablehlo.multiply", [&](int cc, int u) {
        if (!IsConstNear(cc, 0.7978845608028654, 1e-6)) return false;
        return Comm(u, "stablehlo.add", [&](int x, int w) {
          return Comm(w, "stablehlo.multiply", [&](int c2, int c3) {
            if (!IsConstNear(c2, 0.044715, 1e-6)) return false;
            return Comm(c3, "stablehlo.multiply", [&](int a, int b) {
              if (a != x) return false;
              return Comm(b, "stablehlo.multiply", [&](int pp, int qq) {
                if (pp != x || qq != x) return false;
                xr = x;
                return true;
              });
            });
          });
        });
      });
      return xr;
    };
    int res = -1;
    Comm(v, "stablehlo.multiply", [&](int x, int h) {  // x * (0.5 (1 + t))
      return Comm(h, "stablehlo.multiply", [&](int half, int t1) {
        if (!IsConstNear(half, 0.5)) return false;
        return Comm(t1, "stablehlo.add", [&](int one, int t) {
          if (!IsConstNear(one, 1.0) || tanh_input(t) != x) return false;
          res = x;
          return true;
        });
      });
    });
    if (res >= 0) return res;
    Comm(v, "stablehlo.multiply", [&](int hx, int t1) {  // (0.5 x) (1 + t)
      int x = -1;
      if (!Comm(hx, "stablehlo.multiply", [&](int half, int xx) {
            if (!IsConstNear(half, 0.5)) return false;
            x = xx;
            return true;
          }))
        return false;
      return Comm(t1, "stablehlo.add", [&](int one, int t) {
        if (!IsConstNear(one, 1.0) || tanh_input(t) != x) return false;
        res = x;
        return true;
      });
    });
    return res;
  }

  // A product with a matched bias whose fp32 result x feeds gelu_tanh(x)
  // rounded to bf16 for the next product (the MLP's up-projection): the
  // GEMM's epilogue writes that bf16 value as a side output
  // (mk_gemm_bias_gelu, mk_gelu_tanh's function of the stored x), so the
  // forward chain is never materialised.  Its ops stay: the backward reads x
  // (and recomputes from it whatever else it needs).  Whether the side
  // output is taken is decided at lowering, where the operand layouts are
  // known (LowerDot); otherwise the convert lowers as before.
  void TryMatchGemmGelu(int cv) {
    const Op& c = ops_[cv];
    if (c.operands.size() != 1 || c.results.size() != 1) return;
    const int M = c.operands[0], CV = c.results[0];
    if (m_.types[CV].dtype != DType::kBF16 || m_.types[M].dtype != DType::kF32) return;
    if (std::count(outputs_.begin(), outputs_.end(), M) || std::count(outputs_.begin(), outputs_.end(), CV)) return;
    const auto mu = live_users(M);
    if (mu.empty() || std::any_of(mu.begin(), mu.end(), [&](int u) { return u != cv; })) return;
    const int X = GeluInput(M);
    if (X < 0 || m_.types[X].rank() != 2 || m_.types[X].dtype != DType::kF32) return;
    auto it = fused_.find(producer_[X]);
    if (it == fused_.end() || it->second.kind != Fused::kGemmEpi || it->second.relu || it->second.gelu_out >= 0) return;
    it->second.gelu_out = CV;
    prog_->patterns.push_back("gemm+bias+gelu(bf16 side output)");
  }

  void TryMatchGelu(int mul_idx) {
    const int M = ops_[mul_idx].results[0];
    if (m_.types[M].dtype != DType::kF32) return;
    int X = -1;
    std::vector<int> interior;
    const bool ok = Comm(M, "stablehlo.multiply", [&](int x, int h) {
      interior.clear();
      return Comm(h, "stablehlo.multiply", [&](int half, int t1) {
        if (!IsConstNear(half, 0.5)) return false;
        return Comm(t1, "stablehlo.add", [&](int one, int t) {
          if (!IsConstNear(one, 1.0) || !is(t, "stablehlo.tanh")) return false;
          const int u = prod(t)->operands[0];
          return Comm(u, "stablehlo.multiply", [&](int c, int v) {
            if (!IsConstNear(c, 0.7978845608028654, 1e-6)) return false;
            return Comm(v, "stablehlo.add", [&](int x2, int w) {
              if (x2 != x) return false;
              return Comm(w, "stablehlo.multiply", [&](int c2, int c3) {
                if (!IsConstNear(c2, 0.044715, 1e-6)) return false;
                int sq = -1;
                const bool cube = Comm(c3, "stablehlo.multiply", [&](int a, int b) {
                  if (a != x) return false;
                  return Comm(b, "stablehlo.multiply", [&](int p, int q) {
                    if (p != x || q != x) return false;
                    sq = b;
                    return true;
                  });
                });
                if (!cube) return false;
                X = x;
                interior = {h, t1, t, u, v, w, c3, sq};
                return true;
              });
            });
          });
        });
      });
    });
    if (!ok) return;
    std::set<int> ops{mul_idx};
    for (int v : interior) ops.insert(producer_[v]);
    int anchor = mul_idx;
    int out_v = M;
    if (users_[M].size() == 1 && uses_[M] == 1 && ops_[users_[M][0]].name == "stablehlo.convert" &&
        m_.types[ops_[users_[M][0]].results[0]].dtype == DType::kBF16) {
      anchor = users_[M][0];
      out_v = ops_[anchor].results[0];
      ops.insert(anchor);
    }
    for (int v : interior)
      if (!uses_within(v, ops)) return;
    if (anchor != mul_idx && !uses_within(M, ops)) return;
    int src = X;
    if (is(X, "stablehlo.convert") && m_.types[prod(X)->operands[0]].dtype == DType::kBF16) src = prod(X)->operands[0];
    const DType in_t = m_.types[src].dtype, out_t = m_.types[out_v].dtype;
    if (in_t != out_t) return;  // kernel io is one dtype (bf16 -> bf16 or f32 -> f32)
    Fused f;
    f.kind = Fused::kGelu;
    f.x = src;
    f.out_dtype = out_t;
    f.deps = {src};
    fused_[anchor] = f;
    for (int o : ops)
      if (o != anchor) absorbed_.insert(o);
    prog_->patterns.push_back(std::string("gelu_tanh(") + DTypeName(out_t) + ")");
  }

  // LayerNorm over the last dim, as the jnp two-pass formulation lowers:
  //   XF = convert?(x); MEAN = sum(XF)/n; XC = XF - bcast(MEAN);
  //   VAR = sum(XC*XC)/n; N = XC * bcast(rsqrt(VAR + eps));
  //   Y = N [* bcast(gamma)] [+ bcast(beta)]  [-> convert to the storage type]
  // The values a differentiated step reads again are recorded: the gamma
  // and beta broadcasts GB / BB, N (Y0), XC, the rsqrt R and its broadcast RB.
  struct LnMatch {
    int anchor = -1, out_v = -1, Y = -1;
    int gamma = -1, beta = -1, GB = -1, BB = -1;
    int Y0 = -1, XC = -1, XF = -1, R = -1, RB = -1;
    float eps = 0;
    std::set<int> ops;  // the forward's ops, anchor included
  };
  bool MatchLnForward(int idx, LnMatch& m) const {
    int Y = ops_[idx].results[0];
    m.anchor = idx;
    m.out_v = Y;
    if (ops_[idx].name == "stablehlo.convert") {  // output rounding folded in
      Y = ops_[idx].operands[0];
      if (users_[Y].size() != 1 || uses_[Y] != 1) return false;
    }
    m.Y = Y;
    const TensorType& yt = m_.types[Y];
    if (yt.dtype != DType::kF32 || yt.rank() < 1) return false;
    const int64_t n = yt.dims.back();
    std::set<int>& ops = m.ops;
    ops = {idx};
    int N = Y;
    // optional + beta
    {
      int rest = -1, bvec = -1, bb = -1;
      std::set<int> bops;
      if (Comm(Y, "stablehlo.add", [&](int a, int b) {
            bops.clear();
            int vec = VectorOnLastDim(b, n, &bops);
            if (vec < 0) return false;
            rest = a;
            bvec = vec;
            bb = b;
            return true;
          })) {
        m.beta = bvec;
        m.BB = bb;
        N = rest;
        ops.insert(producer_[Y]);
        ops.insert(bops.begin(), bops.end());
      }
    }
    // optional * gamma
    {
      int rest = -1, gvec = -1, gb = -1;
      std::set<int> gops;
      int N2 = N;
      if (Comm(N2, "stablehlo.multiply", [&](int a, int b) {
            gops.clear();
            int vec = VectorOnLastDim(b, n, &gops);
            if (vec < 0) return false;
            // the other side must itself be XC * bcast(rsqrt(...))
            if (!is(a, "stablehlo.multiply")) return false;
            rest = a;
            gvec = vec;
            gb = b;
            return true;
          })) {
        m.gamma = gvec;
        m.GB = gb;
        ops.insert(producer_[N2]);
        ops.insert(gops.begin(), gops.end());
        N = rest;
      }
    }
    // N = XC * bcast(rsqrt(VAR + eps))
    const bool core = Comm(N, "stablehlo.multiply", [&](int xc, int r) {
      std::set<int> cops;
      int rs = r;
      while (is(rs, "stablehlo.broadcast_in_dim") || is(rs, "stablehlo.reshape")) {
        cops.insert(producer_[rs]);
        rs = prod(rs)->operands[0];
      }
      if (!is(rs, "stablehlo.rsqrt")) return false;
      cops.insert(producer_[rs]);
      int var = -1;
      double e = 0;
      if (!Comm(prod(rs)->operands[0], "stablehlo.add", [&](int a, int c) {
            if (!scalar_of(c, &e)) return false;
            var = a;
            return true;
          }))
        return false;
      cops.insert(producer_[prod(rs)->operands[0]]);
      // XC = XF - bcast(MEAN(XF))
      int xf = -1;
      if (!NonComm(xc, "stablehlo.subtract", [&](int a, int mv) {
            std::set<int> mops;
            int in = RowMeanOf(mv, n, mops);
            if (in < 0 || in != a) return false;
            xf = a;
            cops.insert(mops.begin(), mops.end());
            return true;
          }))
        return false;
      cops.insert(producer_[xc]);
      // VAR = mean(XC * XC) over the same rows
      std::set<int> vops;
      int sq = RowMeanOf(var, n, vops);
      if (sq < 0 || !is(sq, "stablehlo.multiply")) return false;
      const Op* sqo = prod(sq);
      if (sqo->operands[0] != xc || sqo->operands[1] != xc) return false;
      vops.insert(producer_[sq]);
      cops.insert(vops.begin(), vops.end());
      ops.insert(producer_[N]);
      ops.insert(cops.begin(), cops.end());
      m.XC = xc;
      m.XF = xf;
      m.R = rs;
      m.RB = r;
      m.eps = float(e);
      return true;
    });
    if (!core) return false;
    m.Y0 = N;
    return true;
  }

  void TryMatchLayerNorm(int idx) {
    LnMatch m;
    if (!MatchLnForward(idx, m)) return;
    // every value computed inside the pattern stays inside it
    for (int o : m.ops)
      for (int r : ops_[o].results)
        if (o != idx && !uses_within(r, m.ops)) return;
    int src = m.XF;
    if (is(m.XF, "stablehlo.convert")) src = prod(m.XF)->operands[0];
    const DType io = m_.types[m.out_v].dtype;
    if (m_.types[src].dtype != io || (io != DType::kBF16 && io != DType::kF32)) return;
    if ((m.gamma >= 0 && m_.types[m.gamma].dtype != io) || (m.beta >= 0 && m_.types[m.beta].dtype != io)) return;
    Fused f;
    f.kind = Fused::kLayerNorm;
    f.x = src;
    f.gamma = m.gamma;
    f.beta = m.beta;
    f.eps = m.eps;
    f.out_dtype = io;
    f.in_dtype = io;
    f.deps = {src};
    if (m.gamma >= 0) f.deps.push_back(m.gamma);
    if (m.beta >= 0) f.deps.push_back(m.beta);
    fused_[idx] = f;
    for (int o : m.ops)
      if (o != idx) absorbed_.insert(o);
    prog_->patterns.push_back(std::string("layernorm(") + DTypeName(io) + ", eps=" + std::to_string(m.eps) + ")");
  }

  // A LayerNorm of fp32 rows [rows, n] (gamma required, beta optional) with
  // the backward that reverse-mode differentiation emits for it, rule by
  // rule (the transposes of the forward's ops, as jax.grad produces them):
  //   dY0 = dy GB;  dgamma = sum_0(dy Y0);  [dbeta = sum_0(dy)]
  //   dR = sum_1(dY0 XC);  dVE = dR (-0.5) (R (R R));  dS2 = dVE (1/n)
  //   dXC = dY0 RB + bcast(dS2) XC + bcast(dS2) XC      (the square's two operands)
  //   dx = [prev +] dXC;  dx += bcast(sum_1(-dXC) (1/n))
  //   [the bias gradient sum_0(dx) of the projection that wrote x]
  // The forward becomes one LayerNorm launch (the output convert folded into
  // its store) and the backward one mk_layernorm_bwd launch, which
  // recomputes the row statistics from x and writes dx (prev as the residual
  // branch), dgamma, dbeta and the bias gradient.  Every value in between
  // must be read by these ops only.
  void TryMatchLayerNormTrain(int idx) {
    LnMatch m;
    if (!MatchLnForward(idx, m) || m.gamma < 0) return;
    const int X = m.XF;
    const TensorType& xt = m_.types[X];
    if (is(X, "stablehlo.convert") || xt.dtype != DType::kF32 || xt.rank() != 2) return;
    if (m_.types[m.gamma].dtype != DType::kF32 || (m.beta >= 0 && m_.types[m.beta].dtype != DType::kF32)) return;
    const DType out_t = m_.types[m.out_v].dtype;
    if (out_t != DType::kF32 && out_t != DType::kBF16) return;
    const int64_t n = xt.dims[1];
    if (n > 2048) return;  // mk_layernorm_bwd's row limit
    auto uniq_users = [&](int v) {
      std::vector<int> r;
      for (int u : live_users(v))
        if (std::find(r.begin(), r.end(), u) == r.end()) r.push_back(u);
      return r;
    };
    auto outside = [&](int v) {
      std::vector<int> r;
      for (int u : uniq_users(v))
        if (!m.ops.count(u)) r.push_back(u);
      return r;
    };
    auto single = [&](int v) {
      const auto u = uniq_users(v);
      return u.size() == 1 ? u[0] : -1;
    };
    auto res = [&](int op) { return ops_[op].results[0]; };
    // op = multiply(a, other) in either order
    auto mul_with = [&](int op, int a, int* other) {
      if (op < 0) return false;
      const Op& o = ops_[op];
      if (o.name != "stablehlo.multiply" || o.operands.size() != 2) return false;
      if (o.operands[0] == a) *other = o.operands[1];
      else if (o.operands[1] == a) *other = o.operands[0];
      else return false;
      return true;
    };
    auto add_of = [&](int op, int a, int b) {
      if (op < 0) return false;
      const Op& o = ops_[op];
      return o.name == "stablehlo.add" && o.operands.size() == 2 &&
             ((o.operands[0] == a && o.operands[1] == b) || (o.operands[0] == b && o.operands[1] == a));
    };
    auto sum_over = [&](int op, int64_t dim) {
      if (op < 0) return false;
      const Op& o = ops_[op];
      double init;
      return o.name == "stablehlo.reduce" && o.operands.size() == 2 && o.results.size() == 1 &&
             reduce_body_op(o) == "stablehlo.add" && scalar_of(o.operands[1], &init) && init == 0.0 &&
             reduce_dims(o) == std::vector<int64_t>{dim} && m_.types[o.operands[0]].dims == xt.dims &&
             m_.types[o.results[0]].dtype == DType::kF32;
    };
    auto rows_bcast = [&](int op) {  // [rows] -> [rows, n] along dim 0
      if (op < 0) return false;
      const Op& o = ops_[op];
      return o.name == "stablehlo.broadcast_in_dim" &&
             attr_ints(o, {"dims", "broadcast_dimensions"}) == std::vector<int64_t>{0} &&
             m_.types[o.results[0]].dims == xt.dims;
    };
    const double inv_n = 1.0 / double(n);
    std::set<int> b;  // the backward's ops
    // dY0 = dy * GB, the broadcast gamma's one reader outside the forward
    const auto gu = outside(m.GB);
    int DY = -1;
    if (gu.size() != 1 || !mul_with(gu[0], m.GB, &DY)) return;
    if (m_.types[DY].dtype != DType::kF32 || m_.types[DY].dims != xt.dims) return;
    const int CTY0 = res(gu[0]);
    b.insert(gu[0]);
    // dgamma = sum_0(dy * Y0)
    const auto yu = outside(m.Y0);
    int o = -1;
    if (yu.size() != 1 || !mul_with(yu[0], m.Y0, &o) || o != DY) return;
    b.insert(yu[0]);
    const int dg_op = single(res(yu[0]));
    if (!sum_over(dg_op, 0)) return;
    b.insert(dg_op);
    const int DG = res(dg_op);
    // dY0's readers: * RB (into dXC) and * XC (into dR)
    const auto cu = uniq_users(CTY0);
    if (cu.size() != 2) return;
    int CTXC1 = -1, CTRB = -1;
    for (int u : cu) {
      if (!mul_with(u, CTY0, &o)) return;
      if (o == m.RB) CTXC1 = res(u);
      else if (o == m.XC) CTRB = res(u);
      b.insert(u);
    }
    if (CTXC1 < 0 || CTRB < 0) return;
    const int dr_op = single(CTRB);
    if (!sum_over(dr_op, 1)) return;
    b.insert(dr_op);
    // dVE = (dR * -0.5) * (R * (R * R))
    const int a1_op = single(res(dr_op));
    if (!mul_with(a1_op, res(dr_op), &o) || !IsConstNear(o, -0.5)) return;
    b.insert(a1_op);
    const auto ru = outside(m.R);
    int R2 = -1, R3 = -1;
    for (int u : ru) {
      const Op& p = ops_[u];
      if (p.name == "stablehlo.multiply" && p.operands[0] == m.R && p.operands[1] == m.R) R2 = res(u);
    }
    if (R2 < 0 || ru.size() != 2) return;
    for (int u : ru)
      if (res(u) != R2 && mul_with(u, m.R, &o) && o == R2) R3 = res(u);
    if (R3 < 0 || single(R2) != producer_[R3]) return;
    b.insert(producer_[R2]);
    b.insert(producer_[R3]);
    const int ve_op = single(res(a1_op));
    if (!mul_with(ve_op, res(a1_op), &o) || o != R3 || single(R3) != ve_op) return;
    b.insert(ve_op);
    // dS2 = dVE * (1/n), broadcast over the row
    const int s2_op = single(res(ve_op));
    if (!mul_with(s2_op, res(ve_op), &o) || !IsConstNear(o, inv_n)) return;
    b.insert(s2_op);
    const int b2_op = single(res(s2_op));
    if (!rows_bcast(b2_op)) return;
    b.insert(b2_op);
    // the square's two cotangents: bcast(dS2) * XC, twice
    const auto b2u = uniq_users(res(b2_op));
    if (b2u.size() != 2) return;
    for (int u : b2u) {
      if (!mul_with(u, res(b2_op), &o) || o != m.XC) return;
      b.insert(u);
    }
    const int M1 = res(b2u[0]), M2 = res(b2u[1]);
    // dXC = (dY0 RB + M) + M'
    const int a2_op = single(CTXC1);
    int Mlast = -1;
    if (add_of(a2_op, CTXC1, M1)) Mlast = M2;
    else if (add_of(a2_op, CTXC1, M2)) Mlast = M1;
    else return;
    if (single(M1) < 0 || single(M2) < 0) return;
    b.insert(a2_op);
    const int xc_op = single(res(a2_op));
    if (!add_of(xc_op, res(a2_op), Mlast)) return;
    b.insert(xc_op);
    const int DXC = res(xc_op);
    // dXC's readers: its negation (into the mean's cotangent) and the
    // accumulation into x's cotangent
    const auto xu = uniq_users(DXC);
    if (xu.size() != 2) return;
    int ng_op = -1, acc_op = -1;
    for (int u : xu) {
      if (ops_[u].name == "stablehlo.negate") ng_op = u;
      else if (ops_[u].name == "stablehlo.add") acc_op = u;
    }
    if (ng_op < 0 || acc_op < 0) return;
    b.insert(ng_op);
    const int dm_op = single(res(ng_op));
    if (!sum_over(dm_op, 1)) return;
    b.insert(dm_op);
    const int s1_op = single(res(dm_op));
    if (!mul_with(s1_op, res(dm_op), &o) || !IsConstNear(o, inv_n)) return;
    b.insert(s1_op);
    const int b3_op = single(res(s1_op));
    if (!rows_bcast(b3_op)) return;
    b.insert(b3_op);
    const int B3 = res(b3_op);
    const int fin = single(B3);
    int PREV = -1;
    if (fin == acc_op) {
      // no other cotangent of x: dx = dXC + bcast(...)
      if (!add_of(fin, DXC, B3)) return;
    } else {
      const Op& q = ops_[acc_op];
      PREV = q.operands[0] == DXC ? q.operands[1] : q.operands[0];
      if (PREV == DXC || m_.types[PREV].dtype != DType::kF32 || m_.types[PREV].dims != xt.dims) return;
      if (single(res(acc_op)) != fin || !add_of(fin, res(acc_op), B3)) return;
      b.insert(acc_op);
    }
    const int DXT = res(fin);
    // optional: dbeta = sum_0(dy), the bias gradient sum_0(dx)
    int DB = -1, CS = -1;
    if (m.beta >= 0)
      for (int u : uniq_users(DY))
        if (sum_over(u, 0) && !b.count(u)) {
          DB = res(u);
          b.insert(u);
          break;
        }
    std::vector<int> dx16;  // dx rounded to bf16 for the products that read it next
    for (int u : uniq_users(DXT)) {
      if (CS < 0 && sum_over(u, 0)) {
        CS = res(u);
        b.insert(u);
      } else if (ops_[u].name == "stablehlo.convert" && m_.types[res(u)].dtype == DType::kBF16 &&
                 !std::count(outputs_.begin(), outputs_.end(), res(u))) {
        dx16.push_back(res(u));
      }
    }
    // every value in between is read by these ops only; the results the
    // fused backward writes are read after it
    // (live readers: the cotangents of the constant 1/n factors are formed
    // and never read)
    std::set<int> all = m.ops;
    all.insert(b.begin(), b.end());
    all.insert(fin);
    auto read_within = [&](int v) {
      if (std::count(outputs_.begin(), outputs_.end(), v)) return false;
      for (int u : live_users(v))
        if (!all.count(u)) return false;
      return true;
    };
    for (int op : m.ops)
      for (int r : ops_[op].results)
        if (op != idx && !read_within(r)) return;
    for (int op : b) {
      const int r = res(op);
      if (r == DG || r == DB || r == CS) {
        for (int u : live_users(r))
          if (u <= fin) return;
        continue;
      }
      if (!read_within(r)) return;
    }
    if (idx >= fin) return;
    // x = a + b, the residual update (fp32 operands read in place, not
    // layout views): added and stored by the forward launch itself, which
    // writes x for the backward and the next update; every reader of x
    // outside the forward comes after it
    int add_op = -1;
    {
      const int p = producer_[X];
      auto in_place = [&](int v) {
        if (m_.types[v].dtype != DType::kF32 || m_.types[v].dims != xt.dims) return false;
        const Op* q = prod(v);
        if (!q) return true;  // a module argument
        static const char* views[] = {"stablehlo.broadcast_in_dim", "stablehlo.reshape", "stablehlo.transpose",
                                      "stablehlo.slice", "stablehlo.concatenate", "stablehlo.convert"};
        for (const char* n : views)
          if (q->name == n) return false;
        return true;
      };
      if (p >= 0 && ops_[p].name == "stablehlo.add" && ops_[p].operands.size() == 2 && !fused_.count(p) &&
          !absorbed_.count(p) && in_place(ops_[p].operands[0]) && in_place(ops_[p].operands[1])) {
        bool later = true;
        for (int u : live_users(X))
          if (!m.ops.count(u) && u < idx) later = false;
        if (later) add_op = p;
      }
    }
    Fused ff;
    ff.kind = Fused::kLayerNorm;
    ff.x = X;
    ff.gamma = m.gamma;
    ff.beta = m.beta;
    ff.eps = m.eps;
    ff.out_dtype = out_t;
    ff.in_dtype = DType::kF32;
    ff.deps = {X, m.gamma};
    if (add_op >= 0) {
      ff.add_a = ops_[add_op].operands[0];
      ff.add_b = ops_[add_op].operands[1];
      ff.deps = {ff.add_a, ff.add_b, m.gamma};
      absorbed_.insert(add_op);
    }
    if (m.beta >= 0) ff.deps.push_back(m.beta);
    fused_[idx] = ff;
    Fused fb;
    fb.kind = Fused::kLayerNormBwd;
    fb.x = X;
    fb.gamma = m.gamma;
    fb.dout = DY;
    fb.dres = PREV;
    fb.dgamma = DG;
    fb.dbeta = DB;
    fb.colsum = CS;
    fb.dx_bf16 = dx16;
    fb.eps = m.eps;
    fb.deps = {X, m.gamma, DY};
    if (PREV >= 0) fb.deps.push_back(PREV);
    fused_[fin] = fb;
    for (int op : m.ops)
      if (op != idx) absorbed_.insert(op);
    for (int op : b) absorbed_.insert(op);
    for (int c : dx16) absorbed_.insert(producer_[c]);
    prog_->patterns.push_back(std::string("layernorm_train(f32 -> ") + DTypeName(out_t) + ", eps=" +
                              std::to_string(m.eps) + (add_op >= 0 ? ", input added" : "") +
                              (PREV >= 0 ? ", residual" : "") +
                              (DB >= 0 ? ", dbeta" : "") + (CS >= 0 ? ", bias gradient" : "") + ")");
  }

  // -------------------------------------------------------------- liveness / DCE
  void Liveness() {
    live_.assign(ops_.size(), false);
    std::vector<int> stack(outputs_.begin(), outputs_.end());
    std::vector<bool> seen(m_.types.size(), false);
    while (!stack.empty()) {
      int v = stack.back();
      stack.pop_back();
      if (v < 0 || seen[v]) continue;
      seen[v] = true;
      int p = producer_[v];
      if (p < 0) continue;
      // a value computed inside a fused pattern is produced by the anchor
      if (!live_[p]) live_[p] = true;
      auto it = fused_.find(p);
      const std::vector<int>& deps = it != fused_.end() ? it->second.deps : ops_[p].operands;
      for (int d : deps) stack.push_back(d);
    }
    // absorbed ops (gemm epilogue internals) never run on their own
    for (int a : absorbed_) live_[a] = false;
  }

  // -------------------------------------------------------------- arena
  BufRef NewTemp(size_t bytes) {
    BufRef r;
    r.space = Space::kArena;
    r.index = int(temps_.size());
    r.offset = 0;
    temps_.push_back({(bytes + 255) & ~size_t(255), -1, -1});
    return r;
  }
  // final placement of the virtual arena buffers: linear scan over steps,
  // first fit in a free list, so buffers with disjoint lifetimes share bytes
  void PackArena() {
    for (size_t s = 0; s < prog_->steps.size(); ++s)
      for (const BufRef& b : prog_->steps[s].bufs)
        if (b.space == Space::kArena) {
          auto& t = temps_[b.index];
          if (t.first < 0) t.first = int(s);
          t.last = int(s);
        }
    struct Block {
      size_t off, size;
    };
    std::vector<Block> free_list;
    size_t top = 0;
    std::vector<size_t> base(temps_.size(), 0);
    std::vector<std::vector<int>> ends(prog_->steps.size() + 1);
    std::vector<std::vector<int>> starts(prog_->steps.size() + 1);
    for (size_t i = 0; i < temps_.size(); ++i)
      if (temps_[i].first >= 0) {
        starts[temps_[i].first].push_back(int(i));
        ends[temps_[i].last].push_back(int(i));
      }
    for (size_t s = 0; s < prog_->steps.size(); ++s) {
      for (int i : starts[s]) {
        const size_t need = temps_[i].size;
        bool placed = false;
        for (size_t k = 0; k < free_list.size(); ++k)
          if (free_list[k].size >= need) {
            base[i] = free_list[k].off;
            free_list[k].off += need;
            free_list[k].size -= need;
            if (free_list[k].size == 0) free_list.erase(free_list.begin() + long(k));
            placed = true;
            break;
          }
        if (!placed) {
          base[i] = top;
          top += need;
        }
      }
      for (int i : ends[s]) free_list.push_back({base[i], temps_[i].size});
    }
    prog_->arena_bytes = top;
    for (auto& st : prog_->steps)
      for (BufRef& b : st.bufs)
        if (b.space == Space::kArena) b.offset += int64_t(base[b.index]);
  }

  // -------------------------------------------------------------- materialization
  // destination for the value `v` when it is materialized by a step
  BufRef DestFor(int v) {
    for (size_t k = 0; k < outputs_.size(); ++k)
      if (outputs_[k] == v && !out_written_[k]) {
        out_written_[k] = true;
        return BufRef{Space::kOutput, int(k), 0};
      }
    return NewTemp(m_.types[v].bytes());
  }
  // rows of value v (its last dim) `pitch` elements apart in `where`
  void SetPaddedView(int v, BufRef where, int64_t pitch) {
    SetDenseView(v, where);
    ValState& s = state_[v];
    const int r = s.view.rank();
    int64_t e = 1;
    for (int d = r - 1; d >= 0; --d) {
      s.view.strides[d] = e;
      e *= d == r - 1 ? pitch : s.view.dims[d];
    }
  }
  // a temp for value v with its rows padded to pad_rows_[v] (0: not padded)
  int64_t PaddedPitch(int v) const {
    const auto it = pad_rows_.find(v);
    return it == pad_rows_.end() ? 0 : it->second;
  }
  BufRef NewPaddedTemp(int v, int64_t pitch) {
    const TensorType& t = m_.types[v];
    return NewTemp(size_t(t.numel() / t.dims.back() * pitch) * DTypeBytes(t.dtype));
  }
  void SetDenseView(int v, BufRef where) {
    ValState& s = state_[v];
    s.kind = ValState::kView;
    s.view.buf = where;
    s.view.dtype = m_.types[v].dtype;
    s.view.dims = m_.types[v].dims;
    s.view.strides = DenseStrides(s.view.dims);
    s.view.offset = 0;
  }

  // ---- narrow copies
  // narrow_[v] is a view of bf16 data that holds exactly the values of the
  // f32 value v (v = widen(narrow_[v])): an attention result rounded to bf16
  // by its kernel, or a product written in bf16 because every reader rounds
  // it to bf16.  While nothing needs v's f32 form it is never written:
  // layout ops carry the narrow view along, a convert back to bf16 is that
  // view, and a sum reads it (widening on load is exact).  A sum is only an
  // allowed reader (allow_sum) where v's f32 values are the kernel's bf16
  // results anyway (the fused attention's outputs and gradients, within
  // that fusion's tolerance); a product whose f32 values a sum reads is
  // written in f32, since the sum of the rounded values would differ.
  bool NarrowOnly(int v, bool allow_sum = true) {
    const int key = 2 * v + (allow_sum ? 1 : 0);
    auto memo = narrow_only_.find(key);
    if (memo != narrow_only_.end()) return memo->second;
    bool ok = m_.types[v].dtype == DType::kF32 && std::count(outputs_.begin(), outputs_.end(), v) == 0;
    bool any = false;
    for (int u : users_[v]) {
      if (!ok) break;
      if (!live_[u]) continue;  // inside a fused step, which reads its own inputs
      any = true;
      const Op& o = ops_[u];
      if (fused_.count(u)) {
        ok = false;
      } else if (o.name == "stablehlo.convert") {
        ok = m_.types[o.results[0]].dtype == DType::kBF16;
      } else if (o.name == "stablehlo.transpose" || o.name == "stablehlo.reshape" ||
                 o.name == "stablehlo.broadcast_in_dim" || o.name == "stablehlo.slice" ||
                 o.name == "stablehlo.concatenate") {
        ok = o.operands[0] == v || o.name == "stablehlo.concatenate";
        ok = ok && NarrowOnly(o.results[0], allow_sum);
      } else if (o.name == "stablehlo.reduce") {
        ok = allow_sum && o.operands.size() == 2 && o.operands[0] == v && reduce_body_op(o) == "stablehlo.add" &&
             m_.types[o.results[0]].dtype == DType::kF32;
      } else {
        ok = false;
      }
    }
    ok = ok && any;
    narrow_only_[key] = ok;
    return ok;
  }

  // The view a layout op (broadcast_in_dim, reshape, transpose, slice) makes
  // of `sv`, its operand's view; a reshape with no strided form copies first.
  View ApplyLayout(const Op& op, View sv) {
    const std::string& n = op.name;
    const TensorType& t = m_.types[op.results[0]];
    View v = sv;
    if (n == "stablehlo.broadcast_in_dim") {
      const auto dims = attr_ints(op, {"dims", "broadcast_dimensions"});
      v.dims = t.dims;
      v.strides.assign(t.rank(), 0);
      for (size_t k = 0; k < dims.size(); ++k) v.strides[dims[k]] = sv.dims[k] == 1 ? 0 : sv.strides[k];
    } else if (n == "stablehlo.reshape") {
      v.dims = t.dims;
      if (!ReshapeStrides(sv.dims, sv.strides, v.dims, v.strides)) {
        if (!sv.dense()) sv = Densify(sv);
        v = sv;
        v.dims = t.dims;
        v.strides = DenseStrides(v.dims);
      }
    } else if (n == "stablehlo.transpose") {
      const auto perm = attr_ints(op, {"dims", "permutation"});
      for (size_t k = 0; k < perm.size(); ++k) {
        v.dims[k] = sv.dims[perm[k]];
        v.strides[k] = sv.strides[perm[k]];
      }
    } else if (n == "stablehlo.slice") {
      const auto st = attr_ints(op, {"start_indices"});
      const auto sd = attr_ints(op, {"strides"});
      v.dims = t.dims;
      for (int k = 0; k < sv.rank(); ++k) {
        v.offset += st.at(k) * sv.strides[k];
        v.strides[k] = sv.strides[k] * (sd.empty() ? 1 : sd[k]);
      }
    } else {
      throw std::string("jam: internal: not a layout op: " + n);
    }
    return v;
  }

  // The concatenate that merges the three attention gradients when each is
  // transpose(0,2,1,3) -> reshape [B·S, H·D] (nothing else reading them)
  // and the three are its operands in order along dim 1; -1 otherwise.
  int MergedQkvConcat(const int g[3], int64_t B, int64_t H, int64_t S, int64_t D) {
    int concat = -1;
    for (int k = 0; k < 3; ++k) {
      if (m_.types[g[k]].dtype != DType::kF32 || !NarrowOnly(g[k])) return -1;
      const auto u1 = live_users(g[k]);
      if (u1.size() != 1 || ops_[u1[0]].name != "stablehlo.transpose" ||
          attr_ints(ops_[u1[0]], {"dims", "permutation"}) != std::vector<int64_t>{0, 2, 1, 3})
        return -1;
      const int t = ops_[u1[0]].results[0];
      const auto u2 = live_users(t);
      if (u2.size() != 1 || ops_[u2[0]].name != "stablehlo.reshape" ||
          m_.types[ops_[u2[0]].results[0]].dims != std::vector<int64_t>{B * S, H * D})
        return -1;
      const int r = ops_[u2[0]].results[0];
      const auto u3 = live_users(r);
      if (u3.size() != 1 || ops_[u3[0]].name != "stablehlo.concatenate") return -1;
      const Op& c = ops_[u3[0]];
      const auto dd = attr_ints(c, {"dim", "dimension"});
      if (c.operands.size() != 3 || c.operands[size_t(k)] != r || dd.empty() || dd[0] != 1) return -1;
      if (concat >= 0 && concat != u3[0]) return -1;
      concat = u3[0];
    }
    return concat;
  }

  // A layout op over a value with a narrow copy, whose result is only read
  // narrow: the result gets the narrow copy's view and no wide form.
  bool PropagateNarrow(const Op& op) {
    if (op.name == "stablehlo.broadcast") return false;
    auto nw = narrow_.find(op.operands[0]);
    if (nw == narrow_.end() || !NarrowOnly(op.results[0])) return false;
    narrow_[op.results[0]] = ApplyLayout(op, nw->second);
    return true;
  }

  // Guarantee that `v` is available as a view; emits steps as needed.
  const View& NeedView(int v) {
    ValState& s = state_[v];
    if (s.kind == ValState::kView) return s.view;
    if (s.kind == ValState::kUnset) {
      auto nw = narrow_.find(v);
      if (nw == narrow_.end())
        throw std::string("jam: value %" + std::to_string(v) + " used before it was lowered");
      // its wide form after all: widen the narrow copy
      const View src = nw->second.dense() ? nw->second : Densify(nw->second);
      BufRef d = DestFor(v);
      EmitConvert(src.at(), src.dtype, d, m_.types[v].dtype, m_.types[v].numel());
      SetDenseView(v, d);
      return state_[v].view;
    }
    const TensorType& t = m_.types[v];
    BufRef dst = DestFor(v);
    if (s.kind == ValState::kScalar) {
      Step st;
      st.kind = StepKind::kFill;
      st.bufs = {dst};
      uint64_t pattern = 0;
      uint8_t bytes[8] = {0};
      EncodeElement(s.fval, s.ival, t.dtype, bytes);
      memcpy(&pattern, bytes, size_t(DTypeBytes(t.dtype)));
      st.i = {DTypeBytes(t.dtype), t.numel(), int64_t(pattern)};
      st.note = "splat";
      Emit(st);
      SetDenseView(v, dst);
      return state_[v].view;
    }
    EmitEw(v, dst);
    SetDenseView(v, dst);
    return state_[v].view;
  }
  // Strides of a reshape of a strided view, when one exists: the dims of
  // both shapes are cut into the shortest runs with equal products (unit
  // dims aside); each input run must be one linear sequence of addresses
  // (every stride the next one times its size), and the output run then
  // walks the same sequence.  A run that is not linear (a transpose's
  // dims merged) has no strided form: false.
  static bool ReshapeStrides(const std::vector<int64_t>& id, const std::vector<int64_t>& is,
                             const std::vector<int64_t>& od, std::vector<int64_t>& os) {
    for (int64_t d : id)
      if (d == 0) return false;
    os.assign(od.size(), 0);
    size_t i = 0, j = 0;
    const size_t ni = id.size(), nj = od.size();
    while (true) {
      while (i < ni && id[i] == 1) ++i;
      while (j < nj && od[j] == 1) ++j;
      if (i >= ni || j >= nj) break;
      int64_t pi = id[i], pj = od[j];
      size_t i2 = i + 1, j2 = j + 1;
      while (pi != pj) {
        if (pi < pj) {
          if (i2 >= ni) return false;
          pi *= id[i2++];
        } else {
          if (j2 >= nj) return false;
          pj *= od[j2++];
        }
      }
      int64_t inner = 0, expect = -1;
      for (size_t k = i2; k-- > i;) {
        if (id[k] == 1) continue;
        if (expect < 0) inner = is[k];
        else if (is[k] != expect) return false;
        expect = is[k] * id[k];
      }
      int64_t st = inner;
      for (size_t k = j2; k-- > j;) {
        os[k] = st;
        st *= od[k];
      }
      i = i2;
      j = j2;
    }
    for (; i < ni; ++i)
      if (id[i] != 1) return false;
    for (; j < nj; ++j)
      if (od[j] != 1) return false;
    // unit dims: the stride a row-major layout would give them (never used
    // for addressing; keeps innermost-stride checks meaningful)
    for (size_t k = nj; k-- > 0;)
      if (od[k] == 1) os[k] = k + 1 < nj ? os[k + 1] * od[k + 1] : 1;
    return true;
  }
  // a dense copy of a view (for consumers that need row-major memory)
  View Densify(const View& src, int64_t elem_bytes_hint = 0) {
    if (src.dense()) return src;
    View out;
    out.dtype = src.dtype;
    out.dims = src.dims;
    out.strides = DenseStrides(src.dims);
    out.buf = NewTemp(size_t(src.numel()) * DTypeBytes(src.dtype));
    EmitCopy(src, out.buf);
    return out;
  }
  void EmitCopy(const View& src, BufRef dst) {
    if (src.dense()) {
      Step st;
      st.kind = StepKind::kCopy;
      st.bufs = {src.at(), dst};
      st.i = {int64_t(src.numel()) * DTypeBytes(src.dtype)};
      Emit(st);
      return;
    }
    if (src.rank() > 6) throw std::string("jam: rank > 6 layout copy is not supported");
    Step st;
    st.kind = StepKind::kCopyStrided;
    st.bufs = {src.at(), dst};
    st.i = {DTypeBytes(src.dtype), src.rank()};
    for (int64_t d : src.dims) st.i.push_back(d);
    st.strides = src.strides;
    Emit(st);
  }
  void Emit(Step st) { prog_->steps.push_back(std::move(st)); }

  // ---- elementwise expression compiler
  static bool IsElementwise(const std::string& n) {
    static const std::set<std::string> s = {
        "stablehlo.add", "stablehlo.subtract", "stablehlo.multiply", "stablehlo.divide",
        "stablehlo.maximum", "stablehlo.minimum", "stablehlo.power", "stablehlo.negate",
        "stablehlo.exponential", "stablehlo.log", "stablehlo.tanh", "stablehlo.sqrt",
        "stablehlo.rsqrt", "stablehlo.abs", "stablehlo.logistic", "stablehlo.compare",
        "stablehlo.select", "stablehlo.clamp", "stablehlo.convert", "stablehlo.floor",
        "stablehlo.ceil", "stablehlo.sign", "stablehlo.and", "stablehlo.or", "stablehlo.not",
        "stablehlo.xor", "stablehlo.round_nearest_even"};
    return s.count(n) > 0;
  }

  struct EwBuild {
    std::vector<int> leaves;              // value ids loaded as inputs
    std::vector<std::array<int32_t, 4>> prog;
    std::vector<uint32_t> consts;
    int next_reg = 0;
    std::vector<int> free_regs;
    std::unordered_map<int, int> memo;    // value id -> register holding it
    std::unordered_map<int, int> refs;    // remaining in-expression references
  };

  int AllocReg(EwBuild& b) {
    if (!b.free_regs.empty()) {
      int r = b.free_regs.back();
      b.free_regs.pop_back();
      return r;
    }
    if (b.next_reg >= 32) throw 1;  // caller splits the expression
    return b.next_reg++;
  }
  void FreeReg(EwBuild& b, int r) {
    if (r >= int(b.leaves.size())) b.free_regs.push_back(r);
  }
  int ConstReg(EwBuild& b, uint32_t bits) {
    int idx = -1;
    for (size_t k = 0; k < b.consts.size(); ++k)
      if (b.consts[k] == bits) idx = int(k);
    if (idx < 0) {
      if (b.consts.size() >= 64) throw 1;
      b.consts.push_back(bits);
      idx = int(b.consts.size()) - 1;
    }
    int r = AllocReg(b);
    b.prog.push_back({MK_EW_CONST, r, idx, 0});
    return r;
  }
  void Ins(EwBuild& b, int op, int dst, int a, int bb = 0) {
    if (b.prog.size() >= 64) throw 1;
    b.prog.push_back({op, dst, a, bb});
  }

  // An unmaterialized elementwise value is part of the expression being
  // built (evaluated once per element, shared through a register); anything
  // materialized is a leaf input.
  bool InExpr(int v) const { return state_[v].kind == ValState::kEw; }

  // First pass over the expression DAG: leaves and reference counts.
  void CollectLeaves(int v, std::vector<int>& leaves, std::unordered_map<int, int>& refs,
                     std::set<int>& seen) {
    if (!seen.insert(v).second) return;
    const ValState& s = state_[v];
    if (s.kind == ValState::kScalar) return;
    if (InExpr(v)) {
      for (int o : ops_[s.op].operands) {
        ++refs[o];
        CollectLeaves(o, leaves, refs, seen);
      }
      return;
    }
    leaves.push_back(v);
  }

  void Release(EwBuild& b, int v) {
    auto it = b.refs.find(v);
    if (it == b.refs.end()) return;
    if (--it->second == 0) {
      auto m = b.memo.find(v);
      if (m != b.memo.end()) FreeReg(b, m->second);
    }
  }

  // Second pass: emit code for v, returns its register.
  int Gen(EwBuild& b, int v, bool root) {
    auto memo = b.memo.find(v);
    if (memo != b.memo.end()) return memo->second;
    const ValState& s = state_[v];
    const DType t = m_.types[v].dtype;
    if (s.kind == ValState::kScalar) {
      int r = ConstReg(b, RegisterBits(s.fval, s.ival, t));
      b.memo[v] = r;
      return r;
    }
    if (!InExpr(v)) {
      auto it = std::find(b.leaves.begin(), b.leaves.end(), v);
      int r = int(it - b.leaves.begin());
      b.memo[v] = r;
      return r;
    }
    const Op& op = ops_[s.op];
    const std::string& n = op.name;
    std::vector<int> regs;
    for (int o : op.operands) regs.push_back(Gen(b, o, false));
    const DType in_t = m_.types[op.operands[0]].dtype;
    const bool fl = IsFloat(in_t);
    const bool in_int = !fl && in_t != DType::kPred;
    int dst = -1;
    auto unary = [&](int opc) {
      dst = AllocReg(b);
      Ins(b, opc, dst, regs[0]);
    };
    auto binary = [&](int opc) {
      dst = AllocReg(b);
      Ins(b, opc, dst, regs[0], regs[1]);
    };
    if (n == "stablehlo.add") binary(fl ? MK_EW_ADD : MK_EW_ADD_S32);
    else if (n == "stablehlo.subtract") binary(fl ? MK_EW_SUB : MK_EW_SUB_S32);
    else if (n == "stablehlo.multiply") binary(fl ? MK_EW_MUL : MK_EW_MUL_S32);
    else if (n == "stablehlo.divide") {
      if (!fl) throw std::string("jam: integer divide is not supported");
      binary(MK_EW_DIV);
    } else if (n == "stablehlo.maximum") binary(fl ? MK_EW_MAX : MK_EW_MAX_S32);
    else if (n == "stablehlo.minimum") binary(fl ? MK_EW_MIN : MK_EW_MIN_S32);
    else if (n == "stablehlo.power") binary(MK_EW_POW);
    else if (n == "stablehlo.negate") unary(fl ? MK_EW_NEG : MK_EW_NEG_S32);
    else if (n == "stablehlo.exponential") unary(MK_EW_EXP);
    else if (n == "stablehlo.log") unary(MK_EW_LOG);
    else if (n == "stablehlo.tanh") unary(MK_EW_TANH);
    else if (n == "stablehlo.sqrt") unary(MK_EW_SQRT);
    else if (n == "stablehlo.rsqrt") unary(MK_EW_RSQRT);
    else if (n == "stablehlo.abs") unary(MK_EW_ABS);
    else if (n == "stablehlo.logistic") unary(MK_EW_LOGISTIC);
    else if (n == "stablehlo.floor") unary(MK_EW_FLOOR);
    else if (n == "stablehlo.ceil") unary(MK_EW_CEIL);
    else if (n == "stablehlo.sign") unary(MK_EW_SIGN);
    else if (n == "stablehlo.round_nearest_even") throw std::string("jam: round_nearest_even is not supported");
    else if (n == "stablehlo.not") {
      if (in_t == DType::kPred) unary(MK_EW_NOT);
      else {
        int m1 = ConstReg(b, RegisterBits(-1, -1, DType::kI32));
        dst = AllocReg(b);
        Ins(b, MK_EW_XOR_B32, dst, regs[0], m1);
        FreeReg(b, m1);
      }
    } else if (n == "stablehlo.and" || n == "stablehlo.or" || n == "stablehlo.xor") {
      if (in_t == DType::kPred)
        binary(n == "stablehlo.and" ? MK_EW_AND : n == "stablehlo.or" ? MK_EW_OR : MK_EW_CMP_NE);
      else
        binary(n == "stablehlo.and" ? MK_EW_AND_B32 : n == "stablehlo.or" ? MK_EW_OR_B32 : MK_EW_XOR_B32);
    } else if (n == "stablehlo.compare") {
      std::string dir;
      if (const Attr* x = op.attr("comparison_direction")) dir = x->s;
      else if (const Attr* x = op.attr("enum0")) dir = x->s;
      int opc;
      if (fl || in_t == DType::kPred) {
        opc = dir == "EQ" ? MK_EW_CMP_EQ : dir == "NE" ? MK_EW_CMP_NE : dir == "LT" ? MK_EW_CMP_LT
            : dir == "LE" ? MK_EW_CMP_LE : dir == "GT" ? MK_EW_CMP_GT : MK_EW_CMP_GE;
      } else {
        if (IsUnsigned(in_t)) throw std::string("jam: unsigned compare is not supported");
        opc = dir == "EQ" ? MK_EW_CMP_EQ_S32 : dir == "NE" ? MK_EW_CMP_NE_S32 : dir == "LT" ? MK_EW_CMP_LT_S32
            : dir == "LE" ? MK_EW_CMP_LE_S32 : dir == "GT" ? MK_EW_CMP_GT_S32 : MK_EW_CMP_GE_S32;
      }
      binary(opc);
    } else if (n == "stablehlo.select") {
      dst = AllocReg(b);
      Ins(b, MK_EW_SELECT, dst, regs[0], regs[1] | (regs[2] << 16));
    } else if (n == "stablehlo.clamp") {
      // clamp(min, x, max)
      const DType xt = m_.types[op.operands[1]].dtype;
      dst = AllocReg(b);
      if (IsFloat(xt)) {
        Ins(b, MK_EW_CLAMP, dst, regs[1], regs[0] | (regs[2] << 16));
      } else {
        Ins(b, MK_EW_MAX_S32, dst, regs[1], regs[0]);
        Ins(b, MK_EW_MIN_S32, dst, dst, regs[2]);
      }
    } else if (n == "stablehlo.convert") {
      const DType ot = t;
      dst = AllocReg(b);
      if (IsFloat(in_t) && IsFloat(ot)) Ins(b, MK_EW_MOV, dst, regs[0]);
      else if (in_int && IsFloat(ot)) Ins(b, IsUnsigned(in_t) ? MK_EW_U32_TO_F32 : MK_EW_S32_TO_F32, dst, regs[0]);
      else if (in_t == DType::kPred && IsFloat(ot)) Ins(b, MK_EW_MOV, dst, regs[0]);
      else if (IsFloat(in_t) && ot == DType::kPred) {
        int z = ConstReg(b, 0);
        Ins(b, MK_EW_CMP_NE, dst, regs[0], z);
        FreeReg(b, z);
      } else if (IsFloat(in_t)) Ins(b, MK_EW_F32_TO_S32, dst, regs[0]);
      else if (in_t == DType::kPred) Ins(b, MK_EW_PRED_TO_S32, dst, regs[0]);
      else if (ot == DType::kPred) Ins(b, MK_EW_S32_TO_PRED, dst, regs[0]);
      else Ins(b, MK_EW_MOV, dst, regs[0]);
    } else {
      throw std::string("jam: no elementwise lowering for " + n);
    }
    // operands whose last in-expression reference this was give their register back
    for (int o : op.operands) Release(b, o);
    // per-op rounding: the StableHLO result type of an interior op is what
    // XLA materialises
    if (!root && (t == DType::kBF16 || t == DType::kF16))
      Ins(b, t == DType::kBF16 ? MK_EW_ROUND_BF16 : MK_EW_ROUND_F16, dst, dst);
    b.memo[v] = dst;
    return dst;
  }

  void EmitEw(int v, BufRef dst) { EmitEwGroup({v}, {dst}); }

  // One program computing every root (same shape) into its destination:
  // the roots' shared subexpressions and inputs are evaluated and loaded
  // once.  Returns false (emitting nothing) when a group of more than one
  // root does not fit the interpreter's limits; a single root is split
  // until it fits.
  bool EmitEwGroup(const std::vector<int>& roots, const std::vector<BufRef>& dsts) {
    const TensorType& t = m_.types[roots[0]];
    for (int attempt = 0; attempt < 64; ++attempt) {
      std::vector<int> leaves;
      std::unordered_map<int, int> refs;
      std::set<int> seen;
      for (int v : roots) CollectLeaves(v, leaves, refs, seen);
      for (int v : roots) ++refs[v];  // a root's register is held until its store
      if (leaves.size() > 8) {
        if (roots.size() > 1) return false;
        SplitLargestChild(roots[0]);
        continue;
      }
      EwBuild b;
      b.leaves = leaves;
      b.refs = refs;
      b.next_reg = int(leaves.size());
      std::vector<int> out_regs;
      try {
        // a root that other roots also read is generated as an interior
        // value (with its per-op rounding); storing it rounds it again to
        // the same bits
        for (int v : roots) out_regs.push_back(Gen(b, v, refs[v] == 1));
      } catch (int) {
        if (roots.size() > 1) return false;
        SplitLargestChild(roots[0]);
        continue;
      }
      if (t.rank() > 6) throw std::string("jam: rank > 6 elementwise is not supported");
      Step st;
      st.kind = StepKind::kEw;
      for (int l : leaves) {
        auto nw = narrow_.find(l);
        const View lv = state_[l].kind == ValState::kUnset && nw != narrow_.end() ? nw->second : NeedView(l);
        if (lv.rank() != t.rank()) throw std::string("jam: elementwise operand rank mismatch");
        st.bufs.push_back(lv.at());
        st.types.push_back(int32_t(lv.dtype));
        for (int d = 0; d < 6; ++d) st.strides.push_back(d < lv.rank() ? lv.strides[d] : 0);
      }
      for (const BufRef& d : dsts) st.bufs.push_back(d);
      st.i = {t.rank()};
      for (int d = 0; d < 6; ++d) st.i.push_back(d < t.rank() ? t.dims[d] : 1);
      st.i.push_back(int64_t(leaves.size()));
      for (size_t k = 0; k < roots.size(); ++k) {
        st.i.push_back(out_regs[k]);
        st.i.push_back(int64_t(m_.types[roots[k]].dtype));
      }
      for (auto& ins : b.prog)
        for (int k = 0; k < 4; ++k) st.prog.push_back(ins[k]);
      for (uint32_t c : b.consts) {
        float f;
        memcpy(&f, &c, 4);
        st.f.push_back(f);
      }
      st.note = ops_[state_[roots[0]].op].name + " chain (" + std::to_string(b.prog.size()) + " instr, " +
                std::to_string(leaves.size()) + " inputs" +
                (roots.size() > 1 ? ", " + std::to_string(roots.size()) + " outputs" : "") + ")";
      Emit(st);
      return true;
    }
    throw std::string("jam: could not split an elementwise expression");
  }

  // Output k (an elementwise value) together with the later outputs of the
  // same shape whose chains read at least one of its inputs, up to four
  // outputs and eight inputs in all: one launch writes them all (the Adam
  // update's new parameter, m and v read p, g, m and v once).
  void EmitOutputGroup(size_t k, BufRef dst) {
    const int v = outputs_[k];
    auto leaf_set = [&](int r) {
      std::vector<int> leaves;
      std::unordered_map<int, int> refs;
      std::set<int> seen;
      CollectLeaves(r, leaves, refs, seen);
      return std::set<int>(leaves.begin(), leaves.end());
    };
    std::vector<int> roots = {v};
    std::vector<BufRef> dsts = {dst};
    std::vector<size_t> ks = {k};
    if (opts_.fuse_elementwise) {
      std::set<int> all = leaf_set(v);
      for (size_t j = k + 1; j < outputs_.size() && roots.size() < 4; ++j) {
        const int w = outputs_[j];
        if (out_written_[j] || state_[w].kind != ValState::kEw || m_.types[w].dims != m_.types[v].dims ||
            std::count(roots.begin(), roots.end(), w))
          continue;
        const std::set<int> lw = leaf_set(w);
        std::set<int> u = all;
        u.insert(lw.begin(), lw.end());
        bool shares = false;
        for (int l : lw) shares = shares || all.count(l);
        if (!shares || u.size() > 8) continue;
        roots.push_back(w);
        dsts.push_back(BufRef{Space::kOutput, int(j), 0});
        ks.push_back(j);
        all = u;
      }
    }
    if (roots.size() > 1 && EmitEwGroup(roots, dsts)) {
      for (size_t i = 1; i < roots.size(); ++i) {
        out_written_[ks[i]] = true;
        SetDenseView(roots[i], dsts[i]);
      }
      return;
    }
    EmitEw(v, dst);
  }

  // materialize the biggest in-expression child of v so the expression shrinks
  void SplitLargestChild(int v) {
    std::function<int(int, std::set<int>&)> size = [&](int w, std::set<int>& seen) -> int {
      if (!InExpr(w) || !seen.insert(w).second) return 0;
      int s = 1;
      for (int o : ops_[state_[w].op].operands) s += size(o, seen);
      return s;
    };
    int best = -1, bs = 0;
    for (int o : ops_[state_[v].op].operands) {
      std::set<int> seen;
      int s = size(o, seen);
      if (s > bs) {
        bs = s;
        best = o;
      }
    }
    if (best < 0) throw std::string("jam: elementwise expression has more than 8 distinct inputs");
    BufRef d = NewTemp(m_.types[best].bytes());
    EmitEw(best, d);
    SetDenseView(best, d);
  }

  // Conversions of module inputs to a narrower float type whose results
  // only non-elementwise ops read (the bf16 copies of a training step's fp32
  // weights for its products) are emitted first, one after another: they
  // depend on nothing else, and as a run of independent steps each group of
  // one shape becomes one batched launch (BatchIndependentEwSteps) instead
  // of a launch in front of every product.
  std::set<int> hoisted_;
  std::set<int> preset_;  // ops whose result an earlier step already wrote (a GEMM's GELU side output)
  void HoistInputConverts() {
    if (!opts_.fuse_elementwise) return;
    for (size_t i = 0; i < ops_.size(); ++i) {
      const Op& op = ops_[i];
      if (!live_[i] || fused_.count(int(i)) || op.name != "stablehlo.convert" || op.operands.size() != 1) continue;
      const int src = op.operands[0], res = op.results[0];
      if (state_[src].kind != ValState::kView || state_[src].view.buf.space != Space::kInput) continue;
      const DType it = m_.types[src].dtype, ot = m_.types[res].dtype;
      if (!(it == DType::kF32 && (ot == DType::kBF16 || ot == DType::kF16))) continue;
      if (std::count(outputs_.begin(), outputs_.end(), res)) continue;
      const auto us = live_users(res);
      bool ok = !us.empty();
      // readers that take it from memory: products and layout ops, also
      // inside a matched pattern (a product with its bias epilogue)
      for (int u : us) ok = ok && !IsElementwise(ops_[u].name);
      if (!ok) continue;
      LowerOp(int(i));   // the lazy conversion
      NeedView(res);     // written now
      hoisted_.insert(int(i));
    }
  }

  // -------------------------------------------------------------- the walk
  void Walk() {
    out_written_.assign(outputs_.size(), false);
    HoistInputConverts();
    for (size_t i = 0; i < ops_.size(); ++i) {
      if (!live_[i] || hoisted_.count(int(i)) || preset_.count(int(i))) continue;
      auto f = fused_.find(int(i));
      if (f != fused_.end()) {
        EmitFused(int(i), f->second);
        continue;
      }
      LowerOp(int(i));
    }
    // program outputs
    for (size_t k = 0; k < outputs_.size(); ++k) {
      if (out_written_[k] && state_[outputs_[k]].kind == ValState::kView &&
          state_[outputs_[k]].view.buf.space == Space::kOutput && state_[outputs_[k]].view.buf.index == int(k))
        continue;
      const int v = outputs_[k];
      if (state_[v].kind != ValState::kView) {
        // materialize straight into this output
        BufRef dst{Space::kOutput, int(k), 0};
        out_written_[k] = true;
        if (state_[v].kind == ValState::kEw) {
          EmitOutputGroup(k, dst);
        } else {
          const TensorType& t = m_.types[v];
          Step st;
          st.kind = StepKind::kFill;
          st.bufs = {dst};
          uint64_t pattern = 0;
          uint8_t bytes[8] = {0};
          EncodeElement(state_[v].fval, state_[v].ival, t.dtype, bytes);
          memcpy(&pattern, bytes, size_t(DTypeBytes(t.dtype)));
          st.i = {DTypeBytes(t.dtype), t.numel(), int64_t(pattern)};
          st.note = "splat output";
          Emit(st);
        }
        SetDenseView(v, dst);
        continue;
      }
      EmitCopy(state_[v].view, BufRef{Space::kOutput, int(k), 0});
      out_written_[k] = true;
    }
  }

  void LowerOp(int idx) {
    const Op& op = ops_[idx];
    const std::string& n = op.name;
    auto res = [&](int k = 0) { return op.results.at(k); };
    if (n == "stablehlo.constant") {
      const TensorType& t = m_.types[res()];
      const Attr* ap = ParsedConst(res());
      if (!ap) {
        Attr a = *op.attr("value");
        std::string err;
        ParseDense(a, t, err);
        throw err;
      }
      const Attr& a = *ap;
      ValState& s = state_[res()];
      if (a.splat || t.numel() == 1) {
        s.kind = ValState::kScalar;
        s.fval = a.fvals.empty() ? double(a.ivals[0]) : a.fvals[0];
        s.ival = a.ivals.empty() ? int64_t(a.fvals[0]) : a.ivals[0];
        return;
      }
      ConstBlob blob;
      blob.type = t;
      blob.bytes.resize(t.bytes());
      const int w = DTypeBytes(t.dtype);
      for (int64_t e = 0; e < t.numel(); ++e)
        EncodeElement(a.fvals[size_t(e)], a.ivals[size_t(e)], t.dtype, &blob.bytes[size_t(e) * w]);
      prog_->consts.push_back(std::move(blob));
      s.kind = ValState::kView;
      s.view.buf = BufRef{Space::kConst, int(prog_->consts.size()) - 1, 0};
      s.view.dtype = t.dtype;
      s.view.dims = t.dims;
      s.view.strides = DenseStrides(t.dims);
      return;
    }
    if (n == "stablehlo.broadcast_in_dim" || n == "stablehlo.broadcast") {
      if (PropagateNarrow(op)) return;
      const int src = op.operands[0];
      const TensorType& t = m_.types[res()];
      if (state_[src].kind == ValState::kScalar) {
        state_[res()] = state_[src];
        return;
      }
      const View& sv = NeedView(src);
      std::vector<int64_t> dims;
      if (n == "stablehlo.broadcast") {  // legacy: prepend broadcast_sizes
        const int lead = t.rank() - sv.rank();
        for (int k = 0; k < sv.rank(); ++k) dims.push_back(lead + k);
      } else {
        dims = attr_ints(op, {"dims", "broadcast_dimensions"});
      }
      View v;
      v.buf = sv.buf;
      v.offset = sv.offset;
      v.dtype = sv.dtype;
      v.dims = t.dims;
      v.strides.assign(t.rank(), 0);
      for (size_t k = 0; k < dims.size(); ++k)
        v.strides[dims[k]] = sv.dims[k] == 1 ? 0 : sv.strides[k];
      SetView(res(), v);
      return;
    }
    if (n == "stablehlo.reshape") {
      if (PropagateNarrow(op)) return;
      const int src = op.operands[0];
      if (state_[src].kind == ValState::kScalar) {
        state_[res()] = state_[src];
        return;
      }
      View sv = NeedView(src);
      View v = sv;
      v.dims = m_.types[res()].dims;
      if (!ReshapeStrides(sv.dims, sv.strides, v.dims, v.strides)) {
        // no strided form: copy to row-major first
        if (!sv.dense()) sv = Densify(sv);
        v = sv;
        v.dims = m_.types[res()].dims;
        v.strides = DenseStrides(v.dims);
      }
      SetView(res(), v);
      return;
    }
    if (n == "stablehlo.transpose") {
      if (PropagateNarrow(op)) return;
      const int src = op.operands[0];
      if (state_[src].kind == ValState::kScalar) {
        state_[res()] = state_[src];
        return;
      }
      const View& sv = NeedView(src);
      const auto perm = attr_ints(op, {"dims", "permutation"});
      View v = sv;
      for (size_t k = 0; k < perm.size(); ++k) {
        v.dims[k] = sv.dims[perm[k]];
        v.strides[k] = sv.strides[perm[k]];
      }
      SetView(res(), v);
      return;
    }
    if (n == "stablehlo.slice") {
      if (PropagateNarrow(op)) return;
      const View& sv = NeedView(op.operands[0]);
      const auto st = attr_ints(op, {"start_indices"});
      const auto sd = attr_ints(op, {"strides"});
      View v = sv;
      v.dims = m_.types[res()].dims;
      for (int k = 0; k < sv.rank(); ++k) {
        v.offset += st.at(k) * sv.strides[k];
        v.strides[k] = sv.strides[k] * (sd.empty() ? 1 : sd[k]);
      }
      SetView(res(), v);
      return;
    }
    if (n == "stablehlo.convert") {
      auto nw = narrow_.find(op.operands[0]);
      if (nw != narrow_.end() && nw->second.dtype == m_.types[res()].dtype) {
        SetView(res(), nw->second);  // bf16 -> f32 -> bf16: the narrow copy itself
        return;
      }
    }
    if (IsElementwise(n)) {
      ValState& s = state_[res()];
      if (!opts_.fuse_elementwise) {
        s.kind = ValState::kEw;
        s.op = idx;
        BufRef d = DestFor(res());
        EmitEw(res(), d);
        SetDenseView(res(), d);
        return;
      }
      s.kind = ValState::kEw;
      s.op = idx;  // evaluated inside the consumers' fused programs
      return;
    }
    if (n == "stablehlo.iota") {
      const TensorType& t = m_.types[res()];
      const auto dd = attr_ints(op, {"dim", "iota_dimension"});
      BufRef d = DestFor(res());
      Step st;
      st.kind = StepKind::kIota;
      st.bufs = {d};
      st.i = {int64_t(t.dtype), t.rank(), dd.empty() ? 0 : dd[0]};
      for (int64_t x : t.dims) st.i.push_back(x);
      Emit(st);
      SetDenseView(res(), d);
      return;
    }
    if (n == "stablehlo.reduce") {
      LowerReduce(idx);
      return;
    }
    if (n == "stablehlo.dot_general" || n == "stablehlo.dot") {
      LowerDot(idx, nullptr);
      return;
    }
    if (n == "stablehlo.gather") {
      LowerGather(idx);
      return;
    }
    if (n == "stablehlo.scatter") {
      LowerScatter(idx);
      return;
    }
    if (n == "stablehlo.concatenate") {
      LowerConcat(idx);
      return;
    }
    throw std::string("jam: unhandled op '" + n + "'");  // lower.mm:308-310
  }

  void SetView(int v, const View& view) {
    ValState& s = state_[v];
    s.kind = ValState::kView;
    s.view = view;
  }

  // ---- reduce (generic single-operand; the arg-reduce pattern is fused)
  void LowerReduce(int idx) {
    const Op& op = ops_[idx];
    if (op.operands.size() != 2 || op.results.size() != 1)
      throw std::string("jam: variadic reduce other than arg-max/arg-min is not supported");
    const std::string body = reduce_body_op(op);
    int rop = body == "stablehlo.add" ? 0 : body == "stablehlo.maximum" ? 1 : body == "stablehlo.minimum" ? 2
            : body == "stablehlo.multiply" ? 3 : -1;
    if (rop < 0) throw std::string("jam: unsupported reduce body op '" + body + "'");  // reduce.mm:91
    double init = 0;
    if (!scalar_of(op.operands[1], &init)) throw std::string("jam: reduce init must be a constant");
    int x = op.operands[0];
    // reduce(convert(x_narrow -> f32)): the kernel widens while loading
    if (state_[x].kind == ValState::kEw && is(x, "stablehlo.convert") &&
        m_.types[x].dtype == DType::kF32) {
      const int src = prod(x)->operands[0];
      const DType st_ = m_.types[src].dtype;
      if (st_ == DType::kBF16 || st_ == DType::kF16) x = src;
    }
    // a reduction of an elementwise value read by nothing else: the value is
    // computed inside the reduction's generated kernel, never stored
    if (opts_.ew_jit && opts_.fuse_elementwise && InExpr(x) && EmitEwReduce(op, x, rop, init, body, uses_[x] > 1))
      return;
    // a sum over an f32 value with a narrow copy reads the copy (the same
    // values; the kernel widens on load)
    auto nw = narrow_.find(x);
    const bool use_narrow = nw != narrow_.end() && m_.types[x].dtype == DType::kF32;
    const DType xt = use_narrow ? nw->second.dtype : m_.types[x].dtype;
    const DType ot = m_.types[op.results[0]].dtype;
    if (!(xt == DType::kF32 || xt == DType::kBF16 || xt == DType::kF16))
      throw std::string("jam: reduce over ") + DTypeName(xt) + " is not supported";
    View xv = use_narrow ? nw->second : NeedView(x);
    const auto dims = reduce_dims(op);
    // move reduced dims last (a transposed view), then make it dense
    std::vector<int> keep, red;
    for (int d = 0; d < xv.rank(); ++d)
      (std::find(dims.begin(), dims.end(), d) != dims.end() ? red : keep).push_back(d);
    View pv = xv;
    int k = 0;
    int64_t rows = 1, cols = 1;
    for (int d : keep) {
      pv.dims[k] = xv.dims[d];
      pv.strides[k++] = xv.strides[d];
      rows *= xv.dims[d];
    }
    for (int d : red) {
      pv.dims[k] = xv.dims[d];
      pv.strides[k++] = xv.strides[d];
      cols *= xv.dims[d];
    }
    // a sum over the leading dims of a row-major array into f32 (bias
    // gradients): mk_col_sum reads the rows in place instead of a transposed
    // copy plus a row reduce.  Its grid has one y-block per 256 kept columns
    // at the finest (f32 vectors), at most 65535 of them; wider sums take the
    // row-reduce path.
    constexpr int64_t kColSumMaxKept = int64_t(65535) * 256;
    bool lead = xv.dense() && rop == 0 && init == 0 && ot == DType::kF32 &&
                (xt == DType::kF32 || xt == DType::kBF16) && rows > 0 && rows <= kColSumMaxKept && cols > 0 &&
                !red.empty() && !keep.empty();
    for (size_t r = 0; lead && r < red.size(); ++r) lead = red[r] == int(r);
    if (lead) {
      BufRef d = DestFor(op.results[0]);
      BufRef ws = NewTemp(mk_col_sum_workspace_bytes(cols, rows));
      Step st;
      st.kind = StepKind::kColSum;
      st.bufs = {xv.at(), d, ws};
      st.i = {int64_t(xt), cols, rows};
      st.note = body;
      Emit(st);
      SetDenseView(op.results[0], d);
      return;
    }
    pv = Densify(pv);
    BufRef d = DestFor(op.results[0]);
    Step st;
    st.kind = StepKind::kRowReduce;
    st.bufs = {pv.at(), d};
    st.i = {int64_t(xt), int64_t(ot), rop, rows, cols};
    st.f = {float(init)};
    st.note = body;
    Emit(st);
    SetDenseView(op.results[0], d);
  }

  // Every reader of v other than `except` converts it to bf16 (directly or
  // through layout ops), and v is no program output.
  bool OnlyBf16Converts(int v, const Op& except) {
    if (std::count(outputs_.begin(), outputs_.end(), v) != 0) return false;
    for (int u : users_[v]) {
      if (&ops_[u] == &except || !live_[u]) continue;
      const Op& o = ops_[u];
      if (fused_.count(u)) return false;
      if (o.name == "stablehlo.convert") {
        if (m_.types[o.results[0]].dtype != DType::kBF16) return false;
      } else if (o.name == "stablehlo.transpose" || o.name == "stablehlo.reshape" ||
                 o.name == "stablehlo.broadcast_in_dim" || o.name == "stablehlo.slice") {
        if (!NarrowOnly(o.results[0], false)) return false;
      } else {
        return false;
      }
    }
    return true;
  }

  // The ew program of value v over its leaves; false when it does not fit
  // the interpreter's limits (eight inputs, its register file).
  bool BuildEwProgram(int v, EwBuild* out, int* reg) {
    std::vector<int> leaves;
    std::unordered_map<int, int> refs;
    std::set<int> seen;
    CollectLeaves(v, leaves, refs, seen);
    ++refs[v];
    if (leaves.size() > 8) return false;
    EwBuild b;
    b.leaves = leaves;
    b.refs = refs;
    b.next_reg = int(leaves.size());
    try {
      *reg = Gen(b, v, true);
    } catch (int) {
      return false;
    }
    *out = std::move(b);
    return true;
  }

  // reduce(x) with x an elementwise expression: one kEwReduce step whose
  // generated kernel evaluates x where the reduction reads it.  Trailing
  // reduced dims (after moving them last): one wave per kept element; a sum
  // over the leading dims into f32 (bias, gamma and beta gradients): column
  // partial sums over row chunks, then their total.  The step keeps a
  // buffer for x for the interpreter fallback (x stored, then the library's
  // reduction).
  bool EmitEwReduce(const Op& op, int x, int rop, double init, const std::string& body, bool store) {
    const TensorType& xt = m_.types[x];
    const DType vt = xt.dtype, ot = m_.types[op.results[0]].dtype;
    auto fl = [](DType d) { return d == DType::kF32 || d == DType::kBF16 || d == DType::kF16; };
    if (!fl(vt) || !fl(ot) || xt.rank() < 1 || xt.rank() > 6) return false;
    const auto rd = reduce_dims(op);
    std::vector<int> keep, red;
    for (int d = 0; d < xt.rank(); ++d)
      (std::find(rd.begin(), rd.end(), d) != rd.end() ? red : keep).push_back(d);
    int64_t nk = 1, nr = 1;
    for (int d : keep) nk *= xt.dims[size_t(d)];
    for (int d : red) nr *= xt.dims[size_t(d)];
    if (red.empty() || nk <= 0 || nr <= 0) return false;
    bool lead = !keep.empty() && rop == 0 && init == 0 && ot == DType::kF32 && (vt == DType::kF32 || vt == DType::kBF16);
    for (size_t r = 0; lead && r < red.size(); ++r) lead = red[r] == int(r);
    std::vector<int> order;
    if (lead) {
      for (int d = 0; d < xt.rank(); ++d) order.push_back(d);
    } else {
      order = keep;
      order.insert(order.end(), red.begin(), red.end());
    }
    // a value that other ops read is stored by the same kernel, which
    // writes it in iteration order: only when that is its own layout
    for (size_t k = 0; store && k < order.size(); ++k)
      if (order[k] != int(k)) return false;
    EwBuild b;
    int reg = 0;
    if (!BuildEwProgram(x, &b, &reg)) return false;
    Step st;
    st.kind = StepKind::kEwReduce;
    for (int l : b.leaves) {
      auto nw = narrow_.find(l);
      const View lv = state_[l].kind == ValState::kUnset && nw != narrow_.end() ? nw->second : NeedView(l);
      if (lv.rank() != xt.rank()) throw std::string("jam: elementwise operand rank mismatch");
      st.bufs.push_back(lv.at());
      st.types.push_back(int32_t(lv.dtype));
      for (int k = 0; k < 6; ++k) st.strides.push_back(k < xt.rank() ? lv.strides[size_t(order[size_t(k)])] : 0);
    }
    // stored: in f32, or only its bf16 rounding when every other reader
    // converts it to bf16 (the sum reads the exact values inside the kernel)
    const bool narrow_store = store && vt == DType::kF32 && OnlyBf16Converts(x, op);
    const BufRef d = DestFor(op.results[0]);
    st.bufs.push_back(d);
    const BufRef xs = store && !narrow_store ? DestFor(x) : NewTemp(xt.bytes());
    st.bufs.push_back(xs);
    const int64_t rows = lead ? nr : nk, cols = lead ? nk : nr;
    const int64_t inner = xt.dims[size_t(order.back())];
    st.bufs.push_back(lead ? NewTemp(size_t(std::max<int64_t>(int64_t(mk_col_sum_workspace_bytes(rows, cols)),
                                                                 EwReduceWorkspaceBytes(rows, cols, inner))))
                           : BufRef{});
    BufRef xn;
    if (narrow_store) {
      xn = NewTemp(size_t(xt.numel()) * 2);
      st.bufs.push_back(xn);
    } else if (store) {
      st.bufs.push_back(xs);
    }
    const float fi = float(init);
    uint32_t ib;
    memcpy(&ib, &fi, 4);
    st.i = {xt.rank()};
    for (int k = 0; k < 6; ++k) st.i.push_back(k < xt.rank() ? xt.dims[size_t(order[size_t(k)])] : 1);
    st.i.push_back(int64_t(b.leaves.size()));
    st.i.insert(st.i.end(), {reg, int64_t(vt), int64_t(ot), rop, rows, cols, lead ? 1 : 0, int64_t(ib),
                             narrow_store ? 2 : store ? 1 : 0});
    for (auto& ins : b.prog)
      for (int k = 0; k < 4; ++k) st.prog.push_back(ins[k]);
    for (uint32_t c : b.consts) {
      float f;
      memcpy(&f, &c, 4);
      st.f.push_back(f);
    }
    st.note = body + " of " + ops_[state_[x].op].name + " chain (" + std::to_string(b.prog.size()) + " instr, " +
              std::to_string(b.leaves.size()) + " inputs, " + (lead ? "leading dims" : "trailing dims") +
              (narrow_store ? ", bf16 copy stored" : store ? ", value stored" : "") + ")";
    Emit(st);
    SetDenseView(op.results[0], d);
    if (narrow_store) {
      View nv;
      nv.buf = xn;
      nv.dtype = DType::kBF16;
      nv.dims = xt.dims;
      nv.strides = DenseStrides(nv.dims);
      narrow_[x] = nv;
      state_[x].kind = ValState::kUnset;  // its f32 form is never written
    } else if (store) {
      SetDenseView(x, xs);
    }
    return true;
  }

  // Map a dot_general to mk_gemm; `epi` optionally carries bias / relu.
  void LowerDot(int idx, const Fused* epi, int result_override = -1) {
    const Op& op = ops_[idx];
    const int res = result_override >= 0 ? result_override : op.results[0];
    const int L = op.operands[0], Rv = op.operands[1];
    DotDims dd = dot_dims(op);
    if (op.name == "stablehlo.dot") {
      dd.lc = {int64_t(m_.types[L].rank()) - 1};
      dd.rc = {0};
    }
    View lv = NeedView(L), rv = NeedView(Rv);
    const DType at = lv.dtype, bt = rv.dtype;
    if (at != bt) throw std::string("jam: dot_general with mixed operand types");
    if (at != DType::kF32 && at != DType::kBF16) throw std::string("jam: dot_general on ") + DTypeName(at) + " is not supported";
    std::vector<int64_t> lf, rf;
    for (int d = 0; d < lv.rank(); ++d)
      if (!std::count(dd.lb.begin(), dd.lb.end(), d) && !std::count(dd.lc.begin(), dd.lc.end(), d)) lf.push_back(d);
    for (int d = 0; d < rv.rank(); ++d)
      if (!std::count(dd.rb.begin(), dd.rb.end(), d) && !std::count(dd.rc.begin(), dd.rc.end(), d)) rf.push_back(d);
    // collapse a group of dims of a view into one (size, stride); false if
    // their memory layout does not allow it
    auto group = [](const View& v, const std::vector<int64_t>& ds, int64_t* size, int64_t* stride) {
      *size = 1;
      *stride = 0;
      std::vector<int64_t> nz;
      for (int64_t d : ds) {
        *size *= v.dims[d];
        if (v.dims[d] != 1) nz.push_back(d);
      }
      if (nz.empty()) {
        *stride = 0;
        return true;
      }
      for (size_t i = 0; i + 1 < nz.size(); ++i)
        if (v.strides[nz[i]] != v.strides[nz[i + 1]] * v.dims[nz[i + 1]]) return false;
      *stride = v.strides[nz.back()];
      return true;
    };
    int64_t B = 1, M, N, K, K2, a_bs = 0, a_ms, a_ks, b_bs = 0, b_ks, b_ns, Bb = 1;
    bool ok = group(lv, dd.lb, &B, &a_bs) && group(lv, lf, &M, &a_ms) && group(lv, dd.lc, &K, &a_ks) &&
              group(rv, dd.rb, &Bb, &b_bs) && group(rv, rf, &N, &b_ns) && group(rv, dd.rc, &K2, &b_ks);
    if (ok && (a_ms != 1 && a_ks != 1 && M != 1 && K != 1)) ok = false;
    if (ok && (b_ks != 1 && b_ns != 1 && K != 1 && N != 1)) ok = false;
    if (!ok) {
      // materialise each operand as dense [batch..., free..., contract...]
      auto canon = [&](View v, std::vector<int64_t> order) {
        View p = v;
        for (size_t k2 = 0; k2 < order.size(); ++k2) {
          p.dims[k2] = v.dims[order[k2]];
          p.strides[k2] = v.strides[order[k2]];
        }
        return Densify(p);
      };
      std::vector<int64_t> lo = dd.lb, ro = dd.rb;
      lo.insert(lo.end(), lf.begin(), lf.end());
      lo.insert(lo.end(), dd.lc.begin(), dd.lc.end());
      ro.insert(ro.end(), dd.rc.begin(), dd.rc.end());
      ro.insert(ro.end(), rf.begin(), rf.end());
      lv = canon(lv, lo);
      rv = canon(rv, ro);
      const size_t nb = dd.lb.size(), nlf = lf.size(), nrc = dd.rc.size();
      std::vector<int64_t> gb, gf, gc, rgb, rgc, rgf;
      for (size_t i = 0; i < nb; ++i) gb.push_back(int64_t(i)), rgb.push_back(int64_t(i));
      for (size_t i = 0; i < nlf; ++i) gf.push_back(int64_t(nb + i));
      for (size_t i = 0; i < dd.lc.size(); ++i) gc.push_back(int64_t(nb + nlf + i));
      for (size_t i = 0; i < nrc; ++i) rgc.push_back(int64_t(nb + i));
      for (size_t i = 0; i < rf.size(); ++i) rgf.push_back(int64_t(nb + nrc + i));
      if (!(group(lv, gb, &B, &a_bs) && group(lv, gf, &M, &a_ms) && group(lv, gc, &K, &a_ks) &&
            group(rv, rgb, &Bb, &b_bs) && group(rv, rgc, &K2, &b_ks) && group(rv, rgf, &N, &b_ns)))
        throw std::string("jam: dot_general operand layout could not be canonicalised");
    }
    if (K != K2 || B != Bb) throw std::string("jam: dot_general dimension mismatch");
    if (M == 1) a_ms = a_ks == 1 ? K : 1;
    if (K == 1) a_ks = 1;
    if (N == 1) b_ns = b_ks == 1 ? K : 1;
    if (B == 1) a_bs = b_bs = 0;
    const DType ct = m_.types[res].dtype;
    // a padded destination (rows c_pitch apart) when the result's last dim is N
    const int64_t pad = (B == 1 && !epi && m_.types[res].dims.back() == N) ? PaddedPitch(res) : 0;
    const int64_t c_pitch = pad > 0 ? pad : N;
    BufRef d = pad > 0 ? NewPaddedTemp(res, pad) : DestFor(res);
    auto set_result = [&](BufRef where) {
      if (pad > 0) SetPaddedView(res, where, pad);
      else SetDenseView(res, where);
    };
    Step st;
    st.kind = StepKind::kGemm;
    // bf16 operands whose rows are not 16-byte aligned (a vocabulary of
    // 50257) rule out the tiled kernel's 16-byte HBM->LDS copies; large such
    // products go to the library GEMM, as the hand-scheduled step's
    // vocabulary products do (the general kernel runs them at a tenth of
    // its rate), the rest to mk_gemm's general kernel
    const auto rows8 = [](int64_t bs, int64_t ms, int64_t ks) { return bs % 8 == 0 && (ms == 1 ? ks : ms) % 8 == 0; };
    if (at == DType::kBF16 && !epi && (ct == DType::kF32 || ct == DType::kBF16) &&
        !(rows8(a_bs, a_ms, a_ks) && rows8(b_bs, b_ns, b_ks)) && double(B) * M * N * K >= double(int64_t(1) << 30))
      st.kind = StepKind::kGemmBlas;
    // one fp32 product with few output tiles and a long contraction (the
    // weight gradients Xᵀ·dY, contracted over the tokens): the K axis is cut
    // into slices summed in order (mk_gemm_splitk), enough of them that the
    // grid covers the CUs (about 400 workgroups of 128x128), each slice at
    // least 256 deep
    // fp32 operands (mk_gemm's general kernel, 128x128 tiles) with fewer
    // output tiles than CUs (config C1's [256,1024]x[1024,4096] has 64, its
    // [256,4096]x[4096,1024] 16) are cut the same way into about 256
    // workgroups, slices at least 128 deep (512 workgroups measured no
    // faster); a fused bias / ReLU then runs as an elementwise pass over the
    // summed product.
    const int64_t tiles128 = ((M + 127) / 128) * ((N + 127) / 128);
    const bool f32_underfill = at == DType::kF32 && tiles128 < 256 && K >= 256;
    if (st.kind == StepKind::kGemm && (!epi || f32_underfill) && B == 1 && ct == DType::kF32 && N % 4 == 0 &&
        (K >= 2 * std::max(M, N) || f32_underfill)) {
      const int64_t tiles = tiles128;
      int64_t splits = 1;
      // bf16 operands: K need not divide evenly (mk_gemm_splitk's uneven
      // slices, a contraction over a vocabulary of 50257)
      const bool any_k = at == DType::kBF16;
      if (f32_underfill)
        while (splits < 16 && tiles * splits < 256 && K % (2 * splits) == 0 && K / (2 * splits) >= 128) splits *= 2;
      else
        while (splits < 8 && tiles * splits < 400 && (any_k || K % (2 * splits) == 0) && K / (2 * splits) >= 256)
          splits *= 2;
      if (splits > 1) {
        st.kind = StepKind::kGemmSplitK;
        st.bufs = {lv.at(), rv.at(), d, NewTemp(mk_gemm_splitk_workspace_bytes(M, N, splits))};
        st.i = {int64_t(at), M, N, K, a_ms, a_ks, b_ks, b_ns, c_pitch, splits, 0};
        st.note = std::to_string(M) + "x" + std::to_string(N) + "x" + std::to_string(K) + " in " +
                  std::to_string(splits) + " slices";
        if (epi) {
          // the bias (+ ReLU) applied by the pass that sums the slices
          const View bv = Densify(NeedView(epi->bias));
          if (bv.dtype != DType::kF32) throw std::string("jam: split product with a non-f32 bias");
          st.bufs.push_back(bv.at());
          st.i[10] = epi->relu ? 2 : 1;
          st.note += epi->relu ? ", + bias + relu" : ", + bias";
        }
        Emit(st);
        set_result(d);
        return;
      }
    }
    // an f32 product every reader rounds to bf16 is written in bf16 (one
    // rounding of the fp32 accumulator, as the module's convert does); with
    // a matched fp32 bias (+ ReLU) the epilogue adds it to the fp32
    // accumulator before that rounding (mk_gemm epilogue 5 / 6), which is
    // the module's f32 add followed by its convert
    bool narrow_out = false;
    if (pad == 0 && ct == DType::kF32 && at == DType::kBF16 && NarrowOnly(res, false) &&
        (!epi || m_.types[epi->bias].dtype == DType::kF32)) {
      narrow_out = true;
      d = NewTemp(size_t(m_.types[res].numel()) * 2);
    }
    st.bufs = {lv.at(), rv.at(), d};
    int epilogue = 0;
    if (epi) {
      const View& bv = NeedView(epi->bias);
      st.bufs.push_back(Densify(bv).at());
      epilogue = (epi->relu ? 2 : 1) | (narrow_out ? 4 : 0);
    }
    st.i = {int64_t(at), int64_t(narrow_out ? DType::kBF16 : ct), B, M, N, K, a_bs, a_ms, a_ks, b_bs, b_ks, b_ns,
            M * N, c_pitch, epilogue};
    st.note = std::to_string(B) + "x" + std::to_string(M) + "x" + std::to_string(N) + "x" + std::to_string(K);
    if (narrow_out) st.note += " -> bf16";
    // the GELU side output (TryMatchGemmGelu) where mk_gemm_bias_gelu takes
    // these layouts: the tiled kernel's operands (bf16, a unit stride, the
    // other a multiple of 8, 16-byte aligned bases) and fp32 C rows of whole
    // 16-byte chunks
    BufRef gelu_buf{};
    if (epi && epi->gelu_out >= 0 && !narrow_out && pad == 0 && B == 1 && at == DType::kBF16 &&
        ct == DType::kF32 && M >= 128 && N >= 128 && K >= 64 && N % 4 == 0 && c_pitch == N) {
      const bool a_ok = (a_ks == 1 && a_ms % 8 == 0 && a_ms >= K) || (a_ms == 1 && a_ks % 8 == 0 && a_ks >= M);
      const bool b_ok = (b_ks == 1 && b_ns % 8 == 0 && b_ns >= K) || (b_ns == 1 && b_ks % 8 == 0 && b_ks >= N);
      if (a_ok && b_ok && lv.at().offset % 16 == 0 && rv.at().offset % 16 == 0 && d.offset % 16 == 0) {
        gelu_buf = NewTemp(size_t(M * N) * 2);
        st.bufs.push_back(gelu_buf);
        st.i.push_back(N);
        st.note += " + gelu side output";
      }
    }
    Emit(st);
    if (gelu_buf.space == Space::kArena) {
      SetDenseView(epi->gelu_out, gelu_buf);
      preset_.insert(producer_[epi->gelu_out]);
    }
    if (narrow_out) {
      View nv;
      nv.buf = d;
      nv.dtype = DType::kBF16;
      nv.dims = m_.types[res].dims;
      nv.strides = DenseStrides(nv.dims);
      narrow_[res] = nv;
      return;
    }
    set_result(d);
  }

  void LowerGather(int idx) {
    const Op& op = ops_[idx];
    const Attr* dn = op.attr("dimension_numbers");
    if (!dn) throw std::string("jam: gather without dimension_numbers");
    auto gi = [&](const char* k) {
      const Attr* a = dn->get(k);
      return a ? a->ints() : std::vector<int64_t>{};
    };
    const auto offset_dims = gi("offset_dims"), collapsed = gi("collapsed_slice_dims"),
               start_map = gi("start_index_map");
    const auto ivd = gi("index_vector_dim");
    const auto slice = attr_ints(op, {"slice_sizes"});
    const int tbl = op.operands[0], ids = op.operands[1];
    const TensorType& tt = m_.types[tbl];
    const TensorType& it = m_.types[ids];
    const TensorType& ot = m_.types[op.results[0]];
    // row gather: table[N, rest...], one collapsed dim 0, full slices elsewhere
    bool row = collapsed == std::vector<int64_t>{0} && start_map == std::vector<int64_t>{0} &&
               int(slice.size()) == tt.rank() && slice[0] == 1;
    for (int d = 1; row && d < tt.rank(); ++d) row = slice[d] == tt.dims[d];
    const int64_t ivdim = ivd.empty() ? it.rank() : ivd[0];
    const int64_t batch_rank = ivdim == it.rank() ? it.rank() : it.rank() - 1;
    if (row) {  // offset dims must be the trailing output dims
      for (size_t k = 0; k < offset_dims.size(); ++k) row = row && offset_dims[k] == batch_rank + int64_t(k);
    }
    if (!row || (ivdim != it.rank() && it.dims[ivdim] != 1))
      throw std::string("jam: only row gathers (embedding lookups) are supported");  // cf. gather_scatter.mm:135-207
    const View& tv = NeedView(tbl);
    const View tvd = Densify(tv);
    const View iv = Densify(NeedView(ids));
    if (it.dtype != DType::kI32 && it.dtype != DType::kI64)
      throw std::string("jam: gather indices must be i32 or i64");
    BufRef d = DestFor(op.results[0]);
    int64_t row_elems = 1;
    for (int k = 1; k < tt.rank(); ++k) row_elems *= tt.dims[k];
    Step st;
    st.kind = StepKind::kGather;
    st.bufs = {tvd.at(), iv.at(), d};
    st.i = {tt.dims[0], row_elems * DTypeBytes(tt.dtype), int64_t(it.dtype), ot.numel() / std::max<int64_t>(row_elems, 1)};
    Emit(st);
    SetDenseView(op.results[0], d);
  }

  void LowerScatter(int idx) {
    const Op& op = ops_[idx];
    if (op.operands.size() != 3) throw std::string("jam: variadic scatter is not supported");
    const std::string body = op.regions.empty() ? "" : reduce_body_op(op);
    if (body != "stablehlo.add") throw std::string("jam: only scatter-add is supported (body '" + body + "')");
    const Attr* dn = op.attr("scatter_dimension_numbers");
    if (!dn) throw std::string("jam: scatter without dimension numbers");
    auto gi = [&](const char* k) {
      const Attr* a = dn->get(k);
      return a ? a->ints() : std::vector<int64_t>{};
    };
    const auto inserted = gi("inserted_window_dims"), todims = gi("scatter_dims_to_operand_dims"),
               uwd = gi("update_window_dims");
    const int tbl = op.operands[0], ids = op.operands[1], upd = op.operands[2];
    const TensorType& tt = m_.types[tbl];
    const TensorType& ut = m_.types[upd];
    bool row = inserted == std::vector<int64_t>{0} && todims == std::vector<int64_t>{0};
    int64_t row_elems = 1;
    for (int k = 1; k < tt.rank(); ++k) row_elems *= tt.dims[k];
    // update windows are the trailing update dims and cover whole rows
    for (size_t k = 0; row && k < uwd.size(); ++k) row = uwd[k] == ut.rank() - int64_t(uwd.size()) + int64_t(k);
    if (!row) throw std::string("jam: only row scatter-adds are supported");  // cf. gather_scatter.mm:262-335
    const DType dt = tt.dtype;
    if (dt != DType::kF32 && dt != DType::kBF16) throw std::string("jam: scatter-add on ") + DTypeName(dt) + " is not supported";
    const View tv = Densify(NeedView(tbl));
    const View iv = Densify(NeedView(ids));
    const View uv = Densify(NeedView(upd));
    const int64_t n_ids = ut.numel() / std::max<int64_t>(row_elems, 1);
    BufRef d = DestFor(op.results[0]);
    BufRef ws = NewTemp(mk_scatter_add_workspace_bytes(tt.dims[0], n_ids));
    Step st;
    st.kind = StepKind::kScatterAdd;
    st.bufs = {tv.at(), iv.at(), uv.at(), d, ws};
    st.i = {int64_t(dt), tt.dims[0], row_elems, int64_t(m_.types[ids].dtype), n_ids};
    Emit(st);
    SetDenseView(op.results[0], d);
  }

  void LowerConcat(int idx) {
    const Op& op = ops_[idx];
    const auto dd = attr_ints(op, {"dim", "dimension"});
    const int64_t dim = dd.empty() ? 0 : dd[0];
    const TensorType& t = m_.types[op.results[0]];
    // operands with narrow copies, read only narrow: when the copies already
    // lie side by side along `dim` (gradients written into place by their
    // kernel), the result is a view of them; else the concatenation is made
    // of the narrow copies (half the bytes of the wide form)
    bool narrow = NarrowOnly(op.results[0]);
    for (int v : op.operands) narrow = narrow && narrow_.count(v);
    if (narrow) {
      const View& v0 = narrow_[op.operands[0]];
      bool tiled = true;
      int64_t at = 0;
      for (int v : op.operands) {
        const View& w = narrow_[v];
        tiled = tiled && w.buf.space == v0.buf.space && w.buf.index == v0.buf.index &&
                w.buf.offset == v0.buf.offset && w.dtype == v0.dtype && w.strides == v0.strides &&
                w.offset == v0.offset + at * v0.strides[size_t(dim)];
        for (int k = 0; tiled && k < t.rank(); ++k)
          if (k != dim) tiled = w.dims[size_t(k)] == t.dims[size_t(k)];
        at += m_.types[v].dims[size_t(dim)];
      }
      View rv = v0;
      rv.dims = t.dims;
      if (tiled) {
        narrow_[op.results[0]] = rv;
        return;
      }
      View out;
      out.dtype = v0.dtype;
      out.dims = t.dims;
      out.strides = DenseStrides(t.dims);
      out.buf = NewTemp(size_t(t.numel()) * DTypeBytes(v0.dtype));
      // copy each operand into its block: a dense destination needs the
      // blocks contiguous, so along an inner dim the narrow result is kept
      // dim-major and handed out as a strided view (as below)
      std::vector<int> order{int(dim)};
      for (int k = 0; k < t.rank(); ++k)
        if (k != dim) order.push_back(k);
      int64_t off = 0;
      for (int v : op.operands) {
        const View& sv = narrow_[v];
        View pv = sv;
        for (size_t k = 0; k < order.size(); ++k) {
          pv.dims[k] = sv.dims[size_t(order[k])];
          pv.strides[k] = sv.strides[size_t(order[k])];
        }
        BufRef part = out.buf;
        part.offset += off;
        EmitCopy(pv, part);
        off += m_.types[v].numel() * DTypeBytes(v0.dtype);
      }
      std::vector<int64_t> pdims;
      for (int k : order) pdims.push_back(t.dims[size_t(k)]);
      const std::vector<int64_t> ps = DenseStrides(pdims);
      out.strides.assign(t.rank(), 0);
      for (size_t k = 0; k < order.size(); ++k) out.strides[size_t(order[k])] = ps[k];
      narrow_[op.results[0]] = out;
      return;
    }
    int64_t outer = 1;
    for (int64_t k = 0; k < dim; ++k) outer *= t.dims[k];
    if (outer != 1) {
      // Along an inner dim the result is stored with `dim` outermost: each
      // operand, viewed with `dim` moved first, is copied densely into its
      // block, and consumers get the permuted (strided) view of the buffer.
      std::vector<int> order{int(dim)};
      for (int k = 0; k < t.rank(); ++k)
        if (k != dim) order.push_back(k);
      BufRef d = NewTemp(t.bytes());
      int64_t off = 0;
      for (int v : op.operands) {
        const View& sv = NeedView(v);
        View pv = sv;
        for (size_t k = 0; k < order.size(); ++k) {
          pv.dims[k] = sv.dims[order[k]];
          pv.strides[k] = sv.strides[order[k]];
        }
        BufRef part = d;
        part.offset += off;
        EmitCopy(pv, part);
        off += int64_t(m_.types[v].bytes());
      }
      std::vector<int64_t> pdims;
      for (int k : order) pdims.push_back(t.dims[k]);
      const std::vector<int64_t> ps = DenseStrides(pdims);
      View rv;
      rv.buf = d;
      rv.offset = 0;
      rv.dtype = t.dtype;
      rv.dims = t.dims;
      rv.strides.assign(t.rank(), 0);
      for (size_t k = 0; k < order.size(); ++k) rv.strides[order[k]] = ps[k];
      SetView(op.results[0], rv);
      return;
    }
    BufRef d = DestFor(op.results[0]);
    int64_t off = 0;
    for (int v : op.operands) {
      const View& sv = NeedView(v);
      BufRef part = d;
      part.offset += off;
      EmitCopy(sv, part);
      off += int64_t(m_.types[v].bytes());
    }
    SetDenseView(op.results[0], d);
  }

  // -------------------------------------------------------------- fused steps
  // a bf16 -> f32 (or other) conversion step of a dense buffer
  void EmitConvert(BufRef src, DType from, BufRef dst, DType to, int64_t n) {
    Step st;
    st.kind = StepKind::kConvert;
    st.bufs = {src, dst};
    st.i = {int64_t(from), int64_t(to), n};
    Emit(st);
  }

  void EmitFused(int anchor, const Fused& f) {
    const Op& op = ops_[anchor];
    auto bf16_rows = [](const View& x) { return x.strides[3] == 1 && x.dtype == DType::kBF16; };
    if (f.kind == Fused::kSdpa) {
      const View& q = NeedView(f.q);
      const View& k = NeedView(f.k);
      const View& v = NeedView(f.v);
      View qv = bf16_rows(q) ? q : Densify(q), kv = bf16_rows(k) ? k : Densify(k),
           vv = bf16_rows(v) ? v : Densify(v);
      const int res = op.results[0];
      const auto& od = m_.types[res].dims;
      // training: O in bf16 (kept for the backward) plus lse, then O in the
      // module's dtype
      const bool bf16_out = m_.types[res].dtype == DType::kBF16 && !f.train;
      const int64_t n = od[0] * od[1] * od[2] * od[3];
      BufRef d = bf16_out ? DestFor(res) : NewTemp(size_t(n) * 2);
      // in a training step whose f32 O is only read back in bf16 (the head
      // merge [B,H,S,D] -> [B,S,H·D] ahead of the output projection), O is
      // written in [B,S,H,D] order: the merge is then a dense view of it
      const bool narrow = f.train && NarrowOnly(res);
      View ov;
      ov.buf = d;
      ov.dtype = DType::kBF16;
      ov.dims = od;
      ov.strides = narrow ? std::vector<int64_t>{od[2] * od[1] * od[3], od[3], od[1] * od[3], 1}
                          : DenseStrides(od);
      Step st;
      st.kind = StepKind::kSdpa;
      st.bufs = {qv.at(), kv.at(), vv.at(), d};
      st.i = {qv.dims[0], qv.dims[1], qv.dims[2], kv.dims[2], qv.dims[3],
              qv.strides[0], qv.strides[1], qv.strides[2],
              kv.strides[0], kv.strides[1], kv.strides[2],
              vv.strides[0], vv.strides[1], vv.strides[2],
              ov.strides[0], ov.strides[1], ov.strides[2], f.causal ? 1 : 0};
      st.f = {f.scale};
      st.note = f.causal ? "causal" : "full";
      BufRef lse;
      if (f.train) {
        lse = NewTemp(size_t(od[0] * od[1] * od[2]) * 4);
        st.bufs.push_back(lse);
        st.note += " +lse";
      }
      Emit(st);
      if (f.train) sdpa_saved_[anchor] = {ov, lse};
      if (bf16_out) {
        SetDenseView(res, d);
      } else if (narrow) {
        narrow_[res] = ov;
      } else {
        BufRef o = DestFor(res);
        EmitConvert(d, DType::kBF16, o, m_.types[res].dtype, n);
        SetDenseView(res, o);
      }
      return;
    }
    if (f.kind == Fused::kXent) {
      // logits rows may be padded (row stride >= cols, unit stride along them)
      View x = NeedView(f.x);
      if (!(x.rank() == 2 && x.strides[1] == 1 && x.strides[0] >= x.dims[1])) x = Densify(x);
      View lab = NeedView(f.labels);
      if (!lab.dense()) lab = Densify(lab);
      const int res = op.results[0];
      BufRef lr = DestFor(res);
      const bool to_bf16 = !f.dlogits_bf16.empty();
      const int dv = to_bf16 ? f.dlogits_bf16[0] : f.dlogits;
      const int64_t dpad = PaddedPitch(dv);
      BufRef dx = dpad > 0 ? NewPaddedTemp(dv, dpad) : DestFor(dv);
      Step st;
      st.kind = StepKind::kSoftmaxXent;
      st.bufs = {x.at(), lab.at(), lr, dx};
      st.i = {int64_t(x.dtype), x.dims[0], x.dims[1], int64_t(lab.dtype),
              int64_t(to_bf16 ? DType::kBF16 : x.dtype), x.strides[0], dpad > 0 ? dpad : x.dims[1]};
      st.f = {f.scale};
      if (x.strides[0] != x.dims[1] || dpad > 0) st.note = "rows padded";
      Emit(st);
      SetDenseView(res, lr);
      auto set_dx = [&](int v) {
        if (dpad > 0) SetPaddedView(v, dx, dpad);
        else SetDenseView(v, dx);
      };
      if (to_bf16) {
        for (int c : f.dlogits_bf16) set_dx(c);
      } else {
        set_dx(f.dlogits);
      }
      return;
    }
    if (f.kind == Fused::kSdpaBwd) {
      const View& q = NeedView(f.q);
      const View& k = NeedView(f.k);
      const View& v = NeedView(f.v);
      const View& g = NeedView(f.dout);
      View qv = bf16_rows(q) ? q : Densify(q), kv = bf16_rows(k) ? k : Densify(k),
           vv = bf16_rows(v) ? v : Densify(v), gv = bf16_rows(g) ? g : Densify(g);
      const auto it = sdpa_saved_.find(f.fwd);
      if (it == sdpa_saved_.end()) throw std::string("jam: attention backward before its forward");
      const int64_t B = qv.dims[0], H = qv.dims[1], Sq = qv.dims[2], Sk = kv.dims[2], D = qv.dims[3];
      BufRef ws = NewTemp(mk_sdpa_bwd_workspace_bytes(B, H, Sq, Sk, D));
      const View& ov = it->second.first;
      // the gradients (bf16 from the kernel, f32 in the module): when each is
      // only read back in bf16 and the three are merged to [B,S,H·D] and
      // concatenated along the features (the fused QKV projection's
      // gradient), they are written straight into that [B·S, 3·H·D] layout
      const int grads_v[3] = {f.dq, f.dk, f.dv};
      const int merged = MergedQkvConcat(grads_v, B, H, Sq, D);
      View gview[3];
      if (merged >= 0 && Sq == Sk) {
        BufRef buf = NewTemp(size_t(B * Sq * 3 * H * D) * 2);
        for (int k = 0; k < 3; ++k) {
          gview[k].buf = buf;
          gview[k].dtype = DType::kBF16;
          gview[k].dims = {B, H, Sq, D};
          gview[k].strides = {Sq * 3 * H * D, D, 3 * H * D, 1};
          gview[k].offset = int64_t(k) * H * D;
        }
      } else {
        for (int k = 0; k < 3; ++k) {
          const int64_t S_k = k == 0 ? Sq : Sk;
          gview[k].buf = NewTemp(size_t(B * H * S_k * D) * 2);
          gview[k].dtype = DType::kBF16;
          gview[k].dims = {B, H, S_k, D};
          gview[k].strides = DenseStrides(gview[k].dims);
        }
      }
      Step st;
      st.kind = StepKind::kSdpaBwd;
      st.bufs = {qv.at(), kv.at(), vv.at(), ov.at(), gv.at(), it->second.second,
                 gview[0].at(), gview[1].at(), gview[2].at(), ws};
      st.i = {B, H, Sq, Sk, D,
              qv.strides[0], qv.strides[1], qv.strides[2],
              kv.strides[0], kv.strides[1], kv.strides[2],
              vv.strides[0], vv.strides[1], vv.strides[2],
              ov.strides[0], ov.strides[1], ov.strides[2],
              gv.strides[0], gv.strides[1], gv.strides[2],
              gview[0].strides[0], gview[0].strides[1], gview[0].strides[2],
              gview[1].strides[0], gview[1].strides[1], gview[1].strides[2],
              gview[2].strides[0], gview[2].strides[1], gview[2].strides[2],
              f.causal ? 1 : 0};
      st.f = {f.scale};
      st.note = std::string(f.causal ? "causal" : "full") + (merged >= 0 ? ", into the merged QKV gradient" : "");
      Emit(st);
      for (int k = 0; k < 3; ++k) {
        const int g = grads_v[k];
        if (m_.types[g].dtype == DType::kF32 && NarrowOnly(g)) {
          narrow_[g] = gview[k];
          continue;
        }
        const View src = gview[k].dense() ? gview[k] : Densify(gview[k]);
        BufRef o = DestFor(g);
        EmitConvert(src.at(), DType::kBF16, o, m_.types[g].dtype, m_.types[g].numel());
        SetDenseView(g, o);
      }
      return;
    }
    if (f.kind == Fused::kArgmax) {
      View x = NeedView(f.x);
      const auto dims = reduce_dims(op);
      const int rd = int(dims[0]);
      // reduced dim last, dense rows
      View pv = x;
      int k = 0;
      int64_t rows = 1;
      for (int d = 0; d < x.rank(); ++d)
        if (d != rd) {
          pv.dims[k] = x.dims[d];
          pv.strides[k++] = x.strides[d];
          rows *= x.dims[d];
        }
      pv.dims[k] = x.dims[rd];
      pv.strides[k] = x.strides[rd];
      pv = Densify(pv);
      const int rv = op.results[0], ri = op.results[1];
      const bool need_vals = live_value(rv);
      BufRef dv = need_vals ? DestFor(rv) : BufRef{};
      BufRef di = DestFor(ri);
      Step st;
      st.kind = StepKind::kArgmax;
      st.bufs = {pv.at(), dv, di};
      st.i = {int64_t(x.dtype), f.is_min ? 1 : 0, rows, x.dims[rd], int64_t(m_.types[ri].dtype), need_vals ? 1 : 0};
      Emit(st);
      if (need_vals) SetDenseView(rv, dv);
      SetDenseView(ri, di);
      return;
    }
    if (f.kind == Fused::kGemmEpi) {
      LowerDot(f.dot, &f, op.results[0]);
      return;
    }
    if (f.kind == Fused::kGelu) {
      const View x = Densify(NeedView(f.x));
      const int res = op.results[0];
      BufRef d = DestFor(res);
      Step st;
      st.kind = StepKind::kGelu;
      st.bufs = {x.at(), d};
      st.i = {int64_t(f.out_dtype), x.numel()};
      Emit(st);
      SetDenseView(res, d);
      return;
    }
    if (f.kind == Fused::kLayerNorm) {
      const bool add = f.add_a >= 0;
      const View x = Densify(NeedView(add ? f.add_a : f.x));
      BufRef g{}, b{};
      if (f.gamma >= 0) g = Densify(NeedView(f.gamma)).at();
      if (f.beta >= 0) b = Densify(NeedView(f.beta)).at();
      const int res = op.results[0];
      BufRef d = DestFor(res);
      const int64_t cols = x.dims.back();
      Step st;
      st.kind = StepKind::kLayerNorm;
      st.bufs = {x.at(), g, b, d};
      st.i = {int64_t(f.out_dtype), x.numel() / std::max<int64_t>(cols, 1), cols};
      if (f.in_dtype != f.out_dtype || add) {
        st.i.push_back(int64_t(f.in_dtype));
        st.note = std::string(DTypeName(f.in_dtype)) + " -> " + DTypeName(f.out_dtype);
      }
      BufRef xs{};
      if (add) {
        // x = a + b written by the step (bufs 4, 5: b and x)
        const View b2 = Densify(NeedView(f.add_b));
        xs = DestFor(f.x);
        st.bufs.push_back(b2.at());
        st.bufs.push_back(xs);
        st.note += ", input added";
      }
      st.f = {f.eps};
      Emit(st);
      if (add) SetDenseView(f.x, xs);
      SetDenseView(res, d);
      return;
    }
    if (f.kind == Fused::kLayerNormBwd) {
      const View x = Densify(NeedView(f.x));
      const View g = Densify(NeedView(f.gamma));
      const View dy = Densify(NeedView(f.dout));
      const int64_t cols = x.dims.back(), rows = x.numel() / std::max<int64_t>(cols, 1);
      BufRef dres{};
      if (f.dres >= 0) dres = Densify(NeedView(f.dres)).at();
      const int res = op.results[0];
      BufRef dx = DestFor(res);
      // dgamma and dbeta are written together (dbeta to scratch when the
      // module does not read it)
      BufRef dg = DestFor(f.dgamma);
      BufRef db = f.dbeta >= 0 ? DestFor(f.dbeta) : NewTemp(size_t(cols) * 4);
      BufRef cs = f.colsum >= 0 ? DestFor(f.colsum) : BufRef{};
      BufRef ws = NewTemp(mk_layernorm_bwd_workspace_bytes(rows, cols));
      Step st;
      st.kind = StepKind::kLayerNormBwd;
      st.bufs = {x.at(), g.at(), dy.at(), dres, dx, dg, db, cs, ws};
      st.i = {int64_t(DType::kF32), rows, cols};
      st.f = {f.eps};
      st.note = std::string(f.dres >= 0 ? "residual" : "no residual") + (f.colsum >= 0 ? ", bias gradient" : "");
      BufRef d16{};
      if (!f.dx_bf16.empty()) {
        d16 = DestFor(f.dx_bf16[0]);
        st.bufs.push_back(d16);
        st.note += ", bf16 copy";
      }
      Emit(st);
      SetDenseView(res, dx);
      for (int c : f.dx_bf16) SetDenseView(c, d16);
      SetDenseView(f.dgamma, dg);
      if (f.dbeta >= 0) SetDenseView(f.dbeta, db);
      if (f.colsum >= 0) SetDenseView(f.colsum, cs);
      return;
    }
    throw std::string("jam: internal: unknown fused pattern");
  }

  bool live_value(int v) const {
    for (int o : outputs_)
      if (o == v) return true;
    for (int u : users_[v])
      if (live_[u]) return true;
    return false;
  }

  struct Temp {
    size_t size;
    int first, last;
  };

  Module& m_;
  CompileOptions opts_;
  std::shared_ptr<Program> prog_;
  std::vector<Op> ops_;
  std::vector<int> outputs_;
  std::set<const Func*> inlined_once_;
  std::vector<int> producer_, uses_;
  std::vector<std::vector<int>> users_;
  // constant op index -> its parsed dense value (each constant is parsed
  // once per Compile, however often the matchers look at it)
  mutable std::unordered_map<int, std::shared_ptr<Attr>> const_cache_;
  std::vector<ValState> state_;
  std::map<int, Fused> fused_;
  std::set<int> absorbed_;
  // values stored with their rows (last dim) padded to this pitch (elements):
  // the logits and the gradient of a fused cross-entropy over a vocabulary
  // whose rows are not 16-byte multiples, so that the products that write
  // and read them take aligned rows
  std::map<int, int64_t> pad_rows_;
  std::vector<bool> reach_;
  std::map<int, std::pair<View, BufRef>> sdpa_saved_;  // training forward anchor -> (bf16 O view, lse)
  std::unordered_map<int, View> narrow_;   // f32 value -> bf16 view of the same values
  std::unordered_map<int, bool> narrow_only_;
  std::vector<bool> live_;
  std::vector<Temp> temps_;
  std::vector<bool> out_written_;
};

}  // namespace

namespace {

// Memory an ew step reads or writes: a byte range of one buffer.  A program
// output that a donated input may carry is the same buffer as that input.
struct Extent {
  int space, index;
  int64_t lo, hi;
};

bool Overlap(const std::vector<Extent>& a, const std::vector<Extent>& b) {
  for (const Extent& x : a)
    for (const Extent& y : b)
      if (x.space == y.space && x.index == y.index && x.lo < y.hi && y.lo < x.hi) return true;
  return false;
}

// Independent ew steps with the same generated kernel in one launch: each
// maximal run of consecutive jitted ew steps that pairwise touch no common
// memory (no step writes what another reads or writes) may run in any order,
// so the run's steps of one kernel become one batched step (placed at its
// first member), up to kEwJitMaxBatch instances each.  The Adam updates of
// a training step's parameters of one shape are such a run.
void BatchIndependentEwSteps(Program& prog) {
  EwJit& jit = *prog.ew_jit;
  std::vector<int> alias_of_output(prog.outputs.size(), -1);
  for (size_t in = 0; in < prog.input_alias.size(); ++in)
    if (prog.input_alias[in] >= 0 && size_t(prog.input_alias[in]) < alias_of_output.size())
      alias_of_output[size_t(prog.input_alias[in])] = int(in);
  auto ext = [&](const BufRef& b, int64_t lo, int64_t hi) {
    Extent e{int(b.space), b.index, b.offset + lo, b.offset + hi};
    if (b.space == Space::kOutput && alias_of_output[size_t(b.index)] >= 0) {
      e.space = int(Space::kInput);
      e.index = alias_of_output[size_t(b.index)];
    }
    if (b.space == Space::kArena) e.index = 0;
    return e;
  };
  struct Acc {
    std::vector<Extent> reads, writes;
  };
  auto access = [&](const Step& st) {
    Acc a;
    const int rank = int(st.i[0]), n_in = int(st.i[7]);
    int64_t n = 1;
    for (int d = 0; d < rank; ++d) n *= st.i[1 + size_t(d)];
    for (int t = 0; t < n_in; ++t) {
      const int64_t elt = DTypeBytes(DType(st.types[size_t(t)]));
      int64_t last = 0;
      bool neg = false;
      for (int d = 0; d < rank; ++d) {
        const int64_t str = st.i[1 + size_t(d)] == 1 ? 0 : st.strides[size_t(t * 6 + d)];
        neg |= str < 0;
        last += (st.i[1 + size_t(d)] - 1) * str;
      }
      a.reads.push_back(neg ? ext(st.bufs[size_t(t)], INT64_MIN / 4, INT64_MAX / 4)
                            : ext(st.bufs[size_t(t)], 0, (last + 1) * elt));
    }
    for (size_t o = size_t(n_in); o < st.bufs.size(); ++o) {
      const int64_t elt = DTypeBytes(DType(st.i[9 + 2 * (o - size_t(n_in))]));
      a.writes.push_back(ext(st.bufs[o], 0, n * elt));
    }
    return a;
  };
  auto batchable = [&](const Step& st) { return st.kind == StepKind::kEw && st.jit >= 0 && st.batch == 1; };
  std::vector<Step> out;
  out.reserve(prog.steps.size());
  std::map<std::pair<int, int>, int> batched_kernel;  // (single kernel, count) -> batched kernel
  auto flush = [&](std::vector<size_t>& run) {
    // groups by kernel, in order of first appearance
    std::vector<std::vector<size_t>> groups;
    std::map<int, size_t> group_of;
    for (size_t j : run) {
      auto it = group_of.find(prog.steps[j].jit);
      if (it == group_of.end()) {
        group_of[prog.steps[j].jit] = groups.size();
        groups.push_back({j});
      } else {
        groups[it->second].push_back(j);
      }
    }
    for (const auto& g : groups) {
      for (size_t c0 = 0; c0 < g.size(); c0 += kEwJitMaxBatch) {
        const size_t cnt = std::min(g.size() - c0, size_t(kEwJitMaxBatch));
        Step st = prog.steps[g[c0]];
        if (cnt > 1) {
          const int single = st.jit;
          auto key = std::make_pair(single, int(cnt));
          auto it = batched_kernel.find(key);
          if (it == batched_kernel.end()) {
            EwKernel bk;
            if (!BatchEwKernel(jit.kernel(single), int(cnt), &bk)) {
              for (size_t m = 0; m < cnt; ++m) out.push_back(prog.steps[g[c0 + m]]);
              continue;
            }
            it = batched_kernel.emplace(key, jit.Add(std::move(bk))).first;
          }
          st.jit = it->second;
          st.batch = int(cnt);
          for (size_t m = 1; m < cnt; ++m)
            st.bufs.insert(st.bufs.end(), prog.steps[g[c0 + m]].bufs.begin(), prog.steps[g[c0 + m]].bufs.end());
          st.note += ", " + std::to_string(cnt) + " independent instances";
        }
        out.push_back(std::move(st));
      }
    }
    run.clear();
  };
  std::vector<size_t> run;
  std::vector<Acc> run_acc;
  for (size_t j = 0; j < prog.steps.size(); ++j) {
    const Step& st = prog.steps[j];
    if (!batchable(st)) {
      flush(run);
      run_acc.clear();
      out.push_back(st);
      continue;
    }
    Acc a = access(st);
    bool indep = true;
    for (const Acc& b : run_acc)
      if (Overlap(a.writes, b.reads) || Overlap(a.writes, b.writes) || Overlap(b.writes, a.reads)) {
        indep = false;
        break;
      }
    if (!indep) {
      flush(run);
      run_acc.clear();
    }
    run.push_back(j);
    run_acc.push_back(std::move(a));
  }
  flush(run);
  prog.steps = std::move(out);
}

}  // namespace

CompileResult Compile(const char* code, size_t size, const CompileOptions& opts) {
  CompileResult r;
  std::unique_ptr<Module> m;
  std::string err;
  if (IsMlirBytecode(code, size)) {
    // A StableHLO portable artifact (what jaxlib serializes): the container
    // is read (bytecode.cc), its VHLO operations, types and attributes are
    // decoded into jam IR (vhlo.cc), and the module is lowered like text.
    bytecode::Module bm;
    std::string berr;
    if (!bytecode::Read(reinterpret_cast<const uint8_t*>(code), size, &bm, &berr)) {
      r.error = "jam: MLIR bytecode: " + berr;
      return r;
    }
    m = FromVhlo(bm, err);
    if (!m) {
      std::string dialects;
      for (size_t d = 0; d < bm.dialects.size(); ++d)
        dialects += (d ? ", " : "") + bm.DialectVersionText(d);
      r.error = err + " (artifact: MLIR bytecode v" + std::to_string(bm.version) + " from '" + bm.producer +
                "', dialects " + dialects + ", " + std::to_string(bm.attrs.size()) + " attributes, " +
                std::to_string(bm.types.size()) + " types; ops " + bm.OpHistogram() + ")";
      return r;
    }
  } else {
    m = ParseText(code, size, err);
    if (!m) {
      r.error = err;
      return r;
    }
  }
  Lowerer L(*m, opts);
  r.program = L.Run(err);
  if (!r.program) {
    r.error = err.empty() ? "jam: lowering failed" : err;
    return r;
  }
  if (opts.ew_jit) {
    // every ew step also as a generated kernel (ew_jit.h); one that cannot
    // be generated keeps the interpreter
    auto jit = std::make_shared<EwJit>();
    jit->strict = opts.ew_jit_strict;
    for (Step& st : r.program->steps) {
      if (st.kind != StepKind::kEw && st.kind != StepKind::kEwReduce) continue;
      EwKernel k;
      std::string why;
      if (GenerateEwKernel(st, &k, &why) && k.blocks > 0) st.jit = jit->Add(std::move(k));
      else if (opts.ew_jit_strict && !why.empty()) {
        r.program = nullptr;
        r.error = "jam: no generated kernel for ew step (" + st.note + "): " + why;
        return r;
      }
    }
    if (jit->size()) {
      r.program->ew_jit = jit;
      if (opts.ew_batch) BatchIndependentEwSteps(*r.program);
      if (opts.ew_jit_eager && !jit->Build()) r.program->patterns.push_back("ew_jit failed: " + jit->error());
    }
  }
  return r;
}

}  // namespace mi::jam
