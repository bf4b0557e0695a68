// Elementwise kernels: fused GELU(tanh), the generic fused elementwise
// program, convert, fill, iota and strided copy (transpose / broadcast).
//
// Streaming kernels move 16 bytes per lane per access (dwordx4) and each
// thread keeps kUnroll independent vectors in flight, so one wave has
// 64 × 16 × kUnroll bytes outstanding — what HBM3E needs to approach peak.
#include "mk_common.h"

#include <cmath>

namespace mk {
namespace {

constexpr int kBlock = 256;
constexpr int kUnroll = 4;

// gelu_tanh(x) = 0.5 x (1 + tanh(u)), u = sqrt(2/pi) (x + 0.044715 x^3).
// Using 1 + tanh(u) = 2 / (1 + exp(-2u)) gives gelu = x / (1 + exp(-2u)),
// which has no cancellation for negative x and needs one exp2 + one rcp.
// exp(-2u) = exp2(x * (c0 + c1 x^2)) with c0 = -2 sqrt(2/pi) log2(e).

template <typename T> struct V16;
template <> struct V16<uint16_t> { using V = u16x8; static constexpr int N = 8; };
template <> struct V16<float> { using V = f32x4; static constexpr int N = 4; };

template <typename T>
__device__ inline float cvt_in(T v) {
  if constexpr (sizeof(T) == 2) return bf16_to_f32(v);
  else return v;
}
template <typename T>
__device__ inline T cvt_out(float v) {
  if constexpr (sizeof(T) == 2) return f32_to_bf16(v);
  else return v;
}

template <typename T>
__global__ __launch_bounds__(kBlock) void gelu_vec_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                          int64_t nvec) {
  using V = typename V16<T>::V;
  constexpr int N = V16<T>::N;
  const V* xv = reinterpret_cast<const V*>(x);
  V* yv = reinterpret_cast<V*>(y);
  const int64_t base = int64_t(blockIdx.x) * (kBlock * kUnroll) + threadIdx.x;
  V a[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    int64_t i = base + int64_t(u) * kBlock;
    if (i < nvec) a[u] = ld_stream(&xv[i]);
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    int64_t i = base + int64_t(u) * kBlock;
    if (i < nvec) {
      V o;
#pragma unroll
      for (int j = 0; j < N; ++j) o.v[j] = cvt_out<T>(gelu_tanh_f32(cvt_in<T>(a[u].v[j])));
      st_stream(&yv[i], o);
    }
  }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void gelu_scalar_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                             int64_t begin, int64_t n) {
  int64_t i = begin + int64_t(blockIdx.x) * kBlock + threadIdx.x;
  if (i < n) y[i] = cvt_out<T>(gelu_tanh_f32(cvt_in<T>(x[i])));
}

// ------------------------------------------------------------------ ew program
constexpr int kEwMaxRank = 6;
constexpr int kEwMaxInputs = 8;
constexpr int kEwMaxRegs = 32;
constexpr int kEwMaxInstr = 64;
constexpr int kEwMaxConsts = 64;
constexpr int kEwMaxOutputs = 4;

struct EwArgs {
  const void* in[kEwMaxInputs];
  int in_type[kEwMaxInputs];
  int in_mode[kEwMaxInputs];  // 0 scalar (offset 0), 1 dense (offset = i), 2 strided
  int64_t in_stride[kEwMaxInputs][kEwMaxRank];
  int64_t dims[kEwMaxRank];
  int rank;
  int n_inputs;
  int n_instr;
  int n_out;                 // 1 .. kEwMaxOutputs dense outputs of the shape
  int out_reg[kEwMaxOutputs];
  int out_type[kEwMaxOutputs];
  void* out[kEwMaxOutputs];
  int need_index;  // some input is strided: decompose the linear index
  int in_vec[kEwMaxInputs];  // vector form: 4 consecutive elements in one 16-byte (f32) / 8-byte (bf16) load
  int out_vec[kEwMaxOutputs];  // vector form: 4 consecutive outputs in one store
  int32_t prog[kEwMaxInstr][4];
  float consts[kEwMaxConsts];
};

__device__ inline float as_f(int32_t i) { return __int_as_float(i); }
__device__ inline int32_t as_i(float f) { return __float_as_int(f); }

// Register file conventions: float types widen to fp32; integer types hold
// their int32 bit pattern (sign- / zero-extended, 64-bit truncated);
// predicates hold 0.0f / 1.0f.
__device__ inline float ew_load(const void* p, int64_t i, int t) {
  switch (t) {
    case MK_PRED: return reinterpret_cast<const uint8_t*>(p)[i] ? 1.f : 0.f;
    case MK_S8: return as_f(int32_t(reinterpret_cast<const int8_t*>(p)[i]));
    case MK_U8: return as_f(int32_t(reinterpret_cast<const uint8_t*>(p)[i]));
    case MK_S16: return as_f(int32_t(reinterpret_cast<const int16_t*>(p)[i]));
    case MK_U16: return as_f(int32_t(reinterpret_cast<const uint16_t*>(p)[i]));
    case MK_S32: case MK_U32: return as_f(reinterpret_cast<const int32_t*>(p)[i]);
    case MK_S64: case MK_U64: return as_f(int32_t(reinterpret_cast<const int64_t*>(p)[i]));
    default: return load_as_f32(p, i, t);
  }
}
__device__ inline void ew_store(void* p, int64_t i, int t, float v) {
  switch (t) {
    case MK_PRED: reinterpret_cast<uint8_t*>(p)[i] = v != 0.f; break;
    case MK_S8: case MK_U8: reinterpret_cast<uint8_t*>(p)[i] = uint8_t(as_i(v)); break;
    case MK_S16: case MK_U16: reinterpret_cast<uint16_t*>(p)[i] = uint16_t(as_i(v)); break;
    case MK_S32: case MK_U32: reinterpret_cast<int32_t*>(p)[i] = as_i(v); break;
    case MK_S64: reinterpret_cast<int64_t*>(p)[i] = int64_t(as_i(v)); break;
    case MK_U64: reinterpret_cast<uint64_t*>(p)[i] = uint64_t(uint32_t(as_i(v))); break;
    default: store_from_f32(p, i, t, v); break;
  }
}

__device__ inline float sign_f(float x) {
  return x > 0.f ? 1.f : (x < 0.f ? -1.f : x);  // keeps ±0 and NaN
}

// Runs the program on the register file r (inputs already in r[0 ..
// n_inputs)).  Each register holds W lanes (W consecutive elements of one
// thread; lane e of register k is r[e][k], each lane its own array so that
// each is indexed by the wave-uniform register number alone); an instruction is decoded once and applied to every lane with the
// same fp32 expression, so W = 4 gives the same bits per element as W = 1
// while paying the decode (scalar loads and the opcode dispatch) once per W
// elements.  NR (a power of two) registers per lane: the host checks that
// every register operand, destination and input is below NR; the operand
// fields are masked to NR - 1 because both are read for every opcode and a
// CONST's first field is a constant index, not a register.
template <int W, int NR>
__device__ __attribute__((always_inline)) inline void ew_run(const EwArgs& A, float* const (&r)[W]) {
  static_assert((NR & (NR - 1)) == 0 && NR <= kEwMaxRegs, "NR: a power of two, at most kEwMaxRegs");
  for (int p = 0; p < A.n_instr; ++p) {
    const int op = A.prog[p][0], dst = A.prog[p][1] & (NR - 1), a = A.prog[p][2] & (NR - 1), b = A.prog[p][3];
    float va[W], vb[W], o[W];
#pragma unroll
    for (int e = 0; e < W; ++e) {
      va[e] = r[e][a];
      vb[e] = r[e][b & (NR - 1)];
    }
    // o[e] = f(va[e], vb[e]) on every lane
    auto each = [&](auto f) __attribute__((always_inline)) {
#pragma unroll
      for (int e = 0; e < W; ++e) o[e] = f(va[e], vb[e]);
    };
    switch (op) {
      case MK_EW_CONST: each([&](float, float) { return A.consts[A.prog[p][2]]; }); break;
      case MK_EW_ADD: each([](float x, float y) { return x + y; }); break;
      case MK_EW_SUB: each([](float x, float y) { return x - y; }); break;
      case MK_EW_MUL: each([](float x, float y) { return x * y; }); break;
      case MK_EW_DIV: each([](float x, float y) { return x / y; }); break;
      case MK_EW_MAX: each([](float x, float y) { return (x != x || y != y) ? __builtin_nanf("") : fmaxf(x, y); }); break;
      case MK_EW_MIN: each([](float x, float y) { return (x != x || y != y) ? __builtin_nanf("") : fminf(x, y); }); break;
      case MK_EW_POW: each([](float x, float y) { return powf(x, y); }); break;
      case MK_EW_NEG: each([](float x, float) { return -x; }); break;
      case MK_EW_EXP: each([](float x, float) { return expf(x); }); break;
      case MK_EW_LOG: each([](float x, float) { return logf(x); }); break;
      case MK_EW_TANH: each([](float x, float) { return tanhf(x); }); break;
      case MK_EW_SQRT: each([](float x, float) { return sqrtf(x); }); break;
      case MK_EW_RSQRT: each([](float x, float) { return 1.f / sqrtf(x); }); break;
      case MK_EW_ABS: each([](float x, float) { return fabsf(x); }); break;
      case MK_EW_LOGISTIC: each([](float x, float) { return 1.f / (1.f + expf(-x)); }); break;
      case MK_EW_CMP_EQ: each([](float x, float y) { return x == y ? 1.f : 0.f; }); break;
      case MK_EW_CMP_NE: each([](float x, float y) { return x != y ? 1.f : 0.f; }); break;
      case MK_EW_CMP_LT: each([](float x, float y) { return x < y ? 1.f : 0.f; }); break;
      case MK_EW_CMP_LE: each([](float x, float y) { return x <= y ? 1.f : 0.f; }); break;
      case MK_EW_CMP_GT: each([](float x, float y) { return x > y ? 1.f : 0.f; }); break;
      case MK_EW_CMP_GE: each([](float x, float y) { return x >= y ? 1.f : 0.f; }); break;
      case MK_EW_SELECT: {
        const int c = (b >> 16) & (NR - 1);
#pragma unroll
        for (int e = 0; e < W; ++e) o[e] = va[e] != 0.f ? vb[e] : r[e][c];
        break;
      }
      case MK_EW_CLAMP: {
        const int c = (b >> 16) & (NR - 1);
#pragma unroll
        for (int e = 0; e < W; ++e) o[e] = fminf(fmaxf(va[e], vb[e]), r[e][c]);
        break;
      }
      case MK_EW_ROUND_BF16: each([](float x, float) { return bf16_to_f32(f32_to_bf16(x)); }); break;
      case MK_EW_ROUND_F16: each([](float x, float) { return f16_to_f32(f32_to_f16(x)); }); break;
      case MK_EW_FLOOR: each([](float x, float) { return floorf(x); }); break;
      case MK_EW_CEIL: each([](float x, float) { return ceilf(x); }); break;
      case MK_EW_SIGN: each([](float x, float) { return sign_f(x); }); break;
      case MK_EW_AND: each([](float x, float y) { return (x != 0.f && y != 0.f) ? 1.f : 0.f; }); break;
      case MK_EW_OR: each([](float x, float y) { return (x != 0.f || y != 0.f) ? 1.f : 0.f; }); break;
      case MK_EW_NOT: each([](float x, float) { return x == 0.f ? 1.f : 0.f; }); break;
      case MK_EW_MOV: each([](float x, float) { return x; }); break;
      case MK_EW_CMP_LT_S32: each([](float x, float y) { return as_i(x) < as_i(y) ? 1.f : 0.f; }); break;
      case MK_EW_CMP_GE_S32: each([](float x, float y) { return as_i(x) >= as_i(y) ? 1.f : 0.f; }); break;
      case MK_EW_ADD_S32: each([](float x, float y) { return as_f(as_i(x) + as_i(y)); }); break;
      case MK_EW_SUB_S32: each([](float x, float y) { return as_f(as_i(x) - as_i(y)); }); break;
      case MK_EW_MUL_S32: each([](float x, float y) { return as_f(as_i(x) * as_i(y)); }); break;
      case MK_EW_S32_TO_F32: each([](float x, float) { return float(as_i(x)); }); break;
      case MK_EW_F32_TO_S32: each([](float x, float) { return as_f(int32_t(x)); }); break;
      case MK_EW_ERF: each([](float x, float) { return erff(x); }); break;
      case MK_EW_CMP_EQ_S32: each([](float x, float y) { return as_i(x) == as_i(y) ? 1.f : 0.f; }); break;
      case MK_EW_CMP_NE_S32: each([](float x, float y) { return as_i(x) != as_i(y) ? 1.f : 0.f; }); break;
      case MK_EW_CMP_LE_S32: each([](float x, float y) { return as_i(x) <= as_i(y) ? 1.f : 0.f; }); break;
      case MK_EW_CMP_GT_S32: each([](float x, float y) { return as_i(x) > as_i(y) ? 1.f : 0.f; }); break;
      case MK_EW_MAX_S32: each([](float x, float y) { return as_f(max(as_i(x), as_i(y))); }); break;
      case MK_EW_MIN_S32: each([](float x, float y) { return as_f(min(as_i(x), as_i(y))); }); break;
      case MK_EW_NEG_S32: each([](float x, float) { return as_f(-as_i(x)); }); break;
      case MK_EW_AND_B32: each([](float x, float y) { return as_f(as_i(x) & as_i(y)); }); break;
      case MK_EW_OR_B32: each([](float x, float y) { return as_f(as_i(x) | as_i(y)); }); break;
      case MK_EW_XOR_B32: each([](float x, float y) { return as_f(as_i(x) ^ as_i(y)); }); break;
      case MK_EW_PRED_TO_S32: each([](float x, float) { return as_f(x != 0.f ? 1 : 0); }); break;
      case MK_EW_S32_TO_PRED: each([](float x, float) { return as_i(x) != 0 ? 1.f : 0.f; }); break;
      case MK_EW_U32_TO_F32: each([](float x, float) { return float(uint32_t(as_i(x))); }); break;
      default: each([](float, float) { return 0.f; }); break;
    }
#pragma unroll
    for (int e = 0; e < W; ++e) r[e][dst] = o[e];
  }
}

// The whole program block travels as a by-value kernel argument (< 2 KiB),
// so a launch needs no device-side staging buffer.
// One element per thread.  IdxT = int32_t when n and every input offset
// fit 31 bits (the index decomposition is then 32-bit division), int64_t
// otherwise.
template <typename IdxT>
__global__ __launch_bounds__(kBlock) void ew_program_kernel(const EwArgs A, int64_t n) {
  const int64_t i64 = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  if (i64 >= n) return;
  const IdxT i = IdxT(i64);
  float reg[kEwMaxRegs];
  float* const r[1] = {reg};
#pragma unroll
  for (int k = 0; k < kEwMaxRegs; ++k) r[0][k] = 0.f;
  const int rank = A.rank;
  IdxT idx[kEwMaxRank];
  if (A.need_index) {
    IdxT rem = i;
    for (int d = rank - 1; d >= 0; --d) {
      const IdxT n_d = IdxT(A.dims[d]);
      idx[d] = rem % n_d;
      rem /= n_d;
    }
  }
  for (int t = 0; t < A.n_inputs; ++t) {
    IdxT off = 0;
    if (A.in_mode[t] == 1) {
      off = i;
    } else if (A.in_mode[t] == 2) {
      for (int d = 0; d < rank; ++d) off += idx[d] * IdxT(A.in_stride[t][d]);
    }
    r[0][t] = ew_load(A.in[t], int64_t(off), A.in_type[t]);
  }
  ew_run<1, kEwMaxRegs>(A, r);
  for (int k = 0; k < A.n_out; ++k) ew_store(A.out[k], i64, A.out_type[k], r[0][A.out_reg[k]]);
}

// The same program on kEwVec consecutive elements of the innermost dim per
// thread (the host uses it when that dim is a multiple of kEwVec and every
// index and input offset fits 32 bits): the multi-dim index is decomposed
// once per thread in 32-bit arithmetic, and the inputs of all kEwVec
// elements are loaded before the program runs on the first of them.
constexpr int kEwVec = 4;
template <int NR>
__global__ __launch_bounds__(kBlock) void ew_program_vec_kernel(const EwArgs A, uint32_t n) {
  const uint32_t i0 = (blockIdx.x * uint32_t(kBlock) + threadIdx.x) * kEwVec;
  if (i0 >= n) return;
  uint32_t idx[kEwMaxRank];
  if (A.need_index) {
    // loops over the maximum rank with static indices keep idx in registers
    uint32_t rem = i0;
#pragma unroll
    for (int d = kEwMaxRank - 1; d >= 0; --d) {
      if (d < A.rank) {
        const uint32_t n_d = uint32_t(A.dims[d]);
        idx[d] = rem % n_d;
        rem /= n_d;
      }
    }
  }
  float reg0[NR], reg1[NR], reg2[NR], reg3[NR];
  float* const r[kEwVec] = {reg0, reg1, reg2, reg3};
#pragma unroll
  for (int e = 0; e < kEwVec; ++e)
#pragma unroll
    for (int k = 0; k < NR; ++k) r[e][k] = 0.f;
#pragma unroll
  for (int t = 0; t < kEwMaxInputs; ++t) {
    if (t >= A.n_inputs) break;
    int32_t off = 0, step = 0;
    if (A.in_mode[t] == 1) {
      off = int32_t(i0);
      step = 1;
    } else if (A.in_mode[t] == 2) {
#pragma unroll
      for (int d = 0; d < kEwMaxRank; ++d)
        if (d < A.rank) off += int32_t(idx[d]) * int32_t(A.in_stride[t][d]);
      step = int32_t(A.in_stride[t][A.rank - 1]);
    }
    if (A.in_vec[t] && A.in_type[t] == MK_F32) {
      const f32x4 w = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(A.in[t]) + off);
#pragma unroll
      for (int e = 0; e < kEwVec; ++e) r[e][t] = w.v[e];
    } else if (A.in_vec[t]) {  // bf16
      const uint2 w = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(A.in[t]) + off);
      r[0][t] = bf16_to_f32(uint16_t(w.x));
      r[1][t] = bf16_to_f32(uint16_t(w.x >> 16));
      r[2][t] = bf16_to_f32(uint16_t(w.y));
      r[3][t] = bf16_to_f32(uint16_t(w.y >> 16));
    } else {
#pragma unroll
      for (int e = 0; e < kEwVec; ++e) r[e][t] = ew_load(A.in[t], off + e * step, A.in_type[t]);
    }
  }
  // the program runs once on 4-lane registers
  ew_run<kEwVec, NR>(A, r);
  for (int k = 0; k < A.n_out; ++k) {
    float o[kEwVec];
#pragma unroll
    for (int e = 0; e < kEwVec; ++e) o[e] = r[e][A.out_reg[k] & (NR - 1)];
    void* out = A.out[k];
    if (A.out_vec[k] && A.out_type[k] == MK_F32) {
      *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(out) + i0) = f32x4{{o[0], o[1], o[2], o[3]}};
    } else if (A.out_vec[k]) {  // bf16
      *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(out) + i0) =
          uint2{f32_to_bf16(o[0]) | (uint32_t(f32_to_bf16(o[1])) << 16),
                f32_to_bf16(o[2]) | (uint32_t(f32_to_bf16(o[3])) << 16)};
    } else {
#pragma unroll
      for (int e = 0; e < kEwVec; ++e) ew_store(out, int64_t(i0) + e, A.out_type[k], o[e]);
    }
  }
}

// ------------------------------------------------------------------ convert / fill / iota
__global__ __launch_bounds__(kBlock) void convert_kernel(const void* __restrict__ in, int in_type,
                                                         void* __restrict__ out, int out_type,
                                                         int64_t n) {
  const int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  if (i >= n) return;
  const bool in_int = in_type == MK_S8 || in_type == MK_S16 || in_type == MK_S32 ||
                      in_type == MK_S64 || in_type == MK_U8 || in_type == MK_U16 ||
                      in_type == MK_U32 || in_type == MK_U64 || in_type == MK_PRED;
  const bool out_int = out_type == MK_S8 || out_type == MK_S16 || out_type == MK_S32 ||
                       out_type == MK_S64 || out_type == MK_U8 || out_type == MK_U16 ||
                       out_type == MK_U32 || out_type == MK_U64;
  if (in_int && out_int) {
    int64_t v;
    switch (in_type) {
      case MK_S8: v = reinterpret_cast<const int8_t*>(in)[i]; break;
      case MK_S16: v = reinterpret_cast<const int16_t*>(in)[i]; break;
      case MK_S32: v = reinterpret_cast<const int32_t*>(in)[i]; break;
      case MK_S64: v = reinterpret_cast<const int64_t*>(in)[i]; break;
      case MK_U8: case MK_PRED: v = reinterpret_cast<const uint8_t*>(in)[i]; break;
      case MK_U16: v = reinterpret_cast<const uint16_t*>(in)[i]; break;
      case MK_U32: v = reinterpret_cast<const uint32_t*>(in)[i]; break;
      default: v = int64_t(reinterpret_cast<const uint64_t*>(in)[i]); break;
    }
    switch (out_type) {
      case MK_S8: reinterpret_cast<int8_t*>(out)[i] = int8_t(v); break;
      case MK_S16: reinterpret_cast<int16_t*>(out)[i] = int16_t(v); break;
      case MK_S32: reinterpret_cast<int32_t*>(out)[i] = int32_t(v); break;
      case MK_S64: reinterpret_cast<int64_t*>(out)[i] = v; break;
      case MK_U8: reinterpret_cast<uint8_t*>(out)[i] = uint8_t(v); break;
      case MK_U16: reinterpret_cast<uint16_t*>(out)[i] = uint16_t(v); break;
      case MK_U32: reinterpret_cast<uint32_t*>(out)[i] = uint32_t(v); break;
      default: reinterpret_cast<uint64_t*>(out)[i] = uint64_t(v); break;
    }
    return;
  }
  if (out_type == MK_PRED) {
    reinterpret_cast<uint8_t*>(out)[i] = load_as_f32(in, i, in_type) != 0.f;
    return;
  }
  if (in_type == MK_F64 && out_type == MK_F32) {
    reinterpret_cast<float*>(out)[i] = float(reinterpret_cast<const double*>(in)[i]);
    return;
  }
  if (out_type == MK_F64) {
    reinterpret_cast<double*>(out)[i] = in_type == MK_F64 ? reinterpret_cast<const double*>(in)[i]
                                                          : double(load_as_f32(in, i, in_type));
    return;
  }
  store_from_f32(out, i, out_type, load_as_f32(in, i, in_type));
}

template <typename W>
__global__ __launch_bounds__(kBlock) void fill_kernel(W* __restrict__ out, W v, int64_t n) {
  const int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  if (i < n) out[i] = v;
}

__global__ __launch_bounds__(kBlock) void iota_kernel(void* __restrict__ out, int out_type, int64_t n,
                                                      int64_t inner, int64_t dim_size) {
  const int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  if (i >= n) return;
  const int64_t c = (i / inner) % dim_size;
  switch (out_type) {
    case MK_S32: reinterpret_cast<int32_t*>(out)[i] = int32_t(c); break;
    case MK_U32: reinterpret_cast<uint32_t*>(out)[i] = uint32_t(c); break;
    case MK_S64: reinterpret_cast<int64_t*>(out)[i] = c; break;
    default: store_from_f32(out, i, out_type, float(c)); break;
  }
}

struct CopyArgs {
  int64_t dims[kEwMaxRank];
  int64_t strides[kEwMaxRank];
  int rank;
};

template <typename W>
__global__ __launch_bounds__(kBlock) void copy_strided_kernel(const W* __restrict__ in,
                                                              W* __restrict__ out, int64_t n,
                                                              CopyArgs a) {
  const int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  if (i >= n) return;
  int64_t rem = i, off = 0;
  for (int d = a.rank - 1; d >= 0; --d) {
    const int64_t q = rem / a.dims[d];
    off += (rem - q * a.dims[d]) * a.strides[d];
    rem = q;
  }
  out[i] = in[off];
}

inline unsigned blocks_for(int64_t n, int per_block) {
  return unsigned((n + per_block - 1) / per_block);
}

}  // namespace
}  // namespace mk

using namespace mk;

extern "C" int mk_gelu_tanh(void* stream, int io_type, int64_t n, const void* x, void* y) {
  clear_error();
  if (n < 0) return fail(MK_ERR_INVALID, "mk_gelu_tanh: negative n");
  if (n == 0) return MK_OK;
  if (!x || !y) return fail(MK_ERR_INVALID, "mk_gelu_tanh: null pointer");
  hipStream_t s = as_stream(stream);
  const bool al = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 15u) == 0;
  if (io_type == MK_BF16 || io_type == MK_F32) {
    const int N = io_type == MK_BF16 ? 8 : 4;
    const int64_t nvec = al ? n / N : 0;
    if (nvec > 0) {
      dim3 g(blocks_for(nvec, kBlock * kUnroll));
      if (io_type == MK_BF16)
        hipLaunchKernelGGL(gelu_vec_kernel<uint16_t>, g, dim3(kBlock), 0, s, (const uint16_t*)x, (uint16_t*)y, nvec);
      else
        hipLaunchKernelGGL(gelu_vec_kernel<float>, g, dim3(kBlock), 0, s, (const float*)x, (float*)y, nvec);
    }
    const int64_t begin = nvec * N;
    if (begin < n) {
      dim3 g(blocks_for(n - begin, kBlock));
      if (io_type == MK_BF16)
        hipLaunchKernelGGL(gelu_scalar_kernel<uint16_t>, g, dim3(kBlock), 0, s, (const uint16_t*)x, (uint16_t*)y, begin, n);
      else
        hipLaunchKernelGGL(gelu_scalar_kernel<float>, g, dim3(kBlock), 0, s, (const float*)x, (float*)y, begin, n);
    }
    return check_launch("mk_gelu_tanh");
  }
  return fail(MK_ERR_UNSUPPORTED, "mk_gelu_tanh: io_type must be bf16/f32");
}

extern "C" int mk_ew_program_multi(void* stream, int rank, const int64_t* dims, int n_inputs,
                                   const void* const* inputs, const int* in_types,
                                   const int64_t* in_strides, int n_instr, const int32_t* program,
                                   const float* consts, int n_consts, int n_outputs, const int* out_regs,
                                   const int* out_types, void* const* outs) {
  clear_error();
  if (rank < 0 || rank > kEwMaxRank) return fail(MK_ERR_INVALID, "mk_ew_program: rank > 6");
  if (n_outputs < 1 || n_outputs > kEwMaxOutputs) return fail(MK_ERR_INVALID, "mk_ew_program: 1 to 4 outputs");
  if (n_inputs < 0 || n_inputs > kEwMaxInputs) return fail(MK_ERR_INVALID, "mk_ew_program: > 8 inputs");
  if (n_instr < 0 || n_instr > kEwMaxInstr) return fail(MK_ERR_INVALID, "mk_ew_program: > 64 instructions");
  if (n_consts < 0 || n_consts > kEwMaxConsts) return fail(MK_ERR_INVALID, "mk_ew_program: > 64 constants");
  for (int k = 0; k < n_outputs; ++k) {
    if (out_regs[k] < 0 || out_regs[k] >= kEwMaxRegs) return fail(MK_ERR_INVALID, "mk_ew_program: bad out_reg");
    if (dtype_bytes(out_types[k]) == 0) return fail(MK_ERR_UNSUPPORTED, "mk_ew_program: bad output dtype");
  }
  int64_t n = 1;
  for (int d = 0; d < rank; ++d) {
    if (dims[d] < 0) return fail(MK_ERR_INVALID, "mk_ew_program: negative dim");
    n *= dims[d];
  }
  if (n == 0) return MK_OK;
  EwArgs a{};
  a.rank = rank;
  a.n_inputs = n_inputs;
  a.n_instr = n_instr;
  a.n_out = n_outputs;
  for (int k = 0; k < n_outputs; ++k) {
    if (!outs[k]) return fail(MK_ERR_INVALID, "mk_ew_program: null output");
    a.out[k] = outs[k];
    a.out_reg[k] = out_regs[k];
    a.out_type[k] = out_types[k];
  }
  for (int d = 0; d < rank; ++d) a.dims[d] = dims[d];
  int need_index = 0;
  for (int t = 0; t < n_inputs; ++t) {
    if (!inputs[t]) return fail(MK_ERR_INVALID, "mk_ew_program: null input");
    a.in[t] = inputs[t];
    a.in_type[t] = in_types[t];
    if (dtype_bytes(in_types[t]) == 0) return fail(MK_ERR_UNSUPPORTED, "mk_ew_program: bad input dtype");
    int64_t expect = 1;
    bool is_dense = true, is_scalar = true;
    for (int d = rank - 1; d >= 0; --d) {
      const int64_t st = in_strides[t * kEwMaxRank + d];
      a.in_stride[t][d] = dims[d] == 1 ? 0 : st;  // size-1 dims never contribute
      if (dims[d] != 1 && st != expect) is_dense = false;
      if (dims[d] != 1 && st != 0) is_scalar = false;
      expect *= dims[d];
    }
    a.in_mode[t] = is_scalar ? 0 : (is_dense ? 1 : 2);
    need_index |= (a.in_mode[t] == 2);
  }
  // highest register the program names (inputs occupy 0 .. n_inputs - 1)
  int max_reg = n_inputs - 1;
  for (int k = 0; k < n_outputs; ++k) max_reg = max(max_reg, out_regs[k]);
  for (int p = 0; p < n_instr; ++p) {
    const int32_t* ins = program + 4 * p;
    if (ins[0] < 0 || ins[0] >= MK_EW_NUM_OPS) return fail(MK_ERR_INVALID, "mk_ew_program: bad opcode");
    if (ins[1] < 0 || ins[1] >= kEwMaxRegs) return fail(MK_ERR_INVALID, "mk_ew_program: bad dst register");
    if (ins[0] == MK_EW_CONST) {
      if (ins[2] < 0 || ins[2] >= n_consts) return fail(MK_ERR_INVALID, "mk_ew_program: bad constant index");
    } else {
      if (ins[2] < 0 || ins[2] >= kEwMaxRegs || (ins[3] & 0xffff) >= kEwMaxRegs ||
          ((ins[3] >> 16) & 0xffff) >= kEwMaxRegs)
        return fail(MK_ERR_INVALID, "mk_ew_program: bad source register");
      max_reg = max(max_reg, max(ins[2], max(ins[3] & 0xffff, (ins[3] >> 16) & 0xffff)));
    }
    max_reg = max(max_reg, ins[1]);
    for (int k = 0; k < 4; ++k) a.prog[p][k] = ins[k];
  }
  for (int c = 0; c < n_consts; ++c) a.consts[c] = consts[c];
  a.need_index = need_index;
  // 32-bit forms: n and every input's largest offset below 2^31; the vector
  // kernel also needs the innermost dim a multiple of kEwVec
  bool narrow = rank >= 1 && n < (int64_t(1) << 31);
  for (int t = 0; narrow && t < n_inputs; ++t) {
    int64_t hi = 0;
    for (int d = 0; d < rank; ++d) {
      const int64_t st = a.in_stride[t][d];
      if (st < 0) narrow = false;
      hi += (dims[d] - 1) * st;
    }
    narrow = narrow && hi < (int64_t(1) << 31) - kEwVec;
  }
  if (narrow) {
    // vector accesses: f32 / bf16 data whose 4 consecutive elements are
    // adjacent (unit innermost stride) and aligned (base aligned, every other
    // stride a multiple of 4 elements)
    auto vec_ok = [&](const void* base, int type, const int64_t* st) {
      const int w = type == MK_F32 ? 4 : type == MK_BF16 ? 2 : 0;
      if (w == 0 || (reinterpret_cast<uintptr_t>(base) & uintptr_t(4 * w - 1)) != 0) return false;
      if (st[rank - 1] != 1) return false;
      for (int d = 0; d + 1 < rank; ++d)
        if (st[d] % kEwVec != 0) return false;
      return true;
    };
    for (int t = 0; t < n_inputs; ++t) a.in_vec[t] = a.in_mode[t] != 0 && vec_ok(a.in[t], a.in_type[t], a.in_stride[t]);
    int64_t dense[kEwMaxRank];
    int64_t acc = 1;
    for (int d = rank - 1; d >= 0; --d) {
      dense[d] = acc;
      acc *= dims[d];
    }
    for (int k = 0; k < n_outputs; ++k) a.out_vec[k] = vec_ok(outs[k], out_types[k], dense);
  }
  // the vector kernel with 16 registers per lane when the program fits (64
  // VGPRs of registers instead of 128: more waves per SIMD)
  if (narrow && dims[rank - 1] % kEwVec == 0 && max_reg < 16)
    hipLaunchKernelGGL(ew_program_vec_kernel<16>, dim3(blocks_for(n / kEwVec, kBlock)), dim3(kBlock), 0,
                       as_stream(stream), a, uint32_t(n));
  else if (narrow && dims[rank - 1] % kEwVec == 0)
    hipLaunchKernelGGL(ew_program_vec_kernel<kEwMaxRegs>, dim3(blocks_for(n / kEwVec, kBlock)), dim3(kBlock), 0,
                       as_stream(stream), a, uint32_t(n));
  else if (narrow)
    hipLaunchKernelGGL(ew_program_kernel<int32_t>, dim3(blocks_for(n, kBlock)), dim3(kBlock), 0,
                       as_stream(stream), a, n);
  else
    hipLaunchKernelGGL(ew_program_kernel<int64_t>, dim3(blocks_for(n, kBlock)), dim3(kBlock), 0,
                       as_stream(stream), a, n);
  return check_launch("mk_ew_program");
}

extern "C" int mk_ew_program(void* stream, int rank, const int64_t* dims, int n_inputs,
                             const void* const* inputs, const int* in_types,
                             const int64_t* in_strides, int n_instr, const int32_t* program,
                             const float* consts, int n_consts, int out_reg, int out_type,
                             void* out) {
  return mk_ew_program_multi(stream, rank, dims, n_inputs, inputs, in_types, in_strides, n_instr, program, consts,
                             n_consts, 1, &out_reg, &out_type, &out);
}

extern "C" int mk_convert(void* stream, int in_type, int out_type, int64_t n, const void* in,
                          void* out) {
  clear_error();
  if (n < 0) return fail(MK_ERR_INVALID, "mk_convert: negative n");
  if (dtype_bytes(in_type) == 0 || dtype_bytes(out_type) == 0)
    return fail(MK_ERR_UNSUPPORTED, "mk_convert: unsupported dtype");
  if (n == 0) return MK_OK;
  if (!in || !out) return fail(MK_ERR_INVALID, "mk_convert: null pointer");
  hipLaunchKernelGGL(convert_kernel, dim3(blocks_for(n, kBlock)), dim3(kBlock), 0, as_stream(stream),
                     in, in_type, out, out_type, n);
  return check_launch("mk_convert");
}

extern "C" int mk_fill(void* stream, int elem_bytes, int64_t n, uint64_t pattern, void* out) {
  clear_error();
  if (n < 0) return fail(MK_ERR_INVALID, "mk_fill: negative n");
  if (n == 0) return MK_OK;
  if (!out) return fail(MK_ERR_INVALID, "mk_fill: null pointer");
  hipStream_t s = as_stream(stream);
  dim3 g(blocks_for(n, kBlock)), b(kBlock);
  switch (elem_bytes) {
    case 1: hipLaunchKernelGGL(fill_kernel<uint8_t>, g, b, 0, s, (uint8_t*)out, uint8_t(pattern), n); break;
    case 2: hipLaunchKernelGGL(fill_kernel<uint16_t>, g, b, 0, s, (uint16_t*)out, uint16_t(pattern), n); break;
    case 4: hipLaunchKernelGGL(fill_kernel<uint32_t>, g, b, 0, s, (uint32_t*)out, uint32_t(pattern), n); break;
    case 8: hipLaunchKernelGGL(fill_kernel<uint64_t>, g, b, 0, s, (uint64_t*)out, pattern, n); break;
    default: return fail(MK_ERR_INVALID, "mk_fill: elem_bytes must be 1, 2, 4 or 8");
  }
  return check_launch("mk_fill");
}

extern "C" int mk_iota(void* stream, int out_type, int rank, const int64_t* dims, int dim, void* out) {
  clear_error();
  if (rank < 1 || rank > kEwMaxRank || dim < 0 || dim >= rank)
    return fail(MK_ERR_INVALID, "mk_iota: need 1 <= rank <= 6 and 0 <= dim < rank");
  if (out_type != MK_S32 && out_type != MK_S64 && out_type != MK_F32 && out_type != MK_BF16 &&
      out_type != MK_U32 && out_type != MK_F16)
    return fail(MK_ERR_UNSUPPORTED, "mk_iota: unsupported out_type");
  int64_t n = 1, inner = 1;
  for (int d = 0; d < rank; ++d) {
    if (dims[d] < 0) return fail(MK_ERR_INVALID, "mk_iota: negative dim");
    n *= dims[d];
    if (d > dim) inner *= dims[d];
  }
  if (n == 0) return MK_OK;
  if (!out) return fail(MK_ERR_INVALID, "mk_iota: null pointer");
  hipLaunchKernelGGL(iota_kernel, dim3(blocks_for(n, kBlock)), dim3(kBlock), 0, as_stream(stream), out,
                     out_type, n, inner, dims[dim]);
  return check_launch("mk_iota");
}

extern "C" int mk_copy_strided(void* stream, int elem_bytes, int rank, const int64_t* dims,
                               const void* in, const int64_t* in_strides, void* out) {
  clear_error();
  if (rank < 0 || rank > kEwMaxRank) return fail(MK_ERR_INVALID, "mk_copy_strided: rank > 6");
  CopyArgs a{};
  a.rank = rank;
  int64_t n = 1;
  for (int d = 0; d < rank; ++d) {
    if (dims[d] < 0) return fail(MK_ERR_INVALID, "mk_copy_strided: negative dim");
    a.dims[d] = dims[d];
    a.strides[d] = in_strides[d];
    n *= dims[d];
  }
  if (n == 0) return MK_OK;
  if (!in || !out) return fail(MK_ERR_INVALID, "mk_copy_strided: null pointer");
  hipStream_t s = as_stream(stream);
  dim3 g(blocks_for(n, kBlock)), b(kBlock);
  switch (elem_bytes) {
    case 1: hipLaunchKernelGGL(copy_strided_kernel<uint8_t>, g, b, 0, s, (const uint8_t*)in, (uint8_t*)out, n, a); break;
    case 2: hipLaunchKernelGGL(copy_strided_kernel<uint16_t>, g, b, 0, s, (const uint16_t*)in, (uint16_t*)out, n, a); break;
    case 4: hipLaunchKernelGGL(copy_strided_kernel<uint32_t>, g, b, 0, s, (const uint32_t*)in, (uint32_t*)out, n, a); break;
    case 8: hipLaunchKernelGGL(copy_strided_kernel<uint64_t>, g, b, 0, s, (const uint64_t*)in, (uint64_t*)out, n, a); break;
    default: return fail(MK_ERR_INVALID, "mk_copy_strided: elem_bytes must be 1, 2, 4 or 8");
  }
  return check_launch("mk_copy_strided");
}
