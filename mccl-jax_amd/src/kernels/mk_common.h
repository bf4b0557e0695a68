// Shared device/host helpers for the gfx950 kernels behind include/mk_kernels.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "mk_kernels.h"

namespace mk {

// ---------------------------------------------------------------- errors
// Per-thread last-error string; entry points return an MK_* code and leave
// the human-readable reason here.
void set_error(const std::string& msg);
void clear_error();
int fail(int code, const std::string& msg);
// Checks hipGetLastError() after a launch; returns MK_OK or MK_ERR_LAUNCH.
int check_launch(const char* what);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// rocBLAS GEMM behind mk_gemm_blas (blas.hip), same operand convention.
int gemm_blas(hipStream_t stream, int ab_type, int c_type, int64_t batch, int64_t M, int64_t N, int64_t K,
              const void* A, int64_t a_bs, int64_t a_ms, int64_t a_ks, const void* B, int64_t b_bs, int64_t b_ks,
              int64_t b_ns, void* C, int64_t c_bs, int64_t c_ms, float alpha, float beta);

// C = sum of the splits dense M x N fp32 slices of W, added in slice order
// (blas.hip), then + bias (c_type, per column; epilogue 1) and max(., 0)
// (epilogue 2), stored as c_type (MK_F32, or MK_BF16 rounded once from the
// fp32 result); N and c_ms multiples of 4, W 16-byte and C 16- (fp32) or
// 8-byte (bf16) aligned.
int splitk_sum(hipStream_t s, const float* W, int64_t splits, int64_t M, int64_t N, void* C, int64_t c_ms,
               const char* what, int c_type = 0, const void* bias = nullptr, int epilogue = 0);

// Tiled bf16 GEMM for large products behind mk_gemm (gemm_tiled.hip), same
// operand convention; returns -1 without launching when the shape, strides or
// alignment do not fit it, else MK_OK or an MK_ERR_* code.  k_rem > 0: the
// last batch contracts over its first k_rem k only (the last, shorter slice
// of a split along K whose slices are K apart).  epilogue | kEpiGeluAux: Y
// (bf16, rows y_ms apart) also receives gelu_tanh of each stored C value
// (batch 1, bf16 or fp32 C whose rows take whole 16-byte chunks).
// epilogue | kEpiGeluBwd (bf16 C, batch 1): C = bf16(stored product *
// gelu_tanh'(Y)) with Y the bf16 pre-activations (rows y_ms apart), and
// colpart row r (N floats) = the column sums of rows 128 r .. 128 r + 127 of
// the stored C (ceil(M / 128) rows).
constexpr int kEpiGeluAux = 8;
constexpr int kEpiGeluBwd = 16;
int gemm_tiled(hipStream_t s, int c_type, int64_t batch, int64_t M, int64_t N, int64_t K, const void* A,
               int64_t a_bs, int64_t a_ms, int64_t a_ks, const void* B, int64_t b_bs, int64_t b_ks,
               int64_t b_ns, void* C, int64_t c_bs, int64_t c_ms, const void* bias, int epilogue,
               int64_t k_rem = 0, void* Y = nullptr, int64_t y_ms = 0, float* colpart = nullptr);

// Flash attention backward behind mk_sdpa_bwd for head_dim 64 / 128
// (attention_bwd.hip); workspace: the per-row statistics.
size_t sdpa_bwd_flash_workspace(int64_t B, int64_t H, int64_t Sq);
int sdpa_bwd_flash(hipStream_t s, int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D,
                   const void* q, int64_t q_bs, int64_t q_hs, int64_t q_ss,
                   const void* k, int64_t k_bs, int64_t k_hs, int64_t k_ss,
                   const void* v, int64_t v_bs, int64_t v_hs, int64_t v_ss,
                   const void* o, int64_t o_bs, int64_t o_hs, int64_t o_ss,
                   const void* dout, int64_t do_bs, int64_t do_hs, int64_t do_ss, const float* lse,
                   void* dq, int64_t dq_bs, int64_t dq_hs, int64_t dq_ss,
                   void* dk, int64_t dk_bs, int64_t dk_hs, int64_t dk_ss,
                   void* dv, int64_t dv_bs, int64_t dv_hs, int64_t dv_ss,
                   float scale, int causal, void* workspace);

// ---------------------------------------------------------------- dtypes
inline int dtype_bytes(int t) {
  switch (t) {
    case MK_PRED: case MK_S8: case MK_U8: return 1;
    case MK_S16: case MK_U16: case MK_F16: case MK_BF16: return 2;
    case MK_S32: case MK_U32: case MK_F32: return 4;
    case MK_S64: case MK_U64: case MK_F64: return 8;
    default: return 0;
  }
}

// ---------------------------------------------------------------- bf16 / f16
// bf16 is carried as raw uint16 bits.  Widening is exact; narrowing is
// round-to-nearest-even with NaN kept quiet (sign preserved).
__host__ __device__ inline float bf16_to_f32(uint16_t h) {
  uint32_t u = uint32_t(h) << 16;
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}
__host__ __device__ inline uint16_t f32_to_bf16_sw(float f) {
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}
// On gfx950 the fptrunc lowers to v_cvt_pk_bf16_f32 (hardware RNE), one
// instruction for two values; the host side uses the integer formulation.
__host__ __device__ inline uint16_t f32_to_bf16(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  __bf16 b = static_cast<__bf16>(f);
  uint16_t u;
  __builtin_memcpy(&u, &b, 2);
  return u;
#else
  return f32_to_bf16_sw(f);
#endif
}
__device__ inline float f16_to_f32(uint16_t h) {
  _Float16 v;
  __builtin_memcpy(&v, &h, 2);
  return float(v);
}
__device__ inline uint16_t f32_to_f16(float f) {
  _Float16 v = _Float16(f);  // RNE on AMDGPU (v_cvt_f16_f32)
  uint16_t h;
  __builtin_memcpy(&h, &v, 2);
  return h;
}

// Generic scalar load/store through an element type known at run time (used
// by the non-hot generic kernels only; hot kernels are templated).
__device__ inline float load_as_f32(const void* p, int64_t i, int t) {
  switch (t) {
    case MK_F32: return reinterpret_cast<const float*>(p)[i];
    case MK_BF16: return bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
    case MK_F16: return f16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
    case MK_S32: return float(reinterpret_cast<const int32_t*>(p)[i]);
    case MK_U32: return float(reinterpret_cast<const uint32_t*>(p)[i]);
    case MK_S64: return float(reinterpret_cast<const int64_t*>(p)[i]);
    case MK_U64: return float(reinterpret_cast<const uint64_t*>(p)[i]);
    case MK_S8: return float(reinterpret_cast<const int8_t*>(p)[i]);
    case MK_U8: case MK_PRED: return float(reinterpret_cast<const uint8_t*>(p)[i]);
    case MK_S16: return float(reinterpret_cast<const int16_t*>(p)[i]);
    case MK_U16: return float(reinterpret_cast<const uint16_t*>(p)[i]);
    case MK_F64: return float(reinterpret_cast<const double*>(p)[i]);
    default: return 0.f;
  }
}
__device__ inline void store_from_f32(void* p, int64_t i, int t, float v) {
  switch (t) {
    case MK_F32: reinterpret_cast<float*>(p)[i] = v; break;
    case MK_BF16: reinterpret_cast<uint16_t*>(p)[i] = f32_to_bf16(v); break;
    case MK_F16: reinterpret_cast<uint16_t*>(p)[i] = f32_to_f16(v); break;
    case MK_S32: reinterpret_cast<int32_t*>(p)[i] = int32_t(v); break;
    case MK_U32: reinterpret_cast<uint32_t*>(p)[i] = uint32_t(v); break;
    case MK_S64: reinterpret_cast<int64_t*>(p)[i] = int64_t(v); break;
    case MK_U64: reinterpret_cast<uint64_t*>(p)[i] = uint64_t(v); break;
    case MK_S8: reinterpret_cast<int8_t*>(p)[i] = int8_t(v); break;
    case MK_U8: reinterpret_cast<uint8_t*>(p)[i] = uint8_t(v); break;
    case MK_PRED: reinterpret_cast<uint8_t*>(p)[i] = uint8_t(v != 0.f); break;
    case MK_S16: reinterpret_cast<int16_t*>(p)[i] = int16_t(v); break;
    case MK_U16: reinterpret_cast<uint16_t*>(p)[i] = uint16_t(v); break;
    case MK_F64: reinterpret_cast<double*>(p)[i] = double(v); break;
    default: break;
  }
}

// ---------------------------------------------------------------- GELU
// gelu_tanh(x) = 0.5 x (1 + tanh(u)), u = sqrt(2/pi) (x + 0.044715 x^3),
// written as x / (1 + exp(-2u)) with exp2; shared by every kernel that
// evaluates it, so fused and unfused paths give the same bits.
__device__ inline float gelu_tanh_f32(float x) {
  constexpr float kC0 = -2.0f * 0.7978845608028654f * 1.4426950408889634f;
  constexpr float kC1 = kC0 * 0.044715f;
  const float t = x * fmaf(x * x, kC1, kC0);
  const float e = exp2f(t);
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

// gelu(x) = x * s, s = 1 / (1 + exp(-2u)), u = c (x + k x^3) (the forward's
// form); gelu'(x) = s + x s (1 - s) 2c (1 + 3k x^2).
__device__ inline float gelu_tanh_grad_f32(float x) {
  constexpr float kC = 0.7978845608028654f, kK = 0.044715f;
  constexpr float kC0 = -2.0f * kC * 1.4426950408889634f;
  const float x2 = x * x;
  const float e = exp2f(x * fmaf(x2, kC0 * kK, kC0));
  const float s = __builtin_amdgcn_rcpf(1.0f + e);
  return s * fmaf(x * (1.0f - s), (2.0f * kC) * fmaf(3.0f * kK, x2, 1.0f), 1.0f);
}

// ---------------------------------------------------------------- wave64
constexpr int kWave = 64;

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}
// The same sum through DPP lane moves instead of ds_bpermute round trips:
// xor 1 and xor 2 (quad_perm), then row_half_mirror and row_mirror (which
// act as xor 4 / xor 8 once the groups below them hold equal values), then
// the four 16-lane row totals read with v_readlane and added.  A fixed order
// (deterministic, though not the butterfly's), and a few VALU cycles per
// step instead of an LDS round trip.
__device__ inline float dpp_f(float v, int ctrl) {
  switch (ctrl) {  // the control word must be a constant
    case 0xB1: return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
    case 0x4E: return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
    case 0x141: return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
    default: return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
  }
}
__device__ inline float wave_sum_dpp(float v) {
  v += dpp_f(v, 0xB1);   // quad_perm [1,0,3,2]
  v += dpp_f(v, 0x4E);   // quad_perm [2,3,0,1]
  v += dpp_f(v, 0x141);  // row_half_mirror
  v += dpp_f(v, 0x140);  // row_mirror
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return (r0 + r1) + (r2 + r3);
}
__device__ inline float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, kWave));
  return v;
}
__device__ inline float wave_min(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fminf(v, __shfl_xor(v, m, kWave));
  return v;
}
__device__ inline float wave_prod(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v *= __shfl_xor(v, m, kWave);
  return v;
}

// 16-byte vector of 8 bf16 / 4 fp32 lanes for dwordx4 global traffic.
struct alignas(16) u16x8 { uint16_t v[8]; };
struct alignas(16) f32x4 { float v[4]; };

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));  // converting f32x2_t to it is v_cvt_pk_bf16_f32 (RNE)

// Streaming (non-temporal) 16-byte load/store: data touched once should not
// evict the L2 working set of other kernels.
template <typename V>
__device__ inline V ld_stream(const V* p) {
  static_assert(sizeof(V) == 16, "16-byte vectors only");
  u32x4_t r = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  V v;
  __builtin_memcpy(&v, &r, 16);
  return v;
}
template <typename V>
__device__ inline void st_stream(V* p, const V& v) {
  static_assert(sizeof(V) == 16, "16-byte vectors only");
  u32x4_t r;
  __builtin_memcpy(&r, &v, 16);
  __builtin_nontemporal_store(r, reinterpret_cast<u32x4_t*>(p));
}

}  // namespace mk
