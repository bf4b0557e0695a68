// Row-wise reductions over the innermost axis: reduce (sum/max/min/prod),
// fused max+argmax (bit-exact), LayerNorm and softmax.
//
// Layout: x is [rows, cols] row-major.  One wave64 owns one row; each lane
// reads 16-byte vectors (8 bf16 / 4 fp32) so a 2 KiB bf16 row is exactly two
// dwordx4 loads per lane and every HBM line is fully used.  Cross-lane
// combination is a 6-step butterfly.  Rows never interact, so the grid is
// rows/4 workgroups of 4 waves — tens of thousands of waves for the C2
// shapes, enough to keep all 256 CUs streaming.
#include "mk_common.h"

#include <algorithm>
#include <type_traits>
#include <cmath>

namespace mk {
namespace {

constexpr int kWavesPerBlock = 4;
constexpr int kBlock = kWavesPerBlock * kWave;

template <typename T> struct Vec;
template <> struct Vec<uint16_t> { static constexpr int N = 8; using V = u16x8; };
template <> struct Vec<float> { static constexpr int N = 4; using V = f32x4; };

template <typename T> __device__ inline float to_f32(T v);
template <> __device__ inline float to_f32<float>(float v) { return v; }
template <> __device__ inline float to_f32<uint16_t>(uint16_t v) { return bf16_to_f32(v); }

// Input element types handled by the templated row kernels: bf16 (uint16_t
// bits, IS_F16=false), f16 (uint16_t bits, IS_F16=true) and f32.
template <typename T, bool IS_F16>
__device__ inline float ld(T v) {
  if constexpr (IS_F16) return f16_to_f32(v);
  else return to_f32<T>(v);
}

template <int OP> __device__ inline float combine(float a, float b) {
  if constexpr (OP == 0) return a + b;
  else if constexpr (OP == 1) return fmaxf(a, b);
  else if constexpr (OP == 2) return fminf(a, b);
  else return a * b;
}
template <int OP> __device__ inline float wave_combine(float v) {
  if constexpr (OP == 0) return wave_sum(v);
  else if constexpr (OP == 1) return wave_max(v);
  else if constexpr (OP == 2) return wave_min(v);
  else return wave_prod(v);
}
template <int OP> __device__ inline float identity() {
  if constexpr (OP == 0) return 0.f;
  else if constexpr (OP == 1) return -INFINITY;
  else if constexpr (OP == 2) return INFINITY;
  else return 1.f;
}

// StableHLO max/min propagate NaN; fmaxf/fminf drop it, so NaN is tracked
// separately for OP 1/2.
template <typename T, bool IS_F16, int OP>
__global__ __launch_bounds__(kBlock) void row_reduce_kernel(const T* __restrict__ x, int64_t rows,
                                                            int64_t cols, float init, void* y,
                                                            int out_type, bool vec_ok) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = int64_t(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * cols;
  float acc = identity<OP>();
  bool nan = false;
  constexpr int N = Vec<T>::N;
  if (vec_ok) {
    using V = typename Vec<T>::V;
    const V* xv = reinterpret_cast<const V*>(xr);
    const int64_t nv = cols / N;
    int64_t i = lane;
    // two vectors in flight per iteration
    for (; i + kWave < nv; i += 2 * kWave) {
      V a = xv[i], b = xv[i + kWave];
#pragma unroll
      for (int j = 0; j < N; ++j) {
        float fa = ld<T, IS_F16>(a.v[j]);
        nan |= (fa != fa);
        acc = combine<OP>(acc, fa);
      }
#pragma unroll
      for (int j = 0; j < N; ++j) {
        float fb = ld<T, IS_F16>(b.v[j]);
        nan |= (fb != fb);
        acc = combine<OP>(acc, fb);
      }
    }
    for (; i < nv; i += kWave) {
      V a = xv[i];
#pragma unroll
      for (int j = 0; j < N; ++j) {
        float fa = ld<T, IS_F16>(a.v[j]);
        nan |= (fa != fa);
        acc = combine<OP>(acc, fa);
      }
    }
  } else {
    for (int64_t c = lane; c < cols; c += kWave) {
      float f = ld<T, IS_F16>(xr[c]);
      nan |= (f != f);
      acc = combine<OP>(acc, f);
    }
  }
  acc = wave_combine<OP>(acc);
  // the vote must run with the whole wave active, before the lane-0 branch
  const bool any_nan = __any(nan);
  if (lane == 0) {
    float r = combine<OP>(acc, init);
    if constexpr (OP == 1 || OP == 2) {
      if (any_nan || init != init) r = __builtin_nanf("");
    }
    store_from_f32(y, row, out_type, r);
  }
}

// (value, index) pair compare for argmax/argmin with XLA semantics.
template <bool IS_MIN>
__device__ inline bool better(float a, int64_t ia, float b, int64_t ib) {
  const bool an = a != a, bn = b != b;
  if (an || bn) {
    if (an && bn) return ia < ib;
    return an;
  }
  if (a == b) return ia < ib;
  return IS_MIN ? (a < b) : (a > b);
}

template <typename T> __device__ inline uint32_t raw_bits(T v) {
  if constexpr (sizeof(T) == 4) {
    uint32_t u;
    __builtin_memcpy(&u, &v, 4);
    return u;
  } else {
    return uint32_t(v);
  }
}
template <typename T> __device__ inline T from_bits(uint32_t u) {
  if constexpr (sizeof(T) == 4) {
    T v;
    __builtin_memcpy(&v, &u, 4);
    return v;
  } else {
    return T(u);
  }
}

template <typename T, bool IS_F16, bool IS_MIN, typename IdxT>
__global__ __launch_bounds__(kBlock) void row_argmax_kernel(const T* __restrict__ x, int64_t rows,
                                                            int64_t cols, T* __restrict__ values,
                                                            IdxT* __restrict__ indices, bool vec_ok) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = int64_t(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * cols;
  float best = 0.f;
  int64_t bi = INT64_MAX;  // "no element yet": loses to any real element
  uint32_t braw = 0;
  constexpr int N = Vec<T>::N;
  // Elements are visited in increasing index within a lane, so only a
  // strictly better element may replace the current one.
  auto consider = [&](T raw, int64_t idx) {
    float f = ld<T, IS_F16>(raw);
    if (bi == INT64_MAX || better<IS_MIN>(f, idx, best, bi)) {
      best = f;
      bi = idx;
      braw = raw_bits<T>(raw);
    }
  };
  if (vec_ok) {
    using V = typename Vec<T>::V;
    const V* xv = reinterpret_cast<const V*>(xr);
    const int64_t nv = cols / N;
    int64_t i = lane;
    for (; i + kWave < nv; i += 2 * kWave) {
      V a = xv[i], b = xv[i + kWave];
#pragma unroll
      for (int j = 0; j < N; ++j) consider(a.v[j], i * N + j);
#pragma unroll
      for (int j = 0; j < N; ++j) consider(b.v[j], (i + kWave) * N + j);
    }
    for (; i < nv; i += kWave) {
      V a = xv[i];
#pragma unroll
      for (int j = 0; j < N; ++j) consider(a.v[j], i * N + j);
    }
  } else {
    for (int64_t c = lane; c < cols; c += kWave) consider(xr[c], c);
  }
  // butterfly: every lane ends with the row winner
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float ob = __shfl_xor(best, m, kWave);
    const int64_t oi = __shfl_xor(bi, m, kWave);
    const uint32_t oraw = __shfl_xor(braw, m, kWave);
    if (oi != INT64_MAX && (bi == INT64_MAX || better<IS_MIN>(ob, oi, best, bi))) {
      best = ob;
      bi = oi;
      braw = oraw;
    }
  }
  if (lane == 0) {
    if (values) values[row] = from_bits<T>(braw);
    indices[row] = IdxT(bi == INT64_MAX ? 0 : bi);
  }
}

// Argmax / argmin of 16-bit floats (bf16, f16) with a row of at most 65536
// elements: each element becomes the 32-bit word (key << 16) | (0xFFFF - i),
// where key orders the values as the XLA reducer does (larger value wins for
// argmax, smaller for argmin, every NaN beats every number, -0 == +0), so
// the row winner -- ties going to the lower index -- is the unsigned max of
// the words.  Two elements are keyed at once with packed 16-bit integer ops.
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));

template <bool IS_MIN, uint32_t INF>
__device__ inline uint32_t order_keys(uint32_t w) {
  constexpr unsigned short kNan = INF + 1;  // smallest NaN magnitude
  const u16x2_t mag = __builtin_bit_cast(u16x2_t, w & 0x7FFF7FFFu);
  const u16x2_t magc = __builtin_elementwise_min(mag, u16x2_t{kNan, kNan});  // NaN -> kNan
  // bit 15 of mag + (0x8000 - kNan) is set exactly for NaN halves
  const uint32_t nanb =
      __builtin_bit_cast(uint32_t, mag + u16x2_t{0x8000 - kNan, 0x8000 - kNan}) & 0x80008000u;
  const uint32_t sgn = w & 0x80008000u;
  // halves whose key is 0x8000 - magnitude: negative numbers for argmax,
  // positive numbers for argmin; the other halves (NaN included) take
  // 0x8000 + magnitude
  const uint32_t low = IS_MIN ? (~(sgn | nanb) & 0x80008000u) : (sgn & ~nanb);
  const uint32_t mask = (low >> 15) * 0xFFFFu;
  const uint32_t kp = __builtin_bit_cast(uint32_t, magc + u16x2_t{0x8000, 0x8000});
  const uint32_t kn = __builtin_bit_cast(uint32_t, u16x2_t{0x8000, 0x8000} - magc);
  return (mask & kn) | (~mask & kp);
}

template <bool IS_F16, bool IS_MIN, typename IdxT>
__global__ __launch_bounds__(kBlock) void row_argmax16_kernel(const uint16_t* __restrict__ x, int64_t rows,
                                                              int cols, uint16_t* __restrict__ values,
                                                              IdxT* __restrict__ indices) {
  constexpr uint32_t kInf = IS_F16 ? 0x7C00u : 0x7F80u;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = int64_t(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint16_t* xr = x + row * cols;
  const u32x4_t* xv = reinterpret_cast<const u32x4_t*>(xr);
  const int nv = cols / 8;
  uint32_t best = 0;  // below every element's word
#pragma unroll 2
  for (int i = lane; i < nv; i += kWave) {
    const u32x4_t a = xv[i];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t k = order_keys<IS_MIN, kInf>(a[j]);
      const uint32_t e = 0xFFFFu - uint32_t(8 * i + 2 * j);  // complement of the low half's index
      const uint32_t p0 = (k << 16) | e, p1 = (k & 0xFFFF0000u) | (e - 1u);
      best = max(best, max(p0, p1));
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) best = max(best, uint32_t(__shfl_xor(int(best), m, kWave)));
  if (lane == 0) {
    const int idx = int(0xFFFFu - (best & 0xFFFFu));
    if (values) values[row] = xr[idx];  // the winner's own bits (NaN payloads included)
    indices[row] = IdxT(idx);
  }
}

// LayerNorm: one wave per row, the whole row held in registers (up to
// kLnMaxPerLane fp32 per lane), two-pass mean/variance, single store.
constexpr int kLnMaxVecs = 8;  // 8 × 8 bf16 = 64 elements per lane → cols ≤ 4096 in registers

// TO: the stored type (T, or bf16 for fp32 rows: four values as one 8-byte
// store, y rows 8-byte aligned).  ADD (fp32 rows): the row is x + x2 (one
// fp32 add per element, the residual stream's update), stored to xsum and
// normalised.
template <typename T, typename TO = T, bool ADD = false>
__global__ __launch_bounds__(kBlock) void layernorm_reg_kernel(const T* __restrict__ x,
                                                               const T* __restrict__ gamma,
                                                               const T* __restrict__ beta,
                                                               int64_t rows, int cols, float eps,
                                                               TO* __restrict__ y, const T* __restrict__ x2 = nullptr,
                                                               T* __restrict__ xsum = nullptr) {
  using V = typename Vec<T>::V;
  constexpr int N = Vec<T>::N;
  static_assert(!ADD || sizeof(T) == 4, "the fused residual add is for fp32 rows");
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = int64_t(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int nv = cols / N;  // vectors per row; host guarantees nv ≤ kLnMaxVecs * 64
  const V* xv = reinterpret_cast<const V*>(x + row * int64_t(cols));
  float r[kLnMaxVecs][N];
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < kLnMaxVecs; ++k) {
    int i = lane + k * kWave;
    if (i < nv) {
      V a = xv[i];
      if constexpr (ADD) {
        const V b = reinterpret_cast<const V*>(x2 + row * int64_t(cols))[i];
#pragma unroll
        for (int j = 0; j < N; ++j) a.v[j] = a.v[j] + b.v[j];
        reinterpret_cast<V*>(xsum + row * int64_t(cols))[i] = a;
      }
#pragma unroll
      for (int j = 0; j < N; ++j) {
        r[k][j] = to_f32<T>(a.v[j]);
        s += r[k][j];
      }
    }
  }
  const float inv_n = 1.f / float(cols);
  const float mean = wave_sum(s) * inv_n;
  float q = 0.f;
#pragma unroll
  for (int k = 0; k < kLnMaxVecs; ++k) {
    if (lane + k * kWave < nv) {
#pragma unroll
      for (int j = 0; j < N; ++j) {
        float d = r[k][j] - mean;
        q += d * d;
      }
    }
  }
  const float var = wave_sum(q) * inv_n;
  const float rstd = 1.f / sqrtf(var + eps);
  const V* gv = reinterpret_cast<const V*>(gamma);
  const V* bv = reinterpret_cast<const V*>(beta);
  constexpr bool kNarrow = sizeof(TO) < sizeof(T);
  static_assert(!kNarrow || N == 4, "narrowing store: fp32 rows to bf16");
  using VO = std::conditional_t<kNarrow, uint2, V>;
  VO* yv = reinterpret_cast<VO*>(y + row * int64_t(cols));
#pragma unroll
  for (int k = 0; k < kLnMaxVecs; ++k) {
    int i = lane + k * kWave;
    if (i < nv) {
      V g{}, b{};
      float o[N];
      if (gamma) g = gv[i];
      if (beta) b = bv[i];
#pragma unroll
      for (int j = 0; j < N; ++j) {
        float gj = gamma ? to_f32<T>(g.v[j]) : 1.f;
        float bj = beta ? to_f32<T>(b.v[j]) : 0.f;
        o[j] = (r[k][j] - mean) * rstd * gj + bj;
      }
      if constexpr (kNarrow) {
        yv[i] = uint2{uint32_t(f32_to_bf16(o[0])) | (uint32_t(f32_to_bf16(o[1])) << 16),
                      uint32_t(f32_to_bf16(o[2])) | (uint32_t(f32_to_bf16(o[3])) << 16)};
      } else {
        V ov;
#pragma unroll
        for (int j = 0; j < N; ++j) {
          if constexpr (sizeof(T) == 2) ov.v[j] = f32_to_bf16(o[j]);
          else ov.v[j] = o[j];
        }
        yv[i] = ov;
      }
    }
  }
}

// bf16 -> fp32 widening of the low / high half of a packed word, spelled
// three ways (shift, byte permute, funnel shift).  The LayerNorm passes each
// use their own spelling, so the compiler cannot merge them into one widened
// copy of the row kept live across the passes: the row stays packed (8 bf16
// per 16-byte vector), fewer registers, more rows in flight.
__device__ inline float lo_a(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ inline float hi_a(uint32_t w) { return __builtin_bit_cast(float, w & 0xFFFF0000u); }
__device__ inline float lo_b(uint32_t w) { return __builtin_bit_cast(float, __builtin_amdgcn_perm(w, 0u, 0x05040C0Cu)); }
__device__ inline float hi_b(uint32_t w) { return __builtin_bit_cast(float, __builtin_amdgcn_perm(w, 0u, 0x07060C0Cu)); }
__device__ inline float lo_c(uint32_t w) { return __builtin_bit_cast(float, __builtin_amdgcn_alignbit(w, 0u, 16u)); }
__device__ inline float hi_c(uint32_t w) { return __builtin_bit_cast(float, __builtin_amdgcn_perm(0u, w, 0x03020C0Cu)); }

// LayerNorm for bf16 rows split over WPR waves of a 256-thread workgroup
// (4 / WPR rows per workgroup): lane t of the row's WPR*64 lanes holds the
// 16-byte vectors t, t + 64 WPR, ... (KV of them), so a row of 4096 needs
// 8 / WPR registers' worth of vectors per lane and many more waves fit on a
// CU than with a whole row per wave.  The two row sums are combined across
// the row's waves through LDS; mean and variance are two-pass as in
// layernorm_reg_kernel.  Rows past the end still take part in the barriers.
template <int WPR, int KV>
__global__ __launch_bounds__(kBlock) void layernorm_bf16_split_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ gamma, const uint16_t* __restrict__ beta,
    int64_t rows, int cols, float eps, uint16_t* __restrict__ y) {
  constexpr int RPB = kWavesPerBlock / WPR;  // rows per workgroup
  __shared__ float red[2][kWavesPerBlock];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const int rloc = wave / WPR, part = wave % WPR;
  const int64_t row = int64_t(blockIdx.x) * RPB + rloc;
  const bool live = row < rows;
  const int nv = cols / 8;
  const int t0 = part * kWave + lane;
  constexpr int kStride = WPR * kWave;
  const u32x4_t* xv = reinterpret_cast<const u32x4_t*>(x + (live ? row : 0) * cols);
  u32x4_t v[KV];
#pragma unroll
  for (int k = 0; k < KV; ++k)
    if (live && t0 + k * kStride < nv) v[k] = xv[t0 + k * kStride];
  const float inv_n = 1.f / float(cols);
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < KV; ++k)
    if (live && t0 + k * kStride < nv)
#pragma unroll
      for (int j = 0; j < 4; ++j) s += lo_a(v[k][j]) + hi_a(v[k][j]);
  s = wave_sum(s);
  if constexpr (WPR > 1) {
    if (lane == 0) red[0][wave] = s;
    __syncthreads();
    s = 0.f;
#pragma unroll
    for (int w = 0; w < WPR; ++w) s += red[0][rloc * WPR + w];
  }
  const float mean = s * inv_n;
  float q = 0.f;
#pragma unroll
  for (int k = 0; k < KV; ++k)
    if (live && t0 + k * kStride < nv)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float d0 = lo_b(v[k][j]) - mean, d1 = hi_b(v[k][j]) - mean;
        q += d0 * d0 + d1 * d1;
      }
  q = wave_sum(q);
  if constexpr (WPR > 1) {
    if (lane == 0) red[1][wave] = q;
    __syncthreads();
    q = 0.f;
#pragma unroll
    for (int w = 0; w < WPR; ++w) q += red[1][rloc * WPR + w];
  }
  if (!live) return;
  const float rstd = 1.f / sqrtf(q * inv_n + eps);
  u32x4_t* yv = reinterpret_cast<u32x4_t*>(y + row * cols);
#pragma unroll
  for (int k = 0; k < KV; ++k) {
    const int i = t0 + k * kStride;
    if (i < nv) {
      const u32x4_t one4 = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
      const u32x4_t gk = gamma ? reinterpret_cast<const u32x4_t*>(gamma)[i] : one4;
      const u32x4_t bk = beta ? reinterpret_cast<const u32x4_t*>(beta)[i] : u32x4_t{0u, 0u, 0u, 0u};
      u32x4_t o;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x2_t e = {(lo_c(v[k][j]) - mean) * rstd * lo_a(gk[j]) + lo_a(bk[j]),
                           (hi_c(v[k][j]) - mean) * rstd * hi_a(gk[j]) + hi_a(bk[j])};
        o[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector(e, bf16x2_t));
      }
      yv[i] = o;
    }
  }
}

// Fallback LayerNorm for any width: three streaming passes over the row.
// With x2 (fp32 rows): the row is x + x2, written to xsum first (the passes
// then read that row back; each lane reads only what it wrote).
template <typename T, typename TO = T>
__global__ __launch_bounds__(kBlock) void layernorm_loop_kernel(const T* __restrict__ x,
                                                                const T* __restrict__ gamma,
                                                                const T* __restrict__ beta,
                                                                int64_t rows, int64_t cols,
                                                                float eps, TO* __restrict__ y,
                                                                const T* x2 = nullptr, T* xsum = nullptr) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = int64_t(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * cols;
  if constexpr (sizeof(T) == 4) {
    if (x2) {
      for (int64_t c = lane; c < cols; c += kWave) xsum[row * cols + c] = xr[c] + x2[row * cols + c];
      xr = xsum + row * cols;
    }
  }
  float s = 0.f;
  for (int64_t c = lane; c < cols; c += kWave) s += to_f32<T>(xr[c]);
  const float mean = wave_sum(s) / float(cols);
  float q = 0.f;
  for (int64_t c = lane; c < cols; c += kWave) {
    float d = to_f32<T>(xr[c]) - mean;
    q += d * d;
  }
  const float rstd = 1.f / sqrtf(wave_sum(q) / float(cols) + eps);
  TO* yr = y + row * cols;
  for (int64_t c = lane; c < cols; c += kWave) {
    float gj = gamma ? to_f32<T>(gamma[c]) : 1.f;
    float bj = beta ? to_f32<T>(beta[c]) : 0.f;
    float v = (to_f32<T>(xr[c]) - mean) * rstd * gj + bj;
    if constexpr (sizeof(TO) == 2) yr[c] = f32_to_bf16(v);
    else yr[c] = v;
  }
}

// Softmax over a row: max pass, sum-of-exp pass, normalise pass.
template <typename T>
__global__ __launch_bounds__(kBlock) void softmax_kernel(const T* __restrict__ x, int64_t rows,
                                                         int64_t cols, T* __restrict__ y) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = int64_t(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * cols;
  float m = -INFINITY;
  for (int64_t c = lane; c < cols; c += kWave) m = fmaxf(m, to_f32<T>(xr[c]));
  m = wave_max(m);
  float s = 0.f;
  for (int64_t c = lane; c < cols; c += kWave) s += __expf(to_f32<T>(xr[c]) - m);
  s = wave_sum(s);
  const float inv = 1.f / s;
  T* yr = y + row * cols;
  for (int64_t c = lane; c < cols; c += kWave) {
    float v = __expf(to_f32<T>(xr[c]) - m) * inv;
    if constexpr (sizeof(T) == 2) yr[c] = f32_to_bf16(v);
    else yr[c] = v;
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline unsigned grid_for_rows(int64_t rows) {
  return unsigned((rows + kWavesPerBlock - 1) / kWavesPerBlock);
}

template <typename T, bool IS_F16>
int launch_reduce(hipStream_t s, int op, int64_t rows, int64_t cols, const void* x, float init,
                  void* y, int out_type) {
  const bool vec_ok = aligned16(x) && (cols % Vec<T>::N) == 0;
  const T* xp = reinterpret_cast<const T*>(x);
  dim3 g(grid_for_rows(rows)), b(kBlock);
  switch (op) {
    case 0: hipLaunchKernelGGL((row_reduce_kernel<T, IS_F16, 0>), g, b, 0, s, xp, rows, cols, init, y, out_type, vec_ok); break;
    case 1: hipLaunchKernelGGL((row_reduce_kernel<T, IS_F16, 1>), g, b, 0, s, xp, rows, cols, init, y, out_type, vec_ok); break;
    case 2: hipLaunchKernelGGL((row_reduce_kernel<T, IS_F16, 2>), g, b, 0, s, xp, rows, cols, init, y, out_type, vec_ok); break;
    case 3: hipLaunchKernelGGL((row_reduce_kernel<T, IS_F16, 3>), g, b, 0, s, xp, rows, cols, init, y, out_type, vec_ok); break;
    default: return fail(MK_ERR_INVALID, "mk_row_reduce: op must be 0..3");
  }
  return check_launch("mk_row_reduce");
}

template <typename T, bool IS_F16, bool IS_MIN>
int launch_argmax(hipStream_t s, int64_t rows, int64_t cols, const void* x, void* values,
                  int index_type, void* indices) {
  const bool vec_ok = aligned16(x) && (cols % Vec<T>::N) == 0;
  dim3 g(grid_for_rows(rows)), b(kBlock);
  const T* xp = reinterpret_cast<const T*>(x);
  T* vp = reinterpret_cast<T*>(values);
  if constexpr (sizeof(T) == 2) {
    if (vec_ok && cols <= 65536) {
      if (index_type == MK_S32)
        hipLaunchKernelGGL((row_argmax16_kernel<IS_F16, IS_MIN, int32_t>), g, b, 0, s, xp, rows, int(cols), vp,
                           reinterpret_cast<int32_t*>(indices));
      else
        hipLaunchKernelGGL((row_argmax16_kernel<IS_F16, IS_MIN, int64_t>), g, b, 0, s, xp, rows, int(cols), vp,
                           reinterpret_cast<int64_t*>(indices));
      return check_launch("mk_row_argmax");
    }
  }
  if (index_type == MK_S32)
    hipLaunchKernelGGL((row_argmax_kernel<T, IS_F16, IS_MIN, int32_t>), g, b, 0, s, xp, rows, cols,
                       vp, reinterpret_cast<int32_t*>(indices), vec_ok);
  else
    hipLaunchKernelGGL((row_argmax_kernel<T, IS_F16, IS_MIN, int64_t>), g, b, 0, s, xp, rows, cols,
                       vp, reinterpret_cast<int64_t*>(indices), vec_ok);
  return check_launch("mk_row_argmax");
}

}  // namespace
}  // namespace mk

using namespace mk;

extern "C" int mk_row_reduce(void* stream, int in_type, int out_type, int op, int64_t rows,
                             int64_t cols, const void* x, float init, void* y) {
  clear_error();
  if (rows < 0 || cols < 0) return fail(MK_ERR_INVALID, "mk_row_reduce: negative shape");
  if (out_type != MK_F32 && out_type != MK_BF16 && out_type != MK_F16)
    return fail(MK_ERR_UNSUPPORTED, "mk_row_reduce: out_type must be f32/bf16/f16");
  if (rows == 0) return MK_OK;
  if (!x || !y) return fail(MK_ERR_INVALID, "mk_row_reduce: null pointer");
  hipStream_t s = as_stream(stream);
  switch (in_type) {
    case MK_BF16: return launch_reduce<uint16_t, false>(s, op, rows, cols, x, init, y, out_type);
    case MK_F16: return launch_reduce<uint16_t, true>(s, op, rows, cols, x, init, y, out_type);
    case MK_F32: return launch_reduce<float, false>(s, op, rows, cols, x, init, y, out_type);
    default: return fail(MK_ERR_UNSUPPORTED, "mk_row_reduce: in_type must be bf16/f16/f32");
  }
}

extern "C" int mk_row_argmax(void* stream, int in_type, int is_min, int64_t rows, int64_t cols,
                             const void* x, void* values, int index_type, void* indices) {
  clear_error();
  if (rows < 0 || cols <= 0)
    return fail(MK_ERR_INVALID, "mk_row_argmax: need rows >= 0 and cols >= 1");
  if (index_type != MK_S32 && index_type != MK_S64)
    return fail(MK_ERR_UNSUPPORTED, "mk_row_argmax: index_type must be s32/s64");
  if (rows == 0) return MK_OK;
  if (!x || !indices) return fail(MK_ERR_INVALID, "mk_row_argmax: null pointer");
  hipStream_t s = as_stream(stream);
  switch (in_type) {
    case MK_BF16:
      return is_min ? launch_argmax<uint16_t, false, true>(s, rows, cols, x, values, index_type, indices)
                    : launch_argmax<uint16_t, false, false>(s, rows, cols, x, values, index_type, indices);
    case MK_F16:
      return is_min ? launch_argmax<uint16_t, true, true>(s, rows, cols, x, values, index_type, indices)
                    : launch_argmax<uint16_t, true, false>(s, rows, cols, x, values, index_type, indices);
    case MK_F32:
      return is_min ? launch_argmax<float, false, true>(s, rows, cols, x, values, index_type, indices)
                    : launch_argmax<float, false, false>(s, rows, cols, x, values, index_type, indices);
    default: return fail(MK_ERR_UNSUPPORTED, "mk_row_argmax: in_type must be bf16/f16/f32");
  }
}

extern "C" int mk_layernorm(void* stream, int io_type, int64_t rows, int64_t cols, const void* x,
                            const void* gamma, const void* beta, float eps, void* y) {
  clear_error();
  if (rows < 0 || cols <= 0) return fail(MK_ERR_INVALID, "mk_layernorm: bad shape");
  if (rows == 0) return MK_OK;
  if (!x || !y) return fail(MK_ERR_INVALID, "mk_layernorm: null pointer");
  hipStream_t s = as_stream(stream);
  dim3 g(grid_for_rows(rows)), b(kBlock);
  auto vec_ok = [&](int n) {
    return (cols % n) == 0 && cols / n <= int64_t(kLnMaxVecs) * kWave && aligned16(x) &&
           aligned16(y) && (!gamma || aligned16(gamma)) && (!beta || aligned16(beta));
  };
  if (io_type == MK_BF16) {
    using T = uint16_t;
    const T *xp = (const T*)x, *gp = (const T*)gamma, *bp = (const T*)beta;
    // rows of up to 4096 / 8192 / 16384 stay in registers over 1 / 2 / 4 waves
    const bool vec = cols % 8 == 0 && cols <= 16384 && rows < (int64_t(1) << 31) && aligned16(x) &&
                     aligned16(y) && (!gamma || aligned16(gamma)) && (!beta || aligned16(beta));
    if (vec && cols <= 4096)
      hipLaunchKernelGGL((layernorm_bf16_split_kernel<1, 8>), g, b, 0, s, xp, gp, bp, rows, int(cols), eps, (T*)y);
    else if (vec && cols <= 8192)
      hipLaunchKernelGGL((layernorm_bf16_split_kernel<2, 8>), dim3(unsigned((rows + 1) / 2)), b, 0, s, xp, gp,
                         bp, rows, int(cols), eps, (T*)y);
    else if (vec && cols <= 16384)
      hipLaunchKernelGGL((layernorm_bf16_split_kernel<4, 8>), dim3(unsigned(rows)), b, 0, s, xp, gp, bp, rows,
                         int(cols), eps, (T*)y);
    else
      hipLaunchKernelGGL(layernorm_loop_kernel<T>, g, b, 0, s, xp, gp, bp, rows, cols, eps, (T*)y);
  } else if (io_type == MK_F32) {
    using T = float;
    const T *xp = (const T*)x, *gp = (const T*)gamma, *bp = (const T*)beta;
    if (vec_ok(4))
      hipLaunchKernelGGL(layernorm_reg_kernel<T>, g, b, 0, s, xp, gp, bp, rows, int(cols), eps, (T*)y);
    else
      hipLaunchKernelGGL(layernorm_loop_kernel<T>, g, b, 0, s, xp, gp, bp, rows, cols, eps, (T*)y);
  } else {
    return fail(MK_ERR_UNSUPPORTED, "mk_layernorm: io_type must be bf16/f32");
  }
  return check_launch("mk_layernorm");
}

extern "C" int mk_layernorm_typed(void* stream, int in_type, int out_type, int64_t rows, int64_t cols,
                                  const void* x, const void* gamma, const void* beta, float eps, void* y) {
  if (in_type == out_type) return mk_layernorm(stream, in_type, rows, cols, x, gamma, beta, eps, y);
  clear_error();
  if (in_type != MK_F32 || out_type != MK_BF16)
    return fail(MK_ERR_UNSUPPORTED, "mk_layernorm_typed: (in, out) must be (bf16, bf16), (f32, f32) or (f32, bf16)");
  if (rows < 0 || cols <= 0) return fail(MK_ERR_INVALID, "mk_layernorm_typed: bad shape");
  if (rows == 0) return MK_OK;
  if (!x || !y) return fail(MK_ERR_INVALID, "mk_layernorm_typed: null pointer");
  hipStream_t s = as_stream(stream);
  dim3 g(grid_for_rows(rows)), b(kBlock);
  const float *xp = (const float*)x, *gp = (const float*)gamma, *bp = (const float*)beta;
  const bool vec = cols % 4 == 0 && cols / 4 <= int64_t(kLnMaxVecs) * kWave && aligned16(x) &&
                   (reinterpret_cast<uintptr_t>(y) & 7u) == 0 && (!gamma || aligned16(gamma)) &&
                   (!beta || aligned16(beta));
  if (vec)
    hipLaunchKernelGGL((layernorm_reg_kernel<float, uint16_t>), g, b, 0, s, xp, gp, bp, rows, int(cols), eps,
                       (uint16_t*)y);
  else
    hipLaunchKernelGGL((layernorm_loop_kernel<float, uint16_t>), g, b, 0, s, xp, gp, bp, rows, cols, eps,
                       (uint16_t*)y);
  return check_launch("mk_layernorm_typed");
}

extern "C" int mk_add_layernorm_typed(void* stream, int in_type, int out_type, int64_t rows, int64_t cols,
                                      const void* a, const void* b, const void* bias, const void* gamma,
                                      const void* beta, float eps, void* sum_out, void* y) {
  if (in_type == MK_BF16 && out_type == MK_BF16)
    return mk_add_layernorm(stream, rows, cols, a, b, bias, gamma, beta, eps, sum_out, y);
  clear_error();
  if (in_type != MK_F32 || (out_type != MK_F32 && out_type != MK_BF16))
    return fail(MK_ERR_UNSUPPORTED, "mk_add_layernorm_typed: (in, out) must be (bf16, bf16), (f32, f32) or (f32, bf16)");
  if (bias) return fail(MK_ERR_UNSUPPORTED, "mk_add_layernorm_typed: no bias for fp32 rows (add it to b)");
  if (rows < 0 || cols <= 0) return fail(MK_ERR_INVALID, "mk_add_layernorm_typed: bad shape");
  if (rows == 0) return MK_OK;
  if (!a || !b || !sum_out || !y) return fail(MK_ERR_INVALID, "mk_add_layernorm_typed: null pointer");
  hipStream_t s = as_stream(stream);
  dim3 g(grid_for_rows(rows)), blk(kBlock);
  const float *ap = (const float*)a, *bp = (const float*)b, *gp = (const float*)gamma, *tp = (const float*)beta;
  float* sp = (float*)sum_out;
  const uintptr_t ymask = out_type == MK_BF16 ? 7u : 15u;
  const bool vec = cols % 4 == 0 && cols / 4 <= int64_t(kLnMaxVecs) * kWave && aligned16(a) && aligned16(b) &&
                   aligned16(sum_out) && (reinterpret_cast<uintptr_t>(y) & ymask) == 0 && (!gamma || aligned16(gamma)) &&
                   (!beta || aligned16(beta));
  if (out_type == MK_BF16) {
    if (vec)
      hipLaunchKernelGGL((layernorm_reg_kernel<float, uint16_t, true>), g, blk, 0, s, ap, gp, tp, rows, int(cols), eps,
                         (uint16_t*)y, bp, sp);
    else
      hipLaunchKernelGGL((layernorm_loop_kernel<float, uint16_t>), g, blk, 0, s, ap, gp, tp, rows, cols, eps,
                         (uint16_t*)y, bp, sp);
  } else {
    if (vec)
      hipLaunchKernelGGL((layernorm_reg_kernel<float, float, true>), g, blk, 0, s, ap, gp, tp, rows, int(cols), eps,
                         (float*)y, bp, sp);
    else
      hipLaunchKernelGGL((layernorm_loop_kernel<float, float>), g, blk, 0, s, ap, gp, tp, rows, cols, eps, (float*)y,
                         bp, sp);
  }
  return check_launch("mk_add_layernorm_typed");
}

extern "C" int mk_softmax_rows(void* stream, int io_type, int64_t rows, int64_t cols,
                               const void* x, void* y) {
  clear_error();
  if (rows < 0 || cols <= 0) return fail(MK_ERR_INVALID, "mk_softmax_rows: bad shape");
  if (rows == 0) return MK_OK;
  if (!x || !y) return fail(MK_ERR_INVALID, "mk_softmax_rows: null pointer");
  hipStream_t s = as_stream(stream);
  dim3 g(grid_for_rows(rows)), b(kBlock);
  if (io_type == MK_BF16)
    hipLaunchKernelGGL(softmax_kernel<uint16_t>, g, b, 0, s, (const uint16_t*)x, rows, cols, (uint16_t*)y);
  else if (io_type == MK_F32)
    hipLaunchKernelGGL(softmax_kernel<float>, g, b, 0, s, (const float*)x, rows, cols, (float*)y);
  else
    return fail(MK_ERR_UNSUPPORTED, "mk_softmax_rows: io_type must be bf16/f32");
  return check_launch("mk_softmax_rows");
}
