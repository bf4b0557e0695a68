// Backward and optimizer kernels of the one-GPU training step (config C5,
// a GPT-2-small decoder): LayerNorm and GELU(tanh) backward, column sums
// (bias gradients), fused softmax cross-entropy (loss and logit gradient in
// one pass pair), attention backward and the Adam update of the reference's
// training loop.
//
// Every reduction here is deterministic: column sums go through per-block
// partial rows in a workspace and a second pass that adds the partials in
// block order, so the same inputs give the same bits on every run.
#include "mk_common.h"

#include <cmath>
#include <initializer_list>
#include <type_traits>

namespace mk {
namespace {

constexpr int kBlock = 256;

typedef unsigned short u16x8_t __attribute__((ext_vector_type(8)));

__device__ inline float lo16(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ inline float hi16(uint32_t w) { return __builtin_bit_cast(float, w & 0xFFFF0000u); }
__device__ inline uint32_t pack_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

template <typename T> __device__ inline float ldf(const T* p, int64_t i);
template <> __device__ inline float ldf<float>(const float* p, int64_t i) { return p[i]; }
template <> __device__ inline float ldf<uint16_t>(const uint16_t* p, int64_t i) { return bf16_to_f32(p[i]); }
template <typename T> __device__ inline void stf(T* p, int64_t i, float v);
template <> __device__ inline void stf<float>(float* p, int64_t i, float v) { p[i] = v; }
template <> __device__ inline void stf<uint16_t>(uint16_t* p, int64_t i, float v) { p[i] = f32_to_bf16(v); }

inline int64_t align256(int64_t n) { return (n + 255) & ~int64_t(255); }

// ---------------------------------------------------------------- GELU bwd
// (gelu_tanh_grad_f32 in mk_common.h)

template <typename T>
__global__ __launch_bounds__(kBlock) void gelu_bwd_kernel(const T* __restrict__ x, const T* __restrict__ dy,
                                                        T* __restrict__ dx, int64_t n) {
  const int64_t stride = int64_t(gridDim.x) * kBlock;
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
    stf<T>(dx, i, ldf<T>(dy, i) * gelu_tanh_grad_f32(ldf<T>(x, i)));
}

// bf16, 8 elements per thread per trip
__global__ __launch_bounds__(kBlock) void gelu_bwd_bf16x8_kernel(const u32x4_t* __restrict__ x,
                                                                const u32x4_t* __restrict__ dy,
                                                                u32x4_t* __restrict__ dx, int64_t nvec) {
  const int64_t stride = int64_t(gridDim.x) * kBlock;
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < nvec; i += stride) {
    const u32x4_t a = x[i], d = dy[i];
    u32x4_t o;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o[j] = pack_bf16(lo16(d[j]) * gelu_tanh_grad_f32(lo16(a[j])), hi16(d[j]) * gelu_tanh_grad_f32(hi16(a[j])));
    dx[i] = o;
  }
}

// ---------------------------------------------------------------- column sums
// Row data moves as 16-byte vectors: NV elements of T, widened to fp32.
template <typename T> struct RowVec;
template <> struct RowVec<uint16_t> {
  using Raw = u32x4_t;
  static constexpr int NV = 8;
  __device__ static void unpack(const u32x4_t& v, float (&f)[NV]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f[2 * j] = lo16(v[j]);
      f[2 * j + 1] = hi16(v[j]);
    }
  }
  __device__ static u32x4_t pack(const float (&f)[NV]) {
    u32x4_t v;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = pack_bf16(f[2 * j], f[2 * j + 1]);
    return v;
  }
};
template <> struct RowVec<float> {
  using Raw = u32x4_t;
  static constexpr int NV = 4;
  __device__ static void unpack(const u32x4_t& v, float (&f)[NV]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t w = v[j];  // bit_cast of the vector element itself reads element 0 (hipcc)
      f[j] = __builtin_bit_cast(float, w);
    }
  }
  __device__ static u32x4_t pack(const float (&f)[NV]) {
    u32x4_t v;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = __builtin_bit_cast(uint32_t, f[j]);
    return v;
  }
};

// bf16 rows as 8-byte vectors (4 values per lane per step): a 768-column
// row is exactly three steps of 64 lanes.
struct Bf16x4 {
  using Raw = uint2;
  static constexpr int NV = 4;
  __device__ static void unpack(const uint2& v, float (&f)[NV]) {
    f[0] = lo16(v.x);
    f[1] = hi16(v.x);
    f[2] = lo16(v.y);
    f[3] = hi16(v.y);
  }
  __device__ static uint2 pack(const float (&f)[NV]) { return uint2{pack_bf16(f[0], f[1]), pack_bf16(f[2], f[3])}; }
};

// Pass 1, column partials over 16-byte vectors.  Block (bx, by) covers rows
// [bx rpb, bx rpb + rpb) and the 64 NV columns from by 64 NV: thread t owns
// column vector t % 64 and visits rows r0 + t / 64, + 4, ..., loading four
// of its rows before using any (Op::load), then Op::apply turns each into NV
// values (computing and storing whatever the pass writes).  The four row
// lanes are added in lane order through LDS into partial row bx.
constexpr int kRowLanes = kBlock / 64;

template <typename T, class Op>
__device__ inline void col_partial_body(const Op& op, int64_t rows, int64_t cols, int64_t rpb,
                                        float* __restrict__ part) {
  constexpr int NV = RowVec<T>::NV, BC = 64 * NV, UNR = 4;
  __shared__ float red[kRowLanes][BC];
  const int cv = threadIdx.x & 63, rl = threadIdx.x >> 6;
  const int64_t r0 = int64_t(blockIdx.x) * rpb, r1 = min(rows, r0 + rpb);
  const int64_t cb = int64_t(blockIdx.y) * BC, c = cb + cv * NV;
  float acc[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) acc[j] = 0.f;
  if (c < cols) {
    for (int64_t r = r0 + rl; r < r1; r += UNR * kRowLanes) {
      typename Op::Raw raw[UNR];
#pragma unroll
      for (int u = 0; u < UNR; ++u)
        if (r + u * kRowLanes < r1) raw[u] = op.load(r + u * kRowLanes, c);
#pragma unroll
      for (int u = 0; u < UNR; ++u)
        if (r + u * kRowLanes < r1) {
          float f[NV];
          op.apply(r + u * kRowLanes, c, raw[u], f);
#pragma unroll
          for (int j = 0; j < NV; ++j) acc[j] += f[j];
        }
    }
  }
#pragma unroll
  for (int j = 0; j < NV; ++j) red[rl][cv * NV + j] = acc[j];
  __syncthreads();
  for (int i = threadIdx.x; i < BC; i += kBlock)
    if (cb + i < cols) {
      float t = red[0][i];
#pragma unroll
      for (int l = 1; l < kRowLanes; ++l) t += red[l][i];
      part[int64_t(blockIdx.x) * cols + cb + i] = t;
    }
}

template <typename T>
struct SumOp {
  using Raw = u32x4_t;
  const T* x;
  int64_t cols;
  __device__ Raw load(int64_t r, int64_t c) const { return *reinterpret_cast<const u32x4_t*>(x + r * cols + c); }
  __device__ void apply(int64_t, int64_t, const Raw& v, float (&f)[RowVec<T>::NV]) const { RowVec<T>::unpack(v, f); }
};

template <typename T>
__global__ __launch_bounds__(kBlock) void col_partial_vec_kernel(const T* __restrict__ x, int64_t rows, int64_t cols,
                                                               int64_t rpb, float* __restrict__ part) {
  col_partial_body<T>(SumOp<T>{x, cols}, rows, cols, rpb, part);
}

// dx = dy * gelu_tanh'(x), stored, and its column partials
template <typename T>
struct GeluBwdOp {
  struct Raw {
    u32x4_t x, dy;
  };
  const T* x;
  const T* dy;
  T* dx;
  int64_t cols;
  __device__ Raw load(int64_t r, int64_t c) const {
    return Raw{*reinterpret_cast<const u32x4_t*>(x + r * cols + c), *reinterpret_cast<const u32x4_t*>(dy + r * cols + c)};
  }
  __device__ void apply(int64_t r, int64_t c, const Raw& v, float (&f)[RowVec<T>::NV]) const {
    constexpr int NV = RowVec<T>::NV;
    float xf[NV], df[NV];
    RowVec<T>::unpack(v.x, xf);
    RowVec<T>::unpack(v.dy, df);
#pragma unroll
    for (int j = 0; j < NV; ++j) f[j] = df[j] * gelu_tanh_grad_f32(xf[j]);
    *reinterpret_cast<u32x4_t*>(dx + r * cols + c) = RowVec<T>::pack(f);
  }
};

template <typename T>
__global__ __launch_bounds__(kBlock) void gelu_bwd_cols_kernel(const T* x, const T* dy, T* dx, int64_t rows,
                                                             int64_t cols, int64_t rpb, float* __restrict__ part) {
  col_partial_body<T>(GeluBwdOp<T>{x, dy, dx, cols}, rows, cols, rpb, part);
}

// Scalar pass 1 for rows that are not whole 16-byte vectors: block b sums
// rows [b rpb, b rpb + rpb) of columns by 2048 + t, + 256, ... in row order.
constexpr int64_t kColChunk = 8 * kBlock;

template <typename T>
__global__ __launch_bounds__(kBlock) void col_partial_kernel(const T* __restrict__ x, int64_t rows, int64_t cols,
                                                           int64_t rpb, float* __restrict__ part) {
  const int64_t r0 = int64_t(blockIdx.x) * rpb, r1 = min(rows, r0 + rpb);
  const int64_t c1 = min(cols, int64_t(blockIdx.y + 1) * kColChunk);
  for (int64_t c = int64_t(blockIdx.y) * kColChunk + threadIdx.x; c < c1; c += kBlock) {
    float acc = 0.f;
    for (int64_t r = r0; r < r1; ++r) acc += ldf<T>(x, r * cols + c);
    part[int64_t(blockIdx.x) * cols + c] = acc;
  }
}

// Pass 2: y[c] = sum of the nparts partial rows, for up to three (partials,
// output) pairs (grid y).  A block covers 16 columns with 16 groups of
// threads; group j adds partials j, j + 16, ... in order (eight loads in
// flight), then the group sums are added in group order: a fixed summation
// tree, so the result is deterministic.
constexpr int kFinCols = 16, kFinGroups = kBlock / kFinCols;

struct FinalJob {
  const float* part[3];
  float* out[3];
};

__global__ __launch_bounds__(kBlock) void col_final_kernel(const FinalJob job, int64_t nparts, int64_t cols) {
  __shared__ float red[kFinGroups][kFinCols];
  const float* __restrict__ part = job.part[blockIdx.y];
  const int cl = threadIdx.x % kFinCols, grp = threadIdx.x / kFinCols;
  const int64_t c = int64_t(blockIdx.x) * kFinCols + cl;
  float acc = 0.f;
  if (c < cols) {
    int64_t p = grp;
    for (; p + 7 * kFinGroups < nparts; p += 8 * kFinGroups) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = part[(p + u * kFinGroups) * cols + c];
#pragma unroll
      for (int u = 0; u < 8; ++u) acc += v[u];
    }
    for (; p < nparts; p += kFinGroups) acc += part[p * cols + c];
  }
  red[grp][cl] = acc;
  __syncthreads();
  if (grp == 0 && c < cols) {
    float t = red[0][cl];
#pragma unroll
    for (int j = 1; j < kFinGroups; ++j) t += red[j][cl];
    job.out[blockIdx.y][c] = t;
  }
}

inline int64_t col_parts(int64_t rows) { return std::min<int64_t>(512, std::max<int64_t>(1, (rows + 15) / 16)); }

// launches pass 2 for n pairs
int col_final(hipStream_t s, int n, const float* const* parts, float* const* outs, int64_t nparts, int64_t cols) {
  FinalJob job{};
  for (int i = 0; i < n; ++i) {
    job.part[i] = parts[i];
    job.out[i] = outs[i];
  }
  const dim3 g(unsigned((cols + kFinCols - 1) / kFinCols), unsigned(n));
  hipLaunchKernelGGL(col_final_kernel, g, dim3(kBlock), 0, s, job, nparts, cols);
  return check_launch("column sum final pass");
}

// ---------------------------------------------------------------- LayerNorm bwd
// One wave per row (rows of up to 64 NV KV columns held in registers as
// fp32, NV consecutive columns per lane per step); the row's mean / rstd are
// recomputed from x exactly as the forward computes them (two-pass).  With
// xh = (x - mean) rstd and g = dy gamma:
//   dx = rstd (g - mean(g) - xh mean(g xh))  (+ dres, the residual branch),
// Block b owns rows [b rpb, b rpb + rpb), its wave w rows r0 + w, + 4, ...;
// on the vector path the next row's loads are issued before the current
// row's arithmetic.  Each lane adds dy xh, dy and the stored dx into
// per-column accumulators, which the block adds in wave order through LDS
// into its partial rows of dgamma, dbeta and colsum(dx).
struct LnBwdArgs {
  const void* x;
  const void* gamma;
  const void* dy;
  const void* dres;
  void* dx;
  uint16_t* dx16;  // fp32 rows: the bf16 rounding of dx as well (may be null)
  int64_t rows, rpb;
  int cols;
  float eps;
  float* part_g;
  float* part_b;
  float* part_s;
};

constexpr int kLnBwdMaxCols = 2048;
constexpr int kLnBwdSliceCols = 1024;

// W waves per block; rows r0 + w, r0 + w + W, ... go to wave w, each wave
// requesting its next row before it reduces the current one.  The column
// partials are merged after the rows, so their cost grows with W: 4 waves
// per block was fastest at 8192 x 768.
template <typename T, typename RV, int KV, bool VEC, int W, bool SLICES = false>
__global__ __launch_bounds__(64 * W) void layernorm_bwd_kernel(const LnBwdArgs a) {
  using Raw = typename RV::Raw;
  constexpr int NV = RV::NV;
  // SLICES (rows of at most kLnBwdSliceCols columns): one LDS slice per wave;
  // otherwise one shared slice merged in wave rounds.  Columns past the
  // slice width are a sink for lanes past the row end.
  constexpr int SC = SLICES ? kLnBwdSliceCols : kLnBwdMaxCols;
  __shared__ __attribute__((aligned(16))) float red[SLICES ? W : 1][3][SC + 8];
  const T* __restrict__ x = static_cast<const T*>(a.x);
  const T* __restrict__ gamma = static_cast<const T*>(a.gamma);
  const T* __restrict__ dy = static_cast<const T*>(a.dy);
  const T* dres = static_cast<const T*>(a.dres);
  T* dx = static_cast<T*>(a.dx);
  const int cols = a.cols;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const float inv_n = 1.f / float(cols);
  float gam[KV][NV], accg[KV][NV], accb[KV][NV], accs[KV][NV];
  // gamma: clamped addresses rather than per-element guards, so the loads
  // are issued together and waited for once (a guarded load per element is
  // a memory round trip each, in series, before the first row)
  if (gamma) {
#pragma unroll
    for (int k = 0; k < KV; ++k)
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int c = (k * 64 + lane) * NV + j;
        gam[k][j] = ldf<T>(gamma, c < cols ? c : cols - 1);
      }
  } else {
#pragma unroll
    for (int k = 0; k < KV; ++k)
#pragma unroll
      for (int j = 0; j < NV; ++j) gam[k][j] = 1.f;
  }
#pragma unroll
  for (int k = 0; k < KV; ++k)
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int c = (k * 64 + lane) * NV + j;
      if (c >= cols) gam[k][j] = 0.f;
      accg[k][j] = accb[k][j] = accs[k][j] = 0.f;
    }
  const int64_t r0 = int64_t(blockIdx.x) * a.rpb, r1 = min(a.rows, r0 + a.rpb);
  // Row loads are unconditional: a row past the block's end reloads the
  // block's last row, a column past the row end loads column 0, and without
  // a residual x stands in for it; the values are discarded or zeroed after
  // unpacking.  Guarded loads would sit in branches, and the compiler then
  // waits for every load in flight (the next row's too) at the joins.
  Raw xr[KV], dr[KV], rr[KV];
  const T* __restrict__ res_src = dres ? dres : x;
  auto fetch = [&](int64_t r) __attribute__((always_inline)) {
    const int64_t rc = r < r1 ? r : r1 - 1;
#pragma unroll
    for (int k = 0; k < KV; ++k) {
      const int c0 = (k * 64 + lane) * NV;
      const int cs = c0 < cols ? c0 : 0;
      xr[k] = *reinterpret_cast<const Raw*>(x + rc * cols + cs);
      dr[k] = *reinterpret_cast<const Raw*>(dy + rc * cols + cs);
      rr[k] = *reinterpret_cast<const Raw*>(res_src + rc * cols + cs);
    }
  };
  // one row: statistics, dx = rstd (dy g - mean(dy g) - xhat mean(dy g xhat)) + dres,
  // and the column partials
  auto process = [&](int64_t r, float (&xv)[KV][NV], const float (&dv)[KV][NV],
                     const float (&rv)[KV][NV]) __attribute__((always_inline)) {
    float sx = 0.f;
#pragma unroll
    for (int k = 0; k < KV; ++k)
#pragma unroll
      for (int j = 0; j < NV; ++j) sx += xv[k][j];
    const float mean = wave_sum_dpp(sx) * inv_n;
    float q = 0.f;
#pragma unroll
    for (int k = 0; k < KV; ++k)
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int c = (k * 64 + lane) * NV + j;
        const float d = (c < cols) ? xv[k][j] - mean : 0.f;
        q += d * d;
      }
    const float rstd = 1.f / sqrtf(wave_sum_dpp(q) * inv_n + a.eps);
    float sg = 0.f, sgx = 0.f;
#pragma unroll
    for (int k = 0; k < KV; ++k)
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int c = (k * 64 + lane) * NV + j;
        const float xh = (c < cols) ? (xv[k][j] - mean) * rstd : 0.f;
        const float g = dv[k][j] * gam[k][j];
        sg += g;
        sgx += g * xh;
        accg[k][j] += dv[k][j] * xh;
        accb[k][j] += dv[k][j];
        xv[k][j] = xh;
      }
    const float mg = wave_sum_dpp(sg) * inv_n, mgx = wave_sum_dpp(sgx) * inv_n;
#pragma unroll
    for (int k = 0; k < KV; ++k) {
      float o[NV];
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        o[j] = rstd * (dv[k][j] * gam[k][j] - mg - xv[k][j] * mgx) + rv[k][j];
        accs[k][j] += o[j];
      }
      const int c0 = (k * 64 + lane) * NV;
      if constexpr (VEC) {
        if (c0 < cols) {
          *reinterpret_cast<Raw*>(dx + r * cols + c0) = RV::pack(o);
          if constexpr (sizeof(T) == 4 && NV == 4) {
            if (a.dx16)
              *reinterpret_cast<uint2*>(a.dx16 + r * cols + c0) = uint2{pack_bf16(o[0], o[1]), pack_bf16(o[2], o[3])};
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < NV; ++j)
          if (c0 + j < cols) {
            stf<T>(dx, r * cols + c0 + j, o[j]);
            if (sizeof(T) == 4 && a.dx16) a.dx16[r * cols + c0 + j] = f32_to_bf16(o[j]);
          }
      }
    }
  };
  if constexpr (VEC) {
    // the next row's loads are issued before the current row is reduced
    int64_t r = r0 + wid;
    fetch(r);
    for (; r < r1; r += W) {
      float xv[KV][NV], dv[KV][NV], rv[KV][NV];
#pragma unroll
      for (int k = 0; k < KV; ++k) {
        RV::unpack(xr[k], xv[k]);
        RV::unpack(dr[k], dv[k]);
        RV::unpack(rr[k], rv[k]);
        const bool in_row = (k * 64 + lane) * NV < cols;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
          xv[k][j] = in_row ? xv[k][j] : 0.f;
          dv[k][j] = in_row ? dv[k][j] : 0.f;
          rv[k][j] = (in_row && dres) ? rv[k][j] : 0.f;
        }
      }
      fetch(r + W);
      process(r, xv, dv, rv);
    }
  } else {
    for (int64_t r = r0 + wid; r < r1; r += W) {
      float xv[KV][NV], dv[KV][NV], rv[KV][NV];
#pragma unroll
      for (int k = 0; k < KV; ++k)
#pragma unroll
        for (int j = 0; j < NV; ++j) {
          const int c = (k * 64 + lane) * NV + j;
          const bool ok = c < cols;
          xv[k][j] = ok ? ldf<T>(x, r * cols + c) : 0.f;
          dv[k][j] = ok ? ldf<T>(dy, r * cols + c) : 0.f;
          rv[k][j] = (ok && dres) ? ldf<T>(dres, r * cols + c) : 0.f;
        }
      process(r, xv, dv, rv);
    }
  }
  // block partial rows: the W waves added in wave order, the three sums in
  // the same rounds.  The rounds are branch-free (lanes past the row end use
  // the sink column), so a wave issues all of its LDS reads of a round
  // before its first add: per-element guards would put each read in its own
  // branch and serialise the round trips (about 2 us per round at 768
  // columns).
  const bool want_gb = a.part_g != nullptr, want_s = a.part_s != nullptr;
  if (!want_gb && !want_s) return;
  int addr[KV][NV];
#pragma unroll
  for (int k = 0; k < KV; ++k)
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int c0 = (k * 64 + lane) * NV, c = c0 + j;
      // vector path (cols % NV == 0): a lane's NV columns stay contiguous,
      // in range or in the sink, so the compiler can use 16-byte LDS ops
      if constexpr (VEC) addr[k][j] = ((c0 < cols) ? c0 : SC) + j;
      else addr[k][j] = (c < cols) ? c : SC;
    }
  if constexpr (SLICES) {
    // every wave writes its own slice at once; after one barrier the
    // threads add the slices per column in wave order (the same order as
    // the rounds below, so the same bits)
#pragma unroll
    for (int k = 0; k < KV; ++k)
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        red[wid][0][addr[k][j]] = accg[k][j];
        red[wid][1][addr[k][j]] = accb[k][j];
        red[wid][2][addr[k][j]] = accs[k][j];
      }
    __syncthreads();
    for (int c = threadIdx.x; c < cols; c += 64 * W) {
      float g = red[0][0][c], b = red[0][1][c], sm = red[0][2][c];
#pragma unroll
      for (int w = 1; w < W; ++w) {
        g += red[w][0][c];
        b += red[w][1][c];
        sm += red[w][2][c];
      }
      const int64_t o = int64_t(blockIdx.x) * cols + c;
      if (want_gb) {
        a.part_g[o] = g;
        a.part_b[o] = b;
      }
      if (want_s) a.part_s[o] = sm;
    }
  } else {
    for (int w = 0; w < W; ++w) {
      if (wid == w) {
        float cur[3][KV][NV];
#pragma unroll
        for (int k = 0; k < KV; ++k)
#pragma unroll
          for (int j = 0; j < NV; ++j) {
            cur[0][k][j] = w > 0 ? red[0][0][addr[k][j]] : 0.f;
            cur[1][k][j] = w > 0 ? red[0][1][addr[k][j]] : 0.f;
            cur[2][k][j] = w > 0 ? red[0][2][addr[k][j]] : 0.f;
          }
#pragma unroll
        for (int k = 0; k < KV; ++k)
#pragma unroll
          for (int j = 0; j < NV; ++j) {
            red[0][0][addr[k][j]] = cur[0][k][j] + accg[k][j];
            red[0][1][addr[k][j]] = cur[1][k][j] + accb[k][j];
            red[0][2][addr[k][j]] = cur[2][k][j] + accs[k][j];
          }
      }
      __syncthreads();
    }
    for (int c = threadIdx.x; c < cols; c += 64 * W) {
      const int64_t o = int64_t(blockIdx.x) * cols + c;
      if (want_gb) {
        a.part_g[o] = red[0][0][c];
        a.part_b[o] = red[0][1][c];
      }
      if (want_s) a.part_s[o] = red[0][2][c];
    }
  }
}

constexpr int64_t kLnBwdBlocks = 512;  // partial rows of the LayerNorm backward

template <int N>
struct IntC {
  static constexpr int value = N;
};

// ---------------------------------------------------------------- softmax xent
// One workgroup per row.  Pass 1: running (max, sum of exp) per thread,
// combined across the workgroup; lse = max + log(sum).  loss = lse - x[label].
// Pass 2: dlogits = (exp(x - lse) - [j == label]) * grad_scale.
template <typename T, typename L>
__global__ __launch_bounds__(kBlock) void softmax_xent_kernel(const T* __restrict__ logits, int64_t cols, int64_t ld_in,
                                                            const L* __restrict__ labels, float grad_scale,
                                                            float* __restrict__ loss, T* __restrict__ dlogits,
                                                            int64_t ld_out) {
  __shared__ float sm[kBlock / 64], ss[kBlock / 64];
  const int64_t row = blockIdx.x;
  const T* xr = logits + row * ld_in;
  float m = -INFINITY, s = 0.f;
  for (int64_t j = threadIdx.x; j < cols; j += kBlock) {
    const float v = ldf<T>(xr, j);
    if (v > m) {
      s = s * __expf(m - v) + 1.f;
      m = v;
    } else if (m != -INFINITY) {
      s += __expf(v - m);
    }
  }
  // combine (m, s) over the wave, then over the 4 waves
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float mo = __shfl_xor(m, off, 64), so = __shfl_xor(s, off, 64);
    const float mn = fmaxf(m, mo);
    s = (mn == -INFINITY) ? 0.f : s * __expf(m - mn) + so * __expf(mo - mn);
    m = mn;
  }
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  if (lane == 0) {
    sm[wv] = m;
    ss[wv] = s;
  }
  __syncthreads();
  float M = sm[0];
#pragma unroll
  for (int w = 1; w < kBlock / 64; ++w) M = fmaxf(M, sm[w]);
  float S = 0.f;
#pragma unroll
  for (int w = 0; w < kBlock / 64; ++w) S += (sm[w] == -INFINITY) ? 0.f : ss[w] * __expf(sm[w] - M);
  const float lse = M + __logf(S);
  const int64_t lab = int64_t(labels[row]);
  const bool lab_ok = lab >= 0 && lab < cols;
  if (threadIdx.x == 0 && loss) loss[row] = lab_ok ? lse - ldf<T>(xr, lab) : lse;
  T* dr = dlogits + row * ld_out;
  for (int64_t j = threadIdx.x; j < cols; j += kBlock) {
    const float p = __expf(ldf<T>(xr, j) - lse);
    stf<T>(dr, j, (p - (j == lab ? 1.f : 0.f)) * grad_scale);
  }
}

// bf16 rows held in registers: one workgroup of kXentThreads per row, the
// row's 16-byte-aligned body as vectors (thread t: vectors t, t + 512, ...,
// NVT of them), the unaligned head and tail (under 8 elements each) as one
// scalar on threads 0..7 and 8..15.  The row is read once: max, sum of
// exp(x - max), then dlogits = (exp(x - lse) - [j == label]) * grad_scale
// written from the same registers (so dlogits may be logits); the label's
// element is rewritten by one thread after a barrier.
constexpr int kXentThreads = 512;
constexpr uint32_t kBf16NegInfPair = 0xFF80FF80u;

template <int NVT, typename L>
__global__ __launch_bounds__(kXentThreads) void softmax_xent_bf16_kernel(const uint16_t* logits, int64_t cols,
                                                                       int64_t ld_in, const L* __restrict__ labels,
                                                                       float grad_scale, float* __restrict__ loss,
                                                                       uint16_t* dlogits, int64_t ld_out) {
  constexpr int NW = kXentThreads / 64;
  constexpr float kL2e = 1.4426950408889634f;
  __shared__ float red[NW];
  const int64_t row = blockIdx.x;
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const uint16_t* xr = logits + row * ld_in;
  uint16_t* dr = dlogits + row * ld_out;
  const int64_t head = min<int64_t>(cols, int64_t(((16u - (reinterpret_cast<uintptr_t>(xr) & 15u)) & 15u) / 2u));
  const int64_t nv = (cols - head) / 8, tail = cols - head - nv * 8;
  const u32x4_t* xv = reinterpret_cast<const u32x4_t*>(xr + head);
  // the label's logit (for the loss) is loaded with the row, by every lane
  // from one in-range address, rather than by one thread after the
  // reductions, where its round trip would end every workgroup
  const int64_t lab = int64_t(labels[row]);
  const bool lab_ok = lab >= 0 && lab < cols;
  const uint16_t xlab_bits = xr[lab_ok ? lab : 0];
  u32x4_t v[NVT];
#pragma unroll
  for (int i = 0; i < NVT; ++i) {
    const int64_t idx = t + int64_t(i) * kXentThreads;
    v[i] = idx < nv ? xv[idx] : u32x4_t{kBf16NegInfPair, kBf16NegInfPair, kBf16NegInfPair, kBf16NegInfPair};
  }
  // this thread's scalar element, if any: head element t (t < 8) or tail element t - 8
  int64_t ej = -1;
  if (t < head) ej = t;
  else if (t >= 8 && t - 8 < tail) ej = head + nv * 8 + (t - 8);
  const float ex = ej >= 0 ? bf16_to_f32(xr[ej]) : -INFINITY;

  auto block_reduce = [&](float x, bool is_max) __attribute__((always_inline)) {
    x = is_max ? wave_max(x) : wave_sum(x);
    if (lane == 0) red[wv] = x;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) r = is_max ? fmaxf(r, red[w]) : r + red[w];
    __syncthreads();
    return r;
  };
  float m = ex;
#pragma unroll
  for (int i = 0; i < NVT; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) m = fmaxf(m, fmaxf(lo16(v[i][j]), hi16(v[i][j])));
  // exponents from x - max (exact at the max), so a row's largest p is
  // exactly 1 / S and a one-class row has p = 1, gradient 0
  const float M = block_reduce(m, true);
  // the exponentials are kept for the gradient (one exp per element)
  const float eex = ej >= 0 ? __builtin_amdgcn_exp2f((ex - M) * kL2e) : 0.f;
  float e[NVT][8];
  float sum = eex;
#pragma unroll
  for (int i = 0; i < NVT; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      e[i][2 * j] = __builtin_amdgcn_exp2f((lo16(v[i][j]) - M) * kL2e);
      e[i][2 * j + 1] = __builtin_amdgcn_exp2f((hi16(v[i][j]) - M) * kL2e);
      sum += e[i][2 * j] + e[i][2 * j + 1];
    }
  const float S = block_reduce(sum, false);
  const float lse = M + __logf(S);
  const float inv_s = 1.f / S;
  if (t == 0 && loss) loss[row] = lab_ok ? lse - bf16_to_f32(xlab_bits) : lse;
  // gradient, from the registers (every read of the row is done: in place is safe)
  u32x4_t* dv = reinterpret_cast<u32x4_t*>(dr + head);
#pragma unroll
  for (int i = 0; i < NVT; ++i) {
    const int64_t idx = t + int64_t(i) * kXentThreads;
    if (idx < nv) {
      u32x4_t o;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = pack_bf16(e[i][2 * j] * inv_s * grad_scale, e[i][2 * j + 1] * inv_s * grad_scale);
      dv[idx] = o;
    }
  }
  if (ej >= 0) dr[ej] = f32_to_bf16(eex * inv_s * grad_scale);
  // the one-hot term touches one element: after every store above, thread 0
  // rewrites it as (p - 1) * grad_scale, p from the label's logit (the same
  // value and rounding as the element's own store)
  if (lab_ok) {
    __syncthreads();
    if (t == 0) {
      const float p = __builtin_amdgcn_exp2f((bf16_to_f32(xlab_bits) - M) * kL2e) * inv_s - 1.f;
      dr[lab] = f32_to_bf16(p * grad_scale);
    }
  }
}

// fp32 logits, bf16 dlogits (the gradient only feeds bf16 products): one
// workgroup of kXentF32Threads per row, the row held in registers (NPT
// elements per thread, element j on thread j % kXentF32Threads), read once
// with coalesced loads; exact row max, then the sum of exp(x - max), then
// dlogits = (exp(x - lse) - [j == label]) * grad_scale stored as bf16.
constexpr int kXentF32Threads = 1024;

template <int NPT, typename L>
__global__ __launch_bounds__(kXentF32Threads) void softmax_xent_f32_bf16_kernel(
    const float* __restrict__ logits, int64_t cols, int64_t ld_in, const L* __restrict__ labels, float grad_scale,
    float* __restrict__ loss, uint16_t* __restrict__ dlogits, int64_t ld_out) {
  constexpr int NW = kXentF32Threads / 64;
  constexpr float kL2e = 1.4426950408889634f;
  __shared__ float red[NW];
  const int64_t row = blockIdx.x;
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const float* xr = logits + row * ld_in;
  uint16_t* dr = dlogits + row * ld_out;
  const int64_t lab = int64_t(labels[row]);
  const bool lab_ok = lab >= 0 && lab < cols;
  const float xlab = xr[lab_ok ? lab : 0];
  float x[NPT];
#pragma unroll
  for (int k = 0; k < NPT; ++k) {
    const int64_t j = t + int64_t(k) * kXentF32Threads;
    x[k] = j < cols ? xr[j] : -INFINITY;
  }
  auto block_reduce = [&](float v, bool is_max) __attribute__((always_inline)) {
    v = is_max ? wave_max(v) : wave_sum(v);
    if (lane == 0) red[wv] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) r = is_max ? fmaxf(r, red[w]) : r + red[w];
    __syncthreads();
    return r;
  };
  float m = x[0];
#pragma unroll
  for (int k = 1; k < NPT; ++k) m = fmaxf(m, x[k]);
  const float M = block_reduce(m, true);
  float sum = 0.f;
#pragma unroll
  for (int k = 0; k < NPT; ++k) sum += __builtin_amdgcn_exp2f((x[k] - M) * kL2e);
  const float S = block_reduce(sum, false);
  const float lse = M + __logf(S);
  const float ls2 = __builtin_amdgcn_logf(S);  // log2 S
  if (t == 0 && loss) loss[row] = lab_ok ? lse - xlab : lse;
#pragma unroll
  for (int k = 0; k < NPT; ++k) {
    const int64_t j = t + int64_t(k) * kXentF32Threads;
    if (j < cols) {
      const float pr = __builtin_amdgcn_exp2f(fmaf(x[k] - M, kL2e, -ls2));
      dr[j] = f32_to_bf16((j == lab ? pr - 1.f : pr) * grad_scale);
    }
  }
}

// The same for rows longer than the registers hold (more than 32
// elements per thread): the row is streamed twice in chunks of C elements
// per thread.  Pass 1 keeps a running (max, sum of exp) per thread, raised
// once per chunk; pass 2 re-reads the row (from the L2 / MALL, where one
// row per CU stays resident between the passes) and writes dlogits.
template <int C, typename L>
__global__ __launch_bounds__(kXentF32Threads) void softmax_xent_f32_bf16_stream_kernel(
    const float* __restrict__ logits, int64_t cols, int64_t ld_in, const L* __restrict__ labels, float grad_scale,
    float* __restrict__ loss, uint16_t* __restrict__ dlogits, int64_t ld_out) {
  constexpr int NW = kXentF32Threads / 64;
  constexpr float kL2e = 1.4426950408889634f;
  constexpr int64_t kChunk = int64_t(C) * kXentF32Threads;
  __shared__ float red[NW];
  const int64_t row = blockIdx.x;
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const float* xr = logits + row * ld_in;
  uint16_t* dr = dlogits + row * ld_out;
  const int64_t lab = int64_t(labels[row]);
  const bool lab_ok = lab >= 0 && lab < cols;
  const float xlab = xr[lab_ok ? lab : 0];
  float m = -INFINITY, sum = 0.f;  // running max and sum of exp2((x - m) log2 e)
  for (int64_t c0 = 0; c0 < cols; c0 += kChunk) {
    float x[C];
#pragma unroll
    for (int k = 0; k < C; ++k) {
      const int64_t j = c0 + t + int64_t(k) * kXentF32Threads;
      x[k] = j < cols ? xr[j] : -INFINITY;
    }
    float cm = x[0];
#pragma unroll
    for (int k = 1; k < C; ++k) cm = fmaxf(cm, x[k]);
    const float mn = fmaxf(m, cm);
    if (mn != -INFINITY) {
      float cs = 0.f;
#pragma unroll
      for (int k = 0; k < C; ++k) cs += __builtin_amdgcn_exp2f((x[k] - mn) * kL2e);
      sum = (m == -INFINITY ? 0.f : sum * __builtin_amdgcn_exp2f((m - mn) * kL2e)) + cs;
      m = mn;
    }
  }
  // combine (m, sum) over the workgroup
  const float wm = wave_max(m);
  const float ws = wave_sum(m == -INFINITY ? 0.f : sum * __builtin_amdgcn_exp2f((m - wm) * kL2e));
  __shared__ float red_s[NW];
  if (lane == 0) {
    red[wv] = wm;
    red_s[wv] = ws;
  }
  __syncthreads();
  float M = red[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) M = fmaxf(M, red[w]);
  float S = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) S += red[w] == -INFINITY ? 0.f : red_s[w] * __builtin_amdgcn_exp2f((red[w] - M) * kL2e);
  const float lse = M + __logf(S);
  const float ls2 = __builtin_amdgcn_logf(S);
  if (t == 0 && loss) loss[row] = lab_ok ? lse - xlab : lse;
  for (int64_t c0 = 0; c0 < cols; c0 += kChunk) {
#pragma unroll
    for (int k = 0; k < C; ++k) {
      const int64_t j = c0 + t + int64_t(k) * kXentF32Threads;
      if (j < cols) {
        const float pr = __builtin_amdgcn_exp2f(fmaf(xr[j] - M, kL2e, -ls2));
        dr[j] = f32_to_bf16((j == lab ? pr - 1.f : pr) * grad_scale);
      }
    }
  }
}

// fp32 logits, bf16 dlogits, rows 16-byte aligned (a padded row pitch): the
// row held in registers as NV 16-byte vectors per thread (vector v on thread
// v % kXentF32Threads), read once; dlogits stored as 8-byte groups of four.
// A last, partial vector is read and written element by element, so nothing
// past `cols` is touched.  Same arithmetic as softmax_xent_f32_bf16_kernel.
template <int NV, typename L>
__global__ __launch_bounds__(kXentF32Threads) void softmax_xent_f32_bf16_vec_kernel(
    const float* __restrict__ logits, int64_t cols, int64_t ld_in, const L* __restrict__ labels, float grad_scale,
    float* __restrict__ loss, uint16_t* __restrict__ dlogits, int64_t ld_out) {
  constexpr int NW = kXentF32Threads / 64;
  constexpr float kL2e = 1.4426950408889634f;
  __shared__ float red[NW];
  const int64_t row = blockIdx.x;
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const float* xr = logits + row * ld_in;
  uint16_t* dr = dlogits + row * ld_out;
  const int64_t lab = int64_t(labels[row]);
  const bool lab_ok = lab >= 0 && lab < cols;
  const float xlab = xr[lab_ok ? lab : 0];
  const int64_t nfull = cols / 4;  // whole vectors; a partial one follows when cols % 4 != 0
  const f32x4* xv = reinterpret_cast<const f32x4*>(xr);
  f32x4 x[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t v = t + int64_t(i) * kXentF32Threads;
    if (v < nfull) {
      x[i] = ld_stream(&xv[v]);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) x[i].v[j] = 4 * v + j < cols ? xr[4 * v + j] : -INFINITY;
    }
  }
  auto block_reduce = [&](float val, bool is_max) __attribute__((always_inline)) {
    val = is_max ? wave_max(val) : wave_sum(val);
    if (lane == 0) red[wv] = val;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) r = is_max ? fmaxf(r, red[w]) : r + red[w];
    __syncthreads();
    return r;
  };
  float m = x[0].v[0];
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) m = fmaxf(m, x[i].v[j]);
  const float M = block_reduce(m, true);
  // the exponentials are kept (in place of the logits) for the gradient
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x[i].v[j] = __builtin_amdgcn_exp2f((x[i].v[j] - M) * kL2e);
      sum += x[i].v[j];
    }
  const float S = block_reduce(sum, false);
  const float lse = M + __logf(S);
  const float inv_s = 1.f / S;
  if (t == 0 && loss) loss[row] = lab_ok ? lse - xlab : lse;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t v = t + int64_t(i) * kXentF32Threads;
    if (4 * v >= cols) continue;
    float g[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float pr = x[i].v[j] * inv_s;
      g[j] = (4 * v + j == lab ? pr - 1.f : pr) * grad_scale;
    }
    if (v < nfull) {
      *reinterpret_cast<uint2*>(dr + 4 * v) = uint2{f32_to_bf16(g[0]) | (uint32_t(f32_to_bf16(g[1])) << 16),
                                                    f32_to_bf16(g[2]) | (uint32_t(f32_to_bf16(g[3])) << 16)};
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (4 * v + j < cols) dr[4 * v + j] = f32_to_bf16(g[j]);
    }
  }
}

// ---------------------------------------------------------------- Adam
// fp32 gradient, four parameters per thread per trip (16-byte loads and
// stores; the bf16 copy as one 8-byte store); same arithmetic as adam_kernel.
__global__ __launch_bounds__(kBlock) void adam_vec4_kernel(int64_t nvec, f32x4* __restrict__ p32,
                                                         uint2* __restrict__ p16, const f32x4* __restrict__ grad,
                                                         f32x4* __restrict__ m, f32x4* __restrict__ v, float lr,
                                                         float b1, float omb1, float b2, float omb2, float eps,
                                                         float bc1, float bc2, const float* __restrict__ hyper) {
  if (hyper) {
    lr = hyper[0];
    bc1 = hyper[1];
    bc2 = hyper[2];
  }
  const int64_t stride = int64_t(gridDim.x) * kBlock;
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < nvec; i += stride) {
    // every array is touched once per step: streaming loads and stores
    const f32x4 g = ld_stream(&grad[i]), m0 = ld_stream(&m[i]), v0 = ld_stream(&v[i]), p0 = ld_stream(&p32[i]);
    f32x4 m1, v1, p1;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      m1.v[j] = b1 * m0.v[j] + omb1 * g.v[j];
      v1.v[j] = b2 * v0.v[j] + omb2 * g.v[j] * g.v[j];
      p1.v[j] = p0.v[j] - lr * (m1.v[j] / bc1) / (sqrtf(v1.v[j] / bc2) + eps);
    }
    st_stream(&m[i], m1);
    st_stream(&v[i], v1);
    st_stream(&p32[i], p1);
    if (p16) p16[i] = uint2{pack_bf16(p1.v[0], p1.v[1]), pack_bf16(p1.v[2], p1.v[3])};
  }
}

// dp_train.py body(): m = b1 m + (1-b1) g; v = b2 v + (1-b2) g g;
// p = p - lr (m / bc1) / (sqrt(v / bc2) + eps), in fp32 with the constants
// b1, 1-b1, b2, 1-b2, eps each one fp32 rounding of the double value (as
// JAX folds the Python-float expressions).  With a master copy the update
// runs on the fp32 master and the bf16 parameter receives its RNE rounding;
// without one the fp32 parameter is updated in place.
template <typename G>
__global__ __launch_bounds__(kBlock) void adam_kernel(int64_t n, float* __restrict__ p32, uint16_t* __restrict__ p16,
                                                    const G* __restrict__ grad, float* __restrict__ m,
                                                    float* __restrict__ v, float lr, float b1, float omb1, float b2,
                                                    float omb2, float eps, float bc1, float bc2,
                                                    const float* __restrict__ hyper) {
  if (hyper) {  // lr, bc1, bc2 as device scalars (inputs of the step)
    lr = hyper[0];
    bc1 = hyper[1];
    bc2 = hyper[2];
  }
  const int64_t stride = int64_t(gridDim.x) * kBlock;
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
    const float g = ldf<G>(grad, i);
    const float mi = b1 * m[i] + omb1 * g;
    const float vi = b2 * v[i] + omb2 * g * g;
    m[i] = mi;
    v[i] = vi;
    const float p = p32[i] - lr * (mi / bc1) / (sqrtf(vi / bc2) + eps);
    p32[i] = p;
    if (p16) p16[i] = f32_to_bf16(p);
  }
}

// ---------------------------------------------------------------- attention bwd
// D[r] = sum_d dO[r, d] O[r, d] for every query row r = (b, h, i)
__global__ __launch_bounds__(kBlock) void attn_rowdot_kernel(const uint16_t* __restrict__ o, int64_t o_bs, int64_t o_hs,
                                                           int64_t o_ss, const uint16_t* __restrict__ dout,
                                                           int64_t d_bs, int64_t d_hs, int64_t d_ss, int64_t H,
                                                           int64_t S, int64_t D, int64_t nrows,
                                                           float* __restrict__ out) {
  const int64_t r = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  if (r >= nrows) return;
  const int64_t bh = r / S, i = r % S, b = bh / H, h = bh % H;
  const uint16_t* orow = o + b * o_bs + h * o_hs + i * o_ss;
  const uint16_t* drow = dout + b * d_bs + h * d_hs + i * d_ss;
  float acc = 0.f;
  for (int64_t d = 0; d < D; d += 8) {
    const u32x4_t a = *reinterpret_cast<const u32x4_t*>(orow + d);
    const u32x4_t c = *reinterpret_cast<const u32x4_t*>(drow + d);
#pragma unroll
    for (int j = 0; j < 4; ++j) acc += lo16(a[j]) * lo16(c[j]) + hi16(a[j]) * hi16(c[j]);
  }
  out[r] = acc;
}

// P[bh, i, j] = exp(scale * S[bh, i, j] - lse[bh, i]) (0 where masked), bf16
__global__ __launch_bounds__(kBlock) void attn_probs_kernel(const float* __restrict__ s, const float* __restrict__ lse,
                                                          int64_t Sq, int64_t Sk, float scale, int causal,
                                                          uint16_t* __restrict__ p, int64_t n) {
  const int64_t stride = int64_t(gridDim.x) * kBlock;
  for (int64_t e = int64_t(blockIdx.x) * kBlock + threadIdx.x; e < n; e += stride) {
    const int64_t j = e % Sk, row = e / Sk, i = row % Sq;
    const float v = (causal && j > i) ? 0.f : __expf(scale * s[e] - lse[row]);
    p[e] = f32_to_bf16(v);
  }
}

// dS = scale * P * (dP - D[row]), bf16, written over P
__global__ __launch_bounds__(kBlock) void attn_dscores_kernel(const float* __restrict__ dp, const float* __restrict__ dsum,
                                                            int64_t Sk, float scale, uint16_t* __restrict__ p,
                                                            int64_t n) {
  const int64_t stride = int64_t(gridDim.x) * kBlock;
  for (int64_t e = int64_t(blockIdx.x) * kBlock + threadIdx.x; e < n; e += stride) {
    const float pv = bf16_to_f32(p[e]);
    p[e] = f32_to_bf16(scale * pv * (dp[e] - dsum[e / Sk]));
  }
}

// ---------------------------------------------------------------- fused forward rows
// sum = a + b + bias (fp32 adds, one bf16 rounding: the stored residual
// stream, as mk_add_rows stores it) and y = LayerNorm(sum) over the rounded
// values, two-pass mean / variance as mk_layernorm; one wave per row, four
// bf16 per lane per step (8-byte vectors), KV steps per row.
template <int KV>
__global__ __launch_bounds__(kBlock) void add_layernorm_kernel(const uint2* __restrict__ a, const uint2* b,
                                                             const uint2* __restrict__ bias,
                                                             const uint2* __restrict__ gamma,
                                                             const uint2* __restrict__ beta, int64_t rows, int cols4,
                                                             float eps, uint2* sum_out, uint2* __restrict__ y) {
  const int lane = threadIdx.x & 63;
  const int64_t r = int64_t(blockIdx.x) * (kBlock / 64) + (threadIdx.x >> 6);
  if (r >= rows) return;  // whole waves
  const float inv_n = 1.f / float(cols4 * 4);
  // Every load is issued up front from an in-range address (column 0 for
  // lanes past the row end, a standing in for an absent b, column vectors
  // for absent bias / gamma / beta) and replaced after the loads: guarded
  // loads would sit in branches, each waited for before the next is issued.
  const uint2* bsrc = b ? b : a;
  uint2 xa[KV], xb[KV], zb[KV], gg[KV], bb[KV];
#pragma unroll
  for (int k = 0; k < KV; ++k) {
    const int c = k * 64 + lane, cs = c < cols4 ? c : 0;
    xa[k] = a[r * cols4 + cs];
    xb[k] = bsrc[r * cols4 + cs];
    zb[k] = bias ? bias[cs] : uint2{0u, 0u};
    gg[k] = gamma ? gamma[cs] : uint2{0x3F803F80u, 0x3F803F80u};  // bf16 1.0
    bb[k] = beta ? beta[cs] : uint2{0u, 0u};
  }
  float v[KV][4];
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < KV; ++k) {
    const int c = k * 64 + lane;
    const uint2 x = xa[k];
    const uint2 y2 = b ? xb[k] : uint2{0u, 0u};
    const uint2 z = zb[k];
    const uint32_t w0 = pack_bf16(lo16(x.x) + lo16(y2.x) + lo16(z.x), hi16(x.x) + hi16(y2.x) + hi16(z.x));
    const uint32_t w1 = pack_bf16(lo16(x.y) + lo16(y2.y) + lo16(z.y), hi16(x.y) + hi16(y2.y) + hi16(z.y));
    const bool in_row = c < cols4;
    if (in_row) sum_out[r * cols4 + c] = uint2{w0, w1};
    v[k][0] = in_row ? lo16(w0) : 0.f;
    v[k][1] = in_row ? hi16(w0) : 0.f;
    v[k][2] = in_row ? lo16(w1) : 0.f;
    v[k][3] = in_row ? hi16(w1) : 0.f;
    s += (v[k][0] + v[k][1]) + (v[k][2] + v[k][3]);
  }
  const float mean = wave_sum_dpp(s) * inv_n;
  float q = 0.f;
#pragma unroll
  for (int k = 0; k < KV; ++k) {
    const bool in_row = k * 64 + lane < cols4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float d = in_row ? v[k][j] - mean : 0.f;
      q += d * d;
    }
  }
  const float rstd = 1.f / sqrtf(wave_sum_dpp(q) * inv_n + eps);
#pragma unroll
  for (int k = 0; k < KV; ++k) {
    const int c = k * 64 + lane;
    if (c < cols4) {
      const uint2 g = gg[k], be = bb[k];
      const float o0 = (v[k][0] - mean) * rstd * lo16(g.x) + lo16(be.x);
      const float o1 = (v[k][1] - mean) * rstd * hi16(g.x) + hi16(be.x);
      const float o2 = (v[k][2] - mean) * rstd * lo16(g.y) + lo16(be.y);
      const float o3 = (v[k][3] - mean) * rstd * hi16(g.y) + hi16(be.y);
      y[r * cols4 + c] = uint2{pack_bf16(o0, o1), pack_bf16(o2, o3)};
    }
  }
}

// pre = x + bias (one bf16 rounding, stored: the activation's input that the
// backward needs) and y = gelu_tanh(pre) from the rounded value; 8 bf16 per
// thread per trip.  pre may alias x.
__global__ __launch_bounds__(kBlock) void bias_gelu_kernel(const u32x4_t* x, const u32x4_t* __restrict__ bias,
                                                         int64_t nvec, int64_t cvec, u32x4_t* pre,
                                                         u32x4_t* __restrict__ y) {
  const int64_t stride = int64_t(gridDim.x) * kBlock;
  // bias column of vector i, advanced with i (no 64-bit division per trip)
  const int64_t i0 = int64_t(blockIdx.x) * kBlock + threadIdx.x, step = stride % cvec;
  int64_t ci = i0 % cvec;
  for (int64_t i = i0; i < nvec; i += stride) {
    const u32x4_t a = x[i], b = bias[ci];
    ci += step;
    if (ci >= cvec) ci -= cvec;
    u32x4_t p, o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      p[j] = pack_bf16(lo16(a[j]) + lo16(b[j]), hi16(a[j]) + hi16(b[j]));
      o[j] = pack_bf16(gelu_tanh_f32(lo16(p[j])), gelu_tanh_f32(hi16(p[j])));
    }
    pre[i] = p;
    y[i] = o;
  }
}

// ---------------------------------------------------------------- row adds
// out[r, c] = a[r, c] (+ b[r, c]) (+ bias[c]), fp32 math, one rounding.
template <typename T>
__global__ __launch_bounds__(kBlock) void add_rows_kernel(const T* __restrict__ a, const T* __restrict__ b,
                                                        const T* __restrict__ bias, int64_t rows, int64_t cols,
                                                        T* __restrict__ out) {
  const int64_t n = rows * cols, stride = int64_t(gridDim.x) * kBlock;
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
    float v = ldf<T>(a, i);
    if (b) v += ldf<T>(b, i);
    if (bias) v += ldf<T>(bias, i % cols);
    stf<T>(out, i, v);
  }
}

// bf16, 8 columns per thread per trip (cols % 8 == 0, 16-byte aligned rows)
__global__ __launch_bounds__(kBlock) void add_rows_bf16x8_kernel(const u32x4_t* __restrict__ a,
                                                               const u32x4_t* __restrict__ b,
                                                               const u32x4_t* __restrict__ bias, int64_t nvec,
                                                               int64_t cvec, u32x4_t* __restrict__ out) {
  const int64_t stride = int64_t(gridDim.x) * kBlock;
  // bias column of vector i, advanced with i (no 64-bit division per trip)
  const int64_t i0 = int64_t(blockIdx.x) * kBlock + threadIdx.x, step = stride % cvec;
  int64_t ci = i0 % cvec;
  for (int64_t i = i0; i < nvec; i += stride) {
    const u32x4_t x = a[i];
    const u32x4_t y = b ? b[i] : u32x4_t{0u, 0u, 0u, 0u};
    const u32x4_t z = bias ? bias[ci] : u32x4_t{0u, 0u, 0u, 0u};
    ci += step;
    if (ci >= cvec) ci -= cvec;
    u32x4_t o;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o[j] = pack_bf16(lo16(x[j]) + lo16(y[j]) + lo16(z[j]), hi16(x[j]) + hi16(y[j]) + hi16(z[j]));
    out[i] = o;
  }
}

inline unsigned grid_for(int64_t n, int64_t per_block = kBlock) {
  return unsigned(std::min<int64_t>((n + per_block - 1) / per_block, 65536));
}

}  // namespace
}  // namespace mk

using namespace mk;

extern "C" int mk_gelu_tanh_bwd(void* stream, int io_type, int64_t n, const void* x, const void* dy, void* dx) {
  clear_error();
  if (n < 0) return fail(MK_ERR_INVALID, "mk_gelu_tanh_bwd: negative n");
  if (n == 0) return MK_OK;
  if (!x || !dy || !dx) return fail(MK_ERR_INVALID, "mk_gelu_tanh_bwd: null pointer");
  hipStream_t s = as_stream(stream);
  if (io_type == MK_BF16) {
    const bool vec = (n % 8) == 0 && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(dy) |
                                       reinterpret_cast<uintptr_t>(dx)) & 15) == 0;
    if (vec)
      hipLaunchKernelGGL(gelu_bwd_bf16x8_kernel, dim3(grid_for(n / 8)), dim3(kBlock), 0, s, (const u32x4_t*)x,
                         (const u32x4_t*)dy, (u32x4_t*)dx, n / 8);
    else
      hipLaunchKernelGGL(gelu_bwd_kernel<uint16_t>, dim3(grid_for(n)), dim3(kBlock), 0, s, (const uint16_t*)x,
                         (const uint16_t*)dy, (uint16_t*)dx, n);
  } else if (io_type == MK_F32) {
    hipLaunchKernelGGL(gelu_bwd_kernel<float>, dim3(grid_for(n)), dim3(kBlock), 0, s, (const float*)x,
                       (const float*)dy, (float*)dx, n);
  } else {
    return fail(MK_ERR_UNSUPPORTED, "mk_gelu_tanh_bwd: io_type must be bf16/f32");
  }
  return check_launch("mk_gelu_tanh_bwd");
}

extern "C" size_t mk_col_sum_workspace_bytes(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  return size_t(align256(col_parts(rows) * cols * 4));
}

namespace {
// rows of `cols` elements of T as whole 16-byte vectors at every row start
template <typename T>
bool rows_are_vectors(int64_t cols, std::initializer_list<const void*> ptrs) {
  uintptr_t al = 0;
  for (const void* p : ptrs) al |= reinterpret_cast<uintptr_t>(p);
  return (cols * int64_t(sizeof(T))) % 16 == 0 && (al & 15) == 0;
}

template <typename T>
int col_sum_launch(hipStream_t s, int64_t rows, int64_t cols, const T* x, float* y, float* part) {
  const int64_t np = col_parts(rows), rpb = (rows + np - 1) / np, nb = (rows + rpb - 1) / rpb;
  if (rows_are_vectors<T>(cols, {x})) {
    constexpr int64_t BC = 64 * RowVec<T>::NV;
    const dim3 g(unsigned(nb), unsigned((cols + BC - 1) / BC));
    if (g.y > 65535) return fail(MK_ERR_UNSUPPORTED, "mk_col_sum: too many columns");
    hipLaunchKernelGGL(col_partial_vec_kernel<T>, g, dim3(kBlock), 0, s, x, rows, cols, rpb, part);
  } else {
    const dim3 g(unsigned(nb), unsigned((cols + kColChunk - 1) / kColChunk));
    if (g.y > 65535) return fail(MK_ERR_UNSUPPORTED, "mk_col_sum: too many columns");
    hipLaunchKernelGGL(col_partial_kernel<T>, g, dim3(kBlock), 0, s, x, rows, cols, rpb, part);
  }
  if (int rc = check_launch("mk_col_sum")) return rc;
  const float* parts[1] = {part};
  float* outs[1] = {y};
  return col_final(s, 1, parts, outs, nb, cols);
}
}  // namespace

extern "C" int mk_col_sum(void* stream, int in_type, int64_t rows, int64_t cols, const void* x, float* y,
                          void* workspace) {
  clear_error();
  if (rows < 0 || cols < 0) return fail(MK_ERR_INVALID, "mk_col_sum: negative shape");
  if (cols == 0) return MK_OK;
  if (!y) return fail(MK_ERR_INVALID, "mk_col_sum: null output");
  hipStream_t s = as_stream(stream);
  if (rows == 0) return mk_fill(stream, 4, cols, 0, y);
  if (!x || !workspace) return fail(MK_ERR_INVALID, "mk_col_sum: null input or workspace");
  float* part = static_cast<float*>(workspace);
  if (in_type == MK_BF16) return col_sum_launch(s, rows, cols, static_cast<const uint16_t*>(x), y, part);
  if (in_type == MK_F32) return col_sum_launch(s, rows, cols, static_cast<const float*>(x), y, part);
  return fail(MK_ERR_UNSUPPORTED, "mk_col_sum: in_type must be bf16/f32");
}

extern "C" int mk_gelu_tanh_bwd_colsum(void* stream, int io_type, int64_t rows, int64_t cols, const void* x,
                                       const void* dy, void* dx, float* dx_colsum, void* workspace) {
  clear_error();
  if (rows < 0 || cols < 0) return fail(MK_ERR_INVALID, "mk_gelu_tanh_bwd_colsum: negative shape");
  if (cols == 0) return MK_OK;
  if (!dx_colsum) return fail(MK_ERR_INVALID, "mk_gelu_tanh_bwd_colsum: null column-sum output");
  if (rows == 0) return mk_fill(stream, 4, cols, 0, dx_colsum);
  if (!x || !dy || !dx || !workspace) return fail(MK_ERR_INVALID, "mk_gelu_tanh_bwd_colsum: null pointer");
  if (io_type != MK_BF16 && io_type != MK_F32)
    return fail(MK_ERR_UNSUPPORTED, "mk_gelu_tanh_bwd_colsum: io_type must be bf16/f32");
  hipStream_t s = as_stream(stream);
  float* part = static_cast<float*>(workspace);
  auto run = [&](auto tag) -> int {
    using T = decltype(tag);
    if (!rows_are_vectors<T>(cols, {x, dy, dx})) {  // two passes: elementwise, then the column sum of dx
      if (int rc = mk_gelu_tanh_bwd(stream, io_type, rows * cols, x, dy, dx)) return rc;
      return col_sum_launch(s, rows, cols, static_cast<const T*>(dx), dx_colsum, part);
    }
    const int64_t np = col_parts(rows), rpb = (rows + np - 1) / np, nb = (rows + rpb - 1) / rpb;
    constexpr int64_t BC = 64 * RowVec<T>::NV;
    const dim3 g(unsigned(nb), unsigned((cols + BC - 1) / BC));
    if (g.y > 65535) return fail(MK_ERR_UNSUPPORTED, "mk_gelu_tanh_bwd_colsum: too many columns");
    hipLaunchKernelGGL(gelu_bwd_cols_kernel<T>, g, dim3(kBlock), 0, s, static_cast<const T*>(x),
                       static_cast<const T*>(dy), static_cast<T*>(dx), rows, cols, rpb, part);
    if (int rc = check_launch("mk_gelu_tanh_bwd_colsum")) return rc;
    const float* parts[1] = {part};
    float* outs[1] = {dx_colsum};
    return col_final(s, 1, parts, outs, nb, cols);
  };
  return io_type == MK_BF16 ? run(uint16_t{}) : run(float{});
}

extern "C" size_t mk_layernorm_bwd_workspace_bytes(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  return size_t(3 * align256(kLnBwdBlocks * cols * 4));
}

namespace {
int layernorm_bwd(void* stream, int io_type, int64_t rows, int64_t cols, const void* x, const void* gamma,
                  const void* dy, const void* dres, float eps, void* dx, void* dx_bf16, float* dgamma, float* dbeta,
                  float* dx_colsum, void* workspace);
}

extern "C" int mk_layernorm_bwd(void* stream, int io_type, int64_t rows, int64_t cols, const void* x,
                                const void* gamma, const void* dy, const void* dres, float eps, void* dx,
                                float* dgamma, float* dbeta, float* dx_colsum, void* workspace) {
  return layernorm_bwd(stream, io_type, rows, cols, x, gamma, dy, dres, eps, dx, nullptr, dgamma, dbeta, dx_colsum,
                       workspace);
}

extern "C" int mk_layernorm_bwd_typed(void* stream, int io_type, int64_t rows, int64_t cols, const void* x,
                                      const void* gamma, const void* dy, const void* dres, float eps, void* dx,
                                      void* dx_bf16, float* dgamma, float* dbeta, float* dx_colsum,
                                      void* workspace) {
  if (dx_bf16 && io_type != MK_F32) {
    clear_error();
    return fail(MK_ERR_UNSUPPORTED, "mk_layernorm_bwd_typed: a bf16 copy of dx is for fp32 rows");
  }
  return layernorm_bwd(stream, io_type, rows, cols, x, gamma, dy, dres, eps, dx, dx_bf16, dgamma, dbeta, dx_colsum,
                       workspace);
}

namespace {
int layernorm_bwd(void* stream, int io_type, int64_t rows, int64_t cols, const void* x, const void* gamma,
                  const void* dy, const void* dres, float eps, void* dx, void* dx_bf16, float* dgamma, float* dbeta,
                  float* dx_colsum, void* workspace) {
  clear_error();
  if (rows < 0 || cols <= 0) return fail(MK_ERR_INVALID, "mk_layernorm_bwd: bad shape");
  if (cols > kLnBwdMaxCols) return fail(MK_ERR_UNSUPPORTED, "mk_layernorm_bwd: rows of at most 2048 columns");
  if ((dgamma == nullptr) != (dbeta == nullptr))
    return fail(MK_ERR_INVALID, "mk_layernorm_bwd: dgamma and dbeta are both given or both NULL");
  if (io_type != MK_BF16 && io_type != MK_F32)
    return fail(MK_ERR_UNSUPPORTED, "mk_layernorm_bwd: io_type must be bf16/f32");
  if (rows == 0) {
    if (dgamma) {
      if (int rc = mk_fill(stream, 4, cols, 0, dgamma)) return rc;
      if (int rc = mk_fill(stream, 4, cols, 0, dbeta)) return rc;
    }
    if (dx_colsum) return mk_fill(stream, 4, cols, 0, dx_colsum);
    return MK_OK;
  }
  if (!x || !dy || !dx || ((dgamma || dx_colsum) && !workspace))
    return fail(MK_ERR_INVALID, "mk_layernorm_bwd: null pointer");
  hipStream_t s = as_stream(stream);
  const int64_t np = std::min<int64_t>(kLnBwdBlocks, std::max<int64_t>(1, (rows + 15) / 16));
  const int64_t rpb = (rows + np - 1) / np, nb = (rows + rpb - 1) / rpb;
  const int64_t slab = align256(kLnBwdBlocks * cols * 4);
  char* ws = static_cast<char*>(workspace);
  LnBwdArgs a;
  a.x = x; a.gamma = gamma; a.dy = dy; a.dres = dres; a.dx = dx;
  a.dx16 = static_cast<uint16_t*>(dx_bf16);
  a.rows = rows; a.rpb = rpb; a.cols = int(cols); a.eps = eps;
  a.part_g = dgamma ? reinterpret_cast<float*>(ws) : nullptr;
  a.part_b = dgamma ? reinterpret_cast<float*>(ws + slab) : nullptr;
  a.part_s = dx_colsum ? reinterpret_cast<float*>(ws + 2 * slab) : nullptr;
  auto launch = [&](auto tag, auto kvt, auto vect) {
    using T = decltype(tag);
    constexpr int KV = decltype(kvt)::value;
    constexpr bool VEC = decltype(vect)::value;
    hipLaunchKernelGGL((layernorm_bwd_kernel<T, RowVec<T>, KV, VEC, kRowLanes>), dim3(unsigned(nb)), dim3(kBlock), 0, s, a);
  };
  // bf16 rows of at most 1024 columns in 8-byte vectors: fewer registers per
  // lane (more rows in flight) and no idle lanes at 768 columns
  const uintptr_t al8 = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(dy) |
                        reinterpret_cast<uintptr_t>(dres) | reinterpret_cast<uintptr_t>(dx);
  if (io_type == MK_BF16 && cols % 4 == 0 && cols <= 1024 && (al8 & 7) == 0) {
    const int64_t kv = (cols + 255) / 256;
    auto go = [&](auto kvt) {
      constexpr int KV = decltype(kvt)::value;
      hipLaunchKernelGGL((layernorm_bwd_kernel<uint16_t, Bf16x4, KV, true, kRowLanes, true>), dim3(unsigned(nb)),
                         dim3(kBlock), 0, s, a);
    };
    if (kv == 1) go(IntC<1>{});
    else if (kv == 2) go(IntC<2>{});
    else if (kv == 3) go(IntC<3>{});
    else go(IntC<4>{});
  } else {
    auto dispatch = [&](auto tag) {
    using T = decltype(tag);
    constexpr int NV = RowVec<T>::NV;
    const int64_t kv = (cols + 64 * NV - 1) / (64 * NV);
    auto with_kv = [&](auto vect) {
      if (kv == 1) launch(tag, IntC<1>{}, vect);
      else if (kv == 2) launch(tag, IntC<2>{}, vect);
      else if (kv == 3 && NV == 4 && decltype(vect)::value) launch(tag, IntC<3>{}, vect);  // fp32 rows of 768
      else if (kv <= 4) launch(tag, IntC<4>{}, vect);
      else if constexpr (NV == 4) launch(tag, IntC<8>{}, vect);  // fp32 only: bf16 rows fit KV 4
    };
    if (rows_are_vectors<T>(cols, {x, dy, dres, dx}) && (reinterpret_cast<uintptr_t>(dx_bf16) & 7u) == 0)
      with_kv(std::true_type{});
    else with_kv(std::false_type{});
    };
    if (io_type == MK_BF16) dispatch(uint16_t{});
    else dispatch(float{});
  }
  if (int rc = check_launch("mk_layernorm_bwd")) return rc;
  const float* parts[3];
  float* outs[3];
  int n = 0;
  if (dgamma) {
    parts[n] = a.part_g; outs[n++] = dgamma;
    parts[n] = a.part_b; outs[n++] = dbeta;
  }
  if (dx_colsum) {
    parts[n] = a.part_s; outs[n++] = dx_colsum;
  }
  return n ? col_final(s, n, parts, outs, nb, cols) : MK_OK;
}
}  // namespace

namespace {
// The cross-entropy kernels for rows `ld_in` / `ld_out` elements apart.
int xent_launch(void* stream, int logits_type, int dlogits_type, int64_t rows, int64_t cols, const void* logits,
                int64_t ld_in, int label_type, const void* labels, float grad_scale, float* loss_rows, void* dlogits,
                int64_t ld_out, const char* what) {
  clear_error();
  if (rows < 0 || cols <= 0) return fail(MK_ERR_INVALID, std::string(what) + ": bad shape");
  if (rows == 0) return MK_OK;
  if (rows >= (int64_t(1) << 31)) return fail(MK_ERR_UNSUPPORTED, std::string(what) + ": too many rows");
  if (!logits || !labels || !dlogits) return fail(MK_ERR_INVALID, std::string(what) + ": null pointer");
  if (ld_in < cols || ld_out < cols) return fail(MK_ERR_INVALID, std::string(what) + ": row pitch below cols");
  if (label_type != MK_S32 && label_type != MK_S64)
    return fail(MK_ERR_UNSUPPORTED, std::string(what) + ": labels must be s32/s64");
  const bool s32 = label_type == MK_S32;
  hipStream_t s = as_stream(stream);
  const dim3 g{unsigned(rows)};
  if (logits_type == MK_F32 && dlogits_type == MK_BF16) {
    // rows 16-byte aligned: the vector kernel; otherwise one element per load
    const bool vec = (reinterpret_cast<uintptr_t>(logits) & 15u) == 0 && ld_in % 4 == 0 &&
                     (reinterpret_cast<uintptr_t>(dlogits) & 7u) == 0 && ld_out % 4 == 0;
    const int64_t nvt = ((cols + 3) / 4 + kXentF32Threads - 1) / kXentF32Threads;  // vectors per thread
    auto vlaunch = [&](auto nt) {
      constexpr int NV = decltype(nt)::value;
      if (s32)
        hipLaunchKernelGGL((softmax_xent_f32_bf16_vec_kernel<NV, int32_t>), g, dim3(kXentF32Threads), 0, s,
                           (const float*)logits, cols, ld_in, (const int32_t*)labels, grad_scale, loss_rows,
                           (uint16_t*)dlogits, ld_out);
      else
        hipLaunchKernelGGL((softmax_xent_f32_bf16_vec_kernel<NV, int64_t>), g, dim3(kXentF32Threads), 0, s,
                           (const float*)logits, cols, ld_in, (const int64_t*)labels, grad_scale, loss_rows,
                           (uint16_t*)dlogits, ld_out);
    };
    const int64_t npt = (cols + kXentF32Threads - 1) / kXentF32Threads;
    auto launch = [&](auto nt) {
      constexpr int NPT = decltype(nt)::value;
      if (s32)
        hipLaunchKernelGGL((softmax_xent_f32_bf16_kernel<NPT, int32_t>), g, dim3(kXentF32Threads), 0, s,
                           (const float*)logits, cols, ld_in, (const int32_t*)labels, grad_scale, loss_rows,
                           (uint16_t*)dlogits, ld_out);
      else
        hipLaunchKernelGGL((softmax_xent_f32_bf16_kernel<NPT, int64_t>), g, dim3(kXentF32Threads), 0, s,
                           (const float*)logits, cols, ld_in, (const int64_t*)labels, grad_scale, loss_rows,
                           (uint16_t*)dlogits, ld_out);
    };
    if (vec && nvt <= 4) vlaunch(IntC<4>{});
    else if (vec && nvt <= 8) vlaunch(IntC<8>{});
    else if (vec && nvt <= 12) vlaunch(IntC<12>{});
    else if (vec && nvt <= 16) vlaunch(IntC<16>{});
    else if (npt <= 8) launch(IntC<8>{});
    else if (npt <= 16) launch(IntC<16>{});
    else if (npt <= 24) launch(IntC<24>{});
    else if (s32)
      hipLaunchKernelGGL((softmax_xent_f32_bf16_stream_kernel<16, int32_t>), g, dim3(kXentF32Threads), 0, s,
                         (const float*)logits, cols, ld_in, (const int32_t*)labels, grad_scale, loss_rows,
                         (uint16_t*)dlogits, ld_out);
    else
      hipLaunchKernelGGL((softmax_xent_f32_bf16_stream_kernel<16, int64_t>), g, dim3(kXentF32Threads), 0, s,
                         (const float*)logits, cols, ld_in, (const int64_t*)labels, grad_scale, loss_rows,
                         (uint16_t*)dlogits, ld_out);
    return check_launch(what);
  }
  if (logits_type != dlogits_type || (logits_type != MK_BF16 && logits_type != MK_F32))
    return fail(MK_ERR_UNSUPPORTED, std::string(what) + ": logits / dlogits types must be bf16/bf16, f32/f32 or f32/bf16");
  // bf16 rows of up to 64K columns: the register-resident kernel.  It takes
  // the unaligned head of a row from the logits' 16-byte phase and stores
  // dlogits with 16-byte vectors at the same offsets, so every row of both
  // must share that phase; otherwise the element-wise kernel below runs.
  const bool same_phase =
      ((reinterpret_cast<uintptr_t>(logits) ^ reinterpret_cast<uintptr_t>(dlogits)) & 15u) == 0 &&
      (ld_in - ld_out) % 8 == 0;
  if (logits_type == MK_BF16 && same_phase && cols <= int64_t(kXentThreads) * 8 * 16) {
    const int64_t nvt = (cols / 8 + kXentThreads - 1) / kXentThreads;  // vectors per thread (bound)
    auto launch = [&](auto nt, auto ltag) {
      constexpr int NVT = decltype(nt)::value;
      using L = decltype(ltag);
      hipLaunchKernelGGL((softmax_xent_bf16_kernel<NVT, L>), g, dim3(kXentThreads), 0, s, (const uint16_t*)logits,
                         cols, ld_in, (const L*)labels, grad_scale, loss_rows, (uint16_t*)dlogits, ld_out);
    };
    auto with_labels = [&](auto nt) {
      if (s32) launch(nt, int32_t{});
      else launch(nt, int64_t{});
    };
    if (nvt <= 4) with_labels(IntC<4>{});
    else if (nvt <= 8) with_labels(IntC<8>{});
    else with_labels(IntC<16>{});
    return check_launch(what);
  }
  auto go = [&](auto tag) {
    using T = decltype(tag);
    if (s32)
      hipLaunchKernelGGL((softmax_xent_kernel<T, int32_t>), g, dim3(kBlock), 0, s, (const T*)logits, cols, ld_in,
                         (const int32_t*)labels, grad_scale, loss_rows, (T*)dlogits, ld_out);
    else
      hipLaunchKernelGGL((softmax_xent_kernel<T, int64_t>), g, dim3(kBlock), 0, s, (const T*)logits, cols, ld_in,
                         (const int64_t*)labels, grad_scale, loss_rows, (T*)dlogits, ld_out);
  };
  if (logits_type == MK_BF16) go(uint16_t{});
  else go(float{});
  return check_launch(what);
}
}  // namespace

extern "C" int mk_softmax_xent_strided(void* stream, int logits_type, int dlogits_type, int64_t rows, int64_t cols,
                                       const void* logits, int64_t ld_logits, int label_type, const void* labels,
                                       float grad_scale, float* loss_rows, void* dlogits, int64_t ld_dlogits) {
  return xent_launch(stream, logits_type, dlogits_type, rows, cols, logits, ld_logits, label_type, labels, grad_scale,
                     loss_rows, dlogits, ld_dlogits, "mk_softmax_xent_strided");
}

extern "C" int mk_softmax_xent_typed(void* stream, int logits_type, int dlogits_type, int64_t rows, int64_t cols,
                                     const void* logits, int label_type, const void* labels, float grad_scale,
                                     float* loss_rows, void* dlogits) {
  if (logits_type != dlogits_type && (logits_type != MK_F32 || dlogits_type != MK_BF16)) {
    clear_error();
    return fail(MK_ERR_UNSUPPORTED, "mk_softmax_xent_typed: mixed types need f32 logits and bf16 dlogits");
  }
  return xent_launch(stream, logits_type, dlogits_type, rows, cols, logits, cols, label_type, labels, grad_scale,
                     loss_rows, dlogits, cols, "mk_softmax_xent_typed");
}

extern "C" int mk_softmax_xent(void* stream, int io_type, int64_t rows, int64_t cols, const void* logits,
                               int label_type, const void* labels, float grad_scale, float* loss_rows,
                               void* dlogits) {
  if (io_type != MK_BF16 && io_type != MK_F32) {
    clear_error();
    return fail(MK_ERR_UNSUPPORTED, "mk_softmax_xent: io_type must be bf16/f32");
  }
  return xent_launch(stream, io_type, io_type, rows, cols, logits, cols, label_type, labels, grad_scale, loss_rows,
                     dlogits, cols, "mk_softmax_xent");
}

namespace {
int adam_launch(void* stream, int64_t n, int param_type, void* param, float* master, int grad_type, const void* grad,
                float* m, float* v, double lr, double b1, double b2, double eps, double bc1, double bc2,
                const float* hyper) {
  if (n < 0) return fail(MK_ERR_INVALID, "mk_adam_update: negative n");
  if (n == 0) return MK_OK;
  if (!param || !grad || !m || !v) return fail(MK_ERR_INVALID, "mk_adam_update: null pointer");
  float* p32;
  uint16_t* p16 = nullptr;
  if (master) {
    if (param_type != MK_BF16) return fail(MK_ERR_UNSUPPORTED, "mk_adam_update: a master copy needs a bf16 param");
    p32 = master;
    p16 = static_cast<uint16_t*>(param);
  } else {
    if (param_type != MK_F32) return fail(MK_ERR_UNSUPPORTED, "mk_adam_update: without a master copy the param is f32");
    p32 = static_cast<float*>(param);
  }
  hipStream_t s = as_stream(stream);
  const dim3 g(grid_for(n)), b(kBlock);
  const float f_lr = float(lr), f_b1 = float(b1), f_omb1 = float(1.0 - b1), f_b2 = float(b2),
              f_omb2 = float(1.0 - b2), f_eps = float(eps), f_bc1 = float(bc1), f_bc2 = float(bc2);
  const uintptr_t al = reinterpret_cast<uintptr_t>(p32) | reinterpret_cast<uintptr_t>(grad) |
                       reinterpret_cast<uintptr_t>(m) | reinterpret_cast<uintptr_t>(v);
  if (grad_type == MK_F32 && n % 4 == 0 && (al & 15) == 0 && (reinterpret_cast<uintptr_t>(p16) & 7) == 0)
    hipLaunchKernelGGL(adam_vec4_kernel, dim3(grid_for(n / 4)), b, 0, s, n / 4, (f32x4*)p32, (uint2*)p16,
                       (const f32x4*)grad, (f32x4*)m, (f32x4*)v, f_lr, f_b1, f_omb1, f_b2, f_omb2, f_eps, f_bc1,
                       f_bc2, hyper);
  else if (grad_type == MK_F32)
    hipLaunchKernelGGL(adam_kernel<float>, g, b, 0, s, n, p32, p16, (const float*)grad, m, v, f_lr, f_b1, f_omb1,
                       f_b2, f_omb2, f_eps, f_bc1, f_bc2, hyper);
  else if (grad_type == MK_BF16)
    hipLaunchKernelGGL(adam_kernel<uint16_t>, g, b, 0, s, n, p32, p16, (const uint16_t*)grad, m, v, f_lr, f_b1,
                       f_omb1, f_b2, f_omb2, f_eps, f_bc1, f_bc2, hyper);
  else
    return fail(MK_ERR_UNSUPPORTED, "mk_adam_update: grad_type must be bf16/f32");
  return check_launch("mk_adam_update");
}
}  // namespace

extern "C" int mk_adam_update(void* stream, int64_t n, int param_type, void* param, float* master, int grad_type,
                              const void* grad, float* m, float* v, double lr, double b1, double b2, double eps,
                              double bc1, double bc2) {
  clear_error();
  return adam_launch(stream, n, param_type, param, master, grad_type, grad, m, v, lr, b1, b2, eps, bc1, bc2, nullptr);
}

extern "C" int mk_adam_update_dev(void* stream, int64_t n, int param_type, void* param, float* master,
                                  int grad_type, const void* grad, float* m, float* v, const float* hyper, double b1,
                                  double b2, double eps) {
  clear_error();
  if (!hyper) return fail(MK_ERR_INVALID, "mk_adam_update_dev: null hyperparameter pointer");
  return adam_launch(stream, n, param_type, param, master, grad_type, grad, m, v, 0.0, b1, b2, eps, 1.0, 1.0, hyper);
}

extern "C" size_t mk_sdpa_bwd_workspace_bytes(int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D) {
  if (B <= 0 || H <= 0 || Sq <= 0 || Sk <= 0) return 0;
  if (D == 64 || D == 128) return sdpa_bwd_flash_workspace(B, H, Sq);
  const int64_t n = B * H * Sq * Sk;
  return size_t(align256(n * 4) + align256(n * 2) + align256(B * H * Sq * 4));
}

extern "C" int mk_sdpa_bwd(void* stream, int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D,
                           const void* q, int64_t q_bs, int64_t q_hs, int64_t q_ss,
                           const void* k, int64_t k_bs, int64_t k_hs, int64_t k_ss,
                           const void* v, int64_t v_bs, int64_t v_hs, int64_t v_ss,
                           const void* o, int64_t o_bs, int64_t o_hs, int64_t o_ss,
                           const void* dout, int64_t do_bs, int64_t do_hs, int64_t do_ss,
                           const float* lse,
                           void* dq, int64_t dq_bs, int64_t dq_hs, int64_t dq_ss,
                           void* dk, int64_t dk_bs, int64_t dk_hs, int64_t dk_ss,
                           void* dv, int64_t dv_bs, int64_t dv_hs, int64_t dv_ss,
                           float scale, int causal, void* workspace) {
  clear_error();
  if (B < 0 || H < 0 || Sq < 0 || Sk < 0) return fail(MK_ERR_INVALID, "mk_sdpa_bwd: negative shape");
  if (D <= 0 || D % 8 != 0 || D > 256) return fail(MK_ERR_UNSUPPORTED, "mk_sdpa_bwd: head_dim must be a multiple of 8, <= 256");
  if (B == 0 || H == 0 || Sq == 0 || Sk == 0) return MK_OK;
  if (!q || !k || !v || !o || !dout || !lse || !dq || !dk || !dv || !workspace)
    return fail(MK_ERR_INVALID, "mk_sdpa_bwd: null pointer");
  if (D == 64 || D == 128)
    return sdpa_bwd_flash(as_stream(stream), B, H, Sq, Sk, D, q, q_bs, q_hs, q_ss, k, k_bs, k_hs, k_ss, v, v_bs, v_hs,
                          v_ss, o, o_bs, o_hs, o_ss, dout, do_bs, do_hs, do_ss, lse, dq, dq_bs, dq_hs, dq_ss, dk, dk_bs,
                          dk_hs, dk_ss, dv, dv_bs, dv_hs, dv_ss, scale, causal, workspace);
  const uintptr_t al = reinterpret_cast<uintptr_t>(o) | reinterpret_cast<uintptr_t>(dout);
  if ((al & 15) != 0 || ((o_bs | o_hs | o_ss | do_bs | do_hs | do_ss) & 7) != 0)
    return fail(MK_ERR_UNSUPPORTED, "mk_sdpa_bwd: o and dO rows must be 16-byte aligned");
  hipStream_t s = as_stream(stream);
  const int64_t n = B * H * Sq * Sk;
  float* F = static_cast<float*>(workspace);  // scores, then dP
  uint16_t* P = reinterpret_cast<uint16_t*>(static_cast<char*>(workspace) + align256(n * 4));  // P, then dS
  float* Dsum = reinterpret_cast<float*>(static_cast<char*>(workspace) + align256(n * 4) + align256(n * 2));
  const int64_t nrows = B * H * Sq;
  hipLaunchKernelGGL(attn_rowdot_kernel, dim3(unsigned((nrows + kBlock - 1) / kBlock)), dim3(kBlock), 0, s,
                     (const uint16_t*)o, o_bs, o_hs, o_ss, (const uint16_t*)dout, do_bs, do_hs, do_ss, H, Sq, D,
                     nrows, Dsum);
  if (int rc = check_launch("mk_sdpa_bwd")) return rc;
  const int64_t SS = Sq * Sk;
  // per batch index: H heads as one batched GEMM (head stride), S / dP rows of Sk
  for (int64_t b = 0; b < B; ++b) {
    const uint16_t* qb = static_cast<const uint16_t*>(q) + b * q_bs;
    const uint16_t* kb = static_cast<const uint16_t*>(k) + b * k_bs;
    float* Fb = F + b * H * SS;
    // S = Q Kᵀ  [Sq x Sk], fp32
    if (int rc = gemm_blas(s, MK_BF16, MK_F32, H, Sq, Sk, D, qb, q_hs, q_ss, 1, kb, k_hs, 1, k_ss, Fb, SS, Sk, 1.f, 0.f))
      return rc;
  }
  hipLaunchKernelGGL(attn_probs_kernel, dim3(grid_for(n)), dim3(kBlock), 0, s, F, lse, Sq, Sk, scale, causal, P, n);
  if (int rc = check_launch("mk_sdpa_bwd")) return rc;
  for (int64_t b = 0; b < B; ++b) {
    const uint16_t* db = static_cast<const uint16_t*>(dout) + b * do_bs;
    const uint16_t* vb = static_cast<const uint16_t*>(v) + b * v_bs;
    const uint16_t* Pb = P + b * H * SS;
    float* Fb = F + b * H * SS;
    // dV = Pᵀ dO  [Sk x D]
    if (int rc = gemm_blas(s, MK_BF16, MK_BF16, H, Sk, D, Sq, Pb, SS, 1, Sk, db, do_hs, do_ss, 1,
                           static_cast<uint16_t*>(dv) + b * dv_bs, dv_hs, dv_ss, 1.f, 0.f))
      return rc;
    // dP = dO Vᵀ  [Sq x Sk], fp32 (over the scores)
    if (int rc = gemm_blas(s, MK_BF16, MK_F32, H, Sq, Sk, D, db, do_hs, do_ss, 1, vb, v_hs, 1, v_ss, Fb, SS, Sk, 1.f, 0.f))
      return rc;
  }
  hipLaunchKernelGGL(attn_dscores_kernel, dim3(grid_for(n)), dim3(kBlock), 0, s, F, Dsum, Sk, scale, P, n);
  if (int rc = check_launch("mk_sdpa_bwd")) return rc;
  for (int64_t b = 0; b < B; ++b) {
    const uint16_t* qb = static_cast<const uint16_t*>(q) + b * q_bs;
    const uint16_t* kb = static_cast<const uint16_t*>(k) + b * k_bs;
    const uint16_t* Pb = P + b * H * SS;
    // dQ = dS K  [Sq x D]
    if (int rc = gemm_blas(s, MK_BF16, MK_BF16, H, Sq, D, Sk, Pb, SS, Sk, 1, kb, k_hs, k_ss, 1,
                           static_cast<uint16_t*>(dq) + b * dq_bs, dq_hs, dq_ss, 1.f, 0.f))
      return rc;
    // dK = dSᵀ Q  [Sk x D]
    if (int rc = gemm_blas(s, MK_BF16, MK_BF16, H, Sk, D, Sq, Pb, SS, 1, Sk, qb, q_hs, q_ss, 1,
                           static_cast<uint16_t*>(dk) + b * dk_bs, dk_hs, dk_ss, 1.f, 0.f))
      return rc;
  }
  return MK_OK;
}

extern "C" int mk_add_rows(void* stream, int io_type, int64_t rows, int64_t cols, const void* a, const void* b,
                           const void* bias, void* out) {
  clear_error();
  if (rows < 0 || cols < 0) return fail(MK_ERR_INVALID, "mk_add_rows: negative shape");
  if (rows == 0 || cols == 0) return MK_OK;
  if (!a || !out) return fail(MK_ERR_INVALID, "mk_add_rows: null pointer");
  hipStream_t s = as_stream(stream);
  const int64_t n = rows * cols;
  if (io_type == MK_BF16) {
    const uintptr_t al = reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
                         reinterpret_cast<uintptr_t>(bias) | reinterpret_cast<uintptr_t>(out);
    if (cols % 8 == 0 && (al & 15) == 0)
      hipLaunchKernelGGL(add_rows_bf16x8_kernel, dim3(grid_for(n / 8)), dim3(kBlock), 0, s, (const u32x4_t*)a,
                         (const u32x4_t*)b, (const u32x4_t*)bias, n / 8, cols / 8, (u32x4_t*)out);
    else
      hipLaunchKernelGGL(add_rows_kernel<uint16_t>, dim3(grid_for(n)), dim3(kBlock), 0, s, (const uint16_t*)a,
                         (const uint16_t*)b, (const uint16_t*)bias, rows, cols, (uint16_t*)out);
  } else if (io_type == MK_F32) {
    hipLaunchKernelGGL(add_rows_kernel<float>, dim3(grid_for(n)), dim3(kBlock), 0, s, (const float*)a,
                       (const float*)b, (const float*)bias, rows, cols, (float*)out);
  } else {
    return fail(MK_ERR_UNSUPPORTED, "mk_add_rows: io_type must be bf16/f32");
  }
  return check_launch("mk_add_rows");
}

extern "C" int mk_add_layernorm(void* stream, int64_t rows, int64_t cols, const void* a, const void* b,
                                const void* bias, const void* gamma, const void* beta, float eps, void* sum_out,
                                void* y) {
  clear_error();
  if (rows < 0 || cols <= 0) return fail(MK_ERR_INVALID, "mk_add_layernorm: bad shape");
  if (rows == 0) return MK_OK;
  if (!a || !sum_out || !y) return fail(MK_ERR_INVALID, "mk_add_layernorm: null pointer");
  if (cols % 4 != 0 || cols > 2048)
    return fail(MK_ERR_UNSUPPORTED, "mk_add_layernorm: cols must be a multiple of 4, at most 2048");
  const uintptr_t al = reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
                       reinterpret_cast<uintptr_t>(bias) | reinterpret_cast<uintptr_t>(gamma) |
                       reinterpret_cast<uintptr_t>(beta) | reinterpret_cast<uintptr_t>(sum_out) |
                       reinterpret_cast<uintptr_t>(y);
  if (al & 7) return fail(MK_ERR_UNSUPPORTED, "mk_add_layernorm: 8-byte aligned operands");
  hipStream_t s = as_stream(stream);
  const int cols4 = int(cols / 4), kv = (cols4 + 63) / 64;
  const dim3 g(unsigned((rows + 3) / 4));
  auto go = [&](auto kvt) {
    constexpr int KV = decltype(kvt)::value;
    hipLaunchKernelGGL((add_layernorm_kernel<KV>), g, dim3(kBlock), 0, s, (const uint2*)a, (const uint2*)b,
                       (const uint2*)bias, (const uint2*)gamma, (const uint2*)beta, rows, cols4, eps,
                       (uint2*)sum_out, (uint2*)y);
  };
  if (kv == 1) go(IntC<1>{});
  else if (kv == 2) go(IntC<2>{});
  else if (kv == 3) go(IntC<3>{});
  else if (kv == 4) go(IntC<4>{});
  else go(IntC<8>{});
  return check_launch("mk_add_layernorm");
}

extern "C" int mk_bias_gelu(void* stream, int64_t rows, int64_t cols, const void* x, const void* bias,
                            void* pre_out, void* y) {
  clear_error();
  if (rows < 0 || cols < 0) return fail(MK_ERR_INVALID, "mk_bias_gelu: negative shape");
  if (rows == 0 || cols == 0) return MK_OK;
  if (!x || !bias || !pre_out || !y) return fail(MK_ERR_INVALID, "mk_bias_gelu: null pointer");
  const uintptr_t al = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(bias) |
                       reinterpret_cast<uintptr_t>(pre_out) | reinterpret_cast<uintptr_t>(y);
  hipStream_t s = as_stream(stream);
  if (cols % 8 != 0 || (al & 15) != 0) {  // two passes: the bias add, then GELU of the stored sum
    if (int rc = mk_add_rows(stream, MK_BF16, rows, cols, x, nullptr, bias, pre_out)) return rc;
    return mk_gelu_tanh(stream, MK_BF16, rows * cols, pre_out, y);
  }
  const int64_t nvec = rows * cols / 8;
  hipLaunchKernelGGL(bias_gelu_kernel, dim3(grid_for(nvec)), dim3(kBlock), 0, s, (const u32x4_t*)x,
                     (const u32x4_t*)bias, nvec, cols / 8, (u32x4_t*)pre_out, (u32x4_t*)y);
  return check_launch("mk_bias_gelu");
}
