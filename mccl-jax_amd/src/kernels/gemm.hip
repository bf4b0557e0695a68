// Batched, strided GEMM on MFMA for dot_general: bf16 (fp32 accumulate) via
// v_mfma_f32_32x32x16_bf16 and true fp32 via v_mfma_f32_32x32x2_f32.
//
// Workgroup tile BM x BN = 128 x 128, 4 waves in a 2 x 2 arrangement, each
// wave 64 x 64 = 2 x 2 MFMA 32x32 blocks.  K advances in BK-deep tiles that
// are staged through LDS in a k-contiguous [row][k] layout (the layout both
// MFMA operands read 8 (bf16) or 1 (fp32) consecutive k from).  Operands that
// are m- / n-contiguous in HBM are transposed while being written to LDS, so
// dot_general never needs a separate transpose kernel (the reference
// materialises transposes, linalg.mm:34-45).  Global loads for tile k+1 are
// issued before tile k is multiplied (register double buffering).
#include "mk_common.h"

namespace mk {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kBM = 128, kBN = 128;

template <typename T> struct Cfg;
template <> struct Cfg<uint16_t> {  // bf16
  static constexpr int BK = 32;
  static constexpr int VEC = 8;       // elements per 16-byte chunk
  static constexpr int KSTEP = 16;    // k per MFMA
  static constexpr int LDS_STRIDE = BK + 8;
};
template <> struct Cfg<float> {
  static constexpr int BK = 32;  // 8 waves: 80.5 against 83.0 us for C1 at 16
  static constexpr int VEC = 4;
  static constexpr int KSTEP = 2;
  static constexpr int LDS_STRIDE = BK + 1;
};

struct GemmArgs {
  const void* A;
  const void* B;
  void* C;
  const void* bias;
  int64_t M, N, K;
  int64_t a_bs, a_ms, a_ks;
  int64_t b_bs, b_ks, b_ns;
  int64_t c_bs, c_ms;
  int tiles_n;
  int epilogue;
  int c_type;
  int vec_a, vec_b;  // 16-byte vector loads allowed along the contiguous dim
};

// Stage one operand tile (ROWS x BK, element (row, k) = src[row*rs + k*ks])
// into registers.  KC: the operand is k-contiguous (ks == 1); otherwise it
// is row-contiguous (rs == 1).
template <typename T, bool KC, int ROWS, int NT = kThreads>
struct TileLoader {
  using C = Cfg<T>;
  static constexpr int BK = C::BK, VEC = C::VEC;
  // k-contiguous: chunks of VEC along k.  row-contiguous: chunks of VEC rows
  // at one k, taken in pairs of k (bf16) so LDS writes are 32-bit.
  static constexpr int KPAIR = sizeof(T) == 2 ? 2 : 1;
  static constexpr int CHUNKS = KC ? ROWS * BK / VEC : (ROWS / VEC) * (BK / KPAIR);
  static constexpr int PER_T = CHUNKS / NT;
  static_assert(CHUNKS % NT == 0, "chunks must divide evenly");
  u32x4_t reg[PER_T][KPAIR];

  __device__ inline void load(const T* src, int64_t rs, int64_t ks, int64_t row0, int64_t rows,
                              int64_t k0, int64_t K, bool vec) {
    // Interior tile (the whole ROWS x BK block in range) with vector access:
    // every chunk is one 16-byte load, issued without a per-chunk bounds
    // branch.  (Loads inside such branches are each waited for before the
    // next is issued.)  The condition is uniform over the workgroup.
    if (vec && row0 + ROWS <= rows && k0 + BK <= K) {
#pragma unroll
      for (int i = 0; i < PER_T; ++i) {
        const int ch = threadIdx.x + i * NT;
        if constexpr (KC) {
          const int r = ch / (BK / VEC), kc = (ch % (BK / VEC)) * VEC;
          reg[i][0] = *reinterpret_cast<const u32x4_t*>(src + (row0 + r) * rs + (k0 + kc));
        } else {
          const int rc = (ch % (ROWS / VEC)) * VEC, kp = (ch / (ROWS / VEC)) * KPAIR;
#pragma unroll
          for (int q = 0; q < KPAIR; ++q)
            reg[i][q] = *reinterpret_cast<const u32x4_t*>(src + (k0 + kp + q) * ks + (row0 + rc));
        }
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      const int ch = threadIdx.x + i * NT;
      if constexpr (KC) {
        const int r = ch / (BK / VEC), kc = (ch % (BK / VEC)) * VEC;
        const int64_t gr = row0 + r, gk = k0 + kc;
        u32x4_t v = {0u, 0u, 0u, 0u};
        if (gr < rows) {
          if (vec && gk + VEC <= K) {
            v = *reinterpret_cast<const u32x4_t*>(src + gr * rs + gk);
          } else {
            T tmp[VEC];
#pragma unroll
            for (int e = 0; e < VEC; ++e) tmp[e] = (gk + e < K) ? src[gr * rs + gk + e] : T(0);
            __builtin_memcpy(&v, tmp, 16);
          }
        }
        reg[i][0] = v;
      } else {
        const int rc = (ch % (ROWS / VEC)) * VEC, kp = (ch / (ROWS / VEC)) * KPAIR;
        const int64_t gr = row0 + rc;
#pragma unroll
        for (int q = 0; q < KPAIR; ++q) {
          const int64_t gk = k0 + kp + q;
          u32x4_t v = {0u, 0u, 0u, 0u};
          if (gk < K) {
            if (vec && gr + VEC <= rows) {
              v = *reinterpret_cast<const u32x4_t*>(src + gk * ks + gr);
            } else {
              T tmp[VEC];
#pragma unroll
              for (int e = 0; e < VEC; ++e) tmp[e] = (gr + e < rows) ? src[gk * ks + gr + e] : T(0);
              __builtin_memcpy(&v, tmp, 16);
            }
          }
          reg[i][q] = v;
        }
      }
    }
  }

  __device__ inline void store(T* lds) const {
    constexpr int LS = C::LDS_STRIDE;
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      const int ch = threadIdx.x + i * NT;
      if constexpr (KC) {
        const int r = ch / (BK / VEC), kc = (ch % (BK / VEC)) * VEC;
        if constexpr (sizeof(T) == 2) {
          *reinterpret_cast<u32x4_t*>(lds + r * LS + kc) = reg[i][0];
        } else {
          const float* f = reinterpret_cast<const float*>(&reg[i][0]);
#pragma unroll
          for (int e = 0; e < VEC; ++e) lds[r * LS + kc + e] = f[e];
        }
      } else {
        const int rc = (ch % (ROWS / VEC)) * VEC, kp = (ch / (ROWS / VEC)) * KPAIR;
        if constexpr (sizeof(T) == 2) {
          const uint16_t* a0 = reinterpret_cast<const uint16_t*>(&reg[i][0]);
          const uint16_t* a1 = reinterpret_cast<const uint16_t*>(&reg[i][1]);
#pragma unroll
          for (int e = 0; e < VEC; ++e)
            *reinterpret_cast<uint32_t*>(lds + (rc + e) * LS + kp) = uint32_t(a0[e]) | (uint32_t(a1[e]) << 16);
        } else {
          const float* f = reinterpret_cast<const float*>(&reg[i][0]);
#pragma unroll
          for (int e = 0; e < VEC; ++e) lds[(rc + e) * LS + kp] = f[e];
        }
      }
    }
  }
};

// NW waves in an (NW / 2) x 2 arrangement: 4 waves of 64 x 64, or 8 waves of
// 32 x 64 (the fp32 products, where one 4-wave workgroup per CU left each
// SIMD a single wave to hide the loads behind).
template <typename T, bool A_KC, bool B_KC, int NW = 4>
__global__ __launch_bounds__(64 * NW, 8 / NW) void gemm_kernel(const GemmArgs p) {
  using C = Cfg<T>;
  constexpr int NT = 64 * NW;
  constexpr int MI = NW == 8 ? 1 : 2;  // 32-row MFMA blocks per wave
  constexpr int BK = C::BK, LS = C::LDS_STRIDE, KSTEP = C::KSTEP;
  __shared__ __attribute__((aligned(16))) T As[2][kBM * LS];
  __shared__ __attribute__((aligned(16))) T Bs[2][kBN * LS];

  const int tile = blockIdx.x;
  const int64_t m0 = int64_t(tile / p.tiles_n) * kBM;
  const int64_t n0 = int64_t(tile % p.tiles_n) * kBN;
  const int64_t bz = blockIdx.y;
  const T* A = reinterpret_cast<const T*>(p.A) + bz * p.a_bs;
  const T* B = reinterpret_cast<const T*>(p.B) + bz * p.b_bs;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 31, g = lane >> 5;
  const int wm = wave >> 1, wn = wave & 1;

  TileLoader<T, A_KC, kBM, NT> la;
  TileLoader<T, B_KC, kBN, NT> lb;
  // B element (n, k) = B[k*b_ks + n*b_ns]: rows are n
  const int64_t a_rs = p.a_ms, a_ks = p.a_ks;
  const int64_t b_rs = p.b_ns, b_ks = p.b_ks;

  f32x16_t acc[MI][2];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int nk = int((p.K + BK - 1) / BK);
  if (nk > 0) {
    la.load(A, a_rs, a_ks, m0, p.M, 0, p.K, p.vec_a);
    lb.load(B, b_rs, b_ks, n0, p.N, 0, p.K, p.vec_b);
  }
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    la.store(As[buf]);
    lb.store(Bs[buf]);
    if (kt + 1 < nk) {
      la.load(A, a_rs, a_ks, m0, p.M, int64_t(kt + 1) * BK, p.K, p.vec_a);
      lb.load(B, b_rs, b_ks, n0, p.N, int64_t(kt + 1) * BK, p.K, p.vec_b);
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < BK; ks += KSTEP) {
      if constexpr (sizeof(T) == 2) {
        bf16x8_t af[MI], bfv[2];
#pragma unroll
        for (int i = 0; i < MI; ++i) {
          u32x4_t v = *reinterpret_cast<const u32x4_t*>(&As[buf][(wm * 32 * MI + i * 32 + c) * LS + ks + 8 * g]);
          __builtin_memcpy(&af[i], &v, 16);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          u32x4_t v = *reinterpret_cast<const u32x4_t*>(&Bs[buf][(wn * 64 + j * 32 + c) * LS + ks + 8 * g]);
          __builtin_memcpy(&bfv[j], &v, 16);
        }
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfv[j], acc[i][j], 0, 0, 0);
      } else {
        float af[MI], bfv[2];
#pragma unroll
        for (int i = 0; i < MI; ++i) af[i] = As[buf][(wm * 32 * MI + i * 32 + c) * LS + ks + g];
#pragma unroll
        for (int j = 0; j < 2; ++j) bfv[j] = Bs[buf][(wn * 64 + j * 32 + c) * LS + ks + g];
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i], bfv[j], acc[i][j], 0, 0, 0);
      }
    }
  }

  // epilogue: acc[i][j] reg r → row 8*(r/4) + 4*g + r%4, col c of block (i, j)
  char* Cb = reinterpret_cast<char*>(p.C);
  const int cbytes = p.c_type == MK_F32 ? 4 : 2;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t n = n0 + wn * 64 + j * 32 + c;
    if (n >= p.N) continue;
    float bias = 0.f;
    if (p.epilogue != 0) bias = load_as_f32(p.bias, n, (p.epilogue & 4) ? MK_F32 : p.c_type);
#pragma unroll
    for (int i = 0; i < MI; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = m0 + wm * 32 * MI + i * 32 + 8 * (r / 4) + 4 * g + (r % 4);
        if (m >= p.M) continue;
        float v = acc[i][j][r];
        if (p.epilogue != 0) v += bias;
        if ((p.epilogue & 3) == 2) v = fmaxf(v, 0.f);
        const int64_t off = bz * p.c_bs + m * p.c_ms + n;
        if (cbytes == 4) reinterpret_cast<float*>(Cb)[off] = v;
        else store_from_f32(Cb, off, p.c_type, v);
      }
    }
  }
}

// 0 none, 1 + bias, 2 + bias then ReLU; 5 / 6: 1 / 2 with an fp32 bias
// whatever C's type
inline bool epilogue_ok(int e) { return e == 0 || e == 1 || e == 2 || e == 5 || e == 6; }

// y[c] = sum of the nrows partial rows of column c, in row order
__global__ __launch_bounds__(256) void colpart_sum_kernel(const float* __restrict__ part, int64_t nrows, int64_t cols,
                                                          float* __restrict__ y) {
  const int64_t c = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (c >= cols) return;
  float s = 0.f;
  for (int64_t r = 0; r < nrows; ++r) s += part[r * cols + c];
  y[c] = s;
}

// fp32 operands: 8 waves per workgroup (two per SIMD when one workgroup
// holds a CU); bf16: 4
template <typename T>
int launch_gemm(hipStream_t s, const GemmArgs& a, int64_t batch, bool a_kc, bool b_kc) {
  constexpr int NW = sizeof(T) == 4 ? 8 : 4;
  const int64_t tiles = ((a.M + kBM - 1) / kBM) * ((a.N + kBN - 1) / kBN);
  const dim3 g{unsigned(tiles), unsigned(batch)}, b{unsigned(64 * NW)};
  if (a_kc && b_kc) hipLaunchKernelGGL((gemm_kernel<T, true, true, NW>), g, b, 0, s, a);
  else if (a_kc && !b_kc) hipLaunchKernelGGL((gemm_kernel<T, true, false, NW>), g, b, 0, s, a);
  else if (!a_kc && b_kc) hipLaunchKernelGGL((gemm_kernel<T, false, true, NW>), g, b, 0, s, a);
  else hipLaunchKernelGGL((gemm_kernel<T, false, false, NW>), g, b, 0, s, a);
  return check_launch("mk_gemm");
}

}  // namespace
}  // namespace mk

using namespace mk;

extern "C" int mk_gemm_bias_gelu(void* stream, int ab_type, int c_type, int64_t M, int64_t N, int64_t K,
                                 const void* A, int64_t a_ms, int64_t a_ks, const void* B, int64_t b_ks,
                                 int64_t b_ns, void* C, int64_t c_ms, const void* bias, int epilogue, void* Y,
                                 int64_t y_ms) {
  clear_error();
  if (M < 0 || N < 0 || K < 0) return fail(MK_ERR_INVALID, "mk_gemm_bias_gelu: negative shape");
  if (ab_type != MK_BF16) return fail(MK_ERR_UNSUPPORTED, "mk_gemm_bias_gelu: ab_type must be bf16");
  if (c_type != MK_BF16 && c_type != MK_F32)
    return fail(MK_ERR_UNSUPPORTED, "mk_gemm_bias_gelu: c_type must be bf16 or f32");
  if (epilogue != 0 && epilogue != 1 && epilogue != 5)
    return fail(MK_ERR_INVALID, "mk_gemm_bias_gelu: epilogue must be 0, 1 or 5");
  if (epilogue != 0 && !bias) return fail(MK_ERR_INVALID, "mk_gemm_bias_gelu: epilogue needs bias");
  if (M == 0 || N == 0) return MK_OK;
  if (!A || !B || !C || !Y) return fail(MK_ERR_INVALID, "mk_gemm_bias_gelu: null pointer");
  const int r = gemm_tiled(as_stream(stream), c_type, 1, M, N, K, A, 0, a_ms, a_ks, B, 0, b_ks, b_ns, C, 0, c_ms,
                           bias, epilogue | kEpiGeluAux, 0, Y, y_ms);
  if (r >= 0) return r;
  return fail(MK_ERR_UNSUPPORTED,
              "mk_gemm_bias_gelu: needs the tiled kernel (bf16 operands with 16-byte aligned rows, M, N >= 128, "
              "K >= 64) and C and Y rows of whole 16-byte chunks");
}

extern "C" size_t mk_gemm_gelu_bwd_workspace_bytes(int64_t M, int64_t N) {
  if (M <= 0 || N <= 0) return 0;
  return size_t(((M + 127) / 128) * N * 4 + 255) & ~size_t(255);
}

extern "C" int mk_gemm_gelu_bwd(void* stream, int ab_type, int64_t M, int64_t N, int64_t K, const void* A,
                                int64_t a_ms, int64_t a_ks, const void* B, int64_t b_ks, int64_t b_ns, void* dx,
                                int64_t dx_ms, const void* pre, int64_t pre_ms, float* dx_colsum, void* workspace) {
  clear_error();
  if (M < 0 || N < 0 || K < 0) return fail(MK_ERR_INVALID, "mk_gemm_gelu_bwd: negative shape");
  if (ab_type != MK_BF16) return fail(MK_ERR_UNSUPPORTED, "mk_gemm_gelu_bwd: ab_type must be bf16");
  if (M == 0 || N == 0) return MK_OK;
  if (!A || !B || !dx || !pre || !dx_colsum || !workspace) return fail(MK_ERR_INVALID, "mk_gemm_gelu_bwd: null pointer");
  hipStream_t s = as_stream(stream);
  float* part = static_cast<float*>(workspace);
  const int r = gemm_tiled(s, MK_BF16, 1, M, N, K, A, 0, a_ms, a_ks, B, 0, b_ks, b_ns, dx, 0, dx_ms, nullptr,
                           kEpiGeluBwd, 0, const_cast<void*>(pre), pre_ms, part);
  if (r < 0)
    return fail(MK_ERR_UNSUPPORTED,
                "mk_gemm_gelu_bwd: needs the tiled kernel (bf16 operands with 16-byte aligned rows, M, N >= 128, "
                "K >= 64) and dx / pre rows of whole 16-byte chunks");
  if (r != MK_OK) return r;
  hipLaunchKernelGGL(colpart_sum_kernel, dim3(unsigned((N + 255) / 256)), dim3(256), 0, s, part, (M + 127) / 128, N,
                     dx_colsum);
  return check_launch("mk_gemm_gelu_bwd");
}

extern "C" int mk_gemm(void* stream, int ab_type, int c_type, int64_t batch, int64_t M, int64_t N,
                       int64_t K, const void* A, int64_t a_bs, int64_t a_ms, int64_t a_ks,
                       const void* B, int64_t b_bs, int64_t b_ks, int64_t b_ns, void* C,
                       int64_t c_bs, int64_t c_ms, const void* bias, int epilogue) {
  clear_error();
  if (batch < 0 || M < 0 || N < 0 || K < 0) return fail(MK_ERR_INVALID, "mk_gemm: negative shape");
  if (ab_type != MK_BF16 && ab_type != MK_F32)
    return fail(MK_ERR_UNSUPPORTED, "mk_gemm: ab_type must be bf16 or f32");
  if (c_type != MK_F32 && c_type != MK_BF16 && c_type != MK_F16)
    return fail(MK_ERR_UNSUPPORTED, "mk_gemm: c_type must be f32, bf16 or f16");
  if (!epilogue_ok(epilogue)) return fail(MK_ERR_INVALID, "mk_gemm: epilogue must be 0, 1, 2, 5 or 6");
  if (epilogue != 0 && !bias) return fail(MK_ERR_INVALID, "mk_gemm: epilogue needs bias");
  if (batch == 0 || M == 0 || N == 0) return MK_OK;
  if (!A || !B || !C) return fail(MK_ERR_INVALID, "mk_gemm: null pointer");
  if (batch >= 65536) return fail(MK_ERR_UNSUPPORTED, "mk_gemm: batch must be < 65536");
  const bool a_kc = a_ks == 1 || K == 1;
  const bool a_mc = a_ms == 1 || M == 1;
  const bool b_kc = b_ks == 1 || K == 1;
  const bool b_nc = b_ns == 1 || N == 1;
  if (!a_kc && !a_mc) return fail(MK_ERR_UNSUPPORTED, "mk_gemm: A needs a unit stride along m or k");
  if (!b_kc && !b_nc) return fail(MK_ERR_UNSUPPORTED, "mk_gemm: B needs a unit stride along k or n");
  const int64_t tiles = ((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN);
  if (tiles >= (int64_t(1) << 31)) return fail(MK_ERR_UNSUPPORTED, "mk_gemm: too many tiles");
  GemmArgs a;
  a.A = A; a.B = B; a.C = C; a.bias = bias;
  a.M = M; a.N = N; a.K = K;
  a.a_bs = a_bs; a.a_ms = a_kc ? a_ms : 1; a.a_ks = a_kc ? 1 : a_ks;
  a.b_bs = b_bs; a.b_ks = b_kc ? 1 : b_ks; a.b_ns = b_kc ? b_ns : 1;
  a.c_bs = c_bs; a.c_ms = c_ms;
  a.tiles_n = int((N + kBN - 1) / kBN);
  a.epilogue = epilogue;
  a.c_type = c_type;
  const int esz = ab_type == MK_BF16 ? 2 : 4;
  auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; };
  const int vec = 16 / esz;
  // vector loads need every chunk start 16-byte aligned: base, batch stride
  // and the non-unit stride must be multiples of the vector width
  a.vec_a = al16(A) && (a_bs % vec == 0) && ((a_kc ? a.a_ms : a.a_ks) % vec == 0);
  a.vec_b = al16(B) && (b_bs % vec == 0) && ((b_kc ? a.b_ns : a.b_ks) % vec == 0);
  hipStream_t s = as_stream(stream);
  if (ab_type == MK_BF16) {
    const int r = gemm_tiled(s, c_type, batch, M, N, K, A, a_bs, a_ms, a_ks, B, b_bs, b_ks, b_ns, C, c_bs,
                             c_ms, bias, epilogue);
    if (r >= 0) return r;
    return launch_gemm<uint16_t>(s, a, batch, a_kc, b_kc);
  }
  return launch_gemm<float>(s, a, batch, a_kc, b_kc);
}

extern "C" size_t mk_gemm_splitk_workspace_bytes(int64_t M, int64_t N, int64_t splits) {
  if (M <= 0 || N <= 0 || splits <= 1) return 0;
  return size_t(M * N * splits * 4);
}

extern "C" int mk_gemm_splitk_typed(void* stream, int ab_type, int c_type, int64_t M, int64_t N, int64_t K,
                                    const void* A, int64_t a_ms, int64_t a_ks, const void* B, int64_t b_ks,
                                    int64_t b_ns, void* C, int64_t c_ms, int64_t splits, void* workspace,
                                    const void* bias, int epilogue) {
  clear_error();
  if (splits < 1 || K < 0 || M < 0 || N < 0) return fail(MK_ERR_INVALID, "mk_gemm_splitk: bad shape or splits");
  if (c_type != MK_F32 && c_type != MK_BF16) return fail(MK_ERR_UNSUPPORTED, "mk_gemm_splitk: c_type must be f32 or bf16");
  if (!epilogue_ok(epilogue)) return fail(MK_ERR_INVALID, "mk_gemm_splitk: epilogue must be 0, 1, 2, 5 or 6");
  if (epilogue != 0 && !bias) return fail(MK_ERR_INVALID, "mk_gemm_splitk: epilogue needs bias");
  if (splits == 1 || M == 0 || N == 0)
    return mk_gemm(stream, ab_type, c_type, 1, M, N, K, A, 0, a_ms, a_ks, B, 0, b_ks, b_ns, C, 0, c_ms, bias,
                   epilogue);
  if (!workspace || !C) return fail(MK_ERR_INVALID, "mk_gemm_splitk: null workspace or output");
  const uintptr_t cal = c_type == MK_F32 ? 15u : 7u;
  if ((N % 4) != 0 || (c_ms % 4) != 0 || (reinterpret_cast<uintptr_t>(C) & cal) ||
      (reinterpret_cast<uintptr_t>(workspace) & 15u))
    return fail(MK_ERR_UNSUPPORTED, "mk_gemm_splitk: N and c_ms multiples of 4, aligned C and workspace");
  float* W = static_cast<float*>(workspace);
  hipStream_t s = as_stream(stream);
  if (K % splits == 0) {
    // slice s reads A[:, s ks : (s+1) ks] and B[s ks : (s+1) ks, :] (element
    // strides along k) and writes W[s]: one batched mk_gemm, then the ordered sum
    const int64_t ks = K / splits;
    if (int rc = mk_gemm(stream, ab_type, MK_F32, splits, M, N, ks, A, ks * a_ks, a_ms, a_ks, B, ks * b_ks, b_ks,
                         b_ns, W, M * N, N, nullptr, 0))
      return rc;
    return splitk_sum(s, W, splits, M, N, C, c_ms, "mk_gemm_splitk", c_type, bias, epilogue);
  }
  // uneven slices: ks apart (a multiple of 8, so every slice starts on a
  // 16-byte boundary of a k-contiguous operand), the last one K - (splits-1) ks
  // long.  Only the tiled kernel takes a per-batch contraction length; a
  // product it does not take runs unsplit (deterministic too, with the fp32
  // additions in another order).
  const int64_t ks = ((K + splits - 1) / splits + 7) / 8 * 8;
  const int64_t rem = K - (splits - 1) * ks;
  const int r = ab_type == MK_BF16 && rem > 0
                    ? gemm_tiled(s, MK_F32, splits, M, N, ks, A, ks * a_ks, a_ms, a_ks, B, ks * b_ks, b_ks, b_ns, W,
                                 M * N, N, nullptr, 0, rem)
                    : -1;
  if (r < 0)
    return mk_gemm(stream, ab_type, c_type, 1, M, N, K, A, 0, a_ms, a_ks, B, 0, b_ks, b_ns, C, 0, c_ms, bias,
                   epilogue);
  if (r != MK_OK) return r;
  return splitk_sum(s, W, splits, M, N, C, c_ms, "mk_gemm_splitk", c_type, bias, epilogue);
}

extern "C" int mk_gemm_splitk(void* stream, int ab_type, int64_t M, int64_t N, int64_t K, const void* A, int64_t a_ms,
                              int64_t a_ks, const void* B, int64_t b_ks, int64_t b_ns, float* C, int64_t c_ms,
                              int64_t splits, void* workspace) {
  return mk_gemm_splitk_typed(stream, ab_type, MK_F32, M, N, K, A, a_ms, a_ks, B, b_ks, b_ns, C, c_ms, splits,
                              workspace, nullptr, 0);
}
