// Causal / non-causal scaled-dot-product attention, forward (flash style)
// for gfx950 on v_mfma_f32_32x32x16_bf16.
//
// Work split: one workgroup = 4 waves = BM = 128 query rows of one (b, h);
// each wave owns 32 query rows for the whole key loop.  Key/value tiles of
// BN = 64 rows are staged through LDS (double buffered; global loads for
// tile t+1 are issued before tile t is computed).
//
// Register layouts (32x32 MFMA, lane l, g = l / 32, c = l % 32):
//   A operand: row c, 8 consecutive k-slots of half g
//   B operand: col c, 8 consecutive k-slots of half g
//   C/D:       reg r holds row 8*(r/4) + 4*g + (r%4), col c
// S is computed transposed, Sᵀ = K · Qᵀ, so every lane holds one query's
// scores (column c) for 32 of the tile's keys: the row max / row sum are
// in-lane reductions plus one exchange with lane l^32.  Those same
// registers, converted to bf16, ARE the B operand of Oᵀ = Vᵀ · Pᵀ: the k-slot
// (g, i) of P corresponds to key 16*j + 4*g + 8*(i/4) + i%4 of the 16-key
// step j, and the A operand (Vᵀ) is read from LDS with the same key mapping,
// so P never leaves registers.  Vᵀ is produced while staging V into LDS
// (pairs of keys packed into one 32-bit LDS word per d).
//
// Online softmax runs in the log2 domain: s2 = s * scale * log2(e),
// p = exp2(s2 - m) on v_exp_f32, row statistics in fp32.  The running max m
// is raised (and O, l rescaled) only when some row's max grows by more than
// kRescaleLog2; otherwise p <= 2^kRescaleLog2 stays far inside fp32/bf16
// range and the rescale is skipped.  The row sum adds the bf16-rounded p
// (the values the P.V product uses) with v_dot2_f32_bf16.
//
// K/V tiles are fetched with raw buffer loads whose descriptor ends at the
// last valid key: rows past Sk read as zeros without a branch.
#include "mk_common.h"

#include <cmath>

namespace mk {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kBM = 128;    // query rows per workgroup
constexpr int kBN = 64;     // keys per tile
constexpr int kThreads = 256;
constexpr float kRescaleLog2 = 8.f;  // lazy-rescale threshold (log2 units)
constexpr int kBufferWord3 = 0x00020000;  // raw buffer descriptor, gfx9 family

struct SdpaArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  float* lse;
  int64_t q_bs, q_hs, q_ss;
  int64_t k_bs, k_hs, k_ss;
  int64_t v_bs, v_hs, v_ss;
  int64_t o_bs, o_hs, o_ss;
  int H, Sq, Sk;
  int n_qtiles;
  int BH;
  float scale_log2;  // scale * log2(e)
};

__device__ inline bf16x8_t as_bf16x8(const u32x4_t& v) {
  bf16x8_t r;
  __builtin_memcpy(&r, &v, 16);
  return r;
}

// descriptor over [base, base + bytes): loads past the end return zeros
__device__ inline __amdgpu_buffer_rsrc_t tile_rsrc(const uint16_t* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), 0, int(bytes), kBufferWord3);
}

template <int D, bool CAUSAL>
__global__ __launch_bounds__(kThreads, 2) void sdpa_fwd_kernel(const SdpaArgs p) {
  constexpr int KS = D + 8;    // K row stride in LDS (elements): conflict-free b128 reads
  constexpr int VS = kBN + 4;  // Vᵀ row stride (elements): conflict-free b64 reads
  constexpr int KCH = kBN * D / 8;           // 16-byte chunks in a K tile
  constexpr int KCH_T = KCH / kThreads;      // per thread
  constexpr int VPAIRS = (kBN / 2) * (D / 8);  // (key pair, d-chunk) tasks in a V tile
  constexpr int VP_T = VPAIRS / kThreads;
  constexpr int NDB = D / 32;  // 32-wide d blocks of O
  constexpr int NKS = D / 16;  // 16-deep k-steps of Q·Kᵀ
  static_assert(KCH % kThreads == 0 && VPAIRS % kThreads == 0, "tile/thread mismatch");

  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][kBN * KS];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[2][D * VS];

  // heaviest (latest) query tiles first; consecutive ids walk over heads so
  // a head's tiles share an XCD when BH % 8 == 0
  const int id = blockIdx.x;
  const int qt = CAUSAL ? (p.n_qtiles - 1 - id / p.BH) : (id / p.BH);
  const int bh = id % p.BH;
  const int b = bh / p.H, h = bh % p.H;

  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int c = lane & 31, g = lane >> 5;
  const int q0 = qt * kBM + wave * 32;  // first query row of this wave
  const int qrow = q0 + c;               // the query this lane's columns belong to

  const uint16_t* qb = p.q + b * p.q_bs + h * p.q_hs;
  const uint16_t* kb = p.k + b * p.k_bs + h * p.k_hs;
  const uint16_t* vb = p.v + b * p.v_bs + h * p.v_hs;

  // Q fragment (B operand of Sᵀ = K·Qᵀ): Q[qrow][16*s + 8*g + i]
  bf16x8_t qf[NKS];
  {
    const bool ok = qrow < p.Sq;
#pragma unroll
    for (int s = 0; s < NKS; ++s) {
      u32x4_t v = {0u, 0u, 0u, 0u};
      if (ok) v = *reinterpret_cast<const u32x4_t*>(qb + int64_t(qrow) * p.q_ss + 16 * s + 8 * g);
      qf[s] = as_bf16x8(v);
    }
  }

  int kv_end = p.Sk;
  if (CAUSAL) {
    const int last_q = min(qt * kBM + kBM, p.Sq);  // one past the block's last query
    kv_end = min(kv_end, last_q);
  }
  const int n_tiles = (kv_end + kBN - 1) / kBN;

  // staging registers for the next tile
  u32x4_t kreg[KCH_T];
  u32x4_t vreg[VP_T][2];

  auto load_tile = [&](int tile) {
    const int kv0 = tile * kBN;
    const int rows = min(kBN, p.Sk - kv0);  // valid keys in the tile (>= 1)
    // byte extent of the valid rows; rows are >= D elements apart
    const __amdgpu_buffer_rsrc_t kr =
        tile_rsrc(kb + int64_t(kv0) * p.k_ss, uint32_t((rows - 1) * p.k_ss + D) * 2u);
    const __amdgpu_buffer_rsrc_t vr =
        tile_rsrc(vb + int64_t(kv0) * p.v_ss, uint32_t((rows - 1) * p.v_ss + D) * 2u);
#pragma unroll
    for (int i = 0; i < KCH_T; ++i) {
      const int ch = t + i * kThreads;
      const int row = ch / (D / 8), col = (ch % (D / 8)) * 8;
      kreg[i] = __builtin_amdgcn_raw_buffer_load_b128(kr, (row * int(p.k_ss) + col) * 2, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < VP_T; ++i) {
      const int task = t + i * kThreads;
      const int pr = task % (kBN / 2), d8 = task / (kBN / 2);
      const int off = (2 * pr * int(p.v_ss) + d8 * 8) * 2;
      vreg[i][0] = __builtin_amdgcn_raw_buffer_load_b128(vr, off, 0, 0);
      vreg[i][1] = __builtin_amdgcn_raw_buffer_load_b128(vr, off + int(p.v_ss) * 2, 0, 0);
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < KCH_T; ++i) {
      const int ch = t + i * kThreads;
      const int row = ch / (D / 8), col = (ch % (D / 8)) * 8;
      *reinterpret_cast<u32x4_t*>(&Ks[buf][row * KS + col]) = kreg[i];
    }
#pragma unroll
    for (int i = 0; i < VP_T; ++i) {
      const int task = t + i * kThreads;
      const int pr = task % (kBN / 2), d8 = task / (kBN / 2);
      const uint16_t* a = reinterpret_cast<const uint16_t*>(&vreg[i][0]);
      const uint16_t* bq = reinterpret_cast<const uint16_t*>(&vreg[i][1]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t w = uint32_t(a[e]) | (uint32_t(bq[e]) << 16);
        *reinterpret_cast<uint32_t*>(&Vt[buf][(d8 * 8 + e) * VS + 2 * pr]) = w;
      }
    }
  };

  f32x16_t o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = 0.f;
  float m_run = -INFINITY;  // running max, log2 domain
  float l_run = 0.f;        // this lane's share of the running row sum

  if (n_tiles > 0) load_tile(0);
  for (int tile = 0; tile < n_tiles; ++tile) {
    const int buf = tile & 1;
    store_tile(buf);
    if (tile + 1 < n_tiles) load_tile(tile + 1);
    __syncthreads();
    const int kv0 = tile * kBN;
    // a wave whose queries all precede the tile has nothing to do here
    if (CAUSAL && kv0 > q0 + 31) continue;

    // ---- Sᵀ = K · Qᵀ for 64 keys (two 32-key blocks)
    f32x16_t sacc[2];
#pragma unroll
    for (int kb2 = 0; kb2 < 2; ++kb2) {
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[kb2][r] = 0.f;
#pragma unroll
      for (int s = 0; s < NKS; ++s) {
        const bf16x8_t a =
            as_bf16x8(*reinterpret_cast<const u32x4_t*>(&Ks[buf][(kb2 * 32 + c) * KS + 16 * s + 8 * g]));
        sacc[kb2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[s], sacc[kb2], 0, 0, 0);
      }
    }

    // ---- masking (diagonal / ragged tiles only)
    const bool need_mask = (CAUSAL && kv0 + kBN - 1 > q0) || (kv0 + kBN > p.Sk);
    if (need_mask) {
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kv0 + kb2 * 32 + 8 * (r / 4) + 4 * g + (r % 4);
          const bool masked = (key >= p.Sk) || (CAUSAL && key > qrow);
          if (masked) sacc[kb2][r] = -INFINITY;
        }
    }

    // ---- online softmax (log2 domain, lazy rescale)
    float mt = sacc[0][0];
#pragma unroll
    for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
      for (int r = 0; r < 16; ++r) mt = fmaxf(mt, sacc[kb2][r]);
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float m_cand = fmaxf(m_run, mt * p.scale_log2);
    // m_run == -inf until the row has seen an unmasked key, so the first
    // such tile always rescales (alpha = exp2(-inf) = 0 on O = 0, l = 0)
    if (__builtin_amdgcn_ballot_w64(m_cand > m_run + kRescaleLog2) != 0) {
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_cand);
      m_run = m_cand;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
    }
    // m_run == -inf only while every key so far is masked for this row
    const float m_use = (m_run == -INFINITY) ? 0.f : m_run;
    // p = exp2(s2 - m), packed two keys per 32-bit word (v_cvt_pk_bf16_f32),
    // summed from the packed words with v_dot2_f32_bf16
    bf16x8_t pf[2][2];
    {
      const bf16x2_t one = {static_cast<__bf16>(1.f), static_cast<__bf16>(1.f)};
      float ls0 = 0.f, ls1 = 0.f;
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
        for (int j2 = 0; j2 < 2; ++j2) {
          u32x4_t w;
#pragma unroll
          for (int i = 0; i < 8; i += 2) {
            const f32x2_t e = {__builtin_amdgcn_exp2f(fmaf(sacc[kb2][8 * j2 + i], p.scale_log2, -m_use)),
                              __builtin_amdgcn_exp2f(fmaf(sacc[kb2][8 * j2 + i + 1], p.scale_log2, -m_use))};
            const bf16x2_t pr = __builtin_convertvector(e, bf16x2_t);
            w[i / 2] = __builtin_bit_cast(uint32_t, pr);
            if (i & 2) ls1 = __builtin_amdgcn_fdot2_f32_bf16(pr, one, ls1, false);
            else ls0 = __builtin_amdgcn_fdot2_f32_bf16(pr, one, ls0, false);
          }
          pf[kb2][j2] = as_bf16x8(w);
        }
      l_run += ls0 + ls1;
    }

    // ---- Oᵀ += Vᵀ · Pᵀ
#pragma unroll
    for (int kb2 = 0; kb2 < 2; ++kb2) {
#pragma unroll
      for (int j2 = 0; j2 < 2; ++j2) {
        const int kbase = kb2 * 32 + 16 * j2 + 4 * g;
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          const uint16_t* row = &Vt[buf][(db * 32 + c) * VS + kbase];
          u32x4_t av;
          const uint2 lo = *reinterpret_cast<const uint2*>(row);
          const uint2 hi = *reinterpret_cast<const uint2*>(row + 8);
          av[0] = lo.x; av[1] = lo.y; av[2] = hi.x; av[3] = hi.y;
          o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(av), pf[kb2][j2], o[db], 0, 0, 0);
        }
      }
    }
  }

  // ---- epilogue: normalise and store O (lane owns query qrow, 4 consecutive d per reg group)
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  if (qrow < p.Sq) {
    const float inv = (l_tot > 0.f) ? 1.f / l_tot : __builtin_nanf("");
    uint16_t* ob = p.o + b * p.o_bs + h * p.o_hs + int64_t(qrow) * p.o_ss;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d = db * 32 + 8 * r4 + 4 * g;
        uint2 w;
        w.x = uint32_t(f32_to_bf16(o[db][4 * r4 + 0] * inv)) | (uint32_t(f32_to_bf16(o[db][4 * r4 + 1] * inv)) << 16);
        w.y = uint32_t(f32_to_bf16(o[db][4 * r4 + 2] * inv)) | (uint32_t(f32_to_bf16(o[db][4 * r4 + 3] * inv)) << 16);
        *reinterpret_cast<uint2*>(ob + d) = w;
      }
    }
    if (p.lse && g == 0) {
      const float lse2 = (l_tot > 0.f) ? m_run + log2f(l_tot) : -INFINITY;
      p.lse[int64_t(bh) * p.Sq + qrow] = lse2 * 0.69314718055994531f;
    }
  }
}

}  // namespace
}  // namespace mk

using namespace mk;

extern "C" int mk_sdpa_fwd(void* stream, int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D,
                           const void* q, int64_t q_bs, int64_t q_hs, int64_t q_ss,
                           const void* k, int64_t k_bs, int64_t k_hs, int64_t k_ss,
                           const void* v, int64_t v_bs, int64_t v_hs, int64_t v_ss,
                           void* o, int64_t o_bs, int64_t o_hs, int64_t o_ss,
                           float scale, int causal, float* lse) {
  clear_error();
  if (B < 0 || H < 0 || Sq < 0 || Sk < 0) return fail(MK_ERR_INVALID, "mk_sdpa_fwd: negative shape");
  if (D != 64 && D != 128) return fail(MK_ERR_UNSUPPORTED, "mk_sdpa_fwd: head_dim must be 64 or 128");
  if (Sq >= (int64_t(1) << 30) || Sk >= (int64_t(1) << 30) || B * H >= (int64_t(1) << 30))
    return fail(MK_ERR_UNSUPPORTED, "mk_sdpa_fwd: sizes too large");
  if (B == 0 || H == 0 || Sq == 0) return MK_OK;
  if (!q || !k || !v || !o) return fail(MK_ERR_INVALID, "mk_sdpa_fwd: null pointer");
  // a length-1 sequence axis may carry any stride; only row 0 is read
  if (Sq == 1) q_ss = o_ss = D;
  if (Sk == 1) k_ss = v_ss = D;
  // 16-byte vector access along d needs every row start 16-byte aligned
  const uintptr_t al = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                       reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(o);
  const int64_t st = q_bs | q_hs | q_ss | k_bs | k_hs | k_ss | v_bs | v_hs | v_ss;
  if ((al & 15u) != 0 || (st & 7) != 0 || ((o_bs | o_hs | o_ss) & 3) != 0)
    return fail(MK_ERR_UNSUPPORTED, "mk_sdpa_fwd: q/k/v need 16-byte aligned rows (strides % 8 == 0), o strides % 4 == 0");
  if (k_ss < D || v_ss < D || k_ss >= (int64_t(1) << 24) || v_ss >= (int64_t(1) << 24))
    return fail(MK_ERR_UNSUPPORTED, "mk_sdpa_fwd: k/v sequence strides must be in [D, 2^24)");
  SdpaArgs a;
  a.q = (const uint16_t*)q; a.k = (const uint16_t*)k; a.v = (const uint16_t*)v; a.o = (uint16_t*)o;
  a.lse = lse;
  a.q_bs = q_bs; a.q_hs = q_hs; a.q_ss = q_ss;
  a.k_bs = k_bs; a.k_hs = k_hs; a.k_ss = k_ss;
  a.v_bs = v_bs; a.v_hs = v_hs; a.v_ss = v_ss;
  a.o_bs = o_bs; a.o_hs = o_hs; a.o_ss = o_ss;
  a.H = int(H); a.Sq = int(Sq); a.Sk = int(Sk);
  a.n_qtiles = int((Sq + kBM - 1) / kBM);
  a.BH = int(B * H);
  a.scale_log2 = scale * 1.4426950408889634f;
  const int64_t blocks = int64_t(a.n_qtiles) * a.BH;
  if (blocks >= (int64_t(1) << 31)) return fail(MK_ERR_UNSUPPORTED, "mk_sdpa_fwd: grid too large");
  hipStream_t s = as_stream(stream);
  const dim3 g{unsigned(blocks)}, bl{unsigned(kThreads)};
  if (D == 128) {
    if (causal) hipLaunchKernelGGL((sdpa_fwd_kernel<128, true>), g, bl, 0, s, a);
    else hipLaunchKernelGGL((sdpa_fwd_kernel<128, false>), g, bl, 0, s, a);
  } else {
    if (causal) hipLaunchKernelGGL((sdpa_fwd_kernel<64, true>), g, bl, 0, s, a);
    else hipLaunchKernelGGL((sdpa_fwd_kernel<64, false>), g, bl, 0, s, a);
  }
  return check_launch("mk_sdpa_fwd");
}
