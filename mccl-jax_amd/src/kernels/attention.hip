// Causal / non-causal scaled-dot-product attention, forward (flash style)
// for gfx950 on v_mfma_f32_32x32x16_bf16.
//
// Work split: one workgroup = 4 waves = BM = 128 query rows of one (b, h);
// each wave owns 32 query rows for the whole key loop.  Key/value tiles of
// BN = 64 rows pass through LDS.
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
// step j.  V stays row-major in LDS; the A operand (Vᵀ) is read with
// ds_read_b64_tr_b16, which hands each lane of a 16-lane group one column of
// a 4-key x 16-d block: two such reads give the 8 k-slots of a lane.
//
// Pipeline (per tile t, one barrier): K runs one tile ahead of its use and
// V one tile behind, so after the barrier of iteration t the workgroup stores
// K[t+1] and V[t] (fetched into registers during iteration t-1) into the LDS
// buffers that K[t-1] and V[t-2] have left, and issues the global loads of
// K[t+2] and V[t+1].  Each wave computes S(t) = K[t]·Qᵀ and then issues the
// MFMAs of O += P(t-1)·V[t-1] in the same instruction stream as the
// exponentials of P(t), so the matrix cores work while the softmax runs.
//
// Online softmax runs in the log2 domain: s2 = s * scale * log2(e),
// p = exp2(s2 - m) on v_exp_f32, row statistics in fp32.  The running max m
// is raised only when some row's max grows by more than kRescaleLog2, and
// then to an integer, so the rescale factor alpha = exp2(m_old - m_new) is a
// power of two: O, l and the pending bf16 P(t-1) are scaled exactly.
// Between raises p <= 2^kRescaleLog2 stays far inside fp32/bf16 range.  The
// row sum adds the bf16-rounded p (the values the P.V product uses) with
// v_dot2_f32_bf16.
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
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;

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

template <bool B>
struct Flag {
  static constexpr bool value = B;
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

// 4 bf16 of one LDS column block (ds_read_b64_tr_b16), as two 32-bit words
__device__ inline uint2 lds_read_tr(const uint16_t* p) {
  const i16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(p));
  return __builtin_bit_cast(uint2, v);
}

template <int D, bool CAUSAL>
__global__ __launch_bounds__(kThreads, 2) void sdpa_fwd_kernel(const SdpaArgs p) {
  constexpr int KS = D + 8;   // K row stride in LDS (elements): conflict-free b128 reads
  constexpr int VS = D + 32;  // V row stride in LDS (elements): conflict-free transposed reads
  constexpr int CH = D / 8;   // 16-byte chunks per row
  constexpr int CH_T = kBN * CH / kThreads;  // chunks per thread per K (or V) tile
  constexpr int NDB = D / 32;  // 32-wide d blocks of O
  constexpr int NKS = D / 16;  // 16-deep k-steps of Q·Kᵀ
  static_assert((kBN * CH) % kThreads == 0, "tile/thread mismatch");

  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][kBN * KS];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[2][kBN * VS];

  // heaviest (latest) query tiles first; consecutive ids walk over heads so
  // a head's tiles share an XCD when BH % 8 == 0
  const int id = blockIdx.x;
  const int qt = CAUSAL ? (p.n_qtiles - 1 - id / p.BH) : (id / p.BH);
  const int bh = id % p.BH;
  const int b = bh / p.H, h = bh % p.H;

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
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
  if (CAUSAL) kv_end = min(kv_end, min(qt * kBM + kBM, p.Sq));  // one past the block's last query
  const int n_tiles = (kv_end + kBN - 1) / kBN;
  // tiles this wave computes (causal: those holding a key <= its last query)
  const int n_rel = CAUSAL ? min(n_tiles, (q0 + 31) / kBN + 1) : n_tiles;

  // ---- staging: global -> registers -> LDS
  u32x4_t kreg[CH_T], vreg[CH_T];
  auto load_k = [&](int tile) {
    const int kv0 = tile * kBN;
    const int rows = min(kBN, p.Sk - kv0);  // valid keys in the tile (>= 1); rows >= D elements apart
    const __amdgpu_buffer_rsrc_t r =
        tile_rsrc(kb + int64_t(kv0) * p.k_ss, uint32_t((rows - 1) * p.k_ss + D) * 2u);
#pragma unroll
    for (int i = 0; i < CH_T; ++i) {
      const int ch = t + i * kThreads;
      kreg[i] = __builtin_amdgcn_raw_buffer_load_b128(r, ((ch / CH) * int(p.k_ss) + (ch % CH) * 8) * 2, 0, 0);
    }
  };
  auto load_v = [&](int tile) {
    const int kv0 = tile * kBN;
    const int rows = min(kBN, p.Sk - kv0);
    const __amdgpu_buffer_rsrc_t r =
        tile_rsrc(vb + int64_t(kv0) * p.v_ss, uint32_t((rows - 1) * p.v_ss + D) * 2u);
#pragma unroll
    for (int i = 0; i < CH_T; ++i) {
      const int ch = t + i * kThreads;
      vreg[i] = __builtin_amdgcn_raw_buffer_load_b128(r, ((ch / CH) * int(p.v_ss) + (ch % CH) * 8) * 2, 0, 0);
    }
  };
  auto store_k = [&](int buf) {
#pragma unroll
    for (int i = 0; i < CH_T; ++i) {
      const int ch = t + i * kThreads;
      *reinterpret_cast<u32x4_t*>(&Ks[buf][(ch / CH) * KS + (ch % CH) * 8]) = kreg[i];
    }
  };
  auto store_v = [&](int buf) {
#pragma unroll
    for (int i = 0; i < CH_T; ++i) {
      const int ch = t + i * kThreads;
      *reinterpret_cast<u32x4_t*>(&Vs[buf][(ch / CH) * VS + (ch % CH) * 8]) = vreg[i];
    }
  };

  // ---- Sᵀ = K · Qᵀ for the 64 keys of an LDS K tile (two 32-key blocks)
  auto qk = [&](int buf, f32x16_t(&s)[2]) {
#pragma unroll
    for (int kb2 = 0; kb2 < 2; ++kb2) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kb2][r] = 0.f;
#pragma unroll
      for (int st = 0; st < NKS; ++st) {
        const bf16x8_t a =
            as_bf16x8(*reinterpret_cast<const u32x4_t*>(&Ks[buf][(kb2 * 32 + c) * KS + 16 * st + 8 * g]));
        s[kb2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[st], s[kb2], 0, 0, 0);
      }
    }
  };

  // lane's element offset in a V tile for the transposed reads: key 4g + r/4,
  // d 16*hi + 4*(r%4) (r = lane % 16, hi = lane / 16 % 2)
  const int vlane = (4 * g + ((lane & 15) >> 2)) * VS + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

  f32x16_t o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = 0.f;
  float m_run = -INFINITY;  // running max, log2 domain
  float l_run = 0.f;        // this lane's share of the running row sum

  // ---- Oᵀ += Vᵀ · Pᵀ over the 64 keys of the LDS V tile in buffer vbuf
  auto pv = [&](const bf16x8_t(&pf)[2][2], int vbuf) {
    const uint16_t* vt = &Vs[vbuf][vlane];
#pragma unroll
    for (int kb2 = 0; kb2 < 2; ++kb2) {
#pragma unroll
      for (int j2 = 0; j2 < 2; ++j2) {
        const int kstep = kb2 * 32 + 16 * j2;
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          const uint2 lo = lds_read_tr(vt + kstep * VS + db * 32);
          const uint2 hi = lds_read_tr(vt + (kstep + 8) * VS + db * 32);
          const u32x4_t av = {lo.x, lo.y, hi.x, hi.y};
          o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(av), pf[kb2][j2], o[db], 0, 0, 0);
        }
      }
    }
  };

  // One tile tt of this wave: S(tt) = K[tt]·Qᵀ, softmax statistics, then the
  // exponentials of P(tt) interleaved with O += P(tt-1)·V[tt-1] (PREV).
  // pf holds P(tt-1) on entry and P(tt) on exit.
  auto step = [&](int tt, bf16x8_t(&pf)[2][2], auto prev) {
    constexpr bool PREV = decltype(prev)::value;
    const int kv0 = tt * kBN;
    f32x16_t s[2];
    qk(tt & 1, s);

    // ---- masking (diagonal / ragged tiles only)
    if ((CAUSAL && kv0 + kBN - 1 > q0) || kv0 + kBN > p.Sk) {
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kv0 + kb2 * 32 + 8 * (r / 4) + 4 * g + (r % 4);
          if (key >= p.Sk || (CAUSAL && key > qrow)) s[kb2][r] = -INFINITY;
        }
    }

    // ---- online softmax statistics (log2 domain, lazy power-of-two rescale)
    float mt = s[0][0];
#pragma unroll
    for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
      for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[kb2][r]);
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float m_cand = fmaxf(m_run, mt * p.scale_log2);
    // m_run == -inf until the row has seen an unmasked key, so the first
    // such tile always rescales (alpha = 0 on O = 0, l = 0)
    if (__builtin_amdgcn_ballot_w64(m_cand > m_run + kRescaleLog2) != 0) {
      const float m_new = ceilf(m_cand);  // integer: alpha is a power of two
      // rows with no unmasked key yet keep m = -inf and alpha = 1
      const float alpha = (m_new == m_run) ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
      if constexpr (PREV) {
        // P(tt-1) still to be applied: bf16 * 2^k is exact
#pragma unroll
        for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
          for (int j2 = 0; j2 < 2; ++j2) {
            u32x4_t w = __builtin_bit_cast(u32x4_t, pf[kb2][j2]);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const f32x2_t e = {__builtin_bit_cast(float, w[i] << 16) * alpha,
                                 __builtin_bit_cast(float, w[i] & 0xffff0000u) * alpha};
              w[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(e, bf16x2_t));
            }
            pf[kb2][j2] = as_bf16x8(w);
          }
      }
    }
    // m_run == -inf only while every key so far is masked for this row
    const float m_use = (m_run == -INFINITY) ? 0.f : m_run;

    // ---- P(tt) = exp2(s2 - m), packed two keys per 32-bit word
    // (v_cvt_pk_bf16_f32), summed from the packed words with v_dot2_f32_bf16;
    // the MFMAs of P(tt-1)·V[tt-1] run meanwhile
    bf16x8_t pn[2][2];
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
            const f32x2_t e = {__builtin_amdgcn_exp2f(fmaf(s[kb2][8 * j2 + i], p.scale_log2, -m_use)),
                               __builtin_amdgcn_exp2f(fmaf(s[kb2][8 * j2 + i + 1], p.scale_log2, -m_use))};
            const bf16x2_t pr = __builtin_convertvector(e, bf16x2_t);
            w[i / 2] = __builtin_bit_cast(uint32_t, pr);
            if (i & 2) ls1 = __builtin_amdgcn_fdot2_f32_bf16(pr, one, ls1, false);
            else ls0 = __builtin_amdgcn_fdot2_f32_bf16(pr, one, ls0, false);
          }
          pn[kb2][j2] = as_bf16x8(w);
        }
      l_run += ls0 + ls1;
    }
    if constexpr (PREV) pv(pf, (tt - 1) & 1);
#pragma unroll
    for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
      for (int j2 = 0; j2 < 2; ++j2) pf[kb2][j2] = pn[kb2][j2];
  };

  // staging of iteration tt: K[tt+1] and V[tt] into LDS, loads of K[tt+2], V[tt+1]
  auto stage = [&](int tt) {
    if (tt + 1 < n_tiles) store_k((tt + 1) & 1);
    store_v(tt & 1);
    if (tt + 2 < n_tiles) load_k(tt + 2);
    if (tt + 1 < n_tiles) load_v(tt + 1);
  };

  bf16x8_t pf[2][2];
  if (n_tiles > 0) {
    // prologue: K[0] in LDS, K[1] and V[0] in flight
    load_k(0);
    store_k(0);
    if (n_tiles > 1) load_k(1);
    load_v(0);
    __syncthreads();
    stage(0);
    step(0, pf, Flag<false>{});  // every wave has n_rel >= 1
    for (int tt = 1; tt < n_tiles; ++tt) {
      __syncthreads();
      stage(tt);
      if (tt < n_rel) step(tt, pf, Flag<true>{});
      else if (tt == n_rel) pv(pf, (tt - 1) & 1);  // the wave's last tile, V still resident
    }
    __syncthreads();  // V[n_tiles-1] was stored in the last iteration
    if (n_rel == n_tiles) pv(pf, (n_tiles - 1) & 1);
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
        const f32x2_t lo = {o[db][4 * r4 + 0] * inv, o[db][4 * r4 + 1] * inv};
        const f32x2_t hi = {o[db][4 * r4 + 2] * inv, o[db][4 * r4 + 3] * inv};
        uint2 w;
        w.x = __builtin_bit_cast(uint32_t, __builtin_convertvector(lo, bf16x2_t));
        w.y = __builtin_bit_cast(uint32_t, __builtin_convertvector(hi, bf16x2_t));
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
