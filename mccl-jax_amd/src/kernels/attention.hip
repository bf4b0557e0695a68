// Causal / non-causal scaled-dot-product attention, forward (flash style)
// for gfx950 on v_mfma_f32_32x32x16_bf16.
//
// Work split: one workgroup = 8 waves = BM = 256 query rows of one (b, h),
// one workgroup per CU; wave w owns query rows 32 w .. 32 w + 31 for the
// whole key loop.  Key/value tiles of BN = 64 rows pass through LDS and are
// shared by the 8 waves.
//
// Register layouts: those of the 32x32 MFMA (attn_common.h).
// S is computed transposed, Sᵀ = K · Qᵀ, so every lane holds one query's
// scores (column c) for 32 of the tile's keys: the row max / row sum are
// in-lane reductions plus one exchange with lane l^32 (v_permlane32_swap,
// a VALU op: no LDS round trip on the softmax's critical path).  Those same
// registers, converted to bf16, ARE the B operand of Oᵀ = Vᵀ · Pᵀ: the k-slot
// (g, i) of P corresponds to key 16*j + 4*g + 8*(i/4) + i%4 of the 16-key
// step j.  V is not transposed in LDS; the A operand (Vᵀ) is read with
// ds_read_b64_tr_b16, which hands each lane of a 16-lane group one column of
// a 4-key x 16-d block: two such reads give the 8 k-slots of a lane.
//
// Ping-pong: waves 0-3 (group A) and 4-7 (group B) share the four SIMDs, one
// of each per SIMD, and alternate between two phases separated by workgroup
// barriers.  In its matrix phase M(t) a wave issues the 32 MFMAs of
// S(t) = K[t]·Qᵀ and O += P(t-1)·V[t-1] back to back, with the LDS operand
// reads running several MFMAs ahead; in its softmax phase X(t) it masks S(t),
// updates the running max / sum and forms P(t).  Group A runs M(t) while
// group B runs X(t-1), then the roles swap, so each SIMD's matrix core always
// has one wave feeding it while the other wave does vector work.
//
// K and V tiles go from HBM/L2 straight into LDS (buffer_load_dwordx4 ... lds:
// lane l of a wave writes bytes [16 l, 16 l + 16) of a 1 KB LDS block, from
// any global address), so no registers stage them.  Since each lane chooses
// its source, the tiles are stored dense with their 16-byte units permuted
// (k_copy_off / v_copy_off below) so that the K reads (32 rows, one chunk
// each) and the transposed V reads (4 rows x 64 bytes per 32 lanes) hit
// distinct banks: D / 8 copies per tile, every lane useful.  The descriptor
// of a tile ends at its last valid key, so rows past Sk are zeros.  The
// copies are issued from inline assembly, so the compiler neither knows nor
// waits for them: the issuing wave waits for its own copies
// (s_waitcnt vmcnt(0)) right before the barrier that hands the data to the
// other waves, and the barriers themselves order LDS only.  Q is waited for
// before the key loop, so no wait the compiler places inside the loop can
// stall on a copy in flight.
//
// Online softmax runs in the log2 domain: s2 = s * scale * log2(e),
// p = exp2(s2 - m) on v_exp_f32, row statistics in fp32.  The running max m
// is raised (and O, l rescaled) only when some row's max grows by more than
// kRescaleLog2; between raises p <= 2^kRescaleLog2 stays far inside
// fp32/bf16 range.  The row sum adds the bf16-rounded p (the values the P.V
// product uses) with v_dot2_f32_bf16.
#include "attn_common.h"

#include <cmath>

namespace mk {
namespace {

using namespace attn;

// one scheduling group of Size instructions of class Mask (0x008 MFMA,
// 0x100 LDS read) at this point of the issue order
template <int Mask, int Size>
__device__ inline void sched_group() { __builtin_amdgcn_sched_group_barrier(Mask, Size, 0); }

constexpr int kBN = 64;     // keys per tile
constexpr float kRescaleLog2 = 8.f;       // lazy-rescale threshold (log2 units)

// ---- K and V tiles in LDS: 64 rows x D bf16, dense (CH = D / 8 16-byte
// chunks per row, 64 CH units per tile), with the units permuted so that the
// operand reads are bank-conflict free AND addressed as a per-lane base plus
// a constant of the k-step (an instruction immediate).  Unit u of a tile
// holds row r, chunk j:
//   K: u = 64 ((r/16) (CH/4) + j/4) + 4 (r % 16) + (j + r/4) % 4
//      one copy holds 16 rows x 4 chunks; its lanes 4 a .. 4 a + 3 fetch the
//      64 contiguous bytes of one row (rotated by r/4, so a quad of lanes is
//      one 64-byte request of the copy).  A K operand read (16 lanes per
//      pass: one chunk of each of 16 consecutive rows) falls on 16 distinct
//      units mod 16, i.e. each of the 64 banks once.
//   V: u = 4 CH (r/4) + 16 (j/4) + 4 (r % 4) + j % 4
//      each group of 4 rows is stored as 64-byte quads, quad-major with the 4
//      rows side by side, so the transposed read (32 lanes per pass: 4 rows x
//      one 64-byte quad) covers 256 distinct bytes.
// Copy n of a tile fills units 64 n .. 64 n + 63 (lane l: unit 64 n + l,
// fetched from the row and chunk below), so a tile is CH copies with no
// padding lanes.
template <int CH>
__device__ inline int k_copy_off(int u, int64_t ss) {  // byte offset in the tile of K unit u
  const int n = u >> 6, a = (u >> 2) & 15;
  const int row = 16 * (n / (CH / 4)) + a, ch = 4 * (n % (CH / 4)) + (((u & 3) - (a >> 2)) & 3);
  return (row * int(ss) + ch * 8) * 2;
}
template <int CH>
__device__ inline int v_copy_off(int u, int64_t ss) {  // byte offset in the tile of V unit u
  const int row = 4 * (u / (4 * CH)) + ((u >> 2) & 3), ch = 4 * ((u >> 4) % (CH / 4)) + (u & 3);
  return (row * int(ss) + ch * 8) * 2;
}
// Element offset of this lane's K operand (row c, chunk g of the k-step; one
// base for even and one for odd k-steps, ODD) and V operand (row
// 4 g + lane % 16 / 4, d 16 (lane / 16 % 2) + 4 (lane % 4)) in the tile; the
// parts of the step, added as immediates:
template <int CH>
__device__ inline int k_lane(int c, int g, int odd) {
  const int x = (g + ((c & 15) >> 2)) & 3;
  return 8 * (64 * (CH / 4) * (c >> 4) + 4 * (c & 15) + (x ^ (2 * odd)));
}
template <int D>
__device__ inline int v_lane(int lane) {
  return 32 * ((lane & 15) >> 2) + 4 * D * (lane >> 5) + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
}
// K: base k_lane(.., s % 2) + k_step(s) for the 16-deep k-step s, + 32 D for
// rows 32..63.
// V: + D kr + 128 db for rows kr.. (kr a multiple of 4), the 32-wide d block db.
constexpr int k_step(int s) { return 512 * (s / 2); }

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
  int head_group;    // > 0: XCD-grouped tile order (sdpa_fwd_kernel), heads per group
  float scale_log2;  // scale * log2(e)
};

// NW waves per workgroup (8: 256 query rows, one workgroup per CU; 4: 128
// rows, two workgroups per CU, for short sequences), in two groups of GW.
template <int D, bool CAUSAL, int NW>
__global__ __launch_bounds__(64 * NW, 8 / NW) void sdpa_fwd_kernel(const SdpaArgs p) {
  constexpr int GW = NW / 2;       // waves per group
  constexpr int kBM = 32 * NW;     // query rows per workgroup
  constexpr int CH = D / 8;      // 16-byte chunks of a row
  constexpr int NK = CH, NV = CH;          // 1 KB copies per tile (64 rows x CH units / 64 lanes)
  constexpr int NKW = (NK + GW - 1) / GW, NVW = (NV + GW - 1) / GW;  // per wave: the GW waves of one group issue a tile
  constexpr int NDB = D / 32;  // 32-wide d blocks of O
  constexpr int NKS = D / 16;  // 16-deep k-steps of Q·Kᵀ

  // K0, K1, V0, V1 in one LDS array (element offsets below)
  constexpr int kOffK1 = NK * 512, kOffV0 = 2 * NK * 512, kOffV1 = 2 * NK * 512 + NV * 512;
  __shared__ __attribute__((aligned(1024))) uint16_t kv_lds[2 * (NK + NV) * 512];
  auto buf_off = [](auto i, auto v) __attribute__((always_inline)) -> int {
    if constexpr (decltype(v)::value) return decltype(i)::value == 0 ? kOffV0 : kOffV1;
    else return decltype(i)::value == 0 ? 0 : kOffK1;
  };
  auto kbuf = [&](auto i) __attribute__((always_inline)) -> uint16_t* { return kv_lds + buf_off(i, Flag<false>{}); };
  auto vbuf = [&](auto i) __attribute__((always_inline)) -> uint16_t* { return kv_lds + buf_off(i, Flag<true>{}); };

  // heaviest (latest) query tiles first; consecutive ids walk over heads so
  // a head's tiles share an XCD when BH % 8 == 0
  const int id = blockIdx.x;
  int qt = CAUSAL ? (p.n_qtiles - 1 - id / p.BH) : (id / p.BH);
  int bh = id % p.BH;
  if (p.head_group > 0) {
    // Workgroups are dealt round-robin to the 8 XCDs (id % 8), each with its
    // own L2.  XCD x owns heads x BH/8 .. (x+1) BH/8 - 1 and runs them
    // head_group heads at a time, heaviest query tiles first within the
    // group: the workgroups of one head that start together stream the same
    // K/V tiles through that XCD's L2 (BH % (8 head_group) == 0).
    const int G = p.head_group, x = id % 8, j = id / 8, hx = p.BH / 8, nq = p.n_qtiles;
    const int r = j % (G * nq), gi = j / (G * nq);
    qt = CAUSAL ? nq - 1 - r / G : r / G;
    bh = x * hx + gi * G + r % G;
  }
  const int b = bh / p.H, h = bh % p.H;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave / GW;  // 0: group A, 1: group B (one phase later)
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
    // Q is in registers before the key loop starts.  Without this wait the
    // compiler waits for Q (vmcnt(0)) at the first use inside the loop, on
    // every trip, which would also wait out the K/V copies in flight.
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), expcnt/lgkmcnt untouched
  }

  int kv_end = p.Sk;
  if (CAUSAL) kv_end = min(kv_end, min(qt * kBM + kBM, p.Sq));  // one past the block's last query
  const int n_tiles = (kv_end + kBN - 1) / kBN;
  // tiles this wave computes (causal: those holding a key <= its last query)
  const int n_rel = CAUSAL ? min(n_tiles, (q0 + 31) / kBN + 1) : n_tiles;

  // ---- staging: global -> LDS.  Copy j (1 KB) of a tile is issued by wave
  // j % GW of the issuing group and fills LDS units 64 j + lane.
  // The lane's byte offset within a tile for copy i: with 8 waves they are
  // kept in registers; the 4-wave variant issues twice as many copies per
  // wave and recomputes them at each copy instead (a few integer ops), which
  // keeps it within 256 VGPRs.
  auto lane_off = [&](int i, auto is_v, int64_t ss) __attribute__((always_inline)) {
    const int u = 64 * (GW * i + (wave % GW)) + lane;
    if constexpr (decltype(is_v)::value) return v_copy_off<CH>(u, ss);
    else return k_copy_off<CH>(u, ss);
  };
  constexpr bool kKeepOff = NW == 8;
  int koff[kKeepOff ? NKW : 1], voff[kKeepOff ? NVW : 1];
  if constexpr (kKeepOff) {
#pragma unroll
    for (int i = 0; i < NKW; ++i) koff[i] = lane_off(i, Flag<false>{}, p.k_ss);
#pragma unroll
    for (int i = 0; i < NVW; ++i) voff[i] = lane_off(i, Flag<true>{}, p.v_ss);
  }
  // LDS byte address of this wave's first copy block in the array; the
  // empty asm at each use keeps the per-copy addresses (this + a constant)
  // from being hoisted out of the key loop, where they would only occupy
  // SGPRs (and spill): m0 costs one scalar add per copy instead.
  const uint32_t lds_wave = lds_addr(kv_lds) + uint32_t(wave % GW) * 1024u;
  auto dma = [&](const uint16_t* base, int64_t ss, const int* off, auto is_v, int n, int nw, int dst_off, int tile) __attribute__((always_inline)) {
    const int kv0 = tile * kBN;
    const int rows = min(kBN, p.Sk - kv0);  // valid keys in the tile (>= 1); rows >= D elements apart
    const i32x4_t r = tile_desc(base + int64_t(kv0) * ss, uint32_t((rows - 1) * ss + D) * 2u);
    uint32_t lw = lds_wave;
    asm volatile("" : "+s"(lw));
#pragma unroll
    for (int i = 0; i < nw; ++i)
      if (GW * i + (wave % GW) < n)  // wave-uniform
        copy_to_lds(r, lw + uint32_t(2 * dst_off + GW * i * 1024), kKeepOff ? off[i] : lane_off(i, is_v, ss));
  };
  auto dma_k = [&](int tile, auto buf) __attribute__((always_inline)) {
    dma(kb, p.k_ss, koff, Flag<false>{}, NK, NKW, buf_off(buf, Flag<false>{}), tile);
  };
  auto dma_v = [&](int tile, auto buf) __attribute__((always_inline)) {
    dma(vb, p.v_ss, voff, Flag<true>{}, NV, NVW, buf_off(buf, Flag<true>{}), tile);
  };

  const int vlane = v_lane<D>(lane);
  const int klane0 = k_lane<CH>(c, g, 0), klane1 = k_lane<CH>(c, g, 1);  // K row c, chunk g of the k-step

  f32x16_t o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = 0.f;
  f32x16_t s[2];            // S(t): from M(t) to X(t)
  bf16x8_t pf[2][2];        // P(t): from X(t) to M(t+1)
  float m_run = -INFINITY;  // running max, log2 domain
  float l_run = 0.f;        // this lane's share of the running row sum

  // ---- matrix phase M(t): S(t) = K[t]·Qᵀ (QK) and O += P(t-1)·V[t-1] (PV).
  // KB names K[t]'s buffer, VB V[t-1]'s.  The LDS reads are issued in the
  // order their MFMAs use them and run ahead by LA MFMAs; the issue order is
  // fixed with scheduling groups (left to itself the scheduler bunched the
  // reads and waited on a read issued just before its MFMA two or three
  // times per eight MFMAs).
  auto mphase = [&](auto kbi, auto vbi, auto do_qk, auto do_pv) __attribute__((always_inline)) {
    constexpr bool QK = decltype(do_qk)::value, PV = decltype(do_pv)::value;
    const uint16_t* ks = kbuf(kbi);
    const uint16_t* vs = vbuf(vbi);
    constexpr int NQ = QK ? 2 * NKS : 0;  // QK MFMAs (two 32-key chains)
    constexpr int NP = PV ? 4 * NDB : 0;  // PV MFMAs
    constexpr int N = NQ + NP;
    constexpr int MQP = NQ < NP ? NQ : NP;
    // MFMA order: QK and PV alternate while both remain, then the rest
    auto is_qk = [](int n) __attribute__((always_inline)) {
      return (QK && PV) ? ((n < 2 * MQP) ? (n % 2 == 0) : (NQ > NP)) : QK;
    };
    auto index = [](int n) __attribute__((always_inline)) {
      return (QK && PV) ? ((n < 2 * MQP) ? n / 2 : MQP + (n - 2 * MQP)) : n;
    };
    // A operand of MFMA n: K rows (QK) or Vᵀ from two transposed reads (PV)
    auto load_op = [&](int n) __attribute__((always_inline)) -> u32x4_t {
      const int i = index(n);
      if (is_qk(n))
        return *reinterpret_cast<const u32x4_t*>(&ks[((i >> 1) & 1 ? klane1 : klane0) + (i & 1) * 32 * D + k_step(i >> 1)]);
      const int kstep = 16 * (i / NDB), db = i % NDB;
      const uint2 lo = lds_read_tr(&vs[vlane + kstep * D + db * 128]);
      const uint2 hi = lds_read_tr(&vs[vlane + (kstep + 8) * D + db * 128]);
      return u32x4_t{lo.x, lo.y, hi.x, hi.y};
    };
    if constexpr (QK) {
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[kb2][r] = 0.f;
    }
    // operands are read LA MFMAs ahead of their use (a ring of LA registers)
    constexpr int LA = 4;
    u32x4_t ring[LA];
#pragma unroll
    for (int n = 0; n < LA && n < N; ++n) ring[n] = load_op(n);
#pragma unroll
    for (int n = 0; n < N; ++n) {
      const u32x4_t a = ring[n % LA];
      if (n + LA < N) ring[n % LA] = load_op(n + LA);
      const int i = index(n);
      if (is_qk(n)) {
        if constexpr (QK) s[i & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), qf[i >> 1], s[i & 1], 0, 0, 0);
      } else {
        if constexpr (PV) {
          const int kb2 = i / (2 * NDB), j2 = (i / NDB) % 2, db = i % NDB;
          o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), pf[kb2][j2], o[db], 0, 0, 0);
        }
      }
    }
    // issue order: the reads of the first LA operands, then MFMA n followed
    // by the reads of operand n + LA (one ds_read_b128 for K, two transposed
    // reads for V)
#pragma unroll
    for (int n = 0; n < LA && n < N; ++n) {
      if (is_qk(n)) sched_group<0x100, 1>();
      else sched_group<0x100, 2>();
    }
#pragma unroll
    for (int n = 0; n < N; ++n) {
      sched_group<0x008, 1>();
      if (n + LA < N) {
        if (is_qk(n + LA)) sched_group<0x100, 1>();
        else sched_group<0x100, 2>();
      }
    }
  };

  // ---- softmax phase X(t): mask S(t), running max / rescale, P(t), row sum
  auto xphase = [&](int tt) __attribute__((always_inline)) {
    const int kv0 = tt * kBN;
    if ((CAUSAL && kv0 + kBN - 1 > q0) || kv0 + kBN > p.Sk) {
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kv0 + kb2 * 32 + 8 * (r / 4) + 4 * g + (r % 4);
          if (key >= p.Sk || (CAUSAL && key > qrow)) s[kb2][r] = -INFINITY;
        }
    }
    float mt = s[0][0];
#pragma unroll
    for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
      for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[kb2][r]);
    {
      float lo, hi;
      lane_halves(mt, lo, hi);
      mt = fmaxf(lo, hi);
    }
    const float m_cand = fmaxf(m_run, mt * p.scale_log2);
    // m_run == -inf until the row has seen an unmasked key, so the first
    // such tile always rescales (alpha = 0 on O = 0, l = 0)
    if (__builtin_amdgcn_ballot_w64(m_cand > m_run + kRescaleLog2) != 0) {
      // rows with no unmasked key yet keep m = -inf and alpha = 1
      const float alpha = (m_cand == m_run) ? 1.f : __builtin_amdgcn_exp2f(m_run - m_cand);
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
        pf[kb2][j2] = as_bf16x8(w);
      }
    l_run += ls0 + ls1;
    // P and l are complete before the phase ends.  The barrier and its LDS
    // fences order memory operations only, so without this the compiler
    // sinks the exponentials (pure VALU work) past the next barrier into this
    // wave's own matrix phase, where in-order issue stalls its MFMA stream
    // while the other wave of the SIMD waits at the following barrier.
    asm volatile("" ::"v"(pf[0][0]), "v"(pf[0][1]), "v"(pf[1][0]), "v"(pf[1][1]), "v"(l_run));
  };

  // M(t) for this wave: QK when t < n_rel, PV when 1 <= t <= n_rel.
  // KP = t % 2 (K[t] in K<KP>, V[t-1] in V<1-KP>).
  auto mstep = [&](int tt, auto kp) __attribute__((always_inline)) {
    constexpr int KP = decltype(kp)::value;
    const bool qk = tt < n_rel, pv = tt >= 1 && tt <= n_rel;
    if (qk && pv) mphase(Int<KP>{}, Int<1 - KP>{}, Flag<true>{}, Flag<true>{});
    else if (qk) mphase(Int<KP>{}, Int<1 - KP>{}, Flag<true>{}, Flag<false>{});
    else if (pv) mphase(Int<KP>{}, Int<1 - KP>{}, Flag<false>{}, Flag<true>{});
  };
  auto xstep = [&](int tt) __attribute__((always_inline)) {
    if (tt >= 0 && tt < n_rel) xphase(tt);
  };

  // Phases M(t) X(t) M(t+1) X(t+1) for an even t.  STEADY: every wave has
  // both products in both M phases and a softmax in both X phases, and no
  // wave's sequence ends here, so the phases are fixed code (the running O
  // stays in the same registers from pair to pair).  Returns true when this
  // wave's last phase has run.
  auto pair = [&](int t, auto steady) __attribute__((always_inline)) -> bool {
    constexpr bool ST = decltype(steady)::value;
    // ---- M(t) (A at t == 0: phase 0's barrier was the one before the loop)
    if (grp == 0) {
      if (t > 0) {
        wait_copies();  // V[t-1] (started in X(t-1)) is read from this phase on
        lds_barrier();
      }
    } else {
      lds_barrier();
    }
    if constexpr (ST) mphase(Int<0>{}, Int<1>{}, Flag<true>{}, Flag<true>{});
    else mstep(t, Int<0>{});
    if (!ST && t == n_tiles && grp == 1) return true;  // B's last phase was M(n_tiles)
    // ---- X(t)
    if (grp == 0) {
      lds_barrier();
      if (ST || t < n_tiles) dma_v(t, Int<0>{});
    } else {
      wait_copies();  // K[t+1] (started in X(t-1)) is read from this phase on
      lds_barrier();
      if (t + 2 < n_tiles) dma_k(t + 2, Int<0>{});
    }
    if constexpr (ST) xphase(t);
    else xstep(t);
    if (!ST && t == n_tiles) return true;
    // ---- M(t+1), t+1 odd
    if (grp == 0) wait_copies();  // V[t]
    lds_barrier();
    if constexpr (ST) mphase(Int<1>{}, Int<0>{}, Flag<true>{}, Flag<true>{});
    else mstep(t + 1, Int<1>{});
    if (!ST && t + 1 == n_tiles && grp == 1) return true;
    // ---- X(t+1)
    if (grp == 0) {
      lds_barrier();
      if (ST || t + 1 < n_tiles) dma_v(t + 1, Int<1>{});
    } else {
      wait_copies();  // K[t+2]
      lds_barrier();
      if (t + 3 < n_tiles) dma_k(t + 3, Int<1>{});
    }
    if constexpr (ST) xphase(t + 1);
    else xstep(t + 1);
    return false;
  };

  // Global phases: group A runs M(t) in phase 2t and X(t) in 2t+1, group B
  // one phase later.  Each wave runs its own M(0) X(0) M(1) X(1) ... with a
  // barrier before every phase; B waits out phase 0 first, so barriers pair
  // up by count.  Copies are started only by the group in its softmax phase,
  // never by the group issuing MFMAs:
  //   A starts V[t] (into V<t%2>, last read in phase 2t-1) at the start of
  //     X(t), phase 2t+1, and waits for it before the barrier of phase 2t+2,
  //     where M(t+1) first reads it;
  //   B starts K[t+2] (into K<t%2>, last read in phase 2t+1) at the start of
  //     X(t), phase 2t+2, and waits for it before the barrier of phase 2t+4,
  //     where M(t+2) first reads it.
  // Phases end at 2 n_tiles + 1 (B's M(n_tiles)).  The pairs from t = 2 up
  // to the last one in which wave 0 (the one with the fewest tiles under the
  // causal mask) still has both products are steady for every wave; the
  // first pair and the ragged tail run the general code.  The steady trip
  // count is the same for all waves, so the barriers still pair up.
  if (n_tiles > 0) {
    if (grp == 1) {  // K[0] before phase 0, K[1] during it (B has no softmax yet)
      dma_k(0, Int<0>{});
      wait_copies();
      lds_barrier();
      if (1 < n_tiles) dma_k(1, Int<1>{});
    } else {
      lds_barrier();
    }
    const int n_rel_min = CAUSAL ? min(n_tiles, (qt * kBM + 31) / kBN + 1) : n_tiles;
    if (!pair(0, Flag<false>{})) {
      int t = 2;
      for (; t + 2 <= n_rel_min; t += 2) pair(t, Flag<true>{});
      for (; t <= n_tiles; t += 2)
        if (pair(t, Flag<false>{})) break;
    }
  }

  // ---- epilogue: normalise and store O (lane owns query qrow, 4 consecutive d per reg group)
  float l_lo, l_hi;
  lane_halves(l_run, l_lo, l_hi);
  const float l_tot = l_lo + l_hi;
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


// ---------------------------------------------------------------- wide waves
// One workgroup = 4 waves (one per SIMD) = 256 query rows of one (b, h); wave
// w owns rows 64 w .. 64 w + 63 as two 32-row blocks.  Every K or Vᵀ operand
// read from LDS feeds two MFMAs (one per row block), which halves the LDS
// read traffic per MFMA of the 8-wave kernel above: there each wave owns 32
// rows, and the waves of a phase read 1 KB of LDS per 32-cycle MFMA, the
// CU's whole LDS read bandwidth (removing the reads there saves a third of
// the time).
// Keys are processed in halves of 32 (half h = keys 32 h .. 32 h + 31), and
// with one wave per SIMD the matrix core is fed from within the wave.  Step h:
//   rescale O if softmax(h) raised a row's max (rare; a wave-uniform branch),
//   O += P(h) · V(h)  with  softmax(S(h+1)) -> P(h+1)   (MFMAs and VALU work
//   on disjoint registers, one basic block: the compiler interleaves them),
//   S(h+2) = K(h+2) · Qᵀ.
// S and P each alternate between two register sets, so the live state is O
// (128 registers at D = 128), Q (64), 2 x 32 scores, 2 x 16 P: the O
// accumulators go to AGPRs, the rest fits the 256 VGPRs.
// K/V tiles of 64 keys are staged as in the 8-wave kernel (same LDS layouts
// and copies, split over the 4 waves), one barrier per tile: at the start of
// step 2t, after which K(t+1) and V(t) are visible and K(t), V(t-1) free.
// Online softmax in the log2 domain with lazy rescale as above, written
// without branches (selects) so that it stays in the interleaved block.
template <int D, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void sdpa_fwd_wide_kernel(const SdpaArgs p) {
  constexpr int NW = 4, QB = 2;     // waves, 32-row blocks per wave
  constexpr int kBM = 64 * NW;      // query rows per workgroup
  constexpr int CH = D / 8;
  constexpr int NK = CH, NV = CH;
  constexpr int NKW = (NK + NW - 1) / NW, NVW = (NV + NW - 1) / NW;
  constexpr int NDB = D / 32, NKS = D / 16;
  constexpr int kOffK1 = NK * 512, kOffV0 = 2 * NK * 512, kOffV1 = 2 * NK * 512 + NV * 512;
  __shared__ __attribute__((aligned(1024))) uint16_t kv_lds[2 * (NK + NV) * 512];

  const int id = blockIdx.x;
  const int qt = CAUSAL ? (p.n_qtiles - 1 - id / p.BH) : (id / p.BH);
  const int bh = id % p.BH;
  const int b = bh / p.H, h = bh % p.H;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 31, g = lane >> 5;
  const int q0 = qt * kBM + wave * 64;  // first query row of this wave

  const uint16_t* qb = p.q + b * p.q_bs + h * p.q_hs;
  const uint16_t* kb = p.k + b * p.k_bs + h * p.k_hs;
  const uint16_t* vb = p.v + b * p.v_bs + h * p.v_hs;

  bf16x8_t qf[QB][NKS];
#pragma unroll
  for (int r = 0; r < QB; ++r) {
    const int qrow = q0 + 32 * r + c;
    const bool ok = qrow < p.Sq;
#pragma unroll
    for (int s = 0; s < NKS; ++s) {
      u32x4_t v = {0u, 0u, 0u, 0u};
      if (ok) v = *reinterpret_cast<const u32x4_t*>(qb + int64_t(qrow) * p.q_ss + 16 * s + 8 * g);
      qf[r][s] = as_bf16x8(v);
    }
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // Q has landed before any copy is in flight
  int kv_end = p.Sk;
  if (CAUSAL) kv_end = min(kv_end, min(qt * kBM + kBM, p.Sq));
  const int n_tiles = (kv_end + kBN - 1) / kBN;
  const int n_rel = CAUSAL ? min(n_tiles, (q0 + 63) / kBN + 1) : n_tiles;  // this wave's tiles
  const int n_half = 2 * n_rel;

  // copies: copy j of a tile by wave j % 4; lane offsets kept in registers
  int koff[NKW], voff[NVW];
#pragma unroll
  for (int i = 0; i < NKW; ++i) koff[i] = k_copy_off<CH>(64 * (NW * i + wave) + lane, p.k_ss);
#pragma unroll
  for (int i = 0; i < NVW; ++i) voff[i] = v_copy_off<CH>(64 * (NW * i + wave) + lane, p.v_ss);
  const uint32_t lds_wave = lds_addr(kv_lds) + uint32_t(wave) * 1024u;
  auto dma = [&](const uint16_t* base, int64_t ss, const int* off, int n, int nw, int dst_off, int tile) __attribute__((always_inline)) {
    const int kv0 = tile * kBN;
    const int rows = min(kBN, p.Sk - kv0);
    const i32x4_t r = tile_desc(base + int64_t(kv0) * ss, uint32_t((rows - 1) * ss + D) * 2u);
    uint32_t lw = lds_wave;
    asm volatile("" : "+s"(lw));
#pragma unroll
    for (int i = 0; i < nw; ++i)
      if (NW * i + wave < n) copy_to_lds(r, lw + uint32_t(2 * dst_off + NW * i * 1024), off[i]);
  };
  auto dma_k = [&](int tile, int buf) __attribute__((always_inline)) {
    dma(kb, p.k_ss, koff, NK, NKW, buf ? kOffK1 : 0, tile);
  };
  auto dma_v = [&](int tile, int buf) __attribute__((always_inline)) {
    dma(vb, p.v_ss, voff, NV, NVW, buf ? kOffV1 : kOffV0, tile);
  };

  const int vlane = v_lane<D>(lane);
  const int klane0 = k_lane<CH>(c, g, 0), klane1 = k_lane<CH>(c, g, 1);

  f32x16_t o[QB][NDB];
#pragma unroll
  for (int r = 0; r < QB; ++r)
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[r][db][e] = 0.f;
  f32x16_t sc[2][QB];     // S(h) in set h % 2
  bf16x8_t pf[2][QB][2];  // P(h) in set h % 2: [row block][16-key step]
  float m_run[QB] = {-INFINITY, -INFINITY}, l_run[QB] = {0.f, 0.f};
  float alpha[QB] = {1.f, 1.f};  // O rescale owed by the last softmax

  // S(hh) = K(hh) · Qᵀ: key half hh % 2 of the tile in K<buffer>; each K
  // operand (16-deep step) is read once and used for both row blocks
  auto qk = [&](int set, int kbuf, int half) __attribute__((always_inline)) {
    const uint16_t* ks = kv_lds + (kbuf ? kOffK1 : 0) + half * 32 * D;
#pragma unroll
    for (int r = 0; r < QB; ++r)
#pragma unroll
      for (int e = 0; e < 16; ++e) sc[set][r][e] = 0.f;
#pragma unroll
    for (int st = 0; st < NKS; ++st) {
      const u32x4_t a = *reinterpret_cast<const u32x4_t*>(&ks[(st & 1 ? klane1 : klane0) + k_step(st)]);
#pragma unroll
      for (int r = 0; r < QB; ++r)
        sc[set][r] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), qf[r][st], sc[set][r], 0, 0, 0);
    }
  };
  // O += P(hh) · V(hh): key half hh % 2 of the tile in V<buffer>; each Vᵀ
  // operand (16-key step, d block; two transposed reads) used twice
  auto pv = [&](int set, int vbuf, int half) __attribute__((always_inline)) {
    const uint16_t* vs = kv_lds + (vbuf ? kOffV1 : kOffV0) + half * 32 * D;
#pragma unroll
    for (int i = 0; i < 2 * NDB; ++i) {
      const int kst = i / NDB, db = i % NDB;
      const uint2 lo = lds_read_tr(&vs[vlane + 16 * kst * D + db * 128]);
      const uint2 hi = lds_read_tr(&vs[vlane + (16 * kst + 8) * D + db * 128]);
      const u32x4_t a = {lo.x, lo.y, hi.x, hi.y};
#pragma unroll
      for (int r = 0; r < QB; ++r)
        o[r][db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), pf[set][r][kst], o[r][db], 0, 0, 0);
    }
  };
  // softmax of S(hh) into P(hh), in two parts.  softmax_max: mask (MASK),
  // running max, alpha (the O rescale owed) and the exponent offset; it ends
  // with the cross-lane exchange (v_permlane32_swap ends a scheduling region).
  // softmax_exp: P = 2^(s scale - m) packed to bf16, row sum; pure VALU work
  // that the compiler can interleave with the MFMAs around it.
  float m_use[QB];
  auto softmax_max = [&](int set, int hh, auto masked) __attribute__((always_inline)) {
    constexpr bool MASK = decltype(masked)::value;
    const int k0 = hh * 32;  // first key of the half
    float mt[QB];
#pragma unroll
    for (int r = 0; r < QB; ++r) {
      const int qrow = q0 + 32 * r + c;
      if constexpr (MASK) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int key = k0 + 8 * (e / 4) + 4 * g + (e % 4);
          if (key >= p.Sk || (CAUSAL && key > qrow)) sc[set][r][e] = -INFINITY;
        }
      }
      mt[r] = sc[set][r][0];
#pragma unroll
      for (int e = 1; e < 16; ++e) mt[r] = fmaxf(mt[r], sc[set][r][e]);
    }
#pragma unroll
    for (int r = 0; r < QB; ++r) {
      float lo, hi;
      lane_halves_sched(mt[r], lo, hi);
      const float m_old = m_run[r];
      const float m_cand = fmaxf(m_old, fmaxf(lo, hi) * p.scale_log2);
      // raise the max only when it grows by more than kRescaleLog2; a row
      // with no unmasked key yet keeps -inf (alpha 1, p = 0)
      const float m_new = (m_cand > m_old + kRescaleLog2) ? m_cand : m_old;
      const bool none = m_new == -INFINITY;
      m_use[r] = none ? 0.f : m_new;
      // alpha = 2^(m_old - m_new): 1 when not raised, 0 from -inf (the
      // exponent is clamped at -256, where exp2 is 0)
      alpha[r] = __builtin_amdgcn_exp2f(none ? 0.f : fmaxf(m_old - m_new, -256.f));
      m_run[r] = m_new;
    }
  };
  auto softmax_exp = [&](int set) __attribute__((always_inline)) {
    const bf16x2_t one = {static_cast<__bf16>(1.f), static_cast<__bf16>(1.f)};
#pragma unroll
    for (int r = 0; r < QB; ++r) {
      float ls0 = 0.f, ls1 = 0.f;
#pragma unroll
      for (int j2 = 0; j2 < 2; ++j2) {
        u32x4_t w;
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
          const f32x2_t e = {__builtin_amdgcn_exp2f(fmaf(sc[set][r][8 * j2 + i], p.scale_log2, -m_use[r])),
                             __builtin_amdgcn_exp2f(fmaf(sc[set][r][8 * j2 + i + 1], p.scale_log2, -m_use[r]))};
          const bf16x2_t pr = __builtin_convertvector(e, bf16x2_t);
          w[i / 2] = __builtin_bit_cast(uint32_t, pr);
          if (i & 2) ls1 = __builtin_amdgcn_fdot2_f32_bf16(pr, one, ls1, false);
          else ls0 = __builtin_amdgcn_fdot2_f32_bf16(pr, one, ls0, false);
        }
        pf[set][r][j2] = as_bf16x8(w);
      }
      l_run[r] = l_run[r] * alpha[r] + (ls0 + ls1);
    }
  };
  auto rescale = [&]() __attribute__((always_inline)) {
    if (__builtin_amdgcn_ballot_w64(alpha[0] != 1.f || alpha[1] != 1.f) != 0) {
#pragma unroll
      for (int r = 0; r < QB; ++r)
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int e = 0; e < 16; ++e) o[r][db][e] *= alpha[r];
    }
  };

  // Step hh (see the header).  HP = hh % 2 (the half within tile hh / 2,
  // and the P / S register sets).  STEADY: every wave has all three parts
  // and no mask.
  auto step = [&](int hh, auto hp, auto steady) __attribute__((always_inline)) {
    constexpr int HP = decltype(hp)::value;
    constexpr bool ST = decltype(steady)::value;
    const int t = hh >> 1;  // tile of half hh
    if constexpr (HP == 0) {
      wait_copies();
      lds_barrier();
      if (t + 2 < n_tiles) dma_k(t + 2, t & 1);
      if (t + 1 < n_tiles) dma_v(t + 1, (t + 1) & 1);
    }
    if (ST || hh < n_half) rescale();
    if constexpr (ST) {
      // P·V of half hh, softmax of hh + 1, S of half hh + 2 (the same half
      // of tile t + 1)
      softmax_max(1 - HP, hh + 1, Flag<false>{});
      pv(HP, t & 1, HP);
      softmax_exp(1 - HP);
      qk(HP, (t + 1) & 1, HP);
    } else {
      if (hh + 1 < n_half) softmax_max(1 - HP, hh + 1, Flag<true>{});
      if (hh < n_half) pv(HP, t & 1, HP);
      if (hh + 1 < n_half) softmax_exp(1 - HP);
      if (hh + 2 < n_half) qk(HP, (t + 1) & 1, HP);
    }
  };

  if (n_tiles > 0) {
    dma_k(0, 0);
    wait_copies();
    lds_barrier();
    if (1 < n_tiles) dma_k(1, 1);
    dma_v(0, 0);
    // S(0), S(1) (every wave has key tile 0), softmax(0)
    qk(0, 0, 0);
    qk(1, 0, 1);
    softmax_max(0, 0, Flag<true>{});
    softmax_exp(0);
    // steady tiles: all waves active and tiles t, t + 1 unmasked for every
    // wave (wave 0 has the fewest tiles under the causal mask; its last one
    // is its diagonal tile)
    const int n_rel_min = CAUSAL ? min(n_tiles, (qt * kBM + 63) / kBN + 1) : n_tiles;
    const int n_steady = max(0, min(n_rel_min - 1, p.Sk / kBN));
    int t = 0;
    for (; t + 1 < n_steady; ++t) {
      step(2 * t, Int<0>{}, Flag<true>{});
      step(2 * t + 1, Int<1>{}, Flag<true>{});
    }
    for (; t < n_tiles; ++t) {
      step(2 * t, Int<0>{}, Flag<false>{});
      step(2 * t + 1, Int<1>{}, Flag<false>{});
    }
  }

  // ---- epilogue (per row block, as in the 8-wave kernel)
#pragma unroll
  for (int r = 0; r < QB; ++r) {
    const int qrow = q0 + 32 * r + c;
    float l_lo, l_hi;
    lane_halves(l_run[r], l_lo, l_hi);
    const float l_tot = l_lo + l_hi;
    if (qrow < p.Sq) {
      const float inv = (l_tot > 0.f) ? 1.f / l_tot : __builtin_nanf("");
      uint16_t* ob = p.o + b * p.o_bs + h * p.o_hs + int64_t(qrow) * p.o_ss;
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const int d = db * 32 + 8 * r4 + 4 * g;
          const f32x2_t lo = {o[r][db][4 * r4 + 0] * inv, o[r][db][4 * r4 + 1] * inv};
          const f32x2_t hi = {o[r][db][4 * r4 + 2] * inv, o[r][db][4 * r4 + 3] * inv};
          uint2 w;
          w.x = __builtin_bit_cast(uint32_t, __builtin_convertvector(lo, bf16x2_t));
          w.y = __builtin_bit_cast(uint32_t, __builtin_convertvector(hi, bf16x2_t));
          *reinterpret_cast<uint2*>(ob + d) = w;
        }
      }
      if (p.lse && g == 0) {
        const float lse2 = (l_tot > 0.f) ? m_run[r] + log2f(l_tot) : -INFINITY;
        p.lse[int64_t(bh) * p.Sq + qrow] = lse2 * 0.69314718055994531f;
      }
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
  a.BH = int(B * H);
  a.scale_log2 = scale * 1.4426950408889634f;
  // 256 query rows per workgroup unless that grid would leave the GPU short
  // of workgroups: then the 4-wave kernel (128 rows, two workgroups per CU).
  // At 256 rows, head_dim 128 runs the 8-wave ping-pong kernel and head_dim
  // 64 the wide-wave kernel (measured, warm clocks, causal B4 H16 S8192:
  // D 128 8-wave 1029 / wide 901 TFLOP/s; D 64 8-wave 775 / wide 922)
  const int64_t blocks256 = ((Sq + 255) / 256) * a.BH;
  const bool rows256 = blocks256 >= 2 * 256;  // 256 CUs
  const int rows = rows256 ? 256 : 128;
  a.n_qtiles = int((Sq + rows - 1) / rows);
  const int64_t blocks = int64_t(a.n_qtiles) * a.BH;
  // XCD-grouped order for long sequences on the 8-wave kernel (measured,
  // causal B4 H16 D128: S=8192 +1.3 to +3%, S=16384 +5 to +7%; at S <= 4096
  // the late start of the last group's heavy tiles costs more than the L2
  // reuse gains, -1% at 4096 and -17% at 2048, so those keep the linear order)
  a.head_group = (rows256 && D == 128 && a.n_qtiles >= 32 && a.BH % 16 == 0) ? 2 : 0;
  if (blocks >= (int64_t(1) << 31)) return fail(MK_ERR_UNSUPPORTED, "mk_sdpa_fwd: grid too large");
  hipStream_t s = as_stream(stream);
  const dim3 g{unsigned(blocks)};
  auto go = [&](auto nwt) {
    constexpr int NW = decltype(nwt)::value;
    const dim3 bl{unsigned(64 * NW)};
    if (D == 128) {
      if (causal) hipLaunchKernelGGL((sdpa_fwd_kernel<128, true, NW>), g, bl, 0, s, a);
      else hipLaunchKernelGGL((sdpa_fwd_kernel<128, false, NW>), g, bl, 0, s, a);
    } else {
      if (causal) hipLaunchKernelGGL((sdpa_fwd_kernel<64, true, NW>), g, bl, 0, s, a);
      else hipLaunchKernelGGL((sdpa_fwd_kernel<64, false, NW>), g, bl, 0, s, a);
    }
  };
  if (!rows256) go(Int<4>{});
  else if (D == 128) go(Int<8>{});
  else if (causal) hipLaunchKernelGGL((sdpa_fwd_wide_kernel<64, true>), g, dim3(256), 0, s, a);
  else hipLaunchKernelGGL((sdpa_fwd_wide_kernel<64, false>), g, dim3(256), 0, s, a);
  return check_launch("mk_sdpa_fwd");
}
