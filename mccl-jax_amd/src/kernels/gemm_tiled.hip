// Large bf16 GEMM on MFMA for dot_general: mk_gemm's kernel for products
// with enough output tiles to fill the chip (gemm.hip keeps the general
// kernel for fp32, odd strides and small products).
//   C[b] = A[b] · B[b] (+ bias)(ReLU), fp32 accumulate, bf16 / f16 / f32 out.
//
// Workgroup tile TM x TN, k in BK-deep tiles, WGM x WGN waves each owning a
// (TM / WGM) x (TN / WGN) block of the tile as 32 x 32 v_mfma_f32_32x32x16_bf16
// blocks.  The MFMA is issued with B's rows as its first operand, so a lane's
// accumulator holds 4 consecutive C columns of one C row (lane (c, g), reg r:
// row c, column 8 (r / 4) + 4 g + r % 4 of its 32 x 32 block).
//
// Operand tiles go from HBM/L2 straight into LDS with buffer_load_dwordx4 ...
// lds (attn_common.h: lane l writes bytes 16 l .. 16 l + 15 of a 1 KB LDS
// block, loaded from any offset of the operand), in S stages: the copies of
// k tile t + S - 1 are issued before tile t is multiplied, one barrier per
// tile.  Each operand keeps the orientation it has in memory:
//   k-contiguous (A[m][k], or B stored as [n][k]): LDS rows of BK k, 16-byte
//     chunk c of row r stored at chunk position c ^ ((r >> 1) & 7) (BK = 64)
//     or c ^ ((r >> 2) & 3) (BK = 32), read with one ds_read_b128 per MFMA
//     operand (8 consecutive k);
//   m- / n-contiguous (A stored as [k][m], B[k][n]): one LDS row of R columns
//     per k, chunk c of k-row r stored at position c ^ 4 (r & 3) (R a
//     multiple of 128) or c ^ 4 ((r >> 1) & 1) (R = 192), read with two
//     ds_read_b64_tr_b16 per operand, which hand each lane one column over 4
//     consecutive k (k-rows 8g .. 8g + 3, then 8g + 4 .. 8g + 7).
// Both forms give lane (c, g) of an MFMA operand column/row c and k = 8 g ..
// 8 g + 7 in order, so any pairing of orientations multiplies correctly.
// The XOR placements make every read conflict-free on gfx950's LDS (64 banks
// of 4 bytes): a ds_read_b128 serves 16 lanes per cycle, which must cover
// all 256 bank bytes, here 16 rows at one chunk; a ds_read_b64_tr_b16 serves
// 32 lanes, here 4 k-rows x 4 chunks.  (An XOR with r & 7, or 2 (r & 3),
// leaves two rows of each group on the same banks and halves the read rate.)
// Chunks past M, N or K are loaded from an out-of-range buffer offset, which
// reads zeros.  A chunk that straddles M or N (an m- / n-contiguous operand
// whose extent is not a multiple of 8) is loaded whole: its extra elements
// lie inside the row pitch (or past the buffer's range, reading zeros) and
// only reach C rows / columns that are never stored.  A chunk that straddles
// K (a k-contiguous operand, K not a multiple of 8) is loaded whole too.  In
// the last k tile the wave that copied a straddling chunk rewrites it in LDS
// (between two barriers) from the operand, element by element, with zeros
// past the end: K-straddling chunks then add exact zeros whatever the row
// pitch held, and the operand's last row, whose straddling chunk ran past
// the buffer range (read as zeros), gets its valid elements back.
//
// Tile order: workgroups are dealt round-robin to the 8 XCDs, each with its
// own L2, so workgroup i takes tile (i % 8) * (tiles / 8) + i / 8 of an
// order that walks groups of 4 tile rows column by column: the tiles an XCD
// runs at once form a compact 4 x 8 block, whose A rows and B columns are
// fetched into that XCD's L2 once for 8 and 4 tiles respectively.
// (The reference's dot_general materialises operand transposes first,
// src/jam/ops/linalg.mm:34-45; no operand is copied in HBM here.)
#include <atomic>

#include "attn_common.h"

namespace mk {
namespace {

using namespace attn;

constexpr int kGroupM = 4;                  // tile rows per group of the tile order
constexpr int kInvalid = int(0x80000000u);  // buffer offset past every accepted range

struct TiledGemm {
  const void* A;
  const void* B;
  void* C;
  const void* bias;
  int64_t M, N, K;
  int64_t k_rem;              // > 0: K of the last batch (a split-K's last, shorter slice)
  int64_t lda, ldb, ldc;      // element stride of A's, B's, C's non-unit dimension
  int64_t a_bs, b_bs, c_bs;   // batch strides (elements)
  uint32_t a_bytes, b_bytes;  // bytes addressable from one batch's A / B base
  int tiles_m, tiles_n;
  int epilogue;               // 0 none, 1 + bias, 2 + bias then ReLU; | 4: the bias is fp32;
                              // | kEpiGeluAux: aux = bf16 gelu_tanh of each stored value
  uint16_t* aux;
  int64_t ld_aux;
  float* colpart;             // kEpiGeluBwd: column sums per 128 rows
  int c_type;
  int c_mode;                 // 0 element stores, 1 4-column vector stores, 2 / 3 staged 16-bit rows
                              // stored as 16-byte chunks / element by element, 4 / 5 staged fp32 rows
                              // stored element by element / as 16-byte chunks
};

// The copies one wave makes of one operand's tile: copy c is j = wave + W c
// (W waves), lane l of it writes LDS chunk position u = 64 j + l of the tile.
//   KC:  LDS row u / (BK / 8), position u % (BK / 8), holding global chunk
//        position ^ kc_swizzle(row)
//   !KC: LDS k-row u / (R / 8), position u % (R / 8), holding global chunk
//        position ^ 2 (k-row & 3)
// Each copy keeps its byte offset for the first k tile (an out-of-range
// offset when its row is outside the operand) and the first k it reads (past
// every K for such a row).  A k tile wholly inside K passes t times the
// per-tile step as the instruction's SGPR offset, so its copies need no
// vector arithmetic; only the tile that crosses K compares each copy's k.
// chunk placement of a k-contiguous LDS row (BK / 8 chunks): the 16 rows one
// ds_read_b128 cycle reads at one chunk land on 16 different 16-byte bank
// groups (rows 2 (64 B) or 4 (32 B) apart share the row's bank offset)
template <int BK>
__device__ inline int kc_swizzle(int row) {
  return BK == 64 ? ((row >> 1) & 7) : ((row >> 2) & 3);
}

// chunk placement of an m- / n-contiguous LDS k-row (R / 8 chunks): the 4
// k-rows x 4 chunks of one ds_read_b64_tr_b16 half-wave land on 16 different
// bank groups; the XOR keeps each chunk inside its aligned group of 8 (R =
// 192) or 16 chunks
template <int R>
__device__ inline int nc_swizzle(int kr) {
  static_assert(R % 64 == 0, "k-row of whole 8-chunk groups");
  return R % 128 == 0 ? 4 * (kr & 3) : 4 * ((kr >> 1) & 1);
}

template <bool KC, int R, int BK, int kC, int W>
struct Copies {
  uint32_t off[kC];
  int32_t k[kC];
  __device__ inline Copies(int wave, int lane, int64_t r0, int64_t rows, int64_t ld) {
#pragma unroll
    for (int c = 0; c < kC; ++c) {
      const int u = 64 * (wave + W * c) + lane;
      int64_t gr, gk;
      if constexpr (KC) {
        constexpr int kCpr = BK / 8;
        const int row = u / kCpr;
        gr = r0 + row;
        gk = 8 * ((u % kCpr) ^ kc_swizzle<BK>(row));
        off[c] = uint32_t((gr * ld + gk) * 2);
      } else {
        constexpr int kCpr = R / 8;
        const int kr = u / kCpr;
        gr = r0 + 8 * ((u % kCpr) ^ nc_swizzle<R>(kr));
        gk = kr;
        off[c] = uint32_t((gk * ld + gr) * 2);
      }
      k[c] = gr < rows ? int32_t(gk) : 0x7fffffff - BK;
      if (gr >= rows) off[c] = uint32_t(kInvalid);  // kInvalid + any step stays past every range
    }
  }
  // offset for the k tile starting at k0 (step: its byte distance from the
  // first), or an offset that reads zeros once the chunk lies past K
  __device__ inline int at(int c, int k0, uint32_t step, int64_t K) const {
    return int64_t(k[c]) + k0 < K ? int(off[c] + step) : kInvalid;
  }
  // Chunks of the last k tile (k0) that straddle the operand's end: along
  // K for a k-contiguous operand (K % 8 != 0), along the rows for an m- /
  // n-contiguous one (rows % 8 != 0).  The copy loaded such a chunk whole,
  // so its elements past the end hold whatever the row pitch held, and in the
  // operand's last row (k-row) the part past the buffer range read as zeros.
  // Called between two barriers once the tile is in LDS: the lane rewrites
  // its chunk from the operand itself, element by element, with zeros past
  // the end (base: the batch's operand base; step: the copy's byte step per
  // k tile).
  __device__ inline void refill_ragged(uint16_t* tile, const char* base, uint32_t step, int kt, int wave, int lane,
                                       int64_t r0, int64_t rows, int64_t K) const {
    const int k0 = BK * kt;
#pragma unroll
    for (int c = 0; c < kC; ++c) {
      const int u = 64 * (wave + W * c) + lane;
      int64_t gr, kk;
      int n;
      bool straddle;
      if constexpr (KC) {
        constexpr int kCpr = BK / 8;
        const int row = u / kCpr;
        gr = r0 + row;
        kk = int64_t(8 * ((u % kCpr) ^ kc_swizzle<BK>(row))) + k0;
        straddle = gr < rows && kk < K && kk + 8 > K;
        n = int(K - kk);
      } else {
        constexpr int kCpr = R / 8;
        const int kr = u / kCpr;
        gr = r0 + 8 * ((u % kCpr) ^ nc_swizzle<R>(kr));
        kk = int64_t(kr) + k0;
        straddle = kk < K && gr < rows && gr + 8 > rows;
        n = int(rows - gr);
      }
      if (straddle) {
        const uint16_t* src = reinterpret_cast<const uint16_t*>(base + (off[c] + uint32_t(kt) * step));
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t lo = 2 * e < n ? uint32_t(src[2 * e]) : 0u;
          const uint32_t hi = 2 * e + 1 < n ? uint32_t(src[2 * e + 1]) : 0u;
          w[e] = lo | (hi << 16);
        }
        *reinterpret_cast<u32x4_t*>(tile + (wave + W * c) * 512 + 8 * lane) = u32x4_t{w[0], w[1], w[2], w[3]};
      }
    }
  }
};

// MFMA operand (8 bf16) for rows rb .. rb + 31 of a tile of R rows and k-step
// ks (k = 16 ks .. 16 ks + 15): lane (c, g) gets row rb + c, k 16 ks + 8 g ..+7.
template <bool KC, int R, int BK>
__device__ inline bf16x8_t read_operand(const uint16_t* t, int rb, int ks, int lane) {
  if constexpr (KC) {
    const int row = rb + (lane & 31), ch = (2 * ks + (lane >> 5)) ^ kc_swizzle<BK>(row);
    return as_bf16x8(*reinterpret_cast<const u32x4_t*>(t + row * BK + 8 * ch));
  } else {
    // 16-lane group: lanes 4q .. 4q + 3 address k-row q of a 4 x 16 block,
    // 8 bytes (4 columns) each; lane i of the group receives column i.
    const int kr = 16 * ks + 8 * (lane >> 5) + ((lane & 15) >> 2);
    const int col = rb + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    const int at = 8 * ((col >> 3) ^ nc_swizzle<R>(kr)) + (col & 7);
    const uint2 lo = lds_read_tr(t + kr * R + at);
    const uint2 hi = lds_read_tr(t + (kr + 4) * R + at);  // k-row kr + 4 has kr's swizzle
    return as_bf16x8(u32x4_t{lo.x, lo.y, hi.x, hi.y});
  }
}

// 4 fp32 -> 4 packed 16-bit values (bf16 or f16, RNE) as two dwords
template <int CT>
__device__ inline uint2 pack4(const float (&v)[4]) {
  if constexpr (CT == MK_BF16)
    return uint2{f32_to_bf16(v[0]) | (uint32_t(f32_to_bf16(v[1])) << 16),
                 f32_to_bf16(v[2]) | (uint32_t(f32_to_bf16(v[3])) << 16)};
  return uint2{f32_to_f16(v[0]) | (uint32_t(f32_to_f16(v[1])) << 16),
               f32_to_f16(v[2]) | (uint32_t(f32_to_f16(v[3])) << 16)};
}

// The GELU side output: bf16 gelu_tanh (mk_gelu_tanh's function) of stored
// values -- a bf16 C chunk of 8 as stored (rounded), fp32 pairs as they are.
__device__ inline uint32_t gelu2_bf16(float x0, float x1) {
  return uint32_t(f32_to_bf16(gelu_tanh_f32(x0))) | (uint32_t(f32_to_bf16(gelu_tanh_f32(x1))) << 16);
}
__device__ inline u32x4_t gelu8_bf16(const u32x4_t& v) {
  u32x4_t o;
#pragma unroll
  for (int q = 0; q < 4; ++q)
    o[q] = gelu2_bf16(__builtin_bit_cast(float, v[q] << 16), __builtin_bit_cast(float, v[q] & 0xFFFF0000u));
  return o;
}

// bias + ReLU on the 4 consecutive columns starting at n (bias read for
// columns < N only)
template <int CT>
__device__ inline void finish4(const TiledGemm& p, int64_t n, float (&v)[4]) {
  if ((p.epilogue & 3) == 0) return;
  const bool bias32 = (p.epilogue & 4) != 0;  // an fp32 bias whatever C's type
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    v[q] += n + q < p.N ? (bias32 ? static_cast<const float*>(p.bias)[n + q] : load_as_f32(p.bias, n + q, CT)) : 0.f;
    if ((p.epilogue & 3) == 2) v[q] = fmaxf(v[q], 0.f);
  }
}

// 16-bit C through LDS.  Lanes l and l + 32 trade halves (v_permlane32_swap)
// so that each holds 8 consecutive columns: from the pair (rg 2h, rg 2h + 1)
// lane g gets the chunk of columns 16 h + 8 g .. + 7 of its block.  Chunks go
// to LDS rows of TN columns at chunk position ^ (row & 15) when a row holds a
// multiple of 16 chunks, else ^ ((row >> 1) & 7) (rows of 8 mod 16 chunks:
// rows 2 apart share the bank offset).  Then the workgroup stores runs of consecutive
// C rows: whole 16-byte chunks when C rows are 16-byte aligned (ROWS16),
// else one element per thread, consecutive threads on consecutive columns.
template <int CT, bool ROWS16, int TM, int TN, int kW, int kWM, int kWN, int kI, int kJ>
__device__ __attribute__((always_inline)) inline void store_staged(const TiledGemm& p,
                                                                   const f32x16_t (&acc)[kI][kJ], uint16_t* st,
                                                                   int64_t m0, int64_t n0, int wm, int wn,
                                                                   int lane, int64_t bz) {
  constexpr int kCpr = TN / 8;
  static_assert(kCpr % 8 == 0, "staging rows of whole 8-chunk groups");
  // chunk position of chunk cn in staging row r: the 16 rows one ds_write_b128
  // cycle writes at one chunk land on 16 different bank groups
  auto pos = [](int r, int cn) { return kCpr % 16 == 0 ? cn ^ (r & 15) : cn ^ ((r >> 1) & 7); };
  const int c = lane & 31, g = lane >> 5;
#pragma unroll
  for (int a = 0; a < kI; ++a) {
    const int ml = wm * kWM + 32 * a + c;
#pragma unroll
    for (int b = 0; b < kJ; ++b) {
      const int nb = wn * kWN + 32 * b;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        uint2 w[2];  // rg 2h, 2h + 1
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int rg = 2 * h + e;
          float v[4] = {acc[a][b][4 * rg], acc[a][b][4 * rg + 1], acc[a][b][4 * rg + 2], acc[a][b][4 * rg + 3]};
          finish4<CT>(p, n0 + nb + 8 * rg + 4 * g, v);
          w[e] = pack4<CT>(v);
        }
        // lane g = 0 ends with (own rg 2h, partner's rg 2h): columns 16 h + 0..7;
        // lane g = 1 with (partner's rg 2h + 1, own rg 2h + 1): 16 h + 8..15
        const auto s0 = __builtin_amdgcn_permlane32_swap(w[0].x, w[1].x, false, false);
        const auto s1 = __builtin_amdgcn_permlane32_swap(w[0].y, w[1].y, false, false);
        const u32x4_t chunk = {static_cast<uint32_t>(s0[0]), static_cast<uint32_t>(s1[0]),
                               static_cast<uint32_t>(s0[1]), static_cast<uint32_t>(s1[1])};
        const int cn = (nb + 16 * h + 8 * g) >> 3;
        *reinterpret_cast<u32x4_t*>(st + ml * TN + 8 * pos(ml, cn)) = chunk;
      }
    }
  }
  lds_barrier();
  constexpr int kThreads = 64 * kW;
  static_assert(TM * kCpr % kThreads == 0, "staged rows split evenly over the threads");
  char* Cz = reinterpret_cast<char*>(p.C) + 2 * bz * p.c_bs;
  if constexpr (!ROWS16) {
    uint16_t* Ce = reinterpret_cast<uint16_t*>(Cz);
    for (int it = 0; it < TM * TN / kThreads; ++it) {
      const int e = it * kThreads + int(threadIdx.x);
      const int row = e / TN, col = e % TN;
      const uint16_t v = st[row * TN + 8 * pos(row, col >> 3) + (col & 7)];
      const int64_t m = m0 + row, n = n0 + col;
      if (m < p.M && n < p.N) Ce[m * p.ldc + n] = v;
    }
    return;
  }
  const bool gelu_bwd = (p.epilogue & kEpiGeluBwd) != 0;
#pragma unroll
  for (int it = 0; it < TM * kCpr / kThreads; ++it) {
    const int e = it * kThreads + int(threadIdx.x);
    const int row = e / kCpr, cn = e % kCpr;
    u32x4_t v = *reinterpret_cast<const u32x4_t*>(st + row * TN + 8 * pos(row, cn));
    const int64_t m = m0 + row, n = n0 + 8 * cn;
    if (gelu_bwd) {
      // v (the product as stored) times gelu'(pre), pre read only inside
      // [M, N); the chunk is written back for the column pass (zeros
      // outside [M, N))
      u32x4_t pre = {0u, 0u, 0u, 0u};
      if (m < p.M && n + 8 <= p.N) {
        pre = *reinterpret_cast<const u32x4_t*>(p.aux + m * p.ld_aux + n);
      } else if (m < p.M && n < p.N) {
#pragma unroll
        for (int q = 0; q < 8; ++q)
          if (n + q < p.N) pre[q / 2] |= uint32_t(p.aux[m * p.ld_aux + n + q]) << (16 * (q & 1));
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const bool in0 = m < p.M && n + 2 * q < p.N, in1 = m < p.M && n + 2 * q + 1 < p.N;
        const float d0 = __builtin_bit_cast(float, v[q] << 16), d1 = __builtin_bit_cast(float, v[q] & 0xFFFF0000u);
        const float x0 = __builtin_bit_cast(float, pre[q] << 16), x1 = __builtin_bit_cast(float, pre[q] & 0xFFFF0000u);
        const uint32_t lo = in0 ? f32_to_bf16(d0 * gelu_tanh_grad_f32(x0)) : 0u;
        const uint32_t hi = in1 ? f32_to_bf16(d1 * gelu_tanh_grad_f32(x1)) : 0u;
        v[q] = lo | (hi << 16);
      }
      *reinterpret_cast<u32x4_t*>(st + row * TN + 8 * pos(row, cn)) = v;
    }
    if (m < p.M && n + 8 <= p.N) {
      *reinterpret_cast<u32x4_t*>(Cz + 2 * (m * p.ldc + n)) = v;
      if (p.epilogue & kEpiGeluAux) *reinterpret_cast<u32x4_t*>(p.aux + m * p.ld_aux + n) = gelu8_bf16(v);
    } else if (m < p.M && n < p.N) {  // the chunk that straddles N: its columns below N only
      uint16_t* Ce = reinterpret_cast<uint16_t*>(Cz) + m * p.ldc + n;
      const u32x4_t gv = gelu8_bf16(v);
#pragma unroll
      for (int q = 0; q < 8; ++q)
        if (n + q < p.N) {
          Ce[q] = uint16_t(v[q / 2] >> (16 * (q & 1)));
          if (p.epilogue & kEpiGeluAux) p.aux[m * p.ld_aux + n + q] = uint16_t(gv[q / 2] >> (16 * (q & 1)));
        }
    }
  }
  if (gelu_bwd) {
    // column sums of the stored values, 128 rows at a time in row order,
    // into partial row (m0 + 128 h) / 128
    lds_barrier();
    for (int t = int(threadIdx.x); t < TN * (TM / 128); t += kThreads) {
      const int col = t % TN, h = t / TN;
      const int64_t n = n0 + col;
      float sum = 0.f;
      for (int row = 128 * h; row < 128 * h + 128; ++row) {
        const uint16_t b = st[row * TN + 8 * pos(row, col >> 3) + (col & 7)];
        sum += __builtin_bit_cast(float, uint32_t(b) << 16);
      }
      if (n < p.N && m0 + 128 * h < p.M) p.colpart[((m0 >> 7) + h) * p.N + n] = sum;
    }
  }
}

// fp32 C through LDS, for C rows that are not 16-byte aligned (an odd N such
// as a vocabulary, where direct stores would go out one dword at a time, 32
// rows per instruction).  The tile is staged in passes of RP rows (whole
// wave rows; RP x TN floats fit the operand buffers): the waves owning those
// rows write their accumulators as 16-byte chunks, chunk c of staging row r
// at position c ^ (r & 15), then every thread stores consecutive columns of
// consecutive rows, so each wave writes 256 contiguous bytes of a C row.
template <bool ROWS16, int TM, int TN, int kW, int kWM, int kWN, int kI, int kJ, int kLdsFloats>
__device__ __attribute__((always_inline)) inline void store_staged_f32(const TiledGemm& p,
                                                                       const f32x16_t (&acc)[kI][kJ], float* st,
                                                                       int64_t m0, int64_t n0, int wm, int wn,
                                                                       int lane, int64_t bz) {
  constexpr int kCpr = TN / 4;
  static_assert(kCpr % 16 == 0, "staging rows of whole 16-chunk groups");
  // rows per pass: the largest multiple of kWM dividing TM whose staging fits
  constexpr int kRP = [] {
    int rp = kWM;
    for (int r = kWM; r <= TM; r += kWM)
      if (TM % r == 0 && r * TN <= kLdsFloats) rp = r;
    return rp;
  }();
  static_assert(kRP * TN <= kLdsFloats, "one wave row of staging fits");
  static_assert(kRP >= kWM && TM % kRP == 0, "passes of whole wave rows");
  constexpr int kThreads = 64 * kW;
  static_assert(kRP * TN % kThreads == 0, "staged rows split evenly over the threads");
  const int c = lane & 31, g = lane >> 5;
  float* Cz = reinterpret_cast<float*>(p.C) + bz * p.c_bs;
#pragma unroll
  for (int pass = 0; pass < TM / kRP; ++pass) {
    if (wm * kWM >= pass * kRP && wm * kWM < (pass + 1) * kRP) {
#pragma unroll
      for (int a = 0; a < kI; ++a) {
        const int ml = wm * kWM + 32 * a + c - pass * kRP;
#pragma unroll
        for (int b = 0; b < kJ; ++b)
#pragma unroll
          for (int rg = 0; rg < 4; ++rg) {
            const int nl = wn * kWN + 32 * b + 8 * rg + 4 * g;
            float v[4] = {acc[a][b][4 * rg], acc[a][b][4 * rg + 1], acc[a][b][4 * rg + 2], acc[a][b][4 * rg + 3]};
            finish4<MK_F32>(p, n0 + nl, v);
            *reinterpret_cast<f32x4*>(st + ml * TN + 4 * ((nl >> 2) ^ (ml & 15))) = f32x4{{v[0], v[1], v[2], v[3]}};
          }
      }
    }
    lds_barrier();
    if constexpr (ROWS16) {
      // 16-byte aligned rows, N a multiple of 4: whole chunks, each wave
      // writing 1 KB of one C row per instruction
      static_assert(kRP * kCpr % kThreads == 0, "staged chunks split evenly over the threads");
#pragma unroll 4
      for (int it = 0; it < kRP * kCpr / kThreads; ++it) {
        const int e = it * kThreads + int(threadIdx.x);
        const int row = e / kCpr, cn = e % kCpr;
        const f32x4 v = *reinterpret_cast<const f32x4*>(st + row * TN + 4 * (cn ^ (row & 15)));
        const int64_t m = m0 + pass * kRP + row, n = n0 + 4 * cn;
        if (m < p.M && n + 4 <= p.N) {
          *reinterpret_cast<f32x4*>(Cz + m * p.ldc + n) = v;
          if (p.epilogue & kEpiGeluAux)
            *reinterpret_cast<uint2*>(p.aux + m * p.ld_aux + n) =
                uint2{gelu2_bf16(v.v[0], v.v[1]), gelu2_bf16(v.v[2], v.v[3])};
        } else if (m < p.M && n < p.N) {  // the chunk that straddles N
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (n + q < p.N) {
              Cz[m * p.ldc + n + q] = v.v[q];
              if (p.epilogue & kEpiGeluAux) p.aux[m * p.ld_aux + n + q] = f32_to_bf16(gelu_tanh_f32(v.v[q]));
            }
        }
      }
    } else {
#pragma unroll 4
      for (int it = 0; it < kRP * TN / kThreads; ++it) {
        const int e = it * kThreads + int(threadIdx.x);
        const int row = e / TN, col = e % TN;
        const float v = st[row * TN + 4 * ((col >> 2) ^ (row & 15)) + (col & 3)];
        const int64_t m = m0 + pass * kRP + row, n = n0 + col;
        if (m < p.M && n < p.N) Cz[m * p.ldc + n] = v;
      }
    }
    lds_barrier();
  }
}

// Stores straight from the accumulators: 4 consecutive columns per lane and
// register group, as one vector store (c_mode 1) or element by element.
template <int CT, int kWM, int kWN, int kI, int kJ>
__device__ __attribute__((always_inline)) inline void store_direct(const TiledGemm& p,
                                                                   const f32x16_t (&acc)[kI][kJ], int64_t m0,
                                                                   int64_t n0, int wm, int wn, int lane,
                                                                   int64_t bz) {
  constexpr int esz = CT == MK_F32 ? 4 : 2;
  const int c = lane & 31, g = lane >> 5;
  char* Cb = reinterpret_cast<char*>(p.C) + esz * bz * p.c_bs;
#pragma unroll
  for (int a = 0; a < kI; ++a) {
    const int64_t m = m0 + wm * kWM + 32 * a + c;
#pragma unroll
    for (int b = 0; b < kJ; ++b)
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const int64_t n = n0 + wn * kWN + 32 * b + 8 * rg + 4 * g;
        float v[4] = {acc[a][b][4 * rg], acc[a][b][4 * rg + 1], acc[a][b][4 * rg + 2], acc[a][b][4 * rg + 3]};
        finish4<CT>(p, n, v);
        if (m >= p.M || n >= p.N) continue;
        char* dst = Cb + esz * (m * p.ldc + n);
        if (p.c_mode == 1) {  // N, ldc, batch stride multiples of 4, C 16-byte aligned
          if constexpr (CT == MK_F32) *reinterpret_cast<float4*>(dst) = float4{v[0], v[1], v[2], v[3]};
          else *reinterpret_cast<uint2*>(dst) = pack4<CT>(v);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (n + q < p.N) store_from_f32(dst, q, CT, v[q]);
        }
      }
  }
}

// Kernel shape: workgroup tile, wave grid, k-tile depth, LDS stages.
template <int TM_, int TN_, int WGM_, int WGN_, int BK_, int S_>
struct Shape {
  static constexpr int TM = TM_, TN = TN_, WGM = WGM_, WGN = WGN_, BK = BK_, S = S_;
};

// s_waitcnt vmcnt(n) for a compile-time n, expcnt / lgkmcnt untouched
template <int N>
__device__ inline void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// RAGGED: an operand chunk straddles K, M or N (the launcher knows): only
// then does the k loop carry the last tile's rewrite, so the common loop is
// unchanged by it (measured: the branch alone cost 2-5% on the C5 shapes).
template <class Sh, bool AKC, bool BKC, bool RAGGED>
__global__ __launch_bounds__(64 * Sh::WGM * Sh::WGN, 1) void gemm_tiled_kernel(const TiledGemm p) {
  constexpr int TM = Sh::TM, TN = Sh::TN, WGN = Sh::WGN, BK = Sh::BK, S = Sh::S;
  constexpr int kW = Sh::WGM * WGN;                      // waves
  constexpr int kWM = TM / Sh::WGM, kWN = TN / WGN;      // wave block
  constexpr int kI = kWM / 32, kJ = kWN / 32;            // MFMA blocks per wave (m, n)
  constexpr int kCa = TM * BK / 512 / kW;                // 1 KB copies per wave per k tile, A
  constexpr int kCb = TN * BK / 512 / kW;                // ... B
  static_assert(BK == 32 || BK == 64, "k tile depth");
  static_assert(kI * 32 * Sh::WGM == TM && kJ * 32 * WGN == TN, "wave blocks tile the workgroup tile");
  static_assert(kCa * kW * 512 == TM * BK && kCb * kW * 512 == TN * BK, "copies split evenly over the waves");
  static_assert(TM * TN <= S * BK * (TM + TN), "staging tile fits the operand buffers");
  __shared__ __attribute__((aligned(1024))) uint16_t lds[S * BK * (TM + TN)];
  uint16_t (*As)[TM * BK] = reinterpret_cast<uint16_t (*)[TM * BK]>(lds);
  uint16_t (*Bs)[TN * BK] = reinterpret_cast<uint16_t (*)[TN * BK]>(lds + S * TM * BK);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WGN, wn = wave % WGN;
  // tile of this workgroup (see the header)
  const uint32_t nt = gridDim.x, per = nt / 8, i = blockIdx.x;
  const uint32_t t = i < 8 * per ? (i % 8) * per + i / 8 : i;
  const uint32_t group = t / (kGroupM * uint32_t(p.tiles_n)), first_m = group * kGroupM;
  const uint32_t gm = min(uint32_t(kGroupM), uint32_t(p.tiles_m) - first_m);
  const uint32_t w_in = t - group * kGroupM * uint32_t(p.tiles_n);
  const int64_t m0 = int64_t(first_m + w_in % gm) * TM;
  const int64_t n0 = int64_t(w_in / gm) * TN;
  const int64_t bz = blockIdx.y;
  // contraction length of this batch
  const int64_t Kb = (p.k_rem > 0 && bz == int64_t(gridDim.y) - 1) ? p.k_rem : p.K;
  const i32x4_t ra = tile_desc(reinterpret_cast<const uint16_t*>(p.A) + bz * p.a_bs, p.a_bytes);
  const i32x4_t rb = tile_desc(reinterpret_cast<const uint16_t*>(p.B) + bz * p.b_bs, p.b_bytes);

  const Copies<AKC, TM, BK, kCa, kW> ca(wave, lane, m0, p.M, p.lda);
  const Copies<BKC, TN, BK, kCb, kW> cb(wave, lane, n0, p.N, p.ldb);
  // byte distance between consecutive k tiles
  const uint32_t a_step = AKC ? 2 * BK : uint32_t(2 * BK * p.lda);
  const uint32_t b_step = BKC ? 2 * BK : uint32_t(2 * BK * p.ldb);
  // this wave's copies [lo, hi) of k tile kt into stage (A's kCa copies first,
  // then B's kCb)
  auto issue = [&](int kt, int stage, int lo, int hi) __attribute__((always_inline)) {
    const int k0 = BK * kt;
    if (k0 + BK <= Kb) {
      const uint32_t sa = uint32_t(kt) * a_step, sb = uint32_t(kt) * b_step;
#pragma unroll
      for (int c = 0; c < kCa + kCb; ++c) {
        if (c < lo || c >= hi) continue;
        if (c < kCa) copy_to_lds_so(ra, lds_addr(&As[stage][(wave + kW * c) * 512]), int(ca.off[c]), sa);
        else copy_to_lds_so(rb, lds_addr(&Bs[stage][(wave + kW * (c - kCa)) * 512]), int(cb.off[c - kCa]), sb);
      }
      return;
    }
#pragma unroll
    for (int c = 0; c < kCa + kCb; ++c) {
      if (c < lo || c >= hi) continue;
      if (c < kCa)
        copy_to_lds(ra, lds_addr(&As[stage][(wave + kW * c) * 512]), ca.at(c, k0, uint32_t(kt) * a_step, Kb));
      else
        copy_to_lds(rb, lds_addr(&Bs[stage][(wave + kW * (c - kCa)) * 512]),
                    cb.at(c - kCa, k0, uint32_t(kt) * b_step, Kb));
    }
  };

  f32x16_t acc[kI][kJ];
#pragma unroll
  for (int a = 0; a < kI; ++a)
#pragma unroll
    for (int b = 0; b < kJ; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;

  // Tile kt lives in stage kt % S.  Before multiplying tile kt a wave waits
  // for its own copies of it (the S - 2 tiles issued after it may still be in
  // flight), then the barrier makes every wave's copies visible and also
  // marks stage (kt - 1) % S, read in the previous iteration, free for the
  // copies of tile kt + S - 1.  Those copies are issued in kParts groups,
  // each after the operand reads of one k-step: a wave that issued all of
  // them at once would stall on the full vector-memory queue (1 KB copies
  // drain at about 60 bytes per clock per CU) with its MFMAs behind them.
  const int nk = int((Kb + BK - 1) / BK);
  constexpr int kNC = kCa + kCb, kParts = BK / 16 < 2 ? BK / 16 : 2;
#pragma unroll
  for (int st = 0; st < S - 1; ++st)
    if (st < nk) issue(st, st, 0, kNC);
  auto desc_base = [](const i32x4_t& r) __attribute__((always_inline)) {
    return reinterpret_cast<const char*>((uint64_t(uint32_t(r.y) & 0xFFFFu) << 32) | uint32_t(r.x));
  };
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + S - 2 < nk) wait_vm<(S - 2) * kNC>();
    else wait_vm<0>();
    lds_barrier();
    if (RAGGED && kt == nk - 1) {
      // the last k tile is in LDS: each wave rewrites the chunks it copied
      // that straddle K, M or N from the operands (zeros past the end), then
      // a second barrier publishes them.  The batch's operand bases come from
      // the copy descriptors; the loop position and lane ids pass through an
      // empty asm, so nothing of the rewrite is computed ahead of the loop
      // (where it would hold registers for the whole k loop).
      int kq = kt, wq = wave, lq = lane;
      asm volatile("" : "+s"(kq), "+s"(wq), "+v"(lq));
      ca.refill_ragged(As[kq % S], desc_base(ra), a_step, kq, wq, lq, m0, p.M, Kb);
      cb.refill_ragged(Bs[kq % S], desc_base(rb), b_step, kq, wq, lq, n0, p.N, Kb);
      lds_barrier();
    }
    const bool more = kt + S - 1 < nk;
    const uint16_t* at = As[kt % S];
    const uint16_t* bt = Bs[kt % S];
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      bf16x8_t af[kI], bfr[kJ];
#pragma unroll
      for (int a = 0; a < kI; ++a) af[a] = read_operand<AKC, TM, BK>(at, wm * kWM + 32 * a, ks, lane);
#pragma unroll
      for (int b = 0; b < kJ; ++b) bfr[b] = read_operand<BKC, TN, BK>(bt, wn * kWN + 32 * b, ks, lane);
      if (more && ks < kParts) issue(kt + S - 1, (kt + S - 1) % S, ks * kNC / kParts, (ks + 1) * kNC / kParts);
#pragma unroll
      for (int a = 0; a < kI; ++a)
#pragma unroll
        for (int b = 0; b < kJ; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[b], af[a], acc[a][b], 0, 0, 0);
    }
  }
  lds_barrier();  // every wave is done with the operand stages before they hold C

  if (p.c_mode == 2 && p.c_type == MK_BF16)
    store_staged<MK_BF16, true, TM, TN, kW, kWM, kWN>(p, acc, lds, m0, n0, wm, wn, lane, bz);
  else if (p.c_mode == 2)
    store_staged<MK_F16, true, TM, TN, kW, kWM, kWN>(p, acc, lds, m0, n0, wm, wn, lane, bz);
  else if (p.c_mode == 3 && p.c_type == MK_BF16)
    store_staged<MK_BF16, false, TM, TN, kW, kWM, kWN>(p, acc, lds, m0, n0, wm, wn, lane, bz);
  else if (p.c_mode == 3)
    store_staged<MK_F16, false, TM, TN, kW, kWM, kWN>(p, acc, lds, m0, n0, wm, wn, lane, bz);
  else if (p.c_mode == 4)
    store_staged_f32<false, TM, TN, kW, kWM, kWN, kI, kJ, S * BK * (TM + TN) / 2>(
        p, acc, reinterpret_cast<float*>(lds), m0, n0, wm, wn, lane, bz);
  else if (p.c_mode == 5)
    store_staged_f32<true, TM, TN, kW, kWM, kWN, kI, kJ, S * BK * (TM + TN) / 2>(
        p, acc, reinterpret_cast<float*>(lds), m0, n0, wm, wn, lane, bz);
  else if (p.c_type == MK_F32)
    store_direct<MK_F32, kWM, kWN>(p, acc, m0, n0, wm, wn, lane, bz);
  else if (p.c_type == MK_BF16)
    store_direct<MK_BF16, kWM, kWN>(p, acc, m0, n0, wm, wn, lane, bz);
  else
    store_direct<MK_F16, kWM, kWN>(p, acc, m0, n0, wm, wn, lane, bz);
}

template <class Sh, bool RG>
void launch_kernel(hipStream_t s, const TiledGemm& a, dim3 g, dim3 b, bool a_kc, bool b_kc) {
  if (a_kc && b_kc) hipLaunchKernelGGL((gemm_tiled_kernel<Sh, true, true, RG>), g, b, 0, s, a);
  else if (a_kc) hipLaunchKernelGGL((gemm_tiled_kernel<Sh, true, false, RG>), g, b, 0, s, a);
  else if (b_kc) hipLaunchKernelGGL((gemm_tiled_kernel<Sh, false, true, RG>), g, b, 0, s, a);
  else hipLaunchKernelGGL((gemm_tiled_kernel<Sh, false, false, RG>), g, b, 0, s, a);
}

template <class Sh>
int launch(hipStream_t s, TiledGemm& a, int64_t batch, bool a_kc, bool b_kc) {
  a.tiles_m = int((a.M + Sh::TM - 1) / Sh::TM);
  a.tiles_n = int((a.N + Sh::TN - 1) / Sh::TN);
  const dim3 g{unsigned(int64_t(a.tiles_m) * a.tiles_n), unsigned(batch)}, b{unsigned(64 * Sh::WGM * Sh::WGN)};
  // a chunk straddles K (k-contiguous operand, K % 8 != 0; the last batch's
  // k_rem counts too), M or N (m- / n-contiguous operand)
  const bool k_ragged = (a_kc || b_kc) && (a.K % 8 != 0 || (a.k_rem > 0 && a.k_rem % 8 != 0));
  const bool ragged = k_ragged || (!a_kc && a.M % 8 != 0) || (!b_kc && a.N % 8 != 0);
  if (ragged) launch_kernel<Sh, true>(s, a, g, b, a_kc, b_kc);
  else launch_kernel<Sh, false>(s, a, g, b, a_kc, b_kc);
  return check_launch("mk_gemm");
}

// Bytes one batch's operand spans from its base: rows (m or n) x K with the
// unit stride along k (kc) or along the rows.
int64_t span_bytes(bool kc, int64_t rows, int64_t K, int64_t ld) {
  return 2 * (kc ? (rows - 1) * ld + K : (K - 1) * ld + rows);
}

// Fills the kernel arguments; false when the shape, strides or alignment do
// not fit the tiled kernel.
bool tiled_args(TiledGemm& a, bool& a_kc, bool& b_kc, int c_type, int64_t batch, int64_t M, int64_t N, int64_t K,
                const void* A, int64_t a_bs, int64_t a_ms, int64_t a_ks, const void* B, int64_t b_bs, int64_t b_ks,
                int64_t b_ns, void* C, int64_t c_bs, int64_t c_ms, const void* bias, int epilogue, int64_t k_rem,
                void* Y, int64_t y_ms, float* colpart) {
  if (M < 128 || N < 128 || K < 64) return false;
  if (k_rem < 0 || k_rem > K || (k_rem > 0 && (batch < 2 || K % 8 != 0))) return false;
  a_kc = a_ks == 1;
  b_kc = b_ks == 1;
  if (!a_kc && a_ms != 1) return false;
  if (!b_kc && b_ns != 1) return false;
  const int64_t lda = a_kc ? a_ms : a_ks, ldb = b_kc ? b_ns : b_ks;
  // every 16-byte chunk a copy loads is aligned: 16-byte bases, strides
  // multiples of 8 elements.  The pitch is then at least the contiguous
  // extent rounded up to 8, so a chunk straddling K, M or N stays inside its
  // row's pitch (or runs past the buffer range, which reads zeros).
  auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; };
  if (!al16(A) || !al16(B) || lda % 8 != 0 || ldb % 8 != 0) return false;
  if (batch > 1 && (a_bs % 8 != 0 || b_bs % 8 != 0)) return false;
  if (lda < (a_kc ? K : M) || ldb < (b_kc ? K : N)) return false;  // overlapping rows
  const int64_t ab = span_bytes(a_kc, M, K, lda), bb = span_bytes(b_kc, N, K, ldb);
  if (ab >= (int64_t(1) << 31) || bb >= (int64_t(1) << 31)) return false;  // 32-bit buffer offsets
  a.A = A; a.B = B; a.C = C; a.bias = bias;
  a.M = M; a.N = N; a.K = K;
  a.k_rem = k_rem;
  a.lda = lda; a.ldb = ldb; a.ldc = c_ms;
  a.a_bs = a_bs; a.b_bs = b_bs; a.c_bs = c_bs;
  a.a_bytes = uint32_t(ab); a.b_bytes = uint32_t(bb);
  a.epilogue = epilogue;
  a.c_type = c_type;
  // C rows 16-byte aligned: whole 16-byte chunks (the one straddling N, when
  // N is not a multiple of the chunk, column by column)
  const bool rows16 = al16(C) && (batch == 1 || c_bs % 8 == 0) && c_ms % 8 == 0;
  const bool rows4 = al16(C) && (batch == 1 || c_bs % 4 == 0) && c_ms % 4 == 0;
  a.c_mode = c_type != MK_F32 ? (rows16 ? 2 : 3) : rows4 ? 5 : 4;
  a.aux = static_cast<uint16_t*>(Y);
  a.ld_aux = y_ms;
  if (epilogue & kEpiGeluAux) {
    // the side output goes out with C's whole chunks: 8 bf16 per bf16 C
    // chunk, 4 per fp32 one, rows aligned to match
    const uintptr_t ya = reinterpret_cast<uintptr_t>(Y);
    const bool ok16 = c_type == MK_BF16 && a.c_mode == 2 && (ya & 15u) == 0 && y_ms % 8 == 0;
    const bool ok32 = c_type == MK_F32 && a.c_mode == 5 && (ya & 7u) == 0 && y_ms % 4 == 0;
    if (batch != 1 || !Y || y_ms < N || !(ok16 || ok32)) return false;
  }
  a.colpart = colpart;
  if (epilogue & kEpiGeluBwd) {
    // pre read in whole 16-byte chunks beside bf16 C's
    const uintptr_t ya = reinterpret_cast<uintptr_t>(Y);
    if ((epilogue & (kEpiGeluAux | 3)) || batch != 1 || c_type != MK_BF16 || a.c_mode != 2 || !Y || !colpart ||
        (ya & 15u) != 0 || y_ms % 8 != 0 || y_ms < N)
      return false;
  }
  return true;
}

// compute units of the current device (cached per device)
int64_t cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

}  // namespace

int gemm_tiled(hipStream_t s, int c_type, int64_t batch, int64_t M, int64_t N, int64_t K, const void* A,
               int64_t a_bs, int64_t a_ms, int64_t a_ks, const void* B, int64_t b_bs, int64_t b_ks,
               int64_t b_ns, void* C, int64_t c_bs, int64_t c_ms, const void* bias, int epilogue, int64_t k_rem,
               void* Y, int64_t y_ms, float* colpart) {
  TiledGemm a;
  bool a_kc, b_kc;
  if (!tiled_args(a, a_kc, b_kc, c_type, batch, M, N, K, A, a_bs, a_ms, a_ks, B, b_bs, b_ks, b_ns, C, c_bs, c_ms,
                  bias, epilogue, k_rem, Y, y_ms, colpart))
    return -1;
  // Kernel shape: the one with the least estimated time.  Each shape has a
  // throughput per CU measured on a large product (8192 x 8192 x 4096: 1240,
  // 1083 and 1017 TFLOP/s) and a number of workgroups a CU holds at once (one
  // 256 x 256 workgroup, two of the smaller ones).  Whole rounds of
  // workgroups over the CUs run at that throughput; a last partial round
  // that leaves every workgroup alone on its CU runs each at about 0.8 of it
  // (a CU's throughput with one 8-wave workgroup instead of two, measured on
  // the 8192 x 768 products with K = 768 .. 3072).
  struct Option {
    int tm, tn, per_cu;
    double rate;
  };
  static const Option options[3] = {{256, 256, 1, 1240.0}, {128, 192, 2, 1083.0}, {128, 128, 2, 1017.0}};
  const int64_t cus = cu_count();
  int best = -1;
  double best_t = 0;
  for (int o = 0; o < 3; ++o) {
    const Option& op = options[o];
    if (M < op.tm || N < op.tn) continue;
    const int64_t tiles = ((M + op.tm - 1) / op.tm) * ((N + op.tn - 1) / op.tn) * batch;
    const int64_t slots = cus * op.per_cu, rem = tiles % slots;
    const double tile = double(op.tm) * op.tn / op.rate;
    double t = double(tiles / slots) * op.per_cu * tile;
    if (rem > 0) t += (op.per_cu > 1 && rem <= cus) ? tile / 0.8 : op.per_cu * tile;
    if (best < 0 || t < best_t) best = o, best_t = t;
  }
  if (best == 0) return launch<Shape<256, 256, 2, 4, 64, 2>>(s, a, batch, a_kc, b_kc);
  if (best == 1) return launch<Shape<128, 192, 4, 2, 64, 2>>(s, a, batch, a_kc, b_kc);
  return launch<Shape<128, 128, 4, 2, 64, 2>>(s, a, batch, a_kc, b_kc);
}

}  // namespace mk
