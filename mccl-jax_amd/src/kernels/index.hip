// Indexing kernels: row gather (embedding lookup) and deterministic
// scatter-add.
//
// Scatter-add determinism: the result must equal applying the updates one
// at a time in increasing update index (XLA:CPU's sequential scatter), so
// for every destination row the fp32 adds happen in that order.  The plan:
//   1. key(i) = ids[i] (or n_rows for a dropped out-of-range id)
//   2. a stable sort of the update indices i by key — stable, so equal keys
//      keep increasing i — and bounds: first / one-past-last sorted position
//      of every row's updates
//   3. one wave per destination row: acc = table[r]; acc += updates[i] for the
//      row's i in sorted (= increasing) order; store.
// Step 3 is the HBM-bound part (reads updates once, table rows once, writes
// output rows once); step 2 touches only O(n_ids + n_rows) 4-byte words.
// Step 2 for keys below 2^16 (n_rows < 65535) is one launch, one workgroup
// per 256 destination rows (bucket_build_kernel); larger tables take the
// general path: keys and indices materialised, an LSD radix sort of 8 bits
// per pass (histogram, scan, scatter launches per pass) and a bounds launch.
// Step 3 streams the update and output rows past the caches (non-temporal
// loads and stores).
#include "mk_common.h"

#include <algorithm>
#include <mutex>
#include <string>
#include <type_traits>

namespace mk {
namespace {

constexpr int kBlock = 256;

// ------------------------------------------------------------------ gather
template <typename IdxT>
__global__ __launch_bounds__(kBlock) void gather_rows16_kernel(const u32x4_t* __restrict__ table,
                                                               int64_t n_rows, int64_t row_vecs,
                                                               const IdxT* __restrict__ ids,
                                                               int64_t n_ids,
                                                               u32x4_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t i = int64_t(blockIdx.x) * (kBlock / 64) + (threadIdx.x >> 6);
  if (i >= n_ids) return;
  int64_t r = int64_t(ids[i]);
  r = r < 0 ? 0 : (r >= n_rows ? n_rows - 1 : r);  // StableHLO gather clamps start indices
  const u32x4_t* src = table + r * row_vecs;
  u32x4_t* dst = out + i * row_vecs;
  for (int64_t c = lane; c < row_vecs; c += 64) dst[c] = src[c];
}

template <typename IdxT>
__global__ __launch_bounds__(kBlock) void gather_rows4_kernel(const uint32_t* __restrict__ table,
                                                              int64_t n_rows, int64_t row_words,
                                                              const IdxT* __restrict__ ids,
                                                              int64_t n_ids,
                                                              uint32_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t i = int64_t(blockIdx.x) * (kBlock / 64) + (threadIdx.x >> 6);
  if (i >= n_ids) return;
  int64_t r = int64_t(ids[i]);
  r = r < 0 ? 0 : (r >= n_rows ? n_rows - 1 : r);
  const uint32_t* src = table + r * row_words;
  uint32_t* dst = out + i * row_words;
  for (int64_t c = lane; c < row_words; c += 64) dst[c] = src[c];
}

// ------------------------------------------------------------------ radix sort
__global__ __launch_bounds__(kBlock) void fill_words(uint32_t* __restrict__ p, int64_t n) {
  const int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  if (i < n) p[i] = 0u;
}

constexpr int kSortItems = 4;
constexpr int kSortTile = kBlock * kSortItems;  // elements per block per pass

// keys[i] = ids[i] (n_rows for an out-of-range id, sorted last and dropped),
// vals[i] = i; threads also zero the 2 n_rows row bounds.
template <typename IdxT>
__global__ __launch_bounds__(kBlock) void scatter_prepare_kernel(const IdxT* __restrict__ ids,
                                                                 int64_t n, int64_t n_rows,
                                                                 uint32_t* __restrict__ keys,
                                                                 uint32_t* __restrict__ vals,
                                                                 uint32_t* __restrict__ bounds) {
  const int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  if (i < 2 * n_rows) bounds[i] = 0u;
  if (i >= n) return;
  const int64_t id = int64_t(ids[i]);
  keys[i] = (id < 0 || id >= n_rows) ? uint32_t(n_rows) : uint32_t(id);
  vals[i] = uint32_t(i);
}

// Per-block digit histogram, stored digit-major: hist[d * nb + block].
__global__ __launch_bounds__(kBlock) void radix_hist_kernel(const uint32_t* __restrict__ keys, int64_t n,
                                                            int shift, uint32_t* __restrict__ hist,
                                                            int nb) {
  __shared__ uint32_t h[256];
  h[threadIdx.x] = 0;
  __syncthreads();
  const int64_t base = int64_t(blockIdx.x) * kSortTile;
#pragma unroll
  for (int k = 0; k < kSortItems; ++k) {
    const int64_t e = base + int64_t(k) * kBlock + threadIdx.x;
    if (e < n) atomicAdd(&h[(keys[e] >> shift) & 255u], 1u);
  }
  __syncthreads();
  hist[int64_t(threadIdx.x) * nb + blockIdx.x] = h[threadIdx.x];
}

// Exclusive scan of `total` words in place, one block of 1024 threads:
// thread t owns the contiguous run [t*per, (t+1)*per); the run sums are
// scanned with wave shuffles and one LDS exchange of the 16 wave totals.
constexpr int kScanBlock = 1024;
__device__ inline uint32_t wave_incl_scan(uint32_t v, int lane) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t o = uint32_t(__shfl_up(int(v), off, 64));
    if (lane >= off) v += o;
  }
  return v;
}
// The histogram is 256 x nb words (a multiple of 16): thread t owns runs of
// 16 contiguous words, read and written as four 16-byte vectors and scanned
// in registers; runs t, t + 1024, ... are handled in rounds, each round
// carrying the total of the previous ones.
__global__ __launch_bounds__(kScanBlock) void scan_exclusive_kernel(uint32_t* __restrict__ data,
                                                                    int64_t total) {
  __shared__ uint32_t wsum[kScanBlock / 64];
  __shared__ uint32_t carry_s;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int64_t runs = total / 16;
  uint32_t carry = 0;  // sum of all earlier rounds
  for (int64_t r0 = 0; r0 < runs; r0 += kScanBlock) {
    const int64_t run = r0 + t;
    u32x4_t v[4] = {};
    if (run < runs) {
#pragma unroll
      for (int k = 0; k < 4; ++k) v[k] = reinterpret_cast<const u32x4_t*>(data + run * 16)[k];
    }
    uint32_t s = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int j = 0; j < 4; ++j) s += v[k][j];
    const uint32_t incl = wave_incl_scan(s, lane);
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    if (wave == 0) {
      const uint32_t w = lane < kScanBlock / 64 ? wsum[lane] : 0u;
      const uint32_t wi = wave_incl_scan(w, lane);
      if (lane < kScanBlock / 64) wsum[lane] = wi - w;  // exclusive prefix of wave totals
      if (lane == kScanBlock / 64 - 1) carry_s = wi;    // this round's total
    }
    __syncthreads();
    uint32_t acc = carry + wsum[wave] + incl - s;
    if (run < runs) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        u32x4_t o;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          o[j] = acc;
          acc += v[k][j];
        }
        reinterpret_cast<u32x4_t*>(data + run * 16)[k] = o;
      }
    }
    carry += carry_s;
    __syncthreads();  // wsum / carry_s are reused by the next round
  }
}

// Stable scatter of one radix pass.  Element order inside a tile is
// k-major (e = base + k*256 + t), which is also the global order, so a rank
// computed in that order is the stable rank.
__global__ __launch_bounds__(kBlock) void radix_scatter_kernel(const uint32_t* __restrict__ keys_in,
                                                               const uint32_t* __restrict__ vals_in,
                                                               int64_t n, int shift,
                                                               const uint32_t* __restrict__ offsets,
                                                               int nb,
                                                               uint32_t* __restrict__ keys_out,
                                                               uint32_t* __restrict__ vals_out) {
  __shared__ uint32_t running[256];            // same-digit elements already placed in this tile
  __shared__ uint32_t wave_cnt[kBlock / 64][256];
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  running[t] = 0;
  const int64_t base = int64_t(blockIdx.x) * kSortTile;
  const uint32_t my_off = offsets[int64_t(t) * nb + blockIdx.x];  // for digit t
  __shared__ uint32_t block_off[256];
  block_off[t] = my_off;
  for (int k = 0; k < kSortItems; ++k) {
#pragma unroll
    for (int w = 0; w < kBlock / 64; ++w) wave_cnt[w][t] = 0;
    __syncthreads();
    const int64_t e = base + int64_t(k) * kBlock + t;
    const bool valid = e < n;
    uint32_t key = 0, val = 0, d = 0;
    if (valid) {
      key = keys_in[e];
      val = vals_in[e];
      d = (key >> shift) & 255u;
    }
    // lanes of this wave holding the same digit
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int bit = 0; bit < 8; ++bit) {
      const uint64_t ones = __ballot(valid && ((d >> bit) & 1u));
      peers &= ((d >> bit) & 1u) ? ones : ~ones;
    }
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const uint32_t rank_w = uint32_t(__popcll(peers & lt_mask));
    if (valid && rank_w == 0) wave_cnt[wave][d] = uint32_t(__popcll(peers));
    __syncthreads();
    if (valid) {
      uint32_t before = running[d];
      for (int w = 0; w < wave; ++w) before += wave_cnt[w][d];
      const uint32_t pos = block_off[d] + before + rank_w;
      keys_out[pos] = key;
      vals_out[pos] = val;
    }
    __syncthreads();
    uint32_t add = 0;
#pragma unroll
    for (int w = 0; w < kBlock / 64; ++w) add += wave_cnt[w][t];
    running[t] += add;
    __syncthreads();
  }
}

// ------------------------------------------------------------------ 16-bit keys: one launch
// Stable rank of one element per thread within a block-wide chunk (thread
// order = element order): the number of elements with the same digit placed
// before it, counting running[d] from earlier chunks; running is then
// advanced by the chunk's digit counts.  Every thread of the block calls it.
template <int NT>
__device__ inline uint32_t chunk_rank(bool valid, uint32_t d, uint32_t* running,
                                      uint32_t (*wave_cnt)[256]) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  for (int i = t; i < (NT / 64) * 256; i += NT) wave_cnt[i / 256][i % 256] = 0;
  __syncthreads();
  uint64_t peers = __ballot(valid);  // lanes of this wave holding the same digit
#pragma unroll
  for (int bit = 0; bit < 8; ++bit) {
    const uint64_t ones = __ballot(valid && ((d >> bit) & 1u));
    peers &= ((d >> bit) & 1u) ? ones : ~ones;
  }
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const uint32_t rank_w = uint32_t(__popcll(peers & lt_mask));
  if (valid && rank_w == 0) wave_cnt[wave][d] = uint32_t(__popcll(peers));
  __syncthreads();
  uint32_t rank = 0;
  if (valid) {
    rank = running[d] + rank_w;
    for (int w = 0; w < wave; ++w) rank += wave_cnt[w][d];
  }
  __syncthreads();
  if (t < 256) {
    uint32_t add = 0;
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) add += wave_cnt[w][t];
    running[t] += add;
  }
  __syncthreads();
  return rank;
}

// bounds[2r] / bounds[2r+1] = first / one-past-last sorted position of key r
// (both 0 when r has no updates; zero-filled beforehand).
__global__ __launch_bounds__(kBlock) void bucket_bounds_kernel(const uint32_t* __restrict__ keys,
                                                               int64_t n, int64_t n_rows,
                                                               uint32_t* __restrict__ bounds) {
  const int64_t j = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  if (j >= n) return;
  const uint32_t k = keys[j];
  if (k >= uint32_t(n_rows)) return;  // dropped ids sort last
  if (j == 0 || keys[j - 1] != k) bounds[2 * int64_t(k)] = uint32_t(j);
  if (j == n - 1 || keys[j + 1] != k) bounds[2 * int64_t(k) + 1] = uint32_t(j + 1);
}

// One wave per destination row.  For fp32 the order of adds per element is
// table, then updates in increasing index — exactly the sequential order.
// For bf16 each add is rounded to bf16 as a bf16 scatter would.
template <bool BF16>
__global__ __launch_bounds__(kBlock) void scatter_accumulate_kernel(
    const void* __restrict__ table, void* __restrict__ out, int64_t n_rows, int64_t row_len,
    const void* __restrict__ updates, const uint32_t* __restrict__ vals,
    const uint32_t* __restrict__ bounds, bool in_place, bool vec_ok) {
  const int lane = threadIdx.x & 63;
  // wave-uniform row index, so the bounds and sorted update ids are scalar loads
  const int64_t r = int64_t(blockIdx.x) * (kBlock / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (r >= n_rows) return;
  const uint32_t b = bounds[2 * r], e = bounds[2 * r + 1];
  if (in_place && b == e) return;  // untouched row already holds its value
  if constexpr (!BF16) {
    const float* tr = reinterpret_cast<const float*>(table) + r * row_len;
    float* orow = reinterpret_cast<float*>(out) + r * row_len;
    const float* up = reinterpret_cast<const float*>(updates);
    if (vec_ok) {
      // up to four float4 columns per lane per sweep (row_len <= 1024 in one);
      // the next update row is loaded while the current one is added
      constexpr int Q = 4;
      const int64_t nv = row_len / 4;
      const f32x4* t4 = reinterpret_cast<const f32x4*>(tr);
      for (int64_t c0 = lane; c0 < nv; c0 += Q * 64) {
        bool ok[Q];
        f32x4 acc[Q], u[Q], un[Q];
#pragma unroll
        for (int q = 0; q < Q; ++q) {
          ok[q] = c0 + q * 64 < nv;
          if (ok[q]) acc[q] = t4[c0 + q * 64];
        }
        auto load_upd = [&](uint32_t j, f32x4(&dst)[Q]) __attribute__((always_inline)) {
          const f32x4* urow = reinterpret_cast<const f32x4*>(up + int64_t(vals[j]) * row_len);
#pragma unroll
          for (int q = 0; q < Q; ++q)
            if (ok[q]) dst[q] = urow[c0 + q * 64];
        };
        if (b < e) load_upd(b, u);
        for (uint32_t j = b; j < e; ++j) {
          if (j + 1 < e) load_upd(j + 1, un);
#pragma unroll
          for (int q = 0; q < Q; ++q)
            if (ok[q])
#pragma unroll
              for (int z = 0; z < 4; ++z) acc[q].v[z] += u[q].v[z];
#pragma unroll
          for (int q = 0; q < Q; ++q) u[q] = un[q];
        }
#pragma unroll
        for (int q = 0; q < Q; ++q)
          if (ok[q]) reinterpret_cast<f32x4*>(orow)[c0 + q * 64] = acc[q];
      }
    } else {
      for (int64_t c = lane; c < row_len; c += 64) {
        float acc = tr[c];
        for (uint32_t j = b; j < e; ++j) acc += up[int64_t(vals[j]) * row_len + c];
        orow[c] = acc;
      }
    }
  } else {
    const uint16_t* tr = reinterpret_cast<const uint16_t*>(table) + r * row_len;
    uint16_t* orow = reinterpret_cast<uint16_t*>(out) + r * row_len;
    const uint16_t* up = reinterpret_cast<const uint16_t*>(updates);
    for (int64_t c = lane; c < row_len; c += 64) {
      float acc = bf16_to_f32(tr[c]);
      for (uint32_t j = b; j < e; ++j)
        acc = bf16_to_f32(f32_to_bf16(acc + bf16_to_f32(up[int64_t(vals[j]) * row_len + c])));
      orow[c] = f32_to_bf16(acc);
    }
  }
}

// Streaming (non-temporal) access for data touched once: the update rows
// and the output rows.  They bypass cache allocation, which raises the
// combined read + write rate of these kernels by about a fifth on MI355X.
__device__ inline f32x4 load_stream(const f32x4* p) {
  typedef float v4 __attribute__((ext_vector_type(4)));
  const v4 x = __builtin_nontemporal_load(reinterpret_cast<const v4*>(p));
  return f32x4{{x.x, x.y, x.z, x.w}};
}
__device__ inline void store_stream(f32x4* p, const f32x4& a) {
  typedef float v4 __attribute__((ext_vector_type(4)));
  __builtin_nontemporal_store(v4{a.v[0], a.v[1], a.v[2], a.v[3]}, reinterpret_cast<v4*>(p));
}

// fp32 rows as float4 vectors, one wave per destination row, all of a row's
// loads in flight together: the bucket's sorted update indices come in with
// one vector load (64 at a time) and are broadcast with v_readlane; the table
// row and up to kScatterU update rows are loaded before any add, and the adds
// run in bucket order (= increasing update index), so the result is the
// sequential one bit for bit.  Columns go in blocks of 64 * RV float4.
constexpr int kScatterU = 4;

template <int RV>
__global__ __launch_bounds__(kBlock) void scatter_accumulate_vec_kernel(
    const f32x4* __restrict__ table, f32x4* __restrict__ out, int64_t n_rows, int64_t nv,
    const f32x4* __restrict__ updates, const uint32_t* __restrict__ vals, const uint32_t* __restrict__ bounds,
    bool in_place) {
  const int lane = threadIdx.x & 63;
  const int64_t r = int64_t(blockIdx.x) * (kBlock / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (r >= n_rows) return;
  const uint32_t b = bounds[2 * r], e = bounds[2 * r + 1];
  if (in_place && b == e) return;  // untouched row already holds its value
  for (int64_t cb = 0; cb < nv; cb += 64 * RV) {
    // lanes past the row end load its last vector (always in bounds) and
    // store nothing, so no load needs a per-lane predicate
    int64_t col[RV];
    bool ok[RV];
#pragma unroll
    for (int q = 0; q < RV; ++q) {
      const int64_t c = cb + q * 64 + lane;
      ok[q] = c < nv;
      col[q] = ok[q] ? c : nv - 1;
    }
    uint32_t myv = (uint32_t(lane) < e - b) ? vals[b + lane] : 0u;  // first chunk of bucket indices
    f32x4 acc[RV];
#pragma unroll
    for (int q = 0; q < RV; ++q) acc[q] = table[r * nv + col[q]];
    for (uint32_t j0 = b; j0 < e; j0 += 64) {
      const uint32_t cnt = min(64u, e - j0);
      if (j0 != b) myv = (uint32_t(lane) < cnt) ? vals[j0 + lane] : 0u;
      for (uint32_t k0 = 0; k0 < cnt; k0 += kScatterU) {
        const uint32_t g = min(uint32_t(kScatterU), cnt - k0);  // wave-uniform group size
        int64_t row[kScatterU];
#pragma unroll
        for (int t = 0; t < kScatterU; ++t)
          row[t] = int64_t(__builtin_amdgcn_readlane(myv, int(k0 + min(uint32_t(t), g - 1))));
        f32x4 u[kScatterU][RV];
        // loads of the group (g rows), then the adds in order
        auto run = [&](auto gn) __attribute__((always_inline)) {
          constexpr int G = decltype(gn)::value;
#pragma unroll
          for (int t = 0; t < G; ++t)
#pragma unroll
            for (int q = 0; q < RV; ++q) u[t][q] = load_stream(updates + row[t] * nv + col[q]);
#pragma unroll
          for (int t = 0; t < G; ++t)
#pragma unroll
            for (int q = 0; q < RV; ++q)
#pragma unroll
              for (int z = 0; z < 4; ++z) acc[q].v[z] += u[t][q].v[z];
        };
        if (g == 4) run(std::integral_constant<int, 4>{});
        else if (g == 3) run(std::integral_constant<int, 3>{});
        else if (g == 2) run(std::integral_constant<int, 2>{});
        else run(std::integral_constant<int, 1>{});
      }
    }
#pragma unroll
    for (int q = 0; q < RV; ++q)
      if (ok[q]) store_stream(out + r * nv + col[q], acc[q]);
  }
}

// ------------------------------------------------------------------ 16-bit keys: bucket build
// One workgroup of kBuildThreads per bucket of 256 destination rows (key >>
// 8 == bucket); it writes the bucket's part of the sorted index list and
// the bounds of its rows, which the accumulate kernels read as they read
// the radix sort's.  The workgroup
//   1. scans all ids once (each wave a contiguous segment, kBuildBatch
//      16-byte loads in flight per lane, L2 resident after the first
//      workgroups; wave-level ballots, no cross-lane shuffles), counting per
//      row of the bucket (LDS atomics), the bucket's matches per segment and
//      the ids of lower buckets, whose count is where the bucket starts in
//      the list; the row counts' exclusive scan gives every row's bounds.
//      The same scan keeps each segment's first kBuildCap / kBuildWaves
//      matches (update index, key & 255) in index order in LDS;
//   2. places the bucket's entries stably by row (ballot ranks per
//      1024-entry chunk, running counts across chunks) into the list.  If a
//      segment had more matches than its region holds, a second scan
//      collects them instead, kBuildCap at a time.
// No workgroup waits for another, so the sort is a single launch.
constexpr int kBuildThreads = 1024, kBuildWaves = kBuildThreads / 64, kBuildCap = 4096, kBuildBatch = 16;

template <typename IdxT>
__global__ __launch_bounds__(kBuildThreads) void bucket_build_kernel(const IdxT* __restrict__ ids, int64_t n_ids,
                                                                     int64_t n_rows, int64_t seg, bool aligned,
                                                                     uint32_t* __restrict__ vals,
                                                                     uint32_t* __restrict__ bounds) {
  __shared__ uint32_t list[kBuildCap];
  __shared__ uint32_t cnt[256], row_start[256], running[256];
  __shared__ uint32_t wave_cnt[kBuildWaves][256];
  __shared__ uint32_t wmatch[kBuildWaves], wbefore[kBuildWaves];
  constexpr int V = 16 / int(sizeof(IdxT));  // ids per 16-byte load
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const uint32_t bucket = blockIdx.x;
  // The ids are cut into kBuildWaves segments; wave w scans segment (w +
  // bucket) % kBuildWaves, so the workgroups, which start together, do not
  // all read the same lines at once (one L2 channel would serve them all).
  const int sg = (wave + int(bucket)) % kBuildWaves;
  const int64_t s0 = min(n_ids, int64_t(sg) * seg), s1 = min(n_ids, s0 + seg);
  if (t < 256) {
    cnt[t] = 0;
    running[t] = 0;
  }
  __syncthreads();

  // Visits the wave's ids in increasing index: f(e0, key, nvalid) for each
  // 64 V chunk, lane l holding ids e0 .. e0 + V - 1 (e0 = chunk + l V), of
  // which the first nvalid are inside the segment (V for every lane of a
  // full chunk); all lanes of the wave call f for the same chunk together.
  // Indices fit 32 bits here (n_ids < 2^24); key = the id, or n_rows for an
  // id outside [0, n_rows).
  auto visit = [&](auto&& f) __attribute__((always_inline)) {
    for (uint32_t c0 = uint32_t(s0); c0 < uint32_t(s1); c0 += uint32_t(kBuildBatch) * 64 * V) {
      IdxT v[kBuildBatch][V];
#pragma unroll
      for (int b = 0; b < kBuildBatch; ++b) {
        const uint32_t c = c0 + uint32_t(b) * 64 * V, e0 = c + uint32_t(lane) * V;
        if (aligned && int64_t(c) + 64 * V <= n_ids) {  // wave-uniform: the whole chunk is inside
          const u32x4_t w = *reinterpret_cast<const u32x4_t*>(ids + e0);
          __builtin_memcpy(v[b], &w, 16);
        } else {
#pragma unroll
          for (int j = 0; j < V; ++j) v[b][j] = int64_t(e0) + j < n_ids ? ids[e0 + j] : IdxT(-1);
        }
      }
#pragma unroll
      for (int b = 0; b < kBuildBatch; ++b) {
        const uint32_t c = c0 + uint32_t(b) * 64 * V;
        if (c >= uint32_t(s1)) break;  // wave-uniform
        const uint32_t e0 = c + uint32_t(lane) * V;
        const int nvalid = c + 64 * V <= uint32_t(s1) ? V : int(min(uint32_t(V), uint32_t(s1) - min(uint32_t(s1), e0)));
        uint32_t key[V];
#pragma unroll
        for (int j = 0; j < V; ++j) {
          if constexpr (sizeof(IdxT) == 4)
            key[j] = uint32_t(v[b][j]) < uint32_t(n_rows) ? uint32_t(v[b][j]) : uint32_t(n_rows);
          else
            key[j] = uint64_t(v[b][j]) < uint64_t(n_rows) ? uint32_t(v[b][j]) : uint32_t(n_rows);
        }
        f(e0, key, nvalid);
      }
    }
  };
  // bits of `mask` below this lane
  auto below = [&](uint64_t mask) __attribute__((always_inline)) {
    return __builtin_amdgcn_mbcnt_hi(uint32_t(mask >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(mask), 0u));
  };

  // 1. counts (ballots: wave-uniform sums, no cross-lane shuffles), and the
  // segment's first kBuildSeg matches, in index order, in its region of list
  constexpr uint32_t kBuildSeg = kBuildCap / kBuildWaves;
  uint32_t nm = 0, nb = 0;
  visit([&](uint32_t e0, const uint32_t (&key)[V], int nvalid) __attribute__((always_inline)) {
    bool m[V];
    uint64_t mask[V], any = 0;
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const uint32_t kb = key[j] >> 8;
      m[j] = j < nvalid && kb == bucket;
      mask[j] = __ballot(m[j]);
      any |= mask[j];
      nb += uint32_t(__popcll(__ballot(j < nvalid && kb < bucket)));
    }
    if (any == 0) return;  // wave-uniform: no id of the bucket in this chunk
    uint32_t rank = nm;  // rank in the segment of this lane's first match
#pragma unroll
    for (int j = 0; j < V; ++j) {
      rank += below(mask[j]);
      nm += uint32_t(__popcll(mask[j]));
    }
#pragma unroll
    for (int j = 0; j < V; ++j)
      if (m[j]) {
        atomicAdd(&cnt[key[j] & 255u], 1u);
        if (rank < kBuildSeg) list[uint32_t(sg) * kBuildSeg + rank] = ((e0 + j) << 8) | (key[j] & 255u);
        ++rank;
      }
  });
  if (lane == 0) {
    wmatch[sg] = nm;
    wbefore[sg] = nb;
  }
  __syncthreads();
  uint32_t start = 0, total = 0, base = 0;  // bucket start in the list, its size, this segment's first rank
  bool spill = false;                         // some segment has more matches than its region holds
  for (int g = 0; g < kBuildWaves; ++g) {
    start += wbefore[g];
    total += wmatch[g];
    base += g < sg ? wmatch[g] : 0u;
    spill |= wmatch[g] > kBuildSeg;
  }
  if (t < 64) {  // exclusive scan of the 256 row counts, 4 per lane of wave 0
    uint32_t c4[4], sum = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      c4[k] = cnt[4 * t + k];
      sum += c4[k];
    }
    uint32_t incl = sum;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const uint32_t o = uint32_t(__shfl_up(int(incl), off, 64));
      if (lane >= off) incl += o;
    }
    uint32_t at = incl - sum;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      row_start[4 * t + k] = at;
      const int64_t r = int64_t(bucket) * 256 + 4 * t + k;
      if (r < n_rows) {
        bounds[2 * r] = start + at;
        bounds[2 * r + 1] = start + at + c4[k];
      }
      at += c4[k];
    }
  }
  __syncthreads();

  // 2. stable placement by row, entry by entry in bucket rank order (ballot
  // ranks per 1024-entry chunk, running counts across chunks and rounds)
  auto place = [&](uint32_t len, auto&& entry) __attribute__((always_inline)) {
    for (uint32_t c0 = 0; c0 < len; c0 += kBuildThreads) {
      const uint32_t i = c0 + uint32_t(t);
      const bool valid = i < len;
      const uint32_t ent = valid ? entry(i) : 0u, d = ent & 255u;
      const uint32_t rank = chunk_rank<kBuildThreads>(valid, d, running, wave_cnt);
      if (valid) vals[start + row_start[d] + rank] = ent >> 8;
    }
  };
  if (!spill) {  // every match is in its segment's region: one round, no second scan
    place(total, [&](uint32_t i) __attribute__((always_inline)) {
      uint32_t g = 0, first = 0;  // segment holding bucket rank i
      while (i >= first + wmatch[g]) first += wmatch[g++];
      return list[g * kBuildSeg + (i - first)];
    });
    return;
  }
  // a segment spilled: rounds of up to kBuildCap entries collected by a
  // second scan
  __syncthreads();  // done reading the regions written by the first scan
  for (uint32_t lo = 0; lo < total; lo += kBuildCap) {
    const uint32_t hi = min(total, lo + kBuildCap), len = hi - lo;
    uint32_t run = base;  // bucket-wide rank of the wave's next match
    visit([&](uint32_t e0, const uint32_t (&key)[V], int nvalid) __attribute__((always_inline)) {
      // rank of (lane, j): matches of earlier lanes (all V slots) and of
      // this lane's earlier slots
      bool m[V];
      uint64_t mask[V];
      uint32_t rank = run;
#pragma unroll
      for (int j = 0; j < V; ++j) {
        m[j] = j < nvalid && (key[j] >> 8) == bucket;
        mask[j] = __ballot(m[j]);
        rank += below(mask[j]);
        run += uint32_t(__popcll(mask[j]));
      }
#pragma unroll
      for (int j = 0; j < V; ++j)
        if (m[j]) {
          if (rank >= lo && rank < hi) list[rank - lo] = ((e0 + j) << 8) | (key[j] & 255u);
          ++rank;
        }
    });
    __syncthreads();
    place(len, [&](uint32_t i) __attribute__((always_inline)) { return list[i]; });
    __syncthreads();  // the list is rewritten by the next round
  }
}

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

struct ScatterWs {
  uint32_t *keys0, *vals0, *keys1, *vals1, *hist, *bounds;
  int nb;
};

inline ScatterWs carve(void* ws, int64_t n_rows, int64_t n_ids) {
  ScatterWs w;
  char* p = reinterpret_cast<char*>(ws);
  const size_t idb = align256(size_t(n_ids) * 4);
  w.nb = int((n_ids + kSortTile - 1) / kSortTile);
  w.keys0 = reinterpret_cast<uint32_t*>(p); p += idb;
  w.vals0 = reinterpret_cast<uint32_t*>(p); p += idb;
  w.keys1 = reinterpret_cast<uint32_t*>(p); p += idb;
  w.vals1 = reinterpret_cast<uint32_t*>(p); p += idb;
  w.hist = reinterpret_cast<uint32_t*>(p); p += align256(size_t(256) * (w.nb > 0 ? w.nb : 1) * 4);
  w.bounds = reinterpret_cast<uint32_t*>(p);
  return w;
}

inline unsigned blocks_for(int64_t n, int per) { return unsigned((n + per - 1) / per); }

}  // namespace
}  // namespace mk

using namespace mk;

extern "C" int mk_gather_rows(void* stream, int64_t n_rows, int64_t row_bytes, const void* table,
                              int index_type, int64_t n_ids, const void* ids, void* out) {
  clear_error();
  if (n_rows <= 0 || row_bytes < 0 || n_ids < 0)
    return fail(MK_ERR_INVALID, "mk_gather_rows: need n_rows >= 1, row_bytes >= 0, n_ids >= 0");
  if (row_bytes % 4 != 0) return fail(MK_ERR_UNSUPPORTED, "mk_gather_rows: row_bytes % 4 != 0");
  if (index_type != MK_S32 && index_type != MK_S64)
    return fail(MK_ERR_UNSUPPORTED, "mk_gather_rows: index_type must be s32/s64");
  if (n_ids == 0 || row_bytes == 0) return MK_OK;
  if (!table || !ids || !out) return fail(MK_ERR_INVALID, "mk_gather_rows: null pointer");
  hipStream_t s = as_stream(stream);
  dim3 g(blocks_for(n_ids, kBlock / 64)), b(kBlock);
  const bool v16 = row_bytes % 16 == 0 &&
                   ((reinterpret_cast<uintptr_t>(table) | reinterpret_cast<uintptr_t>(out)) & 15u) == 0;
  if (v16) {
    if (index_type == MK_S32)
      hipLaunchKernelGGL(gather_rows16_kernel<int32_t>, g, b, 0, s, (const u32x4_t*)table, n_rows,
                         row_bytes / 16, (const int32_t*)ids, n_ids, (u32x4_t*)out);
    else
      hipLaunchKernelGGL(gather_rows16_kernel<int64_t>, g, b, 0, s, (const u32x4_t*)table, n_rows,
                         row_bytes / 16, (const int64_t*)ids, n_ids, (u32x4_t*)out);
  } else {
    if (index_type == MK_S32)
      hipLaunchKernelGGL(gather_rows4_kernel<int32_t>, g, b, 0, s, (const uint32_t*)table, n_rows,
                         row_bytes / 4, (const int32_t*)ids, n_ids, (uint32_t*)out);
    else
      hipLaunchKernelGGL(gather_rows4_kernel<int64_t>, g, b, 0, s, (const uint32_t*)table, n_rows,
                         row_bytes / 4, (const int64_t*)ids, n_ids, (uint32_t*)out);
  }
  return check_launch("mk_gather_rows");
}

extern "C" size_t mk_scatter_add_workspace_bytes(int64_t n_rows, int64_t n_ids) {
  if (n_rows < 0 || n_ids < 0) return 0;
  const int64_t nb = (n_ids + kSortTile - 1) / kSortTile;
  return 4 * align256(size_t(n_ids) * 4) + align256(size_t(256) * size_t(nb > 0 ? nb : 1) * 4) +
         align256(size_t(n_rows) * 8);
}

namespace mk {
namespace {

// Validates the arguments shared by both scatter-add entry points; MK_OK
// means "go on", anything else is returned as is (with *done = true for a
// valid call that has nothing to do).
int scatter_check(const char* name, int dtype, int64_t n_rows, int64_t row_len, int index_type, int64_t n_ids,
                  bool* done) {
  *done = false;
  const std::string n(name);
  if (n_rows < 0 || row_len < 0 || n_ids < 0) return fail(MK_ERR_INVALID, n + ": negative size");
  if (dtype != MK_F32 && dtype != MK_BF16) return fail(MK_ERR_UNSUPPORTED, n + ": dtype must be f32/bf16");
  if (index_type != MK_S32 && index_type != MK_S64) return fail(MK_ERR_UNSUPPORTED, n + ": index_type must be s32/s64");
  if (n_rows >= (int64_t(1) << 31) || n_ids >= (int64_t(1) << 31))
    return fail(MK_ERR_UNSUPPORTED, n + ": n_rows and n_ids must be < 2^31");
  *done = n_rows == 0 || row_len == 0;
  return MK_OK;
}

// Scratch of the allocation-free scatter-add: one copy per GPU, for the
// whole process.  Host code never uses this name as an address (on the host
// it is a stand-in, not device memory): scratch_on() looks up each device's
// own copy with hipGetSymbolAddress.
__device__ __align__(256) unsigned char scratch[MK_SCATTER_ADD_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the device that owns `stream` (looked up
// once per device, with that device current).  nullptr and the error set on
// failure.
void* scratch_on(hipStream_t stream) {
  int dev = -1;
  hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    fail(MK_ERR_INVALID, "mk_scatter_add_rows_noalloc: cannot tell the stream's device");
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev]) return g_scratch_ptr[dev];
  int cur = -1;
  (void)hipGetDevice(&cur);
  if (cur != dev) (void)hipSetDevice(dev);
  void* p = nullptr;
  e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (cur != dev && cur >= 0) (void)hipSetDevice(cur);
  if (e != hipSuccess || !p) {
    (void)hipGetLastError();
    fail(MK_ERR_LAUNCH, std::string("mk_scatter_add_rows_noalloc: hipGetSymbolAddress: ") + hipGetErrorString(e));
    return nullptr;
  }
  g_scratch_ptr[dev] = p;
  return p;
}

int scatter_add_launch(hipStream_t s, int dtype, int64_t n_rows, int64_t row_len, const void* table,
                       int index_type, int64_t n_ids, const void* ids, const void* updates, void* out,
                       void* workspace, const char* name);

}  // namespace
}  // namespace mk

extern "C" int mk_scatter_add_rows(void* stream, int dtype, int64_t n_rows, int64_t row_len,
                                   const void* table, int index_type, int64_t n_ids,
                                   const void* ids, const void* updates, void* out,
                                   void* workspace) {
  clear_error();
  bool done = false;
  if (int rc = scatter_check("mk_scatter_add_rows", dtype, n_rows, row_len, index_type, n_ids, &done)) return rc;
  if (done) return MK_OK;
  if (!table || !out || (n_ids > 0 && (!ids || !updates || !workspace)))
    return fail(MK_ERR_INVALID, "mk_scatter_add_rows: null pointer");
  return scatter_add_launch(as_stream(stream), dtype, n_rows, row_len, table, index_type, n_ids, ids, updates, out,
                            workspace, "mk_scatter_add_rows");
}

extern "C" int mk_scatter_add_rows_noalloc(void* stream, int dtype, int64_t n_rows, int64_t row_len,
                                           const void* table, int index_type, int64_t n_ids,
                                           const void* ids, const void* updates, void* out) {
  clear_error();
  bool done = false;
  if (int rc = scatter_check("mk_scatter_add_rows_noalloc", dtype, n_rows, row_len, index_type, n_ids, &done))
    return rc;
  if (done) return MK_OK;
  const size_t need = mk_scatter_add_workspace_bytes(n_rows, n_ids);
  if (need > size_t(MK_SCATTER_ADD_SCRATCH_BYTES))
    return fail(MK_ERR_UNSUPPORTED, "mk_scatter_add_rows_noalloc: needs " + std::to_string(need) +
                                        " bytes of scratch, more than the " +
                                        std::to_string(size_t(MK_SCATTER_ADD_SCRATCH_BYTES)) +
                                        " bytes it has; use mk_scatter_add_rows with a workspace");
  if (!table || !out || (n_ids > 0 && (!ids || !updates)))
    return fail(MK_ERR_INVALID, "mk_scatter_add_rows_noalloc: null pointer");
  hipStream_t s = as_stream(stream);
  void* ws = scratch_on(s);
  if (!ws) return MK_ERR_LAUNCH;
  return scatter_add_launch(s, dtype, n_rows, row_len, table, index_type, n_ids, ids, updates, out, ws,
                            "mk_scatter_add_rows_noalloc");
}

namespace mk {
namespace {

// Queues the whole scatter-add on `s`.  `workspace` holds at least
// mk_scatter_add_workspace_bytes(n_rows, n_ids) bytes; every part of it that
// is read is written first by the same call (the row bounds are written or
// cleared before they are read), so leftovers of an earlier call do not
// matter.
int scatter_add_launch(hipStream_t s, int dtype, int64_t n_rows, int64_t row_len, const void* table,
                       int index_type, int64_t n_ids, const void* ids, const void* updates, void* out,
                       void* workspace, const char* name) {
  ScatterWs w = carve(workspace, n_rows, n_ids);
  // bounds start at zero (rows without updates have an empty range); the
  // bucket build writes every row's, the radix path's prepare kernel clears
  // them
  if (n_ids == 0)
    hipLaunchKernelGGL((fill_words), dim3(blocks_for(2 * n_rows, kBlock)), dim3(kBlock), 0, s, w.bounds, 2 * n_rows);
  if (n_ids > 0 && n_rows < 65535 && n_ids < (int64_t(1) << 24)) {
    // 16-bit keys (n_rows itself included, for dropped ids): one launch
    const int V = index_type == MK_S32 ? 4 : 2;
    const int64_t chunk = int64_t(kBuildWaves) * 64 * V;
    const int64_t seg = (n_ids + chunk - 1) / chunk * 64 * V;
    const bool aligned = (reinterpret_cast<uintptr_t>(ids) & 15u) == 0;
    const dim3 g(unsigned((n_rows + 255) / 256)), b(kBuildThreads);
    if (index_type == MK_S32)
      hipLaunchKernelGGL(bucket_build_kernel<int32_t>, g, b, 0, s, (const int32_t*)ids, n_ids, n_rows, seg, aligned, w.vals0, w.bounds);
    else
      hipLaunchKernelGGL(bucket_build_kernel<int64_t>, g, b, 0, s, (const int64_t*)ids, n_ids, n_rows, seg, aligned, w.vals0, w.bounds);
  } else if (n_ids > 0) {
    const unsigned gi = blocks_for(n_ids, kBlock);
    const unsigned gp = blocks_for(std::max<int64_t>(n_ids, 2 * n_rows), kBlock);
    if (index_type == MK_S32)
      hipLaunchKernelGGL(scatter_prepare_kernel<int32_t>, dim3(gp), dim3(kBlock), 0, s, (const int32_t*)ids, n_ids, n_rows, w.keys0, w.vals0, w.bounds);
    else
      hipLaunchKernelGGL(scatter_prepare_kernel<int64_t>, dim3(gp), dim3(kBlock), 0, s, (const int64_t*)ids, n_ids, n_rows, w.keys0, w.vals0, w.bounds);
    // keys are in [0, n_rows]: sort only the bits that can be set
    int bits = 0;
    while ((int64_t(1) << bits) <= n_rows) ++bits;
    uint32_t *kin = w.keys0, *vin = w.vals0, *kout = w.keys1, *vout = w.vals1;
    for (int shift = 0; shift < bits; shift += 8) {
      hipLaunchKernelGGL(radix_hist_kernel, dim3(w.nb), dim3(kBlock), 0, s, kin, n_ids, shift, w.hist, w.nb);
      hipLaunchKernelGGL(scan_exclusive_kernel, dim3(1), dim3(kScanBlock), 0, s, w.hist, int64_t(256) * w.nb);
      hipLaunchKernelGGL(radix_scatter_kernel, dim3(w.nb), dim3(kBlock), 0, s, kin, vin, n_ids, shift, w.hist, w.nb, kout, vout);
      uint32_t* tk = kin; kin = kout; kout = tk;
      uint32_t* tv = vin; vin = vout; vout = tv;
    }
    hipLaunchKernelGGL(bucket_bounds_kernel, dim3(gi), dim3(kBlock), 0, s, kin, n_ids, n_rows, w.bounds);
    w.vals0 = vin;  // sorted values
  }
  const bool in_place = table == out;
  const bool vec_ok = dtype == MK_F32 && row_len % 4 == 0 &&
                      ((reinterpret_cast<uintptr_t>(table) | reinterpret_cast<uintptr_t>(out) |
                        reinterpret_cast<uintptr_t>(updates)) & 15u) == 0;
  dim3 g(blocks_for(n_rows, kBlock / 64));
  if (dtype == MK_F32 && vec_ok) {
    const int64_t nv = row_len / 4;
    auto go = [&](auto kern) {
      hipLaunchKernelGGL(kern, g, dim3(kBlock), 0, s, (const f32x4*)table, (f32x4*)out, n_rows, nv,
                         (const f32x4*)updates, w.vals0, w.bounds, in_place);
    };
    if (nv <= 64) go(scatter_accumulate_vec_kernel<1>);
    else if (nv <= 128) go(scatter_accumulate_vec_kernel<2>);
    else if (nv <= 192) go(scatter_accumulate_vec_kernel<3>);
    else go(scatter_accumulate_vec_kernel<4>);
  } else if (dtype == MK_F32)
    hipLaunchKernelGGL(scatter_accumulate_kernel<false>, g, dim3(kBlock), 0, s, table, out, n_rows, row_len, updates, w.vals0, w.bounds, in_place, vec_ok);
  else
    hipLaunchKernelGGL(scatter_accumulate_kernel<true>, g, dim3(kBlock), 0, s, table, out, n_rows, row_len, updates, w.vals0, w.bounds, in_place, false);
  return check_launch(name);
}

}  // namespace
}  // namespace mk
