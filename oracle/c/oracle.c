/*
 * C restatement of the bit-exact parts of the hot path — ORACLE, TEST
 * INFRASTRUCTURE ONLY (used by tests/, smoke() and bench.py's cpu_baseline).
 *
 * Sequential loops, no threading, no reordering: the point is to state the
 * order of operations the GPU kernels must reproduce bit for bit.
 *   oracle_scatter_add_f32   — updates applied one at a time in increasing
 *                              index, fp32 adds (restates XLA:CPU's
 *                              sequential scatter; replaces the order-
 *                              unspecified MPSGraph scatter-add of
 *                              src/jam/ops/gather_scatter.mm:322-327)
 *   oracle_scatter_add_bf16  — same, rounding to bf16 (RNE) after every add
 *   oracle_argmax_rows_bf16  — first index of the max/min, NaN wins
 *                              (src/jam/ops/reduce.mm:29-77 pattern)
 *   oracle_row_sum_bf16      — float64 row sums of bf16 rows
 *   oracle_gather_rows       — clamped row copy (gather_scatter.mm:180-196)
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

void oracle_scatter_add_f32(float* table, int64_t n_rows, int64_t row_len, const int32_t* ids,
                            int64_t n_ids, const float* updates) {
  for (int64_t i = 0; i < n_ids; ++i) {
    const int64_t r = ids[i];
    if (r < 0 || r >= n_rows) continue;
    float* dst = table + r * row_len;
    const float* src = updates + i * row_len;
    for (int64_t c = 0; c < row_len; ++c) dst[c] = dst[c] + src[c];
  }
}

void oracle_scatter_add_bf16(uint16_t* table, int64_t n_rows, int64_t row_len, const int32_t* ids,
                             int64_t n_ids, const uint16_t* updates) {
  for (int64_t i = 0; i < n_ids; ++i) {
    const int64_t r = ids[i];
    if (r < 0 || r >= n_rows) continue;
    uint16_t* dst = table + r * row_len;
    const uint16_t* src = updates + i * row_len;
    for (int64_t c = 0; c < row_len; ++c)
      dst[c] = f32_to_bf16(bf16_to_f32(dst[c]) + bf16_to_f32(src[c]));
  }
}

void oracle_argmax_rows_bf16(const uint16_t* x, int64_t rows, int64_t cols, int is_min,
                             int64_t* idx, uint16_t* vals) {
  for (int64_t r = 0; r < rows; ++r) {
    const uint16_t* row = x + r * cols;
    int64_t bi = 0;
    float bv = bf16_to_f32(row[0]);
    for (int64_t c = 1; c < cols; ++c) {
      const float v = bf16_to_f32(row[c]);
      int take;
      if (isnan(v) || isnan(bv)) take = isnan(v) && !isnan(bv);
      else take = is_min ? (v < bv) : (v > bv);  /* equal keeps the lower index */
      if (take) { bv = v; bi = c; }
    }
    idx[r] = bi;
    if (vals) vals[r] = row[bi];
  }
}

void oracle_row_sum_bf16(const uint16_t* x, int64_t rows, int64_t cols, double* out) {
  for (int64_t r = 0; r < rows; ++r) {
    double s = 0.0;
    for (int64_t c = 0; c < cols; ++c) s += (double)bf16_to_f32(x[r * cols + c]);
    out[r] = s;
  }
}

void oracle_gather_rows(const uint8_t* table, int64_t n_rows, int64_t row_bytes, const int32_t* ids,
                        int64_t n_ids, uint8_t* out) {
  for (int64_t i = 0; i < n_ids; ++i) {
    int64_t r = ids[i];
    if (r < 0) r = 0;
    if (r >= n_rows) r = n_rows - 1;
    memcpy(out + i * row_bytes, table + r * row_bytes, (size_t)row_bytes);
  }
}
