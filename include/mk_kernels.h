/*
 * mk_kernels.h — C-ABI of the hand-written gfx950 (MI355X) HIP kernels.
 *
 * This is the "thin C-ABI" the jam compiler lowers StableHLO into.  Every
 * entry point takes device pointers, explicit element counts / strides and a
 * hipStream_t passed as `void*`; none of them allocates device memory except
 * where a `workspace` argument is documented (callers size it with the
 * matching *_workspace_bytes query).  All launches are asynchronous on the
 * given stream.  Return value: MK_OK (0) or an MK_ERR_* code; the message for
 * the last failure on the calling thread is available from mk_last_error().
 *
 * Each entry point replaces one group of MPSGraph calls of the reference
 * (Lazarus-931/mccl-jax, Metal backend); the replaced call sites are cited as
 * path:line into that repository.
 */
#ifndef MI355X_MK_KERNELS_H_
#define MI355X_MK_KERNELS_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types.  Numeric values equal PJRT_Buffer_Type's so the plugin can
 * pass them through unchanged (third_party/xla/pjrt/c/pjrt_c_api.h:626-660). */
typedef enum mk_dtype {
  MK_PRED = 1, MK_S8 = 2, MK_S16 = 3, MK_S32 = 4, MK_S64 = 5,
  MK_U8 = 6, MK_U16 = 7, MK_U32 = 8, MK_U64 = 9,
  MK_F16 = 10, MK_F32 = 11, MK_F64 = 12, MK_BF16 = 13
} mk_dtype;

enum {
  MK_OK = 0,
  MK_ERR_INVALID = 1,     /* bad shape / stride / pointer / dtype combination */
  MK_ERR_UNSUPPORTED = 2, /* valid request this build has no kernel for       */
  MK_ERR_LAUNCH = 3       /* hipLaunchKernel / hipGetLastError failure         */
};

/* Message of the last failing call on this thread ("" when none). */
const char* mk_last_error(void);
/* ABI version of this header (bumped on incompatible change). */
int mk_abi_version(void);
/* Number of visible HIP devices (0 on a host without a GPU; never fails). */
int mk_device_count(void);

/* ------------------------------------------------------------------------
 * a4  dot_general → batched GEMM on MFMA.
 * Replaces: src/jam/ops/linalg.mm:98 (matrixMultiplicationWithPrimaryTensor)
 *           and the operand transposes/reshapes at linalg.mm:34-45,68-90.
 *
 * C[b][m][n] = sum_k A[b][m][k] * B[b][k][n]  (+ bias[n]) (then ReLU)
 *   A element (b,m,k) at  A + b*a_bs + m*a_ms + k*a_ks   (elements, not bytes)
 *   B element (b,k,n) at  B + b*b_bs + k*b_ks + n*b_ns
 *   C element (b,m,n) at  C + b*c_bs + m*c_ms + n        (row-major rows)
 * One of (a_ms, a_ks) and one of (b_ks, b_ns) must be 1 (unit stride); the
 * other operand stride is the leading dimension.  ab_type ∈ {MK_F32, MK_BF16}
 * (MK_F16 returns MK_ERR_UNSUPPORTED); c_type ∈ {MK_F32, MK_BF16, MK_F16};
 * accumulation is always fp32 (true fp32 MFMA for MK_F32 operands).
 * epilogue: 0 none, 1 +bias, 2 +bias then max(.,0).  bias has c_type, may be
 * NULL when epilogue == 0.  5 / 6: as 1 / 2 with an fp32 bias whatever c_type
 * (an fp32 product plus fp32 bias that the module only reads rounded to
 * bf16, written as bf16: the bias added to the fp32 accumulator, one
 * rounding).
 * ---------------------------------------------------------------------- */
int mk_gemm(void* stream, int ab_type, int c_type,
            int64_t batch, int64_t M, int64_t N, int64_t K,
            const void* A, int64_t a_bs, int64_t a_ms, int64_t a_ks,
            const void* B, int64_t b_bs, int64_t b_ks, int64_t b_ns,
            void* C, int64_t c_bs, int64_t c_ms,
            const void* bias, int epilogue);

/* mk_gemm (batch 1, epilogue 0, 1 or 5) whose epilogue also writes
 * Y[m][n] = bf16(gelu_tanh(C[m][n] as stored)) -- mk_gelu_tanh's function of
 * the stored (for bf16 C: rounded) value -- rows y_ms apart: the MLP's
 * up-projection, its bias and its activation in one pass (the reference's
 * dot_general, add and GELU chain, linalg.mm:47-105 and elementwise.mm).
 * Runs only on the tiled kernel: bf16 operands with 16-byte aligned rows,
 * M, N >= 128, K >= 64, c_type bf16 (C and Y rows 16-byte aligned) or f32
 * (C rows 16-byte, Y rows 8-byte aligned); MK_ERR_UNSUPPORTED otherwise. */
int mk_gemm_bias_gelu(void* stream, int ab_type, int c_type, int64_t M, int64_t N, int64_t K, const void* A,
                      int64_t a_ms, int64_t a_ks, const void* B, int64_t b_ks, int64_t b_ns, void* C,
                      int64_t c_ms, const void* bias, int epilogue, void* Y, int64_t y_ms);

/* The MLP's backward through its activation in the product that forms the
 * incoming gradient: D = A·B (bf16 operands, fp32 accumulate, rounded to
 * bf16 as mk_gemm stores it), dx = bf16(D * gelu_tanh'(pre)) (the function
 * of mk_gelu_tanh_bwd) with pre the bf16 pre-activations (rows pre_ms
 * apart), and dx_colsum[c] = sum_r dx[r][c] over the stored dx (fp32, rows
 * in a fixed order: deterministic) -- the dot_general, the GELU backward
 * chain and the bias gradient's reduce (linalg.mm:47-105, elementwise.mm,
 * reduce.mm:97-106) in one pass plus a small column pass.  Runs only on the
 * tiled kernel: M, N >= 128, K >= 64, 16-byte aligned operand, dx and pre
 * rows (MK_ERR_UNSUPPORTED otherwise).  Workspace:
 * mk_gemm_gelu_bwd_workspace_bytes(M, N). */
size_t mk_gemm_gelu_bwd_workspace_bytes(int64_t M, int64_t N);
int mk_gemm_gelu_bwd(void* stream, int ab_type, int64_t M, int64_t N, int64_t K, const void* A, int64_t a_ms,
                     int64_t a_ks, const void* B, int64_t b_ks, int64_t b_ns, void* dx, int64_t dx_ms,
                     const void* pre, int64_t pre_ms, float* dx_colsum, void* workspace);

/* Split-K form of mk_gemm for fp32 outputs with few output tiles and a long
 * contraction (the weight gradients dW = Xᵀ dY of the training step: the
 * dot_general of linalg.mm:47-105 with the token axis contracted).  The K
 * axis is cut into `splits` equal slices; one batched mk_gemm writes the
 * slices' products to the workspace (splits x M x N fp32) and a second pass
 * adds them in slice order into C (deterministic: the result does not depend
 * on scheduling).  K % splits == 0; N and c_ms multiples of 4; C and
 * workspace 16-byte aligned; C is overwritten.  splits == 1 is a plain
 * mk_gemm call (no workspace).  Operand convention as mk_gemm.
 * Replaces, for these products: src/jam/ops/linalg.mm:98. */
size_t mk_gemm_splitk_workspace_bytes(int64_t M, int64_t N, int64_t splits);
int mk_gemm_splitk(void* stream, int ab_type, int64_t M, int64_t N, int64_t K, const void* A,
                   int64_t a_ms, int64_t a_ks, const void* B, int64_t b_ks, int64_t b_ns, float* C,
                   int64_t c_ms, int64_t splits, void* workspace);

/* mk_gemm_splitk with the output type chosen (c_type MK_F32, or MK_BF16:
 * the ordered fp32 slice sum rounded once to bf16), mk_gemm's epilogue
 * applied to the sum (0 none, 1 + bias, 2 + bias then max(., 0); bias has
 * c_type; config C1's fp32 layers, whose 64 and 16 output tiles are cut
 * along K) and, for bf16 operands
 * the tiled kernel takes (16-byte aligned rows), any K: when K % splits != 0
 * the slices are ceil(K / splits) rounded up to a multiple of 8 apart and the
 * last one is shorter (the vocabulary products of the training step, which
 * contract over 50257 classes).  A product with K % splits != 0 that the
 * tiled kernel does not take runs unsplit (mk_gemm).  Same workspace size
 * and rules as mk_gemm_splitk otherwise (bf16 C: 8-byte aligned).
 * Replaces, for these products: src/jam/ops/linalg.mm:98. */
int mk_gemm_splitk_typed(void* stream, int ab_type, int c_type, int64_t M, int64_t N, int64_t K, const void* A,
                         int64_t a_ms, int64_t a_ks, const void* B, int64_t b_ks, int64_t b_ns, void* C,
                         int64_t c_ms, int64_t splits, void* workspace, const void* bias, int epilogue);

/* Plain GEMM through rocBLAS (the linear layers of the training step and
 * their gradients: with no epilogue to fuse, a library GEMM does the work).  Same operand convention as
 * mk_gemm (row-major C with row stride c_ms, one unit stride per operand),
 * C = alpha A B + beta C; no bias.  ab_type ∈ {MK_BF16 (c_type MK_BF16 /
 * MK_F16 / MK_F32), MK_F32 (c_type MK_F32)}, fp32 accumulation.  Operands
 * with overlapping rows (leading stride below the row length) are rejected.
 * Replaces, for these products: src/jam/ops/linalg.mm:98. */
int mk_gemm_blas(void* stream, int ab_type, int c_type,
                 int64_t batch, int64_t M, int64_t N, int64_t K,
                 const void* A, int64_t a_bs, int64_t a_ms, int64_t a_ks,
                 const void* B, int64_t b_bs, int64_t b_ks, int64_t b_ns,
                 void* C, int64_t c_bs, int64_t c_ms, float alpha, float beta);

/* Split-K form of mk_gemm_blas for fp32 outputs with few output tiles and a
 * long contraction (the weight gradients dW = Xᵀ dY of the training step,
 * linalg.mm:47-105's dot_general with the token axis contracted): the K axis
 * is cut into `splits` equal slices, one batched GEMM writes the slices'
 * products to the workspace (splits x M x N fp32) and a second pass adds
 * them in slice order into C (deterministic).  K % splits == 0; N and c_ms
 * multiples of 4; C and workspace 16-byte aligned; beta 0 (C overwritten).
 * splits == 1 is a plain mk_gemm_blas call (no workspace). */
size_t mk_gemm_blas_splitk_workspace_bytes(int64_t M, int64_t N, int64_t splits);
int mk_gemm_blas_splitk(void* stream, int ab_type, int64_t M, int64_t N, int64_t K, const void* A,
                        int64_t a_ms, int64_t a_ks, const void* B, int64_t b_ks, int64_t b_ns, float* C,
                        int64_t c_ms, int64_t splits, void* workspace);

/* ------------------------------------------------------------------------
 * a5+a6  fused scaled-dot-product attention (flash attention, forward).
 * Replaces the unfused chain the reference emits for the jnp attention
 * pattern: linalg.mm:98 (Q·Kᵀ) → elementwise.mm:87 (softMaxWithTensor,
 * matched by TrySoftmax elementwise.mm:71-89) → linalg.mm:98 (P·V), with the
 * causal mask built by shape.mm:249-256 (iota), binary.mm:84-109 (compare)
 * and binary.mm:77-82 (select).  The [S,S] score matrix never exists.
 *
 * O[b,h,i,:] = softmax_j( scale * Q[b,h,i,:]·K[b,h,j,:] , j ≤ i if causal ) · V[b,h,j,:]
 * (causal = jnp.tril of the [Sq, Sk] score matrix, top-left aligned; a row
 * with no visible key yields NaN, as softmax over all -inf does).
 * Tensors are bf16 with D contiguous; the other strides are in elements:
 *   X element (b,h,s,d) at X + b*x_bs + h*x_hs + s*x_ss + d.
 * D ∈ {64, 128}; k_ss, v_ss in [D, 2^24) (any stride when the length is 1).
 * Scores, running max and accumulation in fp32; the probabilities are
 * rounded to bf16 (as XLA's bf16 softmax rounds exp) and the row sum adds
 * those rounded values, so O = Σ bf16(p)·V / Σ bf16(p).
 * lse (optional, may be NULL): fp32 [B,H,Sq] row log-sum-exp (natural log) of
 * the scaled, masked scores, written densely: log of that same row sum plus
 * the row max (within 2^-8 of the exact value).
 * ---------------------------------------------------------------------- */
int mk_sdpa_fwd(void* stream, int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D,
                const void* q, int64_t q_bs, int64_t q_hs, int64_t q_ss,
                const void* k, int64_t k_bs, int64_t k_hs, int64_t k_ss,
                const void* v, int64_t v_bs, int64_t v_hs, int64_t v_ss,
                void* o, int64_t o_bs, int64_t o_hs, int64_t o_ss,
                float scale, int causal, float* lse);

/* ------------------------------------------------------------------------
 * a8  row reduction over the innermost (contiguous) axis.
 * Replaces: src/jam/ops/reduce.mm:97-106 (reductionSum/Max/Min/Product).
 * y[r] = op_{c<cols} x[r*cols + c]; in_type ∈ {MK_BF16, MK_F16, MK_F32},
 * out_type ∈ {MK_F32, MK_BF16, MK_F16}; fp32 accumulation.
 * op: 0 sum, 1 max, 2 min, 3 product.  init is folded in (StableHLO reduce
 * init operand; the reference ignores it, reduce.mm:79-108).
 * ---------------------------------------------------------------------- */
int mk_row_reduce(void* stream, int in_type, int out_type, int op,
                  int64_t rows, int64_t cols, const void* x, float init, void* y);

/* ------------------------------------------------------------------------
 * a9  fused row max + argmax / min + argmin (bit-exact).
 * Replaces: src/jam/ops/reduce.mm:29-43 (DetectArgReduce) and 61-66
 * (reductionMaximum + reductionArgMaximum).  Semantics are XLA's variadic
 * reduce as emitted by jnp.argmax: larger value wins (smaller for argmin),
 * NaN beats every number, ties go to the lower index.
 * in_type ∈ {MK_BF16, MK_F16, MK_F32}; values (same dtype as x) may be NULL;
 * index_type ∈ {MK_S32, MK_S64}.
 * ---------------------------------------------------------------------- */
int mk_row_argmax(void* stream, int in_type, int is_min, int64_t rows, int64_t cols,
                  const void* x, void* values, int index_type, void* indices);

/* ------------------------------------------------------------------------
 * a7+a8  fused LayerNorm over the innermost axis (one HBM pass).
 * Replaces the reduce(reduce.mm:97-106) + elementwise(elementwise.mm:91-171)
 * chain of the "LayerNorm" composition validated in docs/ops.md:79.
 * y = (x - mean) * rsqrt(var + eps) * gamma + beta, stats in fp32 (two-pass
 * in registers), x/gamma/beta/y of io_type ∈ {MK_BF16, MK_F32}.
 * gamma / beta may be NULL (treated as 1 / 0).
 * ---------------------------------------------------------------------- */
int mk_layernorm(void* stream, int io_type, int64_t rows, int64_t cols,
                 const void* x, const void* gamma, const void* beta, float eps, void* y);

/* mk_layernorm with the stored type separate from the input's: x, gamma,
 * beta of in_type, y of out_type, (in, out) ∈ {(bf16, bf16), (f32, f32),
 * (f32, bf16)}.  (f32, bf16) is the LayerNorm of an fp32 residual stream
 * whose result only feeds a bf16 matrix product (the convert that
 * reduce.mm / elementwise.mm would run as its own node folded into the
 * store: one rounding of the fp32 result). */
int mk_layernorm_typed(void* stream, int in_type, int out_type, int64_t rows, int64_t cols, const void* x,
                       const void* gamma, const void* beta, float eps, void* y);

/* ------------------------------------------------------------------------
 * a7  fused GELU (tanh approximation), fp32 math, one rounding on store.
 * Replaces the multiply/add/tanh chain of elementwise.mm:91-171 for the
 * "GELU-tanh" composition (docs/ops.md:79).
 * y = 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))); io_type ∈ {MK_BF16, MK_F32}.
 * ---------------------------------------------------------------------- */
int mk_gelu_tanh(void* stream, int io_type, int64_t n, const void* x, void* y);

/* ------------------------------------------------------------------------
 * a7  generic fused elementwise program (register-resident interpreter).
 * Replaces one MPSGraph node per elementwise op (elementwise.mm:91-171,
 * binary.mm:65-109, shape.mm:270-293 convert, structural.mm:87-96 broadcast)
 * with ONE launch per fused chain.  Every element of the output shape runs
 * the same straight-line program over fp32 registers.
 *
 * Shapes: the output has `rank` ≤ 6 dims (`dims`); input t is addressed with
 * element strides in_strides[t*6 + d] (0 for broadcast dims) — so
 * broadcast_in_dim / transpose feeding the chain are folded into addressing.
 * Program: n_instr instructions of 4 int32 {opcode, dst, a, b} plus a third
 * operand for select/clamp packed in the high 16 bits of `b` (see
 * mk_ew_op).  Registers 0..n_inputs-1 are preloaded with the inputs: float
 * types widen to fp32, integer types are held as their int32 bit pattern
 * (sign- or zero-extended; 64-bit truncated), predicates as 0.0f / 1.0f.
 * Stores convert back the same way.  Constants come from `consts` (32-bit
 * patterns, read as fp32) via MK_EW_CONST.  Register `out_reg` is stored, converted
 * to out_type.  At most 32 registers, 64 instructions, 8 inputs.
 * ---------------------------------------------------------------------- */
typedef enum mk_ew_op {
  MK_EW_CONST = 0,  /* r[dst] = consts[a]                       */
  MK_EW_ADD, MK_EW_SUB, MK_EW_MUL, MK_EW_DIV, MK_EW_MAX, MK_EW_MIN, MK_EW_POW,
  MK_EW_NEG, MK_EW_EXP, MK_EW_LOG, MK_EW_TANH, MK_EW_SQRT, MK_EW_RSQRT, MK_EW_ABS,
  MK_EW_LOGISTIC,
  MK_EW_CMP_EQ, MK_EW_CMP_NE, MK_EW_CMP_LT, MK_EW_CMP_LE, MK_EW_CMP_GT, MK_EW_CMP_GE,
  MK_EW_SELECT,     /* r[dst] = r[a] != 0 ? r[b & 0xffff] : r[b >> 16]          */
  MK_EW_CLAMP,      /* r[dst] = min(max(r[b & 0xffff], r[a]), r[b >> 16])       */
  MK_EW_ROUND_BF16, /* r[dst] = fp32(bf16_rne(r[a])) — per-op bf16 rounding    */
  MK_EW_ROUND_F16,  /* r[dst] = fp32(f16_rne(r[a]))                            */
  MK_EW_FLOOR, MK_EW_CEIL, MK_EW_SIGN,
  MK_EW_AND, MK_EW_OR, MK_EW_NOT,   /* on 0/1 predicates                        */
  MK_EW_MOV,
  MK_EW_CMP_LT_S32, MK_EW_CMP_GE_S32, /* integer compares on raw int32 bits    */
  MK_EW_ADD_S32, MK_EW_SUB_S32, MK_EW_MUL_S32,
  MK_EW_S32_TO_F32, MK_EW_F32_TO_S32,  /* C-style truncation toward zero        */
  MK_EW_ERF,
  MK_EW_CMP_EQ_S32, MK_EW_CMP_NE_S32, MK_EW_CMP_LE_S32, MK_EW_CMP_GT_S32,
  MK_EW_MAX_S32, MK_EW_MIN_S32, MK_EW_NEG_S32,
  MK_EW_AND_B32, MK_EW_OR_B32, MK_EW_XOR_B32, /* bitwise on raw 32-bit patterns */
  MK_EW_PRED_TO_S32,                   /* 0/1 predicate -> int32 0/1            */
  MK_EW_S32_TO_PRED,                   /* int32 != 0 -> predicate               */
  MK_EW_U32_TO_F32,
  MK_EW_NUM_OPS
} mk_ew_op;

int mk_ew_program(void* stream, int rank, const int64_t* dims,
                  int n_inputs, const void* const* inputs, const int* in_types,
                  const int64_t* in_strides,
                  int n_instr, const int32_t* program, const float* consts, int n_consts,
                  int out_reg, int out_type, void* out);

/* mk_ew_program with 1 to 4 outputs of the same shape, each dense row-major:
 * register out_regs[k] is stored to outs[k] as out_types[k].  Every input
 * element is loaded before any output element is stored, so an output may
 * be the memory of an input read at the same index (in place).  The sibling
 * outputs of one fused chain (an optimizer's new parameter and moments, or
 * values a backward pass keeps) take one launch that reads the shared
 * inputs once, instead of one launch per output. */
int mk_ew_program_multi(void* stream, int rank, const int64_t* dims,
                        int n_inputs, const void* const* inputs, const int* in_types,
                        const int64_t* in_strides,
                        int n_instr, const int32_t* program, const float* consts, int n_consts,
                        int n_outputs, const int* out_regs, const int* out_types, void* const* outs);

/* ------------------------------------------------------------------------
 * a10  row gather (embedding lookup), bit-exact copy.
 * Replaces: src/jam/ops/gather_scatter.mm:185-196 (gatherWithUpdatesTensor
 * axis:0) including the index clamp to [0, n_rows-1] at 180-183.
 * out[i, :] = table[clamp(ids[i], 0, n_rows-1), :]; row_bytes % 4 == 0.
 * ids: int32 (index_type MK_S32) or int64 (MK_S64).
 * ---------------------------------------------------------------------- */
int mk_gather_rows(void* stream, int64_t n_rows, int64_t row_bytes, const void* table,
                   int index_type, int64_t n_ids, const void* ids, void* out);

/* ------------------------------------------------------------------------
 * a11  deterministic scatter-add of rows (bit-exact vs in-order fp32).
 * Replaces: src/jam/ops/gather_scatter.mm:322-327 (scatterNDWithDataTensor
 * mode:Add), whose GPU accumulation order is unspecified.
 * out[r, :] = table[r, :] + sum over i with ids[i]==r, in increasing i, of
 *             updates[i, :]   (fp32 adds applied sequentially in that order)
 * ids outside [0, n_rows) are dropped (StableHLO scatter semantics, JAX's
 * FILL_OR_DROP mode).  table and out may alias (in-place).  dtype ∈ {MK_F32,
 * MK_BF16}: bf16 rounds after every add, exactly as a sequential bf16 scatter.
 * workspace: device memory of mk_scatter_add_workspace_bytes(n_rows, n_ids).
 * ---------------------------------------------------------------------- */
size_t mk_scatter_add_workspace_bytes(int64_t n_rows, int64_t n_ids);
int mk_scatter_add_rows(void* stream, int dtype, int64_t n_rows, int64_t row_len,
                        const void* table, int index_type, int64_t n_ids, const void* ids,
                        const void* updates, void* out, void* workspace);

/* ------------------------------------------------------------------------
 * a11  scatter-add that allocates nothing.  No counterpart in the reference:
 * it exists for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same contract and same kernels as mk_scatter_add_rows, but the workspace
 * is a fixed device array of the library, MK_SCATTER_ADD_SCRATCH_BYTES per
 * GPU, held until the process ends.  Calls whose
 * mk_scatter_add_workspace_bytes(n_rows, n_ids) exceeds it fail with
 * MK_ERR_UNSUPPORTED (C4's 65536 ids into 50257 rows need about 1.5 MB).
 * Every call on a GPU shares that GPU's array: calls that overlap on one GPU
 * (other streams, other threads) race and must be serialised by the caller.
 * ---------------------------------------------------------------------- */
#define MK_SCATTER_ADD_SCRATCH_BYTES (8u << 20)
int mk_scatter_add_rows_noalloc(void* stream, int dtype, int64_t n_rows, int64_t row_len,
                                const void* table, int index_type, int64_t n_ids, const void* ids,
                                const void* updates, void* out);

/* ------------------------------------------------------------------------
 * a6  iota.  Replaces src/jam/ops/shape.mm:249-256 (coordinateAlongAxis +
 * castTensor).  out[idx] = idx[dim] for every index of the row-major shape.
 * out_type ∈ {MK_S32, MK_S64, MK_F32, MK_BF16, MK_U32}.
 * ---------------------------------------------------------------------- */
int mk_iota(void* stream, int out_type, int rank, const int64_t* dims, int dim, void* out);

/* ------------------------------------------------------------------------
 * a12  strided copy (transpose / broadcast / slice materialisation).
 * Replaces shape.mm:28-40 (transposeTensor), shape.mm:163-172 and
 * structural.mm:87-96 (broadcastTensor) when the consumer cannot fold the
 * layout into its own addressing.  out is dense row-major over `dims`;
 * in element (i0..ir) at in + sum_d i_d * in_strides[d] (elements, may be 0).
 * elem_bytes ∈ {1, 2, 4, 8}; rank ≤ 6.
 * ---------------------------------------------------------------------- */
int mk_copy_strided(void* stream, int elem_bytes, int rank, const int64_t* dims,
                    const void* in, const int64_t* in_strides, void* out);

/* ------------------------------------------------------------------------
 * a5  standalone row softmax (fallback when the SDPA pattern does not match).
 * Replaces src/jam/ops/elementwise.mm:87 (softMaxWithTensor).
 * y[r,:] = softmax(x[r,:]); io_type ∈ {MK_BF16, MK_F32}; fp32 math.
 * ---------------------------------------------------------------------- */
int mk_softmax_rows(void* stream, int io_type, int64_t rows, int64_t cols,
                    const void* x, void* y);

/* ------------------------------------------------------------------------
 * dtype conversion (a7 `convert`, shape.mm:270-293), element-wise, dense.
 * Float→int truncates toward zero; unsigned sources convert as unsigned
 * (the unsigned fix-up of shape.mm:280-291); float→bf16/f16 is RNE.
 * ---------------------------------------------------------------------- */
int mk_convert(void* stream, int in_type, int out_type, int64_t n, const void* in, void* out);

/* Fill n elements of elem_bytes (1,2,4,8) with the bit pattern `pattern`
 * (a kernel, so it is safe inside captured HIP graphs). */
int mk_fill(void* stream, int elem_bytes, int64_t n, uint64_t pattern, void* out);

/* ========================================================================
 * Backward and optimizer kernels of the one-GPU training step (config C5:
 * the jitted value_and_grad + Adam step of temp/dp_train.py:67-76 on a
 * GPT-2-small decoder).  In the reference these ops reach MPSGraph through
 * the same handlers as the forward (dot_general linalg.mm:47-105, reduce
 * reduce.mm:79-108, elementwise elementwise.mm:91-171, scatter
 * gather_scatter.mm:262-335) applied to the StableHLO that jax.grad emits;
 * here each backward composition is one entry point.
 * ====================================================================== */

/* out[r, c] = a[r, c] + b[r, c] + bias[c] over a dense [rows, cols] array,
 * fp32 math and one rounding (b and / or bias may be NULL; out may alias a
 * or b).  The residual and bias adds of the step: the broadcast add of a
 * bias (structural.mm:87-96 broadcast feeding elementwise.mm add) and the
 * residual add, folded into one pass.  io_type ∈ {MK_BF16, MK_F32}. */
int mk_add_rows(void* stream, int io_type, int64_t rows, int64_t cols, const void* a, const void* b,
                const void* bias, void* out);

/* Residual add and LayerNorm in one pass, bf16 rows:
 *   sum = a + b + bias[c]      (fp32 adds, one RNE rounding; as mk_add_rows)
 *   y   = (sum - mean) rstd gamma + beta over each row of the rounded sum
 *         (two-pass mean / variance, as mk_layernorm)
 * The pre-LN block's `x + proj(h) + bias` feeding the next LayerNorm
 * (elementwise.mm add, then the LayerNorm pattern of reduce.mm:79-108),
 * both results stored (the sum is the residual stream the backward reads).
 * b, bias, gamma (1), beta (0) may be NULL; cols % 4 == 0, cols <= 2048;
 * 8-byte aligned operands. */
int mk_add_layernorm(void* stream, int64_t rows, int64_t cols, const void* a, const void* b,
                     const void* bias, const void* gamma, const void* beta, float eps, void* sum_out,
                     void* y);

/* mk_add_layernorm with input and output types: (bf16, bf16) is
 * mk_add_layernorm; for fp32 rows (a, b, gamma, beta, sum_out fp32, y fp32
 * or bf16) sum = a + b (one fp32 add, no bias: b already holds it) is stored
 * and normalised as mk_layernorm_typed normalises a row -- the residual
 * update of a pre-LN block in an fp32 module, then the next LayerNorm whose
 * result feeds a bf16 product. */
int mk_add_layernorm_typed(void* stream, int in_type, int out_type, int64_t rows, int64_t cols, const void* a,
                           const void* b, const void* bias, const void* gamma, const void* beta, float eps,
                           void* sum_out, void* y);

/* pre = x + bias[c] (bf16, one rounding) and y = gelu_tanh(pre) (as
 * mk_gelu_tanh on the stored pre) in one pass: the MLP's bias add and
 * activation (elementwise.mm add + the GELU chain).  pre may alias x. */
int mk_bias_gelu(void* stream, int64_t rows, int64_t cols, const void* x, const void* bias, void* pre_out,
                 void* y);

/* dx = dy * gelu_tanh'(x), gelu_tanh as mk_gelu_tanh; fp32 math, one rounding
 * on store.  io_type ∈ {MK_BF16, MK_F32}.  dx may alias dy. */
int mk_gelu_tanh_bwd(void* stream, int io_type, int64_t n, const void* x, const void* dy, void* dx);

/* y[c] = sum_r x[r, c] (fp32 out, fp32 accumulation) — bias gradients, the
 * reduce over the batch axis that jax.grad emits for a broadcast bias add
 * (reduce.mm:97-106 over axis 0).  Deterministic: per-block partial rows in
 * the workspace, then added in block order.  in_type ∈ {MK_BF16, MK_F32}. */
size_t mk_col_sum_workspace_bytes(int64_t rows, int64_t cols);
int mk_col_sum(void* stream, int in_type, int64_t rows, int64_t cols, const void* x, float* y,
               void* workspace);

/* mk_gelu_tanh_bwd over a dense [rows, cols] array fused with mk_col_sum of
 * its output: dx = dy * gelu_tanh'(x) and dx_colsum[c] = sum_r dx[r, c] (the
 * MLP bias gradient) in one pass over x and dy.  Workspace as mk_col_sum's;
 * dx may alias dy. */
int mk_gelu_tanh_bwd_colsum(void* stream, int io_type, int64_t rows, int64_t cols, const void* x,
                            const void* dy, void* dx, float* dx_colsum, void* workspace);

/* LayerNorm backward for y = (x - mean) rstd gamma + beta over rows of `cols`
 * (mean / rstd recomputed from x as mk_layernorm computes them):
 *   dx = rstd (g - mean(g) - xh mean(g xh)) + dres,  g = dy gamma, xh = (x - mean) rstd
 *   dgamma = sum_rows dy xh,  dbeta = sum_rows dy,  dx_colsum = sum_rows dx
 * (fp32, deterministic).  dres (may be NULL; may alias dx) is the residual
 * branch's gradient, so the pre-LN block's dx = dres + LN'(dy) is one pass;
 * dx_colsum (may be NULL) is the bias gradient of the preceding projection.
 * io_type ∈ {MK_BF16, MK_F32} for x, gamma, dy, dres, dx; cols ≤ 2048; gamma
 * may be NULL (1); dgamma / dbeta both NULL skips them; the workspace is
 * needed when dgamma or dx_colsum is given. */
size_t mk_layernorm_bwd_workspace_bytes(int64_t rows, int64_t cols);
int mk_layernorm_bwd(void* stream, int io_type, int64_t rows, int64_t cols, const void* x,
                     const void* gamma, const void* dy, const void* dres, float eps, void* dx,
                     float* dgamma, float* dbeta, float* dx_colsum, void* workspace);

/* mk_layernorm_bwd that also stores dx_bf16 (may be NULL; fp32 rows only):
 * the bf16 rounding (RNE) of each dx element, the operand of the bf16
 * products that read this gradient next (the convert node of the
 * reference's graph folded into the same pass). */
int mk_layernorm_bwd_typed(void* stream, int io_type, int64_t rows, int64_t cols, const void* x,
                           const void* gamma, const void* dy, const void* dres, float eps, void* dx,
                           void* dx_bf16, float* dgamma, float* dbeta, float* dx_colsum, void* workspace);

/* Softmax cross-entropy over rows of logits, loss and gradient together:
 *   lse_r = log sum_j exp(x[r, j]);  loss_rows[r] = lse_r - x[r, labels[r]]
 *   dlogits[r, j] = (exp(x[r, j] - lse_r) - [j == labels[r]]) * grad_scale
 * (grad_scale = 1/rows gives the gradient of the mean loss, as
 * optax.softmax_cross_entropy_with_integer_labels(...).mean() under jax.grad).
 * io_type ∈ {MK_BF16, MK_F32} for logits / dlogits (dlogits may alias logits);
 * label_type ∈ {MK_S32, MK_S64}.  A label outside [0, cols) has no target
 * term: loss_rows[r] = lse_r and dlogits = softmax * grad_scale, which is what
 * the one-hot form sum(select(iota == label, x, 0)) computes for it.
 * loss_rows (fp32 [rows]) may be NULL. */
int mk_softmax_xent(void* stream, int io_type, int64_t rows, int64_t cols, const void* logits,
                    int label_type, const void* labels, float grad_scale, float* loss_rows,
                    void* dlogits);

/* mk_softmax_xent with fp32 logits and bf16 dlogits (logits_type MK_F32,
 * dlogits_type MK_BF16; equal types are mk_softmax_xent):
 * the gradient of a jitted step whose only readers are bf16 products, so
 * the fp32 gradient and its conversion are never written.  Same loss and
 * label rules; dlogits is rounded to bf16 once. */
int mk_softmax_xent_typed(void* stream, int logits_type, int dlogits_type, int64_t rows, int64_t cols,
                          const void* logits, int label_type, const void* labels, float grad_scale,
                          float* loss_rows, void* dlogits);

/* mk_softmax_xent_typed over rows `ld_logits` / `ld_dlogits` elements apart
 * (each >= cols; only the first cols elements of a row are read or written):
 * a vocabulary of 50257 classes kept in rows padded to 16-byte multiples, so
 * that the products reading the gradient take aligned operand rows.  Type
 * pairs bf16/bf16, f32/f32 (dlogits may alias logits when the pitches are
 * equal) and f32/bf16; same loss, gradient and label rules.
 * Replaces, for the fused loss of a jitted step: src/jam/ops/elementwise.mm:71-89
 * (the softmax of the logits and its gradient through the one-hot select). */
int mk_softmax_xent_strided(void* stream, int logits_type, int dlogits_type, int64_t rows, int64_t cols,
                            const void* logits, int64_t ld_logits, int label_type, const void* labels,
                            float grad_scale, float* loss_rows, void* dlogits, int64_t ld_dlogits);

/* One Adam step, the update of temp/dp_train.py:71-75:
 *   m = b1 m + (1-b1) g;  v = b2 v + (1-b2) g^2
 *   p = p - lr (m / bc1) / (sqrt(v / bc2) + eps)       (bc1 = 1-b1^t, bc2 = 1-b2^t)
 * computed in fp32; the hyperparameters come in as doubles and b1, 1-b1, b2,
 * 1-b2, eps, lr, bc1, bc2 are each rounded once to fp32 (how JAX folds the
 * Python-float constants of that loop).  With `master` (fp32) the update runs
 * on the master copy and the bf16 param receives its RNE rounding
 * (param_type MK_BF16); with master NULL the param is fp32 and updated in
 * place.  grad_type ∈ {MK_F32, MK_BF16}; m, v fp32; all arrays n elements. */
int mk_adam_update(void* stream, int64_t n, int param_type, void* param, float* master, int grad_type,
                   const void* grad, float* m, float* v, double lr, double b1, double b2, double eps,
                   double bc1, double bc2);

/* mk_adam_update with lr, bc1, bc2 read from device memory, hyper = {lr, bc1,
 * bc2} (fp32): the step's scalar inputs of temp/dp_train.py:93-95 (host
 * computed, passed as replicated f32 device scalars), so a captured launch
 * sequence takes new values on every replay. */
int mk_adam_update_dev(void* stream, int64_t n, int param_type, void* param, float* master, int grad_type,
                       const void* grad, float* m, float* v, const float* hyper, double b1, double b2,
                       double eps);

/* Attention backward for O = softmax(scale Q Kᵀ [causal]) V (mk_sdpa_fwd's
 * convention, lse from its forward): with P = exp(scale S - lse) (0 where
 * masked), D_r = dO_r · O_r and dS = scale P (dO Vᵀ - D):
 *   dV = Pᵀ dO,  dQ = dS K,  dK = dSᵀ Q     (bf16 out, fp32 accumulation)
 * — the transposed dot_generals, select and reduce that jax.grad emits for
 * the attention pattern.  D ∈ {64, 128}: flash style on MFMA kernels, P and
 * dS recomputed per tile from lse, nothing Sq x Sk in memory, deterministic
 * (no atomics); the workspace holds D_r and lse per row (B H Sq 8 bytes,
 * rounded up to 64-row tiles); q/k/v/o/dout rows 16-byte aligned, dq/dk/dv
 * strides multiples of 4.  Other D (a multiple of 8, ≤ 256): S, dP (fp32)
 * and P, dS (bf16) materialised for all heads in the workspace, products on
 * the rocBLAS GEMM of mk_gemm_blas; o and dout rows 16-byte aligned.
 * Strides as mk_sdpa_fwd (elements, D contiguous). */
size_t mk_sdpa_bwd_workspace_bytes(int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D);
int mk_sdpa_bwd(void* stream, int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D,
                const void* q, int64_t q_bs, int64_t q_hs, int64_t q_ss,
                const void* k, int64_t k_bs, int64_t k_hs, int64_t k_ss,
                const void* v, int64_t v_bs, int64_t v_hs, int64_t v_ss,
                const void* o, int64_t o_bs, int64_t o_hs, int64_t o_ss,
                const void* dout, int64_t do_bs, int64_t do_hs, int64_t do_ss,
                const float* lse,
                void* dq, int64_t dq_bs, int64_t dq_hs, int64_t dq_ss,
                void* dk, int64_t dk_bs, int64_t dk_hs, int64_t dk_ss,
                void* dv, int64_t dv_bs, int64_t dv_hs, int64_t dv_ss,
                float scale, int causal, void* workspace);

#ifdef __cplusplus
}
#endif

#endif /* MI355X_MK_KERNELS_H_ */
