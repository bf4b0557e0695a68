// Plain (unfused) GEMMs through rocBLAS: the linear layers of the training
// step and their gradients, which have no epilogue worth fusing.  The
// row-major, element-strided operand convention of mk_gemm is mapped onto
// rocBLAS's column-major gemm: C[M,N] = A[M,K] B[K,N] is the column-major
// product C^T[N,M] = B^T[N,K] A^T[K,M], and each operand is passed as stored
// (no copies), transposed where its unit stride says so.
#include "mk_common.h"

#include <rocblas/rocblas.h>

#include <algorithm>
#include <mutex>
#include <vector>

namespace mk {
namespace {

std::mutex g_blas_mu;
std::vector<rocblas_handle> g_handles;  // one per device, kept for the process

rocblas_handle handle_for_current_device(int* err) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    *err = fail(MK_ERR_LAUNCH, "mk_gemm_blas: hipGetDevice failed");
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(g_blas_mu);
  if (int(g_handles.size()) <= dev) g_handles.resize(dev + 1, nullptr);
  if (!g_handles[dev]) {
    rocblas_handle h = nullptr;
    if (rocblas_create_handle(&h) != rocblas_status_success) {
      *err = fail(MK_ERR_LAUNCH, "mk_gemm_blas: rocblas_create_handle failed");
      return nullptr;
    }
    rocblas_set_pointer_mode(h, rocblas_pointer_mode_host);
    g_handles[dev] = h;
  }
  return g_handles[dev];
}

bool blas_type(int t, rocblas_datatype* out) {
  if (t == MK_BF16) *out = rocblas_datatype_bf16_r;
  else if (t == MK_F32) *out = rocblas_datatype_f32_r;
  else if (t == MK_F16) *out = rocblas_datatype_f16_r;
  else return false;
  return true;
}

}  // namespace

// shared with the attention backward (train.hip)
int gemm_blas(hipStream_t stream, int ab_type, int c_type, int64_t batch, int64_t M, int64_t N, int64_t K,
              const void* A, int64_t a_bs, int64_t a_ms, int64_t a_ks, const void* B, int64_t b_bs, int64_t b_ks,
              int64_t b_ns, void* C, int64_t c_bs, int64_t c_ms, float alpha, float beta) {
  if (batch < 0 || M < 0 || N < 0 || K < 0) return fail(MK_ERR_INVALID, "mk_gemm_blas: negative shape");
  if (batch == 0 || M == 0 || N == 0) return MK_OK;
  if (!A || !B || !C) return fail(MK_ERR_INVALID, "mk_gemm_blas: null pointer");
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX || batch > INT32_MAX)
    return fail(MK_ERR_UNSUPPORTED, "mk_gemm_blas: dimensions beyond int32");
  rocblas_datatype ab, ct;
  if (!blas_type(ab_type, &ab) || !blas_type(c_type, &ct) || ab_type == MK_F16 ||
      (ab_type == MK_F32 && c_type != MK_F32))
    return fail(MK_ERR_UNSUPPORTED, "mk_gemm_blas: operands bf16 (out bf16/f16/f32) or f32 (out f32)");
  // rocBLAS "A" = our Bᵀ as an N x K column-major matrix
  rocblas_operation op_a;
  int64_t lda;
  if (b_ns == 1) { op_a = rocblas_operation_none; lda = b_ks; }
  else if (b_ks == 1) { op_a = rocblas_operation_transpose; lda = b_ns; }
  else return fail(MK_ERR_UNSUPPORTED, "mk_gemm_blas: B needs a unit stride along k or n");
  // rocBLAS "B" = our Aᵀ as a K x M column-major matrix
  rocblas_operation op_b;
  int64_t ldb;
  if (a_ks == 1) { op_b = rocblas_operation_none; ldb = a_ms; }
  else if (a_ms == 1) { op_b = rocblas_operation_transpose; ldb = a_ks; }
  else return fail(MK_ERR_UNSUPPORTED, "mk_gemm_blas: A needs a unit stride along m or k");
  // a stored matrix's leading dimension must cover its rows; where it has a
  // single column the stride is never used and is set to the row count
  auto fix_ld = [](int64_t& ld, int64_t rows, int64_t cols) {
    if (cols == 1 && ld < rows) ld = rows;
    return ld >= rows;
  };
  int64_t ldc = c_ms;
  if (!fix_ld(lda, op_a == rocblas_operation_none ? N : K, op_a == rocblas_operation_none ? K : N) ||
      !fix_ld(ldb, op_b == rocblas_operation_none ? K : M, op_b == rocblas_operation_none ? M : K) ||
      !fix_ld(ldc, N, M))
    return fail(MK_ERR_UNSUPPORTED, "mk_gemm_blas: overlapping rows (leading stride below the row length)");
  if (lda > INT32_MAX || ldb > INT32_MAX || ldc > INT32_MAX)
    return fail(MK_ERR_UNSUPPORTED, "mk_gemm_blas: leading dimension beyond int32");
  int err = MK_OK;
  rocblas_handle h = handle_for_current_device(&err);
  if (!h) return err;
  // a device's handle is shared: binding the stream and queueing the GEMM
  // happen under one lock, so concurrent callers cannot swap streams between
  std::lock_guard<std::mutex> lk(g_blas_mu);
  if (rocblas_set_stream(h, stream) != rocblas_status_success)
    return fail(MK_ERR_LAUNCH, "mk_gemm_blas: rocblas_set_stream failed");
  const rocblas_status st = rocblas_gemm_strided_batched_ex(
      h, op_a, op_b, rocblas_int(N), rocblas_int(M), rocblas_int(K), &alpha, B, ab, rocblas_int(lda), b_bs, A, ab,
      rocblas_int(ldb), a_bs, &beta, C, ct, rocblas_int(ldc), c_bs, C, ct, rocblas_int(ldc), c_bs,
      rocblas_int(batch), rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
  if (st != rocblas_status_success)
    return fail(MK_ERR_LAUNCH, std::string("mk_gemm_blas: rocblas_gemm_strided_batched_ex: ") +
                                   rocblas_status_to_string(st));
  return MK_OK;
}

namespace {
// C[m, n] = sum over slices s of W[s][m][n] (dense M x N slices), slices added
// in order: the result does not depend on scheduling.
// S > 0: the slice count is a compile-time constant, so a vector's S loads
// are issued together (with a runtime count each load is waited for before
// the next); S == 0: any count.  Same order of adds either way.
template <int S, bool BF16>
__global__ __launch_bounds__(256) void splitk_sum_kernel(const float* __restrict__ w, int64_t splits, int64_t M,
                                                        int64_t N, void* __restrict__ c, int64_t c_ms,
                                                        const void* __restrict__ bias, int epilogue) {
  const int64_t nvec = M * N / 4, slab = M * N / 4;
  const int64_t stride = int64_t(gridDim.x) * 256;
  const f32x4* wv = reinterpret_cast<const f32x4*>(w);
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < nvec; i += stride) {
    f32x4 a;
    if constexpr (S > 0) {
      f32x4 b[S];
#pragma unroll
      for (int s = 0; s < S; ++s) b[s] = wv[s * slab + i];
      a = b[0];
#pragma unroll
      for (int s = 1; s < S; ++s)
#pragma unroll
        for (int j = 0; j < 4; ++j) a.v[j] += b[s].v[j];
    } else {
      a = wv[i];
      for (int64_t s = 1; s < splits; ++s) {
        const f32x4 b = wv[s * slab + i];
#pragma unroll
        for (int j = 0; j < 4; ++j) a.v[j] += b.v[j];
      }
    }
    const int64_t e = i * 4, m = e / N, n = e % N;
    if (epilogue != 0) {
      const bool bias16 = BF16 && (epilogue & 4) == 0;  // | 4: an fp32 bias with bf16 C
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        a.v[j] += bias16 ? bf16_to_f32(static_cast<const uint16_t*>(bias)[n + j]) : static_cast<const float*>(bias)[n + j];
        if ((epilogue & 3) == 2) a.v[j] = fmaxf(a.v[j], 0.f);
      }
    }
    if constexpr (BF16)
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(c) + m * c_ms + n) =
          uint2{f32_to_bf16(a.v[0]) | (uint32_t(f32_to_bf16(a.v[1])) << 16),
                f32_to_bf16(a.v[2]) | (uint32_t(f32_to_bf16(a.v[3])) << 16)};
    else
      *reinterpret_cast<f32x4*>(static_cast<float*>(c) + m * c_ms + n) = a;
  }
}

template <bool BF16>
void splitk_sum_launch(hipStream_t s, const float* W, int64_t splits, int64_t M, int64_t N, void* C, int64_t c_ms,
                       unsigned blocks, const void* bias, int epi) {
  const dim3 g(blocks), b(256);
  if (splits == 2) hipLaunchKernelGGL((splitk_sum_kernel<2, BF16>), g, b, 0, s, W, splits, M, N, C, c_ms, bias, epi);
  else if (splits == 4) hipLaunchKernelGGL((splitk_sum_kernel<4, BF16>), g, b, 0, s, W, splits, M, N, C, c_ms, bias, epi);
  else if (splits == 8) hipLaunchKernelGGL((splitk_sum_kernel<8, BF16>), g, b, 0, s, W, splits, M, N, C, c_ms, bias, epi);
  else hipLaunchKernelGGL((splitk_sum_kernel<0, BF16>), g, b, 0, s, W, splits, M, N, C, c_ms, bias, epi);
}
}  // namespace

int splitk_sum(hipStream_t s, const float* W, int64_t splits, int64_t M, int64_t N, void* C, int64_t c_ms,
               const char* what, int c_type, const void* bias, int epilogue) {
  const int64_t nvec = M * N / 4;
  const unsigned blocks = unsigned(std::min<int64_t>((nvec + 255) / 256, 4096));
  if (c_type == MK_BF16) splitk_sum_launch<true>(s, W, splits, M, N, C, c_ms, blocks, bias, epilogue);
  else splitk_sum_launch<false>(s, W, splits, M, N, C, c_ms, blocks, bias, epilogue);
  return check_launch(what);
}

}  // namespace mk

extern "C" size_t mk_gemm_blas_splitk_workspace_bytes(int64_t M, int64_t N, int64_t splits) {
  if (M <= 0 || N <= 0 || splits <= 1) return 0;
  return size_t(M * N * splits * 4);
}

extern "C" int mk_gemm_blas_splitk(void* stream, int ab_type, int64_t M, int64_t N, int64_t K, const void* A,
                                   int64_t a_ms, int64_t a_ks, const void* B, int64_t b_ks, int64_t b_ns, float* C,
                                   int64_t c_ms, int64_t splits, void* workspace) {
  mk::clear_error();
  if (splits < 1 || K < 0 || M < 0 || N < 0) return mk::fail(MK_ERR_INVALID, "mk_gemm_blas_splitk: bad shape or splits");
  hipStream_t s = mk::as_stream(stream);
  if (splits == 1 || M == 0 || N == 0)
    return mk::gemm_blas(s, ab_type, MK_F32, 1, M, N, K, A, 0, a_ms, a_ks, B, 0, b_ks, b_ns, C, 0, c_ms, 1.f, 0.f);
  if (K % splits != 0) return mk::fail(MK_ERR_UNSUPPORTED, "mk_gemm_blas_splitk: K must be a multiple of splits");
  if (!workspace || !C) return mk::fail(MK_ERR_INVALID, "mk_gemm_blas_splitk: null workspace or output");
  if ((N % 4) != 0 || (c_ms % 4) != 0 || ((reinterpret_cast<uintptr_t>(C) | reinterpret_cast<uintptr_t>(workspace)) & 15))
    return mk::fail(MK_ERR_UNSUPPORTED, "mk_gemm_blas_splitk: N and c_ms multiples of 4, 16-byte aligned C and workspace");
  const int64_t ks = K / splits;
  // slice s reads A[:, s ks : (s+1) ks] and B[s ks : (s+1) ks, :] (element strides along k) and writes W[s]
  float* W = static_cast<float*>(workspace);
  if (int rc = mk::gemm_blas(s, ab_type, MK_F32, splits, M, N, ks, A, ks * a_ks, a_ms, a_ks, B, ks * b_ks, b_ks, b_ns,
                             W, M * N, N, 1.f, 0.f))
    return rc;
  return mk::splitk_sum(s, W, splits, M, N, C, c_ms, "mk_gemm_blas_splitk");
}

extern "C" int mk_gemm_blas(void* stream, int ab_type, int c_type, int64_t batch, int64_t M, int64_t N, int64_t K,
                            const void* A, int64_t a_bs, int64_t a_ms, int64_t a_ks,
                            const void* B, int64_t b_bs, int64_t b_ks, int64_t b_ns,
                            void* C, int64_t c_bs, int64_t c_ms, float alpha, float beta) {
  mk::clear_error();
  return mk::gemm_blas(mk::as_stream(stream), ab_type, c_type, batch, M, N, K, A, a_bs, a_ms, a_ks, B, b_bs, b_ks,
                       b_ns, C, c_bs, c_ms, alpha, beta);
}
