#pragma once
#include "common.h"

namespace crbq {
// C = beta*C + alpha*op(A)*op(B) on fp32 MFMA.  lower: only C[m][n] with
// n <= m is written (tiles wholly above the diagonal are skipped).
// stop: optional device flag; when *stop != 0 the kernel does nothing.
// tri: one operand is triangular and only the K range where it can be
// nonzero is summed (its other entries must hold zeros):
//   GEMM_TRI_KEND_N  op(B)[k][n] = 0 for k > n  (B lower with TB, or upper)
//   GEMM_TRI_KBEG_N  op(B)[k][n] = 0 for k < n  (B lower, no transpose)
//   GEMM_TRI_KEND_M  op(A)[m][k] = 0 for k > m  (A lower, no transpose)
enum { GEMM_TRI_NONE = 0, GEMM_TRI_KEND_N = 1, GEMM_TRI_KBEG_N = 2, GEMM_TRI_KEND_M = 3 };
int sgemm_launch(bool ta, bool tb, bool lower, int64_t M, int64_t N, int64_t K,
                 float alpha, const float* A, int64_t lda, const float* B,
                 int64_t ldb, float beta, float* C, int64_t ldc,
                 const int* stop, hipStream_t s, int tri = GEMM_TRI_NONE);
}  // namespace crbq
