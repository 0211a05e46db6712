#pragma once
#include "common.h"

namespace crbq {
// C = beta*C + alpha*op(A)*op(B) on fp32 MFMA.  lower: only C[m][n] with
// n <= m is written (tiles wholly above the diagonal are skipped).
// stop: optional device flag; when *stop != 0 the kernel does nothing.
int sgemm_launch(bool ta, bool tb, bool lower, int64_t M, int64_t N, int64_t K,
                 float alpha, const float* A, int64_t lda, const float* B,
                 int64_t ldb, float beta, float* C, int64_t ldc,
                 const int* stop, hipStream_t s);
}  // namespace crbq
