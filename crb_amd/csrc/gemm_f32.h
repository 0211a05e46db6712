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

// One product for sgemm2_launch.
struct GemmArgs {
  bool ta, tb, lower;
  int64_t M, N, K;
  float alpha;
  const float* A;
  int64_t lda;
  const float* B;
  int64_t ldb;
  float beta;
  float* C;
  int64_t ldc;
  int tri;
};
// Two independent products (neither writes what the other reads): x a
// lower-tile product op(A) B^T with M == N, y a plain op(A) B (triangular K
// allowed).  One launch when both pick the same tile size, with x's tiles
// first; otherwise the two launches of sgemm_launch in order.
int sgemm2_launch(const GemmArgs& x, const GemmArgs& y, const int* stop, hipStream_t s);
// nseg (1..4) plain products op(A) B with no transposes, no triangle and
// one shape (M, N, K): one launch, each product computed as its own
// sgemm_launch would; otherwise one sgemm_launch per product in order.
int sgemm_seg_launch(int nseg, const GemmArgs* gs, hipStream_t s);
}  // namespace crbq
