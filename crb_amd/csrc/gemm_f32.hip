// fp32 GEMM on the CDNA4 fp32 matrix cores (v_mfma_f32_16x16x4_f32).
//
// C = beta*C + alpha*op(A)*op(B).  Used for the GPTQ trailing update
// W[:, ed:] -= Err @ U[st:ed, ed:] (bigptq.py:264) and for the panel, SYRK
// and inverse updates of the blocked Cholesky/inverse (bigptq.py:117-128).
// The reference disables TF32 (bigptq.py:11-12); these products are full
// fp32 MFMA with fp32 accumulation.
//
// Tiling: 128x128 output tile per 256-thread workgroup (4 wavefronts in a
// 2x2 arrangement, 64x64 each = 4x4 MFMA 16x16 tiles), K staged through LDS
// 16 at a time in k-major layout so every MFMA operand read is one
// conflict-free ds_read_b32 per lane.
#include "gemm_f32.h"

namespace crbq {

constexpr int GB_M = 128, GB_N = 128, GB_K = 16, G_PAD = 4;

template <bool TA, bool TB, bool LOWER>
__global__ __launch_bounds__(256) void k_sgemm(
    int M, int N, int K, float alpha, const float* A, int64_t lda,
    const float* B, int64_t ldb, float beta, float* C,
    int64_t ldc, const int* __restrict__ stop) {
  if (stop && *stop) return;
  const int m0 = blockIdx.y * GB_M, n0 = blockIdx.x * GB_N;
  if (LOWER && n0 > m0 + GB_M - 1) return;  // tile entirely above diagonal
  __shared__ float As[GB_K][GB_M + G_PAD];
  __shared__ float Bs[GB_K][GB_N + G_PAD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  f4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};

  for (int k0 = 0; k0 < K; k0 += GB_K) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int idx = tid + 256 * e;
      int m, k;
      if (TA) { k = idx >> 7; m = idx & 127; }
      else    { m = idx >> 4; k = idx & 15; }
      const int gm = m0 + m, gk = k0 + k;
      float v = 0.f;
      if (gm < M && gk < K) v = TA ? A[(int64_t)gk * lda + gm] : A[(int64_t)gm * lda + gk];
      As[k][m] = v;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int idx = tid + 256 * e;
      int n, k;
      if (TB) { n = idx >> 4; k = idx & 15; }
      else    { k = idx >> 7; n = idx & 127; }
      const int gn = n0 + n, gk = k0 + k;
      float v = 0.f;
      if (gn < N && gk < K) v = TB ? B[(int64_t)gn * ldb + gk] : B[(int64_t)gk * ldb + gn];
      Bs[k][n] = v;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < GB_K; kk += 4) {
      const int kr = kk + (lane >> 4), c16 = lane & 15;
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[kr][wm + i * 16 + c16];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Bs[kr][wn + j * 16 + c16];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }
  // D[row][col]: col = lane%16, row = 4*(lane/16) + r.
  const int c16 = lane & 15, r4 = (lane >> 4) * 4;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int gm = m0 + wm + i * 16 + r4 + r;
        const int gn = n0 + wn + j * 16 + c16;
        if (gm < M && gn < N && (!LOWER || gn <= gm)) {
          float* p = C + (int64_t)gm * ldc + gn;
          const float prod = alpha * acc[i][j][r];
          *p = (beta == 0.f) ? prod : beta * (*p) + prod;
        }
      }
}

int sgemm_launch(bool ta, bool tb, bool lower, int64_t M, int64_t N, int64_t K,
                 float alpha, const float* A, int64_t lda, const float* B,
                 int64_t ldb, float beta, float* C, int64_t ldc,
                 const int* stop, hipStream_t s) {
  if (M <= 0 || N <= 0) return CRBQ_OK;
  if (M > (1 << 30) || N > (1 << 30) || K > (1 << 30) || K < 0) return CRBQ_ERR_ARG;
  dim3 grid((unsigned)((N + GB_N - 1) / GB_N), (unsigned)((M + GB_M - 1) / GB_M));
  if (grid.y > 65535) return CRBQ_ERR_ARG;
  const int m = (int)M, n = (int)N, k = (int)K;
#define CRBQ_GEMM_CASE(TA_, TB_, LO_)                                              \
  if (ta == TA_ && tb == TB_ && lower == LO_) {                                    \
    k_sgemm<TA_, TB_, LO_><<<grid, 256, 0, s>>>(m, n, k, alpha, A, lda, B, ldb,    \
                                                beta, C, ldc, stop);               \
    CRBQ_LAUNCH_CHECK();                                                           \
    return CRBQ_OK;                                                                \
  }
  CRBQ_GEMM_CASE(false, false, false)
  CRBQ_GEMM_CASE(false, true, false)
  CRBQ_GEMM_CASE(true, false, false)
  CRBQ_GEMM_CASE(true, true, false)
  CRBQ_GEMM_CASE(false, true, true)
  CRBQ_GEMM_CASE(false, false, true)
#undef CRBQ_GEMM_CASE
  return CRBQ_ERR_ARG;
}

}  // namespace crbq

extern "C" int crbq_sgemm(int transa, int transb, int64_t M, int64_t N,
                          int64_t K, float alpha, const float* A, int64_t lda,
                          const float* B, int64_t ldb, float beta, float* C,
                          int64_t ldc, void* stream) {
  if (!A || !B || !C) return CRBQ_ERR_ARG;
  return crbq::sgemm_launch(transa != 0, transb != 0, false, M, N, K, alpha, A,
                            lda, B, ldb, beta, C, ldc, nullptr,
                            (hipStream_t)stream);
}
