// fp32 GEMM on the CDNA4 fp32 matrix cores (v_mfma_f32_16x16x4_f32).
//
// C = beta*C + alpha*op(A)*op(B).  Used for the GPTQ trailing update
// W[:, ed:] -= Err @ U[st:ed, ed:] (bigptq.py:264) and for the panel, SYRK
// and inverse updates of the blocked Cholesky/inverse (bigptq.py:117-128).
// The reference disables TF32 (bigptq.py:11-12); these products are full
// fp32 MFMA with fp32 accumulation.
//
// Tiling: 128x128 output tile per 256-thread workgroup (4 wavefronts in a
// 2x2 arrangement, 64x64 each = 4x4 MFMA 16x16 tiles); small products use
// 64x64 tiles (wavefronts of 32x32).  K is staged through
// double-buffered LDS 32 at a time; every operand keeps its global layout in
// LDS so a tile moves as float4 copies, and the next K chunk's global loads
// are in flight while the current chunk's 128 MFMAs per wavefront run.
#include "gemm_f32.h"

namespace crbq {

constexpr int GB_K = 32;          // K staged per chunk
constexpr int P_MK = GB_K + 4;    // pitch of a row-of-K layout (m- or n-major)

// LDS floats of one operand tile of a BT x BT output tile (either layout).
template <int BT>
struct TileCfg {
  static constexpr int P_KM = BT + 16;                // pitch of a K-major layout: the 4 lane
                                                      // groups (k .. k+3) hit disjoint banks
  static constexpr int ELEMS = BT * P_MK > GB_K * P_KM ? BT * P_MK : GB_K * P_KM;
  static constexpr int NE = BT * GB_K / 4 / 256;      // float4 per thread per operand
  static constexpr int WT = BT / 2;                   // wavefront tile side (2 x 2 waves)
  static constexpr int MT = WT / 16;                  // MFMA tiles per wavefront side
};

// Load the float4 at (row, col..col+3) of a row-major matrix, zero-filling
// anything outside rows x cols.
__device__ __forceinline__ float4 ld4(const float* p, int64_t ld, int row, int col, int rows,
                                      int cols, bool vec) {
  if (row >= rows) return make_float4(0.f, 0.f, 0.f, 0.f);
  const float* q = p + (int64_t)row * ld + col;
  if (vec && col + 3 < cols) return *(const float4*)q;
  float4 v;
  v.x = col + 0 < cols ? q[0] : 0.f;
  v.y = col + 1 < cols ? q[1] : 0.f;
  v.z = col + 2 < cols ? q[2] : 0.f;
  v.w = col + 3 < cols ? q[3] : 0.f;
  return v;
}

// Tile of op(X) for K chunk k0.  KMAJ: X is stored [k][mn] (row = k);
// otherwise X is stored [mn][k].  Thread f-th float4 -> (row, col).
template <int BT, bool KMAJ>
__device__ __forceinline__ void load_tile(const float* X, int64_t ld, int mn0, int k0, int MN,
                                          int K, bool vec, float4 (&r)[TileCfg<BT>::NE]) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int e = 0; e < TileCfg<BT>::NE; ++e) {
    const int f = tid + 256 * e;
    if (KMAJ) {
      const int k = f / (BT / 4), c = (f % (BT / 4)) * 4;
      r[e] = ld4(X, ld, k0 + k, mn0 + c, K, MN, vec);
    } else {
      const int m = f >> 3, c = (f & 7) * 4;
      r[e] = ld4(X, ld, mn0 + m, k0 + c, MN, K, vec);
    }
  }
}

// The same tile when it lies wholly inside the matrix and rows are 16-byte
// aligned: unconditional float4 loads.
template <int BT, bool KMAJ>
__device__ __forceinline__ void load_tile_in(const float* X, int64_t ld, int mn0, int k0,
                                             float4 (&r)[TileCfg<BT>::NE]) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int e = 0; e < TileCfg<BT>::NE; ++e) {
    const int f = tid + 256 * e;
    if (KMAJ) {
      const int k = f / (BT / 4), c = (f % (BT / 4)) * 4;
      r[e] = *(const float4*)(X + (int64_t)(k0 + k) * ld + mn0 + c);
    } else {
      const int m = f >> 3, c = (f & 7) * 4;
      r[e] = *(const float4*)(X + (int64_t)(mn0 + m) * ld + k0 + c);
    }
  }
}

template <int BT, bool KMAJ>
__device__ __forceinline__ void store_tile(float* S, const float4 (&r)[TileCfg<BT>::NE]) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int e = 0; e < TileCfg<BT>::NE; ++e) {
    const int f = tid + 256 * e;
    if (KMAJ) {
      const int k = f / (BT / 4), c = (f % (BT / 4)) * 4;
      *(float4*)&S[k * TileCfg<BT>::P_KM + c] = r[e];
    } else {
      const int m = f >> 3, c = (f & 7) * 4;
      *(float4*)&S[m * P_MK + c] = r[e];
    }
  }
}

// Output tile of linear workgroup id.  Plain products go row by row, with
// the ids regrouped so that the workgroups one XCD receives (every 8th id)
// cover consecutive tiles and share operand panels in that XCD's L2.  When
// one operand is triangular the tiles go longest K range first, so the
// short ones fill the tail; the lower-triangle product enumerates only the
// tiles on or below the diagonal.
__device__ __forceinline__ void gemm_tile(int id, int nwg, int TM, int TN, int tri, bool lower,
                                          int& tm, int& tn) {
  if (lower) {                         // id -> (tm >= tn), row tm holds tm + 1 tiles
    int r = (int)((sqrtf(8.f * (float)id + 1.f) - 1.f) * 0.5f);
    while ((r + 1) * (r + 2) / 2 <= id) ++r;
    while (r * (r + 1) / 2 > id) --r;
    tm = r;
    tn = id - r * (r + 1) / 2;
    return;
  }
  if (tri == GEMM_TRI_KEND_N) { tn = TN - 1 - id / TM; tm = id % TM; return; }
  if (tri == GEMM_TRI_KBEG_N) { tn = id / TM; tm = id % TM; return; }
  if (tri == GEMM_TRI_KEND_M) { tm = TM - 1 - id / TN; tn = id % TN; return; }
  const int q = nwg / 8, r = nwg % 8, x = id % 8, k = id / 8;
  const int lin = (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + k;
  tm = lin / TN;
  tn = lin % TN;
}

template <int BT, bool TA, bool TB, bool LOWER>
__global__ __launch_bounds__(256) void k_sgemm(
    int M, int N, int K, float alpha, const float* A, int64_t lda,
    const float* B, int64_t ldb, float beta, float* C,
    int64_t ldc, const int* __restrict__ stop, int va, int vb, int tri) {
  using Cfg = TileCfg<BT>;
  constexpr int P_KM = Cfg::P_KM, WT = Cfg::WT, MT = Cfg::MT, NE = Cfg::NE;
  if (stop && *stop) return;
  int tm, tn;
  gemm_tile(blockIdx.x, gridDim.x, (M + BT - 1) / BT, (N + BT - 1) / BT, tri, LOWER, tm, tn);
  const int m0 = tm * BT, n0 = tn * BT;
  // K range of this tile when one operand is triangular (its zero part is
  // skipped; the products skipped are exact zeros)
  int kbeg = 0, kend = K;
  if (tri == GEMM_TRI_KEND_N) kend = min(K, n0 + BT);
  else if (tri == GEMM_TRI_KBEG_N) kbeg = min(K, n0) / GB_K * GB_K;
  else if (tri == GEMM_TRI_KEND_M) kend = min(K, m0 + BT);
  __shared__ __attribute__((aligned(16))) float As[2][Cfg::ELEMS];
  __shared__ __attribute__((aligned(16))) float Bs[2][Cfg::ELEMS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = (wave >> 1) * WT, wn = (wave & 1) * WT;
  const int c16 = lane & 15, kq = lane >> 4;
  // A is K-major in memory iff TA; B is K-major iff !TB
  constexpr bool AK = TA, BK = !TB;
  f4_t acc[MT][MT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};

  const int nch = kend > kbeg ? (kend - kbeg + GB_K - 1) / GB_K : 0;
  // interior tile: every chunk but a ragged last one loads without bounds checks
  const bool in_mn = va && vb && m0 + BT <= M && n0 + BT <= N;
  const int nfull = in_mn ? (kend - kbeg) / GB_K : 0;
  float4 ra[NE], rb[NE];
  if (nch > 0) {
    load_tile<BT, AK>(A, lda, m0, kbeg, M, K, va, ra);
    load_tile<BT, BK>(B, ldb, n0, kbeg, N, K, vb, rb);
    store_tile<BT, AK>(As[0], ra);
    store_tile<BT, BK>(Bs[0], rb);
  }
  __syncthreads();
  for (int c = 0; c < nch; ++c) {
    const int buf = c & 1;
    if (c + 1 < nfull) {
      load_tile_in<BT, AK>(A, lda, m0, kbeg + (c + 1) * GB_K, ra);
      load_tile_in<BT, BK>(B, ldb, n0, kbeg + (c + 1) * GB_K, rb);
    } else if (c + 1 < nch) {
      load_tile<BT, AK>(A, lda, m0, kbeg + (c + 1) * GB_K, M, K, va, ra);
      load_tile<BT, BK>(B, ldb, n0, kbeg + (c + 1) * GB_K, N, K, vb, rb);
    }
    const float* as = As[buf];
    const float* bs = Bs[buf];
#pragma unroll
    for (int kk = 0; kk < GB_K; kk += 4) {
      const int k = kk + kq;
      float a[MT], b[MT];
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const int m = wm + i * 16 + c16;
        a[i] = AK ? as[k * P_KM + m] : as[m * P_MK + k];
      }
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        const int n = wn + j * 16 + c16;
        b[j] = BK ? bs[k * P_KM + n] : bs[n * P_MK + k];
      }
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < MT; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (c + 1 < nch) {
      store_tile<BT, AK>(As[buf ^ 1], ra);
      store_tile<BT, BK>(Bs[buf ^ 1], rb);
    }
    __syncthreads();
  }
  // D[row][col]: col = lane%16, row = 4*(lane/16) + r.
  const int r4 = kq * 4;
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < MT; ++j)
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

static inline bool vec_ok(const float* p, int64_t ld) {
  return ((((uintptr_t)p) & 15) == 0) && ((ld & 3) == 0);
}

template <int BT>
static int sgemm_go(bool ta, bool tb, bool lower, int64_t M, int64_t N, int64_t K,
                    float alpha, const float* A, int64_t lda, const float* B, int64_t ldb,
                    float beta, float* C, int64_t ldc, const int* stop, hipStream_t s,
                    int tri) {
  const int64_t TM = (M + BT - 1) / BT, TN = (N + BT - 1) / BT;
  // lower: the square tile grid's lower triangle (M == N)
  if (lower && TM != TN) return CRBQ_ERR_ARG;
  const int64_t nwg = lower ? TM * (TM + 1) / 2 : TM * TN;
  if (nwg > 0x7fffffff) return CRBQ_ERR_ARG;
  const dim3 grid((unsigned)nwg);
  const int m = (int)M, n = (int)N, k = (int)K;
  const int va = vec_ok(A, lda), vb = vec_ok(B, ldb);
#define CRBQ_GEMM_CASE(TA_, TB_, LO_)                                                  \
  if (ta == TA_ && tb == TB_ && lower == LO_) {                                        \
    k_sgemm<BT, TA_, TB_, LO_><<<grid, 256, 0, s>>>(m, n, k, alpha, A, lda, B, ldb,    \
                                                    beta, C, ldc, stop, va, vb, tri);  \
    CRBQ_LAUNCH_CHECK();                                                               \
    return CRBQ_OK;                                                                    \
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

// Products that give fewer 128 x 128 tiles than the GPU has CUs run on
// 64 x 64 tiles (4x the workgroups, a quarter of the work each), and those
// with fewer than 64 such tiles on 32 x 32 tiles, which shortens the small
// products of the factorization's lower levels (latency chains of a few
// workgroups each).
int sgemm_launch(bool ta, bool tb, bool lower, int64_t M, int64_t N, int64_t K,
                 float alpha, const float* A, int64_t lda, const float* B,
                 int64_t ldb, float beta, float* C, int64_t ldc,
                 const int* stop, hipStream_t s, int tri) {
  if (M <= 0 || N <= 0) return CRBQ_OK;
  if (M > (1 << 30) || N > (1 << 30) || K > (1 << 30) || K < 0) return CRBQ_ERR_ARG;
  const int64_t t128 = ((M + 127) / 128) * ((N + 127) / 128);
  const int64_t t64 = ((M + 63) / 64) * ((N + 63) / 64);
  if (t64 < 128)
    return sgemm_go<32>(ta, tb, lower, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, stop, s,
                        tri);
  if (t128 < 256)
    return sgemm_go<64>(ta, tb, lower, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, stop, s,
                        tri);
  return sgemm_go<128>(ta, tb, lower, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, stop, s,
                       tri);
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
