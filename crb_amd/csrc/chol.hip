// Inverse-Hessian factor of BRAGPTQ.fasterquant (bigptq.py:101-129).
//
// The reference computes L = chol(H), H^-1 = cholesky_inverse(L) and
// U = chol(H^-1, upper) (4C^3/3 flops).  Here U comes from one factorization
// of the index-reversed matrix: with J the reversal permutation,
//   J H J = L' L'^T   =>   H^-1 = (J L'^-1 J)^T (J L'^-1 J),
// and J L'^-1 J is upper triangular with a positive diagonal, so it is U
// (the Cholesky factor is unique).  2C^3/3 flops.
//
// L'^-1 is formed in the same right-looking blocked sweep as L' (nb = 128):
// step j factors the diagonal block (one workgroup, in LDS, also inverting
// it: D_j = L'_jj^-1), then on fp32 MFMA
//   X[j, 0:j]        = D_j X[j, 0:j]                    (row block of L'^-1)
//   P                = A[j+1:, j] D_j^T                 (panel of L')
//   A[j+1:, j+1:]   -= P P^T          (lower tiles)     (SYRK)
//   X[j+1:, 0:j]    -= P X[j, 0:j]                      (inverse update)
//   X[j+1:, j]       = -P D_j
// where X shares A's storage: column block j of L' is consumed at step j,
// and the same storage then holds column block j of L'^-1.
// A pivot that is not > 0 (or NaN) sets *info (LAPACK potrf semantics) and
// every later kernel of the sweep returns at once; the host then adds the
// reference's extra damping and retries (bigptq.py:114-126).
#include "gemm_f32.h"

namespace crbq {

constexpr int NB = 128;

__global__ __launch_bounds__(256) void k_dead(float* H, int64_t ldh, int C, uint8_t* dead) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= C) return;
  float* p = H + (int64_t)i * ldh + i;
  const bool d = *p == 0.f;                     // bigptq.py:103-104
  dead[i] = d;
  if (d) *p = 1.f;
}

__global__ __launch_bounds__(256) void k_zero_dead(float* W, int64_t ldw, int R, int C,
                                                   const uint8_t* __restrict__ dead) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)R * C) return;
  const int c = (int)(idx % C);
  if (dead[c]) W[(idx / C) * ldw + c] = 0.f;    // bigptq.py:105
}

// H_ii += factor * mean(diag H); retry mode: 1e-6 when that is 0.
__global__ __launch_bounds__(1024) void k_damp(float* H, int64_t ldh, int C, float factor,
                                               int retry, float* out) {
  __shared__ double red[1024];
  const int tid = threadIdx.x;
  double s = 0.0;
  for (int i = tid; i < C; i += 1024) s += (double)H[(int64_t)i * ldh + i];
  red[tid] = s;
  __syncthreads();
  for (int o = 512; o > 0; o >>= 1) {
    if (tid < o) red[tid] += red[tid + o];
    __syncthreads();
  }
  const float mean = (float)red[0] / (float)C;
  float v = factor * mean;
  if (retry && v == 0.f) v = 1e-6f;             // bigptq.py:120-121
  for (int i = tid; i < C; i += 1024) {
    float* p = H + (int64_t)i * ldh + i;
    *p = *p + v;
  }
  if (tid == 0 && out) *out = v;
}

__global__ void k_set_int(int* p, int v) { *p = v; }

// A[i][j] = H[C-1-i][C-1-j], lower triangle only
__global__ __launch_bounds__(256) void k_reverse_lower(const float* __restrict__ H, int64_t ldh,
                                                       int C, float* A, int64_t lda) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int i = (int)(idx / C), j = (int)(idx % C);
  if (i >= C || j > i) return;
  A[(int64_t)i * lda + j] = H[(int64_t)(C - 1 - i) * ldh + (C - 1 - j)];
}

// U[i][j] = X[C-1-i][C-1-j] for j >= i, 0 below the diagonal
__global__ __launch_bounds__(256) void k_reverse_to_u(const float* __restrict__ X, int64_t ldx,
                                                      int C, float* U, int64_t ldu) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int i = (int)(idx / C), j = (int)(idx % C);
  if (i >= C) return;
  U[(int64_t)i * ldu + j] = j >= i ? X[(int64_t)(C - 1 - i) * ldx + (C - 1 - j)] : 0.f;
}

// Last resort (bigptq.py:124-128): L = diag(sqrt(clamp(diag H, 1e-8))),
// H^-1 = diag(1 / L_ii^2), U = diag(sqrt(1 / L_ii^2)).
__global__ __launch_bounds__(256) void k_fallback_u(const float* __restrict__ H, int64_t ldh,
                                                    int C, float* U, int64_t ldu) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int i = (int)(idx / C), j = (int)(idx % C);
  if (i >= C) return;
  float v = 0.f;
  if (i == j) {
    const float l = sqrtf(fmaxf(H[(int64_t)i * ldh + i], 1e-8f));
    const float inv = 1.f / (l * l);
    v = sqrtf(inv);
  }
  U[(int64_t)i * ldu + j] = v;
}

// Diagonal block: Cholesky and triangular inverse of one NB x NB block,
// blocked by 8.  256 threads as a 16 x 16 grid; thread (ty, tx) keeps the
// 8 x 8 sub-block rows ty*8.., cols tx*8.. in registers.  Step kb of the
// factorization: the owner of diagonal block (kb, kb) factors and inverts
// it in registers; the owners of column kb form the panel
// P_I = A_I,kb D_kb^T; every lower block right of column kb takes the
// rank-8 update A_IJ -= P_I P_J^T.  The inverse X = L^-1 is the same
// right-looking sweep on the identity: X_kb,J = D_kb B_kb,J, then
// B_I,J -= L_I,kb X_kb,J.  Rows past bj are padded with the identity.
__device__ __forceinline__ void chol8(float (&a)[8][8], float (&x)[8][8], int& bad) {
  bad = -1;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const float p = a[k][k];
    if (!(p > 0.f) && bad < 0) bad = k;
    const float d = sqrtf(p), di = 1.f / d;
    a[k][k] = d;
#pragma unroll
    for (int r = k + 1; r < 8; ++r) a[r][k] = a[r][k] * di;
#pragma unroll
    for (int c = k + 1; c < 8; ++c)
#pragma unroll
      for (int r = c; r < 8; ++r) a[r][c] = a[r][c] - a[r][k] * a[c][k];
  }
#pragma unroll
  for (int r = 0; r < 8; ++r)
#pragma unroll
    for (int c = 0; c < 8; ++c) x[r][c] = r == c ? 1.f : 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const float di = 1.f / a[k][k];
#pragma unroll
    for (int c = 0; c <= k; ++c) x[k][c] = x[k][c] * di;
#pragma unroll
    for (int r = k + 1; r < 8; ++r)
#pragma unroll
      for (int c = 0; c <= k; ++c) x[r][c] = x[r][c] - a[r][k] * x[k][c];
  }
}

__global__ __launch_bounds__(256) void k_potrf_diag(float* A, int64_t lda, int off, int bj,
                                                    float* D, int* info) {
  if (*info) return;
  __shared__ __attribute__((aligned(16))) float pan[NB][8];     // column panel of L
  __shared__ __attribute__((aligned(16))) float Dk[NB / 8][8][8];  // inverses of diag blocks
  __shared__ __attribute__((aligned(16))) float xr[8][NB];      // row panel of X
  __shared__ int fail;
  const int tid = threadIdx.x, ty = tid >> 4, tx = tid & 15;
  const int i0 = ty * 8, j0 = tx * 8;
  const int nkb = (bj + 7) / 8;
  float a[8][8], x[8][8];
#pragma unroll
  for (int r = 0; r < 8; ++r)
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int i = i0 + r, j = j0 + c;
      a[r][c] = (i < bj && j <= i) ? A[(int64_t)(off + i) * lda + off + j]
                                   : (i == j ? 1.f : 0.f);
    }
  if (tid == 0) fail = 0;
  __syncthreads();
  for (int kb = 0; kb < nkb; ++kb) {
    if (ty == kb && tx == kb) {                       // factor + invert the diagonal block
      int bad;
      chol8(a, x, bad);
      if (bad >= 0 && i0 + bad < bj) {
        fail = 1;
        atomicCAS(info, 0, off + i0 + bad + 1);
      }
#pragma unroll
      for (int r = 0; r < 8; ++r)
#pragma unroll
        for (int c = 0; c < 8; ++c) Dk[kb][r][c] = c <= r ? x[r][c] : 0.f;
    }
    __syncthreads();
    if (fail) return;
    if (tx == kb && ty > kb) {                        // panel P_I = A_I,kb D_kb^T
      float p[8][8];
#pragma unroll
      for (int r = 0; r < 8; ++r)
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          float v = 0.f;
#pragma unroll
          for (int m = 0; m <= c; ++m) v = v + a[r][m] * Dk[kb][c][m];
          p[r][c] = v;
        }
#pragma unroll
      for (int r = 0; r < 8; ++r)
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          a[r][c] = p[r][c];
          pan[i0 + r][c] = p[r][c];
        }
    }
    __syncthreads();
    if (ty >= tx && tx > kb) {                        // A_IJ -= P_I P_J^T
      float pi[8][8];
#pragma unroll
      for (int r = 0; r < 8; ++r)
#pragma unroll
        for (int m = 0; m < 8; ++m) pi[r][m] = pan[i0 + r][m];
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        float pj[8];
#pragma unroll
        for (int m = 0; m < 8; ++m) pj[m] = pan[j0 + c][m];
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          float v = a[r][c];
#pragma unroll
          for (int m = 0; m < 8; ++m) v = v - pi[r][m] * pj[m];
          a[r][c] = v;
        }
      }
    }
  }
  // a: L blocks (I >= J).  X = L^-1, right-looking on the identity.
#pragma unroll
  for (int r = 0; r < 8; ++r)
#pragma unroll
    for (int c = 0; c < 8; ++c) x[r][c] = (i0 + r == j0 + c) ? 1.f : 0.f;
  for (int kb = 0; kb < nkb; ++kb) {
    __syncthreads();                                  // previous step's readers are done
    if (ty == kb && tx <= kb) {                       // X_kb,J = D_kb B_kb,J
      float y[8][8];
#pragma unroll
      for (int r = 0; r < 8; ++r)
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          float v = 0.f;
#pragma unroll
          for (int m = 0; m <= r; ++m) v = v + Dk[kb][r][m] * x[m][c];
          y[r][c] = v;
        }
#pragma unroll
      for (int r = 0; r < 8; ++r)
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          x[r][c] = y[r][c];
          xr[r][j0 + c] = y[r][c];
        }
    }
    if (tx == kb && ty > kb) {                        // publish L_I,kb
#pragma unroll
      for (int r = 0; r < 8; ++r)
#pragma unroll
        for (int m = 0; m < 8; ++m) pan[i0 + r][m] = a[r][m];
    }
    __syncthreads();
    if (ty > kb && tx <= kb) {                        // B_I,J -= L_I,kb X_kb,J
      float li[8][8];
#pragma unroll
      for (int r = 0; r < 8; ++r)
#pragma unroll
        for (int m = 0; m < 8; ++m) li[r][m] = pan[i0 + r][m];
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        float xc[8];
#pragma unroll
        for (int m = 0; m < 8; ++m) xc[m] = xr[m][j0 + c];
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          float v = x[r][c];
#pragma unroll
          for (int m = 0; m < 8; ++m) v = v - li[r][m] * xc[m];
          x[r][c] = v;
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < 8; ++r)
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int i = i0 + r, j = j0 + c;
      if (i < bj && j < bj) {
        const float v = j <= i ? x[r][c] : 0.f;
        D[i * NB + j] = v;
        A[(int64_t)(off + i) * lda + off + j] = v;
      }
    }
}

static inline unsigned nblocks(int64_t n) { return (unsigned)((n + 255) / 256); }

struct HinvWs {
  float* A;        // C x C (ld = C)
  float* P;        // C x NB panel
  float* D;        // NB x NB
  int* info;
  float* scal;
  uint8_t* dead;   // C
};

static void carve_hinv(WsCarver& c, int64_t C, HinvWs& w) {
  w.A = c.take<float>((size_t)C * C);
  w.P = c.take<float>((size_t)C * NB);
  w.D = c.take<float>((size_t)NB * NB);
  w.info = c.take<int>(4);
  w.scal = c.take<float>(4);
  w.dead = c.take<uint8_t>((size_t)C);
}

// One full attempt: factor and invert A in place.  Returns a launch status;
// the factorization outcome is in *w.info.
static int chol_inv_sweep(float* A, int64_t lda, int C, HinvWs& w, hipStream_t s) {
  const int nblk = (C + NB - 1) / NB;
  for (int j = 0; j < nblk; ++j) {
    const int off = j * NB, bj = std::min(NB, C - off), rest = C - off - bj;
    k_potrf_diag<<<1, 256, 0, s>>>(A, lda, off, bj, w.D, w.info);
    CRBQ_LAUNCH_CHECK();
    int st;
    if (off > 0) {           // X[j, 0:j] = D_j X[j, 0:j]  (in place)
      st = sgemm_launch(false, false, false, bj, off, bj, 1.f, w.D, NB, A + (int64_t)off * lda,
                        lda, 0.f, A + (int64_t)off * lda, lda, w.info, s);
      if (st) return st;
    }
    if (rest > 0) {
      float* Apan = A + (int64_t)(off + bj) * lda + off;
      // P = A[j+1:, j] D_j^T
      st = sgemm_launch(false, true, false, rest, bj, bj, 1.f, Apan, lda, w.D, NB, 0.f, w.P,
                        NB, w.info, s);
      if (st) return st;
      // A[j+1:, j+1:] -= P P^T (lower)
      st = sgemm_launch(false, true, true, rest, rest, bj, -1.f, w.P, NB, w.P, NB, 1.f,
                        A + (int64_t)(off + bj) * lda + off + bj, lda, w.info, s);
      if (st) return st;
      if (off > 0) {         // X[j+1:, 0:j] -= P X[j, 0:j]
        st = sgemm_launch(false, false, false, rest, off, bj, -1.f, w.P, NB,
                          A + (int64_t)off * lda, lda, 1.f, A + (int64_t)(off + bj) * lda, lda,
                          w.info, s);
        if (st) return st;
      }
      // X[j+1:, j] = -P D_j
      st = sgemm_launch(false, false, false, rest, bj, bj, -1.f, w.P, NB, w.D, NB, 0.f, Apan,
                        lda, w.info, s);
      if (st) return st;
    }
  }
  return CRBQ_OK;
}

}  // namespace crbq

using namespace crbq;

extern "C" size_t crbq_hinv_workspace_size(int64_t C) {
  WsCarver c(nullptr, 0);
  HinvWs w;
  carve_hinv(c, C, w);
  return c.off + 256;
}

static int hinv_check(float* H, int64_t ldh, int64_t C, float* W, int64_t R, int64_t ldw,
                      float* U, int64_t ldu) {
  if (!H || !U || C <= 0 || ldh < C || ldu < C) return CRBQ_ERR_ARG;
  if (W && (R <= 0 || ldw < C)) return CRBQ_ERR_ARG;
  if (C > (1 << 20)) return CRBQ_ERR_ARG;
  return CRBQ_OK;
}

// dead columns, damping and one factorization attempt; U written assuming
// success (the finish step checks *info and redoes it on failure)
extern "C" int crbq_hinv_upper_async(float* H, int64_t ldh, int64_t C, float* W, int64_t R,
                                     int64_t ldw, float percdamp, float* U, int64_t ldu,
                                     void* ws, size_t ws_bytes, void* stream) {
  int st = hinv_check(H, ldh, C, W, R, ldw, U, ldu);
  if (st) return st;
  WsCarver c(ws, ws_bytes);
  HinvWs w;
  carve_hinv(c, C, w);
  if (!c.ok()) return CRBQ_ERR_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  const int Ci = (int)C;
  k_dead<<<nblocks(C), 256, 0, s>>>(H, ldh, Ci, w.dead);
  CRBQ_LAUNCH_CHECK();
  if (W) {
    k_zero_dead<<<nblocks(R * C), 256, 0, s>>>(W, ldw, (int)R, Ci, w.dead);
    CRBQ_LAUNCH_CHECK();
  }
  k_damp<<<1, 1024, 0, s>>>(H, ldh, Ci, percdamp, 0, w.scal);      // bigptq.py:109-111
  CRBQ_LAUNCH_CHECK();
  k_set_int<<<1, 1, 0, s>>>(w.info, 0);
  k_reverse_lower<<<nblocks(C * C), 256, 0, s>>>(H, ldh, Ci, w.A, C);
  CRBQ_LAUNCH_CHECK();
  st = chol_inv_sweep(w.A, C, Ci, w, s);
  if (st) return st;
  k_reverse_to_u<<<nblocks(C * C), 256, 0, s>>>(w.A, C, Ci, U, ldu);
  CRBQ_LAUNCH_CHECK();
  return CRBQ_OK;
}

// Synchronises `stream`, reads the first attempt's outcome and, if the
// Cholesky failed, runs the reference's retries and fallback
// (bigptq.py:114-126) synchronously.
extern "C" int crbq_hinv_upper_finish(float* H, int64_t ldh, int64_t C, float* U, int64_t ldu,
                                      void* ws, size_t ws_bytes, int* retries, int* fallback,
                                      void* stream) {
  int st = hinv_check(H, ldh, C, nullptr, 0, 0, U, ldu);
  if (st) return st;
  WsCarver c(ws, ws_bytes);
  HinvWs w;
  carve_hinv(c, C, w);
  if (!c.ok()) return CRBQ_ERR_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  const int Ci = (int)C;
  int hinfo = 0;
  CRBQ_HIP(hipMemcpyAsync(&hinfo, w.info, sizeof(int), hipMemcpyDeviceToHost, s));
  CRBQ_HIP(hipStreamSynchronize(s));
  int nretry = 0;
  bool ok = hinfo == 0;
  for (int attempt = 1; !ok && attempt <= 10; ++attempt) {        // bigptq.py:115-123
    ++nretry;
    k_damp<<<1, 1024, 0, s>>>(H, ldh, Ci, 1e-3f, 1, w.scal);
    CRBQ_LAUNCH_CHECK();
    if (attempt == 10) break;                                       // 10 attempts in all
    k_set_int<<<1, 1, 0, s>>>(w.info, 0);
    k_reverse_lower<<<nblocks(C * C), 256, 0, s>>>(H, ldh, Ci, w.A, C);
    CRBQ_LAUNCH_CHECK();
    st = chol_inv_sweep(w.A, C, Ci, w, s);
    if (st) return st;
    CRBQ_HIP(hipMemcpyAsync(&hinfo, w.info, sizeof(int), hipMemcpyDeviceToHost, s));
    CRBQ_HIP(hipStreamSynchronize(s));
    ok = hinfo == 0;
    if (ok) {
      k_reverse_to_u<<<nblocks(C * C), 256, 0, s>>>(w.A, C, Ci, U, ldu);
      CRBQ_LAUNCH_CHECK();
    }
  }
  if (!ok) {
    k_fallback_u<<<nblocks(C * C), 256, 0, s>>>(H, ldh, Ci, U, ldu);
    CRBQ_LAUNCH_CHECK();
  }
  if (retries) *retries = nretry;
  if (fallback) *fallback = ok ? 0 : 1;
  return CRBQ_OK;
}

extern "C" int crbq_hinv_upper(float* H, int64_t ldh, int64_t C, float* W, int64_t R,
                               int64_t ldw, float percdamp, float* U, int64_t ldu, void* ws,
                               size_t ws_bytes, int* retries, int* fallback, void* stream) {
  int st = crbq_hinv_upper_async(H, ldh, C, W, R, ldw, percdamp, U, ldu, ws, ws_bytes, stream);
  if (st) return st;
  return crbq_hinv_upper_finish(H, ldh, C, U, ldu, ws, ws_bytes, retries, fallback, stream);
}
