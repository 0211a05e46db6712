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

// Diagonal block: Cholesky and triangular inverse in LDS.
__global__ __launch_bounds__(256) void k_potrf_diag(float* A, int64_t lda, int off, int bj,
                                                    float* D, int* info) {
  if (*info) return;
  __shared__ float L[NB][NB + 1];
  __shared__ float X[NB][NB + 1];
  __shared__ int fail;
  const int tid = threadIdx.x;
  for (int idx = tid; idx < NB * NB; idx += 256) {
    const int i = idx / NB, k = idx % NB;
    L[i][k] = (i < bj && k <= i) ? A[(int64_t)(off + i) * lda + off + k] : 0.f;
    X[i][k] = (i == k) ? 1.f : 0.f;
  }
  if (tid == 0) fail = 0;
  __syncthreads();
  for (int k = 0; k < bj; ++k) {
    if (tid == 0) {
      const float p = L[k][k];
      if (!(p > 0.f)) {
        fail = 1;
        atomicCAS(info, 0, off + k + 1);
      }
      L[k][k] = sqrtf(p);
    }
    __syncthreads();
    if (fail) return;
    const float d = L[k][k];
    for (int i = k + 1 + tid; i < bj; i += 256) L[i][k] = L[i][k] / d;
    __syncthreads();
    const int m = bj - k - 1;
    for (int idx = tid; idx < m * m; idx += 256) {
      const int ii = idx / m, cc = idx % m;
      if (cc <= ii) {
        const int i = k + 1 + ii, c = k + 1 + cc;
        L[i][c] = L[i][c] - L[i][k] * L[c][k];
      }
    }
    __syncthreads();
  }
  // X = L^-1 by right-looking forward substitution on the identity
  for (int k = 0; k < bj; ++k) {
    const float d = L[k][k];
    for (int c = tid; c <= k; c += 256) X[k][c] = X[k][c] / d;
    __syncthreads();
    const int m = bj - k - 1, w = k + 1;
    for (int idx = tid; idx < m * w; idx += 256) {
      const int i = k + 1 + idx / w, c = idx % w;
      X[i][c] = X[i][c] - L[i][k] * X[k][c];
    }
    __syncthreads();
  }
  for (int idx = tid; idx < bj * bj; idx += 256) {
    const int i = idx / bj, c = idx % bj;
    const float v = c <= i ? X[i][c] : 0.f;
    D[i * NB + c] = v;
    A[(int64_t)(off + i) * lda + off + c] = v;
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

extern "C" int crbq_hinv_upper(float* H, int64_t ldh, int64_t C, float* W, int64_t R,
                               int64_t ldw, float percdamp, float* U, int64_t ldu, void* ws,
                               size_t ws_bytes, int* retries, int* fallback, void* stream) {
  if (!H || !U || C <= 0 || ldh < C || ldu < C) return CRBQ_ERR_ARG;
  if (W && (R <= 0 || ldw < C)) return CRBQ_ERR_ARG;
  if (C > (1 << 20)) return CRBQ_ERR_ARG;
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
  int nretry = 0;
  bool ok = false;
  for (int attempt = 0; attempt < 10; ++attempt) {                // bigptq.py:115-123
    k_set_int<<<1, 1, 0, s>>>(w.info, 0);
    k_reverse_lower<<<nblocks(C * C), 256, 0, s>>>(H, ldh, Ci, w.A, C);
    CRBQ_LAUNCH_CHECK();
    int st = chol_inv_sweep(w.A, C, Ci, w, s);
    if (st) return st;
    int hinfo = 0;
    CRBQ_HIP(hipMemcpyAsync(&hinfo, w.info, sizeof(int), hipMemcpyDeviceToHost, s));
    CRBQ_HIP(hipStreamSynchronize(s));
    if (hinfo == 0) { ok = true; break; }
    ++nretry;
    k_damp<<<1, 1024, 0, s>>>(H, ldh, Ci, 1e-3f, 1, w.scal);
    CRBQ_LAUNCH_CHECK();
  }
  if (ok) k_reverse_to_u<<<nblocks(C * C), 256, 0, s>>>(w.A, C, Ci, U, ldu);
  else k_fallback_u<<<nblocks(C * C), 256, 0, s>>>(H, ldh, Ci, U, ldu);
  CRBQ_LAUNCH_CHECK();
  if (retries) *retries = nretry;
  if (fallback) *fallback = ok ? 0 : 1;
  return CRBQ_OK;
}
