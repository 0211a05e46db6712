// Inverse-Hessian factor of BRAGPTQ.fasterquant (bigptq.py:101-129).
//
// The reference computes L = chol(H), H^-1 = cholesky_inverse(L) and
// U = chol(H^-1, upper) (4C^3/3 flops).  Here U comes from one factorization
// of the index-reversed matrix: with J the reversal permutation,
//   J H J = L' L'^T   =>   H^-1 = (J L'^-1 J)^T (J L'^-1 J),
// and J L'^-1 J is upper triangular with a positive diagonal, so it is U
// (the Cholesky factor is unique).  2C^3/3 flops.
//
// L'^-1 is formed recursively together with L' (block boundaries at
// multiples of NB = 128).  For A = [A11 0; A21 A22] split near the middle:
//   X11 = chol_inv(A11)                     (L11^-1, recursively)
//   T   = A21 X11^T                         (= L21, the panel of L')
//   A22 = A22 - T T^T      (lower tiles)    (Schur complement)
//   A21 = T X11                             (= L21 L11^-1)
//   X22 = chol_inv(A22)                     (recursively)
//   X21 = -X22 A21
// so X = [X11 0; X21 X22] = L'^-1 overwrites A.  Blocks of NB or fewer
// rows are factored and inverted by one workgroup (k_chol_inv_diag).  About
// 3/4 of the 2C^3/3 flops are in the four products of the top level,
// which run as large fp32 MFMA GEMMs; the triangular factors' zero halves
// are skipped.  The upper triangle of A is kept at zero so the triangular
// operands can be read as full matrices.
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

// A[i][j] = H[C-1-i][C-1-j] in the lower triangle, 0 above it
__global__ __launch_bounds__(256) void k_reverse_lower(const float* __restrict__ H, int64_t ldh,
                                                       int C, float* A, int64_t lda) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int i = (int)(idx / C), j = (int)(idx % C);
  if (i >= C) return;
  A[(int64_t)i * lda + j] = j <= i ? H[(int64_t)(C - 1 - i) * ldh + (C - 1 - j)] : 0.f;
}

// Y[r][c] = X[r][c] for an M x N block (row strides ldx, ldy)
__global__ __launch_bounds__(256) void k_copy2d(const float* __restrict__ X, int64_t ldx, int M,
                                                int N, float* Y, int64_t ldy,
                                                const int* __restrict__ stop) {
  if (*stop) return;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int r = (int)(idx / N), c = (int)(idx % N);
  if (r >= M) return;
  Y[(int64_t)r * ldy + c] = X[(int64_t)r * ldx + c];
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

// Diagonal block: Cholesky factor L and its inverse X = L^-1 of one
// bj x bj block (bj <= NB; rows past bj are padded with the identity), in
// place.  256 threads = 4 wavefronts.
//  * Factorization in LDS: the 128 columns form 16 panels of 8; panel b
//    belongs to wavefront b % 4.  The owner factors its panel in registers
//    (lane l holds rows l and l + 64; pivots broadcast with readlane) and
//    publishes it, and after one barrier every wavefront applies the
//    rank-8 update to its own later panels.
//  * Inverse: recursive doubling in LDS.  With X_A, X_C the inverses of two
//    adjacent diagonal blocks of size s and B the block below X_A,
//    X_B = -X_C (B X_A); s = 1, 2, 4, ..., 64.
// This factorization need not follow the reference's rounding step for
// step (LAPACK's blocked potrf does not either), so it uses fused
// multiply-adds and one reciprocal per pivot.
constexpr int LDP = NB + 1;            // LDS pitch of the block (column reads conflict-free)
constexpr int PANP = 12;               // LDS pitch of a panel row (8 used, 16-byte aligned)

__device__ __forceinline__ float rdlane(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

struct DiagSmem {
  float Ls[NB][LDP];
  float pan[2][NB][PANP];
  float Ts[64 * 64];
  int fail;
};

// Panel b of the factorization: the owner wavefront factors columns
// 8b..8b+7 (rows in its lanes' registers, pivots broadcast with readlane),
// every wavefront then applies the rank-8 update to its later panels in
// LDS.  Returns false after a bad pivot.
__device__ __forceinline__ bool chol_panel(int B, DiagSmem& sm, int lane, int w, int off, int bj,
                                           int* info) {
  float (*pb)[PANP] = sm.pan[B & 1];
  if (w == (B & 3)) {
    float pc[2][8];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int q = 0; q < 8; ++q) pc[s][q] = sm.Ls[lane + 64 * s][8 * B + q];
    const bool hi = B >= 8;            // the panel's diagonal rows are in slot 1
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const int c = 8 * B + p;
      const float piv = rdlane(hi ? pc[1][p] : pc[0][p], c & 63);
      if (!(piv > 0.f) && lane == 0 && c < bj) {
        sm.fail = 1;
        atomicCAS(info, 0, off + c + 1);
      }
      const float d = __builtin_amdgcn_sqrtf(piv);
      const float rd = __builtin_amdgcn_rcpf(d);
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int i = lane + 64 * s;
        pc[s][p] = i > c ? pc[s][p] * rd : (i == c ? d : 0.f);
      }
#pragma unroll
      for (int q = p + 1; q < 8; ++q) {
        const float lq = rdlane(hi ? pc[1][p] : pc[0][p], (8 * B + q) & 63);   // L[8B+q][c]
#pragma unroll
        for (int s = 0; s < 2; ++s) pc[s][q] = fmaf(-pc[s][p], lq, pc[s][q]);
      }
    }
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int i = lane + 64 * s;
#pragma unroll
      for (int q = 0; q < 8; ++q) sm.Ls[i][8 * B + q] = pc[s][q];
      *(float4*)&pb[i][0] = make_float4(pc[s][0], pc[s][1], pc[s][2], pc[s][3]);
      *(float4*)&pb[i][4] = make_float4(pc[s][4], pc[s][5], pc[s][6], pc[s][7]);
    }
  }
  __syncthreads();
  if (sm.fail) return false;
  // rank-8 update of this wavefront's later panels; rows < 64 lie above
  // every column >= 64
  float pi[2][8];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const float4 u = *(const float4*)&pb[lane + 64 * s][0];
    const float4 v = *(const float4*)&pb[lane + 64 * s][4];
    pi[s][0] = u.x; pi[s][1] = u.y; pi[s][2] = u.z; pi[s][3] = u.w;
    pi[s][4] = v.x; pi[s][5] = v.y; pi[s][6] = v.z; pi[s][7] = v.w;
  }
  for (int gb = w; gb < 16; gb += 4) {
    if (gb <= B) continue;
    // all 8 columns at once: loads first, then 16 independent FMA chains
    float pj[8][8], t0[8], t1[8];
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) {
      const int j = 8 * gb + cc;
      const float4 u = *(const float4*)&pb[j][0];
      const float4 v = *(const float4*)&pb[j][4];
      pj[cc][0] = u.x; pj[cc][1] = u.y; pj[cc][2] = u.z; pj[cc][3] = u.w;
      pj[cc][4] = v.x; pj[cc][5] = v.y; pj[cc][6] = v.z; pj[cc][7] = v.w;
      t0[cc] = sm.Ls[lane][j];
      t1[cc] = sm.Ls[lane + 64][j];
    }
#pragma unroll
    for (int q = 0; q < 8; ++q)
#pragma unroll
      for (int cc = 0; cc < 8; ++cc) {
        t0[cc] = fmaf(-pi[0][q], pj[cc][q], t0[cc]);
        t1[cc] = fmaf(-pi[1][q], pj[cc][q], t1[cc]);
      }
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) {
      sm.Ls[lane][8 * gb + cc] = t0[cc];
      sm.Ls[lane + 64][8 * gb + cc] = t1[cc];
    }
  }
  return true;
}

// one level of the recursive-doubling inverse (pairs of S x S blocks)
template <int S>
__device__ __forceinline__ void inv_level(DiagSmem& sm, int tid) {
  constexpr int NPAIR = NB / (2 * S);
  if constexpr (S < 4) {
    constexpr int NE = NPAIR * S * S;
    for (int e = tid; e < NE; e += 256) {
      const int q = e / (S * S), r = (e / S) % S, c = e % S, cb = 2 * S * q;
      float t = 0.f;
#pragma unroll
      for (int k = 0; k < S; ++k) t = fmaf(sm.Ls[cb + S + r][cb + k], sm.Ls[cb + k][cb + c], t);
      sm.Ts[e] = t;
    }
    __syncthreads();
    for (int e = tid; e < NE; e += 256) {
      const int q = e / (S * S), r = (e / S) % S, c = e % S, cb = 2 * S * q;
      float t = 0.f;
#pragma unroll
      for (int k = 0; k < S; ++k) t = fmaf(sm.Ls[cb + S + r][cb + S + k], sm.Ts[q * S * S + k * S + c], t);
      sm.Ls[cb + S + r][cb + c] = -t;
    }
    __syncthreads();
  } else if constexpr (S < 16) {
    constexpr int TPS = S / 4;                 // 4x4 tiles per block side
    constexpr int NT = NPAIR * TPS * TPS;
    // T = B X_A (X_A lower: rows k < j0 of X_A are zero in the tile's columns)
    for (int e = tid; e < NT; e += 256) {
      const int q = e / (TPS * TPS), ti = (e / TPS) % TPS, tj = e % TPS, cb = 2 * S * q;
      const int i0 = 4 * ti, j0 = 4 * tj;
      float t[4][4];
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) t[r][c] = 0.f;
#pragma unroll
      for (int k = 0; k < S; ++k) {
        float b[4], x[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) b[r] = sm.Ls[cb + S + i0 + r][cb + k];
#pragma unroll
        for (int c = 0; c < 4; ++c) x[c] = sm.Ls[cb + k][cb + j0 + c];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int c = 0; c < 4; ++c) t[r][c] = fmaf(b[r], x[c], t[r][c]);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) sm.Ts[q * S * S + (i0 + r) * S + j0 + c] = t[r][c];
    }
    __syncthreads();
    // X_B = -X_C T
    for (int e = tid; e < NT; e += 256) {
      const int q = e / (TPS * TPS), ti = (e / TPS) % TPS, tj = e % TPS, cb = 2 * S * q;
      const int i0 = 4 * ti, j0 = 4 * tj;
      const float* T = sm.Ts + q * S * S;
      float t[4][4];
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) t[r][c] = 0.f;
#pragma unroll
      for (int k = 0; k < S; ++k) {
        float xc[4], tv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) xc[r] = sm.Ls[cb + S + i0 + r][cb + S + k];
#pragma unroll
        for (int c = 0; c < 4; ++c) tv[c] = T[k * S + j0 + c];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int c = 0; c < 4; ++c) t[r][c] = fmaf(xc[r], tv[c], t[r][c]);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) sm.Ls[cb + S + i0 + r][cb + j0 + c] = -t[r][c];
    }
    __syncthreads();
  } else {
    // 16 x 16 output tiles on v_mfma_f32_16x16x4_f32, one tile per
    // wavefront at a time: lane l supplies A[l%16][k + l/16] and
    // B[k + l/16][l%16] and receives D[4*(l/16) + r][l%16], r = 0..3.
    constexpr int TPS = S / 16;
    constexpr int NT = NPAIR * TPS * TPS;
    const int lane = tid & 63, wv = tid >> 6, lr = lane & 15, lk = lane >> 4;
    for (int e = wv; e < NT; e += 4) {        // T = B X_A, k >= 16 tj
      const int q = e / (TPS * TPS), ti = (e / TPS) % TPS, tj = e % TPS, cb = 2 * S * q;
      f4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
      for (int k = 16 * tj; k < S; k += 4) {
        const float av = sm.Ls[cb + S + 16 * ti + lr][cb + k + lk];
        const float bv = sm.Ls[cb + k + lk][cb + 16 * tj + lr];
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) sm.Ts[q * S * S + (16 * ti + 4 * lk + r) * S + 16 * tj + lr] = acc[r];
    }
    __syncthreads();
    for (int e = wv; e < NT; e += 4) {        // X_B = -X_C T, k < 16 (ti + 1)
      const int q = e / (TPS * TPS), ti = (e / TPS) % TPS, tj = e % TPS, cb = 2 * S * q;
      const float* T = sm.Ts + q * S * S;
      f4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
      for (int k = 0; k < 16 * (ti + 1); k += 4) {
        const float av = sm.Ls[cb + S + 16 * ti + lr][cb + S + k + lk];
        const float bv = T[(k + lk) * S + 16 * tj + lr];
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) sm.Ls[cb + S + 16 * ti + 4 * lk + r][cb + 16 * tj + lr] = -acc[r];
    }
    __syncthreads();
  }
  if constexpr (2 * S < NB) inv_level<2 * S>(sm, tid);
}

__global__ __launch_bounds__(256) void k_chol_inv_diag(float* A, int64_t lda, int off, int bj,
                                                       int* info) {
  if (*info) return;
  __shared__ DiagSmem sm;
  // the wavefront index as a scalar, so branches on it are uniform
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  // ---- load the block (lower triangle), identity padding, zero above;
  // 16 coalesced 4-float groups per thread, all in flight together
  {
    const bool vec = ((lda & 3) == 0) && ((((uintptr_t)A) & 15) == 0);
    float v[16][4];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int f = tid + 256 * u, i = f >> 5, j0 = (f & 31) * 4;
      const float* src = A + (int64_t)(off + i) * lda + off + j0;
      if (vec && i < bj && j0 + 3 < bj) {
        const float4 q = *(const float4*)src;
        v[u][0] = q.x; v[u][1] = q.y; v[u][2] = q.z; v[u][3] = q.w;
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) v[u][c] = (i < bj && j0 + c < bj) ? src[c] : 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int f = tid + 256 * u, i = f >> 5, j0 = (f & 31) * 4;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int j = j0 + c;
        sm.Ls[i][j] = (i < bj && j <= i) ? v[u][c] : (i == j ? 1.f : 0.f);
      }
    }
  }
  if (tid == 0) sm.fail = 0;
  __syncthreads();
  // ---- factorization (L overwrites the block, zeros above the diagonal)
  for (int B = 0; B < 16; ++B)
    if (!chol_panel(B, sm, lane, w, off, bj, info)) return;
  __syncthreads();
  if (tid < NB) sm.Ls[tid][tid] = 1.f / sm.Ls[tid][tid];
  __syncthreads();
  // ---- inverse by recursive doubling
  inv_level<1>(sm, tid);
  // ---- write X (zero above the diagonal)
#pragma unroll 8
  for (int e = tid; e < NB * NB; e += 256) {
    const int i = e >> 7, j = e & (NB - 1);
    if (i < bj && j < bj) A[(int64_t)(off + i) * lda + off + j] = j <= i ? sm.Ls[i][j] : 0.f;
  }
}

static inline unsigned nblocks(int64_t n) { return (unsigned)((n + 255) / 256); }

struct HinvWs {
  float* A;        // C x C (ld = C)
  float* T;        // panel of the recursion: half x half (ld = half)
  int* info;
  float* scal;
  uint8_t* dead;   // C
};

// rows in the first half of an n-row split (a multiple of NB, >= n - it)
static inline int split_rows(int n) {
  const int nblk = (n + NB - 1) / NB;
  return (nblk + 1) / 2 * NB;
}

static void carve_hinv(WsCarver& c, int64_t C, HinvWs& w) {
  const int64_t h = C > NB ? split_rows((int)C) : 0;
  w.A = c.take<float>((size_t)C * C);
  w.T = c.take<float>((size_t)std::max<int64_t>(h * h, 1));
  w.info = c.take<int>(4);
  w.scal = c.take<float>(4);
  w.dead = c.take<uint8_t>((size_t)C);
}

// X = L^-1 of the n x n diagonal block at offset o of A (lda), in place.
// The factorization outcome is in *w.info; after a failure every later
// kernel returns at once.
static int chol_inv_rec(float* A, int64_t lda, int o, int n, HinvWs& w, hipStream_t s) {
  if (n <= NB) {
    k_chol_inv_diag<<<1, 256, 0, s>>>(A, lda, o, n, w.info);
    CRBQ_LAUNCH_CHECK();
    return CRBQ_OK;
  }
  const int m = split_rows(n), n2 = n - m;
  float* A11 = A + (int64_t)o * lda + o;
  float* A21 = A11 + (int64_t)m * lda;
  float* A22 = A21 + m;
  const int* stop = w.info;
  int st = chol_inv_rec(A, lda, o, m, w, s);
  if (st) return st;
  // T = A21 X11^T
  st = sgemm_launch(false, true, false, n2, m, m, 1.f, A21, lda, A11, lda, 0.f, w.T, m, stop, s,
                    GEMM_TRI_KEND_N);
  if (st) return st;
  // A22 -= T T^T (lower tiles)
  st = sgemm_launch(false, true, true, n2, n2, m, -1.f, w.T, m, w.T, m, 1.f, A22, lda, stop, s);
  if (st) return st;
  // A21 = T X11
  st = sgemm_launch(false, false, false, n2, m, m, 1.f, w.T, m, A11, lda, 0.f, A21, lda, stop, s,
                    GEMM_TRI_KBEG_N);
  if (st) return st;
  st = chol_inv_rec(A, lda, o + m, n2, w, s);
  if (st) return st;
  // X21 = -X22 A21, through T
  st = sgemm_launch(false, false, false, n2, m, n2, -1.f, A22, lda, A21, lda, 0.f, w.T, m, stop,
                    s, GEMM_TRI_KEND_M);
  if (st) return st;
  k_copy2d<<<nblocks((int64_t)n2 * m), 256, 0, s>>>(w.T, m, n2, m, A21, lda, stop);
  CRBQ_LAUNCH_CHECK();
  return CRBQ_OK;
}

// One full attempt: factor and invert A in place.  Returns a launch status;
// the factorization outcome is in *w.info.
static int chol_inv_sweep(float* A, int64_t lda, int C, HinvWs& w, hipStream_t s) {
  return chol_inv_rec(A, lda, 0, C, w, s);
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
