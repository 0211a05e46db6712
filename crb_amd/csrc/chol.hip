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
//   A21 = T X11                             (= L21 L11^-1; one launch with
//                                            the Schur update)
//   X22 = chol_inv(A22)                     (recursively)
//   X21 = -X22 A21
// so X = [X11 0; X21 X22] = L'^-1 overwrites A.  Blocks of NB or fewer
// rows are factored and inverted by one workgroup (k_chol_inv_diag), nodes
// of up to 2 NB rows, all five steps, by one workgroup too
// (k_chol_inv_node).  About
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

__global__ __launch_bounds__(256) void k_zero_dead(float* W, int64_t ldw, int R, int C,
                                                   const uint8_t* __restrict__ dead) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)R * C) return;
  const int c = (int)(idx % C);
  if (dead[c]) W[(idx / C) * ldw + c] = 0.f;    // bigptq.py:105
}

// H_ii += factor * mean(diag H); retry mode: 1e-6 when that is 0.
// dead (optional): first the dead columns, H_ii == 0, flagged and set to 1
// (the mean sees the 1s).  info (optional): the factorization's failure
// flag, cleared.  One workgroup; thread t handles the entries i = t + 1024 u
// in ascending u, DG of them per round loaded together (each is a row
// stride from the last, one cache line apart), few registers so the
// workgroup finds room beside other kernels' waves.  The sum: per thread in
// ascending i in fp64, then a fixed tree over the threads.
constexpr int DG = 4;
__global__ __launch_bounds__(1024) void k_damp(float* H, int64_t ldh, int C, float factor,
                                               int retry, float* out, uint8_t* dead,
                                               int* info) {
  __shared__ double red[1024];
  const int tid = threadIdx.x;
  const int64_t step = ldh + 1;
  if (info && tid == 0) *info = 0;
  double s = 0.0;
  for (int i0 = tid; i0 < C; i0 += 1024 * DG) {
    float v[DG];
#pragma unroll
    for (int u = 0; u < DG; ++u) {
      const int i = i0 + 1024 * u;
      v[u] = i < C ? H[(int64_t)i * step] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < DG; ++u) {
      const int i = i0 + 1024 * u;
      if (i < C) {
        if (dead) {
          const bool d = v[u] == 0.f;           // bigptq.py:103-104
          dead[i] = d;
          if (d) {
            v[u] = 1.f;
            H[(int64_t)i * step] = 1.f;
          }
        }
        s += (double)v[u];
      }
    }
  }
  red[tid] = s;
  __syncthreads();
  for (int o = 512; o > 0; o >>= 1) {
    if (tid < o) red[tid] += red[tid + o];
    __syncthreads();
  }
  const float mean = (float)red[0] / (float)C;
  float v = factor * mean;
  if (retry && v == 0.f) v = 1e-6f;             // bigptq.py:120-121
  for (int i0 = tid; i0 < C; i0 += 1024 * DG) {
    float h[DG];
#pragma unroll
    for (int u = 0; u < DG; ++u) {
      const int i = i0 + 1024 * u;
      h[u] = i < C ? H[(int64_t)i * step] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < DG; ++u) {
      const int i = i0 + 1024 * u;
      if (i < C) H[(int64_t)i * step] = h[u] + v;
    }
  }
  if (tid == 0 && out) *out = v;
}

__global__ void k_set_int(int* p, int v) { *p = v; }

// Grid of the row-wise copies below: x = row, y = 1024-column chunk.
static inline dim3 rows_grid(int64_t C) {
  return dim3((unsigned)C, (unsigned)((C + 1023) / 1024));
}

// Row i of the index-reversed copy: Y[i][j] = X[C-1-i][C-1-j] where keep(i, j)
// holds, 0 elsewhere (rows_grid).  With vec (C, the row strides and both
// bases multiples of 4 floats) each thread moves 4 consecutive j with one
// 16-byte load of the source row (columns C-4-j .. C-1-j, reversed) and one
// 16-byte store; runs wholly outside keep skip the load.
template <bool LOWER>
__device__ __forceinline__ void reverse_row(const float* __restrict__ X, int64_t ldx, int C,
                                            float* Y, int64_t ldy, bool vec) {
  const int i = blockIdx.x;
  const float* x = X + (int64_t)(C - 1 - i) * ldx;
  float* y = Y + (int64_t)i * ldy;
  auto keep = [i](int j) { return LOWER ? j <= i : j >= i; };
  if (vec) {
    const int j0 = blockIdx.y * 1024 + threadIdx.x * 4;
    if (j0 >= C) return;
    float4 q = make_float4(0.f, 0.f, 0.f, 0.f);
    if (keep(j0) || keep(j0 + 3)) {
      const float4 v = *(const float4*)(x + (C - 4 - j0));
      q = make_float4(keep(j0) ? v.w : 0.f, keep(j0 + 1) ? v.z : 0.f, keep(j0 + 2) ? v.y : 0.f,
                      keep(j0 + 3) ? v.x : 0.f);
    }
    *(float4*)(y + j0) = q;
    return;
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int j = blockIdx.y * 1024 + k * 256 + threadIdx.x;
    if (j < C) y[j] = keep(j) ? x[C - 1 - j] : 0.f;
  }
}
static inline bool reverse_vec(const float* X, int64_t ldx, int64_t C, const float* Y,
                               int64_t ldy) {
  return (C & 3) == 0 && ((ldx | ldy) & 3) == 0 && ((((uintptr_t)X) | ((uintptr_t)Y)) & 15) == 0;
}

// A[i][j] = H[C-1-i][C-1-j] in the lower triangle, 0 above it (rows_grid)
__global__ __launch_bounds__(256) void k_reverse_lower(const float* __restrict__ H, int64_t ldh,
                                                       int C, float* A, int64_t lda, int vec) {
  reverse_row<true>(H, ldh, C, A, lda, vec != 0);
}

// U[i][j] = X[C-1-i][C-1-j] for j >= i, 0 below the diagonal (rows_grid)
__global__ __launch_bounds__(256) void k_reverse_to_u(const float* __restrict__ X, int64_t ldx,
                                                      int C, float* U, int64_t ldu, int vec) {
  reverse_row<false>(X, ldx, C, U, ldu, vec != 0);
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
// place in LDS.  256 threads = 4 wavefronts.  The block is split
// recursively like the whole matrix (X11, T = A21 X11^T, A22 -= T T^T,
// A21 = T X11, X22, X21 = -X22 A21):
//  * 16 x 16 leaves: one wavefront, lane i & 15 holding row i in
//    registers; Cholesky by columns and the inverse by right-looking
//    forward substitution, the values other lanes hold taken by DPP row
//    broadcasts fused into the fma (v_fmac_f32_dpp).
//  * 32 x 32 blocks: one wavefront runs both leaves and the four 16 x 16
//    products (v_mfma_f32_16x16x4f32), so no workgroup barrier is needed.
//  * the 64 and 128 levels: the products' 16 x 16 output tiles are spread
//    over the 4 wavefronts, one barrier between dependent products.
// This factorization need not follow the reference's rounding step for
// step (LAPACK's blocked potrf does not either), so it uses fused
// multiply-adds and hardware square root and reciprocal per pivot.
constexpr int LDP = NB + 1;            // LDS pitch of the block (column reads conflict-free)
constexpr int TSP = NB / 2 + 1;        // LDS pitch of the product scratch T

struct DiagSmem {
  float Ls[NB][LDP];
  float Ts[(NB / 2) * TSP];
  int fail;
};

// Orders one wavefront's LDS accesses on both sides (lanes exchange data
// through LDS between the phases of a single-wavefront block).
__device__ __forceinline__ void wave_lds_sync() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

__device__ __forceinline__ f4_t mfma4(float a, float b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Value of lane L of each 16-lane row in every lane of that row (DPP
// row_newbcast).  In the leaves the four rows of a wavefront hold the same
// data, so this is lane L's value in VGPRs, with no scalar registers.
// bound_ctrl set: every lane's source lane is valid, so the old value is
// never read and no zero needs to be moved into the destination first.
template <int L>
__device__ __forceinline__ float row_bcast(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x150 + L, 0xf, 0xf,
                                                    true));
}
__device__ __forceinline__ float row_bcast(float v, int l) {   // l is a constant after unrolling
  switch (l) {
    case 0: return row_bcast<0>(v);   case 1: return row_bcast<1>(v);
    case 2: return row_bcast<2>(v);   case 3: return row_bcast<3>(v);
    case 4: return row_bcast<4>(v);   case 5: return row_bcast<5>(v);
    case 6: return row_bcast<6>(v);   case 7: return row_bcast<7>(v);
    case 8: return row_bcast<8>(v);   case 9: return row_bcast<9>(v);
    case 10: return row_bcast<10>(v); case 11: return row_bcast<11>(v);
    case 12: return row_bcast<12>(v); case 13: return row_bcast<13>(v);
    case 14: return row_bcast<14>(v); default: return row_bcast<15>(v);
  }
}

// d - (lane L of s's row) * m as one v_fmac_f32 whose first source is the
// row broadcast (DPP row_newbcast, negated): the same fma as
// fmaf(-row_bcast<L>(s), m, d), one instruction instead of two.  A DPP
// read of a VGPR needs two wait states after the VALU instruction that
// wrote it, and the compiler's hazard recognizer does not look inside asm:
// NB puts them before the instruction (s was just written), NA after it (a
// compiler-generated DPP read of d follows).
// The wait states sit in the same asm statement as the DPP instruction, so
// the scheduler cannot move the write in between.
#define CRBQ_FMAC_BCAST "v_fmac_f32_dpp %0, -%1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf bound_ctrl:1"
template <int L, bool NB, bool NA>
__device__ __forceinline__ float fnma_row_bcast(float d, float s, float m) {
  if (NB && NA)
    asm volatile("s_nop 1\n\t" CRBQ_FMAC_BCAST "\n\ts_nop 1" : "+v"(d) : "v"(s), "v"(m), "n"(L));
  else if (NB)
    asm volatile("s_nop 1\n\t" CRBQ_FMAC_BCAST : "+v"(d) : "v"(s), "v"(m), "n"(L));
  else if (NA)
    asm volatile(CRBQ_FMAC_BCAST "\n\ts_nop 1" : "+v"(d) : "v"(s), "v"(m), "n"(L));
  else
    asm volatile(CRBQ_FMAC_BCAST : "+v"(d) : "v"(s), "v"(m), "n"(L));
  return d;
}
#undef CRBQ_FMAC_BCAST
template <bool NB, bool NA>
__device__ __forceinline__ float fnma_row_bcast(float d, float s, float m, int l) {
  switch (l) {   // l is a constant after unrolling
    case 0: return fnma_row_bcast<0, NB, NA>(d, s, m);
    case 1: return fnma_row_bcast<1, NB, NA>(d, s, m);
    case 2: return fnma_row_bcast<2, NB, NA>(d, s, m);
    case 3: return fnma_row_bcast<3, NB, NA>(d, s, m);
    case 4: return fnma_row_bcast<4, NB, NA>(d, s, m);
    case 5: return fnma_row_bcast<5, NB, NA>(d, s, m);
    case 6: return fnma_row_bcast<6, NB, NA>(d, s, m);
    case 7: return fnma_row_bcast<7, NB, NA>(d, s, m);
    case 8: return fnma_row_bcast<8, NB, NA>(d, s, m);
    case 9: return fnma_row_bcast<9, NB, NA>(d, s, m);
    case 10: return fnma_row_bcast<10, NB, NA>(d, s, m);
    case 11: return fnma_row_bcast<11, NB, NA>(d, s, m);
    case 12: return fnma_row_bcast<12, NB, NA>(d, s, m);
    case 13: return fnma_row_bcast<13, NB, NA>(d, s, m);
    case 14: return fnma_row_bcast<14, NB, NA>(d, s, m);
    default: return fnma_row_bcast<15, NB, NA>(d, s, m);
  }
}

// 16 x 16 leaf at (o, o): L = chol(A), then X = L^-1 written over it (zeros
// above the diagonal).  One wavefront; each 16-lane row repeats lanes 0..15.
//  * Cholesky with lane i holding row i: at column j the pivot comes from
//    lane j and L[k][j] from lane k (row broadcasts); lanes i <= j keep
//    scratch in column j, never read.
//  * Inverse with lane c holding column c of X: forward substitution
//    X[r][c] = (delta_rc - sum_{k<r} L[r][k] X[k][c]) / L[r][r], the L
//    values broadcast from lane r, so no lane masks are needed.
__device__ __forceinline__ void leaf16(DiagSmem& sm, int o, int lane, int off, int bj,
                                       int* info) {
  const int i = lane & 15;
  float a[16], rdg[16];
#pragma unroll
  for (int c = 0; c < 16; ++c) a[c] = sm.Ls[o + i][o + c];
  unsigned badm = 0u;   // bad pivots as bits (the same in every lane)
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const float piv = row_bcast(a[j], j);
    badm |= (!(piv > 0.f) && o + j < bj) ? (1u << j) : 0u;
    const float rd = __builtin_amdgcn_rcpf(__builtin_amdgcn_sqrtf(piv));
    rdg[j] = rd;
    a[j] *= rd;
    // a[k] -= L[i][j] L[k][j]; the first update reads a[j] right after its
    // scaling, and the next column's pivot reads a[j + 1] (written by the
    // first update) at most two updates later
#pragma unroll
    for (int k = j + 1; k < 16; ++k) {
      if (k == j + 1 && k == 15) a[k] = fnma_row_bcast<true, true>(a[k], a[j], a[j], k);
      else if (k == j + 1) a[k] = fnma_row_bcast<true, false>(a[k], a[j], a[j], k);
      else if (k == 15) a[k] = fnma_row_bcast<false, true>(a[k], a[j], a[j], k);
      else a[k] = fnma_row_bcast<false, false>(a[k], a[j], a[j], k);
    }
  }
  const unsigned bm = __builtin_amdgcn_readfirstlane(badm);
  const int bad = bm ? __builtin_ctz(bm) : 16;   // first bad pivot
  if (bad < 16 && lane == 0) {
    sm.fail = 1;
    atomicCAS(info, 0, off + o + bad + 1);
  }
  // right-looking: once y[r] is known every later row's accumulator takes
  // its term, so each accumulator receives k = 0, 1, ... in the same order
  // as a row-by-row dot product would, while the dependent chain is one
  // multiply and one fma per row
  float y[16], acc[16];
#pragma unroll
  for (int s = 0; s < 16; ++s) acc[s] = i == s ? 1.f : 0.f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    y[r] = acc[r] * rdg[r];
#pragma unroll
    for (int s = r + 1; s < 16; ++s) acc[s] = fnma_row_bcast<false, false>(acc[s], a[r], y[r], s);
  }
  if (lane < 16) {
#pragma unroll
    for (int r = 0; r < 16; ++r) sm.Ls[o + r][o + i] = y[r];
  }
}

// 32 x 32 block at (o, o) by one wavefront: lane l supplies A[l%16][k + l/16]
// and B[k + l/16][l%16] to each MFMA and receives D[4*(l/16) + r][l%16].
__device__ __forceinline__ void block32(DiagSmem& sm, int o, int lane, int off, int bj,
                                        int* info) {
  const int lr = lane & 15, lk = lane >> 4, p = o + 16;
  leaf16(sm, o, lane, off, bj, info);
  wave_lds_sync();
  f4_t t = {0.f, 0.f, 0.f, 0.f};              // T = A21 X11^T
#pragma unroll
  for (int k = 0; k < 16; k += 4) t = mfma4(sm.Ls[p + lr][o + k + lk], sm.Ls[o + lr][o + k + lk], t);
#pragma unroll
  for (int r = 0; r < 4; ++r) sm.Ts[(4 * lk + r) * TSP + lr] = t[r];
  wave_lds_sync();
  f4_t s = {0.f, 0.f, 0.f, 0.f}, u = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < 16; k += 4) {
    const float tv = sm.Ts[lr * TSP + k + lk];
    s = mfma4(tv, tv, s);                      // T T^T
    u = mfma4(tv, sm.Ls[o + k + lk][o + lr], u);   // T X11
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int rr = 4 * lk + r;
    if (lr <= rr) sm.Ls[p + rr][p + lr] -= s[r];
    sm.Ls[p + rr][o + lr] = u[r];
  }
  wave_lds_sync();
  leaf16(sm, p, lane, off, bj, info);
  wave_lds_sync();
  f4_t x = {0.f, 0.f, 0.f, 0.f};              // X21 = -X22 A21
#pragma unroll
  for (int k = 0; k < 16; k += 4) x = mfma4(sm.Ls[p + lr][p + k + lk], sm.Ls[p + k + lk][o + lr], x);
#pragma unroll
  for (int r = 0; r < 4; ++r) sm.Ls[p + 4 * lk + r][o + lr] = -x[r];
  wave_lds_sync();
}

// Lower-triangle tile e (row-major over ti >= tj) of an NTL x NTL tile grid.
__device__ __forceinline__ void lower_tile(int e, int& ti, int& tj) {
  ti = 0;
  while ((ti + 1) * (ti + 2) / 2 <= e) ++ti;
  tj = e - ti * (ti + 1) / 2;
}

// The products of a level with H-row halves at (o, o), 16 x 16 tiles over
// the 4 wavefronts.  Full-depth products (the triangular operands' zero
// halves included) so that every operand read of a tile can be issued
// before its MFMA chain, with a wavefront's tiles interleaved.  Ends with a
// barrier.
template <int H>
__device__ __forceinline__ void level_panel(DiagSmem& sm, int o, int wv, int lane) {
  constexpr int NTL = H / 16, TPW = NTL * NTL / 4, NL = NTL * (NTL + 1) / 2;
  constexpr int LPW = (NL + 3) / 4;
  const int lr = lane & 15, lk = lane >> 4, p = o + H;
  {                                            // T = A21 X11^T
    f4_t t[TPW];
    int ti[TPW], tj[TPW];
#pragma unroll
    for (int q = 0; q < TPW; ++q) {
      ti[q] = (wv + 4 * q) / NTL;
      tj[q] = (wv + 4 * q) % NTL;
      t[q] = f4_t{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int k = 0; k < H; k += 4)
#pragma unroll
      for (int q = 0; q < TPW; ++q)
        t[q] = mfma4(sm.Ls[p + 16 * ti[q] + lr][o + k + lk],
                     sm.Ls[o + 16 * tj[q] + lr][o + k + lk], t[q]);
#pragma unroll
    for (int q = 0; q < TPW; ++q)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        sm.Ts[(16 * ti[q] + 4 * lk + r) * TSP + 16 * tj[q] + lr] = t[q][r];
  }
  __syncthreads();
  {                                            // A22 -= T T^T (lower tiles)
    f4_t s[LPW];
    int ti[LPW], tj[LPW];
#pragma unroll
    for (int q = 0; q < LPW; ++q) {
      const int e = wv + 4 * q;
      lower_tile(e < NL ? e : NL - 1, ti[q], tj[q]);
      s[q] = f4_t{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int k = 0; k < H; k += 4)
#pragma unroll
      for (int q = 0; q < LPW; ++q)
        s[q] = mfma4(sm.Ts[(16 * ti[q] + lr) * TSP + k + lk],
                     sm.Ts[(16 * tj[q] + lr) * TSP + k + lk], s[q]);
    f4_t u[TPW];                               // A21 = T X11
    int ui[TPW], uj[TPW];
#pragma unroll
    for (int q = 0; q < TPW; ++q) {
      ui[q] = (wv + 4 * q) / NTL;
      uj[q] = (wv + 4 * q) % NTL;
      u[q] = f4_t{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int k = 0; k < H; k += 4)
#pragma unroll
      for (int q = 0; q < TPW; ++q)
        u[q] = mfma4(sm.Ts[(16 * ui[q] + lr) * TSP + k + lk],
                     sm.Ls[o + k + lk][o + 16 * uj[q] + lr], u[q]);
#pragma unroll
    for (int q = 0; q < LPW; ++q) {
      if (wv + 4 * q < NL) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int rr = 16 * ti[q] + 4 * lk + r, cc = 16 * tj[q] + lr;
          if (cc <= rr) sm.Ls[p + rr][p + cc] -= s[q][r];
        }
      }
    }
#pragma unroll
    for (int q = 0; q < TPW; ++q)
#pragma unroll
      for (int r = 0; r < 4; ++r) sm.Ls[p + 16 * ui[q] + 4 * lk + r][o + 16 * uj[q] + lr] = u[q][r];
  }
  __syncthreads();
}

// X21 = -X22 A21 of a level (full depth, as above); results are held in
// registers until every wavefront has read A21.  Ends with a barrier.
template <int H>
__device__ __forceinline__ void level_x21(DiagSmem& sm, int o, int wv, int lane) {
  constexpr int NTL = H / 16, TPW = NTL * NTL / 4;
  const int lr = lane & 15, lk = lane >> 4, p = o + H;
  f4_t x[TPW];
  int ti[TPW], tj[TPW];
#pragma unroll
  for (int q = 0; q < TPW; ++q) {
    ti[q] = (wv + 4 * q) / NTL;
    tj[q] = (wv + 4 * q) % NTL;
    x[q] = f4_t{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int k = 0; k < H; k += 4)
#pragma unroll
    for (int q = 0; q < TPW; ++q)
      x[q] = mfma4(sm.Ls[p + 16 * ti[q] + lr][p + k + lk], sm.Ls[p + k + lk][o + 16 * tj[q] + lr],
                   x[q]);
  __syncthreads();
#pragma unroll
  for (int q = 0; q < TPW; ++q)
#pragma unroll
    for (int r = 0; r < 4; ++r) sm.Ls[p + 16 * ti[q] + 4 * lk + r][o + 16 * tj[q] + lr] = -x[q][r];
  __syncthreads();
}

// 64 x 64 block at (o, o).  Returns false after a bad pivot (uniformly).
__device__ __forceinline__ bool block64(DiagSmem& sm, int o, int wv, int lane, int off, int bj,
                                        int* info) {
  if (wv == 0) block32(sm, o, lane, off, bj, info);
  __syncthreads();
  if (sm.fail) return false;
  level_panel<32>(sm, o, wv, lane);
  if (wv == 0) block32(sm, o + 32, lane, off, bj, info);
  __syncthreads();
  if (sm.fail) return false;
  level_x21<32>(sm, o, wv, lane);
  return true;
}

// Load the bj x bj diagonal block at (off, off) into sm.Ls: lower triangle,
// identity padding, zero above; 16 coalesced 4-float groups per thread,
// all in flight together.  Ends with a barrier.
__device__ __forceinline__ void diag_load(DiagSmem& sm, const float* A, int64_t lda, int off,
                                          int bj, bool vec) {
  const int tid = threadIdx.x;
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
  if (tid == 0) sm.fail = 0;
  __syncthreads();
}

// X = L^-1 of the block in sm.Ls (L is not kept).  Returns false after a
// bad pivot (uniformly; *info is set).
__device__ __forceinline__ bool diag_core(DiagSmem& sm, int w, int lane, int off, int bj,
                                          int* info) {
  if (!block64(sm, 0, w, lane, off, bj, info)) return false;
  level_panel<64>(sm, 0, w, lane);
  if (!block64(sm, 64, w, lane, off, bj, info)) return false;
  level_x21<64>(sm, 0, w, lane);
  return true;
}

// Write X (zero above the diagonal) back to the block, 16-byte stores where
// aligned.
__device__ __forceinline__ void diag_store(const DiagSmem& sm, float* A, int64_t lda, int off,
                                           int bj, bool vec) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const int f = tid + 256 * u, i = f >> 5, j0 = (f & 31) * 4;
    float* dst = A + (int64_t)(off + i) * lda + off + j0;
    float q[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) q[c] = j0 + c <= i ? sm.Ls[i][j0 + c] : 0.f;
    if (vec && i < bj && j0 + 3 < bj) {
      *(float4*)dst = make_float4(q[0], q[1], q[2], q[3]);
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (i < bj && j0 + c < bj) dst[c] = q[c];
    }
  }
}

__device__ __forceinline__ bool diag_vec(const float* A, int64_t lda, int off) {
  return ((lda & 3) == 0) && ((((uintptr_t)A) & 15) == 0) && ((off & 3) == 0);
}

__global__ __launch_bounds__(256) void k_chol_inv_diag(float* A, int64_t lda, int off, int bj,
                                                       int* info) {
  if (*info) return;
  __shared__ DiagSmem sm;
  // the wavefront index as a scalar, so branches on it are uniform
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool vec = diag_vec(A, lda, off);
  diag_load(sm, A, lda, off, bj, vec);
  if (!diag_core(sm, w, lane, off, bj, info)) return;
  diag_store(sm, A, lda, off, bj, vec);
}

// A node of 129 to 256 rows in one workgroup: the recursion's five steps
// for a split at m = 128 (n2 = n - 128 rows in the second half)
//   X11 = chol_inv(A11)                     (diagonal block in LDS)
//   T   = A21 X11^T                         (A21 staged in LDS, T over it)
//   A22 -= T T^T, Q = T X11                 (Q over T; A22 loaded into the
//                                            block buffer, S subtracted there)
//   X22 = chol_inv(A22)
//   X21 = -X22 Q                            (written over A21)
// instead of five launches, each of which waits for a free CU when other
// work holds them.  The products are 16 x 16 MFMA tiles over k in
// ascending steps of 4 with the same operands as the GEMM launches they
// replace (v_mfma_f32_16x16x4_f32, lane l supplying row l % 16 at k + l / 16)
// and the same epilogues (T = acc, Q = acc, A22 = A22 - acc, X21 = -acc), so
// X is bitwise what those launches give; the zero parts of the triangular
// operands are skipped (exact zeros leave the sums unchanged).  Tiles go
// to the 4 wavefronts in pairs of a short and a long K range (tile
// columns or rows w and 7 - w), so every wavefront issues the same number
// of MFMAs.
struct NodeSmem {
  DiagSmem d;                // the diagonal block (X11, then A22 / X22)
  float P[NB][LDP];          // A21, then T, then Q
};

__global__ __launch_bounds__(256) void k_chol_inv_node(float* A, int64_t lda, int off, int n,
                                                       int* info) {
  if (*info) return;
  __shared__ NodeSmem nm;
  DiagSmem& sm = nm.d;
  float (*P)[LDP] = nm.P;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lk = lane >> 4;
  const int n2 = n - NB;                          // 1 .. 128
  const bool vec = diag_vec(A, lda, off);
  // ---- X11
  diag_load(sm, A, lda, off, NB, vec);
  if (!diag_core(sm, w, lane, off, NB, info)) return;
  diag_store(sm, A, lda, off, NB, vec);
  // ---- A21 (n2 x 128) into P, zero rows past n2
  float* A21 = A + (int64_t)(off + NB) * lda + off;
  {
    float v[16][4];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int f = tid + 256 * u, i = f >> 5, j0 = (f & 31) * 4;
      const float* src = A21 + (int64_t)i * lda + j0;
      if (vec && i < n2) {
        const float4 q = *(const float4*)src;
        v[u][0] = q.x; v[u][1] = q.y; v[u][2] = q.z; v[u][3] = q.w;
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) v[u][c] = i < n2 ? src[c] : 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int f = tid + 256 * u, i = f >> 5, j0 = (f & 31) * 4;
#pragma unroll
      for (int c = 0; c < 4; ++c) P[i][j0 + c] = v[u][c];
    }
  }
  __syncthreads();
  // wavefront w's tile columns (T, Q) or rows (X21): w and 7 - w, 8 tiles each
  const int ca = w, cb = 7 - w;
  // ---- T = A21 X11^T: column tile j sums k < 16 (j + 1)
  {
    f4_t ta[8], tb[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) { ta[i] = f4_t{0.f, 0.f, 0.f, 0.f}; tb[i] = ta[i]; }
    const int ka = 16 * (ca + 1), kb = 16 * (cb + 1);   // ka < kb
    for (int k = 0; k < kb; k += 4) {
      const float ba = sm.Ls[16 * ca + lr][k + lk], bb = sm.Ls[16 * cb + lr][k + lk];
      float a[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) a[i] = P[16 * i + lr][k + lk];
      if (k < ka) {
#pragma unroll
        for (int i = 0; i < 8; ++i) ta[i] = mfma4(a[i], ba, ta[i]);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) tb[i] = mfma4(a[i], bb, tb[i]);
    }
    __syncthreads();                              // every read of A21 done
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        P[16 * i + 4 * lk + r][16 * ca + lr] = ta[i][r];
        P[16 * i + 4 * lk + r][16 * cb + lr] = tb[i][r];
      }
  }
  __syncthreads();
  // ---- S = T T^T (the 36 lower tiles, full K) and Q = T X11 (column tile j
  // sums k >= 16 j)
  f4_t sacc[9];
  int si[9], sj[9];
#pragma unroll
  for (int q = 0; q < 9; ++q) {
    lower_tile(w + 4 * q, si[q], sj[q]);
    sacc[q] = f4_t{0.f, 0.f, 0.f, 0.f};
  }
  for (int k = 0; k < NB; k += 4) {
#pragma unroll
    for (int q = 0; q < 9; ++q)
      sacc[q] = mfma4(P[16 * si[q] + lr][k + lk], P[16 * sj[q] + lr][k + lk], sacc[q]);
  }
  f4_t ua[8], ub[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) { ua[i] = f4_t{0.f, 0.f, 0.f, 0.f}; ub[i] = ua[i]; }
  {
    const int ka = 16 * ca, kb = 16 * cb;         // start of the K range; ka < kb
    for (int k = ka; k < NB; k += 4) {
      const float ba = sm.Ls[k + lk][16 * ca + lr], bb = sm.Ls[k + lk][16 * cb + lr];
      float a[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) a[i] = P[16 * i + lr][k + lk];
#pragma unroll
      for (int i = 0; i < 8; ++i) ua[i] = mfma4(a[i], ba, ua[i]);
      if (k >= kb) {
#pragma unroll
        for (int i = 0; i < 8; ++i) ub[i] = mfma4(a[i], bb, ub[i]);
      }
    }
  }
  __syncthreads();                                // every read of T and X11 done
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      P[16 * i + 4 * lk + r][16 * ca + lr] = ua[i][r];
      P[16 * i + 4 * lk + r][16 * cb + lr] = ub[i][r];
    }
  // ---- A22 - S into the block buffer (rows and columns past n2: identity
  // padding, where S is 0), then X22
  diag_load(sm, A, lda, off + NB, n2, vec);       // ends with a barrier
#pragma unroll
  for (int q = 0; q < 9; ++q)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int rr = 16 * si[q] + 4 * lk + r, cc = 16 * sj[q] + lr;
      if (cc <= rr) sm.Ls[rr][cc] = sm.Ls[rr][cc] - sacc[q][r];
    }
  __syncthreads();
  if (!diag_core(sm, w, lane, off + NB, n2, info)) return;
  diag_store(sm, A, lda, off + NB, n2, vec);
  // ---- X21 = -X22 Q: row tile i sums k < 16 (i + 1)
  {
    f4_t xa[8], xb[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) { xa[j] = f4_t{0.f, 0.f, 0.f, 0.f}; xb[j] = xa[j]; }
    const int ra = ca, rb = cb;
    const int ka = 16 * (ra + 1), kb = 16 * (rb + 1);
    for (int k = 0; k < kb; k += 4) {
      const float aa = sm.Ls[16 * ra + lr][k + lk], ab = sm.Ls[16 * rb + lr][k + lk];
      float b[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) b[j] = P[k + lk][16 * j + lr];
      if (k < ka) {
#pragma unroll
        for (int j = 0; j < 8; ++j) xa[j] = mfma4(aa, b[j], xa[j]);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) xb[j] = mfma4(ab, b[j], xb[j]);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int ia = 16 * ra + 4 * lk + r, ib = 16 * rb + 4 * lk + r, c = 16 * j + lr;
        if (ia < n2) A21[(int64_t)ia * lda + c] = -xa[j][r];
        if (ib < n2) A21[(int64_t)ib * lda + c] = -xb[j][r];
      }
  }
}

static inline unsigned nblocks(int64_t n) { return (unsigned)((n + 255) / 256); }

struct HinvWs {
  float* A;        // C x C (ld = C)
  float* T;        // panel of the recursion: half x half (ld = half)
  float* Q;        // A21 X11 of every node on the current recursion path (q_floats)
  int* info;
  float* scal;
  uint8_t* dead;   // C
};

// rows in the first half of an n-row split (a multiple of NB, >= n - it)
static inline int split_rows(int n) {
  const int nblk = (n + NB - 1) / NB;
  return (nblk + 1) / 2 * NB;
}

// Floats of Q an n-row node needs: its own n2 x m product, held while the
// X22 recursion runs, stacked on what that recursion needs (the X11
// recursion runs before it and reuses the same space).
static int64_t q_floats(int64_t n) {
  if (n <= NB) return 0;
  const int64_t m = split_rows((int)n), n2 = n - m;
  return std::max(q_floats(m), n2 * m + q_floats(n2));
}

static void carve_hinv(WsCarver& c, int64_t C, HinvWs& w) {
  const int64_t h = C > NB ? split_rows((int)C) : 0;
  w.A = c.take<float>((size_t)C * C);
  w.T = c.take<float>((size_t)std::max<int64_t>(h * h, 1));
  w.Q = c.take<float>((size_t)std::max<int64_t>(q_floats(C), 1));
  w.info = c.take<int>(4);
  w.scal = c.take<float>(4);
  w.dead = c.take<uint8_t>((size_t)C);
}

// X = L^-1 of the n x n diagonal block at offset o of A (lda), in place.
// Q: q_floats(n) floats of scratch.  The factorization outcome is in
// *w.info; after a failure every later kernel returns at once.
static int chol_inv_rec(float* A, int64_t lda, int o, int n, HinvWs& w, float* Q,
                        hipStream_t s) {
  if (n <= NB) {
    k_chol_inv_diag<<<1, 256, 0, s>>>(A, lda, o, n, w.info);
    CRBQ_LAUNCH_CHECK();
    return CRBQ_OK;
  }
  if (n <= 2 * NB) {                  // split at NB: the whole node in one workgroup
    k_chol_inv_node<<<1, 256, 0, s>>>(A, lda, o, n, w.info);
    CRBQ_LAUNCH_CHECK();
    return CRBQ_OK;
  }
  const int m = split_rows(n), n2 = n - m;
  float* A11 = A + (int64_t)o * lda + o;
  float* A21 = A11 + (int64_t)m * lda;
  float* A22 = A21 + m;
  const int* stop = w.info;
  int st = chol_inv_rec(A, lda, o, m, w, Q, s);
  if (st) return st;
  // T = A21 X11^T
  st = sgemm_launch(false, true, false, n2, m, m, 1.f, A21, lda, A11, lda, 0.f, w.T, m, stop, s,
                    GEMM_TRI_KEND_N);
  if (st) return st;
  // A22 -= T T^T (lower tiles) and Q = T X11 (A21 is dead after T; X21
  // will go there), in one launch: both only read T and X11
  {
    const GemmArgs schur = {false, true, true, n2, n2, m, -1.f, w.T, m, w.T, m, 1.f, A22, lda,
                            GEMM_TRI_NONE};
    const GemmArgs q = {false, false, false, n2, m, m, 1.f, w.T, m, A11, lda, 0.f, Q, m,
                        GEMM_TRI_KBEG_N};
    st = sgemm2_launch(schur, q, stop, s);
    if (st) return st;
  }
  st = chol_inv_rec(A, lda, o + m, n2, w, Q + (int64_t)n2 * m, s);
  if (st) return st;
  // X21 = -X22 Q
  return sgemm_launch(false, false, false, n2, m, n2, -1.f, A22, lda, Q, m, 0.f, A21, lda, stop,
                      s, GEMM_TRI_KEND_M);
}

// One full attempt: factor and invert A in place.  Returns a launch status;
// the factorization outcome is in *w.info.
static int chol_inv_sweep(float* A, int64_t lda, int C, HinvWs& w, hipStream_t s) {
  return chol_inv_rec(A, lda, 0, C, w, w.Q, s);
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
  // dead columns, damping (bigptq.py:103-111) and the failure flag cleared
  k_damp<<<1, 1024, 0, s>>>(H, ldh, Ci, percdamp, 0, w.scal, w.dead, w.info);
  CRBQ_LAUNCH_CHECK();
  if (W) {
    k_zero_dead<<<nblocks(R * C), 256, 0, s>>>(W, ldw, (int)R, Ci, w.dead);
    CRBQ_LAUNCH_CHECK();
  }
  k_reverse_lower<<<rows_grid(C), 256, 0, s>>>(H, ldh, Ci, w.A, C,
                                                reverse_vec(H, ldh, C, w.A, C));
  CRBQ_LAUNCH_CHECK();
  st = chol_inv_sweep(w.A, C, Ci, w, s);
  if (st) return st;
  k_reverse_to_u<<<rows_grid(C), 256, 0, s>>>(w.A, C, Ci, U, ldu,
                                               reverse_vec(w.A, C, C, U, ldu));
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
    k_damp<<<1, 1024, 0, s>>>(H, ldh, Ci, 1e-3f, 1, w.scal, nullptr, nullptr);
    CRBQ_LAUNCH_CHECK();
    if (attempt == 10) break;                                       // 10 attempts in all
    k_set_int<<<1, 1, 0, s>>>(w.info, 0);
    k_reverse_lower<<<rows_grid(C), 256, 0, s>>>(H, ldh, Ci, w.A, C,
                                                reverse_vec(H, ldh, C, w.A, C));
    CRBQ_LAUNCH_CHECK();
    st = chol_inv_sweep(w.A, C, Ci, w, s);
    if (st) return st;
    CRBQ_HIP(hipMemcpyAsync(&hinfo, w.info, sizeof(int), hipMemcpyDeviceToHost, s));
    CRBQ_HIP(hipStreamSynchronize(s));
    ok = hinfo == 0;
    if (ok) {
      k_reverse_to_u<<<rows_grid(C), 256, 0, s>>>(w.A, C, Ci, U, ldu,
                                               reverse_vec(w.A, C, C, U, ldu));
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
