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

// K loop of an interior 128 x 128 tile (A not transposed) as one asm block.
// Left to the compiler, each 4-deep k-step's fragment reads were issued two
// MFMAs before their first use, so every step waited out the LDS latency
// (~0.8 of the matrix units busy); and once the accumulators are asm
// operands, any asm statement inside a compiler-visible loop makes the
// register allocator carry them in VGPRs and copy them in and out of the
// AGPRs around it.  So the whole loop is one block with a fixed schedule:
//  * chunk c (32 deep) runs from LDS buffer c & 1: 8 k-steps of 4, each
//    waiting for the fragments the previous step read and issuing its 16
//    MFMAs (v_mfma_f32_16x16x4_f32, 4 x 4 tiles of 16 x 16) with the 8
//    ds_read_b32 of the next step between the first 8 of them (two
//    fragment sets in alternation);
//  * at its start the 8 buffer loads of chunk c + 1 (4 float4 per operand
//    and thread) go into staging registers; after 5 k-steps they are
//    written to the other buffer (its last reader, chunk c - 1, finished
//    before the previous barrier) between MFMAs;
//  * the chunk ends with one barrier, then the next chunk's first reads.
// Past the last chunk the loads run beyond kend; the buffer descriptors'
// record counts end at the operands' last elements, so those loads return
// zeros or in-range elements, and their LDS copy is never read.
// A is [m][k] in LDS (pitch P_MK = 36), B [k][n] (pitch BT + 16 = 144) when
// BK, else [n][k] (pitch 36); a buffer is 4608 floats.  ab / bb: this lane's
// byte address of A[wm + lane % 16][lane / 16] and of B's first fragment in
// buffer 0; wa / wb: the byte address of this thread's first float4 of the
// staged tile (float4 e at + 4608 e bytes).
#define SG_BUF "18432"
#define SG_MF(i, j, s)                                                                    \
  "v_mfma_f32_16x16x4_f32 %[c" #i #j "], %[f" #s "a" #i "], %[f" #s "b" #j "], %[c" #i #j "]\n"
#define SG_RA(s, i, kk, b)                                                                \
  "ds_read_b32 %[f" #s "a" #i "], %[ab] offset:((" #i ")*576+(" #kk "))*4+(" #b ")*" SG_BUF "\n"
#define SG_RBK(s, j, kk, b)                                                               \
  "ds_read_b32 %[f" #s "b" #j "], %[bb] offset:((" #kk ")*144+(" #j ")*16)*4+(" #b ")*" SG_BUF "\n"
#define SG_RBN(s, j, kk, b)                                                               \
  "ds_read_b32 %[f" #s "b" #j "], %[bb] offset:((" #j ")*576+(" #kk "))*4+(" #b ")*" SG_BUF "\n"
#define SG_WA(e, w) "ds_write_b128 %[wa], %[r" #e "] offset:" #e "*4608+(" #w ")*" SG_BUF "\n"
#define SG_WB(e, w) "ds_write_b128 %[wb], %[r" #e "b] offset:" #e "*4608+(" #w ")*" SG_BUF "\n"
#define SG_ROW(i, s) SG_MF(i, 0, s) SG_MF(i, 1, s) SG_MF(i, 2, s) SG_MF(i, 3, s)
// 8 MFMAs (rows 0, 1 of set s) with the reads of step nk (buffer b) into set n
#define SG_HR(s, n, nk, RB, b)                                                            \
  SG_MF(0, 0, s) SG_RA(n, 0, nk, b) SG_MF(0, 1, s) SG_RA(n, 1, nk, b) SG_MF(0, 2, s)     \
  SG_RA(n, 2, nk, b) SG_MF(0, 3, s) SG_RA(n, 3, nk, b) SG_MF(1, 0, s) RB(n, 0, nk, b)    \
  SG_MF(1, 1, s) RB(n, 1, nk, b) SG_MF(1, 2, s) RB(n, 2, nk, b) SG_MF(1, 3, s)           \
  RB(n, 3, nk, b)
#define SG_STEP(s, n, nk, RB, b)                                                          \
  "s_waitcnt lgkmcnt(0)\n" SG_HR(s, n, nk, RB, b) SG_ROW(2, s) SG_ROW(3, s)
// the same with the staged chunk written to buffer w between rows 2 and 3
#define SG_STEPW(s, n, nk, RB, b, w)                                                      \
  "s_waitcnt lgkmcnt(0)\n" SG_HR(s, n, nk, RB, b)                                        \
  SG_MF(2, 0, s) SG_WA(0, w) SG_MF(2, 1, s) SG_WA(1, w) SG_MF(2, 2, s) SG_WA(2, w)       \
  SG_MF(2, 3, s) SG_WA(3, w) SG_MF(3, 0, s) SG_WB(0, w) SG_MF(3, 1, s) SG_WB(1, w)       \
  SG_MF(3, 2, s) SG_WB(2, w) SG_MF(3, 3, s) SG_WB(3, w)
#define SG_FIRST(RB, b)                                                                   \
  SG_RA(0, 0, 0, b) SG_RA(0, 1, 0, b) SG_RA(0, 2, 0, b) SG_RA(0, 3, 0, b)                \
  RB(0, 0, 0, b) RB(0, 1, 0, b) RB(0, 2, 0, b) RB(0, 3, 0, b)
#define SG_LOADS                                                                          \
  "buffer_load_dwordx4 %[r0], %[va], %[rsa], %[sa0] offen\n"                             \
  "buffer_load_dwordx4 %[r1], %[va], %[rsa], %[sa1] offen\n"                             \
  "buffer_load_dwordx4 %[r2], %[va], %[rsa], %[sa2] offen\n"                             \
  "buffer_load_dwordx4 %[r3], %[va], %[rsa], %[sa3] offen\n"                             \
  "buffer_load_dwordx4 %[r0b], %[vb], %[rsb], %[sb0] offen\n"                            \
  "buffer_load_dwordx4 %[r1b], %[vb], %[rsb], %[sb1] offen\n"                            \
  "buffer_load_dwordx4 %[r2b], %[vb], %[rsb], %[sb2] offen\n"                            \
  "buffer_load_dwordx4 %[r3b], %[vb], %[rsb], %[sb3] offen\n"                            \
  "v_add_u32 %[va], %[ka], %[va]\n"                                                      \
  "v_add_u32 %[vb], %[kb], %[vb]\n"
// chunk from buffer b, staging the next one into buffer w
#define SG_CHUNK(RB, b, w)                                                                \
  SG_LOADS                                                                               \
  SG_STEP(0, 1, 4, RB, b) SG_STEP(1, 0, 8, RB, b) SG_STEP(0, 1, 12, RB, b)               \
  SG_STEP(1, 0, 16, RB, b) "s_waitcnt vmcnt(0)\n" SG_STEPW(0, 1, 20, RB, b, w)           \
  SG_STEP(1, 0, 24, RB, b) SG_STEP(0, 1, 28, RB, b)                                      \
  "s_waitcnt lgkmcnt(0)\n" SG_ROW(0, 1) SG_ROW(1, 1) SG_ROW(2, 1) SG_ROW(3, 1)          \
  "s_barrier\n"                                                                          \
  "s_add_u32 %[cnt], %[cnt], 1\n"                                                        \
  "s_cmp_ge_u32 %[cnt], %[n]\n"                                                          \
  "s_cbranch_scc1 .Lsgend%=\n"                                                           \
  SG_FIRST(RB, w)
#define SG_LOOP(RB)                                                                       \
  "s_mov_b32 %[cnt], 0\n" SG_FIRST(RB, 0)                                                \
  ".Lsgloop%=:\n" SG_CHUNK(RB, 0, 1) SG_CHUNK(RB, 1, 0) "s_branch .Lsgloop%=\n"          \
  ".Lsgend%=:\n"                                                                         \
  "s_waitcnt vmcnt(0) lgkmcnt(0)\n"                                                      \
  "s_nop 7\ns_nop 7\ns_nop 7\n"
#define SG_OPERANDS                                                                       \
  : [c00] "+{a[0:3]}"(acc[0][0]), [c01] "+{a[4:7]}"(acc[0][1]),                          \
    [c02] "+{a[8:11]}"(acc[0][2]), [c03] "+{a[12:15]}"(acc[0][3]),                       \
    [c10] "+{a[16:19]}"(acc[1][0]), [c11] "+{a[20:23]}"(acc[1][1]),                      \
    [c12] "+{a[24:27]}"(acc[1][2]), [c13] "+{a[28:31]}"(acc[1][3]),                      \
    [c20] "+{a[32:35]}"(acc[2][0]), [c21] "+{a[36:39]}"(acc[2][1]),                      \
    [c22] "+{a[40:43]}"(acc[2][2]), [c23] "+{a[44:47]}"(acc[2][3]),                      \
    [c30] "+{a[48:51]}"(acc[3][0]), [c31] "+{a[52:55]}"(acc[3][1]),                      \
    [c32] "+{a[56:59]}"(acc[3][2]), [c33] "+{a[60:63]}"(acc[3][3]),                      \
    [f0a0] "=&v"(t[0]), [f0a1] "=&v"(t[1]), [f0a2] "=&v"(t[2]), [f0a3] "=&v"(t[3]),      \
    [f0b0] "=&v"(t[4]), [f0b1] "=&v"(t[5]), [f0b2] "=&v"(t[6]), [f0b3] "=&v"(t[7]),      \
    [f1a0] "=&v"(t[8]), [f1a1] "=&v"(t[9]), [f1a2] "=&v"(t[10]), [f1a3] "=&v"(t[11]),    \
    [f1b0] "=&v"(t[12]), [f1b1] "=&v"(t[13]), [f1b2] "=&v"(t[14]), [f1b3] "=&v"(t[15]),  \
    [r0] "=&v"(r[0]), [r1] "=&v"(r[1]), [r2] "=&v"(r[2]), [r3] "=&v"(r[3]),              \
    [r0b] "=&v"(r[4]), [r1b] "=&v"(r[5]), [r2b] "=&v"(r[6]), [r3b] "=&v"(r[7]),          \
    [cnt] "=&s"(cnt), [va] "+v"(va), [vb] "+v"(vb)                                       \
  : [ab] "v"(ab), [bb] "v"(bb), [wa] "v"(wa), [wb] "v"(wb), [rsa] "s"(rsa),              \
    [rsb] "s"(rsb), [sa0] "s"(sa[0]), [sa1] "s"(sa[1]), [sa2] "s"(sa[2]),                \
    [sa3] "s"(sa[3]), [sb0] "s"(sb[0]), [sb1] "s"(sb[1]), [sb2] "s"(sb[2]),              \
    [sb3] "s"(sb[3]), [ka] "s"(ka), [kb] "s"(kb), [n] "s"(n)                             \
  : "memory", "scc"

typedef int sg_i4_t __attribute__((ext_vector_type(4)));
// Raw buffer descriptor: 48-bit base, stride 0, nrec bytes.
__device__ __forceinline__ sg_i4_t sg_rsrc(const float* base, unsigned nrec) {
  const uint64_t a = (uint64_t)base;
  return sg_i4_t{__builtin_amdgcn_readfirstlane((int)(uint32_t)a),
                 __builtin_amdgcn_readfirstlane((int)((a >> 32) & 0xffff)),
                 __builtin_amdgcn_readfirstlane((int)nrec), 0x00020000};
}

// The K loop over n chunks (chunk 0 already in LDS buffer 0).
template <bool BK>
__device__ __forceinline__ void sg_loop128(f4_t (&acc)[4][4], unsigned ab, unsigned bb,
                                           unsigned wa, unsigned wb, sg_i4_t rsa, sg_i4_t rsb,
                                           int va, int vb, const int (&sa)[4],
                                           const int (&sb)[4], int ka, int kb, int n) {
  float t[16];
  f4_t r[8];
  int cnt;
  if constexpr (BK) asm volatile(SG_LOOP(SG_RBK) SG_OPERANDS);
  else asm volatile(SG_LOOP(SG_RBN) SG_OPERANDS);
}

__device__ __forceinline__ unsigned lds_addr(const float* p) {
  return (unsigned)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// One BT x BT output tile (number bid of the product's nwg tiles) of
// C = beta C + alpha op(A) op(B), staged through the LDS buffers As, Bs.
template <int BT, bool TA, bool TB, bool LOWER>
__device__ __forceinline__ void sgemm_tile(
    int M, int N, int K, float alpha, const float* A, int64_t lda,
    const float* B, int64_t ldb, float beta, float* C,
    int64_t ldc, int va, int vb, int tri, float (*As)[TileCfg<BT>::ELEMS],
    float (*Bs)[TileCfg<BT>::ELEMS], int bid, int nwg) {
  using Cfg = TileCfg<BT>;
  constexpr int P_KM = Cfg::P_KM, WT = Cfg::WT, MT = Cfg::MT, NE = Cfg::NE;
  int tm, tn;
  gemm_tile(bid, nwg, (M + BT - 1) / BT, (N + BT - 1) / BT, tri, LOWER, tm, tn);
  const int m0 = tm * BT, n0 = tn * BT;
  // K range of this tile when one operand is triangular (its zero part is
  // skipped; the products skipped are exact zeros)
  int kbeg = 0, kend = K;
  if (tri == GEMM_TRI_KEND_N) kend = min(K, n0 + BT);
  else if (tri == GEMM_TRI_KBEG_N) kbeg = min(K, n0) / GB_K * GB_K;
  else if (tri == GEMM_TRI_KEND_M) kend = min(K, m0 + BT);
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
  bool done = false;
  if constexpr (BT == 128 && !AK) {
    // the asm K loop: interior tiles whose chunks are all full, with every
    // byte offset of both operand regions below 2^31
    const int64_t ea = ((int64_t)(M - m0) * lda + K) * 4;
    const int64_t eb = BK ? ((int64_t)(K - kbeg + 2 * GB_K) * ldb + N) * 4
                          : ((int64_t)(N - n0) * ldb + K) * 4;
    if (nch > 0 && nfull == nch && ea < ((int64_t)1 << 31) && eb < ((int64_t)1 << 31)) {
      static_assert(P_MK == 36 && P_KM == 144 && Cfg::ELEMS == 4608, "offsets in the asm");
      const unsigned ab = lds_addr(As[0]) + (unsigned)(((wm + c16) * P_MK + kq) * 4);
      const unsigned bb = lds_addr(Bs[0]) + (unsigned)((BK ? kq * P_KM + wn + c16
                                                           : (wn + c16) * P_MK + kq) * 4);
      const unsigned wa = lds_addr(As[0]) + (unsigned)(((tid >> 3) * P_MK + (tid & 7) * 4) * 4);
      const unsigned wb = lds_addr(Bs[0]) + (unsigned)((BK ? (tid >> 5) * P_KM + (tid & 31) * 4
                                                           : (tid >> 3) * P_MK + (tid & 7) * 4) * 4);
      const int la = (int)lda, lb = (int)ldb;
      const sg_i4_t rsa = sg_rsrc(A + (int64_t)m0 * lda + kbeg,
                                  (unsigned)(((int64_t)(M - m0 - 1) * lda + (K - kbeg)) * 4));
      const sg_i4_t rsb =
          BK ? sg_rsrc(B + (int64_t)kbeg * ldb + n0,
                       (unsigned)(((int64_t)(K - kbeg - 1) * ldb + (N - n0)) * 4))
             : sg_rsrc(B + (int64_t)n0 * ldb + kbeg,
                       (unsigned)(((int64_t)(N - n0 - 1) * ldb + (K - kbeg)) * 4));
      // chunk 1's offsets (chunk 0 is in LDS); float4 e of a thread at + s[e]
      const int va0 = ((tid >> 3) * la + (tid & 7) * 4) * 4 + GB_K * 4;
      const int vb0 = BK ? ((tid >> 5) * lb + (tid & 31) * 4) * 4 + GB_K * lb * 4
                         : ((tid >> 3) * lb + (tid & 7) * 4) * 4 + GB_K * 4;
      int sa[4], sb[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sa[e] = __builtin_amdgcn_readfirstlane(e * 32 * la * 4);
        sb[e] = __builtin_amdgcn_readfirstlane(BK ? e * 8 * lb * 4 : e * 32 * lb * 4);
      }
      const int ka = GB_K * 4;
      const int kb = __builtin_amdgcn_readfirstlane(BK ? GB_K * lb * 4 : GB_K * 4);
      sg_loop128<BK>(acc, ab, bb, wa, wb, rsa, rsb, va0, vb0, sa, sb, ka, kb, nch);
      done = true;
    }
  }
  for (int c = 0; !done && c < nch; ++c) {
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

// operands of one product (the arguments of sgemm_tile)
struct SgP {
  int M, N, K;
  float alpha, beta;
  const float* A;
  const float* B;
  float* C;
  int64_t lda, ldb, ldc;
  int va, vb, tri;
};

template <int BT, bool TA, bool TB, bool LOWER>
__device__ __forceinline__ void sgemm_tile(const SgP& p, float (*As)[TileCfg<BT>::ELEMS],
                                           float (*Bs)[TileCfg<BT>::ELEMS], int bid, int nwg) {
  sgemm_tile<BT, TA, TB, LOWER>(p.M, p.N, p.K, p.alpha, p.A, p.lda, p.B, p.ldb, p.beta, p.C,
                                p.ldc, p.va, p.vb, p.tri, As, Bs, bid, nwg);
}

template <int BT, bool TA, bool TB, bool LOWER>
__global__ __launch_bounds__(256) void k_sgemm(SgP p, const int* __restrict__ stop) {
  if (stop && *stop) return;
  __shared__ __attribute__((aligned(16))) float As[2][TileCfg<BT>::ELEMS];
  __shared__ __attribute__((aligned(16))) float Bs[2][TileCfg<BT>::ELEMS];
  sgemm_tile<BT, TA, TB, LOWER>(p, As, Bs, blockIdx.x, gridDim.x);
}

// Two independent products in one grid: workgroups [0, n1) compute p1's
// tiles, the others p2's, in one set of LDS buffers.  The factorization's
// Schur update A22 -= T T^T (p1, full K on every tile) and Q = T X11 (p2,
// tiles in decreasing K) both only read T; launched together, the Schur
// update's last round of tiles shares the CUs with the start of the other
// product instead of running alone, and one launch of the dependent chain
// goes away.
template <int BT, bool TA1, bool TB1, bool LO1, bool TA2, bool TB2, bool LO2>
__global__ __launch_bounds__(256) void k_sgemm2(SgP p1, int n1, SgP p2,
                                                const int* __restrict__ stop) {
  if (stop && *stop) return;
  __shared__ __attribute__((aligned(16))) float As[2][TileCfg<BT>::ELEMS];
  __shared__ __attribute__((aligned(16))) float Bs[2][TileCfg<BT>::ELEMS];
  if ((int)blockIdx.x < n1)
    sgemm_tile<BT, TA1, TB1, LO1>(p1, As, Bs, blockIdx.x, n1);
  else
    sgemm_tile<BT, TA2, TB2, LO2>(p2, As, Bs, (int)blockIdx.x - n1, (int)gridDim.x - n1);
}

// Up to SG_NSEG products of one shape, one per blockIdx.y: the block loop
// of sublayers that share the factor updates each one's weights with its
// own error rows against the same U rows, all in one launch.  Every
// product's tiles are those of its own k_sgemm launch (same tile size,
// same grid, same sums).
constexpr int SG_NSEG = 4;
struct SgSeg {
  SgP p[SG_NSEG];
};

template <int BT>
__global__ __launch_bounds__(256) void k_sgemm_seg(SgSeg g) {
  __shared__ __attribute__((aligned(16))) float As[2][TileCfg<BT>::ELEMS];
  __shared__ __attribute__((aligned(16))) float Bs[2][TileCfg<BT>::ELEMS];
  sgemm_tile<BT, false, false, false>(g.p[blockIdx.y], As, Bs, blockIdx.x, gridDim.x);
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
  SgP p;
  p.M = (int)M; p.N = (int)N; p.K = (int)K;
  p.alpha = alpha; p.beta = beta;
  p.A = A; p.B = B; p.C = C;
  p.lda = lda; p.ldb = ldb; p.ldc = ldc;
  p.va = vec_ok(A, lda); p.vb = vec_ok(B, ldb); p.tri = tri;
#define CRBQ_GEMM_CASE(TA_, TB_, LO_)                                 \
  if (ta == TA_ && tb == TB_ && lower == LO_) {                       \
    k_sgemm<BT, TA_, TB_, LO_><<<grid, 256, 0, s>>>(p, stop);         \
    CRBQ_LAUNCH_CHECK();                                              \
    return CRBQ_OK;                                                   \
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

// Products that give fewer than 512 tiles of 128 x 128 (two per CU) run on
// 64 x 64 tiles (4x the workgroups, a quarter of the work each), and those
// with fewer than 512 tiles of 64 x 64 on 32 x 32 tiles.  The products of
// the factorization below its top two levels (2048 and smaller) are
// latency chains of one or two rounds of workgroups, which smaller tiles
// shorten (factor at C = 16384: 33.2 -> 31.4 ms; the sums are unchanged,
// since every tile size adds the k-steps of an element in the same order).
static int tile_of(int64_t M, int64_t N) {
  const int64_t t128 = ((M + 127) / 128) * ((N + 127) / 128);
  const int64_t t64 = ((M + 63) / 64) * ((N + 63) / 64);
  return t64 < 512 ? 32 : t128 < 512 ? 64 : 128;
}

int sgemm_launch(bool ta, bool tb, bool lower, int64_t M, int64_t N, int64_t K,
                 float alpha, const float* A, int64_t lda, const float* B,
                 int64_t ldb, float beta, float* C, int64_t ldc,
                 const int* stop, hipStream_t s, int tri) {
  if (M <= 0 || N <= 0) return CRBQ_OK;
  if (M > (1 << 30) || N > (1 << 30) || K > (1 << 30) || K < 0) return CRBQ_ERR_ARG;
  const int bt = tile_of(M, N);
  if (bt == 32)
    return sgemm_go<32>(ta, tb, lower, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, stop, s,
                        tri);
  if (bt == 64)
    return sgemm_go<64>(ta, tb, lower, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, stop, s,
                        tri);
  return sgemm_go<128>(ta, tb, lower, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, stop, s,
                       tri);
}

static SgP sg_params(const GemmArgs& g);

template <int BT>
static int sgemm_seg_go(int nseg, const GemmArgs* gs, hipStream_t s) {
  const int64_t nwg = ((gs[0].M + BT - 1) / BT) * ((gs[0].N + BT - 1) / BT);
  if (nwg > 0x7fffffff) return CRBQ_ERR_ARG;
  SgSeg g{};
  for (int i = 0; i < nseg; ++i) g.p[i] = sg_params(gs[i]);
  k_sgemm_seg<BT><<<dim3((unsigned)nwg, (unsigned)nseg), 256, 0, s>>>(g);
  CRBQ_LAUNCH_CHECK();
  return CRBQ_OK;
}

int sgemm_seg_launch(int nseg, const GemmArgs* gs, hipStream_t s) {
  if (nseg < 1 || nseg > SG_NSEG) return CRBQ_ERR_ARG;
  const GemmArgs& g0 = gs[0];
  bool same = true;
  for (int i = 0; i < nseg; ++i) {
    const GemmArgs& g = gs[i];
    same = same && !g.ta && !g.tb && !g.lower && g.tri == GEMM_TRI_NONE && g.M == g0.M &&
           g.N == g0.N && g.K == g0.K;
  }
  if (!same || nseg == 1 || g0.M <= 0 || g0.N <= 0 || g0.M > (1 << 30) ||
      g0.N > (1 << 30) || g0.K < 0 || g0.K > (1 << 30)) {
    for (int i = 0; i < nseg; ++i) {
      const GemmArgs& g = gs[i];
      const int st = sgemm_launch(g.ta, g.tb, g.lower, g.M, g.N, g.K, g.alpha, g.A, g.lda, g.B,
                                  g.ldb, g.beta, g.C, g.ldc, nullptr, s, g.tri);
      if (st) return st;
    }
    return CRBQ_OK;
  }
  const int bt = tile_of(g0.M, g0.N);
  if (bt == 32) return sgemm_seg_go<32>(nseg, gs, s);
  if (bt == 64) return sgemm_seg_go<64>(nseg, gs, s);
  return sgemm_seg_go<128>(nseg, gs, s);
}

static SgP sg_params(const GemmArgs& g) {
  SgP p;
  p.M = (int)g.M; p.N = (int)g.N; p.K = (int)g.K;
  p.alpha = g.alpha; p.beta = g.beta;
  p.A = g.A; p.B = g.B; p.C = g.C;
  p.lda = g.lda; p.ldb = g.ldb; p.ldc = g.ldc;
  p.va = vec_ok(g.A, g.lda); p.vb = vec_ok(g.B, g.ldb); p.tri = g.tri;
  return p;
}

template <int BT>
static int sgemm2_go(const GemmArgs& x, const GemmArgs& y, const int* stop, hipStream_t s) {
  const int64_t TX = (x.M + BT - 1) / BT;
  const int64_t n1 = TX * (TX + 1) / 2;
  const int64_t n2 = ((y.M + BT - 1) / BT) * ((y.N + BT - 1) / BT);
  if (n1 + n2 > 0x7fffffff) return CRBQ_ERR_ARG;
  k_sgemm2<BT, false, true, true, false, false, false>
      <<<(unsigned)(n1 + n2), 256, 0, s>>>(sg_params(x), (int)n1, sg_params(y), stop);
  CRBQ_LAUNCH_CHECK();
  return CRBQ_OK;
}

int sgemm2_launch(const GemmArgs& x, const GemmArgs& y, const int* stop, hipStream_t s) {
  const auto one = [&](const GemmArgs& g) {
    return sgemm_launch(g.ta, g.tb, g.lower, g.M, g.N, g.K, g.alpha, g.A, g.lda, g.B, g.ldb,
                        g.beta, g.C, g.ldc, stop, s, g.tri);
  };
  const bool pair = !x.ta && x.tb && x.lower && x.M == x.N && x.tri == GEMM_TRI_NONE &&
                    !y.ta && !y.tb && !y.lower;
  const bool sizes = x.M > 0 && x.N > 0 && y.M > 0 && y.N > 0 && x.K >= 0 && y.K >= 0 &&
                     x.M <= (1 << 30) && x.K <= (1 << 30) && y.M <= (1 << 30) &&
                     y.N <= (1 << 30) && y.K <= (1 << 30);
  const int bt = sizes ? tile_of(x.M, x.N) : 0;
  if (!pair || !sizes || bt != tile_of(y.M, y.N)) {
    const int st = one(x);
    return st ? st : one(y);
  }
  if (bt == 32) return sgemm2_go<32>(x, y, stop, s);
  if (bt == 64) return sgemm2_go<64>(x, y, stop, s);
  return sgemm2_go<128>(x, y, stop, s);
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
