// Hessian accumulation of BRAGPTQ.add_batch (bigptq.py:37-53) on MFMA.
//
// S[I, J] += X[:, I]^T X[:, J] over token rows of X, for the upper-triangle
// tiles I <= J of the fp32 C x C accumulator S.  The reference casts
// the activations to fp32 and runs an SGEMM with TF32 off; f16/bf16 products
// are exact in fp32, so the f16/bf16 MFMA (v_mfma_f32_16x16x32_{f16,bf16},
// fp32 accumulate) computes the same sums up to summation order.  fp32
// inputs use v_mfma_f32_16x16x4_f32.
//
// Each MFMA lane needs 8 consecutive tokens of one channel.  Three ways to
// get them from the token-major activations X[t][c]:
//  * token-major stages (k_syrk16k / k_syrk16k_pers with TM, used when C is
//    a multiple of 256 and X's rows are 16-byte aligned): 64-token stages of
//    X go straight into LDS as they are (direct-to-LDS buffer loads), and
//    the lanes read their operands with LDS transpose reads
//    (ds_read_b64_tr_b16): no copy of X;
//  * channel-major path (k_xpose16, then the same kernels on the copy, used
//    for other channel counts when the workspace can hold a transposed
//    copy): X is transposed once into the workspace and each lane reads its
//    operand with one ds_read_b128;
//  * in-place path (k_syrk16p): a loading thread reads a 4-token x
//    8-channel unit with four 16-byte loads and transposes it in registers
//    with v_perm_b32 before one 8-byte LDS store per channel.
// The first two issue the same MFMAs on the same operands for the same
// token splits, so their sums are bitwise equal.
#include <stdlib.h>

#include <atomic>
#include <mutex>
#include <vector>

#include "common.h"

namespace crbq {

constexpr int HT = 128;      // output tile of the fp32-input kernel
constexpr int HK32 = 16;     // tokens per LDS stage (fp32 input)

__device__ __forceinline__ void tile_of(int idx, int nt, int& ti, int& tj) {
  // idx over the upper triangle row by row: row ti has nt - ti tiles
  int i = 0, rem = idx;
  while (rem >= nt - i) { rem -= nt - i; ++i; }
  ti = i;
  tj = i + rem;
}

template <typename T8>
__device__ __forceinline__ f4_t mfma16(T8 a, T8 b, f4_t c);
template <>
__device__ __forceinline__ f4_t mfma16<h8_t>(h8_t a, h8_t b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f4_t mfma16<b8_t>(b8_t a, b8_t b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// 16-bit inputs (T8 = h8_t or b8_t; storage is 2 bytes per element):
// 256 x 256 output tile per workgroup (k_syrk16p below).
// Split-K: workgroup (tile, s) sums tokens [s*span, (s+1)*span) and, when
// the grid is split, split 0 adds into S and split s > 0 writes its
// partial tile to P[s - 1] for k_sum_splits.
constexpr int ST = 256;                 // output tile (channels)

// FAST: C and ldx are multiples of 8 and X is 16-byte aligned, so every
// in-range 8-channel group is one 16-byte load.
template <bool FAST>
__device__ __forceinline__ void load_unit(const uint16_t* __restrict__ X, int64_t ntok,
                                          int64_t ldx, int C, int64_t t0, int cbase,
                                          bool cvec, uint32_t (&in)[4][4]) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t t = t0 + r;
    if (FAST) {
      uint4 v = make_uint4(0u, 0u, 0u, 0u);
      if (t < ntok && cbase < C) v = *(const uint4*)(X + t * ldx + cbase);
      in[r][0] = v.x; in[r][1] = v.y; in[r][2] = v.z; in[r][3] = v.w;
    } else if (t < ntok && cvec) {
      const uint4 v = *(const uint4*)(X + t * ldx + cbase);
      in[r][0] = v.x; in[r][1] = v.y; in[r][2] = v.z; in[r][3] = v.w;
    } else {
      uint16_t h[8];
#pragma unroll
      for (int q = 0; q < 8; ++q)
        h[q] = (t < ntok && cbase + q < C) ? X[t * ldx + cbase + q] : (uint16_t)0;
#pragma unroll
      for (int q = 0; q < 4; ++q) in[r][q] = (uint32_t)h[2 * q] | ((uint32_t)h[2 * q + 1] << 16);
    }
  }
}

// transpose a 4-token x 8-channel unit in registers, store it channel-major
template <int PITCH>
__device__ __forceinline__ void store_unit(uint16_t (*Xs)[PITCH], int crow, int tcol,
                                           const uint32_t (&in)[4][4]) {
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
    uint2 o;
    o.x = __builtin_amdgcn_perm(in[1][c >> 1], in[0][c >> 1], sel);
    o.y = __builtin_amdgcn_perm(in[3][c >> 1], in[2][c >> 1], sel);
    *(uint2*)&Xs[crow + c][tcol] = o;
  }
}

template <int U>
struct StageRegsT {
  uint32_t u[U][4][4];
};

template <bool FAST, int U>
__device__ __forceinline__ void load_stage(const uint16_t* __restrict__ X, int64_t kend,
                                           int64_t ldx, int C, int64_t t0, int cbase, bool cvec,
                                           StageRegsT<U>& r) {
#pragma unroll
  for (int q = 0; q < U; ++q)
    load_unit<FAST>(X, kend, ldx, C, t0 + 32 * q, cbase, cvec, r.u[q]);
}

template <int U, int PITCH>
__device__ __forceinline__ void store_stage(uint16_t (*Xs)[PITCH], int crow, int tcol,
                                            const StageRegsT<U>& r) {
#pragma unroll
  for (int q = 0; q < U; ++q) store_unit<PITCH>(Xs, crow, tcol + 32 * q, r.u[q]);
}

// Upper-triangle tile of linear index lin, in bands of 4 tile rows: within
// a band the tile columns ascend and each column lists the band's rows, so
// 32 consecutive indices form a 4 x 8 block of tiles that shares 12
// operand panels.
__device__ __forceinline__ void tile_band(int lin, int nt, int& ti, int& tj) {
  for (int r0 = 0; r0 < nt; r0 += 4) {
    const int r1 = min(r0 + 4, nt) - 1;
    for (int c = r0; c < nt; ++c) {
      const int cnt = min(r1, c) - r0 + 1;
      if (lin < cnt) { ti = r0 + lin; tj = c; return; }
      lin -= cnt;
    }
  }
  ti = tj = 0;
}

// Workgroup id -> linear tile index such that the workgroups one XCD
// receives (every 8th id) take consecutive indices.
__device__ __forceinline__ int xcd_chunk(int id, int nwg) {
  const int q = nwg / 8, r = nwg % 8, x = id % 8, k = id / 8;
  return (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + k;
}

// Producer/consumer variant: 12 wavefronts per 256 x 256 tile.
//  * 8 consumer wavefronts (2 x 4, 128 x 64 outputs each) only read operand
//    fragments from LDS and issue MFMAs.
//  * 4 producer wavefronts load X, transpose 4-token x 8-channel units in
//    registers and store them channel-major into a ring of 3 LDS stages of
//    SKQ tokens; loads run two stages ahead of their LDS store, so global
//    latency stays off the MFMA wavefronts.
// One barrier per stage: at iteration c the consumers read stage c while
// the producers store stage c + 2 (its buffer was last read at c - 1) and
// issue the loads of stage c + 4.
// Barrier for LDS traffic only: waits for this wavefront's LDS operations,
// not for its outstanding global loads (__syncthreads waits for both, which
// would drain the producers' prefetch at every stage).
__device__ __forceinline__ void sync_lds() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

constexpr int SKQ = 32;                 // tokens per stage
constexpr int SKQP = SKQ + 8;           // padded LDS row (halves)
constexpr int SYRKP_THREADS = 768;
constexpr int NSTAGE = 3;
constexpr int NSET = 4;                 // stages in flight in producer registers

template <typename T8>
__device__ __forceinline__ void syrk_stage_p(const uint16_t (*XI)[SKQP],
                                             const uint16_t (*XJ)[SKQP], int wm, int wn,
                                             int r16, int kof, f4_t (&acc)[8][4]) {
  T8 b[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) b[j] = *(const T8*)&XJ[wn + j * 16 + r16][kof];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const T8 a = *(const T8*)&XI[wm + i * 16 + r16][kof];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = mfma16<T8>(a, b[j], acc[i][j]);
  }
}

template <typename T8, bool FAST>
__global__ __launch_bounds__(SYRKP_THREADS) void k_syrk16p(const uint16_t* __restrict__ X,
                                                           int64_t ntok, int64_t ldx, int C,
                                                           float* S, int64_t lds, int nt,
                                                           int64_t span, float* P) {
  __shared__ __attribute__((aligned(16))) uint16_t Xs[NSTAGE][2][ST][SKQP];
  int ti, tj;
  tile_band(xcd_chunk(blockIdx.x, gridDim.x), nt, ti, tj);
  const int64_t k_beg = (int64_t)blockIdx.y * span;
  const int64_t k_end = k_beg + span < ntok ? k_beg + span : ntok;
  const int nch = k_end > k_beg ? (int)((k_end - k_beg + SKQ - 1) / SKQ) : 0;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool diag = ti == tj;
  if (wave >= 8) {
    // ---------------- producers ----------------
    const int p = tid - 512, tg = p & 7, cg = p >> 3;   // 8 token groups x 32 channel groups
    const bool vecok = ((ldx & 7) == 0) && ((((uintptr_t)X) & 15) == 0);
    const int cb0 = ti * ST + cg * 8, cb1 = tj * ST + cg * 8;
    const bool cv0 = vecok && cb0 + 8 <= C, cv1 = vecok && cb1 + 8 <= C;
    const int64_t t_lane = k_beg + tg * 4;
    StageRegsT<1> r[NSET][2];                           // [set][side]
    auto load = [&](int stage, int set) {
      const int64_t t0 = t_lane + (int64_t)stage * SKQ;
      load_stage<FAST, 1>(X, k_end, ldx, C, t0, cb0, cv0, r[set][0]);
      if (!diag) load_stage<FAST, 1>(X, k_end, ldx, C, t0, cb1, cv1, r[set][1]);
    };
    auto store = [&](int stage, int set) {
      const int b = stage % NSTAGE;
      store_stage<1, SKQP>(Xs[b][0], cg * 8, tg * 4, r[set][0]);
      if (!diag) store_stage<1, SKQP>(Xs[b][1], cg * 8, tg * 4, r[set][1]);
    };
    // stages 0 and 1 go straight to LDS; stage 2 + q is held in set q
    if (nch > 0) load(0, 0);
    if (nch > 0) store(0, 0);
    if (nch > 1) load(1, 0);
    if (nch > 1) store(1, 0);
#pragma unroll
    for (int q = 0; q < NSET; ++q)
      if (2 + q < nch) load(2 + q, q);
    sync_lds();
    // at iteration c: store stage c + 2 (set c % NSET), load stage
    // c + 2 + NSET into the same set; unrolled by NSET so the set index is
    // static
    for (int c0 = 0; c0 < nch; c0 += NSET) {
#pragma unroll
      for (int q = 0; q < NSET; ++q) {
        const int c = c0 + q;
        if (c >= nch) break;
        if (c + 2 < nch) store(c + 2, q);
        if (c + 2 + NSET < nch) load(c + 2 + NSET, q);
        sync_lds();
      }
    }
    return;
  }
  // ---------------- consumers ----------------
  const int lane = tid & 63;
  const int wm = (wave >> 2) * 128, wn = (wave & 3) * 64;
  f4_t acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};
  const int r16 = lane & 15, kof = (lane >> 4) * 8;
  sync_lds();
  for (int c = 0; c < nch; ++c) {
    const int b = c % NSTAGE;
    syrk_stage_p<T8>(Xs[b][0], diag ? Xs[b][0] : Xs[b][1], wm, wn, r16, kof, acc);
    sync_lds();
  }
  const int c16 = lane & 15, r4 = (lane >> 4) * 4;
  // split 0 adds into S, split s > 0 writes P[s - 1]; k_sum_splits then
  // adds P[0..] in split order, so S + acc_0 + acc_1 + ... either way
  const bool part = P && blockIdx.y > 0;
  float* out = part ? P + (size_t)(blockIdx.y - 1) * (size_t)C * lds : S;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int gi = ti * ST + wm + i * 16 + r4 + r;
        const int gj = tj * ST + wn + j * 16 + c16;
        if (gi < C && gj < C && gi <= gj) {
          float* q = out + (int64_t)gi * lds + gj;
          *q = part ? acc[i][j][r] : *q + acc[i][j][r];
        }
      }
}

// ---------------------------------------------------------------------------
// Channel-major path.  X[t][c] is first transposed into a workspace
// Xt[c][t] (k_xpose16), zero-padded to Cp = 256-multiple channels and tpad =
// 64-multiple tokens; k_syrk16k then reads operand rows that are already
// token-contiguous, so every 16-byte chunk goes from L2 straight into LDS
// (a direct-to-LDS buffer load) and every stage touches whole 128-byte
// lines.  For the same split boundaries both paths issue the same MFMAs on
// the same 32-token slices in the same order, so their sums are bitwise
// equal.

// Workgroups of a k_xpose16 launch for nw 64x64 blocks (4 per workgroup and
// pass): up to 16384, 64 per CU; on the fc2 input (262144 x 16384) this
// grid moves the 17 GB in 3.39 ms against 3.51 ms with 4096 workgroups.
inline unsigned xpose_blocks(int64_t nw) {
  const int64_t b = (nw + 3) / 4;
  return (unsigned)(b < 16384 ? b : 16384);
}

// X[t][c] -> Xt[c][t] for c < Cp, t < tpad; zeros where t >= ntok or
// c >= C.  A wavefront moves 64 tokens x 64 channels; each lane transposes
// an 8-token x 8-channel block in registers (v_perm_b32), reading 16 bytes
// of 8 token rows and writing 16 bytes of 8 channel rows, so both sides are
// whole 128-byte lines per 8 lanes.
template <bool FAST>
__global__ __launch_bounds__(256) void k_xpose16(const uint16_t* __restrict__ X, int64_t ntok,
                                                 int64_t ldx, int C, uint16_t* __restrict__ Xt,
                                                 int64_t ldt, int64_t tpad, int Cp) {
  const int lane = threadIdx.x & 63;
  const int tg = lane & 7, cg = lane >> 3;
  const int nwc = Cp / 64;
  const int64_t nw = (tpad / 64) * nwc;
  for (int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); w < nw;
       w += (int64_t)gridDim.x * 4) {
    const int64_t wt = w / nwc;
    const int c0 = (int)(w - wt * nwc) * 64 + cg * 8;
    const int64_t t0 = wt * 64 + tg * 8;
    uint32_t in[8][4];
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int64_t t = t0 + r;
      if (FAST) {
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (t < ntok && c0 < C) v = *(const uint4*)(X + t * ldx + c0);
        in[r][0] = v.x; in[r][1] = v.y; in[r][2] = v.z; in[r][3] = v.w;
      } else {
        uint16_t h[8];
#pragma unroll
        for (int q = 0; q < 8; ++q)
          h[q] = (t < ntok && c0 + q < C) ? X[t * ldx + c0 + q] : (uint16_t)0;
#pragma unroll
        for (int q = 0; q < 4; ++q) in[r][q] = (uint32_t)h[2 * q] | ((uint32_t)h[2 * q + 1] << 16);
      }
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
      uint4 o;
      o.x = __builtin_amdgcn_perm(in[1][c >> 1], in[0][c >> 1], sel);
      o.y = __builtin_amdgcn_perm(in[3][c >> 1], in[2][c >> 1], sel);
      o.z = __builtin_amdgcn_perm(in[5][c >> 1], in[4][c >> 1], sel);
      o.w = __builtin_amdgcn_perm(in[7][c >> 1], in[6][c >> 1], sel);
      *(uint4*)(Xt + (int64_t)(c0 + c) * ldt + t0) = o;
    }
  }
}

constexpr int KQ = 64;                  // tokens per stage: one 128-byte line per row
constexpr int SYRKD_THREADS = 512;
typedef int i4_t __attribute__((ext_vector_type(4)));

// 16-byte chunk slot of chunk c in LDS row r (rows are 128 bytes, unpadded):
// the MFMA reads of 8 consecutive rows at one chunk hit 8 distinct slots.
__device__ __forceinline__ int xt_slot(int c, int r) { return c ^ (r & 7); }

// Raw buffer descriptor (gfx950 layout): 48-bit base, stride 0, nrec bytes.
__device__ __forceinline__ i4_t xt_rsrc(const uint16_t* base, int nrec) {
  const uint64_t a = (uint64_t)base;
  return i4_t{__builtin_amdgcn_readfirstlane((int)(uint32_t)a),
              __builtin_amdgcn_readfirstlane((int)((a >> 32) & 0xffff)),
              __builtin_amdgcn_readfirstlane(nrec), 0x00020000};
}

// Load k (0..7) of one wavefront's share of a stage: 8-row group
// g = 4w + (k & 3) of operand panel k >> 2 (1 KB: one buffer_load_dwordx4
// ... lds, whose 64 lanes write 16 bytes each at M0 + 16 * lane).  Lane l
// fills slot l & 7 of row l >> 3 of the group, so it reads the chunk that
// belongs there.  Inline assembly: the compiler does not see these loads,
// so it does not make operand reads of the other buffer wait for them; the
// caller waits for them (vmcnt).  No "memory" clobber: the load writes a
// buffer no operand read of the current stage touches, and its order
// against the barriers (volatile asm) is kept.
__device__ __forceinline__ void xt_load(uint16_t* buf, int stage, int wave, int k, i4_t rs0,
                                        i4_t rs1, int voff, int gstep) {
  const int g = wave * 4 + (k & 3);
  const int soff = __builtin_amdgcn_readfirstlane(g * gstep + stage * KQ * 2);
  const unsigned d = __builtin_amdgcn_readfirstlane(
      (unsigned)(uintptr_t)(__attribute__((address_space(3))) void*)(buf + ((k >> 2) * ST +
                                                                              g * 8) * KQ));
  const i4_t rs = (k >> 2) ? rs1 : rs0;
  asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds" :: "v"(voff), "s"(rs), "s"(soff),
               "{m0}"(d));
}

// SYRK on Xt, 256 x 256 upper tiles, 8 wavefronts.  Each wavefront computes
// a 128 x 64 block of outputs (v_mfma_f32_16x16x32, two 32-token slices per
// stage) from a 2-stage LDS ring of 64-token stages, and also loads a
// quarter of every stage with direct-to-LDS buffer loads (L2 straight into
// LDS, no VGPR round trip, no loader wavefronts, so each wavefront may use
// 256 registers).  During stage c a wavefront issues its 8 loads of stage
// c + 1, one after each 16-row A fragment of the stage's first 32-token
// slice (between the MFMAs: a burst of 64 loads per CU at the top of the
// stage held the wavefronts in VMEM issue), into the buffer every
// wavefront finished reading at the barrier that ended stage c - 1; each
// wavefront waits for its own loads (vmcnt(0)) before the barrier that
// ends stage c.  In the last stage the loads repeat stage nch - 1 into the
// other buffer, which is not read again, so every stage issues the same 8
// loads without a branch.  The next A fragment is read before the current
// one's MFMAs, and a scheduling barrier after each fragment's group keeps
// that order.
// Requires Cp = nt * 256 rows in Xt, ldt, span and tpad multiples of KQ, and
// 256 * ldt * 2 < 2^31 (a tile's panel is addressed with 32-bit offsets).
//
// Pacing (THR, the persistent kernel): the workgroups of one XCD share
// their operand panels through that XCD's L2, but drift apart by more
// stages than the L2 holds (a panel line read by one is gone before the
// next asks for it).  Each workgroup adds 1 to its XCD's stage counter at
// the top of every stage (a returning atomic in the XCD's L2, workgroup
// scope: every workgroup that uses the counter runs on that XCD) and, at
// the end of the stage, lets stage g start only once the counter reaches
// nwx * (g - lag): no workgroup runs more than lag stages ahead of the
// XCD's slowest.  (The add's result is awaited right away; issuing it as
// assembly awaited only at the stage end measured slower, 61 against
// 59.6 ms on the fc2 shape, with occasional 68 ms runs.)  The wait is bounded (maxspin polls), so it is a pace and
// never a dependence: results do not depend on it.
struct SyrkPace {
  unsigned* ctr;     // the XCD's stage counter
  unsigned nwx;      // workgroups counted on the XCD
  int lag, maxspin;
  unsigned g;        // paced stages this workgroup has finished
  bool on;           // pace this tile (uniform over the workgroup)
};

// Top of a paced stage: this workgroup's add to its XCD's stage counter
// (the counter's value before it is returned to thread 0).
template <bool THR>
__device__ __forceinline__ unsigned pace_top(SyrkPace& pc, int tid) {
  unsigned snap = 0;
  if (THR && pc.on && tid == 0)
    snap = __hip_atomic_fetch_add(pc.ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  return snap;
}
// End of a paced stage: thread 0 polls the counter until the XCD's slowest
// workgroup is at most lag stages behind, or maxspin polls have passed.
template <bool THR>
__device__ __forceinline__ void pace_end(SyrkPace& pc, int tid, unsigned snap) {
  if (THR && pc.on && tid == 0) {
    ++pc.g;
    const unsigned need = pc.g > (unsigned)pc.lag ? pc.nwx * (pc.g - pc.lag) : 0u;
    unsigned seen = snap + 1u;
    for (int it = 0; seen < need && it < pc.maxspin; ++it) {
      __builtin_amdgcn_s_sleep(1);
      seen = __hip_atomic_fetch_add(pc.ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  }
}

template <typename T8, bool THR>
__device__ __forceinline__ void syrk_tile(uint16_t (*Xs)[2][ST][KQ], const uint16_t* Xt,
                                          int64_t ldt, int ti, int tj, int64_t k_beg, int nch,
                                          f4_t (&acc)[8][4], SyrkPace& pc) {
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int nrec = (int)((int64_t)ST * ldt * 2);
  const i4_t rs0 = xt_rsrc(Xt + (int64_t)ti * ST * ldt + k_beg, nrec);
  const i4_t rs1 = xt_rsrc(Xt + (int64_t)tj * ST * ldt + k_beg, nrec);
  // lane -> (row l >> 3 of the group, slot l & 7) -> source chunk
  const int lr = lane >> 3;
  const int voff = (lr * (int)ldt + xt_slot(lane & 7, lr) * 8) * 2;
  const int gstep = 8 * (int)ldt * 2;
  const int wm = (wave >> 2) * 128, wn = (wave & 3) * 64;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};
  const int r16 = lane & 15;
  if (nch > 0) {
#pragma unroll
    for (int k = 0; k < 8; ++k) xt_load(&Xs[0][0][0][0], 0, wave, k, rs0, rs1, voff, gstep);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  sync_lds();
  for (int c = 0; c < nch; ++c) {
    const unsigned snap = pace_top<THR>(pc, tid);
    const int nxt = c + 1 < nch ? c + 1 : nch - 1;     // stage loaded during this one
    uint16_t* nbuf = &Xs[(c + 1) & 1][0][0][0];
    const uint16_t (*XA)[KQ] = Xs[c & 1][0];
    const uint16_t (*XB)[KQ] = Xs[c & 1][1];
#pragma unroll
    for (int h = 0; h < KQ / 32; ++h) {
      // rows wm + 16i + r16 and wn + 16j + r16 share r16's low 3 bits
      const int slot = xt_slot((lane >> 4) + 4 * h, r16) * 8;
      T8 bb[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) bb[j] = *(const T8*)&XB[wn + j * 16 + r16][slot];
      T8 an = *(const T8*)&XA[wm + r16][slot];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const T8 a = an;
        if (i < 7) an = *(const T8*)&XA[wm + (i + 1) * 16 + r16][slot];
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16<T8>(a, bb[j], acc[i][j]);
        if (h == 0) {
          xt_load(nbuf, nxt, wave, i, rs0, rs1, voff, gstep);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    // the pace check overlaps this wavefront's loads still in flight
    pace_end<THR>(pc, tid, snap);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    sync_lds();
  }
}

// Token-major stages: the activations X[t][c] are staged as they are, with
// no transposed copy.  An operand's stage is 64 token rows of its panel's
// 256 channels (512 bytes per row, 32 16-byte chunks, chunk c in slot
// c ^ tm_swz(t)); a wavefront's direct-to-LDS load fills two rows.  The MFMA
// operands come from ds_read_b64_tr_b16, which gives lane j of a 16-lane
// group, as its result q (q = 0..3), the 16-bit element j % 4 of the 8 bytes
// addressed by lane 4q + j / 4 of the group.  With lane s of the group
// addressing row t0 + s / 4 at channel RB + 4 (s % 4), lane j receives
// channel RB + j at tokens t0 .. t0 + 3; reads at t0 and t0 + 4 give the 8
// consecutive tokens of the MFMA operand layout, the values the
// channel-major path reads with one ds_read_b128, so both paths issue the
// same MFMAs on the same operands and their sums are bitwise equal.
// tm_swz depends on bits 0, 1 and 3 of the row: the 8 rows one half of a
// wavefront reads (bits 0-1 from the lane, bit 3 from its 16-lane group)
// land on 8 distinct groups of 8 banks.
__device__ __forceinline__ int tm_swz(int t) { return ((t & 3) | ((t >> 1) & 4)) << 1; }

typedef __fp16 tr4_t __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef __attribute__((address_space(3))) tr4_t lds_tr4_t;

// 8 tokens x 1 channel per lane (the MFMA operand) from a token-major stage:
// p is this lane's byte address of its first 4-token read in LDS.
template <typename T8>
__device__ __forceinline__ T8 tm_frag(const char* p) {
  typedef __attribute__((address_space(3))) const char lchar;
  lchar* q = (lchar*)(const void*)p;
  const tr4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_tr4_t*)(q));
  const tr4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_tr4_t*)(q + 4 * ST * 2));
  struct P { tr4_t a, b; } v{lo, hi};
  return __builtin_bit_cast(T8, v);
}

// Descriptor of the stage of rows [t0, t0 + KQ) of panel pn of token-major
// X: rows at or beyond ntok read as zeros (their offsets lie beyond nrec).
__device__ __forceinline__ i4_t tm_rsrc(const uint16_t* X, int64_t ldx, int64_t t0,
                                        int64_t ntok, int pn) {
  int64_t rows = ntok - t0;
  rows = rows < 0 ? 0 : (rows > KQ ? KQ : rows);
  return xt_rsrc(X + t0 * ldx + (int64_t)pn * ST, (int)(rows * ldx * 2));
}

// Load k (0..7) of one wavefront's share of a token-major stage: rows
// 2g, 2g + 1 (g = 4 wave + (k & 3)) of operand k >> 2.  Lane l fills slot
// l & 31 of row 2g + (l >> 5), so it reads the chunk slot ^ tm_swz(row).
// The row offset is part of the lane offset voff[k & 3] (the buffer range
// check, which turns rows at or beyond ntok into zeros, covers the lane
// offset).
__device__ __forceinline__ void tm_load(uint16_t* buf, int wave, int k, i4_t rs0, i4_t rs1,
                                        const int (&voff)[4]) {
  const int g = wave * 4 + (k & 3);
  const unsigned d = __builtin_amdgcn_readfirstlane(
      (unsigned)(uintptr_t)(__attribute__((address_space(3))) void*)(buf + ((k >> 2) * KQ +
                                                                              2 * g) * ST));
  const i4_t rs = (k >> 2) ? rs1 : rs0;
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" :: "v"(voff[k & 3]), "s"(rs),
               "{m0}"(d));
}

// syrk_tile on token-major X (row stride ldx, ntok valid rows; stages at
// k_beg + 64 c): the same stage loop, loads and pacing, with token-major
// stages.  Requires C a multiple of 256, X 16-byte aligned and ldx a
// multiple of 8 below 2^24.
template <typename T8, bool THR>
__device__ __forceinline__ void syrk_tile_tm(uint16_t (*Xs)[2][ST][KQ], const uint16_t* X,
                                             int64_t ldx, int64_t ntok, int ti, int tj,
                                             int64_t k_beg, int nch, f4_t (&acc)[8][4],
                                             SyrkPace& pc) {
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  // direct-to-LDS loads: lane -> (row lr of the pair, slot) -> source chunk
  const int lr = lane >> 5, slot = lane & 31;
  int voff[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    const int row = 2 * (wave * 4 + kk) + lr;
    voff[kk] = (row * (int)ldx + (slot ^ tm_swz(row)) * 8) * 2;
  }
  // fragment reads: lane (group gq, s) addresses row 8 gq + s / 4 at
  // channel RB + 4 (s % 4)
  const int gq = lane >> 4, s = lane & 15;
  const int trow = 8 * gq + (s >> 2);
  const int fsw = tm_swz(trow);
  const int wm = (wave >> 2) * 128, wn = (wave & 3) * 64;
  int aoff[8], boff[4];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int ch = wm + 16 * i + 4 * (s & 3);
    aoff[i] = trow * ST * 2 + (((ch >> 3) ^ fsw) << 4) + (ch & 7) * 2;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int ch = wn + 16 * j + 4 * (s & 3);
    boff[j] = (KQ + trow) * ST * 2 + (((ch >> 3) ^ fsw) << 4) + (ch & 7) * 2;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};
  if (nch > 0) {
    const i4_t r0 = tm_rsrc(X, ldx, k_beg, ntok, ti), r1 = tm_rsrc(X, ldx, k_beg, ntok, tj);
#pragma unroll
    for (int k = 0; k < 8; ++k) tm_load(&Xs[0][0][0][0], wave, k, r0, r1, voff);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  sync_lds();
  for (int c = 0; c < nch; ++c) {
    const unsigned snap = pace_top<THR>(pc, tid);
    const int nxt = c + 1 < nch ? c + 1 : nch - 1;     // stage loaded during this one
    const int64_t tn = k_beg + (int64_t)nxt * KQ;
    const i4_t r0 = tm_rsrc(X, ldx, tn, ntok, ti), r1 = tm_rsrc(X, ldx, tn, ntok, tj);
    uint16_t* nbuf = &Xs[(c + 1) & 1][0][0][0];
    const char* cur = (const char*)&Xs[c & 1][0][0][0];
#pragma unroll
    for (int h = 0; h < KQ / 32; ++h) {
      const char* ch = cur + h * 32 * ST * 2;
      T8 bb[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) bb[j] = tm_frag<T8>(ch + boff[j]);
      T8 an = tm_frag<T8>(ch + aoff[0]);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const T8 a = an;
        if (i < 7) an = tm_frag<T8>(ch + aoff[i + 1]);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16<T8>(a, bb[j], acc[i][j]);
        if (h == 0) {
          tm_load(nbuf, wave, i, r0, r1, voff);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    pace_end<THR>(pc, tid, snap);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    sync_lds();
  }
}

// tile (split 0 adds into S, split s > 0 writes P[s - 1]; k_sum_splits then
// adds P[0..] in split order, so S + acc_0 + acc_1 + ... either way)
__device__ __forceinline__ void syrk_store(const f4_t (&acc)[8][4], int ti, int tj, int C,
                                           float* S, int64_t lds, float* P, int split) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int wm = (wave >> 2) * 128, wn = (wave & 3) * 64;
  const int c16 = lane & 15, r4 = (lane >> 4) * 4;
  const bool part = P && split > 0;
  float* out = part ? P + (size_t)(split - 1) * (size_t)C * lds : S;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int gi = ti * ST + wm + i * 16 + r4 + r;
        const int gj = tj * ST + wn + j * 16 + c16;
        if (gi < C && gj < C && gi <= gj) {
          float* q = out + (int64_t)gi * lds + gj;
          *q = part ? acc[i][j][r] : *q + acc[i][j][r];
        }
      }
}

// One workgroup per (tile, split): grid (tiles, splits).  TM: X is the
// token-major activation (ld its row stride, ntok valid rows); otherwise
// the channel-major copy (ld its row stride, zero-padded to tpad tokens).
template <typename T8, bool TM>
__global__ __launch_bounds__(SYRKD_THREADS) void k_syrk16k(const uint16_t* __restrict__ X,
                                                           int64_t ld, int64_t ntok,
                                                           int64_t tpad, int C, float* S,
                                                           int64_t lds, int nt, int64_t span,
                                                           float* P) {
  __shared__ __attribute__((aligned(1024))) uint16_t Xs[2][2][ST][KQ];   // [buffer][side]
  int ti, tj;
  tile_band(xcd_chunk(blockIdx.x, gridDim.x), nt, ti, tj);
  const int64_t k_beg = (int64_t)blockIdx.y * span;
  const int64_t k_end = k_beg + span < tpad ? k_beg + span : tpad;
  const int nch = k_end > k_beg ? (int)((k_end - k_beg) / KQ) : 0;
  f4_t acc[8][4];
  SyrkPace pc{nullptr, 0u, 0, 0, 0u, false};
  if constexpr (TM) syrk_tile_tm<T8, false>(Xs, X, ld, ntok, ti, tj, k_beg, nch, acc, pc);
  else syrk_tile<T8, false>(Xs, X, ld, ti, tj, k_beg, nch, acc, pc);
  syrk_store(acc, ti, tj, C, S, lds, P, blockIdx.y);
}

// Control words of the persistent SYRK, one 256-byte line each, zeroed
// before every launch: per XCD a stage counter (pacing), an item claim
// counter and an arrival counter.
constexpr int PCTL_LINE = 64;                                  // u32 per line
constexpr size_t PCTL_BYTES = (size_t)3 * 8 * PCTL_LINE * sizeof(unsigned);
constexpr int PACE_LAG = 4;
constexpr int PACE_MAXSPIN = 64;
// above any need (up to 63 workgroups per XCD x 2^20 paced stages), and
// 63 of them plus the stage counts stay below 2^32
constexpr unsigned PACE_RETIRE = 1u << 26;

__global__ void k_zero_u32(unsigned* p, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0u;
}

// Persistent SYRK: about one workgroup per CU.  The work items (tile,
// split) are listed per XCD as the launched grid assigns them (the
// xcd_chunk range of tile indices of XCD x, split by split); a workgroup
// claims the next item of its own XCD's list (hardware register XCC_ID)
// with an atomic counter and, when that list is empty, items of the other
// lists, so every item runs exactly once wherever the workgroups land.
// The workgroups of an XCD are paced (SyrkPace) so that those working on a
// 4 x 8 block of tiles read the same operand lines while they are in L2.
template <typename T8, bool TM>
__global__ __launch_bounds__(SYRKD_THREADS) void k_syrk16k_pers(
    const uint16_t* __restrict__ X, int64_t ld, int64_t ntok, int64_t tpad, int C, float* S,
    int64_t lds, int nt, int64_t span, int ns, float* P, unsigned* ctl) {
  __shared__ __attribute__((aligned(1024))) uint16_t Xs[2][2][ST][KQ];
  __shared__ int bcast[2];
  int xx;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xx));
  const int x = xx & 7;
  const int ntiles = nt * (nt + 1) / 2;
  const int q = ntiles / 8, r = ntiles % 8;
  unsigned* ctr = ctl + x * PCTL_LINE;
  unsigned* claim = ctl + 8 * PCTL_LINE;
  unsigned* arrive = ctl + 16 * PCTL_LINE + x * PCTL_LINE;
  if (threadIdx.x == 0) {
    // the XCD's workgroups that started with this one: counted after a
    // short settle time (workgroups that start later are not waited for)
    __hip_atomic_fetch_add(arrive, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    __builtin_amdgcn_s_sleep(127);
    __builtin_amdgcn_s_sleep(127);
    bcast[1] = (int)__hip_atomic_fetch_add(arrive, 0u, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  __syncthreads();
  SyrkPace pc{ctr, (unsigned)bcast[1], PACE_LAG, PACE_MAXSPIN, 0u, false};
  // Only the full rounds of the own list are paced: a workgroup leaves the
  // pace for good (adding PACE_RETIRE, above any stage count a paced
  // workgroup can need, so it never holds one back) when it first takes a
  // tile of its list's last round or of another XCD's list.
  bool pacing = true;
  int xs = x;                                    // list being drained
  for (int lists = 0; lists < 8;) {
    const int lin0 = xs < r ? xs * (q + 1) : r * (q + 1) + (xs - r) * q;
    const int nl = xs < r ? q + 1 : q;
    if (threadIdx.x == 0)
      bcast[0] = (int)__hip_atomic_fetch_add(claim + xs * PCTL_LINE, 1u, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const int it = bcast[0];
    __syncthreads();
    const bool paced = pacing && xs == x && it + (int)pc.nwx < nl * ns;
    if (pacing && !paced) {
      pacing = false;
      if (threadIdx.x == 0)
        __hip_atomic_fetch_add(ctr, PACE_RETIRE, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    if (it >= nl * ns) {
      ++lists;
      xs = (xs + 1) & 7;
      continue;
    }
    const int split = it / nl;
    int ti, tj;
    tile_band(lin0 + it % nl, nt, ti, tj);
    const int64_t k_beg = (int64_t)split * span;
    const int64_t k_end = k_beg + span < tpad ? k_beg + span : tpad;
    const int nch = k_end > k_beg ? (int)((k_end - k_beg) / KQ) : 0;
    f4_t acc[8][4];
    pc.on = paced;
    if constexpr (TM) syrk_tile_tm<T8, true>(Xs, X, ld, ntok, ti, tj, k_beg, nch, acc, pc);
    else syrk_tile<T8, true>(Xs, X, ld, ti, tj, k_beg, nch, acc, pc);
    syrk_store(acc, ti, tj, C, S, lds, P, split);
  }
}

// S[i][j] += sum_s P[s][i][j] in split order, upper triangle.  Grid: x =
// row, y = 1024-column chunk; 256 threads, 4 columns each.
// Upper tile id of an nt x nt grid of FT x FT tiles, row by row from the
// last (k_sum_splits, k_finalize).
constexpr int FT = 64;
__device__ __forceinline__ void upper_tile(int id, int nt, int& ti, int& tj) {
  const int k = nt * (nt + 1) / 2 - 1 - id;          // lower-triangle index (r >= b)
  int r = (int)((sqrtf(8.f * (float)k + 1.f) - 1.f) * 0.5f);
  while ((r + 1) * (r + 2) / 2 <= k) ++r;
  while (r * (r + 1) / 2 > k) --r;
  const int b = k - r * (r + 1) / 2;
  ti = nt - 1 - r;
  tj = nt - 1 - b;
}

// S[i][j] += P[0][i][j] + P[1][i][j] + ... (in that order) for j >= i,
// over the 64 x 64 tiles of the upper triangle (the same sums as the
// SYRK's split partials need), 16-byte accesses where S's rows allow.
__global__ __launch_bounds__(256) void k_sum_splits(const float* __restrict__ P, int nsplit,
                                                    int C, float* S, int64_t lds, int nt,
                                                    int vec) {
  int ti, tj;
  upper_tile(blockIdx.x, nt, ti, tj);
  const int r0 = ti * FT, c0 = tj * FT;
  const size_t pstride = (size_t)C * lds;
  const int tid = threadIdx.x;
  if (vec && r0 + FT <= C && c0 + FT <= C) {
    // thread: rows tid / 16 + 16 k, columns 4 (tid % 16) .. + 3
    const int rr = tid >> 4, cc = (tid & 15) * 4;
    float4 v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = *(const float4*)(S + (int64_t)(r0 + rr + 16 * k) * lds + c0 + cc);
    for (int sp = 0; sp < nsplit; ++sp) {
      float4 q[4];
#pragma unroll
      for (int k = 0; k < 4; ++k)
        q[k] = *(const float4*)(P + sp * pstride + (int64_t)(r0 + rr + 16 * k) * lds + c0 + cc);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        v[k].x = v[k].x + q[k].x; v[k].y = v[k].y + q[k].y;
        v[k].z = v[k].z + q[k].z; v[k].w = v[k].w + q[k].w;
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int i = r0 + rr + 16 * k, j = c0 + cc;
      float* d = S + (int64_t)i * lds + j;
      if (j >= i) {
        *(float4*)d = v[k];
      } else if (j + 3 >= i) {                  // the float4 straddles the diagonal
        const float e[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (j + c >= i) d[c] = e[c];
      }
    }
    return;
  }
  const int tx = tid & 63, ty = tid >> 6;
  for (int k = 0; k < FT; k += 4) {
    const int i = r0 + ty + k, j = c0 + tx;
    if (i >= C || j >= C || j < i) continue;
    float v = S[(int64_t)i * lds + j];
    for (int sp = 0; sp < nsplit; ++sp) v = v + P[sp * pstride + (int64_t)i * lds + j];
    S[(int64_t)i * lds + j] = v;
  }
}

static void sum_splits(const float* P, int nsplit, int64_t C, float* S, int64_t lds,
                       hipStream_t s) {
  const int nt = (int)((C + FT - 1) / FT);
  const int vec = (lds & 3) == 0 && ((((uintptr_t)S) | ((uintptr_t)P)) & 15) == 0;
  k_sum_splits<<<(unsigned)((int64_t)nt * (nt + 1) / 2), 256, 0, s>>>(P, nsplit, (int)C, S, lds,
                                                                      nt, vec);
}

// fp32 inputs: LDS in natural token-major layout, A[i][k] = X[k][i].
__global__ __launch_bounds__(256) void k_syrk32(const float* __restrict__ X, int64_t ntok,
                                                int64_t ldx, int C, float* S, int64_t lds,
                                                int nt) {
  __shared__ float Xs[2][HK32][HT + 4];
  int ti, tj;
  tile_of(blockIdx.x, nt, ti, tj);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  const bool diag = ti == tj;
  f4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};
  for (int64_t t0 = 0; t0 < ntok; t0 += HK32) {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int idx = tid + 256 * e;           // 0..4095 = 2 sides x 16 tokens x 128 ch
      const int side = idx >> 11, k = (idx >> 7) & 15, c = idx & 127;
      if (diag && side) continue;
      const int gc = (side ? tj : ti) * HT + c;
      const int64_t t = t0 + k;
      Xs[side][k][c] = (t < ntok && gc < C) ? X[t * ldx + gc] : 0.f;
    }
    __syncthreads();
    const int sj = diag ? 0 : 1;
#pragma unroll
    for (int kk = 0; kk < HK32; kk += 4) {
      const int kr = kk + (lane >> 4), c16 = lane & 15;
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = Xs[0][kr][wm + i * 16 + c16];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Xs[sj][kr][wn + j * 16 + c16];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }
  const int c16 = lane & 15, r4 = (lane >> 4) * 4;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int gi = ti * HT + wm + i * 16 + r4 + r;
        const int gj = tj * HT + wn + j * 16 + c16;
        if (gi < C && gj < C && gi <= gj) {
          float* p = S + (int64_t)gi * lds + gj;
          *p = *p + acc[i][j][r];
        }
      }
}

// H = scale * sym(S) from the upper triangle of S, in 64 x 64 tiles: the
// workgroup of upper tile (ti, tj) stages it in LDS and writes it and its
// mirror (tj, ti) with row-contiguous stores (16-byte accesses when rows
// are 16-byte aligned and the tile lies inside the matrix).  Grid: the
// nt (nt + 1) / 2 upper tiles, row by row from the last.  H may alias S: a
// workgroup reads only its own upper tile, all of it before any store, and
// lower tiles are never read.

__global__ __launch_bounds__(256) void k_finalize(const float* S, int64_t lds, int C,
                                                  float scale, float* H, int64_t ldh, int nt,
                                                  int vec) {
  int ti, tj;
  upper_tile(blockIdx.x, nt, ti, tj);
  __shared__ float T[FT][FT + 1];
  const int tid = threadIdx.x;
  const int r0 = ti * FT, c0 = tj * FT;
  const bool diag = ti == tj;
  if (vec && r0 + FT <= C && c0 + FT <= C) {
    // thread: rows tid / 16 + 16 k, columns 4 (tid % 16) .. + 3
    const int rr = tid >> 4, cc = (tid & 15) * 4;
    float4 v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      v[k] = *(const float4*)(S + (int64_t)(r0 + rr + 16 * k) * lds + c0 + cc);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int r = rr + 16 * k;
      T[r][cc] = scale * v[k].x;
      T[r][cc + 1] = scale * v[k].y;
      T[r][cc + 2] = scale * v[k].z;
      T[r][cc + 3] = scale * v[k].w;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int r = rr + 16 * k;
      float q[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) q[e] = (!diag || r <= cc + e) ? T[r][cc + e] : T[cc + e][r];
      *(float4*)(H + (int64_t)(r0 + r) * ldh + c0 + cc) = make_float4(q[0], q[1], q[2], q[3]);
    }
    if (diag) return;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int r = rr + 16 * k;
      *(float4*)(H + (int64_t)(c0 + r) * ldh + r0 + cc) =
          make_float4(T[cc][r], T[cc + 1][r], T[cc + 2][r], T[cc + 3][r]);
    }
    return;
  }
  const int tx = tid & 63, ty = tid >> 6;
#pragma unroll
  for (int k = 0; k < FT; k += 4) {
    const int r = r0 + ty + k, c = c0 + tx;
    float v = 0.f;
    if (r < C && c < C && r <= c) v = scale * S[(int64_t)r * lds + c];
    T[ty + k][tx] = v;
  }
  __syncthreads();
  if (diag) {
#pragma unroll
    for (int k = 0; k < FT; k += 4) {
      const int r = ty + k, c = tx;
      if (r0 + r < C && c0 + c < C)
        H[(int64_t)(r0 + r) * ldh + c0 + c] = r <= c ? T[r][c] : T[c][r];
    }
    return;
  }
#pragma unroll
  for (int k = 0; k < FT; k += 4) {
    const int r = r0 + ty + k, c = c0 + tx;
    if (r < C && c < C) H[(int64_t)r * ldh + c] = T[ty + k][tx];
  }
#pragma unroll
  for (int k = 0; k < FT; k += 4) {
    const int r = c0 + ty + k, c = r0 + tx;
    if (r < C && c < C) H[(int64_t)r * ldh + c] = T[tx][ty + k];
  }
}

}  // namespace crbq

namespace crbq {
// CUs of the current device, per device (thread-safe: one query each)
static int num_cus() {
  constexpr int MAXDEV = 64;
  static std::atomic<int> cus[MAXDEV] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAXDEV) return 256;
  int v = cus[dev].load(std::memory_order_relaxed);
  if (v > 0) return v;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      v <= 0)
    v = 256;
  cus[dev].store(v, std::memory_order_relaxed);
  return v;
}

// Split count for the 16-bit kernel: minimise the modelled time of
// ceil(tiles*ns / CUs) rounds of ceil(T/ns) tokens plus the partial-tile
// write/read traffic (ns * C^2 floats, twice).
static int choose_splits(int64_t ntok, int64_t C, int cus) {
  const int64_t nt = (C + ST - 1) / ST;
  const int64_t tiles = nt * (nt + 1) / 2;
  const double tok_s = 2.0 * ST * ST / (4096.0 * 2.4e9 * 0.6);   // one WG, one token
  double best_t = 0.0;
  int best = 1;
  for (int ns = 1; ns <= 16; ++ns) {
    if (ns > 1 && ntok / ns < 2048) break;
    const int64_t rounds = (tiles * ns + cus - 1) / cus;
    const int64_t per = (ntok + ns - 1) / ns;
    double t = (double)rounds * (double)per * tok_s;
    if (ns > 1) t += 2.0 * ns * (double)C * C * 4.0 / 5e12;
    if (ns == 1 || t < best_t) { best_t = t; best = ns; }
  }
  return best;
}
}  // namespace crbq

namespace crbq {
// SYRK launch timing (crbq_syrk_timing): while enabled, every SYRK kernel
// launch of crbq_hessian_accum is bracketed by two HIP events recorded on
// the launch's stream.
struct SyrkRec {
  hipEvent_t a, b;
  int64_t C;
};
static std::mutex g_tmu;
static bool g_timing = false;
static std::vector<SyrkRec> g_recs;

struct SyrkTimer {
  SyrkRec r{nullptr, nullptr, 0};
  bool on = false;
  SyrkTimer(hipStream_t s, int64_t C) {
    {
      std::lock_guard<std::mutex> g(g_tmu);
      on = g_timing;
    }
    if (!on) return;
    r.C = C;
    if (hipEventCreate(&r.a) != hipSuccess || hipEventCreate(&r.b) != hipSuccess ||
        hipEventRecord(r.a, s) != hipSuccess)
      on = false;
  }
  void stop(hipStream_t s) {
    if (!on || hipEventRecord(r.b, s) != hipSuccess) return;
    std::lock_guard<std::mutex> g(g_tmu);
    g_recs.push_back(r);
    on = false;
  }
};

// Geometry of the channel-major path: a call of ntok tokens runs in passes
// of at most tch tokens, each transposed into Xt[Cp][ldt].  A pass's Xt is
// at most 8 GiB, and ldt <= 2^21 keeps a tile's 256-row panel of Xt below
// the 2^31-byte reach of a buffer load's offsets.  The environment variable
// CRBQ_XT_PASS_TOKENS lowers the pass length (tests use it to run several
// passes on small inputs).
struct XtPlan {
  int64_t Cp, tch, ldt;
  size_t xt_bytes;    // 256-byte aligned
};
static XtPlan xt_plan(int64_t ntok, int64_t C) {
  XtPlan p;
  p.Cp = (C + ST - 1) / ST * ST;
  int64_t cap = ((int64_t)1 << 33) / (2 * p.Cp);
  cap = cap < ((int64_t)1 << 21) ? cap : ((int64_t)1 << 21);
  if (const char* e = getenv("CRBQ_XT_PASS_TOKENS")) {
    const long long v = atoll(e);
    if (v > 0 && v < cap) cap = v;
  }
  cap = cap / KQ * KQ;
  if (cap < KQ) cap = KQ;
  p.tch = ntok < cap ? ntok : cap;
  p.ldt = (p.tch + KQ - 1) / KQ * KQ;
  p.xt_bytes = ((size_t)p.Cp * (size_t)p.ldt * 2 + 255) & ~(size_t)255;
  return p;
}
}  // namespace crbq

namespace crbq {
// SYRK of a channel-major operand Xt[Cp][ldt] (rows >= C and tokens in
// [ntok, tpad) zero, tpad a multiple of KQ, ldt >= tpad): token splits
// chosen by the cost model within the partial-tile capacity pcap, split 0
// adding into S and the others summed after it in split order.
// Channel counts from which the persistent paced SYRK is used (its
// control words at the end of the workspace): the fc2-sized inputs, whose
// SYRK fills the GPU for tens of milliseconds.  Smaller SYRKs keep the
// launched grid, whose short workgroups leave CUs to other streams' work.
constexpr int64_t PERS_MIN_C = 8192;
static size_t syrk_ctl_bytes(int64_t C) { return C >= PERS_MIN_C ? PCTL_BYTES + 256 : 0; }

// tmaj: X is the token-major activation itself (ld its row stride, ntok
// valid rows, tpad = ntok rounded up to KQ; C a multiple of 256); else the
// channel-major copy (ld its row stride, ntok unused).
static int syrk_xt(const uint16_t* X, int64_t ld, int64_t ntok, bool tmaj, int64_t tpad,
                   int64_t C, float* S, int64_t lds, float* Pbuf, size_t pcap, int dtype,
                   hipStream_t s) {
  const int nt = (int)((C + ST - 1) / ST);
  const int64_t ntiles = (int64_t)nt * (nt + 1) / 2;
  // control words of the persistent kernel at the end of the workspace
  unsigned* ctl = nullptr;
  if (C >= PERS_MIN_C && Pbuf && pcap >= syrk_ctl_bytes(C)) {
    const uintptr_t end = (uintptr_t)Pbuf + pcap - PCTL_BYTES;
    ctl = (unsigned*)(end & ~(uintptr_t)255);
    pcap = (size_t)((uintptr_t)ctl - (uintptr_t)Pbuf);
  }
  int ns = choose_splits(tpad, C, num_cus());
  while (ns > 1 && (size_t)ns * (size_t)C * (size_t)lds * sizeof(float) > pcap) --ns;
  int64_t span = (tpad + ns - 1) / ns;
  span = (span + KQ - 1) / KQ * KQ;
  ns = (int)((tpad + span - 1) / span);
  float* P = ns > 1 ? Pbuf : nullptr;
  if (ctl) {
    k_zero_u32<<<1, 256, 0, s>>>(ctl, (int)(PCTL_BYTES / sizeof(unsigned)));
    CRBQ_LAUNCH_CHECK();
  }
  SyrkTimer tm(s, C);
  if (ctl) {
    const unsigned nwg = (unsigned)num_cus();
#define CRBQ_PERS_GO(T8_, TM_)                                                              \
  k_syrk16k_pers<T8_, TM_><<<nwg, SYRKD_THREADS, 0, s>>>(X, ld, ntok, tpad, (int)C, S, lds, \
                                                         nt, span, ns, P, ctl)
    if (dtype == CRBQ_F16) {
      if (tmaj) CRBQ_PERS_GO(h8_t, true); else CRBQ_PERS_GO(h8_t, false);
    } else {
      if (tmaj) CRBQ_PERS_GO(b8_t, true); else CRBQ_PERS_GO(b8_t, false);
    }
#undef CRBQ_PERS_GO
  } else {
    dim3 grid((unsigned)ntiles, (unsigned)ns);
#define CRBQ_GRID_GO(T8_, TM_)                                                                 \
  k_syrk16k<T8_, TM_><<<grid, SYRKD_THREADS, 0, s>>>(X, ld, ntok, tpad, (int)C, S, lds, nt, \
                                                     span, P)
    if (dtype == CRBQ_F16) {
      if (tmaj) CRBQ_GRID_GO(h8_t, true); else CRBQ_GRID_GO(h8_t, false);
    } else {
      if (tmaj) CRBQ_GRID_GO(b8_t, true); else CRBQ_GRID_GO(b8_t, false);
    }
#undef CRBQ_GRID_GO
  }
  CRBQ_LAUNCH_CHECK();
  tm.stop(s);
  if (P) {
    sum_splits(P, ns - 1, C, S, lds, s);
    CRBQ_LAUNCH_CHECK();
  }
  return CRBQ_OK;
}
}  // namespace crbq

extern "C" size_t crbq_hessian_workspace_size(int64_t ntok, int64_t C) {
  if (ntok <= 0 || C <= 0) return 0;
  if (C % crbq::ST == 0) {
    // token-major stages: split partials and control words only
    const int64_t tpad = (ntok + crbq::KQ - 1) / crbq::KQ * crbq::KQ;
    const int ns = crbq::choose_splits(tpad, C, crbq::num_cus());
    return (ns > 1 ? (size_t)ns * (size_t)C * (size_t)C * sizeof(float) : 0) +
           crbq::syrk_ctl_bytes(C);
  }
  const crbq::XtPlan pl = crbq::xt_plan(ntok, C);
  const int64_t tpad = (pl.tch + crbq::KQ - 1) / crbq::KQ * crbq::KQ;
  const int ns = crbq::choose_splits(tpad, C, crbq::num_cus());
  return pl.xt_bytes + (ns > 1 ? (size_t)ns * (size_t)C * (size_t)C * sizeof(float) : 0) +
         crbq::syrk_ctl_bytes(C);
}

extern "C" int crbq_hessian_accum(const void* X, int dtype, int64_t ntok, int64_t ldx,
                                  int64_t C, float* S, int64_t lds, void* ws, size_t ws_bytes,
                                  void* stream) {
  if (!X || !S || C <= 0 || ntok < 0 || ldx < C || lds < C) return CRBQ_ERR_ARG;
  if (C > (1 << 20)) return CRBQ_ERR_ARG;
  if (ntok == 0) return CRBQ_OK;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == CRBQ_F32) {
    const int nt = (int)((C + crbq::HT - 1) / crbq::HT);
    const int64_t ntiles = (int64_t)nt * (nt + 1) / 2;
    if (ntiles > 0x7fffffff) return CRBQ_ERR_ARG;
    crbq::k_syrk32<<<(unsigned)ntiles, 256, 0, s>>>((const float*)X, ntok, ldx, (int)C, S,
                                                    lds, nt);
    CRBQ_LAUNCH_CHECK();
    return CRBQ_OK;
  }
  if (dtype != CRBQ_F16 && dtype != CRBQ_BF16) return CRBQ_ERR_ARG;
  const int nt = (int)((C + crbq::ST - 1) / crbq::ST);
  const int64_t ntiles = (int64_t)nt * (nt + 1) / 2;
  if (ntiles > 0x7fffffff) return CRBQ_ERR_ARG;
  const bool fast = (C % 8 == 0) && (ldx % 8 == 0) && ((((uintptr_t)X) & 15) == 0);
  if (fast && C % crbq::ST == 0 && ldx < ((int64_t)1 << 24)) {
    // token-major stages straight from X (no transposed copy); the
    // workspace holds the split partials and the control words
    const int64_t tpad = (ntok + crbq::KQ - 1) / crbq::KQ * crbq::KQ;
    return crbq::syrk_xt((const uint16_t*)X, ldx, ntok, true, tpad, C, S, lds, (float*)ws,
                         ws ? ws_bytes : 0, dtype, s);
  }
  const crbq::XtPlan pl = crbq::xt_plan(ntok, C);
  if (ws && ws_bytes >= pl.xt_bytes) {
    // channel-major path: transpose each pass into the workspace, then SYRK
    uint16_t* Xt = (uint16_t*)ws;
    float* Pbuf = (float*)((char*)ws + pl.xt_bytes);
    const size_t pcap = ws_bytes - pl.xt_bytes;
    for (int64_t t0 = 0; t0 < ntok; t0 += pl.tch) {
      const int64_t n = ntok - t0 < pl.tch ? ntok - t0 : pl.tch;
      const int64_t tpad = (n + crbq::KQ - 1) / crbq::KQ * crbq::KQ;
      const uint16_t* Xc = (const uint16_t*)X + t0 * ldx;
      const int64_t nw = (tpad / 64) * (pl.Cp / 64);
      const unsigned nblk = crbq::xpose_blocks(nw);
      if (fast)
        crbq::k_xpose16<true><<<nblk, 256, 0, s>>>(Xc, n, ldx, (int)C, Xt, pl.ldt, tpad,
                                                   (int)pl.Cp);
      else
        crbq::k_xpose16<false><<<nblk, 256, 0, s>>>(Xc, n, ldx, (int)C, Xt, pl.ldt, tpad,
                                                    (int)pl.Cp);
      CRBQ_LAUNCH_CHECK();
      const int st = crbq::syrk_xt(Xt, pl.ldt, 0, false, tpad, C, S, lds, Pbuf, pcap, dtype, s);
      if (st) return st;
    }
    return CRBQ_OK;
  }
  // token-major path (workspace too small for the transposed copy)
  int ns = crbq::choose_splits(ntok, C, crbq::num_cus());
  // the partial buffers are laid out like S (row stride lds)
  while (ns > 1 && (!ws || (size_t)ns * (size_t)C * (size_t)lds * sizeof(float) > ws_bytes)) --ns;
  int64_t span = (ntok + ns - 1) / ns;
  span = (span + crbq::SKQ - 1) / crbq::SKQ * crbq::SKQ;
  ns = (int)((ntok + span - 1) / span);
  float* P = ns > 1 ? (float*)ws : nullptr;
  dim3 grid((unsigned)ntiles, (unsigned)ns);
  crbq::SyrkTimer tm(s, C);
#define CRBQ_SYRK_GO(T8_, F_)                                                            \
  crbq::k_syrk16p<T8_, F_><<<grid, crbq::SYRKP_THREADS, 0, s>>>(                         \
      (const uint16_t*)X, ntok, ldx, (int)C, S, lds, nt, span, P)
  if (dtype == CRBQ_F16) {
    if (fast) CRBQ_SYRK_GO(h8_t, true); else CRBQ_SYRK_GO(h8_t, false);
  } else {
    if (fast) CRBQ_SYRK_GO(b8_t, true); else CRBQ_SYRK_GO(b8_t, false);
  }
#undef CRBQ_SYRK_GO
  CRBQ_LAUNCH_CHECK();
  tm.stop(s);
  if (P) {
    crbq::sum_splits(P, ns - 1, C, S, lds, s);
    CRBQ_LAUNCH_CHECK();
  }
  return CRBQ_OK;
}

extern "C" int crbq_hessian_cm_shape(int64_t ntok, int64_t C, int64_t* rows, int64_t* ldt) {
  if (!rows || !ldt || ntok <= 0 || C <= 0 || C > (1 << 20)) return CRBQ_ERR_ARG;
  const int64_t tpad = (ntok + crbq::KQ - 1) / crbq::KQ * crbq::KQ;
  if (tpad > ((int64_t)1 << 21)) return CRBQ_ERR_ARG;
  *rows = (C + crbq::ST - 1) / crbq::ST * crbq::ST;
  *ldt = tpad;
  return CRBQ_OK;
}

extern "C" int crbq_hessian_transpose(const void* X, int dtype, int64_t ntok, int64_t ldx,
                                      int64_t C, void* Xt, int64_t ldt, int64_t t0,
                                      void* stream) {
  if (!X || !Xt || ntok <= 0 || C <= 0 || C > (1 << 20) || ldx < C) return CRBQ_ERR_ARG;
  if (dtype != CRBQ_F16 && dtype != CRBQ_BF16) return CRBQ_ERR_ARG;
  if (t0 < 0 || t0 % crbq::KQ || ldt % crbq::KQ || ldt > ((int64_t)1 << 21)) return CRBQ_ERR_ARG;
  const int64_t tpad = (ntok + crbq::KQ - 1) / crbq::KQ * crbq::KQ;
  if (t0 + tpad > ldt) return CRBQ_ERR_ARG;
  if ((((uintptr_t)Xt) & 15) != 0) return CRBQ_ERR_ARG;
  const int64_t Cp = (C + crbq::ST - 1) / crbq::ST * crbq::ST;
  const bool fast = (C % 8 == 0) && (ldx % 8 == 0) && ((((uintptr_t)X) & 15) == 0);
  const int64_t nw = (tpad / 64) * (Cp / 64);
  const unsigned nblk = crbq::xpose_blocks(nw);
  uint16_t* dst = (uint16_t*)Xt + t0;
  hipStream_t s = (hipStream_t)stream;
  if (fast)
    crbq::k_xpose16<true><<<nblk, 256, 0, s>>>((const uint16_t*)X, ntok, ldx, (int)C, dst, ldt,
                                               tpad, (int)Cp);
  else
    crbq::k_xpose16<false><<<nblk, 256, 0, s>>>((const uint16_t*)X, ntok, ldx, (int)C, dst,
                                                ldt, tpad, (int)Cp);
  CRBQ_LAUNCH_CHECK();
  return CRBQ_OK;
}

extern "C" size_t crbq_hessian_cm_workspace_size(int64_t ntok, int64_t C) {
  if (ntok <= 0 || C <= 0) return 0;
  const int64_t tpad = (ntok + crbq::KQ - 1) / crbq::KQ * crbq::KQ;
  const int ns = crbq::choose_splits(tpad, C, crbq::num_cus());
  return (ns > 1 ? (size_t)ns * (size_t)C * (size_t)C * sizeof(float) : 0) +
         crbq::syrk_ctl_bytes(C);
}

extern "C" int crbq_hessian_accum_cm(const void* Xt, int dtype, int64_t ntok, int64_t ldt,
                                     int64_t C, float* S, int64_t lds, void* ws,
                                     size_t ws_bytes, void* stream) {
  if (!Xt || !S || C <= 0 || C > (1 << 20) || ntok < 0 || lds < C) return CRBQ_ERR_ARG;
  if (dtype != CRBQ_F16 && dtype != CRBQ_BF16) return CRBQ_ERR_ARG;
  if (ntok == 0) return CRBQ_OK;
  const int64_t tpad = (ntok + crbq::KQ - 1) / crbq::KQ * crbq::KQ;
  if (ldt % crbq::KQ || ldt < tpad || ldt > ((int64_t)1 << 21)) return CRBQ_ERR_ARG;
  if ((((uintptr_t)Xt) & 15) != 0) return CRBQ_ERR_ARG;
  const int nt = (int)((C + crbq::ST - 1) / crbq::ST);
  if ((int64_t)nt * (nt + 1) / 2 > 0x7fffffff) return CRBQ_ERR_ARG;
  return crbq::syrk_xt((const uint16_t*)Xt, ldt, 0, false, tpad, C, S, lds, (float*)ws,
                       ws ? ws_bytes : 0,
                       dtype, (hipStream_t)stream);
}

extern "C" int crbq_syrk_timing(int on) {
  std::lock_guard<std::mutex> g(crbq::g_tmu);
  crbq::g_timing = on != 0;
  return CRBQ_OK;
}

extern "C" int crbq_syrk_timing_collect(float* ms, int64_t* C, int max, int* n) {
  if (!n || max < 0 || (max > 0 && (!ms || !C))) return CRBQ_ERR_ARG;
  std::vector<crbq::SyrkRec> recs;
  {
    std::lock_guard<std::mutex> g(crbq::g_tmu);
    recs.swap(crbq::g_recs);
  }
  int k = 0, rc = CRBQ_OK;
  for (const crbq::SyrkRec& r : recs) {
    float t = 0.f;
    if (hipEventSynchronize(r.b) != hipSuccess || hipEventElapsedTime(&t, r.a, r.b) != hipSuccess)
      rc = CRBQ_ERR_HIP;
    if (k < max) {
      ms[k] = t;
      C[k] = r.C;
    }
    ++k;
    (void)hipEventDestroy(r.a);
    (void)hipEventDestroy(r.b);
  }
  *n = k;
  return rc;
}

extern "C" int crbq_hessian_finalize(const float* S, int64_t lds, int64_t C, float scale,
                                     float* H, int64_t ldh, void* stream) {
  if (!S || !H || C <= 0 || C > (1 << 20) || lds < C || ldh < C) return CRBQ_ERR_ARG;
  const int nt = (int)((C + crbq::FT - 1) / crbq::FT);
  const int vec = ((lds | ldh) & 3) == 0 && ((((uintptr_t)S) | ((uintptr_t)H)) & 15) == 0;
  crbq::k_finalize<<<(unsigned)(nt * (nt + 1) / 2), 256, 0, (hipStream_t)stream>>>(
      S, lds, (int)C, scale, H, ldh, nt, vec);
  CRBQ_LAUNCH_CHECK();
  return CRBQ_OK;
}
