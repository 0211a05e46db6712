// The 128-column block loop of BRAGPTQ.fasterquant (bigptq.py:131-264) on
// gfx950: salient-column search, bell-shaped split, binarization, Err/Loss
// and the GPTQ trailing update.
//
// Search of one block (utils/structure.py:8-20 -> utils/autosearch.py:28-83
// -> utils/mask.py:7-18), all on the device with no host round trip:
//   k_colscore   column scores sum_r |T| (fp64 per-workgroup partials);
//                the last workgroup ranks the columns (torch.topk order)
//   k_phase_a_rows  lanes = 64 rows, wavefront = salient candidate i:
//                order-2 residual binarization error of {top i cols} +
//                complement (group sums from fp64 chunk sums, two passes,
//                closed-form error); the last workgroup takes
//                i* = first strict minimum
//   k_qpass1, k_qlist, k_qselect
//                exact np.quantile of |T * ~M3| at the 81 float32
//                percentiles: level-1 histogram of the top 12 bits of the
//                non-negative float's bit pattern, the bins of the 162
//                order statistics, the elements of those bins gathered into
//                per-bin lists, one selection workgroup per statistic; then
//                numpy's float32 index/lerp arithmetic
//   k_phase_c    per row a sorted copy with fp64 prefix sums; the
//                workgroup's (row, split candidate k) pairs over its lanes:
//                order-1 errors of the two bell groups in closed form;
//                the last workgroup takes k* = first strict minimum,
//                split = p[k*]
//   k_quantize   one wavefront per row: masks, binarization per group,
//                Q, Err = (w-q)/d, Loss = (w-q)^2/d^2
// then sgemm_launch for W[:, ed:] -= Err @ U[st:ed, ed:].
//
// T = W^2 / diag(U_blk)^2 (hessian metric) or W (magnitude) is recomputed
// from W on every pass instead of being stored.
#include <atomic>
#include <mutex>

#include "binarize.h"
#include "gemm_f32.h"

namespace crbq {

constexpr int NQ = 81;       // percentiles linspace(0.10, 0.90, 81)
constexpr int NT = 2 * NQ;   // order statistics needed (lo, hi per percentile)
constexpr int NCMAX = 128;   // widest block
constexpr int UPMAX = 64;    // largest supported up_lim
#ifndef CRBQ_Q_RPW
#define CRBQ_Q_RPW 32
#endif
constexpr int Q_RPW = CRBQ_Q_RPW;   // rows per workgroup in the quantile passes
#ifndef CRBQ_CS_MAXWG
#define CRBQ_CS_MAXWG 128
#endif
constexpr int CS_MAXWG = CRBQ_CS_MAXWG;   // colscore partials
#ifndef CRBQ_PX_MAXWG
#define CRBQ_PX_MAXWG 256
#endif
constexpr int PX_MAXWG = CRBQ_PX_MAXWG;  // phase A / C partials
constexpr int H1_BITS = 12, H2_BITS = 10, H3_BITS = 10;   // 12 + 10 + 10 = 32
constexpr int H1 = 1 << H1_BITS, H2 = 1 << H2_BITS, H3 = 1 << H3_BITS;
constexpr int SH1 = H2_BITS + H3_BITS, SH2 = H3_BITS;     // key = b1<<SH1 | b2<<SH2 | b3
constexpr int NONE = 0x7fffffff;
// The level-2 histogram of the radix select, the one most elements reach,
// is kept once per XCD: a workgroup adds into the copy of the XCD it runs
// on (hardware register XCC_ID) with workgroup-scope atomics, which
// complete in that XCD's L2 instead of travelling to memory as device-scope
// atomics do; the level-2 scan sums the copies.  Kernel boundaries write
// the L2s back, so the next launch sees every copy.
constexpr int NXCD = 8;

// torch.linspace(0.10, 0.90, 81) on the CPU (utils/autosearch.py:65), float32.
__constant__ float c_q[NQ];

struct Ctrl {        // small per-block control record (device)
  int istar;
  int kstar;
  int ncand_a;
  int pad;
  float split;
  uint32_t cnt[4];   // arrival counters of the last-workgroup reductions
};
enum { CNT_CS = 0, CNT_A = 1, CNT_C = 2 };

struct Tgt {         // one order statistic being selected
  int64_t rank;      // absolute rank in the sorted flattened block
  int bin1, r1;      // level-1 bin and rank within it
  int slot1;         // leader target index of bin1 (the first target in it)
};

struct SearchWs {
  double* colpart;   // [nwg_cs][NCMAX]
  int* rank;         // [NCMAX]
  Ctrl* ctrl;
  double* parta;     // [nwg_a][UPMAX]
  double* partc;     // [nwg_c][96]
  uint32_t* hist1;   // [H1]
  Tgt* tgt;          // [NT]
  float* gam;        // [NQ]
  int* list_off;     // [NT]: start of each leader target's element list
  int* list_cnt;     // [NT]: elements appended to it
  uint32_t* lists;   // [R * NCMAX]: bit patterns of the elements of every target bin
  float* tval;       // [NT]
  float* pvals;      // [NQ]
};

// Sublayers of one shape (q/k/v/out of an attention block, Llama's
// gate/up) run one block loop together: every search and quantize launch
// covers up to NSEG of them, blockIdx.y selecting the sublayer (its
// weights, inverse factor, search scratch and trace), and each sublayer's
// work is exactly that of a launch of its own (same workgroups, same
// reductions, same bits).
constexpr int NSEG = 4;
struct SegSearch {
  const float* W[NSEG];
  const float* U[NSEG];   // the block's diagonal corner of each factor
  SearchWs s[NSEG];
  crbq_block_trace* tr[NSEG];
};

static inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

static void carve_search(WsCarver& c, int64_t R, SearchWs& s) {
  s.colpart = c.take<double>((size_t)CS_MAXWG * NCMAX);
  s.rank = c.take<int>(NCMAX);
  s.ctrl = c.take<Ctrl>(1);
  s.parta = c.take<double>((size_t)PX_MAXWG * UPMAX);
  s.partc = c.take<double>((size_t)PX_MAXWG * 96);
  s.hist1 = c.take<uint32_t>(H1);
  s.tgt = c.take<Tgt>(NT);
  s.gam = c.take<float>(NQ);
  s.list_off = c.take<int>(NT);
  s.list_cnt = c.take<int>(NT);
  s.lists = c.take<uint32_t>((size_t)R * NCMAX);
  s.tval = c.take<float>(NT);
  s.pvals = c.take<float>(NQ);
}

__device__ __forceinline__ int xcd_id() {
  int x;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
  return x & (NXCD - 1);
}

// Salient-search target T (utils/structure.py:9-12).
__device__ __forceinline__ float target_of(float w, float d2, int metric) {
  if (metric == CRBQ_METRIC_HESSIAN) {
    const float w2 = w * w;
    return w2 / d2;
  }
  return w;
}

// ---------------------------------------------------------------------------
// last-workgroup reductions
// ---------------------------------------------------------------------------
// Every workgroup calls this after writing its partial results.  It returns
// true in exactly one workgroup, the last to arrive, which then sees every
// other workgroup's partials, and resets the counter for the next launch.
// The partials travel through device-coherent accesses (pstore / pload:
// agent-scope atomic stores and loads, written through to and read from
// the point of coherence of all XCDs), so the arrival needs no cache-wide
// release / acquire fences (an L2 write-back and invalidate per workgroup):
// every thread waits for its own partial stores to be acknowledged before
// the barrier that precedes the arrival on the counter, and the last
// workgroup reads the partials only after its arrival returned.
__device__ __forceinline__ void pstore(double* p, double v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ double pload(const double* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ bool last_block(uint32_t* cnt) {
  __shared__ bool last;
  // The waitcnt builtin is no memory access, so a compiler barrier keeps
  // every partial store of this thread ahead of it; the hardware then waits
  // until those stores are acknowledged (vmcnt counts them: they are vector
  // memory stores), i.e. written through to the coherence point.
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): this thread's stores acknowledged
  asm volatile("" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev = atomicAdd(cnt, 1u);
    last = prev == gridDim.x - 1;
    if (last) atomicExch(cnt, 0u);
  }
  __syncthreads();
  return last;
}

// Fixed-order sum of nwg partials (row stride `stride` doubles) for `ncand`
// candidates with NK * PARTS threads: thread (k, pp) adds partials
// g = pp * G .. pp * G + G - 1 (G = ceil(nwg / PARTS) <= GMAX) of candidate
// k in order, loading all of them before the first add (the partials were
// written by other workgroups, so every load goes out to memory: one round
// trip instead of one per batch), then the PARTS subtotals in order.
// Result in out[0..ncand).
template <int NK, int PARTS, int GMAX>
__device__ void reduce_partials(const double* part, int stride, int nwg, int ncand,
                                double (*red)[NK], double* out) {
  const int t = threadIdx.x, k = t % NK, pp = t / NK;
  const int G = (nwg + PARTS - 1) / PARTS;
  double v = 0.0;
  if (k < ncand && pp < PARTS) {
    double x[GMAX];
#pragma unroll
    for (int j = 0; j < GMAX; ++j) {
      const int g = pp * G + j;
      x[j] = (j < G && g < nwg) ? pload(&part[(size_t)g * stride + k]) : 0.0;
    }
#pragma unroll
    for (int j = 0; j < GMAX; ++j) v += x[j];
  }
  if (pp < PARTS) red[pp][k] = v;
  __syncthreads();
  if (t < ncand) {
    double a = 0.0;
    for (int q = 0; q < PARTS; ++q) a += red[q][t];
    out[t] = a;
  }
  __syncthreads();
}

// Index of the first strict minimum of v[0..n) (the reference's
// `if e < best` scan from best = inf), or -1 when no value is below
// infinity (NaN never wins); computed by the calling wavefront, every lane
// gets the result.  Each lane scans its indices in ascending order, then
// pairs combine keeping the smaller value and, on equal values, the
// smaller index.
__device__ int wave_argmin(const double* v, int n) {
  const int lane = threadIdx.x & 63;
  double b = INFINITY;
  int bi = 0x7fffffff;
  for (int j = lane; j < n; j += 64)
    if (v[j] < b) { b = v[j]; bi = j; }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const double ob = __shfl_xor(b, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    if (ob < b || (ob == b && oi < bi)) { b = ob; bi = oi; }
  }
  return bi == 0x7fffffff ? -1 : bi;
}

// ---------------------------------------------------------------------------
// column scores -> ranks (torch.topk order); zeroing of this block's
// selection histograms
// ---------------------------------------------------------------------------
#ifndef CRBQ_CS_PH
#define CRBQ_CS_PH 8
#endif
constexpr int CS_PH = CRBQ_CS_PH;            // row phases per workgroup
constexpr int CS_THREADS = NCMAX * CS_PH;
__global__ __launch_bounds__(CS_THREADS) void k_colscore(
    SegSearch seg, int64_t ldw, int R, int nc, int64_t ldu,
    int metric) {
  const float* __restrict__ W = seg.W[blockIdx.y];
  const float* __restrict__ U = seg.U[blockIdx.y];
  const SearchWs s = seg.s[blockIdx.y];
  __shared__ double part[CS_PH][NCMAX];
  __shared__ double red[CS_PH][NCMAX];
  __shared__ double sc[NCMAX];
  const int tid = threadIdx.x, col = tid & (NCMAX - 1), ph = tid / NCMAX;
  double acc = 0.0;
  if (col < nc) {
    const float dg = U[(int64_t)col * ldu + col];
    const float d2 = dg * dg;
#pragma unroll 4
    for (int r = CS_PH * blockIdx.x + ph; r < R; r += CS_PH * gridDim.x)
      acc += (double)fabsf(target_of(W[(int64_t)r * ldw + col], d2, metric));
  }
  part[ph][col] = acc;
  // zero the level-1 histogram used later by this block (grid-stride)
  const size_t gsz = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + tid; i < (size_t)H1; i += gsz) s.hist1[i] = 0u;
  if (blockIdx.x == 0 && tid < NT) s.list_cnt[tid] = 0;       // k_qlist's list counters
  __syncthreads();
  if (ph == 0) {
    double v = 0.0;
#pragma unroll
    for (int q = 0; q < CS_PH; ++q) v += part[q][col];
    pstore(&s.colpart[(size_t)blockIdx.x * NCMAX + col], v);
  }
  if (!last_block(&s.ctrl->cnt[CNT_CS])) return;
  reduce_partials<NCMAX, CS_PH, CS_MAXWG / CS_PH>(s.colpart, NCMAX, gridDim.x, NCMAX, red, sc);
  // rank of column c by descending score, ties to the lower column: phase
  // ph counts the columns k = ph, ph + CS_PH, ... that precede c
  __shared__ int cntp[CS_PH][NCMAX];
  {
    const int c = col;
    const double v = sc[c];
    int r = 0;
    if (c < nc)
      for (int k = ph; k < nc; k += CS_PH) r += (sc[k] > v) || (sc[k] == v && k < c);
    cntp[ph][c] = r;
  }
  __syncthreads();
  if (tid < NCMAX) {
    const int c = tid;
    int r = NCMAX;
    if (c < nc) {
      r = 0;
#pragma unroll
      for (int q = 0; q < CS_PH; ++q) r += cntp[q][c];
    }
    s.rank[c] = r;
  }
}

// ---------------------------------------------------------------------------
// phase A: error of order-2 residual binarization of {rank < i} and its
// complement, for candidates i = 1..up_lim-1 (utils/autosearch.py:44-55);
// the last workgroup picks i* = first strict minimum (default
// max(1, up_lim // 3), :43)
// ---------------------------------------------------------------------------
struct ParA {           // a group's fp32 parameters for the residual pass
  float m1, hi, lo, m2, a1;   // hi = fl(a1 + m1), lo = fl(-a1 + m1)
};

// The kernel (k_phase_a_rows) follows the sorting helpers below.

// ---------------------------------------------------------------------------
// exact float32 np.quantile of S = |T * ~M3| (utils/autosearch.py:62-68)
// ---------------------------------------------------------------------------
// The passes' per-thread elements: element i = tid + 256 k of the
// workgroup's rows (row r0 + i / nc, column i % nc).  Every load of W is
// issued before any is used, so the loads overlap instead of each waiting
// out a memory latency.
constexpr int QE = Q_RPW * NCMAX / 256;
static_assert(QE * 256 == Q_RPW * NCMAX, "quantile pass geometry");

__device__ __forceinline__ void q_load(const float* __restrict__ W, int64_t ldw, int r0, int r1,
                                       int nc, float (&w)[QE], int (&col)[QE]) {
  const int n = (r1 - r0) * nc;
#pragma unroll
  for (int k = 0; k < QE; ++k) {
    const int i = threadIdx.x + 256 * k;
    col[k] = -1;
    w[k] = 0.f;
    if (i < n) {
      const int r = r0 + i / nc, c = i - (i / nc) * nc;
      col[k] = c;
      w[k] = W[(int64_t)r * ldw + c];
    }
  }
}

// rank and squared U diagonal of every column into LDS
__device__ __forceinline__ void q_cols(const float* __restrict__ U, int64_t ldu, int nc,
                                       const SearchWs& s, int* rk, float* d2s) {
  const int c = threadIdx.x;
  if (c < NCMAX) {
    rk[c] = s.rank[c];
    if (c < nc) { const float dg = U[(int64_t)c * ldu + c]; d2s[c] = dg * dg; }
  }
}

// Level-1: histogram of bits [31:20] of the (non-negative) float pattern.
__global__ __launch_bounds__(256) void k_qpass1(
    SegSearch seg, int64_t ldw, int R, int nc, int64_t ldu,
    int metric) {
  const float* __restrict__ W = seg.W[blockIdx.y];
  const float* __restrict__ U = seg.U[blockIdx.y];
  const SearchWs s = seg.s[blockIdx.y];
  __shared__ uint32_t lh[H1];
  __shared__ float d2s[NCMAX];
  __shared__ int rk[NCMAX];
  const int tid = threadIdx.x;
  const int r0 = blockIdx.x * Q_RPW, r1 = min(R, r0 + Q_RPW);
  float w[QE];
  int col[QE];
  q_load(W, ldw, r0, r1, nc, w, col);
  for (int i = tid; i < H1; i += 256) lh[i] = 0u;
  const int istar = s.ctrl->istar;
  q_cols(U, ldu, nc, s, rk, d2s);
  __syncthreads();
#pragma unroll
  for (int k = 0; k < QE; ++k) {
    const int c = col[k];
    if (c < 0 || rk[c] < istar) continue;  // M3 zeros are counted below
    const float v = fabsf(target_of(w[k], d2s[c], metric));
    atomicAdd(&lh[__float_as_uint(v) >> SH1], 1u);
  }
  __syncthreads();
  for (int i = tid; i < H1; i += 256)
    if (lh[i]) atomicAdd(&s.hist1[i], lh[i]);
  if (blockIdx.x == 0 && tid == 0) {
    int nsal = 0;
    for (int c = 0; c < nc; ++c) nsal += rk[c] < istar;
    if (nsal) atomicAdd(&s.hist1[0], (uint32_t)R * (uint32_t)nsal);
  }
}

// Inclusive scan of a 32-bit value over the 64 lanes: row_shr 1, 2, 4, 8
// inside rows of 16 (zero fill), then row_bcast15 / row_bcast31 carry the
// row totals.
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp_u32_rows(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWS, 0xF, true);
}
__device__ __forceinline__ uint32_t wave_scan_u32(uint32_t v) {
  v += dpp_u32_rows<0x111, 0xF>(v);          // row_shr:1
  v += dpp_u32_rows<0x112, 0xF>(v);          // row_shr:2
  v += dpp_u32_rows<0x114, 0xF>(v);          // row_shr:4
  v += dpp_u32_rows<0x118, 0xF>(v);          // row_shr:8
  v += dpp_u32_rows<0x142, 0xA>(v);          // row_bcast:15 into rows 1, 3
  v += dpp_u32_rows<0x143, 0xC>(v);          // row_bcast:31 into rows 2, 3
  return v;
}

// Block-wide exclusive scan of H (multiple of 256) counters in LDS: each of
// the first 256 threads sums H / 256 consecutive counters, the 4 wavefronts
// scan their sums with DPP, and one barrier shares the wavefront totals.
// Every thread of the workgroup (256 or more) must call it, for the
// barriers.
template <int H>
__device__ void block_scan(const uint32_t* src, uint32_t* cum, uint32_t* tmp /* 256 */) {
  constexpr int PER = H / 256;
  const int tid = threadIdx.x, wv = tid >> 6;
  const bool act = tid < 256;
  uint32_t loc[PER];
  uint32_t sum = 0;
#pragma unroll
  for (int k = 0; k < PER; ++k) loc[k] = act ? src[tid * PER + k] : 0u;
#pragma unroll
  for (int k = 0; k < PER; ++k) sum += loc[k];
  const uint32_t inc = wave_scan_u32(sum);
  if (act && (tid & 63) == 63) tmp[wv] = inc;
  __syncthreads();
  if (act) {
    uint32_t run = inc - sum;
    for (int w = 0; w < wv; ++w) run += tmp[w];
#pragma unroll
    for (int k = 0; k < PER; ++k) { cum[tid * PER + k] = run; run += loc[k]; }
  }
  __syncthreads();
}

// Find b with cum[b] <= r < cum[b+1] (cum exclusive, H entries, total n).
template <int H>
__device__ __forceinline__ int find_bin(const uint32_t* cum, uint32_t r) {
  int lo = 0, hi = H - 1;
  while (lo < hi) {                 // last b with cum[b] <= r
    const int mid = (lo + hi + 1) >> 1;
    if (cum[mid] <= r) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// Elements of the target bins into their bin's list.  Every workgroup
// first places the NT order statistics in the level-1 histogram itself (the
// 4096 counters come from L2; repeating this small scan per workgroup costs
// less than a launch of its own): an exclusive scan of the counters, numpy
// 'linear' ranks, each target's bin by binary search, a leader per bin (its
// first target) and the lists' offsets (exclusive scan of the leaders' bin
// counts; bin 0's count also holds the salient columns' zeros, which are
// not stored).  Workgroup 0 publishes the targets for the selection.  Then
// each workgroup counts its elements per list in LDS, reserves room with
// one global atomic per list, and writes the elements' bit patterns (the
// order inside a list does not matter to the selection).  The list counters
// are cleared by k_colscore.
__global__ __launch_bounds__(256) void k_qlist(
    SegSearch seg, int64_t ldw, int R, int nc, int64_t ldu,
    int metric) {
  const float* __restrict__ W = seg.W[blockIdx.y];
  const float* __restrict__ U = seg.U[blockIdx.y];
  const SearchWs s = seg.s[blockIdx.y];
  __shared__ uint32_t cum[H1];
  __shared__ int lead[H1];
  __shared__ uint32_t tmp[256];
  __shared__ float d2s[NCMAX];
  __shared__ int rk[NCMAX];
  __shared__ int cnt[NT];
  __shared__ int base[NT];
  __shared__ int loff[NT];
  __shared__ int bins[NT];
  const int tid = threadIdx.x;
  const int r0 = blockIdx.x * Q_RPW, r1 = min(R, r0 + Q_RPW);
  const int64_t n = (int64_t)R * nc;
  float w[QE];
  int col[QE];
  q_load(W, ldw, r0, r1, nc, w, col);
  const int istar = s.ctrl->istar;
  q_cols(U, ldu, nc, s, rk, d2s);
  for (int i = tid; i < H1; i += 256) lead[i] = NONE;
  if (tid < NT) cnt[tid] = 0;
  block_scan<H1>(s.hist1, cum, tmp);
  if (tid < NT) {
    // numpy 'linear': virtual index (n-1)*q in float32, floor, fractional gamma
    const int q = tid >> 1;
    const float vi = (float)(n - 1) * c_q[q];
    int64_t lo, hi;
    float g;
    if (vi >= (float)(n - 1)) { lo = hi = n - 1; g = 0.f; }
    else {
      const float fl = floorf(vi);
      lo = (int64_t)fl; hi = lo + 1; g = vi - fl;
    }
    const int64_t rnk = (tid & 1) ? hi : lo;
    const int b = find_bin<H1>(cum, (uint32_t)rnk);
    bins[tid] = b;
    atomicMin(&lead[b], tid);
    if (blockIdx.x == 0) {
      Tgt& t = s.tgt[tid];
      t.rank = rnk;
      t.bin1 = b;
      t.r1 = (int)((uint32_t)rnk - cum[b]);
      if (!(tid & 1)) s.gam[q] = g;
    }
  }
  __syncthreads();
  {
    uint32_t c = 0;
    if (tid < NT) {
      const int b = bins[tid];
      if (lead[b] == tid) c = (b + 1 < H1 ? cum[b + 1] : (uint32_t)n) - cum[b];
    }
    const uint32_t inc = wave_scan_u32(c);
    if ((tid & 63) == 63) tmp[tid >> 6] = inc;
    __syncthreads();
    uint32_t off = inc - c;
    for (int v = 0; v < (tid >> 6); ++v) off += tmp[v];
    if (tid < NT) {
      loff[tid] = (int)off;
      if (blockIdx.x == 0) {
        s.list_off[tid] = (int)off;
        s.tgt[tid].slot1 = lead[bins[tid]];
      }
    }
  }
  int slot[QE], pos[QE];
  uint32_t key[QE];
#pragma unroll
  for (int k = 0; k < QE; ++k) {
    const int c = col[k];
    slot[k] = -1;
    pos[k] = 0;
    key[k] = 0u;
    if (c < 0 || rk[c] < istar) continue;  // salient columns: implicit zeros
    const float v = fabsf(target_of(w[k], d2s[c], metric));
    key[k] = __float_as_uint(v);
    const int sl = lead[key[k] >> SH1];
    if (sl != NONE) {
      slot[k] = sl;
      pos[k] = atomicAdd(&cnt[sl], 1);
    }
  }
  __syncthreads();
  if (tid < NT && cnt[tid] > 0) base[tid] = loff[tid] + atomicAdd(&s.list_cnt[tid], cnt[tid]);
  __syncthreads();
#pragma unroll
  for (int k = 0; k < QE; ++k)
    if (slot[k] >= 0) s.lists[base[slot[k]] + pos[k]] = key[k];
}

// One workgroup per target: the r1-th smallest bit pattern of its level-1
// bin, from the bin's list, by two histogram rounds (bits [19:10], then
// bits [9:0] among the elements with the chosen [19:10]).  In bin 0 the
// salient columns' R * nsal zeros come first.
constexpr int QS_T = 1024;           // threads per target
constexpr int QS_UNROLL = 8;
constexpr int QS_LDS = 32768;        // lists up to this long are staged in LDS (128 KB)
template <bool ROUND_B>
__device__ void qselect_hist(const uint32_t* list, int n, int b2, uint32_t* h) {
  for (int i0 = threadIdx.x; i0 < n; i0 += QS_T * QS_UNROLL) {
    uint32_t k[QS_UNROLL];
#pragma unroll
    for (int u = 0; u < QS_UNROLL; ++u) {
      const int i = i0 + QS_T * u;
      k[u] = i < n ? list[i] : 0xffffffffu;
    }
#pragma unroll
    for (int u = 0; u < QS_UNROLL; ++u) {
      if (i0 + QS_T * u >= n) continue;
      const uint32_t mid = (k[u] >> SH2) & (H2 - 1);
      if (!ROUND_B) atomicAdd(&h[mid], 1u);
      else if ((int)mid == b2) atomicAdd(&h[k[u] & (H3 - 1)], 1u);
    }
  }
}

__global__ __launch_bounds__(QS_T) void k_qselect(SegSearch seg, int R, int nc) {
  const SearchWs s = seg.s[blockIdx.y];
  static_assert(H2 == H3, "one histogram buffer for both rounds");
  __shared__ uint32_t h[H2];
  __shared__ uint32_t cum[H2];
  __shared__ uint32_t tmp[256];
  __shared__ int nsal;
  const int t = blockIdx.x, tid = threadIdx.x;
  const Tgt g = s.tgt[t];
  if (tid == 0) nsal = 0;
  __syncthreads();
  if (g.bin1 == 0 && tid < nc && s.rank[tid] < s.ctrl->istar) atomicAdd(&nsal, 1);
  __syncthreads();
  uint32_t r = (uint32_t)g.r1;
  if (g.bin1 == 0) {
    const uint32_t nz = (uint32_t)R * (uint32_t)nsal;
    if (r < nz) {                            // one of the salient columns' zeros
      if (tid == 0) s.tval[t] = 0.f;
      return;
    }
    r -= nz;
  }
  const uint32_t* glist = s.lists + s.list_off[g.slot1];
  const int n = s.list_cnt[g.slot1];
  __shared__ uint32_t stage[QS_LDS];
  const uint32_t* list = glist;
  if (n <= QS_LDS) {                         // one read of the list from memory
    for (int i0 = tid; i0 < n; i0 += QS_T * QS_UNROLL) {
      uint32_t k[QS_UNROLL];
#pragma unroll
      for (int u = 0; u < QS_UNROLL; ++u) k[u] = i0 + QS_T * u < n ? glist[i0 + QS_T * u] : 0u;
#pragma unroll
      for (int u = 0; u < QS_UNROLL; ++u)
        if (i0 + QS_T * u < n) stage[i0 + QS_T * u] = k[u];
    }
    list = stage;
  }
  for (int i = tid; i < H2; i += QS_T) h[i] = 0u;
  __syncthreads();
  qselect_hist<false>(list, n, 0, h);
  __syncthreads();
  block_scan<H2>(h, cum, tmp);
  __shared__ int b2s, r2s;
  if (tid == 0) {
    const int b = find_bin<H2>(cum, r);
    b2s = b;
    r2s = (int)(r - cum[b]);
  }
  for (int i = tid; i < H3; i += QS_T) h[i] = 0u;
  __syncthreads();
  const int b2 = b2s;
  qselect_hist<true>(list, n, b2, h);
  __syncthreads();
  block_scan<H3>(h, cum, tmp);
  if (tid == 0) {
    const int b3 = find_bin<H3>(cum, (uint32_t)r2s);
    const uint32_t key = ((uint32_t)g.bin1 << SH1) | ((uint32_t)b2 << SH2) | (uint32_t)b3;
    s.tval[t] = __uint_as_float(key);
  }
}

// numpy _lerp in float32 (numpy/lib/_function_base_impl.py)
__device__ __forceinline__ float np_lerp(float a, float b, float t) {
  const float diff = b - a;
  float r = diff * t;
  r = a + r;
  if (t >= 0.5f) {
    const float omt = 1.f - t;
    float q = diff * omt;
    r = b - q;
  }
  return r;
}

// ---------------------------------------------------------------------------
// phase C: order-1 errors of the two bell groups for each of the 81 split
// candidates (utils/autosearch.py:71-80), in closed form.
//
// One wavefront per row: the row's non-salient targets are bitonic-sorted
// (2 per lane) and fp64 prefix sums of v and v^2 are formed.  A group
// {|v| < p} or {|v| >= p} is then one or two ranges of the sorted row, and
// order-1 residual binarization of a group is
//   mu = sum v / n,  alpha = sum |v - mu| / n,
//   q(v) = mu + alpha*sign(v - mu),  err = sum (v - q(v))^2,
// where the ranges v < mu, v == mu, v > mu come from binary searches with
// the same fp32 comparisons the elementwise code makes, and every sum is a
// difference of prefix sums: sum (v - t)^2 = Q - 2 t S + n t^2.
// ---------------------------------------------------------------------------
#ifndef CRBQ_PC_WAVES
#define CRBQ_PC_WAVES 16
#endif
constexpr int PC_WAVES = CRBQ_PC_WAVES;

struct SortedRow {
  float v[NCMAX];        // ascending; first n valid
  double S[NCMAX + 1];   // exclusive prefix sums of v
  double Q[NCMAX + 1];   // exclusive prefix sums of v^2
  int n;
};

struct Stat { double n, s, q; };
__device__ __forceinline__ Stat rstat(const SortedRow& r, int l, int h) {
  if (h <= l) return Stat{0.0, 0.0, 0.0};
  return Stat{(double)(h - l), r.S[h] - r.S[l], r.Q[h] - r.Q[l]};
}
__device__ __forceinline__ double sqdev(const Stat& a, double t) {   // sum (v - t)^2
  return a.q - 2.0 * t * a.s + a.n * t * t;
}

// Number of v[0, n) below x (STRICT: the lower bound) or not above x (the
// upper bound) in a sorted row, n <= 128: 8 fixed halving steps instead of
// a data-dependent loop, since the lanes of a wavefront search different
// rows and thresholds; independent searches interleave their LDS reads.
template <bool STRICT>
__device__ __forceinline__ int bcount(const float* v, int n, float x) {
  int pos = 0;
#pragma unroll
  for (int step = NCMAX; step >= 1; step >>= 1) {
    const float y = v[min(pos + step - 1, NCMAX - 1)];
    const bool take = pos + step <= n && (STRICT ? y < x : y <= x);
    pos += take ? step : 0;
  }
  return pos;
}

// sum over the group made of sorted ranges [l1,h1) and [l2,h2) and its size
__device__ __forceinline__ double group_sum2(const SortedRow& r, int l1, int h1, int l2, int h2,
                                             int& n) {
  n = max(h1 - l1, 0) + max(h2 - l2, 0);
  return rstat(r, l1, h1).s + rstat(r, l2, h2).s;
}

// order-1 error of that group (binary.py:18-39 with order 1) given its mean
// mu and the row's lower / upper bounds lb / ub of mu
__device__ double group_err1(const SortedRow& r, int l1, int h1, int l2, int h2, int n,
                             float mu, int lb, int ub) {
  if (n == 0) return 0.0;
  const float nf = (float)n;
  double sabs = 0.0, err = 0.0;
  Stat parts[2][3];
  const int L[2] = {l1, l2}, Hh[2] = {h1, h2};
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const int l = L[g], h = Hh[g];
    const int b1 = min(max(lb, l), max(h, l)), b2 = min(max(ub, l), max(h, l));
    parts[g][0] = rstat(r, l, b1);      // v < mu
    parts[g][1] = rstat(r, b1, b2);     // v == mu
    parts[g][2] = rstat(r, b2, h);      // v > mu
    sabs += (parts[g][2].s - parts[g][2].n * (double)mu) + (parts[g][0].n * (double)mu - parts[g][0].s);
  }
  const float alpha = (float)sabs / nf;
  const float hi = alpha + mu, lo = -alpha + mu;
#pragma unroll
  for (int g = 0; g < 2; ++g)
    err += sqdev(parts[g][0], (double)lo) + sqdev(parts[g][1], (double)mu) +
           sqdev(parts[g][2], (double)hi);
  return err;
}

// Error of split candidate thr on a sorted row of n non-salient targets
// (utils/autosearch.py:72-80): M1 = {-thr < v < thr} = [a, b),
// M2 = [0, a) + [b, n), each binarized at order 1 (utils/mask.py:7-18).
__device__ double split_err(const SortedRow& r, int n, float thr) {
  const int a = bcount<false>(r.v, n, -thr);
  const int b = max(bcount<true>(r.v, n, thr), a);
  int n1, n2;
  const double s1 = group_sum2(r, a, b, 0, 0, n1), s2 = group_sum2(r, 0, a, b, n, n2);
  const float mu1 = n1 ? (float)s1 / (float)n1 : 0.f, mu2 = n2 ? (float)s2 / (float)n2 : 0.f;
  const int lb1 = bcount<true>(r.v, n, mu1), ub1 = bcount<false>(r.v, n, mu1);
  const int lb2 = bcount<true>(r.v, n, mu2), ub2 = bcount<false>(r.v, n, mu2);
  return group_err1(r, a, b, 0, 0, n1, mu1, lb1, ub1) + group_err1(r, 0, a, b, n, n2, mu2, lb2, ub2);
}

// Partner value of a xor-j exchange inside the wavefront, without the LDS
// crossbar.  For j = 16, 32 the permlane swap returns {own, partner} in some
// order, which is all a compare-exchange needs (min and max of the pair).
template <int J>
__device__ __forceinline__ void xchg_pair(float x, float& a, float& b) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  const int lane = threadIdx.x & 63;
  if (J == 1) {
    a = x; b = __builtin_bit_cast(float, dpp_u32<DPP_XOR1>(u));
  } else if (J == 2) {
    a = x; b = __builtin_bit_cast(float, dpp_u32<DPP_XOR2>(u));
  } else if (J == 4 || J == 8) {
    // row_shl:J brings lane + J, row_shr:J lane - J (rows of 16 lanes)
    const float up = __builtin_bit_cast(float, dpp_u32<0x100 + J>(u));
    const float dn = __builtin_bit_cast(float, dpp_u32<0x110 + J>(u));
    a = x; b = (lane & J) ? dn : up;
  } else {
    unsigned p = u, q = u;
    if (J == 16) permlane16_swap(p, q);
    else permlane32_swap(p, q);
    a = __builtin_bit_cast(float, p); b = __builtin_bit_cast(float, q);
  }
}

template <int J>
__device__ __forceinline__ void bitonic_step(float& x0, float& x1, int k) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int slot = 0; slot < 2; ++slot) {
    float& x = slot ? x1 : x0;
    const int pos = lane + 64 * slot;
    float a, b;
    xchg_pair<J>(x, a, b);
    const bool up = ((pos & k) == 0);
    const bool lower = (pos & J) == 0;
    x = (lower == up) ? fminf(a, b) : fmaxf(a, b);
  }
}

// bitonic sort of 128 values held 2 per lane (position lane + 64*slot)
__device__ __forceinline__ void wave_sort128(float& x0, float& x1) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int k = 2; k <= 128; k <<= 1) {
    if (k >= 128) {                          // partner is the other slot of this lane
      const float a = fminf(x0, x1), b = fmaxf(x0, x1);
      x0 = a;
      x1 = b;
    }
    if (k >= 64) bitonic_step<32>(x0, x1, k);
    if (k >= 32) bitonic_step<16>(x0, x1, k);
    if (k >= 16) bitonic_step<8>(x0, x1, k);
    if (k >= 8) bitonic_step<4>(x0, x1, k);
    if (k >= 4) bitonic_step<2>(x0, x1, k);
    bitonic_step<1>(x0, x1, k);
  }
  (void)lane;
}

// inclusive fp64 scan over the 64 lanes: row_shr 1, 2, 4, 8 inside rows of
// 16 (zero fill), then row_bcast15 / row_bcast31 carry the row totals
template <int CTRL, int ROWS>
__device__ __forceinline__ double dpp_f64_rows(double v) {
  const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
  const unsigned lo = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)b, CTRL, ROWS, 0xF,
                                                            true);
  const unsigned hi = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)(b >> 32), CTRL,
                                                            ROWS, 0xF, true);
  return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}
__device__ __forceinline__ double wave_scan_f64(double v) {
  v = v + dpp_f64_rows<0x111, 0xF>(v);       // row_shr:1
  v = v + dpp_f64_rows<0x112, 0xF>(v);       // row_shr:2
  v = v + dpp_f64_rows<0x114, 0xF>(v);       // row_shr:4
  v = v + dpp_f64_rows<0x118, 0xF>(v);       // row_shr:8
  v = v + dpp_f64_rows<0x142, 0xA>(v);       // row_bcast:15 into rows 1, 3
  v = v + dpp_f64_rows<0x143, 0xC>(v);       // row_bcast:31 into rows 2, 3
  return v;
}
__device__ __forceinline__ double lane63_f64(double v) {
  const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
  const unsigned lo = __builtin_amdgcn_readlane((unsigned)b, 63);
  const unsigned hi = __builtin_amdgcn_readlane((unsigned)(b >> 32), 63);
  return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}

// exclusive fp64 prefix sums of the sorted row into r.S / r.Q
__device__ __forceinline__ void wave_prefix(SortedRow& r, float x0, float x1, int n) {
  const int lane = threadIdx.x & 63;
  double s0 = lane < n ? (double)x0 : 0.0, s1 = lane + 64 < n ? (double)x1 : 0.0;
  double q0 = s0 * s0, q1 = s1 * s1;
  s0 = wave_scan_f64(s0);
  s1 = wave_scan_f64(s1);
  q0 = wave_scan_f64(q0);
  q1 = wave_scan_f64(q1);
  const double tS = lane63_f64(s0), tQ = lane63_f64(q0);
  s1 += tS;
  q1 += tQ;
  r.S[lane + 1] = s0;
  r.S[lane + 65] = s1;
  r.Q[lane + 1] = q0;
  r.Q[lane + 65] = q1;
  if (lane == 0) { r.S[0] = 0.0; r.Q[0] = 0.0; }
  r.v[lane] = x0;
  r.v[lane + 64] = x1;
}

// Phase C: per row (one wavefront) the non-salient targets sorted with
// fp64 prefix sums of v and v^2; then the workgroup's (row, candidate k)
// pairs over all its lanes, each two binary searches per group and range
// sums (group_err1); the last workgroup takes k* = first strict minimum.
__global__ __launch_bounds__(64 * PC_WAVES) void k_phase_c(
    SegSearch seg, int64_t ldw, int R, int nc, int64_t ldu,
    int metric) {
  const float* __restrict__ W = seg.W[blockIdx.y];
  const float* __restrict__ U = seg.U[blockIdx.y];
  const SearchWs s = seg.s[blockIdx.y];
  crbq_block_trace* const tr = seg.tr[blockIdx.y];
  __shared__ SortedRow rows[PC_WAVES];
  __shared__ double red[10][96];
  __shared__ double e[128];
  __shared__ float pv[NQ];
  __shared__ double errs[PC_WAVES][NQ];
  __shared__ double acc[NQ];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int istar = s.ctrl->istar;
  for (int k = tid; k < NQ; k += 64 * PC_WAVES) {
    pv[k] = np_lerp(s.tval[2 * k], s.tval[2 * k + 1], s.gam[k]);
    if (blockIdx.x == 0) s.pvals[k] = pv[k];
    acc[k] = 0.0;
  }
  const int c0 = lane, c1 = lane + 64;
  const bool in0 = c0 < nc && s.rank[c0] >= istar, in1 = c1 < nc && s.rank[c1] >= istar;
  float d20 = 1.f, d21 = 1.f;
  if (c0 < nc) { const float dg = U[(int64_t)c0 * ldu + c0]; d20 = dg * dg; }
  if (c1 < nc) { const float dg = U[(int64_t)c1 * ldu + c1]; d21 = dg * dg; }
  const int n = (int)wave_sum_f((in0 ? 1.f : 0.f) + (in1 ? 1.f : 0.f));
  SortedRow& sr = rows[wv];
  for (int r0 = blockIdx.x * PC_WAVES; r0 < R; r0 += gridDim.x * PC_WAVES) {
    const int row = r0 + wv;
    __syncthreads();                       // previous rows' errs consumed
    if (row < R) {
      float x0 = in0 ? target_of(W[(int64_t)row * ldw + c0], d20, metric) : INFINITY;
      float x1 = in1 ? target_of(W[(int64_t)row * ldw + c1], d21, metric) : INFINITY;
      wave_sort128(x0, x1);
      wave_prefix(sr, x0, x1, n);
      if (lane == 0) sr.n = n;
    }
    __syncthreads();
    // the workgroup's (row, candidate) pairs spread over all its lanes
    for (int pq = tid; pq < PC_WAVES * NQ; pq += 64 * PC_WAVES) {
      const int q = pq / NQ, k = pq - q * NQ;
      if (r0 + q < R) {
        errs[q][k] = split_err(rows[q], n, pv[k]);
      }
    }
    __syncthreads();
    const int nr = min(PC_WAVES, R - r0);
    for (int k = tid; k < NQ; k += 64 * PC_WAVES) {
      double v = acc[k];
      for (int w = 0; w < nr; ++w) v += errs[w][k];
      acc[k] = v;
    }
  }
  __syncthreads();
  for (int k = tid; k < NQ; k += 64 * PC_WAVES) pstore(&s.partc[(size_t)blockIdx.x * 96 + k], acc[k]);
  if (!last_block(&s.ctrl->cnt[CNT_C])) return;
  reduce_partials<96, 10, (PX_MAXWG + 9) / 10>(s.partc, 96, gridDim.x, NQ, red, e);
  if (tid < 64) {
    const int am = wave_argmin(e, NQ);
    const int ks = am < 0 ? NQ / 2 : am;                             // :71 median
    if (tid == 0) {
      s.ctrl->kstar = ks;
      s.ctrl->split = pv[ks];
      if (tr) { tr->k_star = ks; tr->split = pv[ks]; }
    }
  }
  if (tr && tid < NQ) { tr->errs_c[tid] = e[tid]; tr->pvals[tid] = pv[tid]; }
}

// ---------------------------------------------------------------------------
// quantize one block: masks -> binarize per group -> Q, Err, Loss
// (bigptq.py:235-264, utils/mask.py:7-18)
// ---------------------------------------------------------------------------
struct QuantArgs {
  float* W; int64_t ldw; int R; int nc;
  const float* U; int64_t ldu;      // U[st, st]
  int metric; int method; int partition; int orders[3];
  CrbConsts k;
  int gptq;                          // 0: RTN (no Err/Loss)
  float* err; int64_t lde;           // R x nc
  float* losses;
  uint8_t* masks; int64_t ldm;       // optional
};
struct QuantSegs {                   // one per sublayer of the launch (blockIdx.y)
  QuantArgs a[NSEG];
  SearchWs s[NSEG];
};

template <int MF, int EPL>
__global__ __launch_bounds__(256) void k_quantize(QuantSegs qs) {
  const QuantArgs& a = qs.a[blockIdx.y];
  const SearchWs& s = qs.s[blockIdx.y];
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.R) return;
  const int istar = a.partition == 3 ? s.ctrl->istar : 0;
  const float split = a.partition == 3 ? s.ctrl->split : 0.f;
  float x[EPL], dd[EPL];
  int grp[EPL];
  bool valid[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    const int c = lane + 64 * e;
    valid[e] = c < a.nc;
    x[e] = valid[e] ? a.W[(int64_t)row * a.ldw + c] : 0.f;
    dd[e] = valid[e] ? a.U[(int64_t)c * a.ldu + c] : 1.f;
    int g = -1;
    if (valid[e]) {
      if (a.partition != 3) g = 0;
      else if (s.rank[c] < istar) g = 2;
      else {
        const float t = fabsf(target_of(x[e], dd[e] * dd[e], a.metric));
        g = t >= split ? 1 : 0;
      }
    }
    grp[e] = g;
  }
  float q[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) q[e] = 0.f;
  const int ngroups = a.partition == 3 ? 3 : 1;
  for (int g = 0; g < ngroups; ++g) {
    bool m[EPL];
    bool any = false;
#pragma unroll
    for (int e = 0; e < EPL; ++e) { m[e] = grp[e] == g; any |= m[e]; }
    (void)any;
    float out[EPL];
    binarize_row<MF, EPL>(a.method, x, m, a.orders[g], a.k, out);
#pragma unroll
    for (int e = 0; e < EPL; ++e) if (m[e]) q[e] = out[e];
  }
  double lsum = 0.0;
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    if (!valid[e]) continue;
    const int c = lane + 64 * e;
    const float w = x[e], d = dd[e];
    const float df = w - q[e];
    if (a.gptq) {
      const float d2 = d * d;
      const float l = (df * df) / d2;
      lsum += (double)l;
      a.err[(int64_t)row * a.lde + c] = df / d;
    }
    a.W[(int64_t)row * a.ldw + c] = q[e];
    if (a.masks) a.masks[(int64_t)row * a.ldm + c] = (uint8_t)(grp[e] + 1);
  }
  if (a.gptq) {
    const float tot = (float)wave_sum(lsum);
    if (lane == 0) a.losses[row] = a.losses[row] + tot / 2.f;
  }
}

// VW consecutive floats through one 16-, 8- or 4-byte access
template <int VW>
__device__ __forceinline__ void vload(const float* p, float* v) {
  if constexpr (VW == 4) { const float4 q = *(const float4*)p; v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w; }
  else if constexpr (VW == 2) { const float2 q = *(const float2*)p; v[0] = q.x; v[1] = q.y; }
  else v[0] = *p;
}
template <int VW>
__device__ __forceinline__ void vstore(float* p, const float* v) {
  if constexpr (VW == 4) *(float4*)p = make_float4(v[0], v[1], v[2], v[3]);
  else if constexpr (VW == 2) *(float2*)p = make_float2(v[0], v[1]);
  else *p = v[0];
}
// k_quantize for blocks of at most 128 columns with QG_LPR lanes per row
// (256 / QG_LPR rows per workgroup) and 128 / QG_LPR elements per lane, in
// runs of VW = min(4, 128 / QG_LPR) consecutive columns: lane r holds columns
// h*VW*QG_LPR + r*VW + j.  Loads and stores move VW floats at a time (W, err
// and their row strides 16-byte aligned, masks 4-byte aligned; the host
// checks).  32 lanes per row (8 rows per workgroup) keeps two wavefronts per
// SIMD on a 4096-row block, which hides more of the reductions' latency than
// 16 lanes (one wavefront per SIMD) or 8.
#ifndef CRBQ_QG_LPR
#define CRBQ_QG_LPR 32
#endif
constexpr int QG_LPR = CRBQ_QG_LPR;          // lanes per row of the block quantize
template <int MF>
__global__ __launch_bounds__(256) void k_quantize_g(QuantSegs qs) {
  const QuantArgs& a = qs.a[blockIdx.y];
  const SearchWs& s = qs.s[blockIdx.y];
  constexpr int LPR = QG_LPR, EPL = 128 / LPR, VW = EPL < 4 ? EPL : 4, NH = EPL / VW;
  const int r = threadIdx.x % LPR;
  const int row = blockIdx.x * (256 / LPR) + threadIdx.x / LPR;
  if (row >= a.R) return;                    // whole lane groups leave together
  const int istar = a.partition == 3 ? s.ctrl->istar : 0;
  const float split = a.partition == 3 ? s.ctrl->split : 0.f;
  float x[EPL], dd[EPL];
  int grp[EPL];
  bool valid[EPL];
  float* wr = a.W + (int64_t)row * a.ldw;
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    const int c0 = h * VW * LPR + r * VW;
    if (c0 + VW - 1 < a.nc) {
      vload<VW>(wr + c0, x + VW * h);
    } else {
#pragma unroll
      for (int j = 0; j < VW; ++j) x[VW * h + j] = c0 + j < a.nc ? wr[c0 + j] : 0.f;
    }
  }
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    const int c = (e / VW) * VW * LPR + r * VW + e % VW;
    valid[e] = c < a.nc;
    dd[e] = valid[e] ? a.U[(int64_t)c * a.ldu + c] : 1.f;
    int g = -1;
    if (valid[e]) {
      if (a.partition != 3) g = 0;
      else if (s.rank[c] < istar) g = 2;
      else {
        const float t = fabsf(target_of(x[e], dd[e] * dd[e], a.metric));
        g = t >= split ? 1 : 0;
      }
    }
    grp[e] = g;
  }
  float q[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) q[e] = 0.f;
  const int ngroups = a.partition == 3 ? 3 : 1;
  for (int g = 0; g < ngroups; ++g) {
    bool m[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) m[e] = grp[e] == g;
    float out[EPL];
    binarize_row<MF, EPL, LPR>(a.method, x, m, a.orders[g], a.k, out);
#pragma unroll
    for (int e = 0; e < EPL; ++e) if (m[e]) q[e] = out[e];
  }
  double lsum = 0.0;
  float ev[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    ev[e] = 0.f;
    if (!valid[e]) continue;
    const float w = x[e], d = dd[e];
    const float df = w - q[e];
    if (a.gptq) {
      const float d2 = d * d;
      const float l = (df * df) / d2;
      lsum += (double)l;
      ev[e] = df / d;
    }
  }
  float* er = a.err + (int64_t)row * a.lde;
  uint8_t* mr = a.masks ? a.masks + (int64_t)row * a.ldm : nullptr;
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    const int c0 = h * VW * LPR + r * VW;
    if (c0 + VW - 1 < a.nc) {
      vstore<VW>(wr + c0, q + VW * h);
      if (a.gptq) vstore<VW>(er + c0, ev + VW * h);
      if (mr) {
        unsigned mb = 0;
#pragma unroll
        for (int j = 0; j < VW; ++j) mb |= (unsigned)(grp[VW * h + j] + 1) << (8 * j);
        if (VW == 4) *(unsigned*)(mr + c0) = mb;
        else if (VW == 2) *(uint16_t*)(mr + c0) = (uint16_t)mb;
        else mr[c0] = (uint8_t)mb;
      }
    } else {
#pragma unroll
      for (int j = 0; j < VW; ++j) {
        if (c0 + j >= a.nc) continue;
        wr[c0 + j] = q[VW * h + j];
        if (a.gptq) er[c0 + j] = ev[VW * h + j];
        if (mr) mr[c0 + j] = (uint8_t)(grp[VW * h + j] + 1);
      }
    }
  }
  if (a.gptq) {
    const float tot = (float)group_sum<LPR>(lsum);
    if (r == 0) a.losses[row] = a.losses[row] + tot / 2.f;
  }
}

// clears the arrival counters of the last-workgroup reductions
// Arrival counters of every segment's search scratch cleared (thread
// 4 i + j: counter j of segment i).
struct SegCtrl {
  Ctrl* c[NSEG];
};
__global__ void k_init_ctrl(SegCtrl g, int nseg) {
  const int t = threadIdx.x;
  if (t < 4 * nseg) g.c[t >> 2]->cnt[t & 3] = 0u;
}

// ---------------------------------------------------------------------------
// Salient-count candidates with the rows on the lanes: lane = row of a
// 64-row group, wavefront = candidate i.  A candidate's salient group (ranks
// [0, i)) and complement (ranks [i, nc)) are then wavefront-uniform ranges,
// so each of the three passes (group sums, |x - m1| with sign counts,
// residual moments) is two select-free loops, and no lane idles.  The group
// sums run in fp64 (exact for these fp32 values unless their exponents span
// more than 29 binades); the other passes sum in fp32 over chunks of 8
// elements, accumulated in fp64, with integer counts.  A workgroup holds one
// row group in LDS and evaluates cw candidates; ncg = ceil(ncand / cw)
// workgroups share a row group, each writing its candidates' partial sums.
// ---------------------------------------------------------------------------
#ifndef CRBQ_PR_CW
#define CRBQ_PR_CW 16
#endif
constexpr int PR_CW = CRBQ_PR_CW;   // most candidates (wavefronts) per workgroup
constexpr int PR_MINW = 9;          // reduce_partials<UPMAX, 9> needs 576 threads
constexpr int PR_XS = NCMAX + 4;    // row stride: 33 16-byte units

struct RowAbs { double ad; int npos, nneg; };
struct RowRes { double e1, e2; int nz; };

__device__ __forceinline__ void row_abs(const float* x, int c0, int c1, float m1, RowAbs& a) {
  int c = c0;
  for (; c + 8 <= c1; c += 8) {
    float p = 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float d = x[c + u] - m1;
      p += fabsf(d);
      a.npos += d > 0.f ? 1 : 0;
      a.nneg += d < 0.f ? 1 : 0;
    }
    a.ad += (double)p;
  }
  float p = 0.f;
  for (; c < c1; ++c) {
    const float d = x[c] - m1;
    p += fabsf(d);
    a.npos += d > 0.f ? 1 : 0;
    a.nneg += d < 0.f ? 1 : 0;
  }
  a.ad += (double)p;
}

// Residual moments over x[c0, c1) of a group with parameters g.  Each
// element takes s1 = x > m1 ? hi : lo with hi = fl(a1 + m1), lo =
// fl(-a1 + m1): the reference's sign(x - m1) * a1 + m1 (binary.py:26,
// 32-34; the product is exact, so the add rounds as the reference's does)
// except where x == m1, whose sign is 0 and s1 = m1.  Those n0 elements
// (known from the sign counts) all contributed the same e0 = fl(fl(m1 -
// lo) - m2) here, and their sums are moved to the reference's e = -m2
// afterwards, so the loop carries no zero test.  e^2 is accumulated with
// fma.
__device__ __forceinline__ void row_res(const float* x, int c0, int c1, const ParA& g, int n0,
                                        RowRes& r) {
  int c = c0;
  for (; c + 8 <= c1; c += 8) {
    float p1 = 0.f, p2 = 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float v = x[c + u];
      const float s1 = v > g.m1 ? g.hi : g.lo;
      const float e = (v - s1) - g.m2;
      p1 += fabsf(e);
      p2 = __builtin_fmaf(e, e, p2);
      r.nz += e != 0.f ? 1 : 0;
    }
    r.e1 += (double)p1;
    r.e2 += (double)p2;
  }
  float p1 = 0.f, p2 = 0.f;
  for (; c < c1; ++c) {
    const float v = x[c];
    const float s1 = v > g.m1 ? g.hi : g.lo;
    const float e = (v - s1) - g.m2;
    p1 += fabsf(e);
    p2 = __builtin_fmaf(e, e, p2);
    r.nz += e != 0.f ? 1 : 0;
  }
  r.e1 += (double)p1;
  r.e2 += (double)p2;
  if (n0 > 0) {
    const float e0 = (g.m1 - g.lo) - g.m2;
    const double m2 = (double)g.m2, d0 = (double)e0;
    r.e1 += (double)n0 * (fabs(m2) - fabs(d0));
    r.e2 += (double)n0 * (m2 * m2 - d0 * d0);
    r.nz += n0 * ((g.m2 != 0.f ? 1 : 0) - (e0 != 0.f ? 1 : 0));
  }
}

// fp64 sum of x[c0, c1): eight loads in flight per step, each step's
// values summed in a tree first
__device__ __forceinline__ double row_sum(const float* x, int c0, int c1) {
  double a = 0.0;
  int c = c0;
  for (; c + 8 <= c1; c += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = x[c + u];
    a += (((double)v[0] + (double)v[1]) + ((double)v[2] + (double)v[3])) +
         (((double)v[4] + (double)v[5]) + ((double)v[6] + (double)v[7]));
  }
  for (; c < c1; ++c) a += (double)x[c];
  return a;
}

// order-2 residual binarization error of {ranks [0, i)} + {ranks [i, nc)}
// of one row x in rank order (binary.py:17-41 via utils/autosearch.py:44-55)
__device__ __forceinline__ double row_cand_err(const float* x, int i, int nc, double ps,
                                               double pc) {
  const float nS = (float)i, nC = (float)(nc - i);
  const float m1S = (float)ps / nS;
  const float m1C = nC > 0.f ? (float)pc / nC : 0.f;
  RowAbs aS = {0.0, 0, 0}, aC = {0.0, 0, 0};
  row_abs(x, 0, i, m1S, aS);
  row_abs(x, i, nc, m1C, aC);
  const float a1S = (float)aS.ad / nS;
  const float a1C = nC > 0.f ? (float)aC.ad / nC : 0.f;
  // sum r = sum x - sum s1, s1 in {fl(a1 + m1), fl(-a1 + m1), m1}
  const float hiS = a1S + m1S, loS = -a1S + m1S, hiC = a1C + m1C, loC = -a1C + m1C;
  const double s1S = aS.npos * (double)hiS + aS.nneg * (double)loS +
                     ((double)nS - aS.npos - aS.nneg) * (double)m1S;
  const double s1C = aC.npos * (double)hiC + aC.nneg * (double)loC +
                     ((double)nC - aC.npos - aC.nneg) * (double)m1C;
  const float m2S = (float)(ps - s1S) / nS;
  const float m2C = nC > 0.f ? (float)(pc - s1C) / nC : 0.f;
  const ParA PS = {m1S, hiS, loS, m2S, a1S}, PC = {m1C, hiC, loC, m2C, a1C};
  RowRes rS = {0.0, 0.0, 0}, rC = {0.0, 0.0, 0};
  row_res(x, 0, i, PS, i - aS.npos - aS.nneg, rS);
  row_res(x, i, nc, PC, (nc - i) - aC.npos - aC.nneg, rC);
  // sum (e - a2 sign(e))^2 = sum e^2 - 2 a2 sum |e| + a2^2 #(e != 0)
  const double a2S = (double)((float)rS.e1 / nS);
  const double a2C = nC > 0.f ? (double)((float)rC.e1 / nC) : 0.0;
  return (rS.e2 - 2.0 * a2S * rS.e1 + a2S * a2S * (double)rS.nz) +
         (rC.e2 - 2.0 * a2C * rC.e1 + a2C * a2C * (double)rC.nz);
}

__global__ __launch_bounds__(64 * PR_CW) void k_phase_a_rows(
    SegSearch seg, int64_t ldw, int R, int nc, int64_t ldu,
    int metric, int ncand, int up_lim, int ncg, int cw) {
  const float* __restrict__ W = seg.W[blockIdx.y];
  const float* __restrict__ U = seg.U[blockIdx.y];
  const SearchWs s = seg.s[blockIdx.y];
  crbq_block_trace* const tr = seg.tr[blockIdx.y];
  constexpr int LMAX = (64 + PR_MINW - 1) / PR_MINW;   // rows loaded per wavefront
  __shared__ __attribute__((aligned(16))) float xs[64][PR_XS];
  __shared__ double cs[NCMAX / 8][64];           // fp64 sums of 8-rank chunks, per row
  __shared__ double red[PR_MINW][UPMAX];
  __shared__ double e[UPMAX];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, nw = blockDim.x >> 6;
  const int cg = (int)blockIdx.x % ncg, nrg = (int)gridDim.x / ncg;
  const int i = cg * cw + wv + 1;                // this wavefront's candidate
  const bool live = wv < cw && i <= ncand;
  const int c0 = lane, c1 = lane + 64;
  const int rk0 = c0 < nc ? s.rank[c0] : -1, rk1 = c1 < nc ? s.rank[c1] : -1;
  float d20 = 1.f, d21 = 1.f;
  if (c0 < nc) { const float dg = U[(int64_t)c0 * ldu + c0]; d20 = dg * dg; }
  if (c1 < nc) { const float dg = U[(int64_t)c1 * ldu + c1]; d21 = dg * dg; }
  double acc = 0.0;
  for (int rg = (int)blockIdx.x / ncg; rg * 64 < R; rg += nrg) {
    const int r0 = rg * 64;
    __syncthreads();                             // previous rows' readers are done
    float v0[LMAX], v1[LMAX];                    // every load issued before the first store
#pragma unroll
    for (int k = 0; k < LMAX; ++k) {
      const int q = wv + k * nw, rq = r0 + q;
      const bool ok = q < 64 && rq < R;
      v0[k] = ok && rk0 >= 0 ? W[(int64_t)rq * ldw + c0] : 0.f;
      v1[k] = ok && rk1 >= 0 ? W[(int64_t)rq * ldw + c1] : 0.f;
    }
#pragma unroll
    for (int k = 0; k < LMAX; ++k) {
      const int q = wv + k * nw;
      if (q < 64) {
        if (rk0 >= 0) xs[q][rk0] = target_of(v0[k], d20, metric);
        if (rk1 >= 0) xs[q][rk1] = target_of(v1[k], d21, metric);
      }
    }
    __syncthreads();
    // chunk sums once per row group, shared by the candidates' group sums
    for (int j = wv; j < NCMAX / 8; j += nw) cs[j][lane] = row_sum(xs[lane], 8 * j, min(nc, 8 * j + 8));
    __syncthreads();
    if (live) {
      // group sums: whole chunks below i, then the ranks of i's chunk
      double ps = 0.0, tot = 0.0;
      const int ji = i >> 3;
      for (int j = 0; j < NCMAX / 8; ++j) {
        const double v = cs[j][lane];
        if (j < ji) ps += v;
        tot += v;
      }
      ps += row_sum(xs[lane], 8 * ji, i);
      const double err = row_cand_err(xs[lane], i, nc, ps, tot - ps);
      const double t = lane63_f64(wave_scan_f64(r0 + lane < R ? err : 0.0));
      acc += t;
    }
  }
  if (live && lane == 0) pstore(&s.parta[(size_t)((int)blockIdx.x / ncg) * UPMAX + (i - 1)], acc);
  if (!last_block(&s.ctrl->cnt[CNT_A])) return;
  reduce_partials<UPMAX, PR_MINW, (PX_MAXWG + PR_MINW - 1) / PR_MINW>(s.parta, UPMAX, nrg,
                                                                      ncand, red, e);
  if (tid < 64) {
    const int am = wave_argmin(e, ncand);
    const int istar = am < 0 ? max(1, up_lim / 3) : am + 1;         // :43
    if (tid == 0) {
      s.ctrl->istar = istar;
      if (tr) tr->i_star = istar;
    }
  }
  if (tr && tid < UPMAX) tr->errs_a[tid] = (tid >= 1 && tid <= ncand) ? e[tid - 1] : 0.0;
}

// ---------------------------------------------------------------------------
// host drivers
// ---------------------------------------------------------------------------
static int search_block(const SegSearch& seg, int nseg, int64_t ldw, int R, int nc,
                        int64_t ldu, int metric, int up_lim, hipStream_t st) {
  const int ncand = up_lim - 1;
  const int nwg_cs = (int)std::min<int64_t>(cdiv(R, CS_PH), CS_MAXWG);
  const int nwg_q = (int)cdiv(R, Q_RPW);
  const int nwg_c = (int)std::min<int64_t>(cdiv(R, PC_WAVES), PX_MAXWG);
  // phase A: ceil(ncand / PR_CW) workgroups of up to PR_CW candidates per
  // 64-row group (at least PR_MINW wavefronts: the reduction's 576 threads)
  const int ncg = (int)cdiv(ncand, PR_CW), cw = (int)cdiv(ncand, ncg);
  const int nrg = (int)std::min<int64_t>(cdiv(R, 64), PX_MAXWG);
  const unsigned y = (unsigned)nseg;
  k_colscore<<<dim3(nwg_cs, y), CS_THREADS, 0, st>>>(seg, ldw, R, nc, ldu, metric);
  k_phase_a_rows<<<dim3(nrg * ncg, y), 64 * std::max(cw, PR_MINW), 0, st>>>(
      seg, ldw, R, nc, ldu, metric, ncand, up_lim, ncg, cw);
  k_qpass1<<<dim3(nwg_q, y), 256, 0, st>>>(seg, ldw, R, nc, ldu, metric);
  k_qlist<<<dim3(nwg_q, y), 256, 0, st>>>(seg, ldw, R, nc, ldu, metric);
  k_qselect<<<dim3(NT, y), QS_T, 0, st>>>(seg, R, nc);
  k_phase_c<<<dim3(nwg_c, y), 64 * PC_WAVES, 0, st>>>(seg, ldw, R, nc, ldu, metric);
  CRBQ_LAUNCH_CHECK();
  return CRBQ_OK;
}

// c_q lives in every device's copy of the code object, so "uploaded" is
// tracked per device (the current device of the call).  Host threads may
// call concurrently: the flags are atomics and the upload is serialized.
constexpr int MAXDEV = 64;
static std::atomic<bool> q_table_ready[MAXDEV] = {};
static std::mutex g_q_mu;
static int ensure_q_table() {
  int dev = 0;
  CRBQ_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= MAXDEV) return CRBQ_ERR_ARG;
  if (q_table_ready[dev].load(std::memory_order_acquire)) return CRBQ_OK;
  std::lock_guard<std::mutex> g(g_q_mu);
  if (q_table_ready[dev].load(std::memory_order_relaxed)) return CRBQ_OK;
  // torch.linspace(0.10, 0.90, 81) (float32, CPU): start + i*step for the
  // first half, end - (steps-1-i)*step for the second, step in float32.
  float q[NQ];
  const float start = 0.10f, end = 0.90f;
  const float step = (end - start) / (float)(NQ - 1);
  const int half = NQ / 2;
  for (int i = 0; i < NQ; ++i)
    q[i] = i < half ? start + step * (float)i : end - step * (float)(NQ - 1 - i);
  CRBQ_HIP(hipMemcpyToSymbol(HIP_SYMBOL(c_q), q, sizeof(q)));
  q_table_ready[dev].store(true, std::memory_order_release);
  return CRBQ_OK;
}

int set_q_table(const float* q) {
  int dev = 0;
  CRBQ_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= MAXDEV) return CRBQ_ERR_ARG;
  std::lock_guard<std::mutex> g(g_q_mu);
  CRBQ_HIP(hipMemcpyToSymbol(HIP_SYMBOL(c_q), q, NQ * sizeof(float)));
  q_table_ready[dev].store(true, std::memory_order_release);
  return CRBQ_OK;
}

static size_t search_ws_bytes(int64_t R) {
  WsCarver c(nullptr, 0);
  SearchWs s;
  carve_search(c, R, s);
  return c.off + 256;
}

static int check_params(const crbq_params* p) {
  if (!p) return CRBQ_ERR_ARG;
  if (p->blocksize < 1 || p->blocksize > NCMAX) return CRBQ_ERR_ARG;
  if (p->partition != 1 && p->partition != 3) return CRBQ_ERR_ARG;
  if (p->method < CRBQ_BRAQ || p->method > CRBQ_CRB_SYMDAMP_NOREFINE) return CRBQ_ERR_ARG;
  if (p->metric != CRBQ_METRIC_HESSIAN && p->metric != CRBQ_METRIC_MAGNITUDE) return CRBQ_ERR_ARG;
  if (p->partition == 3 && (p->up_lim < 2 || p->up_lim > UPMAX)) return CRBQ_ERR_ARG;
  for (int g = 0; g < 3; ++g) if (p->orders[g] < 1 || p->orders[g] > 8) return CRBQ_ERR_ARG;
  if (p->refine_iters < 0 || p->refine_iters > 64) return CRBQ_ERR_ARG;
  return CRBQ_OK;
}

}  // namespace crbq

using namespace crbq;

extern "C" size_t crbq_block_search_workspace_size(int64_t R, int32_t up_lim) {
  (void)up_lim;
  return search_ws_bytes(R);
}

namespace crbq {
__global__ __launch_bounds__(256) void k_emit_masks(const float* __restrict__ W, int64_t ldw,
                                                    int R, int nc, const float* __restrict__ U,
                                                    int64_t ldu, int metric, uint8_t* masks,
                                                    int64_t ldm, SearchWs s) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)R * nc) return;
  const int r = (int)(i / nc), c = (int)(i % nc);
  uint8_t code;
  if (s.rank[c] < s.ctrl->istar) code = 3;
  else {
    const float dg = U[(int64_t)c * ldu + c];
    const float t = fabsf(target_of(W[(int64_t)r * ldw + c], dg * dg, metric));
    code = t >= s.ctrl->split ? 2 : 1;
  }
  masks[(int64_t)r * ldm + c] = code;
}
}  // namespace crbq

extern "C" int crbq_block_search(const float* W, int64_t R, int32_t ncols, int64_t ldw,
                                 const float* Ublk, int64_t ldu, int32_t metric,
                                 int32_t up_lim, uint8_t* masks, int64_t ldm,
                                 crbq_block_trace* trace, void* ws, size_t ws_bytes,
                                 void* stream) {
  if (!W || !Ublk || R <= 0 || ncols <= 0 || ncols > NCMAX) return CRBQ_ERR_ARG;
  if (up_lim < 2 || up_lim > UPMAX) return CRBQ_ERR_ARG;
  if (ncols < up_lim) return CRBQ_ERR_TOPK;
  if (R * (int64_t)NCMAX >= (1 << 24)) return CRBQ_ERR_ARG;
  if (metric != CRBQ_METRIC_HESSIAN && metric != CRBQ_METRIC_MAGNITUDE) return CRBQ_ERR_ARG;
  if (masks && ldm < ncols) return CRBQ_ERR_ARG;
  WsCarver c(ws, ws_bytes);
  SearchWs s;
  carve_search(c, R, s);
  if (!c.ok()) return CRBQ_ERR_WORKSPACE;
  int st = ensure_q_table();
  if (st) return st;
  hipStream_t hs = (hipStream_t)stream;
  SegCtrl sc{};
  sc.c[0] = s.ctrl;
  k_init_ctrl<<<1, 64, 0, hs>>>(sc, 1);
  SegSearch seg{};
  seg.W[0] = W;
  seg.U[0] = Ublk;
  seg.s[0] = s;
  seg.tr[0] = trace;
  st = search_block(seg, 1, ldw, (int)R, ncols, ldu, metric, up_lim, hs);
  if (st) return st;
  if (masks) {
    const int64_t n = R * (int64_t)ncols;
    k_emit_masks<<<(unsigned)cdiv(n, 256), 256, 0, hs>>>(W, ldw, (int)R, ncols, Ublk, ldu,
                                                         metric, masks, ldm, s);
    CRBQ_LAUNCH_CHECK();
  }
  return CRBQ_OK;
}

extern "C" int crbq_set_percentiles(const float* q81) {
  if (!q81) return CRBQ_ERR_ARG;
  return set_q_table(q81);
}

// Column blocks per super-block of the two-level GPTQ update: inside a
// super-block each block's error updates only the rest of the super-block
// (K = blocksize); at its end one GEMM with K = SB_BLOCKS * blocksize updates
// every later column.  Same sums as the reference's per-block
// W[:, ed:] -= Err @ U[st:ed, ed:] (bigptq.py:264), regrouped.
constexpr int SB_BLOCKS = 8;

extern "C" size_t crbq_fasterquant_workspace_size(int64_t R, int64_t C, const crbq_params* p) {
  const int bs = p ? p->blocksize : NCMAX;
  const int64_t sb = std::min<int64_t>((int64_t)SB_BLOCKS * bs, C);
  return search_ws_bytes(R) + (size_t)R * (size_t)sb * sizeof(float) + 512;
}

namespace crbq {
// The block loop over nseg sublayers of one shape (nseg = 1: one
// sublayer).  Segment i has its own weights Ws[i], factor Us[i] (segments
// may share one), losses, masks, traces and its own part of the workspace
// (search scratch and the super-block's error rows), so its results are
// those of a call of its own.
static int fasterquant_impl(int nseg, float* const* Ws, int64_t R, int64_t C, int64_t ldw,
                            const float* const* Us, int64_t ldu, const crbq_params* p,
                            float* const* losses, uint8_t* const* masks, int64_t ldm,
                            crbq_block_trace* const* traces, void* ws, size_t ws_bytes,
                            void* stream) {
  int st = check_params(p);
  if (st) return st;
  if (nseg < 1 || nseg > NSEG || !Ws || !Us || !losses) return CRBQ_ERR_ARG;
  if (R <= 0 || C <= 0 || ldw < C || ldu < C) return CRBQ_ERR_ARG;
  for (int i = 0; i < nseg; ++i)
    if (!Ws[i] || !Us[i] || !losses[i]) return CRBQ_ERR_ARG;
  // one launch updates every segment's outputs: two segments given the
  // same buffer would race (factors may be shared: they are only read)
  for (int i = 0; i < nseg; ++i)
    for (int j = 0; j < i; ++j)
      if (Ws[i] == Ws[j] || losses[i] == losses[j] ||
          (masks && masks[i] && masks[i] == masks[j]) ||
          (traces && traces[i] && traces[i] == traces[j]))
        return CRBQ_ERR_ARG;
  const bool any_masks = masks && masks[0];
  for (int i = 0; i < nseg; ++i)
    if (masks && ((masks[i] != nullptr) != any_masks)) return CRBQ_ERR_ARG;
  if (R * (int64_t)NCMAX >= (1 << 24)) return CRBQ_ERR_ARG;
  if (any_masks && ldm < C) return CRBQ_ERR_ARG;
  const int bs = p->blocksize;
  const int64_t SB = std::min<int64_t>((int64_t)SB_BLOCKS * bs, C);
  WsCarver c(ws, ws_bytes);
  SearchWs s[NSEG];
  float* err[NSEG] = {};
  for (int i = 0; i < nseg; ++i) {
    carve_search(c, R, s[i]);
    err[i] = c.take<float>((size_t)R * SB);
  }
  if (!c.ok()) return CRBQ_ERR_WORKSPACE;
  if (p->partition == 3) {
    // every block must be at least up_lim wide (torch.topk k <= n)
    const int64_t last = C - (C - 1) / bs * bs;
    if (last < p->up_lim || bs < p->up_lim) return CRBQ_ERR_TOPK;
  }
  st = ensure_q_table();
  if (st) return st;
  hipStream_t hs = (hipStream_t)stream;
  SegCtrl sc{};
  for (int i = 0; i < nseg; ++i) sc.c[i] = s[i].ctrl;
  k_init_ctrl<<<1, 64, 0, hs>>>(sc, nseg);
  CrbConsts k;
  k.lam = p->lam;
  k.omg = (float)(1.0 - (double)p->corr_damp);
  k.sym = false;
  k.skip = false;
  k.iters = p->refine_iters;
  const bool gptq = !p->disable_gptq;
  const int mf = method_family(p->method);
  const unsigned y = (unsigned)nseg;
  int bi = 0;
  for (int64_t sb0 = 0; sb0 < C; sb0 += SB) {
    const int64_t sb1 = std::min<int64_t>(sb0 + SB, C);
    for (int64_t st0 = sb0; st0 < sb1; st0 += bs, ++bi) {
      const int nc = (int)std::min<int64_t>(bs, sb1 - st0);
      if (p->partition == 3) {
        SegSearch seg{};
        for (int i = 0; i < nseg; ++i) {
          seg.W[i] = Ws[i] + st0;
          seg.U[i] = Us[i] + st0 * ldu + st0;
          seg.s[i] = s[i];
          seg.tr[i] = traces && traces[i] ? traces[i] + bi : nullptr;
        }
        st = search_block(seg, nseg, ldw, (int)R, nc, ldu, p->metric, p->up_lim, hs);
        if (st) return st;
      }
      QuantSegs qs{};
      bool vec = ldw % 4 == 0 && SB % 4 == 0 && (!any_masks || ldm % 4 == 0);
      for (int i = 0; i < nseg; ++i) {
        QuantArgs& a = qs.a[i];
        a.W = Ws[i] + st0; a.ldw = ldw; a.R = (int)R; a.nc = nc;
        a.U = Us[i] + st0 * ldu + st0; a.ldu = ldu;
        a.metric = p->metric; a.method = p->method; a.partition = p->partition;
        for (int g = 0; g < 3; ++g) a.orders[g] = p->orders[g];
        a.k = k;
        a.gptq = gptq;
        a.err = err[i] + (st0 - sb0); a.lde = SB;
        a.losses = losses[i];
        a.masks = any_masks ? masks[i] + st0 : nullptr; a.ldm = ldm;
        qs.s[i] = s[i];
        vec = vec && ((uintptr_t)a.W % 16 == 0) && ((uintptr_t)a.err % 16 == 0) &&
              (!a.masks || (uintptr_t)a.masks % 4 == 0);
      }
#define CRBQ_QUANT_GO(MF_)                                                          \
  do {                                                                              \
    if (vec && nc <= 128)                                                           \
      k_quantize_g<MF_><<<dim3((unsigned)cdiv(R, 256 / QG_LPR), y), 256, 0, hs>>>(qs); \
    else                                                                            \
      k_quantize<MF_, 2><<<dim3((unsigned)cdiv(R, 4), y), 256, 0, hs>>>(qs);       \
  } while (0)
      if (mf == MF_BRAQ) CRBQ_QUANT_GO(MF_BRAQ);
      else if (mf == MF_CRBOG) CRBQ_QUANT_GO(MF_CRBOG);
      else CRBQ_QUANT_GO(MF_CRB);
#undef CRBQ_QUANT_GO
      CRBQ_LAUNCH_CHECK();
      const int64_t ed = st0 + nc;
      if (gptq && ed < sb1) {            // rest of this super-block
        GemmArgs g[NSEG];
        for (int i = 0; i < nseg; ++i)
          g[i] = GemmArgs{false, false, false, R, sb1 - ed, nc, -1.f, qs.a[i].err, SB,
                          Us[i] + st0 * ldu + ed, ldu, 1.f, Ws[i] + ed, ldw, GEMM_TRI_NONE};
        st = sgemm_seg_launch(nseg, g, hs);
        if (st) return st;
      }
    }
    if (gptq && sb1 < C) {               // every later column, K = sb1 - sb0
      GemmArgs g[NSEG];
      for (int i = 0; i < nseg; ++i)
        g[i] = GemmArgs{false, false, false, R, C - sb1, sb1 - sb0, -1.f, err[i], SB,
                        Us[i] + sb0 * ldu + sb1, ldu, 1.f, Ws[i] + sb1, ldw, GEMM_TRI_NONE};
      st = sgemm_seg_launch(nseg, g, hs);
      if (st) return st;
    }
  }
  return CRBQ_OK;
}

// Scratch of the allocation-free entry point: one copy per device, in the
// code object's device memory, held until the process ends.  Host code
// never uses this name as an address (on the host it is only a stand-in):
// it asks for each device's address once, with that device current, and
// passes that pointer to the kernels.
static __device__ __align__(256) unsigned char scratch[CRBQ_NOALLOC_SCRATCH_BYTES];
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[MAXDEV] = {};

static bool noalloc_ready_on_current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAXDEV) return false;
  if (!q_table_ready[dev].load(std::memory_order_acquire)) return false;
  std::lock_guard<std::mutex> g(g_scratch_mu);
  return g_scratch_ptr[dev] != nullptr;
}

static int scratch_of_current_device(void** out) {
  int dev = 0;
  CRBQ_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= MAXDEV) return CRBQ_ERR_ARG;
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    CRBQ_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    if (!ptr) return CRBQ_ERR_HIP;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return CRBQ_OK;
}
}  // namespace crbq

extern "C" int crbq_fasterquant(float* W, int64_t R, int64_t C, int64_t ldw, const float* U,
                                int64_t ldu, const crbq_params* p, float* losses,
                                uint8_t* masks, int64_t ldm, crbq_block_trace* traces,
                                void* ws, size_t ws_bytes, void* stream) {
  return crbq::fasterquant_impl(1, &W, R, C, ldw, &U, ldu, p, &losses, &masks, ldm, &traces,
                                ws, ws_bytes, stream);
}

extern "C" size_t crbq_fasterquant_batched_workspace_size(int32_t nseg, int64_t R, int64_t C,
                                                          const crbq_params* p) {
  if (nseg < 1 || nseg > crbq::NSEG) return 0;
  return (size_t)nseg * crbq_fasterquant_workspace_size(R, C, p);
}

extern "C" int crbq_fasterquant_batched(int32_t nseg, float* const* W, int64_t R, int64_t C,
                                        int64_t ldw, const float* const* U, int64_t ldu,
                                        const crbq_params* p, float* const* losses,
                                        uint8_t* const* masks, int64_t ldm,
                                        crbq_block_trace* const* traces, void* ws,
                                        size_t ws_bytes, void* stream) {
  return crbq::fasterquant_impl(nseg, W, R, C, ldw, U, ldu, p, losses, masks, ldm, traces, ws,
                                ws_bytes, stream);
}

extern "C" int crbq_fasterquant_noalloc(float* W, int64_t R, int64_t C, int64_t ldw,
                                        const float* U, int64_t ldu, const crbq_params* p,
                                        float* losses, uint8_t* masks, int64_t ldm,
                                        crbq_block_trace* traces, void* stream) {
  const int st = crbq::check_params(p);
  if (st) return st;
  if (R <= 0 || C <= 0) return CRBQ_ERR_ARG;
  if (crbq_fasterquant_workspace_size(R, C, p) > CRBQ_NOALLOC_SCRATCH_BYTES)
    return CRBQ_ERR_TOO_LARGE;
  {
    // The per-device set-up (the percentile table's copy to the device and
    // the scratch address query) happens on a device's first call and
    // cannot be recorded into a graph: under capture it must already be done.
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    CRBQ_HIP(hipStreamIsCapturing((hipStream_t)stream, &cs));
    if (cs != hipStreamCaptureStatusNone && !crbq::noalloc_ready_on_current_device())
      return CRBQ_ERR_CAPTURE;
  }
  void* ws = nullptr;
  const int sst = crbq::scratch_of_current_device(&ws);
  if (sst) return sst;
  return crbq::fasterquant_impl(1, &W, R, C, ldw, &U, ldu, p, &losses, &masks, ldm, &traces,
                                ws, CRBQ_NOALLOC_SCRATCH_BYTES, stream);
}

// ---------------------------------------------------------------------------
// standalone Binarization.quantize
// ---------------------------------------------------------------------------
namespace crbq {
template <int MF, int EPL>
__global__ __launch_bounds__(256) void k_binarize(const float* x, int R, int nc, int64_t ldx,
                                                  const uint8_t* __restrict__ mask, int64_t ldm,
                                                  int order, int method, CrbConsts k, float* out,
                                                  int64_t ldo) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= R) return;
  float v[EPL], o[EPL];
  bool m[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    const int c = lane + 64 * e;
    const bool ok = c < nc;
    v[e] = ok ? x[(int64_t)row * ldx + c] : 0.f;
    m[e] = ok && mask[(int64_t)row * ldm + c] != 0;
  }
  binarize_row<MF, EPL>(method, v, m, order, k, o);
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    const int c = lane + 64 * e;
    if (c < nc) out[(int64_t)row * ldo + c] = o[e];
  }
}
// The same with the row's scales written to scales[row * lds ..] by lane 0
// (a check of the per-row scales, so one wavefront per row and no
// tuning: rows of up to 64 * EPL columns).
template <int MF, int EPL>
__global__ __launch_bounds__(256) void k_binarize_scales(const float* x, int R, int nc,
                                                         int64_t ldx,
                                                         const uint8_t* __restrict__ mask,
                                                         int64_t ldm, int order, int method,
                                                         CrbConsts k, float* out, int64_t ldo,
                                                         float* scales, int64_t lds, int nsc) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= R) return;
  float v[EPL], o[EPL];
  bool m[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    const int c = lane + 64 * e;
    const bool ok = c < nc;
    v[e] = ok ? x[(int64_t)row * ldx + c] : 0.f;
    m[e] = ok && mask[(int64_t)row * ldm + c] != 0;
  }
  float sc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) sc[i] = 0.f;
  binarize_row<MF, EPL>(method, v, m, order, k, o, sc);
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    const int c = lane + 64 * e;
    if (c < nc) out[(int64_t)row * ldo + c] = o[e];
  }
  if (lane == 0)
    for (int i = 0; i < nsc; ++i) scales[(int64_t)row * lds + i] = sc[i];
}

// Rows of at most EPL * LPR columns, LPR lanes per row (256 / LPR rows per
// workgroup), EPL elements per lane: lane r of a row holds columns
// h * 4 LPR + 4r .. h * 4 LPR + 4r + 3 for h < EPL / 4, moved with 16-byte
// accesses (x, out and their row strides 16-byte aligned, mask rows 4-byte
// aligned; the host checks).  Row reductions stay inside the row's lane
// group.
// One row of k_binarize_g.  FULL: the row is exactly 4 LPR NH columns, so
// every chunk is in range and the loads, mask tests and stores carry no
// per-chunk guards (a guarded chunk makes the compiler keep the mask as
// packed bytes across the branches and unpack it again).
template <int MF, int LPR, int EPL, bool FULL>
__device__ __forceinline__ void binarize_g_row(const float* xr, const uint8_t* mr, float* orow,
                                               int r, int nc, int order, int method,
                                               const CrbConsts& k) {
  constexpr int NH = EPL / 4;
  float v[EPL], o[EPL];
  bool m[EPL];
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    const int c0 = h * 4 * LPR + r * 4;
    if (FULL || c0 + 3 < nc) {
      const float4 q = *(const float4*)(xr + c0);
      const unsigned mb = *(const unsigned*)(mr + c0);
      v[4 * h] = q.x; v[4 * h + 1] = q.y; v[4 * h + 2] = q.z; v[4 * h + 3] = q.w;
#pragma unroll
      for (int j = 0; j < 4; ++j) m[4 * h + j] = ((mb >> (8 * j)) & 0xFF) != 0;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool ok = c0 + j < nc;
        v[4 * h + j] = ok ? xr[c0 + j] : 0.f;
        m[4 * h + j] = ok && mr[c0 + j] != 0;
      }
    }
  }
  binarize_row<MF, EPL, LPR>(method, v, m, order, k, o);
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    const int c0 = h * 4 * LPR + r * 4;
    if (FULL || c0 + 3 < nc) {
      *(float4*)(orow + c0) = make_float4(o[4 * h], o[4 * h + 1], o[4 * h + 2], o[4 * h + 3]);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (c0 + j < nc) orow[c0 + j] = o[4 * h + j];
    }
  }
}

template <int MF, int LPR, int EPL>
__global__ __launch_bounds__(256) void k_binarize_g(const float* x, int R, int nc, int64_t ldx,
                                                    const uint8_t* __restrict__ mask, int64_t ldm,
                                                    int order, int method, CrbConsts k,
                                                    float* out, int64_t ldo) {
  const int r = threadIdx.x % LPR;
  const int row = blockIdx.x * (256 / LPR) + threadIdx.x / LPR;
  if (row >= R) return;                      // whole lane groups leave together
  const float* xr = x + (int64_t)row * ldx;
  const uint8_t* mr = mask + (int64_t)row * ldm;
  float* orow = out + (int64_t)row * ldo;
  if (nc == EPL * LPR)
    binarize_g_row<MF, LPR, EPL, true>(xr, mr, orow, r, nc, order, method, k);
  else
    binarize_g_row<MF, LPR, EPL, false>(xr, mr, orow, r, nc, order, method, k);
}
}  // namespace crbq

#ifndef CRBQ_BIN_LPR
#define CRBQ_BIN_LPR 8
#endif
extern "C" int crbq_binarize(const float* x, int64_t R, int32_t ncols, int64_t ldx,
                             const uint8_t* mask, int64_t ldm, int32_t order, int32_t method,
                             float lam, float corr_damp, int32_t refine_iters, float* out,
                             int64_t ldo, void* stream) {
  if (!x || !mask || !out || R <= 0 || ncols <= 0 || ncols > 1024) return CRBQ_ERR_ARG;
  if (order < 1 || order > 8 || refine_iters < 0 || refine_iters > 64) return CRBQ_ERR_ARG;
  if (method < CRBQ_BRAQ || method > CRBQ_CRB_SYMDAMP_NOREFINE) return CRBQ_ERR_ARG;
  if (R > (int64_t)4 * 65535 * 1024) return CRBQ_ERR_ARG;
  CrbConsts k;
  k.lam = lam;
  k.omg = (float)(1.0 - (double)corr_damp);
  k.sym = false;
  k.skip = false;
  k.iters = refine_iters;
  hipStream_t hs = (hipStream_t)stream;
  const int r = (int)R;
  const bool vec = ((uintptr_t)x % 16 == 0) && ((uintptr_t)out % 16 == 0) && ldx % 4 == 0 &&
                   ldo % 4 == 0 && ((uintptr_t)mask % 4 == 0) && ldm % 4 == 0;
  const unsigned g4 = (unsigned)cdiv(R, 4);
#define CRBQ_BIN_GO(MF_)                                                                   \
  do {                                                                                     \
    if (vec && ncols <= 128)                                                               \
      k_binarize_g<MF_, CRBQ_BIN_LPR, 128 / CRBQ_BIN_LPR>                                    \
          <<<(unsigned)cdiv(R, 256 / CRBQ_BIN_LPR), 256, 0, hs>>>(x, r, ncols, ldx, mask, ldm, \
                                                                order, method, k, out, ldo); \
    else if (vec && ncols <= 256)                                                          \
      k_binarize_g<MF_, 32, 8><<<(unsigned)cdiv(R, 8), 256, 0, hs>>>(x, r, ncols, ldx, mask, \
                                                                      ldm, order, method, k, \
                                                                      out, ldo);           \
    else if (ncols <= 128)                                                                 \
      k_binarize<MF_, 2><<<g4, 256, 0, hs>>>(x, r, ncols, ldx, mask, ldm, order, method, k, \
                                             out, ldo);                                    \
    else if (ncols <= 256)                                                                 \
      k_binarize<MF_, 4><<<g4, 256, 0, hs>>>(x, r, ncols, ldx, mask, ldm, order, method, k, \
                                             out, ldo);                                    \
    else if (ncols <= 512)                                                                 \
      k_binarize<MF_, 8><<<g4, 256, 0, hs>>>(x, r, ncols, ldx, mask, ldm, order, method, k, \
                                             out, ldo);                                    \
    else                                                                                   \
      k_binarize<MF_, 16><<<g4, 256, 0, hs>>>(x, r, ncols, ldx, mask, ldm, order, method,  \
                                              k, out, ldo);                                \
  } while (0)
  const int mf = method_family(method);
  if (mf == MF_BRAQ) CRBQ_BIN_GO(MF_BRAQ);
  else if (mf == MF_CRBOG) CRBQ_BIN_GO(MF_CRBOG);
  else CRBQ_BIN_GO(MF_CRB);
#undef CRBQ_BIN_GO
  CRBQ_LAUNCH_CHECK();
  return CRBQ_OK;
}

extern "C" int crbq_binarize_scales(const float* x, int64_t R, int32_t ncols, int64_t ldx,
                                    const uint8_t* mask, int64_t ldm, int32_t order,
                                    int32_t method, float lam, float corr_damp,
                                    int32_t refine_iters, float* out, int64_t ldo,
                                    float* scales, int64_t lds, void* stream) {
  if (!x || !mask || !out || !scales || R <= 0 || ncols <= 0 || ncols > 1024)
    return CRBQ_ERR_ARG;
  if (order < 1 || order > 8 || refine_iters < 0 || refine_iters > 64) return CRBQ_ERR_ARG;
  if (method < CRBQ_BRAQ || method > CRBQ_CRB_SYMDAMP_NOREFINE) return CRBQ_ERR_ARG;
  if (R > (int64_t)4 * 65535 * 1024) return CRBQ_ERR_ARG;
  const int mf = method_family(method);
  const bool passes = mf == MF_BRAQ || (mf == MF_CRBOG && order == 1);
  const int nsc = passes ? 2 * order : 4;
  if (lds < nsc) return CRBQ_ERR_ARG;
  CrbConsts k;
  k.lam = lam;
  k.omg = (float)(1.0 - (double)corr_damp);
  k.sym = false;
  k.skip = false;
  k.iters = refine_iters;
  hipStream_t hs = (hipStream_t)stream;
  const unsigned g4 = (unsigned)cdiv(R, 4);
  const int r = (int)R;
#define CRBQ_BSC_GO(MF_, EPL_)                                                               \
  k_binarize_scales<MF_, EPL_><<<g4, 256, 0, hs>>>(x, r, ncols, ldx, mask, ldm, order, method, \
                                                   k, out, ldo, scales, lds, nsc)
#define CRBQ_BSC_MF(MF_)                                          \
  do {                                                            \
    if (ncols <= 128) CRBQ_BSC_GO(MF_, 2);                        \
    else if (ncols <= 256) CRBQ_BSC_GO(MF_, 4);                   \
    else if (ncols <= 512) CRBQ_BSC_GO(MF_, 8);                   \
    else CRBQ_BSC_GO(MF_, 16);                                    \
  } while (0)
  if (mf == MF_BRAQ) CRBQ_BSC_MF(MF_BRAQ);
  else if (mf == MF_CRBOG) CRBQ_BSC_MF(MF_CRBOG);
  else CRBQ_BSC_MF(MF_CRB);
#undef CRBQ_BSC_MF
#undef CRBQ_BSC_GO
  CRBQ_LAUNCH_CHECK();
  return CRBQ_OK;
}
