// Packed low-bit storage of CRB/BRAQ-quantized weights and its GEMV.
//
// The reference stores the quantized layer as fake-quantized fp16/bf16
// weights (bigptq.py:278-280).  Within one 128-column block of one row,
// those weights take at most 2 distinct values in each non-salient group
// (mask1, mask2: order-1 binarization, mu +- alpha) and at most 4 on the
// salient columns (mask3: order 2, mu + a1 s1 + a2 s2); the salient columns
// of a block are whole columns, the same for every row
// (utils/structure.py:8-20).  So the layer is stored exactly as
//   codes [R][nblk * 32] bytes : 2 bits per weight, element j of a block at
//                                byte j / 4, bits 2 (j % 4) .. +1;
//   lut   [R][nblk][8]         : the block row's values in the weight
//                                dtype: mask1 {lo, hi}, mask2 {lo, hi},
//                                mask3 4 values, each ascending;
//   sal   [nblk][16] bytes     : salient-column bitmap of each block;
// with weight = lut[r][b][4 * sal + code], code = (mask2 ? 2 : 0) + rank
// for non-salient weights and rank (0..3) for salient ones: 3 bits per
// weight instead of 16, and unpacking reproduces the weights bit for bit.
#include <algorithm>

#include "common.h"

namespace crbq {

constexpr int PB = 128;   // packing block (columns)

// Order-preserving 16-bit keys: -0 sorts just below +0, so the two zeros
// are distinct values and round-trip exactly.
__device__ __forceinline__ int key16(uint32_t u) {
  return (u & 0x8000u) ? (int)(~u & 0xffffu) : (int)(u | 0x8000u);
}
__device__ __forceinline__ uint16_t unkey16(int k) {
  return (k & 0x8000) ? (uint16_t)(k & 0x7fff) : (uint16_t)(~k & 0xffff);
}
__device__ __forceinline__ int wave_min_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, CRBQ_WAVE));
  return v;
}
__device__ __forceinline__ int wave_or_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v |= __shfl_xor(v, o, CRBQ_WAVE);
  return v;
}

__global__ void k_zero_status(int* status, int* ex_count) {
  *status = 0;
  *ex_count = 0;
}

__device__ __forceinline__ float half_bits_to_float(uint32_t u, bool bf16) {
  return bf16 ? __uint_as_float(u << 16)
              : (float)__builtin_bit_cast(_Float16, (unsigned short)(u & 0xffffu));
}

constexpr int NDV = 8;    // distinct values a group's table is chosen from

// One wavefront per (row, block); lane l holds elements l and 64 + l.
// Per group (mask 1 and 2: 2 table entries, mask 3: 4) the table keeps the
// most frequent values among the group's NDV smallest distinct values (ties
// to the smaller key), in ascending order; every other element is an
// exception: code = the group's first entry, and (flat index r * C + c, raw
// value, value - first entry in fp32) appended to the exception list.
__global__ __launch_bounds__(256) void k_pack(const uint16_t* __restrict__ Q, int64_t ldq,
                                              const uint8_t* __restrict__ M, int64_t ldm,
                                              int R, int C, int nblk, bool bf16,
                                              uint8_t* __restrict__ codes, int64_t ldc,
                                              uint16_t* __restrict__ lut,
                                              uint8_t* __restrict__ sal,
                                              int64_t* __restrict__ ex_idx,
                                              uint16_t* __restrict__ ex_val,
                                              float* __restrict__ ex_delta, int ex_cap,
                                              int* ex_count, int* status) {
  const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (w >= (int64_t)R * nblk) return;   // whole wavefronts
  const int r = (int)(w / nblk), b = (int)(w % nblk), lane = threadIdx.x & 63;
  int key[2], grp[2];
  bool sal0[2], inside[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int c = b * PB + s * 64 + lane;
    inside[s] = c < C;
    key[s] = inside[s] ? key16(Q[(int64_t)r * ldq + c]) : 0;
    grp[s] = inside[s] ? M[(int64_t)r * ldm + c] : 0;
    sal0[s] = inside[s] && M[c] == 3;          // row 0 defines the salient columns
  }
  int err = 0;
  const uint64_t my0 = __ballot(grp[0] == 3), my1 = __ballot(grp[1] == 3);
  if (my0 != __ballot(sal0[0]) || my1 != __ballot(sal0[1])) err |= 2;
#pragma unroll
  for (int s = 0; s < 2; ++s)
    if (inside[s] && (grp[s] < 1 || grp[s] > 3)) err |= 4;
  int code[2] = {0, 0};
  bool exc[2] = {false, false};
  uint32_t lv[8];
#pragma unroll
  for (int G = 1; G <= 3; ++G) {
    const int cap = G == 3 ? 4 : 2, base = G == 1 ? 0 : (G == 2 ? 2 : 4);
    // the group's NDV smallest distinct keys and their counts (uniform)
    int cand[NDV], cnt[NDV], nd = 0, prev = -1;
#pragma unroll
    for (int k = 0; k < NDV; ++k) {
      int m = 0x10000;
#pragma unroll
      for (int s = 0; s < 2; ++s)
        if (grp[s] == G && key[s] > prev) m = min(m, key[s]);
      m = wave_min_i(m);
      cand[k] = m;
      cnt[k] = 0;
      if (m < 0x10000) {
        cnt[k] = __popcll(__ballot(grp[0] == G && key[0] == m)) +
                 __popcll(__ballot(grp[1] == G && key[1] == m));
        nd = k + 1;
        prev = m;
      }
    }
    // keep the cap most frequent (ties: smaller key), in ascending key order
    bool keep[NDV];
#pragma unroll
    for (int k = 0; k < NDV; ++k) {
      int better = 0;
#pragma unroll
      for (int q = 0; q < NDV; ++q)
        better += (q < nd && (cnt[q] > cnt[k] || (cnt[q] == cnt[k] && q < k))) ? 1 : 0;
      keep[k] = k < nd && better < cap;
    }
    int keys[4], found = 0;
#pragma unroll
    for (int k = 0; k < NDV; ++k)
      if (keep[k] && found < 4) keys[found++] = cand[k];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      if (grp[s] != G) continue;
      int rk = -1;
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (k < found && keys[k] == key[s]) rk = k;
      exc[s] = rk < 0;
      code[s] = (G == 2 ? 2 : 0) + (rk < 0 ? 0 : rk);
    }
#pragma unroll
    for (int k = 0; k < cap; ++k)
      lv[base + k] = found ? unkey16(keys[k < found ? k : found - 1]) : 0u;
  }
  // exceptions (rare): append to the list
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    if (!exc[s]) continue;
    const int c = b * PB + s * 64 + lane;
    const uint32_t v = unkey16(key[s]);
    const uint32_t t = lv[(grp[s] == 3 ? 4 : 0) + code[s]];
    const int e = atomicAdd(ex_count, 1);
    if (e < ex_cap) {
      ex_idx[e] = (int64_t)r * C + c;
      ex_val[e] = (uint16_t)v;
      ex_delta[e] = half_bits_to_float(v, bf16) - half_bits_to_float(t, bf16);
    } else {
      err |= 1;
    }
  }
  err = wave_or_i(err);
  if (lane == 0 && err) atomicOr(status, err);
  // byte t (lanes 0..31) packs elements 4t .. 4t+3, all in slot t / 16
  uint32_t byte = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int src = (4 * lane + i) & 63;
    const int c0 = __shfl(code[0], src, CRBQ_WAVE), c1 = __shfl(code[1], src, CRBQ_WAVE);
    byte |= (uint32_t)((lane < 16 ? c0 : c1) & 3) << (2 * i);
  }
  if (lane < 32) codes[(int64_t)r * ldc + b * 32 + lane] = (uint8_t)byte;
  if (lane < 4) {
    uint32_t v = lv[0] | (lv[1] << 16);
    if (lane == 1) v = lv[2] | (lv[3] << 16);
    if (lane == 2) v = lv[4] | (lv[5] << 16);
    if (lane == 3) v = lv[6] | (lv[7] << 16);
    ((uint32_t*)(lut + ((int64_t)r * nblk + b) * 8))[lane] = v;
  }
  if (r == 0 && lane == 0) {
    uint64_t* sp = (uint64_t*)(sal + (int64_t)b * 16);
    sp[0] = my0;
    sp[1] = my1;
  }
}

// One thread per code byte (4 weights).
__global__ __launch_bounds__(256) void k_unpack(const uint8_t* __restrict__ codes, int64_t ldc,
                                                const uint16_t* __restrict__ lut,
                                                const uint8_t* __restrict__ sal, int R, int C,
                                                int nblk, uint16_t* __restrict__ Q, int64_t ldq) {
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= (int64_t)R * nblk * 32) return;
  const int t = (int)(id & 31);
  const int64_t rb = id >> 5;
  const int r = (int)(rb / nblk), b = (int)(rb % nblk);
  const uint32_t cb = codes[(int64_t)r * ldc + b * 32 + t];
  const uint32_t sb = (uint32_t)(sal[(int64_t)b * 16 + (t >> 1)] >> (4 * (t & 1))) & 0xfu;
  const uint16_t* L = lut + ((int64_t)r * nblk + b) * 8;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = b * PB + 4 * t + i;
    if (c < C) Q[(int64_t)r * ldq + c] = L[4 * ((sb >> i) & 1) + ((cb >> (2 * i)) & 3)];
  }
}

// Exceptions of the packed form: the exact values over the unpacked ones.
__global__ __launch_bounds__(256) void k_unpack_ex(const int64_t* __restrict__ ex_idx,
                                                   const uint16_t* __restrict__ ex_val,
                                                   int64_t n_ex, int C, int64_t n,
                                                   uint16_t* __restrict__ Q, int64_t ldq) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= n_ex) return;
  const int64_t i = ex_idx[e];
  if (i < 0 || i >= n) return;           // indices outside R x C are ignored
  Q[(i / C) * ldq + i % C] = ex_val[e];
}

// y[t][r] += delta_e * x[t][c] for every exception e = (r, c), one thread
// per token, exceptions in list order (deterministic for a given list).
__global__ __launch_bounds__(256) void k_apply_ex(const int64_t* __restrict__ ex_idx,
                                                  const float* __restrict__ ex_delta,
                                                  int64_t n_ex, int C, int64_t n,
                                                  const uint16_t* __restrict__ x, int64_t ldx,
                                                  bool bf16, int T, float* __restrict__ y,
                                                  int64_t ldy) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= T) return;
  for (int64_t e = 0; e < n_ex; ++e) {
    const int64_t i = ex_idx[e];
    if (i < 0 || i >= n) continue;       // indices outside R x C are ignored
    const int r = (int)(i / C), c = (int)(i % C);
    y[(int64_t)t * ldy + r] += ex_delta[e] * half_bits_to_float(x[(int64_t)t * ldx + c], bf16);
  }
}

constexpr int GV_MAXVEC = 16;

// The codes of pair p (elements 2p, 2p+1 of a lane's 8) are bits 4p..4p+1
// and 4p+2..4p+3 of the 16-bit code word cw.  code_spread adds a copy of cw
// 14 bits higher, so that pair p's two codes sit at bits 4p..4p+1 and
// 4p+16..4p+17 for every p in 0..3, and one shift and one mask take them to
// bits 0-1 and 16-17 (bits 16-31 of the argument are dropped).
__device__ __forceinline__ uint32_t code_spread(uint32_t cw) {
  return (cw & 0xffffu) | (cw << 14);
}

// Two weights (elements 2p, 2p+1 of a lane's 8) from the block's table L:
// v_perm_b32 picks the 16-bit entries of codes (c_a, c_b) among the four
// non-salient entries and among the four salient ones; selb (sal_sel of the
// pair's two salient bits) takes each half from the salient or the
// non-salient pick.  d is code_spread of the code word.
__device__ __forceinline__ uint32_t decode_pair(uint32_t d, int p, uint4 L, uint32_t selb) {
  const uint32_t t = (d >> (4 * p)) & 0x00030003u;     // c_a | c_b << 16
  const uint32_t sel = t * 0x202u + 0x01000100u;
  const uint32_t wn = __builtin_amdgcn_perm(L.y, L.x, sel);
  const uint32_t ws = __builtin_amdgcn_perm(L.w, L.z, sel);
  return __builtin_amdgcn_perm(ws, wn, selb);
}

// The final selector of pair q (columns 2q, 2q + 1) of a lane's 32 columns
// from their salient bits sb: bytes 0-1 from the salient pick (perm source
// bytes 4-7) if column 2q is salient, bytes 2-3 likewise for 2q + 1.
__device__ __forceinline__ uint32_t sal_sel(uint32_t sb, int q) {
  const uint32_t s2 = (sb >> (2 * q)) & 3u;
  return 0x03020100u + (s2 & 1u) * 0x0404u + (s2 >> 1) * 0x04040000u;
}

// The 16 lanes of a DPP row (lanes 16 i .. 16 i + 15) decode the same 32
// columns (one row of W each), so their selectors are the same: lane r of
// the row builds pair r's (sal_sel(sb, r)) and the others read it with a
// row broadcast (DPP row_newbcast), one move instead of the bit arithmetic.
template <int Q>
__device__ __forceinline__ uint32_t row_bcast_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x150 + Q, 0xf, 0xf, true);
}
__device__ __forceinline__ uint32_t pair_sel(uint32_t mine, int q) {   // q constant when unrolled
  switch (q) {
    case 0: return row_bcast_u32<0>(mine);   case 1: return row_bcast_u32<1>(mine);
    case 2: return row_bcast_u32<2>(mine);   case 3: return row_bcast_u32<3>(mine);
    case 4: return row_bcast_u32<4>(mine);   case 5: return row_bcast_u32<5>(mine);
    case 6: return row_bcast_u32<6>(mine);   case 7: return row_bcast_u32<7>(mine);
    case 8: return row_bcast_u32<8>(mine);   case 9: return row_bcast_u32<9>(mine);
    case 10: return row_bcast_u32<10>(mine); case 11: return row_bcast_u32<11>(mine);
    case 12: return row_bcast_u32<12>(mine); case 13: return row_bcast_u32<13>(mine);
    case 14: return row_bcast_u32<14>(mine); default: return row_bcast_u32<15>(mine);
  }
}

template <typename T8>
__device__ __forceinline__ f4_t mfma_gv(T8 a, T8 b, f4_t c);
template <>
__device__ __forceinline__ f4_t mfma_gv<h8_t>(h8_t a, h8_t b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f4_t mfma_gv<b8_t>(b8_t a, b8_t b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// y[v][r] = sum_c W[r][c] x[v][c] for up to 16 vectors, W packed, x in the
// weights' 16-bit dtype, fp32 sums, on v_mfma_f32_16x16x32.  A workgroup
// takes 16 rows; its 16 wavefronts split the row's 128-column blocks into
// contiguous ranges.  Per block, lane l takes the 32 contiguous columns
// 32 (l >> 4) .. +31 of row l & 15 (8 bytes of codes, 4 of salient bits,
// the row-block's table) and the same columns of vector l & 15 (64 bytes),
// and feeds them to four MFMAs as 8-column slices: the MFMA sums over k in
// any order as long as A and B agree, so the columns need not be in the
// instruction's natural k order.  Decoding is the only per-weight vector
// work whatever nvec.  The wavefronts' 16 x 16 partial products are
// summed in LDS.
constexpr int GV_WAVES = 16;

template <typename T8>
__device__ __forceinline__ void gv_block(const uint8_t* crow, const uint4* lrow,
                                         const uint8_t* sal, const uint16_t* xv, int b, int kq,
                                         int C, bool row_ok, bool vec_ok, f4_t& acc) {
  const int c = b * PB + kq * 32;                // this lane's 32 columns
  const uint2 cw = row_ok ? *(const uint2*)(crow + b * 32 + kq * 8) : make_uint2(0u, 0u);
  const uint32_t sb = *(const uint32_t*)(sal + (int64_t)b * 16 + kq * 4);
  const uint4 L = row_ok ? lrow[b] : make_uint4(0u, 0u, 0u, 0u);
  uint4 xs[4];
  if (c + 32 <= C) {                             // all blocks but a ragged last one
    const uint4* xp = (const uint4*)(xv + c);
#pragma unroll
    for (int k = 0; k < 4; ++k) xs[k] = vec_ok ? xp[k] : make_uint4(0u, 0u, 0u, 0u);
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t h[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int cc = c + 8 * k + e;
        h[e] = vec_ok && cc < C ? xv[cc] : 0u;
      }
      xs[k] = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                         h[6] | (h[7] << 16));
    }
  }
  const uint32_t mine = sal_sel(sb, (int)(threadIdx.x & 15));
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t cws = code_spread((k < 2 ? cw.x : cw.y) >> (16 * (k & 1)));
    uint4 a;
    a.x = decode_pair(cws, 0, L, pair_sel(mine, 4 * k));
    a.y = decode_pair(cws, 1, L, pair_sel(mine, 4 * k + 1));
    a.z = decode_pair(cws, 2, L, pair_sel(mine, 4 * k + 2));
    a.w = decode_pair(cws, 3, L, pair_sel(mine, 4 * k + 3));
    acc = mfma_gv<T8>(__builtin_bit_cast(T8, a), __builtin_bit_cast(T8, xs[k]), acc);
  }
}

template <typename T8>
__global__ __launch_bounds__(64 * GV_WAVES) void k_gemv_packed(
    const uint8_t* __restrict__ codes, int64_t ldc, const uint16_t* __restrict__ lut,
    const uint8_t* __restrict__ sal, int R, int C, int nblk, const uint16_t* __restrict__ x,
    int64_t ldx, int nvec, float* __restrict__ y, int64_t ldy) {
  __shared__ float red[GV_WAVES][16][17];
  const int r0 = blockIdx.x * 16;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row = r0 + (lane & 15), kq = lane >> 4, vec = lane & 15;
  const bool row_ok = row < R, vec_ok = vec < nvec;
  const int b_beg = (int)((int64_t)nblk * wave / GV_WAVES);
  const int b_end = (int)((int64_t)nblk * (wave + 1) / GV_WAVES);
  const uint8_t* crow = codes + (int64_t)(row_ok ? row : 0) * ldc;
  const uint4* lrow = (const uint4*)(lut + (int64_t)(row_ok ? row : 0) * nblk * 8);
  const uint16_t* xv = x + (int64_t)(vec_ok ? vec : 0) * ldx;
  f4_t acc = {0.f, 0.f, 0.f, 0.f};
  int b = b_beg;
  for (; b + 1 < b_end; b += 2) {
    gv_block<T8>(crow, lrow, sal, xv, b, kq, C, row_ok, vec_ok, acc);
    gv_block<T8>(crow, lrow, sal, xv, b + 1, kq, C, row_ok, vec_ok, acc);
  }
  if (b < b_end) gv_block<T8>(crow, lrow, sal, xv, b, kq, C, row_ok, vec_ok, acc);
  // acc[i] = partial y[vector lane & 15][row r0 + 4 (lane >> 4) + i]
#pragma unroll
  for (int i = 0; i < 4; ++i) red[wave][4 * (lane >> 4) + i][lane & 15] = acc[i];
  __syncthreads();
  const int t = threadIdx.x;
  if (t < 256) {
    const int rr = t >> 4, v = t & 15;
    if (v < nvec && r0 + rr < R) {
      float s0 = 0.f;
#pragma unroll
      for (int w = 0; w < GV_WAVES; ++w) s0 += red[w][rr][v];
      y[(int64_t)v * ldy + r0 + rr] = s0;
    }
  }
}

// Y[t][r] = sum_c W[r][c] X[t][c] for many tokens (prefill), W packed:
// the GEMV's decode, with each decoded fragment reused for a tile of
// tokens.  A workgroup of GM_WAVES wavefronts covers 16 * GM_WAVES rows x
// TT tokens (64, or 128 for more than 64 tokens); per 128-column block each wavefront decodes its 16 rows'
// 128 columns (lane l: row l & 15, columns 32 (l >> 4) .. +31, four
// 8-column MFMA slices) and multiplies them with every 16-token group of
// the X tile, which the whole workgroup stages in LDS (rows padded to 136
// halves so a 16-lane group's 16-byte reads of 16 tokens fall on disjoint
// banks).  The X tile of the next block (with 64-token tiles also its codes,
// salient bits and table) is loaded into registers while the current one is
// used.  When row and token tiles alone would leave CUs idle
// the block range is split over gridDim.z workgroups, each writing an fp32
// partial [T][R] slice that k_gemm_packed_sum adds in split order.
constexpr int GM_WAVES = 8;
constexpr int GM_ROWS = 16 * GM_WAVES;
constexpr int GM_XP = PB + 8;                     // LDS pitch of an X tile row (halves)

static inline int gemm_packed_tt(int64_t T) { return T > 64 ? 128 : 64; }

template <typename T8, int GM_TT>
__global__ __launch_bounds__(64 * GM_WAVES) void k_gemm_packed(
    const uint8_t* __restrict__ codes, int64_t ldc, const uint16_t* __restrict__ lut,
    const uint8_t* __restrict__ sal, int R, int C, int nblk, const uint16_t* __restrict__ x,
    int64_t ldx, int T, int bps, float* __restrict__ y, int64_t ldy) {
  __shared__ __attribute__((aligned(16))) uint16_t Xs[2][GM_TT][GM_XP];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int r0 = blockIdx.x * GM_ROWS, t0 = blockIdx.y * GM_TT;
  const int b_beg = blockIdx.z * bps, b_end = min(nblk, b_beg + bps);
  const int row = r0 + wave * 16 + (lane & 15), kq = lane >> 4;
  const bool row_ok = row < R;
  const uint8_t* crow = codes + (int64_t)(row_ok ? row : 0) * ldc;
  const uint4* lrow = (const uint4*)(lut + (int64_t)(row_ok ? row : 0) * nblk * 8);
  // X tile loader: thread -> (token xt, XPT 8-column chunks from xc)
  constexpr int XPT = GM_TT * PB / 8 / (64 * GM_WAVES);     // 16-byte chunks per thread
  constexpr int TPR = PB / 8 / XPT;                         // threads per token row
  const int xt = tid / TPR, xc = (tid % TPR) * XPT * 8;
  const int tok = t0 + xt;
  const bool tok_ok = tok < T;
  const uint16_t* xrow = x + (int64_t)(tok_ok ? tok : 0) * ldx;
  auto load_x = [&](int b, uint4 (&u)[XPT]) {
    const int c = b * PB + xc;
    if (tok_ok && c + 8 * XPT <= C) {
#pragma unroll
      for (int k = 0; k < XPT; ++k) u[k] = *(const uint4*)(xrow + c + 8 * k);
    } else {
#pragma unroll
      for (int k = 0; k < XPT; ++k) {
        uint32_t h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = tok_ok && c + 8 * k + e < C ? xrow[c + 8 * k + e] : 0u;
        u[k] = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                          h[6] | (h[7] << 16));
      }
    }
  };
  f4_t acc[GM_TT / 16];
#pragma unroll
  for (int g = 0; g < GM_TT / 16; ++g) acc[g] = f4_t{0.f, 0.f, 0.f, 0.f};
  // With 64-token tiles a block's codes, salient bits and table are loaded
  // with its X tile, one block ahead, so that the decode never waits on
  // them (rows past R read row 0 through crow and lrow: an MFMA output row
  // depends only on its own weight row, and those rows are not stored);
  // 128-token tiles spread each decode over 8 token groups and load them
  // after the barrier.
  constexpr bool codes_ahead = GM_TT == 64;
  uint4 u[XPT];
  uint2 cwn = make_uint2(0u, 0u);
  uint32_t sbn = 0u;
  uint4 Ln = make_uint4(0u, 0u, 0u, 0u);
  auto load_codes = [&](int b) {
    cwn = *(const uint2*)(crow + b * 32 + kq * 8);
    sbn = *(const uint32_t*)(sal + (int64_t)b * 16 + kq * 4);
    Ln = lrow[b];
  };
  if (b_beg < b_end) {
    if constexpr (codes_ahead) load_codes(b_beg);
    load_x(b_beg, u);
  }
  for (int b = b_beg; b < b_end; ++b) {
    const int buf = (b - b_beg) & 1;
#pragma unroll
    for (int k = 0; k < XPT; ++k) *(uint4*)&Xs[buf][xt][xc + 8 * k] = u[k];
    __syncthreads();
    uint2 cw;
    uint32_t sb;
    uint4 L;
    if constexpr (codes_ahead) {
      cw = cwn;
      sb = sbn;
      L = Ln;
      if (b + 1 < b_end) {
        load_codes(b + 1);
        load_x(b + 1, u);
      }
    } else {
      if (b + 1 < b_end) load_x(b + 1, u);
      cw = row_ok ? *(const uint2*)(crow + b * 32 + kq * 8) : make_uint2(0u, 0u);
      sb = *(const uint32_t*)(sal + (int64_t)b * 16 + kq * 4);
      L = row_ok ? lrow[b] : make_uint4(0u, 0u, 0u, 0u);
    }
    T8 a[4];
    const uint32_t mine = sal_sel(sb, lane & 15);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t cws = code_spread((k < 2 ? cw.x : cw.y) >> (16 * (k & 1)));
      uint4 q;
      q.x = decode_pair(cws, 0, L, pair_sel(mine, 4 * k));
      q.y = decode_pair(cws, 1, L, pair_sel(mine, 4 * k + 1));
      q.z = decode_pair(cws, 2, L, pair_sel(mine, 4 * k + 2));
      q.w = decode_pair(cws, 3, L, pair_sel(mine, 4 * k + 3));
      a[k] = __builtin_bit_cast(T8, q);
    }
#pragma unroll
    for (int g = 0; g < GM_TT / 16; ++g) {
      if (t0 + g * 16 >= T) break;                // token groups past the end (uniform)
      const uint16_t* xr = &Xs[buf][g * 16 + (lane & 15)][kq * 32];
#pragma unroll
      for (int k = 0; k < 4; ++k)
        acc[g] = mfma_gv<T8>(a[k], *(const T8*)(xr + 8 * k), acc[g]);
    }
    // the other buffer is written next; this one is only read again after
    // the following iteration's barrier
  }
  // acc[g][i] = y[token t0 + 16 g + (lane & 15)][row r0 + 16 wave + 4 (lane >> 4) + i]
  float* out = y + (size_t)blockIdx.z * (size_t)T * (size_t)ldy;
  const int rb = r0 + wave * 16 + 4 * kq;
#pragma unroll
  for (int g = 0; g < GM_TT / 16; ++g) {
    const int t = t0 + g * 16 + (lane & 15);
    if (t >= T) continue;
    float* o = out + (int64_t)t * ldy + rb;
    if (rb + 3 < R && ((((uintptr_t)o) & 15) == 0)) {
      *(float4*)o = make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (rb + i < R) o[i] = acc[g][i];
    }
  }
}

// y[t][r] = sum_s P[s][t][r] in split order
__global__ __launch_bounds__(256) void k_gemm_packed_sum(const float* __restrict__ P, int ns,
                                                         int T, int R, int64_t ldp,
                                                         float* __restrict__ y, int64_t ldy) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)T * R) return;
  const int t = (int)(idx / R), r = (int)(idx % R);
  float v = 0.f;
  for (int s = 0; s < ns; ++s) v += P[((int64_t)s * T + t) * ldp + r];
  y[(int64_t)t * ldy + r] = v;
}

// Split of the block range: as many splits as keep the workgroups within
// 512 (two per CU of an MI355X, one round: a few workgroups past it would
// run as a second round), at least 8 blocks per split; a function of the
// shapes only, so the workspace size is known without a device.
constexpr int GM_TARGET_WG = 512;
static inline int gemm_packed_splits(int64_t R, int64_t C, int64_t T, int* bps) {
  const int64_t nblk = (C + PB - 1) / PB;
  const int64_t tt = gemm_packed_tt(T);
  const int64_t tiles = ((R + GM_ROWS - 1) / GM_ROWS) * ((T + tt - 1) / tt);
  int64_t ns = GM_TARGET_WG / tiles;
  ns = std::max<int64_t>(1, std::min<int64_t>(ns, nblk / 8));
  const int64_t per = (nblk + ns - 1) / ns;
  *bps = (int)per;
  return (int)((nblk + per - 1) / per);
}

}  // namespace crbq

extern "C" int crbq_pack(const void* Q, int dtype, int64_t R, int64_t C, int64_t ldq,
                         const uint8_t* masks, int64_t ldm, uint8_t* codes, int64_t ldc,
                         void* lut, uint8_t* sal, int64_t* ex_idx, void* ex_val,
                         float* ex_delta, int ex_cap, int* ex_count, int* status,
                         void* stream) {
  if (!Q || !masks || !codes || !lut || !sal || !status || !ex_count) return CRBQ_ERR_ARG;
  if (ex_cap < 0 || (ex_cap > 0 && (!ex_idx || !ex_val || !ex_delta))) return CRBQ_ERR_ARG;
  if (dtype != CRBQ_F16 && dtype != CRBQ_BF16) return CRBQ_ERR_ARG;
  if (R <= 0 || C <= 0 || R > 0x7fffffff || C > 0x7fffffff || ldq < C || ldm < C)
    return CRBQ_ERR_ARG;
  const int64_t nblk = (C + crbq::PB - 1) / crbq::PB;
  if (ldc < nblk * 32 || (ldc & 7) || (((uintptr_t)lut) & 15) || (((uintptr_t)sal) & 7) ||
      (((uintptr_t)codes) & 7))
    return CRBQ_ERR_ARG;
  hipStream_t s = (hipStream_t)stream;
  crbq::k_zero_status<<<1, 1, 0, s>>>(status, ex_count);
  CRBQ_LAUNCH_CHECK();
  const int64_t waves = R * nblk;
  crbq::k_pack<<<(unsigned)((waves + 3) / 4), 256, 0, s>>>(
      (const uint16_t*)Q, ldq, masks, ldm, (int)R, (int)C, (int)nblk, dtype == CRBQ_BF16, codes,
      ldc, (uint16_t*)lut, sal, ex_idx, (uint16_t*)ex_val, ex_delta, ex_cap, ex_count, status);
  CRBQ_LAUNCH_CHECK();
  return CRBQ_OK;
}

extern "C" int crbq_unpack(const uint8_t* codes, int64_t ldc, const void* lut, const uint8_t* sal,
                           const int64_t* ex_idx, const void* ex_val, int64_t n_ex, int dtype,
                           int64_t R, int64_t C, void* Q, int64_t ldq, void* stream) {
  if (!codes || !lut || !sal || !Q) return CRBQ_ERR_ARG;
  if (n_ex < 0 || (n_ex > 0 && (!ex_idx || !ex_val))) return CRBQ_ERR_ARG;
  if (dtype != CRBQ_F16 && dtype != CRBQ_BF16) return CRBQ_ERR_ARG;
  if (R <= 0 || C <= 0 || R > 0x7fffffff || C > 0x7fffffff || ldq < C) return CRBQ_ERR_ARG;
  const int64_t nblk = (C + crbq::PB - 1) / crbq::PB;
  if (ldc < nblk * 32) return CRBQ_ERR_ARG;
  const int64_t n = R * nblk * 32;
  hipStream_t s = (hipStream_t)stream;
  crbq::k_unpack<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(
      codes, ldc, (const uint16_t*)lut, sal, (int)R, (int)C, (int)nblk, (uint16_t*)Q, ldq);
  CRBQ_LAUNCH_CHECK();
  if (n_ex > 0) {
    crbq::k_unpack_ex<<<(unsigned)((n_ex + 255) / 256), 256, 0, s>>>(
        ex_idx, (const uint16_t*)ex_val, n_ex, (int)C, R * C, (uint16_t*)Q, ldq);
    CRBQ_LAUNCH_CHECK();
  }
  return CRBQ_OK;
}

static int apply_ex(const int64_t* ex_idx, const float* ex_delta, int64_t n_ex, int64_t R,
                    int64_t C, const void* x, int64_t ldx, int dtype, int64_t T, float* y,
                    int64_t ldy, hipStream_t s) {
  if (n_ex <= 0) return CRBQ_OK;
  crbq::k_apply_ex<<<(unsigned)((T + 255) / 256), 256, 0, s>>>(
      ex_idx, ex_delta, n_ex, (int)C, R * C, (const uint16_t*)x, ldx, dtype == CRBQ_BF16,
      (int)T, y, ldy);
  CRBQ_LAUNCH_CHECK();
  return CRBQ_OK;
}

extern "C" int crbq_gemv_packed(const uint8_t* codes, int64_t ldc, const void* lut,
                                const uint8_t* sal, const int64_t* ex_idx,
                                const float* ex_delta, int64_t n_ex, int dtype, int64_t R,
                                int64_t C, const void* x, int64_t ldx, int nvec, float* y,
                                int64_t ldy, void* stream) {
  if (!codes || !lut || !sal || !x || !y) return CRBQ_ERR_ARG;
  if (n_ex < 0 || (n_ex > 0 && (!ex_idx || !ex_delta))) return CRBQ_ERR_ARG;
  if (dtype != CRBQ_F16 && dtype != CRBQ_BF16) return CRBQ_ERR_ARG;
  if (R <= 0 || C <= 0 || R > 0x7fffffff || C > 0x7fffffff) return CRBQ_ERR_ARG;
  if (nvec < 1 || nvec > crbq::GV_MAXVEC || ldx < C || ldy < R) return CRBQ_ERR_ARG;
  const int64_t nblk = (C + crbq::PB - 1) / crbq::PB;
  if (ldc < nblk * 32 || (ldc & 7) || (ldx & 7) || (((uintptr_t)x) & 15) ||
      (((uintptr_t)lut) & 15) || (((uintptr_t)codes) & 7) || (((uintptr_t)sal) & 3))
    return CRBQ_ERR_ARG;
  const unsigned grid = (unsigned)((R + 15) / 16);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == CRBQ_BF16)
    crbq::k_gemv_packed<b8_t><<<grid, 64 * crbq::GV_WAVES, 0, s>>>(
        codes, ldc, (const uint16_t*)lut, sal, (int)R, (int)C, (int)nblk, (const uint16_t*)x,
        ldx, nvec, y, ldy);
  else
    crbq::k_gemv_packed<h8_t><<<grid, 64 * crbq::GV_WAVES, 0, s>>>(
        codes, ldc, (const uint16_t*)lut, sal, (int)R, (int)C, (int)nblk, (const uint16_t*)x,
        ldx, nvec, y, ldy);
  CRBQ_LAUNCH_CHECK();
  return apply_ex(ex_idx, ex_delta, n_ex, R, C, x, ldx, dtype, nvec, y, ldy, s);
}

extern "C" size_t crbq_gemm_packed_workspace_size(int64_t R, int64_t C, int64_t ntok) {
  if (R <= 0 || C <= 0 || ntok <= 0) return 0;
  int bps = 0;
  const int ns = crbq::gemm_packed_splits(R, C, ntok, &bps);
  return ns > 1 ? (size_t)ns * (size_t)ntok * (size_t)R * sizeof(float) : 0;
}

extern "C" int crbq_gemm_packed(const uint8_t* codes, int64_t ldc, const void* lut,
                                const uint8_t* sal, const int64_t* ex_idx,
                                const float* ex_delta, int64_t n_ex, int dtype, int64_t R,
                                int64_t C, const void* x, int64_t ldx, int64_t ntok, float* y,
                                int64_t ldy, void* ws, size_t ws_bytes, void* stream) {
  if (!codes || !lut || !sal || !x || !y) return CRBQ_ERR_ARG;
  if (n_ex < 0 || (n_ex > 0 && (!ex_idx || !ex_delta))) return CRBQ_ERR_ARG;
  if (dtype != CRBQ_F16 && dtype != CRBQ_BF16) return CRBQ_ERR_ARG;
  if (R <= 0 || C <= 0 || ntok <= 0 || R > 0x7fffffff || C > 0x7fffffff || ntok > 0x7fffffff ||
      ldx < C || ldy < R)
    return CRBQ_ERR_ARG;
  const int64_t nblk = (C + crbq::PB - 1) / crbq::PB;
  if (ldc < nblk * 32 || (ldc & 7) || (ldx & 7) || (((uintptr_t)x) & 15) ||
      (((uintptr_t)lut) & 15) || (((uintptr_t)codes) & 7) || (((uintptr_t)sal) & 3))
    return CRBQ_ERR_ARG;
  int bps = 0;
  const int ns = crbq::gemm_packed_splits(R, C, ntok, &bps);
  const size_t need = ns > 1 ? (size_t)ns * (size_t)ntok * (size_t)R * sizeof(float) : 0;
  if (need && (!ws || ws_bytes < need)) return CRBQ_ERR_WORKSPACE;
  float* out = ns > 1 ? (float*)ws : y;
  const int64_t ldo = ns > 1 ? R : ldy;
  const int tt = crbq::gemm_packed_tt(ntok);
  dim3 grid((unsigned)((R + crbq::GM_ROWS - 1) / crbq::GM_ROWS),
            (unsigned)((ntok + tt - 1) / tt), (unsigned)ns);
  if (grid.y > 65535) return CRBQ_ERR_ARG;
  hipStream_t s = (hipStream_t)stream;
#define CRBQ_GM_LAUNCH(T8, TT)                                                                  \
  crbq::k_gemm_packed<T8, TT><<<grid, 64 * crbq::GM_WAVES, 0, s>>>(                             \
      codes, ldc, (const uint16_t*)lut, sal, (int)R, (int)C, (int)nblk, (const uint16_t*)x,     \
      ldx, (int)ntok, bps, out, ldo)
  if (dtype == CRBQ_BF16) {
    if (tt == 128) CRBQ_GM_LAUNCH(b8_t, 128); else CRBQ_GM_LAUNCH(b8_t, 64);
  } else {
    if (tt == 128) CRBQ_GM_LAUNCH(h8_t, 128); else CRBQ_GM_LAUNCH(h8_t, 64);
  }
#undef CRBQ_GM_LAUNCH
  CRBQ_LAUNCH_CHECK();
  if (ns > 1) {
    const int64_t n = ntok * R;
    crbq::k_gemm_packed_sum<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(
        out, ns, (int)ntok, (int)R, R, y, ldy);
    CRBQ_LAUNCH_CHECK();
  }
  return apply_ex(ex_idx, ex_delta, n_ex, R, C, x, ldx, dtype, ntok, y, ldy, s);
}
