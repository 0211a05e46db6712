// Hessian accumulation of BRAGPTQ.add_batch (bigptq.py:37-53) on MFMA.
//
// S[I, J] += X[:, I]^T X[:, J] over token rows of X, for the upper-triangle
// tiles I <= J of the fp32 C x C accumulator S.  The reference casts
// the activations to fp32 and runs an SGEMM with TF32 off; f16/bf16 products
// are exact in fp32, so the f16/bf16 MFMA (v_mfma_f32_16x16x32_{f16,bf16},
// fp32 accumulate) computes the same sums up to summation order.  fp32
// inputs use v_mfma_f32_16x16x4_f32.
//
// Token-major X[t][c] is staged through LDS channel-major (Xs[c][t]) so each
// MFMA lane reads its 8 consecutive tokens with one ds_read_b128: every
// thread loads an 8-token x 8-channel block with eight 16-byte loads and
// transposes it in registers with v_perm_b32 before one 16-byte LDS store
// per channel.
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

// 16-bit inputs (T8 = h8_t or b8_t; storage is 2 bytes per element).
// 256 x 256 output tile per 512-thread workgroup; the 8 wavefronts form a
// 2 x 4 grid, each owning 128 x 64 outputs (8 x 4 MFMA 16x16x32 tiles).
// Tokens are staged SK at a time through double-buffered LDS: per stage
// thread t loads SK/32 4-token x 8-channel units of side I (t < 256) or J,
// ahead in registers, so global latency is covered by MFMA work
// (SK MFMAs per wavefront per stage).
// Split-K: workgroup (tile, s) sums tokens [s*span, (s+1)*span) and, when
// the grid is split, writes its partial tile to P[s] for k_sum_splits.
#ifndef CRBQ_SYRK_SK
#define CRBQ_SYRK_SK 64
#endif
#ifndef CRBQ_SYRK_DIST
#define CRBQ_SYRK_DIST 1
#endif
constexpr int ST = 256;                 // output tile (channels)
constexpr int SK = CRBQ_SYRK_SK;        // tokens per stage (multiple of 32)
constexpr int SKP = SK + 8;             // padded LDS row (halves)
constexpr int UNITS = SK / 32;          // 4-token x 8-channel units per thread per stage
constexpr int SYRK_THREADS = 512;

__device__ __forceinline__ void load_unit(const uint16_t* __restrict__ X, int64_t ntok,
                                          int64_t ldx, int C, int64_t t0, int cbase,
                                          bool cvec, uint32_t (&in)[4][4]) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t t = t0 + r;
    if (t < ntok && cvec) {
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
__device__ __forceinline__ void store_unit(uint16_t (*Xs)[SKP], int crow, int tcol,
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

struct StageRegs {
  uint32_t u[UNITS][4][4];
};

__device__ __forceinline__ void load_stage(const uint16_t* __restrict__ X, int64_t kend,
                                           int64_t ldx, int C, int64_t t0, int cbase, bool cvec,
                                           StageRegs& r) {
#pragma unroll
  for (int q = 0; q < UNITS; ++q) load_unit(X, kend, ldx, C, t0 + 32 * q, cbase, cvec, r.u[q]);
}

__device__ __forceinline__ void store_stage(uint16_t (*Xs)[SKP], int crow, int tcol,
                                            const StageRegs& r) {
#pragma unroll
  for (int q = 0; q < UNITS; ++q) store_unit(Xs, crow, tcol + 32 * q, r.u[q]);
}

template <typename T8>
__device__ __forceinline__ void syrk_stage(const uint16_t (*XI)[SKP], const uint16_t (*XJ)[SKP],
                                           int wm, int wn, int r16, int kof0, f4_t (&acc)[8][4]) {
#pragma unroll
  for (int ks = 0; ks < SK; ks += 32) {
    const int kof = ks + kof0;
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
}

template <typename T8>
__global__ __launch_bounds__(SYRK_THREADS) void k_syrk16(const uint16_t* __restrict__ X,
                                                         int64_t ntok, int64_t ldx, int C,
                                                         float* S, int64_t lds, int nt,
                                                         int64_t span, float* P) {
  __shared__ __attribute__((aligned(16))) uint16_t Xs[2][2][ST][SKP];
  int ti, tj;
  tile_of(blockIdx.x, nt, ti, tj);
  const int64_t k_beg = (int64_t)blockIdx.y * span;
  const int64_t k_end = k_beg + span < ntok ? k_beg + span : ntok;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = (wave >> 2) * 128, wn = (wave & 3) * 64;
  const bool diag = ti == tj;
  // token group fastest across lanes: the 8 channel rows a store
  // instruction touches then fall on distinct LDS bank groups
  const int side = tid >> 8, lt = tid & 255;
  const int tg = lt & 7, cg = lt >> 3;             // 8 token groups x 32 channel groups
  const int cbase = (side ? tj : ti) * ST + cg * 8;
  const bool cvec = (cbase + 8 <= C) && ((ldx & 7) == 0) && ((((uintptr_t)X) & 15) == 0);
  const bool loader = !(diag && side);
  f4_t acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};
  const int nch = k_end > k_beg ? (int)((k_end - k_beg + SK - 1) / SK) : 0;
  const int64_t t_lane = k_beg + tg * 4;
  const int r16 = lane & 15, kof0 = (lane >> 4) * 8;
#if CRBQ_SYRK_DIST == 1
  StageRegs ra;
  if (nch > 0 && loader) {
    load_stage(X, k_end, ldx, C, t_lane, cbase, cvec, ra);
    store_stage(Xs[0][side], cg * 8, tg * 4, ra);
  }
  __syncthreads();
  for (int c = 0; c < nch; ++c) {
    const int buf = c & 1;
    const bool more = c + 1 < nch;
    if (more && loader) load_stage(X, k_end, ldx, C, t_lane + (int64_t)(c + 1) * SK, cbase,
                                   cvec, ra);
    syrk_stage<T8>(Xs[buf][0], diag ? Xs[buf][0] : Xs[buf][1], wm, wn, r16, kof0, acc);
    if (more && loader) store_stage(Xs[buf ^ 1][side], cg * 8, tg * 4, ra);
    __syncthreads();
  }
#else
  // two stages in flight in registers (ra: next, rb: the one after)
  StageRegs ra, rb;
  if (nch > 0 && loader) {
    load_stage(X, k_end, ldx, C, t_lane, cbase, cvec, ra);
    store_stage(Xs[0][side], cg * 8, tg * 4, ra);
  }
  if (nch > 1 && loader) load_stage(X, k_end, ldx, C, t_lane + SK, cbase, cvec, ra);
  if (nch > 2 && loader) load_stage(X, k_end, ldx, C, t_lane + 2 * SK, cbase, cvec, rb);
  __syncthreads();
  for (int c = 0; c < nch; c += 2) {
    syrk_stage<T8>(Xs[0][0], diag ? Xs[0][0] : Xs[0][1], wm, wn, r16, kof0, acc);
    if (loader && c + 1 < nch) store_stage(Xs[1][side], cg * 8, tg * 4, ra);
    if (loader && c + 3 < nch)
      load_stage(X, k_end, ldx, C, t_lane + (int64_t)(c + 3) * SK, cbase, cvec, ra);
    __syncthreads();
    if (c + 1 >= nch) break;
    syrk_stage<T8>(Xs[1][0], diag ? Xs[1][0] : Xs[1][1], wm, wn, r16, kof0, acc);
    if (loader && c + 2 < nch) store_stage(Xs[0][side], cg * 8, tg * 4, rb);
    if (loader && c + 4 < nch)
      load_stage(X, k_end, ldx, C, t_lane + (int64_t)(c + 4) * SK, cbase, cvec, rb);
    __syncthreads();
  }
#endif
  const int c16 = lane & 15, r4 = (lane >> 4) * 4;
  float* out = P ? P + (size_t)blockIdx.y * (size_t)C * lds : S;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int gi = ti * ST + wm + i * 16 + r4 + r;
        const int gj = tj * ST + wn + j * 16 + c16;
        if (gi < C && gj < C && gi <= gj) {
          float* p = out + (int64_t)gi * lds + gj;
          *p = P ? acc[i][j][r] : *p + acc[i][j][r];
        }
      }
}

// S[i][j] += sum_s P[s][i][j] in split order, upper triangle
__global__ __launch_bounds__(256) void k_sum_splits(const float* __restrict__ P, int nsplit,
                                                    int C, float* S, int64_t lds) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int i = (int)(idx / C), j = (int)(idx % C);
  if (i >= C || j < i) return;
  float v = S[(int64_t)i * lds + j];
  for (int s = 0; s < nsplit; ++s) v = v + P[(size_t)s * C * lds + (int64_t)i * lds + j];
  S[(int64_t)i * lds + j] = v;
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

__global__ __launch_bounds__(256) void k_finalize(const float* S, int64_t lds, int C,
                                                  float scale, float* H, int64_t ldh) {
  // H may alias S: each thread owns the pair (i, j), (j, i) with i <= j.
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int i = (int)(idx / C), j = (int)(idx % C);
  if (i >= C || j < i) return;
  const float v = scale * S[(int64_t)i * lds + j];
  H[(int64_t)i * ldh + j] = v;
  H[(int64_t)j * ldh + i] = v;
}

}  // namespace crbq

namespace crbq {
static int num_cus() {
  static int cus = 0;
  if (!cus) {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
      cus = v;
    else
      cus = 256;
  }
  return cus;
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

extern "C" size_t crbq_hessian_workspace_size(int64_t ntok, int64_t C) {
  if (ntok <= 0 || C <= 0) return 0;
  const int ns = crbq::choose_splits(ntok, C, crbq::num_cus());
  return ns > 1 ? (size_t)ns * (size_t)C * (size_t)C * sizeof(float) : 0;
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
  int ns = crbq::choose_splits(ntok, C, crbq::num_cus());
  // the partial buffers are laid out like S (row stride lds)
  while (ns > 1 && (!ws || (size_t)ns * (size_t)C * (size_t)lds * sizeof(float) > ws_bytes)) --ns;
  int64_t span = (ntok + ns - 1) / ns;
  span = (span + crbq::SK - 1) / crbq::SK * crbq::SK;
  ns = (int)((ntok + span - 1) / span);
  float* P = ns > 1 ? (float*)ws : nullptr;
  dim3 grid((unsigned)ntiles, (unsigned)ns);
  if (dtype == CRBQ_F16)
    crbq::k_syrk16<h8_t><<<grid, crbq::SYRK_THREADS, 0, s>>>((const uint16_t*)X, ntok, ldx, (int)C, S, lds, nt,
                                              span, P);
  else
    crbq::k_syrk16<b8_t><<<grid, crbq::SYRK_THREADS, 0, s>>>((const uint16_t*)X, ntok, ldx, (int)C, S, lds, nt,
                                              span, P);
  CRBQ_LAUNCH_CHECK();
  if (P) {
    crbq::k_sum_splits<<<(unsigned)((C * C + 255) / 256), 256, 0, s>>>(P, ns, (int)C, S, lds);
    CRBQ_LAUNCH_CHECK();
  }
  return CRBQ_OK;
}

extern "C" int crbq_hessian_finalize(const float* S, int64_t lds, int64_t C, float scale,
                                     float* H, int64_t ldh, void* stream) {
  if (!S || !H || C <= 0 || lds < C || ldh < C) return CRBQ_ERR_ARG;
  const int64_t n = C * C;
  crbq::k_finalize<<<(unsigned)((n + 255) / 256), 256, 0, (hipStream_t)stream>>>(
      S, lds, (int)C, scale, H, ldh);
  CRBQ_LAUNCH_CHECK();
  return CRBQ_OK;
}
