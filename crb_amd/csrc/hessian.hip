// Hessian accumulation of BRAGPTQ.add_batch (bigptq.py:37-53) on MFMA.
//
// S[I, J] += X[:, I]^T X[:, J] over token rows of X, for the upper-triangle
// 128x128 tiles I <= J of the fp32 C x C accumulator S.  The reference casts
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

constexpr int HT = 128;      // output tile
constexpr int HK = 64;       // tokens per LDS stage (16-bit inputs)
constexpr int HKP = HK + 8;  // padded LDS row (halves)
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

// 16-bit inputs (T8 = h8_t or b8_t; storage is 2 bytes per element)
template <typename T8>
__global__ __launch_bounds__(256) void k_syrk16(const uint16_t* __restrict__ X, int64_t ntok,
                                                int64_t ldx, int C, float* S, int64_t lds,
                                                int nt) {
  __shared__ __attribute__((aligned(16))) uint16_t Xs[2][HT][HKP];
  int ti, tj;
  tile_of(blockIdx.x, nt, ti, tj);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  const bool diag = ti == tj;
  // loader role: threads 0..127 -> tile I, 128..255 -> tile J
  const int side = tid >> 7, lt = tid & 127;
  const int cg = lt & 15, tg = lt >> 4;           // channel group (8), token group (8)
  const int cbase = (side ? tj : ti) * HT + cg * 8;
  const bool cvec = (cbase + 8 <= C) && ((ldx & 7) == 0) && ((((uintptr_t)X) & 15) == 0);
  f4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};

  for (int64_t t0 = 0; t0 < ntok; t0 += HK) {
    if (!(diag && side)) {
      uint32_t in[8][4];
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const int64_t t = t0 + tg * 8 + r;
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
      // transpose: out[c] dword m = (X[2m][c], X[2m+1][c])
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
        uint4 o;
        o.x = __builtin_amdgcn_perm(in[1][c >> 1], in[0][c >> 1], sel);
        o.y = __builtin_amdgcn_perm(in[3][c >> 1], in[2][c >> 1], sel);
        o.z = __builtin_amdgcn_perm(in[5][c >> 1], in[4][c >> 1], sel);
        o.w = __builtin_amdgcn_perm(in[7][c >> 1], in[6][c >> 1], sel);
        *(uint4*)&Xs[side][cg * 8 + c][tg * 8] = o;
      }
    }
    __syncthreads();
    const uint16_t(*XI)[HKP] = Xs[0];
    const uint16_t(*XJ)[HKP] = diag ? Xs[0] : Xs[1];
#pragma unroll
    for (int ks = 0; ks < HK; ks += 32) {
      const int kof = ks + (lane >> 4) * 8, r16 = lane & 15;
      T8 a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = *(const T8*)&XI[wm + i * 16 + r16][kof];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = *(const T8*)&XJ[wn + j * 16 + r16][kof];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16<T8>(a[i], b[j], acc[i][j]);
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

extern "C" int crbq_hessian_accum(const void* X, int dtype, int64_t ntok, int64_t ldx,
                                  int64_t C, float* S, int64_t lds, void* stream) {
  if (!X || !S || C <= 0 || ntok < 0 || ldx < C || lds < C) return CRBQ_ERR_ARG;
  if (C > (1 << 20)) return CRBQ_ERR_ARG;
  if (ntok == 0) return CRBQ_OK;
  const int nt = (int)((C + crbq::HT - 1) / crbq::HT);
  const int64_t ntiles = (int64_t)nt * (nt + 1) / 2;
  if (ntiles > 0x7fffffff) return CRBQ_ERR_ARG;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case CRBQ_F16:
      crbq::k_syrk16<h8_t><<<(unsigned)ntiles, 256, 0, s>>>((const uint16_t*)X, ntok, ldx,
                                                            (int)C, S, lds, nt);
      break;
    case CRBQ_BF16:
      crbq::k_syrk16<b8_t><<<(unsigned)ntiles, 256, 0, s>>>((const uint16_t*)X, ntok, ldx,
                                                            (int)C, S, lds, nt);
      break;
    case CRBQ_F32:
      crbq::k_syrk32<<<(unsigned)ntiles, 256, 0, s>>>((const float*)X, ntok, ldx, (int)C, S,
                                                      lds, nt);
      break;
    default:
      return CRBQ_ERR_ARG;
  }
  CRBQ_LAUNCH_CHECK();
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
