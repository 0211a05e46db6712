// Per-row binarizers of the three in-scope techniques: a row is held by an
// aligned group of LPR lanes (64: one wavefront per row; 16: four rows per
// wavefront), EPL elements per lane.  Elementwise arithmetic is fp32 in the
// reference's operation order (compiled with -ffp-contract=off so nothing is
// fused); row reductions are fp32 sums as the reference's torch.sum is: each
// lane adds its EPL elements in order, then the lanes are combined pairwise
// (DPP / permlane tree, every lane of the group ending with the same bits).
// The order differs from torch's, so sums agree to fp32 rounding.
// A product a * B with B = sign(.) in {-1, 0, +1} is exact, so the
// reference's fl(x - fl(a * B)) and fl(x + fl(a * B)) are one rounding of
// an exact value: fma(-a, B, x) and fma(a, B, x) give the same bits in one
// instruction.
#pragma once
#include "common.h"

namespace crbq {

struct CrbConsts {
  float lam;    // fp32(lam)                   (binary.py:1589  A = d + lam)
  float omg;    // fp32(1 - corr_damp)        (binary.py:1584-1587)
  bool sym;     // symmetric_damp
  bool skip;    // skip_refinement
  int iters;    // refinement rounds (reference: 1)
};

// Pairwise sum of a lane's terms (depth log2(EPL) instead of EPL - 1
// dependent adds).
template <int N>
__device__ __forceinline__ float tree_sum(float (&t)[N]) {
#pragma unroll
  for (int w = 1; w < N; w <<= 1)
#pragma unroll
    for (int e = 0; e + w < N; e += 2 * w) t[e] = t[e] + t[e + w];
  return t[0];
}

template <int EPL, int LPR = 64>
__device__ __forceinline__ float rsum(const float (&v)[EPL], const bool (&m)[EPL]) {
  float t[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) t[e] = m[e] ? v[e] : 0.f;
  return group_sum_f<LPR>(tree_sum(t));
}

template <int EPL, int LPR = 64>
__device__ __forceinline__ float rsum_abs(const float (&v)[EPL], const bool (&m)[EPL]) {
  float t[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) t[e] = m[e] ? fabsf(v[e]) : 0.f;
  return group_sum_f<LPR>(tree_sum(t));
}

// x / d for an integer-valued d in [1, 1024] given r = 1 / d (IEEE): the
// product and one fma correction give the correctly rounded quotient, the
// same bits as x / d (checked for every fp32 significand and every such d:
// tests/test_arith.py), for 3 instructions instead of a full division.
__device__ __forceinline__ float div_cnt(float x, float d, float r) {
  const float q = x * r;
  const float e = __builtin_fmaf(-q, d, x);
  return __builtin_fmaf(e, r, q);
}

// sum of values that are already 0 outside the mask
template <int EPL, int LPR = 64>
__device__ __forceinline__ float rsum_z(const float (&v)[EPL]) {
  float t[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) t[e] = v[e];
  return group_sum_f<LPR>(tree_sum(t));
}

// sum of a * b where every product is exact (one factor a sign in
// {-1, 0, +1}): fma(a, b, s) is fl(s + fl(a * b)) in one instruction
template <int EPL, int LPR = 64>
__device__ __forceinline__ float rdot_sign(const float (&a)[EPL], const float (&b)[EPL]) {
  float t[EPL / 2];
#pragma unroll
  for (int e = 0; e < EPL / 2; ++e) t[e] = __builtin_fmaf(a[2 * e + 1], b[2 * e + 1], a[2 * e] * b[2 * e]);
  return group_sum_f<LPR>(tree_sum(t));
}

// Row count of the mask: an integer add-with-carry per element (the mask
// bit is the carry-in), then the lane sums as exact integer-valued floats.
template <int EPL, int LPR = 64>
__device__ __forceinline__ float rcount(const bool (&m)[EPL]) {
  unsigned c = 0;
#pragma unroll
  for (int e = 0; e < EPL; ++e) c += m[e] ? 1u : 0u;
  return group_sum_f<LPR>((float)c);  // integer-valued, exact
}

// high_order_residual, binary.py:18-39.
// scales (optional): (mu_k, alpha_k) of each pass k at scales[2k], [2k+1].
template <int EPL, int LPR = 64>
__device__ void hor_row(const float (&x)[EPL], const bool (&m)[EPL], int order,
                        float (&acc)[EPL], float* scales = nullptr) {
  const float cnt = rcount<EPL, LPR>(m);
  const float rc = 1.f / fmaxf(cnt, 1.f);
#pragma unroll
  for (int e = 0; e < EPL; ++e) acc[e] = 0.f;
  for (int od = 0; od < order; ++od) {
    float c[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) c[e] = x[e] - acc[e];            // residual
    const float mu = cnt > 0.f ? div_cnt(rsum<EPL, LPR>(c, m), cnt, rc) : 0.f;  // nanmean, NaN->0
#pragma unroll
    for (int e = 0; e < EPL; ++e) c[e] = c[e] - mu;
    const float alpha = cnt > 0.f ? div_cnt(rsum_abs<EPL, LPR>(c, m), cnt, rc) : 0.f;
    if (scales) { scales[2 * od] = mu; scales[2 * od + 1] = alpha; }
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      const float b = __builtin_fmaf(tsign(c[e]), alpha, mu);
      acc[e] = m[e] ? acc[e] + b : 0.f;
    }
  }
}

// The lanes of a row hold the same d, c12, c1w, c2w (row sums end equal on
// every lane of the group), so the two quotients are split over each pair
// of adjacent lanes: the even lane divides n1, the odd lane n2, and a DPP
// swap hands each lane the other's (the same IEEE quotients, one division
// per lane instead of two).
__device__ __forceinline__ void crb_solve(float d, float c12, float c1w, float c2w,
                                          const CrbConsts& k, float& a1, float& a2) {
  // binary.py:1582-1596 (solve_alphas_vec)
  if (k.sym) c12 = c12 * k.omg;
  else c12 = (c12 > 0.f) ? c12 * k.omg : c12;
  const float A = d + k.lam;
  const float den = A * A - c12 * c12;
  const bool ok = fabsf(den) > 1e-12f;
  const float sden = ok ? den : 1.f;
  const float n1 = A * c1w - c12 * c2w;
  const float n2 = A * c2w - c12 * c1w;
  const bool odd = (threadIdx.x & 1) != 0;
  const float q = (odd ? n2 : n1) / sden;
  const float o = __builtin_bit_cast(float, dpp_u32<DPP_XOR1>(__builtin_bit_cast(unsigned, q)));
  a1 = ok ? clamp0(odd ? o : q) : 0.f;
  a2 = ok ? clamp0(odd ? q : o) : 0.f;
}

// coupled_residual_binarization_stable_v7, binary.py:1544-1638.
// Outside the mask cen = 0, so B1 = sign(cen) = 0 there and every
// cen - a*B term is 0 too: those values need no mask, and their sums none
// either (the reference multiplies them by the mask, giving the same zeros).
// Only the signs taken of shifted values (B2 and the refined B1) and the
// output are masked explicitly.
// scales (optional): (mean, mu correction, a1, a2) of the row (binary.py:
// 1599 mean, 1582-1596 a1 / a2, 1633-1635 mu correction); order 1 gives
// (mean, 0, a1, 0).
template <int EPL, int LPR = 64>
__device__ void crb_row(const float (&x)[EPL], const bool (&m)[EPL], int order,
                        const CrbConsts& k, float (&out)[EPL],
                        float* scales = nullptr) {
  const float d = rcount<EPL, LPR>(m);
  const float ds = fmaxf(d, 1.f);
  const float rds = 1.f / ds;
  const float mean = div_cnt(rsum<EPL, LPR>(x, m), ds, rds);
  float cen[EPL], B1[EPL], B2[EPL], t[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) cen[e] = m[e] ? x[e] - mean : 0.f;
#pragma unroll
  for (int e = 0; e < EPL; ++e) B1[e] = tsign(cen[e]);
  float ac[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) ac[e] = fabsf(cen[e]);
  const float sabs = rsum_z<EPL, LPR>(ac);
  if (order == 1) {                                                 // :1570-1576
    const float a1 = div_cnt(sabs, ds, rds);
#pragma unroll
    for (int e = 0; e < EPL; ++e) out[e] = m[e] ? __builtin_fmaf(a1, B1[e], mean) : 0.f;
    if (scales) { scales[0] = mean; scales[1] = 0.f; scales[2] = a1; scales[3] = 0.f; }
    return;
  }
  const float a10 = div_cnt(sabs, ds, rds);                          // step 2
#pragma unroll
  for (int e = 0; e < EPL; ++e) t[e] = __builtin_fmaf(-a10, B1[e], cen[e]);   // step 3
  const float rmean = div_cnt(rsum_z<EPL, LPR>(t), ds, rds);
#pragma unroll
  for (int e = 0; e < EPL; ++e) B2[e] = tsign_m(m[e], t[e] - rmean);
  float c12, c1w, c2w, a1, a2;
  {                                                                 // step 4
    c12 = rdot_sign<EPL, LPR>(B1, B2);
    // cen * B1 = |cen| elementwise (B1 = sign(cen) here): the same sum as a10's
    c1w = sabs;
    c2w = rdot_sign<EPL, LPR>(cen, B2);
  }
  crb_solve(d, c12, c1w, c2w, k, a1, a2);
  if (!k.skip && k.iters > 0) {
    auto round = [&]() {
#pragma unroll
      for (int e = 0; e < EPL; ++e) t[e] = __builtin_fmaf(-a1, B1[e], cen[e]);  // step 5
      const float t5m = div_cnt(rsum_z<EPL, LPR>(t), ds, rds);
#pragma unroll
      for (int e = 0; e < EPL; ++e) B2[e] = tsign_m(m[e], t[e] - t5m);
      c2w = rdot_sign<EPL, LPR>(cen, B2);
      c12 = rdot_sign<EPL, LPR>(B1, B2);
      crb_solve(d, c12, c1w, c2w, k, a1, a2);
#pragma unroll
      for (int e = 0; e < EPL; ++e) t[e] = __builtin_fmaf(-a2, B2[e], cen[e]);  // step 6
      const float t6m = div_cnt(rsum_z<EPL, LPR>(t), ds, rds);
#pragma unroll
      for (int e = 0; e < EPL; ++e) B1[e] = tsign_m(m[e], t[e] - t6m);
      c1w = rdot_sign<EPL, LPR>(cen, B1);
      c12 = rdot_sign<EPL, LPR>(B1, B2);
      crb_solve(d, c12, c1w, c2w, k, a1, a2);
    };
    // the reference's single round (binary.py:1607-1631) straight-line, so
    // its registers need no loop-carried copies; more rounds loop
    round();
    for (int it = 1; it < k.iters; ++it) round();
  }
#pragma unroll
  for (int e = 0; e < EPL; ++e) {                                   // step 7
    const float ap = __builtin_fmaf(a1, B1[e], a2 * B2[e]);
    t[e] = cen[e] - ap;
  }
  const float muc = div_cnt(rsum_z<EPL, LPR>(t), ds, rds);
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    float v = mean + muc;
    v = __builtin_fmaf(a1, B1[e], v);
    v = __builtin_fmaf(a2, B2[e], v);
    out[e] = m[e] ? v : 0.f;
  }
  if (scales) { scales[0] = mean; scales[1] = muc; scales[2] = a1; scales[3] = a2; }
}

// coupled_residual_binarization (CRBOG), binary.py:577-687.
// scales (optional): order 1 as hor_row; order 2 (mean, 0, a1, a2).
template <int EPL, int LPR = 64>
__device__ void crbog_row(const float (&x)[EPL], const bool (&m)[EPL], int order,
                          float (&out)[EPL], float* scales = nullptr) {
  if (order == 1) { hor_row<EPL, LPR>(x, m, 1, out, scales); return; }       // :595-630
  const float n = rcount<EPL, LPR>(m);
#pragma unroll
  for (int e = 0; e < EPL; ++e) out[e] = 0.f;
  if (scales) { scales[0] = 0.f; scales[1] = 0.f; scales[2] = 0.f; scales[3] = 0.f; }
  if (n == 0.f) return;                                             // :647-649
  const float rn = 1.f / n;
  const float mean = div_cnt(rsum<EPL, LPR>(x, m), n, rn);
  float cen[EPL], B1[EPL], B2[EPL], t[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) { cen[e] = x[e] - mean; B1[e] = tsign(cen[e]); }
  float a1 = div_cnt(rsum_abs<EPL, LPR>(cen, m), n, rn);
#pragma unroll
  for (int e = 0; e < EPL; ++e) { t[e] = __builtin_fmaf(-a1, B1[e], cen[e]); B2[e] = tsign(t[e]); }
  float a2 = div_cnt(rsum_abs<EPL, LPR>(t, m), n, rn);
#pragma unroll
  for (int e = 0; e < EPL; ++e) t[e] = B1[e] * B2[e];
  const double c12 = (double)rsum<EPL, LPR>(t, m);
#pragma unroll
  for (int e = 0; e < EPL; ++e) t[e] = cen[e] * B1[e];
  const double c1w = (double)rsum<EPL, LPR>(t, m);
#pragma unroll
  for (int e = 0; e < EPL; ++e) t[e] = cen[e] * B2[e];
  const double c2w = (double)rsum<EPL, LPR>(t, m);
  const double dn = (double)n;
  const double det = dn * dn - c12 * c12;
  if (fabs(det) > 1e-12) {
    double n1 = (c1w * dn - c2w * c12) / det;
    double n2 = (c2w * dn - c1w * c12) / det;
    a1 = (float)((0.0 > n1) ? 0.0 : n1);                            // python max(x, 0.0)
    a2 = (float)((0.0 > n2) ? 0.0 : n2);
  }
  if (scales) { scales[0] = mean; scales[2] = a1; scales[3] = a2; }
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    float v = __builtin_fmaf(a1, B1[e], mean);
    v = __builtin_fmaf(a2, B2[e], v);
    out[e] = m[e] ? v : 0.f;
  }
}

// Method families of Binarization.quantize (binary.py:2874-2890): kernels
// are instantiated per family so each carries only its own registers.
enum { MF_BRAQ = 0, MF_CRB = 1, MF_CRBOG = 2 };
__host__ __device__ inline int method_family(int method) {
  return method == CRBQ_BRAQ ? MF_BRAQ : (method == CRBQ_CRBOG ? MF_CRBOG : MF_CRB);
}

// Binarization.quantize dispatch, binary.py:2874-2890, within a family.
// scales (optional): the per-row scales as hor_row / crb_row / crbog_row
// write them.
template <int MF, int EPL, int LPR = 64>
__device__ __forceinline__ void binarize_row(int method, const float (&x)[EPL],
                                             const bool (&m)[EPL], int order,
                                             const CrbConsts& base, float (&out)[EPL],
                                             float* scales = nullptr) {
  if (MF == MF_BRAQ) {
    hor_row<EPL, LPR>(x, m, order, out, scales);
  } else if (MF == MF_CRBOG) {
    crbog_row<EPL, LPR>(x, m, order, out, scales);
  } else {
    CrbConsts k = base;
    k.skip = (method == CRBQ_CRB_NOREFINE || method == CRBQ_CRB_SYMDAMP_NOREFINE);
    k.sym = (method == CRBQ_CRB_SYMDAMP || method == CRBQ_CRB_SYMDAMP_NOREFINE);
    crb_row<EPL, LPR>(x, m, order, k, out, scales);
  }
}

}  // namespace crbq
