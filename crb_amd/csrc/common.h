// Shared device/host helpers of the crbq library (gfx950 only).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/crbq.h"

#define CRBQ_WAVE 64

#define CRBQ_HIP(expr)                                   \
  do {                                                   \
    hipError_t e_ = (expr);                              \
    if (e_ != hipSuccess) return CRBQ_ERR_HIP;           \
  } while (0)

#define CRBQ_LAUNCH_CHECK() CRBQ_HIP(hipGetLastError())

typedef float f4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef __bf16 b8_t __attribute__((ext_vector_type(8)));

namespace crbq {

// torch.sign: (0 < x) - (x < 0); +-0 and NaN give 0.  |x| > 0 is false
// exactly for +-0 and NaN, and copysign gives +-1 otherwise.
__device__ __forceinline__ float tsign(float x) {
  return fabsf(x) > 0.f ? __builtin_copysignf(1.f, x) : 0.f;
}
// tsign(x) inside a mask, 0 outside
__device__ __forceinline__ float tsign_m(bool m, float x) {
  return (m && fabsf(x) > 0.f) ? __builtin_copysignf(1.f, x) : 0.f;
}

// torch.clamp(x, min=0): NaN propagates.
__device__ __forceinline__ float clamp0(float x) { return x < 0.f ? 0.f : x; }

// Sum over the 64 lanes of a wavefront without the LDS crossbar: DPP
// quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror and row_mirror
// within each 16-lane row, then v_permlane16_swap (rows 0<->1, 2<->3) and
// v_permlane32_swap (lanes 0-31 <-> 32-63).  Every lane ends with the
// bitwise-same value: a DPP level adds commuted operand pairs (lane i adds
// v_j, lane j adds v_i, with all lanes of the partner group already equal),
// and a swap level returns (lower-group value, upper-group value) in the
// same order to both lanes of a pair.
// bound_ctrl set: a lane whose source lies outside its row (row_shl /
// row_shr) reads 0, the same value the old operand 0 gave it, and no zero
// has to be moved into the destination first.
template <int CTRL>
__device__ __forceinline__ unsigned dpp_u32(unsigned v) {
  return (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, true);
}
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140;

// v_permlane16_swap_b32 / v_permlane32_swap_b32 on the pair (a, b) (a is
// VDST, b is SRC0): after the swap, with a = b = v on entry, every lane holds
// in a the value of the lower lane group of its pair (rows 0/2 for 16, lanes
// 0-31 for 32) and in b the value of the upper group.  Issued as inline
// assembly: the compiler's optimizer folds the builtins' second result into
// the first when they are used as floats, which is wrong across lanes.  The
// s_nop guards cover the VALU-write -> permlane-read hazard and a DPP read
// of the results, which the hazard recognizer does not see inside asm.
__device__ __forceinline__ void permlane16_swap(unsigned& a, unsigned& b) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void permlane32_swap(unsigned& a, unsigned& b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}

template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
  const unsigned lo = dpp_u32<CTRL>((unsigned)b), hi = dpp_u32<CTRL>((unsigned)(b >> 32));
  return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}
// (value of the lower lane group, value of the upper group) of a pair
template <bool W32>
__device__ __forceinline__ void swap_f64(double v, double& a, double& b) {
  const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
  unsigned la = (unsigned)u, lb = (unsigned)u, ha = (unsigned)(u >> 32), hb = ha;
  if (W32) { permlane32_swap(la, lb); permlane32_swap(ha, hb); }
  else { permlane16_swap(la, lb); permlane16_swap(ha, hb); }
  a = __builtin_bit_cast(double, ((unsigned long long)ha << 32) | la);
  b = __builtin_bit_cast(double, ((unsigned long long)hb << 32) | lb);
}
__device__ __forceinline__ void swap16_f64(double v, double& a, double& b) {
  swap_f64<false>(v, a, b);
}
__device__ __forceinline__ void swap32_f64(double v, double& a, double& b) {
  swap_f64<true>(v, a, b);
}

// Sum over aligned groups of LPR lanes (2, 4, 8, 16, 32 or 64): the first
// log2(LPR) levels of the sequence above.
template <int LPR>
__device__ __forceinline__ double group_sum(double v) {
  static_assert(LPR == 2 || LPR == 4 || LPR == 8 || LPR == 16 || LPR == 32 || LPR == 64, "LPR");
  v = v + dpp_f64<DPP_XOR1>(v);
  if (LPR == 2) return v;
  v = v + dpp_f64<DPP_XOR2>(v);
  if (LPR == 4) return v;
  v = v + dpp_f64<DPP_HALF_MIRROR>(v);
  if (LPR == 8) return v;
  v = v + dpp_f64<DPP_MIRROR>(v);
  if (LPR == 16) return v;
  double a, b;
  swap16_f64(v, a, b);
  v = a + b;
  if (LPR == 32) return v;
  swap32_f64(v, a, b);
  return a + b;
}
template <int LPR>
__device__ __forceinline__ float group_sum_f(float v) {
  static_assert(LPR == 2 || LPR == 4 || LPR == 8 || LPR == 16 || LPR == 32 || LPR == 64, "LPR");
  auto f = [](unsigned u) { return __builtin_bit_cast(float, u); };
  auto u = [](float x) { return __builtin_bit_cast(unsigned, x); };
  v = v + f(dpp_u32<DPP_XOR1>(u(v)));
  if (LPR == 2) return v;
  v = v + f(dpp_u32<DPP_XOR2>(u(v)));
  if (LPR == 4) return v;
  v = v + f(dpp_u32<DPP_HALF_MIRROR>(u(v)));
  if (LPR == 8) return v;
  v = v + f(dpp_u32<DPP_MIRROR>(u(v)));
  if (LPR == 16) return v;
  unsigned a = u(v), b = a;
  permlane16_swap(a, b);
  v = f(a) + f(b);
  if (LPR == 32) return v;
  a = u(v);
  b = a;
  permlane32_swap(a, b);
  return f(a) + f(b);
}
__device__ __forceinline__ double wave_sum(double v) { return group_sum<64>(v); }
__device__ __forceinline__ float wave_sum_f(float v) { return group_sum_f<64>(v); }

// Align a workspace carve-out to 256 bytes.
struct WsCarver {
  char* base;
  size_t off;
  size_t cap;
  explicit WsCarver(void* b, size_t c) : base((char*)b), off(0), cap(c) {}
  template <typename T>
  T* take(size_t n) {
    off = (off + 255) & ~(size_t)255;
    T* p = (T*)(base ? base + off : nullptr);
    off += n * sizeof(T);
    return p;
  }
  bool ok() const { return base != nullptr && off <= cap; }
};

}  // namespace crbq
