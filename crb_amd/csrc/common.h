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

// torch.sign: (0 < x) - (x < 0); +-0 and NaN give 0.
__device__ __forceinline__ float tsign(float x) {
  return (float)((0.f < x) - (x < 0.f));
}

// torch.clamp(x, min=0): NaN propagates.
__device__ __forceinline__ float clamp0(float x) { return x < 0.f ? 0.f : x; }

// Butterfly sum over the 64 lanes of a wavefront.  Every lane ends with the
// bitwise-same value (each level adds two commuted operands).
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, CRBQ_WAVE);
  return v;
}
__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, CRBQ_WAVE);
  return v;
}

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
