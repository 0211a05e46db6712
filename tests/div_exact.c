// Division by a count through its reciprocal plus one fma correction:
// q0 = x * r, q1 = fma(fma(-q0, d, x), r, q0) with r = 1 / d (IEEE), for
// every fp32 significand x in [1, 2) and every integer d in 1..1024, against
// the IEEE quotient x / d (scaling x by a power of two scales every step
// exactly, so this covers all normal x).  Prints "bad N of M".
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

int main(void) {
  long bad = 0, tot = 0;
  for (int d = 1; d <= 1024; ++d) {
    volatile float df = (float)d;
    const float r = 1.0f / df;
    for (uint32_t m = 0; m < (1u << 23); ++m) {
      const uint32_t u = 0x3f800000u | m;
      float x;
      memcpy(&x, &u, 4);
      const float q0 = x * r;
      const float e = fmaf(-q0, df, x);
      const float q1 = fmaf(e, r, q0);
      ++tot;
      if (q1 != x / df) ++bad;
    }
  }
  printf("bad %ld of %ld\n", bad, tot);
  return 0;
}
