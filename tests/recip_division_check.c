/*
 * Exhaustive check of the append kernel's reciprocal-based quotient
 * (rtn_i8_recip in superl8_serve_amd/csrc/s8kv_device.h) on its whole input
 * domain: for every fp16 absmax m > 0 and every fp16 y with |y| <= m (both
 * signs), with s = m / 127 and rs = 1 / s (IEEE fp32), q0 = y * rs,
 * r = fma(-q0, s, y), q1 = fma(r, rs, q0): q1 must equal the IEEE quotient
 * y / s, and the kernel's rounding of it -- the encoding of q1 + 1.5 * 2^23
 * minus 0x4B400000, with no clamp -- must equal rint(y / s) clamped to
 * [-127, 127].  Prints "pairs N mismatches K".  Build with -ffp-contract=off.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float half_to_float(uint16_t h) {
  const uint32_t e = (h >> 10) & 31, m = h & 1023;
  const float v = e == 0 ? ldexpf((float)m, -24) : ldexpf((float)(m | 1024), (int)e - 25);
  return (h >> 15) ? -v : v;
}

int main(void) {
  static float vals[0x7C00];
  for (uint32_t h = 0; h < 0x7C00; ++h) vals[h] = half_to_float((uint16_t)h);  /* finite, >= 0, ascending */
  long long pairs = 0, bad = 0;
  for (int mi = 1; mi < 0x7C00; ++mi) {
    volatile float s = vals[mi] / 127.0f;
    volatile float rs = 1.0f / s;
    for (int yi = 0; yi <= mi; ++yi) {
      for (int neg = 0; neg < 2; ++neg) {
        const float y = neg ? -vals[yi] : vals[yi];
        volatile float exact = y / s;
        volatile float q0 = y * rs;
        const float r = fmaf(-q0, s, y);
        const float q1 = fmaf(r, rs, q0);
        volatile float biased = q1 + 12582912.0f;
        const float fb = biased;
        uint32_t bits;
        memcpy(&bits, &fb, 4);
        const int code = (int)(bits - 0x4B400000u);
        const float ref = fminf(127.0f, fmaxf(-127.0f, rintf(exact)));
        ++pairs;
        if (q1 != exact || code != (int)ref) {
          if (bad < 3) printf("mismatch: m=%a y=%a y/s=%a q1=%a\n", vals[mi], y, exact, q1);
          ++bad;
        }
      }
    }
  }
  printf("pairs %lld mismatches %lld\n", pairs, bad);
  return bad != 0;
}
