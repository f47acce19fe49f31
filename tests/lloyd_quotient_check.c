/*
 * Check of the K8V3 append's reciprocal-based quotient u = v / norm
 * (rows_lloydmax3_store in superl8_serve_amd/csrc/s8kv_append.hip): with
 * rn = 1 / norm (IEEE fp32), q0 = v * rn, r = fma(-q0, norm, v) and
 * u = fma(r, rn, q0), u must equal the IEEE quotient v / norm.
 *
 * v is an fp16 value and norm a positive fp32 >= |v| (at most
 * sqrt(128) * 65504).  Every step scales exactly with powers of two of v and
 * of norm while no value leaves the normal range, which holds there (the
 * smallest nonzero |v| is 2^-24, so q0, r and u stay far above 2^-126), and
 * negating v negates every step.  So the pairs with v one of the 1024 fp16
 * significands in [1, 2) and norm any of the 2^23 fp32 significands in
 * [1, 2) stand for all of them: 8.6e9 pairs, every one checked.  A second
 * pass draws 2^26 pairs over the whole domain (every fp16 v, subnormals and
 * signs included, norm from |v| up to 2^20) as a check of that reduction.
 * Prints "pairs N mismatches K".  Build with -O2 -mfma -ffp-contract=off
 * (and -fopenmp to spread the first pass over threads).
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float bits_to_float(uint32_t b) {
  float f;
  memcpy(&f, &b, 4);
  return f;
}

static float half_to_float(uint16_t h) {
  const uint32_t e = (h >> 10) & 31, m = h & 1023;
  const float v = e == 0 ? ldexpf((float)m, -24) : ldexpf((float)(m | 1024), (int)e - 25);
  return (h >> 15) ? -v : v;
}

static int quotient_ok(float v, float norm) {
  const float rn = 1.0f / norm;
  const float q0 = v * rn;
  const float r = fmaf(-q0, norm, v);
  const float u = fmaf(r, rn, q0);
  return u == v / norm;
}

int main(void) {
  long long pairs = 0, bad = 0;
#pragma omp parallel for schedule(dynamic) reduction(+ : pairs, bad)
  for (int vm = 0; vm < 1024; ++vm) {
    const float v = bits_to_float(0x3F800000u | ((uint32_t)vm << 13));  /* fp16 significand 1.vm */
    long long bad_v = 0;
    for (uint32_t nm = 0; nm < (1u << 23); ++nm) bad_v += !quotient_ok(v, bits_to_float(0x3F800000u | nm));
    pairs += 1ll << 23;
    bad += bad_v;
  }
  /* whole-domain sample: xorshift64 */
  uint64_t st = 0x9E3779B97F4A7C15ull;
  for (long long i = 0; i < (1ll << 26); ++i) {
    st ^= st << 13;
    st ^= st >> 7;
    st ^= st << 17;
    const uint16_t h = (uint16_t)(st & 0x7FFF);
    if (h == 0 || h >= 0x7C00) continue;  /* nonzero finite fp16 magnitudes */
    float v = half_to_float(h);
    if (st & 0x8000) v = -v;
    /* norm = |v| * 2^k * (1 + f), k in [0, 20], f a random significand */
    const float norm = ldexpf(fabsf(v), (int)((st >> 16) % 21)) * bits_to_float(0x3F800000u | (uint32_t)((st >> 40) & 0x7FFFFF));
    if (!(norm >= fabsf(v)) || isinf(norm)) continue;
    ++pairs;
    bad += !quotient_ok(v, norm);
  }
  printf("pairs %lld mismatches %lld\n", pairs, bad);
  return bad != 0;
}
