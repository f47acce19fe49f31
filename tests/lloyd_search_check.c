/*
 * Check of the three-test codeword search (lloyd3_search and its codebook
 * condition lloyd3_search_ok in superl8_serve_amd/csrc/s8kv_device.h) against
 * the sequential scan it replaces: code = first index j minimising
 * fl|u - c_j| (strict "<" while scanning j = 0 .. 7).
 *
 * Usage: lloyd_search_check c0 c1 ... c7   (the codebook, as C float literals)
 * For a codebook that meets the condition, every fp32 u in [-1, 1] (both
 * signs, 2.1e9 values) and NaN are checked; otherwise the program reports
 * "rejected" and exits 2.  Prints "values N mismatches K".
 * Build with -O2 -ffp-contract=off (and -fopenmp to use threads).
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float cb[8];

static int search_ok(void) {
  int ok = cb[0] >= -4.0f && cb[7] <= 4.0f;
  for (int j = 1; j < 8; ++j) ok = ok && (cb[j] - cb[j - 1] >= 0x1p-19f);
  return ok;
}

static int scan(float u) {
  float best = fabsf(u - cb[0]);
  int c = 0;
  for (int j = 1; j < 8; ++j) {
    const float d = fabsf(u - cb[j]);
    if (d < best) {
      best = d;
      c = j;
    }
  }
  return c;
}

static int search(float u) {
  const int b2 = fabsf(u - cb[4]) < fabsf(u - cb[3]);
  const float c62 = b2 ? cb[6] : cb[2], c51 = b2 ? cb[5] : cb[1];
  const float c73 = b2 ? cb[7] : cb[3], c40 = b2 ? cb[4] : cb[0];
  const int b1 = fabsf(u - c62) < fabsf(u - c51);
  const float hi = b1 ? c73 : c51, lo = b1 ? c62 : c40;
  const int b0 = fabsf(u - hi) < fabsf(u - lo);
  return 4 * b2 + 2 * b1 + b0;
}

int main(int argc, char** argv) {
  if (argc != 9) {
    fprintf(stderr, "usage: %s c0 .. c7\n", argv[0]);
    return 64;
  }
  for (int j = 0; j < 8; ++j) cb[j] = strtof(argv[j + 1], NULL);
  if (!search_ok()) {
    printf("rejected\n");
    return 2;
  }
  long long values = 0, bad = 0;
  const int64_t top = 0x3F800000;  /* 1.0f */
#pragma omp parallel for schedule(static) reduction(+ : values, bad)
  for (int64_t b = 0; b <= top; ++b) {
    for (int neg = 0; neg < 2; ++neg) {
      const uint32_t bits = (uint32_t)b | (neg ? 0x80000000u : 0u);
      float u;
      memcpy(&u, &bits, 4);
      ++values;
      if (search(u) != scan(u)) ++bad;
    }
  }
  const float nan = nanf("");
  ++values;
  bad += search(nan) != scan(nan);
  printf("values %lld mismatches %lld\n", values, bad);
  return bad != 0;
}
