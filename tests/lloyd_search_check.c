/*
 * Check of the three-test codeword search (lloyd3_search and its codebook
 * condition lloyd3_search_ok in superl8_serve_amd/csrc/s8kv_device.h) and of
 * its threshold form (the append kernel's compares against T_j, found by
 * lloyd3_threshold's bisection in superl8_serve_amd/csrc/s8kv_append.hip)
 * against the sequential scan they replace: code = first index j minimising
 * fl|u - c_j| (strict "<" while scanning j = 0 .. 7).
 *
 * Usage: lloyd_search_check c0 c1 ... c7 [lower]   (the codebook, as C float
 * literals; "lower" moves T_4 one fp32 step down, a planted mistake the check
 * must report)
 * For a codebook that meets the condition, every fp32 u in [-1, 1] (both
 * signs, 2.1e9 values) and NaN are checked with both forms; otherwise the
 * program reports "rejected" and exits 2.  Prints the thresholds, then
 * "values N mismatches K" (K counts values where either form differs).
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

/* ordered key of an fp32 bit pattern (its own inverse) */
static int32_t key(int32_t bits) { return bits ^ ((bits >> 31) & 0x7FFFFFFF); }
static int32_t f2i(float f) { int32_t i; memcpy(&i, &f, 4); return i; }
static float i2f(int32_t i) { float f; memcpy(&f, &i, 4); return f; }

/* least fp32 u with fl|u - b| < fl|u - a| on [a, b], by bisection over keys */
static float threshold(float a, float b) {
  int32_t lo = key(f2i(a)), hi = key(f2i(b));
  for (int it = 0; it < 32; ++it) {
    const uint32_t d = (uint32_t)hi - (uint32_t)lo;
    if (d <= 1u) break;
    const int32_t mid = (int32_t)((uint32_t)lo + (d >> 1));
    const float u = i2f(key(mid));
    if (fabsf(u - b) < fabsf(u - a)) hi = mid;
    else lo = mid;
  }
  return i2f(key(hi));
}

static float thr[8];

static int thr_search(float u) {
  const int b2 = u >= thr[4];
  const int b1 = u >= (b2 ? thr[6] : thr[2]);
  const float t_hi = b2 ? thr[7] : thr[3], t_lo = b2 ? thr[5] : thr[1];
  const int b0 = u >= (b1 ? t_hi : t_lo);
  return 4 * b2 + 2 * b1 + b0;
}

int main(int argc, char** argv) {
  if (argc != 9 && !(argc == 10 && strcmp(argv[9], "lower") == 0)) {
    fprintf(stderr, "usage: %s c0 .. c7 [lower]\n", argv[0]);
    return 64;
  }
  for (int j = 0; j < 8; ++j) cb[j] = strtof(argv[j + 1], NULL);
  if (!search_ok()) {
    printf("rejected\n");
    return 2;
  }
  for (int j = 1; j < 8; ++j) thr[j] = threshold(cb[j - 1], cb[j]);
  if (argc == 10) thr[4] = i2f(key(key(f2i(thr[4])) - 1));
  printf("thresholds");
  for (int j = 1; j < 8; ++j) printf(" %a", thr[j]);
  printf("\n");
  long long values = 0, bad = 0;
  const int64_t top = 0x3F800000;  /* 1.0f */
#pragma omp parallel for schedule(static) reduction(+ : values, bad)
  for (int64_t b = 0; b <= top; ++b) {
    for (int neg = 0; neg < 2; ++neg) {
      const uint32_t bits = (uint32_t)b | (neg ? 0x80000000u : 0u);
      float u;
      memcpy(&u, &bits, 4);
      ++values;
      const int c = scan(u);
      if (search(u) != c || thr_search(u) != c) ++bad;
    }
  }
  const float nan = nanf("");
  ++values;
  bad += search(nan) != scan(nan) || thr_search(nan) != scan(nan);
  printf("values %lld mismatches %lld\n", values, bad);
  return bad != 0;
}
