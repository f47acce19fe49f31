// Host-side helpers for the C ABI: per-thread error text and argument checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/superl8_kv.h"

namespace s8kv {

void set_error(const char* fmt, ...);

// A fresh 40-bit launch tag (never zero) for arrival counters.
unsigned long long next_launch_tag();

// Compute units of the current device (cached per device id).
int device_cus();

inline bool is_pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }

inline int log2i(int64_t x) {
  int r = 0;
  while ((int64_t(1) << r) < x) ++r;
  return r;
}

inline bool head_dim_ok(int d) { return d == 32 || d == 64 || d == 128 || d == 256; }

// Bytes of a per-layer cache tensor must fit the 32-bit buffer-descriptor range.
inline bool fits_u32(int64_t bytes) { return bytes >= 0 && bytes < (int64_t(1) << 32); }
// A byte count as a buffer descriptor's 32-bit size (4 GiB - 1 at most).
inline uint32_t cap_u32(uint64_t n) { return (uint32_t)(n < 0xFFFFFFFFull ? n : 0xFFFFFFFFull); }

inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return S8KV_ERR_LAUNCH;
  }
  return S8KV_OK;
}

}  // namespace s8kv

#define S8KV_REQUIRE(cond, code, ...)     \
  do {                                    \
    if (!(cond)) {                        \
      ::s8kv::set_error(__VA_ARGS__);     \
      return (code);                      \
    }                                     \
  } while (0)
