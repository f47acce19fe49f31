// Error reporting, version, launch tags and device queries for the C ABI.
#include <stdarg.h>
#include <stdio.h>
#include <unistd.h>

#include <atomic>
#include <chrono>

#include "s8kv_host.h"

namespace s8kv {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

// A fresh 40-bit launch tag (never zero): a per-process sequence, seeded from
// the clock and the process id, through the splitmix64 finaliser.
unsigned long long next_launch_tag() {
  static std::atomic<unsigned long long> seq{0};
  static const unsigned long long seed =
      (unsigned long long)std::chrono::steady_clock::now().time_since_epoch().count() * 0x9E3779B97F4A7C15ull ^
      ((unsigned long long)getpid() << 32);
  for (;;) {
    unsigned long long z = seed + 0x9E3779B97F4A7C15ull * (seq.fetch_add(1) + 1);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    z &= (1ull << 40) - 1;
    if (z != 0) return z;
  }
}

// Compute units of the current device (cached per device id).
int device_cus() {
  constexpr int kMaxDevices = 64;
  static int cached[kMaxDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  if (dev >= 0 && dev < kMaxDevices && cached[dev] > 0) return cached[dev];
  int cus = 256;
  int v = 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0) cus = v;
  if (dev >= 0 && dev < kMaxDevices) cached[dev] = cus;
  return cus;
}

}  // namespace s8kv

extern "C" int s8kv_version(void) { return 100; }

extern "C" const char* s8kv_last_error(void) { return s8kv::g_err; }
