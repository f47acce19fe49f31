// Error reporting and version for the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "s8kv_host.h"

namespace s8kv {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

}  // namespace s8kv

extern "C" int s8kv_version(void) { return 100; }

extern "C" const char* s8kv_last_error(void) { return s8kv::g_err; }
