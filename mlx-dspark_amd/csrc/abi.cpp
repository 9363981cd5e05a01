// ABI-level helpers: the per-thread error message and the version number.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace dsk {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

}  // namespace dsk

extern "C" const char* dsk_last_error(void) { return dsk::g_err; }

extern "C" int dsk_abi_version(void) { return 1; }
