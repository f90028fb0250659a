// C ABI housekeeping: version and the thread-local last-error message.

#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace ss {

static thread_local char g_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

}  // namespace ss

extern "C" int ss_abi_version(void) { return SS_ABI_VERSION; }

extern "C" const char* ss_last_error(void) { return ss::g_error; }
