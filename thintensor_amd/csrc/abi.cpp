// Library-wide C ABI helpers: version and per-thread error messages.
#include <stdarg.h>
#include <stdio.h>

#include "../../include/thintensor_hip.h"

namespace tt {

static thread_local char g_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

}  // namespace tt

extern "C" int tt_version(void) { return 1; }

extern "C" const char* tt_last_error(void) { return tt::g_error; }
