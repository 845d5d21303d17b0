// C-ABI housekeeping: version, last-error string.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace cortex {
static thread_local char g_err[512] = {0};
void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}
}  // namespace cortex

extern "C" {
int cortex_version(void) { return 1; }
const char* cortex_last_error(void) { return cortex::g_err; }
}
