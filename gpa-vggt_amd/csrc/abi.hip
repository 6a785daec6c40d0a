// Library-wide C ABI pieces: version query and the per-thread error message.
#include <stdarg.h>
#include <stdio.h>

#include "gpa_common.h"

namespace {
thread_local char g_last_error[512] = "";
}

void gpa_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void gpa_clear_error() { g_last_error[0] = '\0'; }

extern "C" int gpa_abi_version(void) { return GPA_ABI_VERSION; }

extern "C" const char* gpa_last_error(void) { return g_last_error; }
