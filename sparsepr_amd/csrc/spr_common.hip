// Error state shared by every entry point of libsparsepr_hip.so.
#include <stdarg.h>
#include <stdio.h>

#include "spr_common.h"

static thread_local char g_last_error[1024] = "";

void spr_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

extern "C" const char* spr_last_error(void) { return g_last_error; }

extern "C" int spr_abi_version(void) { return 2; }
