// Library-wide entry points of libsaeflow_hip.so: ABI version and the thread-local error text.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace {
thread_local char g_err[512] = "";
}

int sf_fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return status;
}

void sf_clear_error() { g_err[0] = '\0'; }

extern "C" int sf_abi_version(void) { return SF_ABI_VERSION; }

extern "C" const char* sf_last_error(void) { return g_err; }
