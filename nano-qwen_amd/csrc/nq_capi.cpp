// Library-wide C-ABI pieces: version and thread-local error text.
#include <stdarg.h>
#include <stdio.h>

#include "nq_internal.hpp"

static thread_local char g_err[512] = "";

void nq_clear_error() { g_err[0] = '\0'; }

int nq_fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int nq_check_launch(hipError_t e) {
  if (e == hipSuccess) return NQ_OK;
  snprintf(g_err, sizeof(g_err), "kernel launch failed: %s", hipGetErrorString(e));
  return -static_cast<int>(e);
}

extern "C" int nq_version(void) { return 100; }

extern "C" const char* nq_last_error(void) { return g_err; }
