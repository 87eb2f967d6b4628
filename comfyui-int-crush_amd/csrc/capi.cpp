// Library identification, thread-local error reporting and launch checking.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/intcrush.h"

static thread_local char g_err[512] = "";

int ic_set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int ic_check_launch(const char* who) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return ic_set_error(IC_ERR_LAUNCH, "%s: %s", who, hipGetErrorString(e));
  return IC_OK;
}

extern "C" {
const char* ic_version(void) { return "intcrush-gfx950 0.1.0"; }
const char* ic_last_error(void) { return g_err; }
}
