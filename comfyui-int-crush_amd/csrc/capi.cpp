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

// Compute units of the current device (cached per device id).
int ic_num_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  if (dev < 64 && cache[dev] > 0) return cache[dev];
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
  if (dev < 64) cache[dev] = n;
  return n;
}

// Dynamic-LDS limit of a kernel, set once per device: done[] holds one flag
// per device id (hipFuncSetAttribute applies to the current device).
hipError_t ic_set_lds_limit(const void* kern, int bytes, unsigned char* done) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev >= 0 && dev < 64 && done[dev]) return hipSuccess;
  e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess && dev >= 0 && dev < 64) done[dev] = 1;  // idempotent; a race only repeats the call
  return e;
}

extern "C" {
const char* ic_version(void) { return "intcrush-gfx950 0.1.0"; }
const char* ic_last_error(void) { return g_err; }
}
