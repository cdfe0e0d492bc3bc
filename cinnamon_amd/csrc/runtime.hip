// C-ABI bookkeeping: version and per-thread error messages.
#include <stdarg.h>
#include <stdio.h>

#include "cin_runtime.h"

namespace {
thread_local char g_err[512] = "";
}

int cin_set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int cin_check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return cin_set_error(CIN_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return CIN_OK;
}

extern "C" {

int cin_abi_version(void) { return 3; }

const char* cin_last_error(void) { return g_err; }

}  // extern "C"
