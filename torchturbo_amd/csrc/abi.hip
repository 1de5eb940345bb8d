// Library-wide ABI helpers: version, per-thread error message, launch check.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace {
thread_local char g_last_error[512] = "";
}

void tt_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int tt_check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    tt_set_error("%s: %s", what, hipGetErrorString(err));
    return TT_ERR_HIP;
  }
  return TT_OK;
}

extern "C" int tt_abi_version(void) { return 1; }

extern "C" const char* tt_last_error(void) { return g_last_error; }
