// Error reporting shared by every kx355 entry point.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace {
thread_local char g_error[512] = "";
}

namespace kx {

int set_error(int code, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, args);
  va_end(args);
  return code;
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return set_error(KX_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(err));
  }
  return KX_OK;
}

}  // namespace kx

extern "C" int kx_abi_version(void) { return 1; }

extern "C" const char* kx_last_error(void) { return g_error; }
