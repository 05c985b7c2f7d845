// Status plumbing for the C ABI: per-thread last-error message and launch checks.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "common.hpp"

namespace {
thread_local char g_last_error[512] = "";
}

namespace sfl {

int set_error(int code, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, args);
  va_end(args);
  return code;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return set_error(SFL_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(err));
  }
  return SFL_OK;
}

}  // namespace sfl

extern "C" const char* sfl_version(void) { return "sfl 0.1 gfx950"; }

extern "C" const char* sfl_last_error(void) { return g_last_error; }
