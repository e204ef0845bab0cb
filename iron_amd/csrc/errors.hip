// Error reporting for the C ABI: every entry point returns 0 or an error code
// and leaves a message retrievable with iron_last_error() on the calling thread.
#include <stdarg.h>
#include <stdio.h>

#include "iron_common.hpp"
#include "../../include/iron_hip.h"

namespace iron {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int fail_einval(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return IRON_EINVAL;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return static_cast<int>(e);
  }
  return 0;
}

}  // namespace iron

extern "C" const char* iron_last_error(void) { return iron::g_last_error; }

extern "C" int iron_abi_version(void) { return IRON_HIP_ABI_VERSION; }
