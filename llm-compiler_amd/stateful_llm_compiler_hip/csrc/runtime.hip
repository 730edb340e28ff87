// Host-side plumbing shared by every entry point: error text and launch checks.
#include <stdarg.h>
#include <stdio.h>

#include "common.hpp"

namespace {
thread_local char g_last_error[512] = "";
}

namespace slc_host {

void set_error(const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, args);
  va_end(args);
}

int check_launch(const char* what) {
  hipError_t status = hipGetLastError();
  if (status != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(status));
    return static_cast<int>(status);
  }
  g_last_error[0] = '\0';
  return SLC_OK;
}

}  // namespace slc_host

extern "C" int slc_hip_version(void) { return 100; }

extern "C" const char* slc_hip_last_error(void) { return g_last_error; }
