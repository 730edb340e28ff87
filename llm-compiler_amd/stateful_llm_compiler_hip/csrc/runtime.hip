// Host-side plumbing shared by every entry point: error text and launch checks.
#include <stdarg.h>
#include <stdio.h>

#include "common.hpp"

namespace {
thread_local char g_last_error[512] = "";
thread_local hipEvent_t g_begin = nullptr;
thread_local hipEvent_t g_end = nullptr;
thread_local int g_repeats = 1;
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

int device_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  if (dev < 64 && cached[dev] > 0) return cached[dev];
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    n = 256;
  if (dev < 64) cached[dev] = n;
  return n;
}

void mark_kernel_begin(hipStream_t stream) {
  if (g_begin != nullptr) hipEventRecord(g_begin, stream);
}

void mark_kernel_end(hipStream_t stream) {
  if (g_end != nullptr) hipEventRecord(g_end, stream);
}

int timed_repeats() { return g_begin != nullptr ? g_repeats : 1; }

}  // namespace slc_host

extern "C" int slc_hip_version(void) { return 200; }

extern "C" const char* slc_hip_last_error(void) { return g_last_error; }

extern "C" void slc_hip_set_timing_events(void* begin, void* end) {
  g_begin = static_cast<hipEvent_t>(begin);
  g_end = static_cast<hipEvent_t>(end);
}

extern "C" void slc_hip_set_timing_repeats(int repeats) { g_repeats = repeats > 1 ? repeats : 1; }
