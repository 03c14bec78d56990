// Error plumbing, version and per-device facts shared by every entry point.
#include <stdarg.h>
#include <stdio.h>

#include "common.hpp"

static thread_local char g_last_error[1024] = "";

int rh_set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int rh_check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return rh_set_error(RH_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return RH_OK;
}

// Compute-unit count of the current device (cached for up to 16 devices).
int rh_device_cus() {
  static int cached[16] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  if (dev < 16 && cached[dev]) return cached[dev];
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  if (dev < 16) cached[dev] = cus;
  return cus;
}

extern "C" int rh_version(void) { return 100; }

extern "C" const char* rh_last_error(void) { return g_last_error; }
