// Thread-local error message + launch checking for the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace {
thread_local char g_err[512] = "";
}

namespace wz {

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(WZ_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return WZ_OK;
}

}  // namespace wz

extern "C" const char* wz_last_error(void) { return g_err; }

extern "C" int wz_device_info(int* cu_count, int* xcd_count) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return wz::set_error(WZ_EINVAL, "wz_device_info: no device");
  hipDeviceProp_t p;
  if (hipGetDeviceProperties(&p, dev) != hipSuccess)
    return wz::set_error(WZ_EINVAL, "wz_device_info: hipGetDeviceProperties failed");
  if (cu_count) *cu_count = p.multiProcessorCount;
  if (xcd_count) *xcd_count = 8;
  return WZ_OK;
}
