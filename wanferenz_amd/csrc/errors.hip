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

namespace wz {
// Compute units of the current device (cached per device; 256 on MI355X).
int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}
}  // namespace wz

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
