// Error reporting and identification for the libtmhd C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "tmhd_internal.h"

namespace tmhd {

namespace {
thread_local char g_last_error[512] = "";
}

int set_error(int status, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

int device_cus() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cus[dev] = n;
  }
  return cus[dev];
}

int check_launch(const char *what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(TMHD_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return TMHD_OK;
}

}  // namespace tmhd

extern "C" const char *tmhd_version(void) { return "tmhd 0.1.0 gfx950"; }

extern "C" const char *tmhd_last_error(void) { return tmhd::g_last_error; }
