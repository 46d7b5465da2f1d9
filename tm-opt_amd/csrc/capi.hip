// Library-wide C-ABI plumbing: thread-local error text, version string and
// the compute-unit count of the current device.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace tmopt {

static thread_local char g_err[1024];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

void clear_error() { g_err[0] = '\0'; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return TMOPT_ELAUNCH;
  }
  return TMOPT_OK;
}

int device_cus() {
  static int cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount,
                              dev) != hipSuccess || n <= 0)
      n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

}  // namespace tmopt

extern "C" const char* tmopt_last_error(void) { return tmopt::g_err; }

extern "C" const char* tmopt_version(void) { return "tmopt_attn 0.1 gfx950"; }
