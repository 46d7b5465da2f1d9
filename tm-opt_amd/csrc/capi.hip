// Library-wide C-ABI plumbing: thread-local error text and version string.
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

}  // namespace tmopt

extern "C" const char* tmopt_last_error(void) { return tmopt::g_err; }

extern "C" const char* tmopt_version(void) { return "tmopt_attn 0.1 gfx950"; }
