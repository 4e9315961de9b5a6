// Error reporting and small ABI-level entry points of libnslg_kv.
#include "nslg_common.h"

#include <stdarg.h>
#include <stdio.h>

namespace nslg {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return NSLG_ELAUNCH;
  }
  return NSLG_OK;
}

}  // namespace nslg

extern "C" int nslg_version(void) { return 100; }

extern "C" const char* nslg_last_error(void) { return nslg::g_err; }
