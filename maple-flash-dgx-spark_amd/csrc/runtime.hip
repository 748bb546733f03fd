// Library-level plumbing: version and per-thread error messages.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace ma {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return status;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MA_ERUNTIME, "%s: launch failed: %s", what, hipGetErrorString(e));
  return MA_OK;
}

}  // namespace ma

extern "C" int ma_version(void) { return 100; }

extern "C" const char* ma_last_error(void) { return ma::g_err; }
