// Error reporting and library-wide entry points of libmiq.
#include <stdarg.h>
#include <stdio.h>

#include "miq_common.h"

namespace miq {

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
  if (e != hipSuccess) return fail(MIQ_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return MIQ_OK;
}

}  // namespace miq

extern "C" const char* miq_last_error(void) { return miq::g_err; }

extern "C" int miq_version(void) { return MIQ_VERSION; }
