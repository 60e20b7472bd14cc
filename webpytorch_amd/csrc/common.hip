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
  // a runtime failure is reported here; the runtime's own last-error state is cleared so that it
  // does not surface later as the failure of an unrelated launch
  if (code == MIQ_ERR_HIP) (void)hipGetLastError();
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MIQ_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return MIQ_OK;
}

int require_lds(const char* what, size_t bytes) {
  // A launch may ask for dynamic LDS up to the device's per-workgroup limit (160 KB on gfx950)
  // with no opt-in call; the limit is read once per device.
  static int limit[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
    return fail(MIQ_ERR_HIP, "%s: cannot query the current device", what);
  if (limit[dev] <= 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0)
      return fail(MIQ_ERR_HIP, "%s: cannot query the LDS limit", what);
    limit[dev] = v;
  }
  if (bytes > (size_t)limit[dev])
    return fail(MIQ_ERR_UNSUPPORTED, "%s: %zu bytes of LDS exceed the device's %d", what, bytes, limit[dev]);
  return MIQ_OK;
}

}  // namespace miq

extern "C" const char* miq_last_error(void) { return miq::g_err; }

extern "C" int miq_version(void) { return MIQ_VERSION; }
