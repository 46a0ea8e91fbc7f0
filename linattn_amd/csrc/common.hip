// Error state and version entry points of the C ABI.
#include <stdarg.h>

#include "common.h"

namespace la {

static thread_local char g_last_error[512] = "";

void set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int num_cus() {
  static thread_local int cached_dev = -1, cached = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (dev != cached_dev) {
    int v = 0;
    cached = hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0
                 ? v
                 : 256;
    cached_dev = dev;
  }
  return cached;
}

}  // namespace la

extern "C" int la_abi_version(void) { return LA_ABI_VERSION; }

extern "C" const char *la_last_error(void) { return la::g_last_error; }
