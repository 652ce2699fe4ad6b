// Error reporting, version and device queries shared by every entry point.
#include "common.h"

#include <string.h>

static thread_local char g_err[512];

void bs_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

void bs_clear_error() { g_err[0] = 0; }

extern "C" const char* bs_last_error(void) { return g_err; }

extern "C" int bs_version(void) { return 1; }

int bs_num_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    cache[dev] = cus;
  }
  return cache[dev];
}
