// Library-wide C ABI pieces: version, per-thread error message, launch checks.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace kda {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int clear_error() {
  g_last_error[0] = '\0';
  return KDA_OK;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(KDA_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return KDA_OK;
}

int device_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

}  // namespace kda

extern "C" int kda_version(void) { return 100; }  // 0.1.0

extern "C" const char* kda_last_error(void) { return kda::g_last_error; }
