// C-ABI plumbing: last-error message, launch status, library version.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "uwc_common.h"

static thread_local char g_last_error[512] = "";

int uwc_fail(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof g_last_error, fmt, ap);
  va_end(ap);
  return UWC_EINVAL;
}

int uwc_launch_status(const char* kernel) {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return UWC_OK;
  snprintf(g_last_error, sizeof g_last_error, "%s launch failed: %s", kernel, hipGetErrorString(e));
  return (int)e;
}

extern "C" const char* uwc_last_error(void) { return g_last_error; }

extern "C" int uwc_version(void) { return 1; }

#ifndef UWC_HEADER_SHA
#define UWC_HEADER_SHA "unstamped"
#endif
// build.sh stamps the header's hash in (-DUWC_HEADER_SHA=...)
extern "C" const char* uwc_header_sha(void) { return UWC_HEADER_SHA; }

// Compute units of the current device, queried once per device (256 on MI355X).
int uwc_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    cached[dev] = v;
  }
  return cached[dev];
}
