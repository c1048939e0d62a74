// sf_api.hip — library-wide entry points: error reporting, version, arch check.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "sf_common.h"

static thread_local char g_last_error[512] = "";

int sf_fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int sf_check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return sf_fail(SF_EHIP, "%s: %s", what, hipGetErrorString(e));
  return SF_OK;
}

extern "C" const char *sf_last_error(void) { return g_last_error; }

extern "C" int sf_abi_version(void) { return SF_ABI_VERSION; }

extern "C" int sf_device_arch_ok(int device) {
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return sf_fail(SF_EHIP, "hipGetDeviceProperties: %s", hipGetErrorString(e));
  return strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}
