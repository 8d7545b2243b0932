// Library facts and the per-thread error state of the C ABI.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "internal.h"

namespace intent {

static thread_local char g_error[512];
static thread_local char g_last_kernel[128];

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_error[0] = '\0'; }

int launch_status(const char* kernel) {
  snprintf(g_last_kernel, sizeof(g_last_kernel), "%s", kernel);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(INTENT_ERR_LAUNCH, "%s: launch failed: %s", kernel, hipGetErrorString(e));
  return INTENT_OK;
}

int launch_status_fmt(const char* fmt, ...) {
  char name[128];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(name, sizeof(name), fmt, ap);
  va_end(ap);
  return launch_status(name);
}

}  // namespace intent

extern "C" int intent_amd_abi_version(void) { return INTENT_AMD_ABI_VERSION; }

extern "C" const char* intent_amd_last_error(void) { return intent::g_error; }

extern "C" const char* intent_amd_last_kernel(void) { return intent::g_last_kernel; }

extern "C" int intent_amd_device_arch(int device, char* buf, int64_t buf_len) {
  if (buf == nullptr || buf_len <= 0) return intent::fail(INTENT_ERR_INVALID_ARGUMENT, "null buffer");
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return intent::fail(INTENT_ERR_LAUNCH, "hipGetDeviceProperties: %s", hipGetErrorString(e));
  snprintf(buf, (size_t)buf_len, "%s", prop.gcnArchName);
  return INTENT_OK;
}
