// Library facts and the per-thread error state of the C ABI.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "internal.h"

namespace intent {

static thread_local char g_error[512];

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_error[0] = '\0'; }

int launch_status(const char* kernel) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(INTENT_ERR_LAUNCH, "%s: launch failed: %s", kernel, hipGetErrorString(e));
  return INTENT_OK;
}

}  // namespace intent

extern "C" int intent_amd_abi_version(void) { return INTENT_AMD_ABI_VERSION; }

extern "C" const char* intent_amd_last_error(void) { return intent::g_error; }

extern "C" int intent_amd_device_arch(int device, char* buf, int64_t buf_len) {
  if (buf == nullptr || buf_len <= 0) return intent::fail(INTENT_ERR_INVALID_ARGUMENT, "null buffer");
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return intent::fail(INTENT_ERR_LAUNCH, "hipGetDeviceProperties: %s", hipGetErrorString(e));
  snprintf(buf, (size_t)buf_len, "%s", prop.gcnArchName);
  return INTENT_OK;
}
