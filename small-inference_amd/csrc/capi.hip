// C-ABI support of libsmallinf_hip.so: version, per-thread error messages, device queries.
#include <cstdarg>
#include <cstdio>

#include "sipa_common.h"

namespace sipa {

static thread_local char g_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

}  // namespace sipa

extern "C" int32_t sipa_abi_version(void) { return SIPA_ABI_VERSION; }

extern "C" const char* sipa_last_error(void) { return sipa::g_error; }

extern "C" int32_t sipa_device_cu_count(int32_t device) {
  static int cached[64] = {0};
  if (device < 0) {
    if (hipGetDevice(&device) != hipSuccess) return sipa::fail(SIPA_EHIP, "hipGetDevice failed");
  }
  if (device < 64 && cached[device] > 0) return cached[device];
  int n = 0;
  const hipError_t e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device);
  if (e != hipSuccess) return sipa::fail(SIPA_EHIP, "CU count of device %d: %s", device, hipGetErrorString(e));
  if (device < 64) cached[device] = n;
  return n;
}
