// Version, status names and the thread-local last-error string of the C ABI.
#include <cstdio>
#include <cstring>

#include "mm_common.h"

namespace mm {

namespace {
thread_local char g_last_error[512] = {0};
}

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  int n = std::snprintf(g_last_error, sizeof(g_last_error), "%s: ", mm_status_name(status));
  if (n < 0) n = 0;
  if (n < static_cast<int>(sizeof(g_last_error)))
    std::vsnprintf(g_last_error + n, sizeof(g_last_error) - n, fmt, ap);
  va_end(ap);
  return status;
}

void clear_error() { g_last_error[0] = '\0'; }

int num_cus() {
  static DeviceCache cache;
  return device_cached(
      cache,
      [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
          n = 0;
        return n;
      },
      256);
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MM_ERR_HIP, "%s launch failed: %s", what, hipGetErrorString(e));
  return MM_OK;
}

}  // namespace mm

extern "C" {

int mm_abi_version(void) { return MM_ABI_VERSION; }

const char* mm_last_error(void) { return mm::g_last_error; }

const char* mm_status_name(int status) {
  switch (status) {
    case MM_OK: return "MM_OK";
    case MM_ERR_NULL_POINTER: return "MM_ERR_NULL_POINTER";
    case MM_ERR_SHAPE: return "MM_ERR_SHAPE";
    case MM_ERR_DSTATE: return "MM_ERR_DSTATE";
    case MM_ERR_DTYPE: return "MM_ERR_DTYPE";
    case MM_ERR_LAYOUT: return "MM_ERR_LAYOUT";
    case MM_ERR_WORKSPACE: return "MM_ERR_WORKSPACE";
    case MM_ERR_HIP: return "MM_ERR_HIP";
    default: return "MM_ERR_UNKNOWN";
  }
}

}  // extern "C"
