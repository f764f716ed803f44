// Error reporting and device queries shared by every entry point.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <mutex>

#include "common.h"

namespace voom {

namespace {
thread_local char g_error[1024] = "";
}

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return VOOM_OK;
  snprintf(g_error, sizeof(g_error), "%s: %s (%d)", what, hipGetErrorString(e),
           static_cast<int>(e));
  return static_cast<int>(e);
}

int device_cu_count() {
  static std::mutex mu;
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

}  // namespace voom

extern "C" const char* voom_last_error(void) { return voom::g_error; }

extern "C" int voom_abi_version(void) { return 6; }
