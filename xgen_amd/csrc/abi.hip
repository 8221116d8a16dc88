// Status reporting shared by every xgen_amd entry point.
#include <stdarg.h>
#include <stdio.h>

#include <atomic>

#include "xgen_common.h"

namespace xgen {

static thread_local char g_last_error[512] = "";

int fail(int status, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

int ok() {
  g_last_error[0] = '\0';
  return XGEN_OK;
}

int launch_status(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(XGEN_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return ok();
}

int device_cu_count() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cached[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  if (dev < kMaxDevices) {
    const int c = cached[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int v = 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
  if (dev < kMaxDevices) cached[dev].store(v, std::memory_order_relaxed);
  return v;
}

}  // namespace xgen

extern "C" int xgen_abi_version(void) { return XGEN_ABI_VERSION; }

extern "C" const char *xgen_status_string(int status) {
  switch (status) {
    case XGEN_OK:
      return "ok";
    case XGEN_ERR_INVALID_ARGUMENT:
      return "invalid argument";
    case XGEN_ERR_UNSUPPORTED:
      return "unsupported shape or layout";
    case XGEN_ERR_HIP:
      return "HIP runtime error";
    default:
      return "unknown status";
  }
}

extern "C" const char *xgen_last_error(void) { return xgen::g_last_error; }
