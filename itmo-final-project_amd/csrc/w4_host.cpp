// Host-side plumbing shared by every C-ABI entry point: thread-local error
// messages and launch checking.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "w4_common.hpp"

namespace w4host {

static thread_local char g_err[512] = "";

void clear_error() { g_err[0] = '\0'; }

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(W4_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return W4_OK;
}

int device_cu_count() {
  // Cached per device: the count drives the static split-K table, so it must
  // not change between calls.
  static thread_local int cached_dev = -1;
  static thread_local int cached_cus = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (dev != cached_dev) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
    cached_dev = dev;
    cached_cus = cus;
  }
  return cached_cus;
}

}  // namespace w4host

extern "C" {

int w4_abi_version(void) { return W4_ABI_VERSION; }

const char* w4_last_error(void) { return w4host::g_err; }

}  // extern "C"
