// Error reporting and ABI metadata for libatma_hip.so.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace atma {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(ATMA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return ATMA_OK;
}

int device_cu_count() {
  static int cached[64];  // 0 = not yet queried; a racing second query writes the same value
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

int dtype_size(int dtype) {
  switch (dtype) {
    case ATMA_F32: return 4;
    case ATMA_BF16: return 2;
    case ATMA_F16: return 2;
    default: return 0;
  }
}

}  // namespace atma

extern "C" int atma_abi_version(void) { return 2; }

extern "C" const char* atma_last_error(void) { return atma::g_last_error; }
