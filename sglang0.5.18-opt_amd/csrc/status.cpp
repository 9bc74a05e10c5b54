// Thread-local error status of the C ABI and small device queries.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "dsa_common.h"

namespace {
thread_local std::string g_last_error;
}

namespace dsa {

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return DSA_OK;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(DSA_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

}  // namespace dsa

extern "C" const char* dsa_last_error(void) { return g_last_error.c_str(); }

extern "C" int dsa_device_cu_count(int* n_cu) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(n_cu, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return dsa::fail(DSA_ERR_LAUNCH, "dsa_device_cu_count: %s", hipGetErrorString(e));
  return dsa::ok();
}
