// The library's own entry points (version, error text) and the error
// bookkeeping the launch layers share.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "common.hpp"

namespace drift {

namespace {
thread_local char last_error[512] = "";
}

int refuse(const char* format, ...) {
  va_list args;
  va_start(args, format);
  vsnprintf(last_error, sizeof last_error, format, args);
  va_end(args);
  return (int)hipErrorInvalidValue;
}

int launched(const char* entry) {
  const hipError_t status = hipGetLastError();
  if (status != hipSuccess)
    snprintf(last_error, sizeof last_error, "%s: launch failed: %s", entry, hipGetErrorString(status));
  return (int)status;
}

void clear_error() { last_error[0] = '\0'; }

}  // namespace drift

extern "C" int drift_abi_version(void) { return DRIFT_ABI_VERSION; }

extern "C" const char* drift_error_string(int code) { return hipGetErrorString((hipError_t)code); }

extern "C" const char* drift_last_error(void) { return drift::last_error; }
