// Status codes and the thread-local error message shared by every entry point.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

enum {
  TPF_OK = 0,
  TPF_ERR_ARG = 1,     // null pointer, bad workspace, bad enum value
  TPF_ERR_SHAPE = 2,   // unsupported or inconsistent dimensions
  TPF_ERR_LAUNCH = 3,  // the HIP runtime rejected a launch
};

namespace tpf {

char* error_buffer();

inline int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(error_buffer(), 512, fmt, ap);
  va_end(ap);
  return code;
}

inline int check_launch(const char* fn) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(TPF_ERR_LAUNCH, "%s: %s", fn, hipGetErrorString(e));
  return TPF_OK;
}

}  // namespace tpf
