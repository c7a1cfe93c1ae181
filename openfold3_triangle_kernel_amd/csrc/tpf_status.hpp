// Status codes and the thread-local error message shared by every entry point.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "tpf_amd.h"  // status codes and the declarations every entry point must match

namespace tpf {

char* error_buffer();

inline int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(error_buffer(), 512, fmt, ap);
  va_end(ap);
  return code;
}

// Compute units of the current device (cached per device; 256 if unknown).
int device_cus();

inline int check_launch(const char* fn) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(TPF_ERR_LAUNCH, "%s: %s", fn, hipGetErrorString(e));
  return TPF_OK;
}

}  // namespace tpf
