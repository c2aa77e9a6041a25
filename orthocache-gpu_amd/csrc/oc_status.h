#pragma once
// Status helpers shared by the C-ABI translation units: fail() records a
// message for oc_last_error() (thread-local) and returns the status code.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "orthocache_hip.h"

namespace oc {

void set_last_error(const char* msg);

__attribute__((format(printf, 2, 3))) inline int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  set_last_error(buf);
  return code;
}

inline int hip_fail(hipError_t e, const char* what) {
  return fail(OC_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

}  // namespace oc
