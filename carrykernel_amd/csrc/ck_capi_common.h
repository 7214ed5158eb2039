// Host-side helpers shared by the extern "C" entry points: status codes and a
// thread-local error message.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "carrykernel_gdn.h"

namespace ck {

inline std::string& last_error() {
  static thread_local std::string msg;
  return msg;
}

inline int fail(int status, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  last_error() = buf;
  return status;
}

inline int ok() {
  last_error().clear();
  return CK_OK;
}

inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(CK_ELAUNCH, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  return ok();
}

inline bool valid_dtype(int d) { return d == CK_DTYPE_F32 || d == CK_DTYPE_BF16 || d == CK_DTYPE_F16; }

}  // namespace ck
