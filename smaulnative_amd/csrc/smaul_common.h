// smaul_common.h -- pieces shared by the translation units of libsmaul_rocm.so:
// the per-thread error channel behind smaul_last_error() and the launch check.
#ifndef SMAUL_COMMON_H
#define SMAUL_COMMON_H

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "smaul_rocm.h"

namespace smaul {

// Message of the calling thread's last failure (one buffer per thread for
// the whole library).
inline thread_local char g_err[512] = "";

inline int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(SMAUL_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return SMAUL_OK;
}

}  // namespace smaul

#endif  // SMAUL_COMMON_H
