// Error reporting shared by the C-ABI translation units of libmuspace_msda.so:
// every entry point returns a MUSPACE_* code and leaves a message in one
// thread-local buffer that muspace_last_error() returns. Plays the role of the
// reference's TVM_FFI_ICHECK exceptions and musaGetLastError check
// (/root/reference/csrc/ffi/tensor_utils.hpp:13-38), without C++ exceptions
// crossing the ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "../../include/muspace_msda.h"

namespace capi {

inline thread_local char g_error[512] = "";

inline int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

inline int ok() {
  g_error[0] = '\0';
  return MUSPACE_OK;
}

inline int check_launch(const char *what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return fail(MUSPACE_ELAUNCH, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  }
  return ok();
}

}  // namespace capi
