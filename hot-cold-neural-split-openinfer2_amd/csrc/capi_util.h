// Host-side helpers for the C ABI: thread-local error string, HIP checks.
#pragma once
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string>

#include "oi2.h"

namespace oi2 {

void set_error(const char* fmt, ...);
void clear_error();

}  // namespace oi2

#define OI2_CHECK_ARG(cond, ...)        \
  do {                                  \
    if (!(cond)) {                      \
      ::oi2::set_error(__VA_ARGS__);    \
      return OI2_EINVAL;                \
    }                                   \
  } while (0)

#define OI2_CHECK_HIP(expr)                                                              \
  do {                                                                                   \
    hipError_t _e = (expr);                                                              \
    if (_e != hipSuccess) {                                                              \
      ::oi2::set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(_e), __FILE__, \
                       __LINE__);                                                        \
      return OI2_EHIP;                                                                   \
    }                                                                                    \
  } while (0)

#define OI2_CHECK_LAUNCH() OI2_CHECK_HIP(hipGetLastError())
