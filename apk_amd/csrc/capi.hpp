// capi.hpp -- shared plumbing of the C ABI (error text, argument checks).
#pragma once
#include <hip/hip_runtime.h>
#include <stdio.h>
#include "apk.h"

namespace apk {

void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

#define APK_REQUIRE(cond, ...)          \
  do {                                  \
    if (!(cond)) {                      \
      ::apk::set_error(__VA_ARGS__);    \
      return APK_EINVAL;                \
    }                                   \
  } while (0)

#define APK_HIP(call)                                                      \
  do {                                                                     \
    hipError_t e_ = (call);                                                \
    if (e_ != hipSuccess) {                                                \
      ::apk::set_error("HIP error at %s:%d: %s", __FILE__, __LINE__,       \
                       hipGetErrorString(e_));                             \
      return APK_EHIP;                                                     \
    }                                                                      \
  } while (0)

// Launch-error check after a <<<>>> launch.
#define APK_LAUNCHED() APK_HIP(hipGetLastError())

inline hipStream_t as_stream(void* s) { return (hipStream_t)s; }

}  // namespace apk
