// Host-side helpers shared by the extern "C" entry points: error recording
// and argument checks.  Every check failure returns a fvx_status code and
// leaves a message for fvx_last_error(); nothing aborts.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/fluxvla_amd.h"

namespace fvx {

int set_error(int code, const char* fmt, ...);
void clear_error();

inline bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

inline int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(FVX_ERR_LAUNCH, "%s: launch failed: %s", what,
                     hipGetErrorString(e));
  return FVX_OK;
}

// Compute units of the current device (cached per device).
inline int device_cus() {
  static int cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] <= 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) !=
            hipSuccess || n <= 0)
      n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

}  // namespace fvx

#define FVX_REQUIRE(cond, code, ...)                    \
  do {                                                  \
    if (!(cond)) return ::fvx::set_error(code, __VA_ARGS__); \
  } while (0)
