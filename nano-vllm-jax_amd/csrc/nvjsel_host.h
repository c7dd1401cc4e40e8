// Host-side helpers shared by the C ABI translation units: error recording,
// device properties and launch checks.
#pragma once
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/nvjsel.h"

namespace nvjsel {

void set_error(const char* fmt, ...);
void clear_error();

// Compute units of the current device (cached per device id).
int device_cu_count();
// Largest LDS allocation one workgroup may request on the current device.
size_t device_max_lds_per_block();

inline int fail(int code, const char* what) {
  set_error("%s", what);
  return code;
}

#define NVJSEL_CHECK_HIP(expr)                                                  \
  do {                                                                          \
    hipError_t e_ = (expr);                                                     \
    if (e_ != hipSuccess) {                                                     \
      (void)hipGetLastError(); /* do not leave a sticky error for the caller */ \
      ::nvjsel::set_error("%s failed: %s", #expr, hipGetErrorString(e_));       \
      return NVJSEL_EHIP;                                                       \
    }                                                                           \
  } while (0)

// Checks the launch that was just issued.
#define NVJSEL_CHECK_LAUNCH(name)                                               \
  do {                                                                          \
    hipError_t e_ = hipGetLastError();                                          \
    if (e_ != hipSuccess) {                                                     \
      ::nvjsel::set_error("launch of %s failed: %s", name, hipGetErrorString(e_)); \
      return NVJSEL_EHIP;                                                       \
    }                                                                           \
  } while (0)

inline bool valid_dtype(int d) { return d == NVJSEL_F32 || d == NVJSEL_BF16 || d == NVJSEL_F16; }
inline size_t dtype_size(int d) { return d == NVJSEL_F32 ? 4 : 2; }

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

}  // namespace nvjsel
