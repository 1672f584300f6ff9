// Host-side helpers of the q36 C-ABI: thread-local error text, argument checks, launch checks.
#pragma once
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "q36_abi.h"

namespace q36 {

void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

// Allow kernel fn `bytes` of dynamic LDS (above 64 KiB: raises the kernel's limit once per device).
int ensure_lds(const void* fn, size_t bytes, const char* what);

inline bool aligned16(const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// After a launch: report the HIP error (if any) as Q36_ELAUNCH.
inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return Q36_ELAUNCH;
  }
  return Q36_OK;
}

#define Q36_REQUIRE(cond, ...)      \
  do {                              \
    if (!(cond)) {                  \
      ::q36::set_error(__VA_ARGS__); \
      return Q36_EINVAL;            \
    }                               \
  } while (0)

}  // namespace q36
