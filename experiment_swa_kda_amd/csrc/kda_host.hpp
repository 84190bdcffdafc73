// Host-side helpers of libkda_mi355x: error reporting and launch checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/kda_mi355x.h"

namespace kda {

// Formats the calling thread's last error and returns `code`.
int set_error(int code, const char* fmt, ...);
void clear_error();

inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(KDA_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return KDA_OK;
}

// Raises a kernel's dynamic-LDS limit to `bytes` on the current device, once per
// (kernel, device); thread-safe.  Returns the HIP error of the first failing call.
hipError_t ensure_lds_limit(const void* kernel, int bytes);

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// True when every pointer is null or 16-byte aligned (the kernels move 16-byte vectors).
inline bool aligned16() { return true; }
template <typename P, typename... R>
inline bool aligned16(P p, R... rest) {
  return ((uintptr_t)p % 16) == 0 && aligned16(rest...);
}

}  // namespace kda

#define KDA_REQUIRE(cond, ...)                                    \
  do {                                                            \
    if (!(cond)) return ::kda::set_error(KDA_ERR_INVALID, __VA_ARGS__); \
  } while (0)

#define KDA_LAUNCH_CHECK(what)                     \
  do {                                             \
    int _rc = ::kda::check_launch(what);           \
    if (_rc != KDA_OK) return _rc;                 \
  } while (0)
