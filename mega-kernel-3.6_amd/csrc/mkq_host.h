// Host-side helpers shared by the C-ABI entry points: error reporting,
// dtype dispatch, cached device properties.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>

#include "../../include/mkq.h"
#include "mkq_device.h"

namespace mkq {

// Records a printf-style message for mkq_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// Number of compute units of the current device (queried once per device).
int cu_count();
// Max dynamic LDS bytes per workgroup of the current device (queried once).
int max_lds_per_block();
int current_device();

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace mkq

#define MKQ_REQUIRE(cond, ...)                                   \
  do {                                                           \
    if (!(cond)) return ::mkq::set_error(MKQ_ERR_INVALID, __VA_ARGS__); \
  } while (0)

#define MKQ_HIP_TRY(expr)                                                            \
  do {                                                                               \
    hipError_t _e = (expr);                                                          \
    if (_e != hipSuccess)                                                            \
      return ::mkq::set_error(MKQ_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(_e)); \
  } while (0)

// Checks the launch that was just enqueued.
#define MKQ_LAUNCH_CHECK(name)                                                        \
  do {                                                                                \
    hipError_t _e = hipGetLastError();                                                \
    if (_e != hipSuccess)                                                             \
      return ::mkq::set_error(MKQ_ERR_HIP, "%s launch failed: %s", name, hipGetErrorString(_e)); \
  } while (0)
