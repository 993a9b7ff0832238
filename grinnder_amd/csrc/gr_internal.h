// Internal helpers shared by the translation units of libgrinnder_amd.so.
#pragma once

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#else
#include <hip/hip_runtime_api.h>
#endif

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/grinnder_amd.h"

namespace gr {

// Records a printf-style message as this thread's last error and returns
// `code`, so call sites can `return fail(GR_EINVAL, "...")`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Clears the last error message of this thread.
void clear_error();

// The last error message of this thread ("" if none).
const char* last_error_cstr();

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace gr

// Evaluates a HIP call; on failure records the call text and error string
// and returns GR_EHIP from the enclosing function.
#define GR_HIP_CHECK(expr)                                                   \
  do {                                                                       \
    hipError_t gr_err_ = (expr);                                             \
    if (gr_err_ != hipSuccess) {                                             \
      return ::gr::fail(GR_EHIP, "%s failed: %s (%s:%d)", #expr,              \
                        hipGetErrorString(gr_err_), __FILE__, __LINE__);     \
    }                                                                        \
  } while (0)

#define GR_REQUIRE(cond, ...)                                                \
  do {                                                                       \
    if (!(cond)) return ::gr::fail(GR_EINVAL, __VA_ARGS__);                  \
  } while (0)
