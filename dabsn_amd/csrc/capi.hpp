// Error reporting shared by the C-ABI entry points.
#pragma once

#include <hip/hip_runtime.h>

namespace dabsn {

// Records a printf-style message returned by dabsn_hip_last_error().
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

}  // namespace dabsn

// Status codes returned by every entry point.
#define DABSN_OK 0
#define DABSN_ERR_HIP (-1)
#define DABSN_ERR_ARG (-2)
#define DABSN_ERR_UNSUPPORTED (-3)

#define DABSN_HIP_CHECK(expr)                                                        \
  do {                                                                               \
    hipError_t e_ = (expr);                                                          \
    if (e_ != hipSuccess) {                                                          \
      dabsn::set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__, \
                       __LINE__);                                                    \
      return DABSN_ERR_HIP;                                                          \
    }                                                                                \
  } while (0)

#define DABSN_REQUIRE(cond, ...)       \
  do {                                 \
    if (!(cond)) {                     \
      dabsn::set_error(__VA_ARGS__);   \
      return DABSN_ERR_ARG;            \
    }                                  \
  } while (0)
