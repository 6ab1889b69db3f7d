// Error reporting shared by the C-ABI entry points.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/dabsn_hip.h"

namespace dabsn {

// Records a printf-style message returned by dabsn_hip_last_error().
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

}  // namespace dabsn

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
