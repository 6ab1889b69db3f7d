// Library-level C-ABI: version, error string and small utility kernels.
#include <stdarg.h>
#include <stdio.h>

#include "../../include/dabsn_hip.h"
#include "capi.hpp"
#include "common.hpp"

namespace dabsn {

static thread_local char g_error[1024] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

__global__ void zero_words_kernel(uint32_t* p, size_t n) {
  size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (; i < n; i += stride) p[i] = 0u;
}

}  // namespace dabsn

extern "C" {

int dabsn_hip_abi_version(void) { return DABSN_HIP_ABI_VERSION; }

const char* dabsn_hip_last_error(void) { return dabsn::g_error; }

int dabsn_hip_zero(void* ptr, size_t bytes, hipStream_t stream) {
  DABSN_REQUIRE(bytes % 4 == 0, "dabsn_hip_zero: size %zu is not a multiple of 4", bytes);
  if (bytes == 0) return DABSN_OK;
  const size_t words = bytes / 4;
  size_t blocks = (words + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(dabsn::zero_words_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     stream, static_cast<uint32_t*>(ptr), words);
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

}  // extern "C"
