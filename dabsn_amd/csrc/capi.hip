// Library-level C-ABI: version, error string and small utility kernels.
#include <stdarg.h>
#include <stdio.h>

#include <hip/hip_ext.h>

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

// CU masks of hipExtStreamCreateWithCUMask: bits in alternating groups of 8. The runtime
// deals mask bits round-robin over the XCDs (8 on MI355X), so a group of 8 consecutive bits
// is one CU of every XCD and each stream gets half of every XCD's CUs.
int dabsn_hip_stream_pair(hipStream_t* a, hipStream_t* b, int* cus_a, int* cus_b) {
  DABSN_REQUIRE(a && b && cus_a && cus_b, "stream pair: null pointer");
  int dev = 0, cus = 0;
  DABSN_HIP_CHECK(hipGetDevice(&dev));
  DABSN_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  DABSN_REQUIRE(cus >= 2 && cus <= 1024, "stream pair: %d CUs", cus);
  uint32_t ma[32] = {0}, mb[32] = {0};
  int na = 0, nb = 0;
  for (int i = 0; i < cus; ++i) {
    if ((i / 8) % 2 == 0) {
      ma[i / 32] |= 1u << (i % 32);
      ++na;
    } else {
      mb[i / 32] |= 1u << (i % 32);
      ++nb;
    }
  }
  DABSN_REQUIRE(na > 0 && nb > 0, "stream pair: %d CUs cannot be split", cus);
  const uint32_t words = static_cast<uint32_t>((cus + 31) / 32);
  DABSN_HIP_CHECK(hipExtStreamCreateWithCUMask(a, words, ma));
  const hipError_t e = hipExtStreamCreateWithCUMask(b, words, mb);
  if (e != hipSuccess) {
    (void)hipStreamDestroy(*a);
    dabsn::set_error("stream pair: %s", hipGetErrorString(e));
    return DABSN_ERR_HIP;
  }
  *cus_a = na;
  *cus_b = nb;
  return DABSN_OK;
}

int dabsn_hip_stream_destroy(hipStream_t stream) {
  DABSN_REQUIRE(stream != nullptr, "stream destroy: null stream");
  DABSN_HIP_CHECK(hipStreamSynchronize(stream));
  DABSN_HIP_CHECK(hipStreamDestroy(stream));
  return DABSN_OK;
}

}  // extern "C"
