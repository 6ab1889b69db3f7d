// Block glue of the inference step: the element work around the read and the MLP branch
// of one DABSN block, each in one pass instead of the two to seven tensor operations the
// block's forward evaluates. Every kernel rounds where those operations round (each
// intermediate tensor is stored in the activation dtype E), so the results equal the
// unfused evaluation up to the summation order of the RMS norm's mean.
//
// Reference: src/dabsn/model.py:336 (y + read_gain * read), read.py:435 / :821
// (out(...) + long_gain * long), model.py:35-45 (MLPRMSNorm), model.py:188-195
// (relu(fc1(norm(h))).square()).
#include "../../include/dabsn_hip.h"
#include "capi.hpp"
#include "common.hpp"

#include <initializer_list>

namespace dabsn {
namespace block {

// out = y + read_gain * (proj + long_gain * long), each product and sum rounded to E.
template <typename E, int V>
__global__ void __launch_bounds__(256) read_mix_kernel(uint32_t chunks, const E* proj,
                                                       const E* lng, const float* long_gain,
                                                       const E* y, const float* read_gain,
                                                       E* out) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i >= chunks) return;
  const size_t o = static_cast<size_t>(i) * V;
  const float lg = long_gain[0], rg = read_gain[0];
  float a[V], l[V], w[V];
  ldv<E, V>(proj + o, a);
  ldv<E, V>(lng + o, l);
  ldv<E, V>(y + o, w);
#pragma unroll
  for (int e = 0; e < V; ++e) {
    const float r = round_to<E>(a[e] + round_to<E>(lg * l[e]));  // the read's output
    w[e] = w[e] + round_to<E>(rg * r);
  }
  stv<E, V>(out + o, w);
}

// One workgroup of 256 threads per row: scale = rsqrt(mean(x^2) + eps) in fp32, then
// out = E(E(x * scale) * weight).
template <typename E>
__global__ void __launch_bounds__(256) rms_norm_kernel(int H, const E* x, const E* weight,
                                                       float eps, E* out) {
  __shared__ float part[4];
  const size_t base = static_cast<size_t>(blockIdx.x) * H;
  float ss = 0.0f;
  for (int h = threadIdx.x; h < H; h += 256) {
    const float v = ld(x, base + h);
    ss += v * v;
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float total = (part[0] + part[1]) + (part[2] + part[3]);
  const float scale = rsqrtf(total * (1.0f / static_cast<float>(H)) + eps);
  for (int h = threadIdx.x; h < H; h += 256) {
    const float n = round_to<E>(ld(x, base + h) * scale);
    st(out, base + h, n * ld(weight, static_cast<size_t>(h)));
  }
}

// out = E(relu(x)^2).
template <typename E, int V>
__global__ void __launch_bounds__(256) relu_square_kernel(uint32_t chunks, const E* x, E* out) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i >= chunks) return;
  const size_t o = static_cast<size_t>(i) * V;
  float v[V];
  ldv<E, V>(x + o, v);
#pragma unroll
  for (int e = 0; e < V; ++e) {
    const float r = v[e] > 0.0f || v[e] != v[e] ? v[e] : 0.0f;  // relu keeps NaN
    v[e] = r * r;
  }
  stv<E, V>(out + o, v);
}

static inline unsigned blocks_for(int64_t n, int per) {
  return static_cast<unsigned>((n + per - 1) / per);
}

static bool vec8(int64_t n, std::initializer_list<const void*> ptrs) {
  if (n % 8 != 0) return false;
  for (const void* p : ptrs)
    if (reinterpret_cast<uintptr_t>(p) & 15u) return false;
  return true;
}

}  // namespace block
}  // namespace dabsn

using namespace dabsn;
using namespace dabsn::block;

extern "C" {

int dabsn_hip_read_mix(int dtype, int64_t n, const void* proj, const void* lng,
                       const float* long_gain, const void* y, const float* read_gain, void* out,
                       hipStream_t stream) {
  DABSN_REQUIRE(dtype == kF32 || dtype == kBF16, "read_mix: bad dtype %d", dtype);
  DABSN_REQUIRE(n >= 0, "read_mix: bad size");
  if (n == 0) return DABSN_OK;
  DABSN_REQUIRE(proj && lng && long_gain && y && read_gain && out, "read_mix: null pointer");
  const bool vec = vec8(n, {proj, lng, y, out});
  const int64_t chunks = n / (vec ? 8 : 1);
  DABSN_REQUIRE(chunks < (1ll << 32), "read_mix: too many elements");
  const dim3 grid(blocks_for(chunks, 256)), block(256);
#define L(E, V)                                                                              \
  hipLaunchKernelGGL((read_mix_kernel<E, V>), grid, block, 0, stream, (uint32_t)chunks,      \
                     (const E*)proj, (const E*)lng, long_gain, (const E*)y, read_gain, (E*)out)
  if (dtype == kBF16) {
    if (vec) L(bf16, 8); else L(bf16, 1);
  } else {
    if (vec) L(float, 8); else L(float, 1);
  }
#undef L
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

int dabsn_hip_rms_norm(int dtype, int64_t rows, int64_t H, const void* x, const void* weight,
                       float eps, void* out, hipStream_t stream) {
  DABSN_REQUIRE(dtype == kF32 || dtype == kBF16, "rms_norm: bad dtype %d", dtype);
  DABSN_REQUIRE(rows >= 0 && H > 0 && H < (1 << 30) && rows < (1ll << 31),
                "rms_norm: bad shape rows=%lld H=%lld", (long long)rows, (long long)H);
  if (rows == 0) return DABSN_OK;
  DABSN_REQUIRE(x && weight && out, "rms_norm: null pointer");
  if (dtype == kBF16)
    hipLaunchKernelGGL(rms_norm_kernel<bf16>, dim3((unsigned)rows), dim3(256), 0, stream, (int)H,
                       (const bf16*)x, (const bf16*)weight, eps, (bf16*)out);
  else
    hipLaunchKernelGGL(rms_norm_kernel<float>, dim3((unsigned)rows), dim3(256), 0, stream,
                       (int)H, (const float*)x, (const float*)weight, eps, (float*)out);
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

int dabsn_hip_relu_square(int dtype, int64_t n, const void* x, void* out, hipStream_t stream) {
  DABSN_REQUIRE(dtype == kF32 || dtype == kBF16, "relu_square: bad dtype %d", dtype);
  DABSN_REQUIRE(n >= 0, "relu_square: bad size");
  if (n == 0) return DABSN_OK;
  DABSN_REQUIRE(x && out, "relu_square: null pointer");
  const bool vec = vec8(n, {x, out});
  const int64_t chunks = n / (vec ? 8 : 1);
  DABSN_REQUIRE(chunks < (1ll << 32), "relu_square: too many elements");
  const dim3 grid(blocks_for(chunks, 256)), block(256);
#define L(E, V)                                                                                 \
  hipLaunchKernelGGL((relu_square_kernel<E, V>), grid, block, 0, stream, (uint32_t)chunks,    \
                     (const E*)x, (E*)out)
  if (dtype == kBF16) {
    if (vec) L(bf16, 8); else L(bf16, 1);
  } else {
    if (vec) L(float, 8); else L(float, 1);
  }
#undef L
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

}  // extern "C"
