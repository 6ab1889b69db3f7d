// Row kernels of the chunked readout + cross-entropy loss.
//
// Reference: src/dabsn/runtime/loss.py:52-137 (ChunkedLinearCrossEntropy): per chunk of rows
// the readout GEMM gives logits [rows, V] in the hidden dtype; the loss upcasts them to fp32
// and forms logsumexp, the target logit and the masked NLL (forward), or
// (softmax - onehot(target)) * valid * scale (backward). The GEMMs stay on hipBLASLt; these
// kernels do each row's upcast, reductions and gradient in one pass over the logits (one
// workgroup per row; the forward keeps a running max and exp-sum per thread), instead of
// an fp32 copy plus logsumexp, gather, softmax and scatter kernels. Targets outside
// [0, V) other than ignore_index raise the error word and count as ignored.
#include <algorithm>

#include "../../include/dabsn_hip.h"
#include "capi.hpp"
#include "common.hpp"

namespace dabsn {
namespace loss {

constexpr int NTH = 256;
constexpr uint32_t kErrTarget = 1u;

__device__ __forceinline__ float block_reduce(float v, float* sh, bool is_max) {
  v = is_max ? wave_max(v) : wave_sum(v);
  __syncthreads();  // sh is reused by consecutive reductions
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = sh[0];
#pragma unroll
  for (int w = 1; w < NTH / 64; ++w) r = is_max ? fmaxf(r, sh[w]) : r + sh[w];
  return r;
}

// Fold one value (or the max of a vector with its exp-sum relative to that max) into a
// running (max, sum of exp(x - max)).
__device__ __forceinline__ void fold(float& m, float& s, float vm, float vs) {
  const float nm = fmaxf(m, vm);
  s = (m == -INFINITY ? 0.0f : s * __expf(m - nm)) + (vm == -INFINITY ? 0.0f : vs * __expf(vm - nm));
  m = nm;
}

// Row max m and sum of exp(x - m) in fp32 in one pass: each thread keeps a running
// (max, sum), rescaled once per VEC-element vector; the block combines the pairs.
template <typename E, int VEC>
__device__ __forceinline__ void row_stats(const E* x, int V, float* sh, float& m, float& s) {
  const int nv = V / VEC;
  m = -INFINITY;
  s = 0.0f;
  for (int c = threadIdx.x; c < nv; c += NTH) {
    float v[VEC];
    ldv<E, VEC>(x + static_cast<size_t>(c) * VEC, v);
    float vm = v[0];
#pragma unroll
    for (int e = 1; e < VEC; ++e) vm = fmaxf(vm, v[e]);
    float vs = 0.0f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) vs += __expf(v[e] - vm);
    fold(m, s, vm, vs);
  }
  for (int c = nv * VEC + threadIdx.x; c < V; c += NTH) fold(m, s, ld(x, c), 1.0f);
  // Block combine: the block max, then every thread's sum rescaled to it.
  const float M = block_reduce(m, sh, true);
  s = block_reduce(m == -INFINITY ? 0.0f : s * __expf(m - M), sh, false);
  m = M;
}

__device__ __forceinline__ bool target_ok(int64_t t, int V, int64_t ignore, uint32_t* err) {
  if (t == ignore) return false;
  if (t < 0 || t >= V) {
    if (threadIdx.x == 0) atomicOr(err, kErrTarget);
    return false;
  }
  return true;
}

template <typename E, int VEC>
__global__ void __launch_bounds__(NTH) ce_fwd_kernel(int V, int64_t ldl, const E* __restrict__ logits,
                                                     const int64_t* __restrict__ targets,
                                                     int64_t ignore, float* __restrict__ lse,
                                                     float* __restrict__ nll, uint32_t* err) {
  __shared__ float sh[NTH / 64];
  const int row = blockIdx.x;
  const E* x = logits + static_cast<size_t>(row) * ldl;
  float m, s;
  row_stats<E, VEC>(x, V, sh, m, s);
  if (threadIdx.x != 0) return;
  const float l = m + logf(s);
  lse[row] = l;
  const int64_t t = targets[row];
  nll[row] = target_ok(t, V, ignore, err) ? l - ld(x, static_cast<size_t>(t)) : 0.0f;
}

// d[row, c] = (exp(x - lse) - [c == target]) * valid * scale[0], fp32, row stride V.
template <typename E, int VEC>
__global__ void __launch_bounds__(NTH) ce_bwd_kernel(int V, int64_t ldl, const E* __restrict__ logits,
                                                     const int64_t* __restrict__ targets,
                                                     int64_t ignore, const float* __restrict__ lse,
                                                     const float* __restrict__ scale,
                                                     float* __restrict__ d, uint32_t* err) {
  const int row = blockIdx.x;
  const E* x = logits + static_cast<size_t>(row) * ldl;
  float* o = d + static_cast<size_t>(row) * V;
  const int64_t t = targets[row];
  const bool valid = target_ok(t, V, ignore, err);
  const float sc = valid ? scale[0] : 0.0f;
  const float l = lse[row];
  const int nv = V / VEC;
  for (int c = threadIdx.x; c < nv; c += NTH) {
    float v[VEC];
    ldv<E, VEC>(x + static_cast<size_t>(c) * VEC, v);
    float r[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const int col = c * VEC + e;
      r[e] = (__expf(v[e] - l) - (col == t ? 1.0f : 0.0f)) * sc;
    }
    if constexpr (VEC % 4 == 0) {
#pragma unroll
      for (int e = 0; e < VEC; e += 4)
        *reinterpret_cast<f32x4*>(o + c * VEC + e) = (f32x4){r[e], r[e + 1], r[e + 2], r[e + 3]};
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) o[c * VEC + e] = r[e];
    }
  }
  for (int c = nv * VEC + threadIdx.x; c < V; c += NTH)
    o[c] = (__expf(ld(x, c) - l) - (c == t ? 1.0f : 0.0f)) * sc;
}

static int checks(int dtype, int64_t rows, int64_t V, int64_t ldl) {
  DABSN_REQUIRE(dtype == kF32 || dtype == kBF16, "cross entropy: bad dtype %d", dtype);
  DABSN_REQUIRE(rows >= 0 && rows < (1ll << 31) && V > 0 && V < (1ll << 31) && ldl >= V,
                "cross entropy: bad shape (rows=%lld, V=%lld, ld=%lld)", (long long)rows,
                (long long)V, (long long)ldl);
  return DABSN_OK;
}

// 8-element vector loads need every row to start 16-byte aligned (bf16: ld a multiple of
// 8; fp32: of 4, the 8-vector being two 16-byte loads); the rest of a row is read singly.
static bool vec_rows(const void* p, int64_t ldl, size_t esize) {
  return (reinterpret_cast<uintptr_t>(p) % 16 == 0) && ((ldl * esize) % 16 == 0);
}

}  // namespace loss
}  // namespace dabsn

using namespace dabsn;
using namespace dabsn::loss;

extern "C" {

int dabsn_hip_ce_fwd(int dtype, int64_t rows, int64_t V, const void* logits, int64_t ldl,
                     const int64_t* targets, int64_t ignore_index, float* lse, float* nll,
                     uint32_t* err, hipStream_t stream) {
  int rc = checks(dtype, rows, V, ldl);
  if (rc != DABSN_OK) return rc;
  if (rows == 0) return DABSN_OK;
  DABSN_REQUIRE(logits && targets && lse && nll && err, "cross entropy: null pointer");
  const size_t es = dtype == kBF16 ? 2 : 4;
  const bool vec = vec_rows(logits, ldl, es);
  const dim3 grid(static_cast<unsigned>(rows));
#define DABSN_LAUNCH(E, VEC)                                                               \
  hipLaunchKernelGGL((ce_fwd_kernel<E, VEC>), grid, dim3(NTH), 0, stream, (int)V, ldl,      \
                     static_cast<const E*>(logits), targets, ignore_index, lse, nll, err)
  if (dtype == kBF16) {
    if (vec) DABSN_LAUNCH(bf16, 8); else DABSN_LAUNCH(bf16, 1);
  } else {
    if (vec) DABSN_LAUNCH(float, 8); else DABSN_LAUNCH(float, 1);
  }
#undef DABSN_LAUNCH
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

int dabsn_hip_ce_bwd(int dtype, int64_t rows, int64_t V, const void* logits, int64_t ldl,
                     const int64_t* targets, int64_t ignore_index, const float* lse,
                     const float* scale, float* dlogits, uint32_t* err, hipStream_t stream) {
  int rc = checks(dtype, rows, V, ldl);
  if (rc != DABSN_OK) return rc;
  if (rows == 0) return DABSN_OK;
  DABSN_REQUIRE(logits && targets && lse && scale && dlogits && err,
                "cross entropy backward: null pointer");
  const size_t es = dtype == kBF16 ? 2 : 4;
  // The 8-wide path also stores 16-byte fp32 vectors into rows of V floats.
  const bool vec = vec_rows(logits, ldl, es) && V % 8 == 0 &&
                   reinterpret_cast<uintptr_t>(dlogits) % 16 == 0;
  const dim3 grid(static_cast<unsigned>(rows));
#define DABSN_LAUNCH(E, VEC)                                                               \
  hipLaunchKernelGGL((ce_bwd_kernel<E, VEC>), grid, dim3(NTH), 0, stream, (int)V, ldl,      \
                     static_cast<const E*>(logits), targets, ignore_index, lse, scale, dlogits, \
                     err)
  if (dtype == kBF16) {
    if (vec) DABSN_LAUNCH(bf16, 8); else DABSN_LAUNCH(bf16, 1);
  } else {
    if (vec) DABSN_LAUNCH(float, 8); else DABSN_LAUNCH(float, 1);
  }
#undef DABSN_LAUNCH
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

}  // extern "C"
