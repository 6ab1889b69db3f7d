// Local field patch gather (dabsn::local_field_gather) and its scatter-add backward.
//
// Reference: src/dabsn/kernels/local_field.py:208-244 (op and registered backward),
// CPU kernels cpu_runtime.cpp:1191-1237.
//   out[b, p, j, :] = x[b, patch[p, j], :]                  x [B, N, D], patch [P, K]
//   gx[b, n, :]     = sum over (p, j) with patch[p, j] == n of gout[b, p, j, :]
// The gather is a copy: 16-byte vectors where a row of D elements allows it. The backward
// sums, for each source cell n, its entries e = p * K + j in increasing e -- the order in
// which the reference's CPU loop adds them -- through an inverse index built on the
// device (count per source, exclusive scan, fill, per-source sort of the entry lists), so
// fp32 results equal that loop's bit for bit and no float atomics are used. Indices
// outside [0, N) raise the workspace error word; their entries read and contribute zero.
#include <algorithm>

#include "../../include/dabsn_hip.h"
#include "capi.hpp"
#include "common.hpp"

namespace dabsn {
namespace field {

constexpr uint32_t kErrIndex = 1u;

__device__ __forceinline__ bool in_range(int64_t s, int N) { return s >= 0 && s < N; }

// Elements copied per thread: V (16 bytes) when every row of D elements is 16-byte aligned.
template <typename E, int V>
__global__ void __launch_bounds__(256) gather_kernel(int64_t total, int N, int D, int PK,
                                                     const E* __restrict__ x,
                                                     const int64_t* __restrict__ patch,
                                                     E* __restrict__ out, uint32_t* err) {
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * V;  // element
  if (i >= total) return;
  const int d = static_cast<int>(i % D);
  const int64_t row = i / D;  // (b, e)
  const int e = static_cast<int>(row % PK);
  const int64_t b = row / PK;
  const int64_t s = patch[e];
  if (!in_range(s, N)) {
    if (d == 0) atomicOr(err, kErrIndex);
#pragma unroll
    for (int v = 0; v < V; ++v) out[i + v] = E(0);
    return;
  }
  const E* src = x + (b * N + s) * D + d;
  if constexpr (V * sizeof(E) == 16) {
    gstore16(out + i, gload16(src));
  } else {
#pragma unroll
    for (int v = 0; v < V; ++v) out[i + v] = src[v];
  }
}

// Workspace of the backward: error word, counts[N], cursor[N], offsets[N + 1], list[P K]
// (int32).
struct BwdLayout {
  size_t counts, cursor, offsets, list, end;
};

static size_t align_up(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

static BwdLayout bwd_layout(int64_t N, int64_t PK) {
  BwdLayout l{};
  size_t o = 256;  // error word first
  l.counts = o; o = align_up(o + static_cast<size_t>(N) * 4);
  l.cursor = o; o = align_up(o + static_cast<size_t>(N) * 4);
  l.offsets = o; o = align_up(o + static_cast<size_t>(N + 1) * 4);
  l.list = o; o = align_up(o + static_cast<size_t>(PK) * 4);
  l.end = o;
  return l;
}

__global__ void __launch_bounds__(256) count_kernel(int PK, int N, const int64_t* __restrict__ patch,
                                                    int* counts, uint32_t* err) {
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (e >= PK) return;
  const int64_t s = patch[e];
  if (!in_range(s, N)) {
    atomicOr(err, kErrIndex);
    return;
  }
  atomicAdd(&counts[s], 1);
}

// offsets = exclusive prefix sum of counts (N + 1 entries), one workgroup: each thread sums
// a contiguous range, the 1024 range totals are scanned in LDS, then each range is written.
__global__ void __launch_bounds__(1024) scan_kernel(int N, const int* __restrict__ counts,
                                                    int* __restrict__ offsets) {
  __shared__ int part[1024];
  const int tid = threadIdx.x;
  const int per = (N + 1023) / 1024;
  const int lo = min(N, tid * per), hi = min(N, lo + per);
  int sum = 0;
  for (int n = lo; n < hi; ++n) sum += counts[n];
  part[tid] = sum;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {  // inclusive Hillis-Steele scan
    const int v = tid >= off ? part[tid - off] : 0;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  int run = tid > 0 ? part[tid - 1] : 0;
  for (int n = lo; n < hi; ++n) {
    offsets[n] = run;
    run += counts[n];
  }
  if (tid == 1023) offsets[N] = part[1023];
}

__global__ void __launch_bounds__(256) fill_kernel(int PK, int N, const int64_t* __restrict__ patch,
                                                   const int* __restrict__ offsets, int* cursor,
                                                   int* __restrict__ list) {
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (e >= PK) return;
  const int64_t s = patch[e];
  if (!in_range(s, N)) return;
  list[offsets[s] + atomicAdd(&cursor[s], 1)] = e;
}

// Each source's entries into increasing order (insertion sort; lists hold about K entries).
__global__ void __launch_bounds__(256) sort_kernel(int N, const int* __restrict__ offsets,
                                                   int* __restrict__ list) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= N) return;
  const int lo = offsets[n], hi = offsets[n + 1];
  for (int i = lo + 1; i < hi; ++i) {
    const int v = list[i];
    int j = i - 1;
    while (j >= lo && list[j] > v) {
      list[j + 1] = list[j];
      --j;
    }
    list[j + 1] = v;
  }
}

// gx[b, n, d] = sum over the entries e of source n, in list order, of gout[b, e, d].
template <typename E>
__global__ void __launch_bounds__(256) scatter_sum_kernel(int64_t total, int N, int D, int PK,
                                                          const E* __restrict__ gout,
                                                          const int* __restrict__ offsets,
                                                          const int* __restrict__ list,
                                                          E* __restrict__ gx) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= total) return;
  const int d = static_cast<int>(i % D);
  const int64_t bn = i / D;
  const int n = static_cast<int>(bn % N);
  const int64_t b = bn / N;
  float acc = 0.0f;
  for (int p = offsets[n]; p < offsets[n + 1]; ++p)
    acc += to_f(gout[(b * PK + list[p]) * D + d]);
  st(gx, static_cast<size_t>(i), acc);
}

static int checks(int dtype, int64_t B, int64_t N, int64_t D, int64_t P, int64_t K) {
  DABSN_REQUIRE(dtype == kF32 || dtype == kBF16, "local field gather: bad dtype %d", dtype);
  DABSN_REQUIRE(B > 0 && N > 0 && D > 0 && P >= 0 && K >= 0, "local field gather: bad shape");
  DABSN_REQUIRE(N < (1ll << 31) && P * K < (1ll << 31) && D < (1ll << 31),
                "local field gather: dimension too large");
  return DABSN_OK;
}

template <typename E>
static int gather_impl(int64_t B, int64_t N, int64_t D, int64_t PK, const E* x,
                       const int64_t* patch, E* out, uint32_t* err, hipStream_t stream) {
  const int64_t total = B * PK * D;
  if (total == 0) return DABSN_OK;
  constexpr int V = 16 / sizeof(E);
  const bool vec = (D % V == 0) && (reinterpret_cast<uintptr_t>(x) % 16 == 0) &&
                   (reinterpret_cast<uintptr_t>(out) % 16 == 0);
  if (vec) {
    hipLaunchKernelGGL((gather_kernel<E, V>), dim3(static_cast<unsigned>((total / V + 255) / 256)),
                       dim3(256), 0, stream, total, (int)N, (int)D, (int)PK, x, patch, out, err);
  } else {
    hipLaunchKernelGGL((gather_kernel<E, 1>), dim3(static_cast<unsigned>((total + 255) / 256)),
                       dim3(256), 0, stream, total, (int)N, (int)D, (int)PK, x, patch, out, err);
  }
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

}  // namespace field
}  // namespace dabsn

using namespace dabsn;
using namespace dabsn::field;

extern "C" {

size_t dabsn_hip_local_field_workspace_bytes(int64_t N, int64_t P, int64_t K, int backward) {
  if (!backward) return 256;
  return bwd_layout(N, P * K).end;
}

int dabsn_hip_local_field_gather(int dtype, int64_t B, int64_t N, int64_t D, int64_t P,
                                 int64_t K, const void* x, const int64_t* patch, void* out,
                                 void* workspace, size_t workspace_bytes, hipStream_t stream) {
  int rc = checks(dtype, B, N, D, P, K);
  if (rc != DABSN_OK) return rc;
  DABSN_REQUIRE(x && workspace && ((out && patch) || P * K == 0),
                "local field gather: null pointer");
  DABSN_REQUIRE(workspace_bytes >= 4, "local field gather: workspace %zu < 4", workspace_bytes);
  uint32_t* err = static_cast<uint32_t*>(workspace);
  rc = dabsn_hip_zero(err, 4, stream);
  if (rc != DABSN_OK) return rc;
  if (dtype == kBF16)
    return gather_impl<bf16>(B, N, D, P * K, static_cast<const bf16*>(x), patch,
                             static_cast<bf16*>(out), err, stream);
  return gather_impl<float>(B, N, D, P * K, static_cast<const float*>(x), patch,
                            static_cast<float*>(out), err, stream);
}

int dabsn_hip_local_field_gather_bwd(int dtype, int64_t B, int64_t N, int64_t D, int64_t P,
                                     int64_t K, const void* grad_out, const int64_t* patch,
                                     void* grad_x, void* workspace, size_t workspace_bytes,
                                     hipStream_t stream) {
  int rc = checks(dtype, B, N, D, P, K);
  if (rc != DABSN_OK) return rc;
  DABSN_REQUIRE(grad_x && workspace && ((grad_out && patch) || P * K == 0),
                "local field gather backward: null pointer");
  const int64_t PK = P * K;
  const BwdLayout l = bwd_layout(N, PK);
  DABSN_REQUIRE(workspace_bytes >= l.end, "local field gather backward: workspace %zu < %zu",
                workspace_bytes, l.end);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  uint32_t* err = reinterpret_cast<uint32_t*>(ws);
  int* counts = reinterpret_cast<int*>(ws + l.counts);
  int* cursor = reinterpret_cast<int*>(ws + l.cursor);
  int* offsets = reinterpret_cast<int*>(ws + l.offsets);
  int* list = reinterpret_cast<int*>(ws + l.list);
  rc = dabsn_hip_zero(ws, l.offsets, stream);  // error word, counts, cursor
  if (rc != DABSN_OK) return rc;
  const unsigned eblocks = static_cast<unsigned>((PK + 255) / 256);
  if (PK > 0) {
    hipLaunchKernelGGL(count_kernel, dim3(eblocks), dim3(256), 0, stream, (int)PK, (int)N, patch,
                       counts, err);
    DABSN_HIP_CHECK(hipGetLastError());
  }
  hipLaunchKernelGGL(scan_kernel, dim3(1), dim3(1024), 0, stream, (int)N, counts, offsets);
  DABSN_HIP_CHECK(hipGetLastError());
  if (PK > 0) {
    hipLaunchKernelGGL(fill_kernel, dim3(eblocks), dim3(256), 0, stream, (int)PK, (int)N, patch,
                       offsets, cursor, list);
    DABSN_HIP_CHECK(hipGetLastError());
    hipLaunchKernelGGL(sort_kernel, dim3(static_cast<unsigned>((N + 255) / 256)), dim3(256), 0,
                       stream, (int)N, offsets, list);
    DABSN_HIP_CHECK(hipGetLastError());
  }
  const int64_t total = B * N * D;
  const dim3 grid(static_cast<unsigned>((total + 255) / 256));
  if (dtype == kBF16)
    hipLaunchKernelGGL(scatter_sum_kernel<bf16>, grid, dim3(256), 0, stream, total, (int)N, (int)D,
                       (int)PK, static_cast<const bf16*>(grad_out), offsets, list,
                       static_cast<bf16*>(grad_x));
  else
    hipLaunchKernelGGL(scatter_sum_kernel<float>, grid, dim3(256), 0, stream, total, (int)N,
                       (int)D, (int)PK, static_cast<const float*>(grad_out), offsets, list,
                       static_cast<float*>(grad_x));
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

}  // extern "C"
