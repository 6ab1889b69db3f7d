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

// V consecutive elements at p (V = 1, or 16 bytes).
template <typename E, int V>
struct Vec {
  E e[V];
};
template <typename E, int V>
__device__ __forceinline__ Vec<E, V> vload(const E* p) {
  Vec<E, V> r;
  if constexpr (V * sizeof(E) == 16) {
    r = __builtin_bit_cast(Vec<E, V>, gload16(p));
  } else {
#pragma unroll
    for (int v = 0; v < V; ++v) r.e[v] = p[v];
  }
  return r;
}
template <typename E, int V>
__device__ __forceinline__ void vstore(E* p, const Vec<E, V>& r) {
  if constexpr (V * sizeof(E) == 16) {
    gstore16(p, __builtin_bit_cast(u32x4, r));
  } else {
#pragma unroll
    for (int v = 0; v < V; ++v) p[v] = r.e[v];
  }
}

// Grid (vectors of one batch row, B): thread j copies V elements (16 bytes when every row of
// D elements is 16-byte aligned) of entry e = j / (D / V). 32-bit index math (P K D < 2^31).
template <typename E, int V>
__global__ void __launch_bounds__(256) gather_kernel(int N, int D, int PK,
                                                     const E* __restrict__ x,
                                                     const int64_t* __restrict__ patch,
                                                     E* __restrict__ out, uint32_t* err) {
  const int b = blockIdx.y;
  const int dv = D / V;
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= PK * dv) return;
  const int e = j / dv, d = (j - e * dv) * V;
  E* dst = out + (static_cast<size_t>(b) * PK + e) * D + d;
  const int64_t s = patch[e];
  if (!in_range(s, N)) {
    if (d == 0) atomicOr(err, kErrIndex);
    vstore<E, V>(dst, Vec<E, V>{});
    return;
  }
  const Vec<E, V> v = vload<E, V>(x + (static_cast<size_t>(b) * N + s) * D + d);
  if constexpr (V * sizeof(E) == 16) {
    // Written once and not read back here: a streaming (non-temporal) store keeps the
    // output out of the caches the neighbours' source rows are read through.
    __builtin_nontemporal_store(__builtin_bit_cast(u32x4, v), reinterpret_cast<u32x4*>(dst));
  } else {
    vstore<E, V>(dst, v);
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

// offsets = exclusive prefix sum of counts (N + 1 entries), one workgroup, over tiles of
// 16 Ki counts staged in LDS with coalesced loads and stores: each thread scans 16
// consecutive counts, the 1024 thread totals are scanned in LDS, and a running carry links
// the tiles. Row i of the tile is stored at i + i / 16 (one pad word per 16) so the
// per-thread runs of 16 fall in different banks.
constexpr int kScanPer = 16, kScanTile = 1024 * kScanPer;

__device__ __forceinline__ int scan_slot(int i) { return i + i / kScanPer; }

__global__ void __launch_bounds__(1024) scan_kernel(int N, const int* __restrict__ counts,
                                                    int* __restrict__ offsets) {
  __shared__ int tile[kScanTile + kScanTile / kScanPer];
  __shared__ int part[1024];
  const int tid = threadIdx.x;
  int carry = 0;
  for (int base = 0; base < N; base += kScanTile) {
    const int len = min(kScanTile, N - base);
    for (int i = tid; i < kScanTile; i += 1024) tile[scan_slot(i)] = i < len ? counts[base + i] : 0;
    __syncthreads();
    int sum = 0;
#pragma unroll
    for (int j = 0; j < kScanPer; ++j) sum += tile[scan_slot(tid * kScanPer + j)];
    part[tid] = sum;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {  // inclusive Hillis-Steele scan
      const int v = tid >= off ? part[tid - off] : 0;
      __syncthreads();
      part[tid] += v;
      __syncthreads();
    }
    int run = carry + (tid > 0 ? part[tid - 1] : 0);
#pragma unroll
    for (int j = 0; j < kScanPer; ++j) {
      const int k = scan_slot(tid * kScanPer + j);
      const int c = tile[k];
      tile[k] = run;
      run += c;
    }
    carry += part[1023];
    __syncthreads();
    for (int i = tid; i < len; i += 1024) offsets[base + i] = tile[scan_slot(i)];
    __syncthreads();
  }
  if (tid == 0) offsets[N] = carry;
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

// gx[b, n, d..d+V) = sum over the entries e of source n, in list order, of gout[b, e, ...].
// Grid (vectors of one batch row, B), as gather_kernel.
template <typename E, int V>
__global__ void __launch_bounds__(256) scatter_sum_kernel(int N, int D, int PK,
                                                          const E* __restrict__ gout,
                                                          const int* __restrict__ offsets,
                                                          const int* __restrict__ list,
                                                          E* __restrict__ gx) {
  const int b = blockIdx.y;
  const int dv = D / V;
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= N * dv) return;
  const int n = j / dv, d = (j - n * dv) * V;
  float acc[V];
#pragma unroll
  for (int v = 0; v < V; ++v) acc[v] = 0.0f;
  const E* gb = gout + static_cast<size_t>(b) * PK * D + d;
  for (int p = offsets[n]; p < offsets[n + 1]; ++p) {
    const Vec<E, V> g = vload<E, V>(gb + static_cast<size_t>(list[p]) * D);
#pragma unroll
    for (int v = 0; v < V; ++v) acc[v] += to_f(g.e[v]);
  }
  Vec<E, V> r;
#pragma unroll
  for (int v = 0; v < V; ++v) r.e[v] = is_bf16<E>::value ? E(f2bf(acc[v])) : E(acc[v]);
  vstore<E, V>(gx + (static_cast<size_t>(b) * N + n) * D + d, r);
}

static int checks(int dtype, int64_t B, int64_t N, int64_t D, int64_t P, int64_t K) {
  DABSN_REQUIRE(dtype == kF32 || dtype == kBF16, "local field gather: bad dtype %d", dtype);
  DABSN_REQUIRE(B > 0 && N > 0 && D > 0 && P >= 0 && K >= 0, "local field gather: bad shape");
  DABSN_REQUIRE(B < 65536 && N * D < (1ll << 31) && P * K * D < (1ll << 31),
                "local field gather: dimension too large");
  return DABSN_OK;
}

// 16-byte vectors when rows of D elements keep both pointers 16-byte aligned.
template <typename E>
static bool vec_ok(int64_t D, const void* a, const void* b) {
  return D % (16 / sizeof(E)) == 0 && reinterpret_cast<uintptr_t>(a) % 16 == 0 &&
         reinterpret_cast<uintptr_t>(b) % 16 == 0;
}

template <typename E>
static int gather_impl(int64_t B, int64_t N, int64_t D, int64_t PK, const E* x,
                       const int64_t* patch, E* out, uint32_t* err, hipStream_t stream) {
  if (PK == 0) return DABSN_OK;
  constexpr int V = 16 / sizeof(E);
  if (vec_ok<E>(D, x, out)) {
    hipLaunchKernelGGL((gather_kernel<E, V>), dim3(static_cast<unsigned>((PK * D / V + 255) / 256),
                       static_cast<unsigned>(B)), dim3(256), 0, stream, (int)N, (int)D, (int)PK, x,
                       patch, out, err);
  } else {
    hipLaunchKernelGGL((gather_kernel<E, 1>), dim3(static_cast<unsigned>((PK * D + 255) / 256),
                       static_cast<unsigned>(B)), dim3(256), 0, stream, (int)N, (int)D, (int)PK, x,
                       patch, out, err);
  }
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

template <typename E>
static int scatter_impl(int64_t B, int64_t N, int64_t D, int64_t PK, const E* gout,
                        const int* offsets, const int* list, E* gx, hipStream_t stream) {
  constexpr int V = 16 / sizeof(E);
  if (vec_ok<E>(D, gout ? static_cast<const void*>(gout) : gx, gx)) {
    hipLaunchKernelGGL((scatter_sum_kernel<E, V>), dim3(static_cast<unsigned>((N * D / V + 255) / 256),
                       static_cast<unsigned>(B)), dim3(256), 0, stream, (int)N, (int)D, (int)PK, gout,
                       offsets, list, gx);
  } else {
    hipLaunchKernelGGL((scatter_sum_kernel<E, 1>), dim3(static_cast<unsigned>((N * D + 255) / 256),
                       static_cast<unsigned>(B)), dim3(256), 0, stream, (int)N, (int)D, (int)PK, gout,
                       offsets, list, gx);
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
  if (dtype == kBF16)
    return scatter_impl<bf16>(B, N, D, PK, static_cast<const bf16*>(grad_out), offsets, list,
                              static_cast<bf16*>(grad_x), stream);
  return scatter_impl<float>(B, N, D, PK, static_cast<const float*>(grad_out), offsets, list,
                             static_cast<float*>(grad_x), stream);
}

}  // extern "C"
