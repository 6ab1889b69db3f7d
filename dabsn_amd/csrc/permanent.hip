// Permanent associative delta scan (dabsn::permanent_delta_scan).
//
// Reference: src/dabsn/kernels/permanent.py:39-51 (definition), 70-119 (analytic reverse),
// CPU kernels cpu_runtime.cpp:1075-1188. Per batch row b a fast-weight state
// S [H_v, H_k] starts at zero and, for t = 0 .. T-1,
//   r_t = S k_t                      (output)
//   S  += beta_t (v_t - r_t) k_t^T   (rank-1 delta update)
// Each value row of S evolves on its own given k_t and beta_t, so the forward gives one
// wave to one (b, row): its 64 lanes hold the row's H columns (H / 64 each, in registers),
// r_t[row] is a wave reduction, the update is elementwise. fp32 state and arithmetic.
//
// Backward (adjoint A = dL/dS_{t+1}, per row a): walking t = T-1 .. 0,
//   Ak = a . k_t,  e = v_t[row] - r_t[row]
//   dv_t[row] = beta_t Ak,  dbeta_t += Ak e  (sum over rows)
//   dk_t += g_t[row] s_t + beta_t e a - beta_t Ak s_t  (sum over rows, s_t = state before t)
//   a = a + g_t[row] k_t - beta_t Ak k_t
// Workgroups of R waves own R rows; each first recomputes its rows' states, keeping r_t and
// every kCkpt-th state s_t (plus the final s_T), then runs the adjoint. The adjoint rebuilds
// s_t from s_{t+1} by undoing the row's update, s_t = s_{t+1} - beta_t (v_t - r_t) k_t, with
// the same e_t the forward used (r_t is taped), and restarts from a kept state at every
// checkpoint, so rounding drift spans at most kCkpt - 1 steps. The reference's reverse
// pass keeps every s_t instead (B H T H floats). The sums over rows are deterministic: the
// R rows of a workgroup are summed through LDS into a per-block partial, and reduce
// kernels add the blocks (dk) and rows (dbeta) in index order.
#include <algorithm>

#include "../../include/dabsn_hip.h"
#include "capi.hpp"
#include "common.hpp"

namespace dabsn {
namespace permanent {

constexpr int kRowsPerBlock = 8;  // backward: waves (value rows) per workgroup
constexpr int kFwdRows = 4;       // forward: waves per workgroup
constexpr int kCkpt = 8;          // backward: steps between kept states

// Kept states of the backward: s_t at index t / kCkpt for t % kCkpt == 0, t < T, and the
// final state s_T at index ceil(T / kCkpt).
__host__ __device__ inline int64_t ckpt_slots(int64_t T) { return (T + kCkpt - 1) / kCkpt + 1; }

// Lane's columns c = lane + 64 j, j < CPL; columns past H read and hold zero.
template <int CPL>
__device__ __forceinline__ void load_cols(const float* row, int lane, int H, float (&x)[CPL]) {
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + 64 * j;
    x[j] = c < H ? row[c] : 0.0f;
  }
}

template <int CPL>
__device__ __forceinline__ float dot_cols(const float (&a)[CPL], const float (&b)[CPL]) {
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < CPL; ++j) s = fmaf(a[j], b[j], s);
  return wave_sum(s);
}

template <int CPL>
__global__ void __launch_bounds__(kFwdRows * 64) perm_fwd_kernel(int T, int H,
                                                                 const float* __restrict__ k,
                                                                 const float* __restrict__ v,
                                                                 const float* __restrict__ beta,
                                                                 float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kFwdRows + (threadIdx.x >> 6);
  const int b = blockIdx.y;
  if (row >= H) return;  // whole waves; no barriers below
  float s[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) s[j] = 0.0f;
  const size_t base = static_cast<size_t>(b) * T * H;
  float kn[CPL];
  if (T > 0) load_cols<CPL>(k + base, lane, H, kn);
  for (int t = 0; t < T; ++t) {
    float kt[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) kt[j] = kn[j];
    if (t + 1 < T) load_cols<CPL>(k + base + static_cast<size_t>(t + 1) * H, lane, H, kn);
    const size_t o = base + static_cast<size_t>(t) * H + row;
    const float r = dot_cols<CPL>(s, kt);
    if (lane == 0) out[o] = r;
    const float e = beta[static_cast<size_t>(b) * T + t] * (v[o] - r);
#pragma unroll
    for (int j = 0; j < CPL; ++j) s[j] = fmaf(e, kt[j], s[j]);
  }
}

// Workspace of the backward: kept states [B][H][ckpt_slots(T)][H], r tape [B][T][H], per-block dk
// partials [B][T][nrb][H], per-row dbeta partials [B][T][H] (fp32, 256-byte aligned).
struct BwdLayout {
  size_t tape, rtape, pdk, pbeta, end;
};

static size_t align_up(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

static BwdLayout bwd_layout(int64_t B, int64_t T, int64_t H) {
  const size_t nrb = static_cast<size_t>((H + kRowsPerBlock - 1) / kRowsPerBlock);
  BwdLayout l{};
  size_t o = 0;
  l.tape = o; o = align_up(o + static_cast<size_t>(B) * H * ckpt_slots(T) * H * 4);
  l.rtape = o; o = align_up(o + static_cast<size_t>(B) * T * H * 4);
  l.pdk = o; o = align_up(o + static_cast<size_t>(B) * T * nrb * H * 4);
  l.pbeta = o; o = align_up(o + static_cast<size_t>(B) * T * H * 4);
  l.end = o;
  return l;
}

template <int CPL>
__global__ void __launch_bounds__(kRowsPerBlock * 64) perm_bwd_kernel(
    int T, int H, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ beta, const float* __restrict__ g, float* __restrict__ dv,
    float* __restrict__ tape, float* __restrict__ rtape, float* __restrict__ pdk,
    float* __restrict__ pbeta) {
  extern __shared__ float red[];  // [kRowsPerBlock][H]
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int rb = blockIdx.x, b = blockIdx.y;
  const int nrb = gridDim.x;
  const int row = rb * kRowsPerBlock + w;
  const bool live = row < H;  // waves past H take part in the barriers with zeros
  const size_t base = static_cast<size_t>(b) * T * H;
  const int64_t nck = ckpt_slots(T);
  float* my_tape = tape + (static_cast<size_t>(b) * H + (live ? row : 0)) * nck * H;

  // Forward recompute: r_t of this row, and the kept states.
  float s[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) s[j] = 0.0f;
  for (int t = 0; t < T; ++t) {
    float kt[CPL];
    load_cols<CPL>(k + base + static_cast<size_t>(t) * H, lane, H, kt);
    if (live && t % kCkpt == 0) {
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int c = lane + 64 * j;
        if (c < H) my_tape[static_cast<size_t>(t / kCkpt) * H + c] = s[j];
      }
    }
    const size_t o = base + static_cast<size_t>(t) * H + (live ? row : 0);
    const float r = dot_cols<CPL>(s, kt);
    if (live && lane == 0) rtape[o] = r;
    const float e = live ? beta[static_cast<size_t>(b) * T + t] * (v[o] - r) : 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) s[j] = fmaf(e, kt[j], s[j]);
  }
  if (live) {
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = lane + 64 * j;
      if (c < H) my_tape[static_cast<size_t>(nck - 1) * H + c] = s[j];
    }
  }

  // Adjoint. s_t is the kept state at checkpoint steps (exact, s_0 = 0 among them), else
  // rebuilt from sn = s_{t+1}: the kept final state at t = T - 1, otherwise the previous
  // iteration's s_t.
  float a[CPL], sn[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    a[j] = 0.0f;
    sn[j] = 0.0f;
  }
  if (live && T % kCkpt != 1) load_cols<CPL>(my_tape + static_cast<size_t>(nck - 1) * H, lane, H, sn);
  for (int t = T - 1; t >= 0; --t) {
    float kt[CPL], st[CPL];
    load_cols<CPL>(k + base + static_cast<size_t>(t) * H, lane, H, kt);
    const size_t o = base + static_cast<size_t>(t) * H + (live ? row : 0);
    const float bt = beta[static_cast<size_t>(b) * T + t];
    const float gr = live ? g[o] : 0.0f;
    const float e = live ? v[o] - rtape[o] : 0.0f;
    if (t % kCkpt == 0) {
      if (live) {
        load_cols<CPL>(my_tape + static_cast<size_t>(t / kCkpt) * H, lane, H, st);
      } else {
#pragma unroll
        for (int j = 0; j < CPL; ++j) st[j] = 0.0f;
      }
    } else {
      const float eb = bt * e;  // the forward's beta_t (v_t - r_t), bit for bit
#pragma unroll
      for (int j = 0; j < CPL; ++j) st[j] = fmaf(-eb, kt[j], sn[j]);
    }
#pragma unroll
    for (int j = 0; j < CPL; ++j) sn[j] = st[j];
    const float ak = dot_cols<CPL>(a, kt);
    if (live && lane == 0) {
      dv[o] = bt * ak;
      pbeta[o] = ak * e;
    }
    // This row's share of dk_t, summed over the workgroup's rows through LDS.
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = lane + 64 * j;
      if (c < H) red[w * H + c] = gr * st[j] + bt * a[j] * e - bt * st[j] * ak;
    }
    __syncthreads();
    for (int c = threadIdx.x; c < H; c += kRowsPerBlock * 64) {
      float sum = 0.0f;
#pragma unroll
      for (int r = 0; r < kRowsPerBlock; ++r) sum += red[r * H + c];
      pdk[((base / H + t) * nrb + rb) * H + c] = sum;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < CPL; ++j) a[j] = fmaf(gr - bt * ak, kt[j], a[j]);
  }
}

// dk[b, t, c] = sum over row blocks of pdk (block order); dbeta[b, t] = sum over rows of
// pbeta (row order). One thread per output element.
__global__ void __launch_bounds__(256) perm_reduce_kernel(int64_t BT, int H, int nrb,
                                                          const float* __restrict__ pdk,
                                                          const float* __restrict__ pbeta,
                                                          float* __restrict__ dk,
                                                          float* __restrict__ dbeta) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < BT * H) {
    const int64_t bt = i / H;
    const int c = static_cast<int>(i % H);
    float sum = 0.0f;
    for (int r = 0; r < nrb; ++r) sum += pdk[(bt * nrb + r) * H + c];
    dk[i] = sum;
  }
  if (i < BT) {
    float sum = 0.0f;
    for (int r = 0; r < H; ++r) sum += pbeta[i * H + r];
    dbeta[i] = sum;
  }
}

static int cpl_for(int64_t H) {
  for (int c : {1, 2, 4, 8, 16, 32})
    if (H <= 64 * c) return c;
  return 0;
}

static int checks(int64_t B, int64_t T, int64_t H, const void* k, const void* v,
                  const void* beta) {
  DABSN_REQUIRE(B > 0 && T >= 0 && H > 0, "permanent scan: bad shape");
  DABSN_REQUIRE(B < 65536 && T < (1 << 30), "permanent scan: dimension too large");
  DABSN_REQUIRE(cpl_for(H) != 0, "permanent scan: H=%lld > 2048 is not supported", (long long)H);
  DABSN_REQUIRE(k && v && beta, "permanent scan: null pointer");
  return DABSN_OK;
}

}  // namespace permanent
}  // namespace dabsn

using namespace dabsn;
using namespace dabsn::permanent;

extern "C" {

int dabsn_hip_permanent_scan_fwd(int64_t B, int64_t T, int64_t H, const float* key,
                                 const float* value, const float* beta, float* out,
                                 hipStream_t stream) {
  int rc = checks(B, T, H, key, value, beta);
  if (rc != DABSN_OK) return rc;
  DABSN_REQUIRE(out, "permanent scan: null output");
  if (T == 0) return DABSN_OK;
  const dim3 grid(static_cast<unsigned>((H + kFwdRows - 1) / kFwdRows), static_cast<unsigned>(B));
  const dim3 block(kFwdRows * 64);
  switch (cpl_for(H)) {
#define DABSN_CASE(C)                                                                        \
  case C:                                                                                    \
    hipLaunchKernelGGL(perm_fwd_kernel<C>, grid, block, 0, stream, (int)T, (int)H, key, value, \
                       beta, out);                                                           \
    break;
    DABSN_CASE(1) DABSN_CASE(2) DABSN_CASE(4) DABSN_CASE(8) DABSN_CASE(16) DABSN_CASE(32)
#undef DABSN_CASE
  }
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

size_t dabsn_hip_permanent_scan_workspace_bytes(int64_t B, int64_t T, int64_t H) {
  if (B <= 0 || T <= 0 || H <= 0) return 0;
  return bwd_layout(B, T, H).end;
}

int dabsn_hip_permanent_scan_bwd(int64_t B, int64_t T, int64_t H, const float* key,
                                 const float* value, const float* beta, const float* grad_out,
                                 float* dkey, float* dvalue, float* dbeta, void* workspace,
                                 size_t workspace_bytes, hipStream_t stream) {
  int rc = checks(B, T, H, key, value, beta);
  if (rc != DABSN_OK) return rc;
  DABSN_REQUIRE(grad_out && dkey && dvalue && dbeta, "permanent scan backward: null pointer");
  if (T == 0) return DABSN_OK;
  const BwdLayout l = bwd_layout(B, T, H);
  DABSN_REQUIRE(workspace && workspace_bytes >= l.end,
                "permanent scan backward: workspace %zu < %zu", workspace_bytes, l.end);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  float* tape = reinterpret_cast<float*>(ws + l.tape);
  float* rtape = reinterpret_cast<float*>(ws + l.rtape);
  float* pdk = reinterpret_cast<float*>(ws + l.pdk);
  float* pbeta = reinterpret_cast<float*>(ws + l.pbeta);
  const int nrb = static_cast<int>((H + kRowsPerBlock - 1) / kRowsPerBlock);
  const dim3 grid(static_cast<unsigned>(nrb), static_cast<unsigned>(B));
  const dim3 block(kRowsPerBlock * 64);
  const size_t lds = static_cast<size_t>(kRowsPerBlock) * H * 4;
  switch (cpl_for(H)) {
#define DABSN_CASE(C)                                                                       \
  case C:                                                                                   \
    hipLaunchKernelGGL(perm_bwd_kernel<C>, grid, block, lds, stream, (int)T, (int)H, key,   \
                       value, beta, grad_out, dvalue, tape, rtape, pdk, pbeta);             \
    break;
    DABSN_CASE(1) DABSN_CASE(2) DABSN_CASE(4) DABSN_CASE(8) DABSN_CASE(16) DABSN_CASE(32)
#undef DABSN_CASE
  }
  DABSN_HIP_CHECK(hipGetLastError());
  const int64_t BT = B * T;
  hipLaunchKernelGGL(perm_reduce_kernel, dim3(static_cast<unsigned>((BT * H + 255) / 256)),
                     dim3(256), 0, stream, BT, (int)H, nrb, pdk, pbeta, dkey, dbeta);
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

}  // extern "C"
