// Diagonal linear recurrences: the registered dabsn::linear_recurrence pair and the
// fused recurrent long-memory scan.
//
// Reference: src/dabsn/kernels/long.py:24-98 (linear recurrence and its analytic
// reverse), long.py:492-579 (long memory as three recurrences plus glue), loop form in
// src/dabsn/read.py:625-636; CPU kernels cpu_runtime.cpp:92-143.
//
// Every (batch row, unit) channel is an independent scalar recurrence over time, so
// one thread owns one channel and walks T; consecutive threads own consecutive units,
// so each time step is one coalesced row access. Loads for a block of time steps are
// issued before the dependent arithmetic so their latency overlaps.
#include "../../include/dabsn_hip.h"
#include "capi.hpp"
#include "common.hpp"

namespace dabsn {
namespace longmem {

constexpr int NT = 64;      // threads per block (one wave: spreads channels over CUs)
constexpr int TB = 8;       // time steps loaded ahead
constexpr int CK = DABSN_LONG_CKPT;

template <typename E>
__global__ void __launch_bounds__(NT) linrec_fwd_kernel(int B, int T, int H, const E* a,
                                                        const E* g, const E* y0, E* y) {
  const int64_t ch = static_cast<int64_t>(blockIdx.x) * NT + threadIdx.x;
  if (ch >= static_cast<int64_t>(B) * H) return;
  const int64_t b = ch / H, h = ch % H;
  float carry = ld(y0, ch);
  const size_t base = static_cast<size_t>(b) * T * H + h;
  for (int t0 = 0; t0 < T; t0 += TB) {
    float av[TB], gv[TB];
#pragma unroll
    for (int i = 0; i < TB; ++i) {
      const int t = t0 + i;
      av[i] = t < T ? ld(a, base + static_cast<size_t>(t) * H) : 0.0f;
      gv[i] = t < T ? ld(g, base + static_cast<size_t>(t) * H) : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < TB; ++i) {
      const int t = t0 + i;
      if (t < T) {
        carry = av[i] * carry + gv[i];
        st(y, base + static_cast<size_t>(t) * H, carry);
      }
    }
  }
}

// Reverse pass: c_t = gy_t + a_{t+1} c_{t+1}; dg_t = c_t; da_t = c_t y_{t-1};
// dy0 = a_0 c_0. y_{t-1} comes from an fp32 forward replay stored in `yprev`.
template <typename E>
__global__ void __launch_bounds__(NT) linrec_bwd_kernel(int B, int T, int H, const E* a,
                                                        const E* g, const E* y0, const E* gy,
                                                        E* da, E* dg, E* dy0, float* yprev) {
  const int64_t ch = static_cast<int64_t>(blockIdx.x) * NT + threadIdx.x;
  if (ch >= static_cast<int64_t>(B) * H) return;
  const int64_t b = ch / H, h = ch % H;
  const size_t base = static_cast<size_t>(b) * T * H + h;
  float carry = ld(y0, ch);
  for (int t = 0; t < T; ++t) {
    const size_t o = base + static_cast<size_t>(t) * H;
    yprev[o] = carry;
    carry = ld(a, o) * carry + ld(g, o);
  }
  float c = 0.0f;
  for (int t = T - 1; t >= 0; --t) {
    const size_t o = base + static_cast<size_t>(t) * H;
    const float a_next = (t + 1 < T) ? ld(a, o + H) : 0.0f;
    c = ld(gy, o) + a_next * c;
    st(dg, o, c);
    st(da, o, c * yprev[o]);
  }
  st(dy0, ch, T > 0 ? ld(a, base) * c : 0.0f);
}

struct Coef {
  float er, rd, ret, rs;
};

__device__ __forceinline__ Coef load_coef(const float* const* logits) {
  Coef c;
  c.er = sigmoidf_(logits[0][0]);
  c.rd = sigmoidf_(logits[1][0]);
  c.ret = sigmoidf_(logits[2][0]);
  c.rs = sigmoidf_(logits[3][0]);
  return c;
}

struct Logits {
  const float* p[4];
};

template <typename E>
__global__ void __launch_bounds__(NT) long_fwd_kernel(int B, int T, int H, const E* w, const E* p,
                                                      Logits lg, const float* L0, const float* E0,
                                                      const float* R0, E* out, float* LF, float* EF,
                                                      float* RF, float* ckpt) {
  const int64_t ch = static_cast<int64_t>(blockIdx.x) * NT + threadIdx.x;
  if (ch >= static_cast<int64_t>(B) * H) return;
  const Coef k = load_coef(lg.p);
  const int64_t b = ch / H, h = ch % H;
  const size_t base = static_cast<size_t>(b) * T * H + h;
  const int nseg = (T + CK - 1) / CK;
  float L = L0[ch], Ev = E0[ch], R = R0[ch];
  for (int t0 = 0; t0 < T; t0 += TB) {
    if (ckpt && (t0 % CK) == 0) {
      const size_t cbase = (static_cast<size_t>(b) * nseg + t0 / CK) * 3 * H + h;
      ckpt[cbase] = L;
      ckpt[cbase + H] = Ev;
      ckpt[cbase + 2 * H] = R;
    }
    float wv[TB], pv[TB];
#pragma unroll
    for (int i = 0; i < TB; ++i) {
      const int t = t0 + i;
      wv[i] = t < T ? ld(w, base + static_cast<size_t>(t) * H) : 0.0f;
      pv[i] = t < T ? ld(p, base + static_cast<size_t>(t) * H) : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < TB; ++i) {
      const int t = t0 + i;
      if (t < T) {
        const float pe = tanhf(fabsf(wv[i] - Ev));
        const float sal = pv[i] * pe;
        Ev = k.er * Ev + (1.0f - k.er) * wv[i];
        R = k.rd * R + (1.0f - k.rd) * (1.0f - pe);
        const float eff = k.ret + (1.0f - k.ret) * k.rs * R;
        L = eff * L + (1.0f - eff) * (sal * wv[i]);
        st(out, base + static_cast<size_t>(t) * H, L);
      }
    }
  }
  LF[ch] = L;
  EF[ch] = Ev;
  RF[ch] = R;
}

// Reverse scan. Segments of CK steps are replayed forward from their fp32 checkpoint
// into registers (fully unrolled, so the per-step arrays stay in VGPRs), then walked
// backward. Gradients w.r.t. the four logits are reduced per block (fixed order).
template <typename E>
__global__ void __launch_bounds__(NT) long_bwd_kernel(int B, int T, int H, const E* w, const E* p,
                                                      Logits lg, const float* ckpt, const E* gout,
                                                      const float* gLF, const float* gEF,
                                                      const float* gRF, E* gw, E* gp, float* gL0,
                                                      float* gE0, float* gR0, float* part) {
  __shared__ float red[4][NT];
  const int64_t ch = static_cast<int64_t>(blockIdx.x) * NT + threadIdx.x;
  const bool ok = ch < static_cast<int64_t>(B) * H;
  const Coef k = load_coef(lg.p);
  float d_er = 0.f, d_rd = 0.f, d_ret = 0.f, d_rs = 0.f;
  if (ok) {
    const int64_t b = ch / H, h = ch % H;
    const size_t base = static_cast<size_t>(b) * T * H + h;
    const int nseg = (T + CK - 1) / CK;
    float gLc = gLF ? gLF[ch] : 0.0f;
    float gEc = gEF ? gEF[ch] : 0.0f;
    float gRc = gRF ? gRF[ch] : 0.0f;
    for (int sg = nseg - 1; sg >= 0; --sg) {
      const int t0 = sg * CK;
      const size_t cbase = (static_cast<size_t>(b) * nseg + sg) * 3 * H + h;
      float L = ckpt[cbase], Ev = ckpt[cbase + H], R = ckpt[cbase + 2 * H];
      float Lp[CK], Ep[CK], Rp[CK], wv[CK], pv[CK];
#pragma unroll
      for (int i = 0; i < CK; ++i) {
        const int t = t0 + i;
        wv[i] = t < T ? ld(w, base + static_cast<size_t>(t) * H) : 0.0f;
        pv[i] = t < T ? ld(p, base + static_cast<size_t>(t) * H) : 0.0f;
      }
#pragma unroll
      for (int i = 0; i < CK; ++i) {
        Lp[i] = L;
        Ep[i] = Ev;
        Rp[i] = R;
        const float pe = tanhf(fabsf(wv[i] - Ev));
        const float sal = pv[i] * pe;
        Ev = k.er * Ev + (1.0f - k.er) * wv[i];
        R = k.rd * R + (1.0f - k.rd) * (1.0f - pe);
        const float eff = k.ret + (1.0f - k.ret) * k.rs * R;
        L = eff * L + (1.0f - eff) * (sal * wv[i]);
      }
#pragma unroll
      for (int i = CK - 1; i >= 0; --i) {
        const int t = t0 + i;
        if (t < T) {
          const size_t o = base + static_cast<size_t>(t) * H;
          const float wt = wv[i], pt = pv[i];
          const float diff = wt - Ep[i];
          const float pe = tanhf(fabsf(diff));
          const float sal = pt * pe;
          const float Rcur = k.rd * Rp[i] + (1.0f - k.rd) * (1.0f - pe);
          const float eff = k.ret + (1.0f - k.ret) * k.rs * Rcur;
          const float gL = ld(gout, o) + gLc;
          const float deff = gL * (Lp[i] - sal * wt);
          const float dsal = gL * (1.0f - eff) * wt;
          float dw = gL * (1.0f - eff) * sal;
          gLc = gL * eff;
          const float dR = gRc + deff * (1.0f - k.ret) * k.rs;
          gRc = dR * k.rd;
          const float dpe = dsal * pt - dR * (1.0f - k.rd);
          st(gp, o, dsal * pe);
          const float darg = dpe * (1.0f - pe * pe) * signf_(diff);
          dw += darg;
          const float dE = gEc;
          dw += (1.0f - k.er) * dE;
          gEc = k.er * dE - darg;
          st(gw, o, dw);
          d_er += dE * (Ep[i] - wt);
          d_rd += dR * (Rp[i] - (1.0f - pe));
          d_ret += deff * (1.0f - k.rs * Rcur);
          d_rs += deff * (1.0f - k.ret) * Rcur;
        }
      }
    }
    gL0[ch] = gLc;
    gE0[ch] = gEc;
    gR0[ch] = gRc;
  }
  // d logit = d coef * sigmoid'(logit)
  red[0][threadIdx.x] = d_er * k.er * (1.0f - k.er);
  red[1][threadIdx.x] = d_rd * k.rd * (1.0f - k.rd);
  red[2][threadIdx.x] = d_ret * k.ret * (1.0f - k.ret);
  red[3][threadIdx.x] = d_rs * k.rs * (1.0f - k.rs);
  __syncthreads();
  if (threadIdx.x < 4) {
    float s = 0.0f;
    for (int i = 0; i < NT; ++i) s += red[threadIdx.x][i];
    part[static_cast<size_t>(blockIdx.x) * 4 + threadIdx.x] = s;
  }
}

static int grid_for(int64_t B, int64_t H) { return static_cast<int>((B * H + NT - 1) / NT); }

}  // namespace longmem
}  // namespace dabsn

using namespace dabsn;
using namespace dabsn::longmem;

#define DABSN_SHAPE_CHECK(B, T, H)                                                             \
  DABSN_REQUIRE((B) > 0 && (T) >= 0 && (H) > 0 && (B) * (T) * (H) < (1ll << 46) &&          \
                    (B) * (H) < (1ll << 31) && (T) < (1ll << 30),                            \
                "bad shape B=%lld T=%lld H=%lld", (long long)(B), (long long)(T), (long long)(H))

extern "C" {

int dabsn_hip_linrec_fwd(int dtype, int64_t B, int64_t T, int64_t H, const void* a, const void* g,
                         const void* y0, void* y, hipStream_t stream) {
  DABSN_SHAPE_CHECK(B, T, H);
  DABSN_REQUIRE(a && g && y0 && (y || T == 0), "linrec: null pointer");
  if (T == 0) return DABSN_OK;
  const int grid = grid_for(B, H);
  if (dtype == kBF16)
    hipLaunchKernelGGL(linrec_fwd_kernel<bf16>, dim3(grid), dim3(NT), 0, stream, (int)B, (int)T,
                       (int)H, (const bf16*)a, (const bf16*)g, (const bf16*)y0, (bf16*)y);
  else if (dtype == kF32)
    hipLaunchKernelGGL(linrec_fwd_kernel<float>, dim3(grid), dim3(NT), 0, stream, (int)B, (int)T,
                       (int)H, (const float*)a, (const float*)g, (const float*)y0, (float*)y);
  else
    DABSN_REQUIRE(false, "linrec: bad dtype %d", dtype);
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

size_t dabsn_hip_linrec_workspace_bytes(int dtype, int64_t B, int64_t T, int64_t H) {
  (void)dtype;
  return static_cast<size_t>(B) * T * H * sizeof(float);
}

int dabsn_hip_linrec_bwd(int dtype, int64_t B, int64_t T, int64_t H, const void* a, const void* g,
                         const void* y0, const void* gy, void* da, void* dg, void* dy0,
                         void* workspace, size_t workspace_bytes, hipStream_t stream) {
  DABSN_SHAPE_CHECK(B, T, H);
  DABSN_REQUIRE(a && g && y0 && gy && da && dg && dy0, "linrec backward: null pointer");
  DABSN_REQUIRE(workspace_bytes >= dabsn_hip_linrec_workspace_bytes(dtype, B, T, H),
                "linrec backward: workspace too small");
  const int grid = grid_for(B, H);
  if (dtype == kBF16)
    hipLaunchKernelGGL(linrec_bwd_kernel<bf16>, dim3(grid), dim3(NT), 0, stream, (int)B, (int)T,
                       (int)H, (const bf16*)a, (const bf16*)g, (const bf16*)y0, (const bf16*)gy,
                       (bf16*)da, (bf16*)dg, (bf16*)dy0, (float*)workspace);
  else if (dtype == kF32)
    hipLaunchKernelGGL(linrec_bwd_kernel<float>, dim3(grid), dim3(NT), 0, stream, (int)B, (int)T,
                       (int)H, (const float*)a, (const float*)g, (const float*)y0,
                       (const float*)gy, (float*)da, (float*)dg, (float*)dy0, (float*)workspace);
  else
    DABSN_REQUIRE(false, "linrec backward: bad dtype %d", dtype);
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

int dabsn_hip_long_fwd(int dtype, int64_t B, int64_t T, int64_t H, const void* w, const void* p,
                       const float* const* logits, const float* L0, const float* E0,
                       const float* R0, void* out, float* LF, float* EF, float* RF, float* ckpt,
                       hipStream_t stream) {
  DABSN_SHAPE_CHECK(B, T, H);
  DABSN_REQUIRE(w && p && logits && L0 && E0 && R0 && (out || T == 0) && LF && EF && RF,
                "long scan: null pointer");
  for (int i = 0; i < 4; ++i) DABSN_REQUIRE(logits[i], "long scan: null logit %d", i);
  Logits lg{{logits[0], logits[1], logits[2], logits[3]}};
  const int grid = grid_for(B, H);
  if (dtype == kBF16)
    hipLaunchKernelGGL(long_fwd_kernel<bf16>, dim3(grid), dim3(NT), 0, stream, (int)B, (int)T,
                       (int)H, (const bf16*)w, (const bf16*)p, lg, L0, E0, R0, (bf16*)out, LF, EF,
                       RF, ckpt);
  else if (dtype == kF32)
    hipLaunchKernelGGL(long_fwd_kernel<float>, dim3(grid), dim3(NT), 0, stream, (int)B, (int)T,
                       (int)H, (const float*)w, (const float*)p, lg, L0, E0, R0, (float*)out, LF,
                       EF, RF, ckpt);
  else
    DABSN_REQUIRE(false, "long scan: bad dtype %d", dtype);
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

int64_t dabsn_hip_long_partials(int64_t B, int64_t H) { return grid_for(B, H); }

int dabsn_hip_long_bwd(int dtype, int64_t B, int64_t T, int64_t H, const void* w, const void* p,
                       const float* const* logits, const float* ckpt, const void* gout,
                       const float* gLF, const float* gEF, const float* gRF, void* gw, void* gp,
                       float* gL0, float* gE0, float* gR0, float* part_logit, hipStream_t stream) {
  DABSN_SHAPE_CHECK(B, T, H);
  DABSN_REQUIRE(w && p && logits && (ckpt || T == 0) && (gout || T == 0) && gL0 && gE0 && gR0 &&
                    part_logit,
                "long scan backward: null pointer");
  for (int i = 0; i < 4; ++i) DABSN_REQUIRE(logits[i], "long scan backward: null logit %d", i);
  Logits lg{{logits[0], logits[1], logits[2], logits[3]}};
  const int grid = grid_for(B, H);
  if (dtype == kBF16)
    hipLaunchKernelGGL(long_bwd_kernel<bf16>, dim3(grid), dim3(NT), 0, stream, (int)B, (int)T,
                       (int)H, (const bf16*)w, (const bf16*)p, lg, ckpt, (const bf16*)gout, gLF,
                       gEF, gRF, (bf16*)gw, (bf16*)gp, gL0, gE0, gR0, part_logit);
  else if (dtype == kF32)
    hipLaunchKernelGGL(long_bwd_kernel<float>, dim3(grid), dim3(NT), 0, stream, (int)B, (int)T,
                       (int)H, (const float*)w, (const float*)p, lg, ckpt, (const float*)gout, gLF,
                       gEF, gRF, (float*)gw, (float*)gp, gL0, gE0, gR0, part_logit);
  else
    DABSN_REQUIRE(false, "long scan backward: bad dtype %d", dtype);
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

}  // extern "C"
