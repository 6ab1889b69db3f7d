// Diagonal linear recurrences: the registered dabsn::linear_recurrence pair and the
// fused recurrent long-memory scan.
//
// Reference: src/dabsn/kernels/long.py:24-98 (linear recurrence and its analytic
// reverse), long.py:492-579 (long memory as three recurrences plus glue), loop form in
// src/dabsn/read.py:625-636; CPU kernels cpu_runtime.cpp:92-143.
//
// linear_recurrence: one thread owns one (batch row, unit) channel and walks T;
// consecutive threads own consecutive units, so each time step is one coalesced row
// access, with a block of time steps loaded ahead of the dependent arithmetic.
//
// Long memory, parallel over time as well as channels. Per channel the forward is three
// chained recurrences: E_t = er E + (1-er) w (constant coefficient), R_t = rd R +
// (1-rd)(1 - pe_t) with pe_t = tanh|w_t - E_{t-1}| (constant coefficient, input known once
// E is), and L_t = eff_t L + (1 - eff_t) sal_t w_t (coefficient eff_t known once R is).
// T is cut into chunks of CK steps. For each recurrence in turn, a chunk-parallel pass
// computes every chunk's end value from a zero start (plus the product of eff_t for L),
// and a per-channel pass over the chunks turns those into the true chunk-start values
// (the checkpoint, [B][nseg][3][H] fp32, kept for the backward). A last chunk pass writes
// the output. The backward composes each chunk's affine map of the three adjoints (see the
// backward kernels below) and carries the maps across chunks in one per-channel pass; both
// of its chunk passes replay the forward recurrence over their chunk from the checkpoint
// (the same step function as the forward, so the replayed states are the forward's bits)
// instead of reading per-step states, which would be 12 bytes per (row, step, unit) written
// once and read twice.
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
      // Clamped, unconditional loads: all TB requests are issued before the first use
      // (values past T are never used).
      const size_t o = base + static_cast<size_t>(min(t0 + i, T - 1)) * H;
      av[i] = ld(a, o);
      gv[i] = ld(g, o);
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

// One step of the three recurrences from the states entering it (L, E, R), in the step
// order of long.py:492-579: pe = tanh|w - E|, then E, R, the retention eff and L advance.
// Every pass that walks the recurrence (forward, and the backward's replays) calls this,
// so the states a replay produces are bit-identical to the forward's.
__device__ __forceinline__ void advance(const Coef& k, float wt, float pt, float& L, float& Ev,
                                        float& R, float& pe, float& eff) {
  pe = tanhf(fabsf(wt - Ev));
  Ev = k.er * Ev + (1.0f - k.er) * wt;
  R = k.rd * R + (1.0f - k.rd) * (1.0f - pe);
  const float sal = pt * pe;
  eff = k.ret + (1.0f - k.ret) * k.rs * R;
  L = eff * L + (1.0f - eff) * (sal * wt);
}

// er^n for n <= CK by repeated multiplication (fixed order).
__device__ __forceinline__ float powi(float x, int n) {
  float r = 1.0f;
  for (int i = 0; i < n; ++i) r *= x;
  return r;
}

struct ChunkIdx {
  int64_t ch;       // b * H + h
  int b, h, k, t0, len, nseg;
  size_t base;      // offset of (b, 0, h) in [B, T, H]
  size_t ibase;     // offset of (b, 0, h) in the inputs w, p (batch rows ldx apart)
  size_t cbase;     // offset of (b, k, 0, h) in the checkpoint [B][nseg][3][H]
};

__device__ __forceinline__ bool chunk_idx(int B, int T, int H, int64_t ldx, ChunkIdx& c) {
  c.ch = static_cast<int64_t>(blockIdx.x) * NT + threadIdx.x;
  if (c.ch >= static_cast<int64_t>(B) * H) return false;
  c.b = static_cast<int>(c.ch / H);
  c.h = static_cast<int>(c.ch % H);
  c.k = blockIdx.y;
  c.t0 = c.k * CK;
  c.len = min(CK, T - c.t0);
  c.nseg = (T + CK - 1) / CK;
  c.base = static_cast<size_t>(c.b) * T * H + c.h;
  c.ibase = static_cast<size_t>(c.b) * ldx + c.h;
  c.cbase = (static_cast<size_t>(c.b) * c.nseg + c.k) * 3 * H + c.h;
  return true;
}

// Forward chunk pass. PHASE 0: E from 0 -> loc0 = E end. PHASE 1: E from its true start,
// R from 0 -> loc0 = R end. PHASE 2: E, R from true starts, L from 0 -> loc0 = L end,
// loc1 = prod eff. PHASE 3: all from true starts (the checkpoint) -> out.
template <typename E, int PHASE>
__global__ void __launch_bounds__(NT) long_fwd_chunk(int B, int T, int H, int64_t ldx,
                                                     const E* w, const E* p, Logits lg,
                                                     const float* ckpt, float* loc0,
                                                     float* loc1, E* out) {
  ChunkIdx c;
  if (!chunk_idx(B, T, H, ldx, c)) return;
  const Coef k = load_coef(lg.p);
  float wv[CK], pv[CK];
#pragma unroll
  for (int i = 0; i < CK; ++i) {
    // Clamped, unconditional loads so all CK requests are in flight at once (steps past
    // the chunk end are never used).
    const size_t o = c.ibase + static_cast<size_t>(c.t0 + min(i, c.len - 1)) * H;
    wv[i] = ld(w, o);
    if (PHASE >= 2) pv[i] = ld(p, o);
  }
  float Ev = PHASE >= 1 ? ckpt[c.cbase + H] : 0.0f;
  float R = PHASE >= 2 ? ckpt[c.cbase + 2 * H] : 0.0f;
  float L = PHASE >= 3 ? ckpt[c.cbase] : 0.0f;
  float prod = 1.0f;
#pragma unroll
  for (int i = 0; i < CK; ++i) {
    if (i < c.len) {
      if (PHASE == 3) {
        float pe, eff;
        advance(k, wv[i], pv[i], L, Ev, R, pe, eff);
        st(out, c.base + static_cast<size_t>(c.t0 + i) * H, L);
        continue;
      }
      const float pe = PHASE >= 1 ? tanhf(fabsf(wv[i] - Ev)) : 0.0f;
      Ev = k.er * Ev + (1.0f - k.er) * wv[i];
      if (PHASE >= 1) R = k.rd * R + (1.0f - k.rd) * (1.0f - pe);
      if (PHASE >= 2) {
        const float sal = pv[i] * pe;
        const float eff = k.ret + (1.0f - k.ret) * k.rs * R;
        L = eff * L + (1.0f - eff) * (sal * wv[i]);
        prod *= eff;
      }
    }
  }
  const size_t li = static_cast<size_t>(c.k) * B * H + c.ch;
  if (PHASE == 0) loc0[li] = Ev;
  if (PHASE == 1) loc0[li] = R;
  if (PHASE == 2) {
    loc0[li] = L;
    loc1[li] = prod;
  }
}

// A sequence of at most one chunk (T <= CK: streaming decode, short query chunks): the
// three recurrences walked once per channel from the given initial state, in the step
// order of long.py:492-579 (as phase 3 above), with the final state taken from the walk.
// The checkpoint (if given) of the one chunk is the initial state.
template <typename E>
__global__ void __launch_bounds__(NT) long_fwd_single(int B, int T, int H, int64_t ldx,
                                                      const E* w, const E* p, Logits lg,
                                                      const float* L0, const float* E0,
                                                      const float* R0, E* out, float* LF,
                                                      float* EF, float* RF, float* ckpt) {
  const int64_t ch = static_cast<int64_t>(blockIdx.x) * NT + threadIdx.x;
  if (ch >= static_cast<int64_t>(B) * H) return;
  const Coef k = load_coef(lg.p);
  const int b = static_cast<int>(ch / H), h = static_cast<int>(ch % H);
  const size_t base = static_cast<size_t>(b) * T * H + h;
  const size_t ibase = static_cast<size_t>(b) * ldx + h;
  float L = L0[ch], Ev = E0[ch], R = R0[ch];
  if (ckpt) {
    float* cp = ckpt + static_cast<size_t>(b) * 3 * H + h;
    cp[0] = L;
    cp[H] = Ev;
    cp[2 * H] = R;
  }
  for (int t = 0; t < T; ++t) {
    const size_t o = base + static_cast<size_t>(t) * H, io = ibase + static_cast<size_t>(t) * H;
    float pe, eff;
    advance(k, ld(w, io), ld(p, io), L, Ev, R, pe, eff);
    st(out, o, L);
  }
  LF[ch] = L;
  EF[ch] = Ev;
  RF[ch] = R;
}

// Per-channel pass over chunks for state S (0 = L, 1 = E, 2 = R): the chunk-start value
// goes to the checkpoint slot S; the state after the last chunk to `fin`.
// x_{k+1} = a_k x_k + loc[k] with a_k = prod[k] (L) or coef^len_k (E: er, R: rd).
template <int S>
__global__ void __launch_bounds__(NT) long_fwd_carry(int B, int T, int H, Logits lg,
                                                     const float* x0, const float* loc,
                                                     const float* prod, float* ckpt, float* fin) {
  const int64_t ch = static_cast<int64_t>(blockIdx.x) * NT + threadIdx.x;
  if (ch >= static_cast<int64_t>(B) * H) return;
  const Coef k = load_coef(lg.p);
  const int b = static_cast<int>(ch / H), h = static_cast<int>(ch % H);
  const int nseg = (T + CK - 1) / CK;
  const float coef = S == 1 ? k.er : k.rd;
  const float a_full = powi(coef, CK);
  float x = x0[ch];
  for (int kk = 0; kk < nseg; ++kk) {
    ckpt[(static_cast<size_t>(b) * nseg + kk) * 3 * H + S * H + h] = x;
    const size_t li = static_cast<size_t>(kk) * B * H + ch;
    const int len = min(CK, T - kk * CK);
    const float a = S == 0 ? prod[li] : (len == CK ? a_full : powi(coef, len));
    x = a * x + loc[li];
  }
  fin[ch] = x;
}

// Backward. Walking time in reverse, one step maps the carried adjoints x = (gL, gR, gE)
// (coming from step t + 1) to the ones leaving step t, affinely:
//   gL' = eff (gL + g_t)
//   gR' = rd gR + rd k a (gL + g_t)                          k = (1 - ret) rs, a = L_{t-1} - sal w
//   gE' = er gE + s (1 - rd) gR + c (gL + g_t)               s = (1 - pe^2) sign(w - E_{t-1})
//                                                              c = s ((1 - rd) k a - (1 - eff) w p)
// i.e. x' = M_t (x + g_t e0) with M_t lower triangular. Over a chunk, x_out = A x_in + v
// with A = M_0 ... M_{len-1} and v = sum_i (M_0 ... M_{i-1}) M_i g_i e0, both accumulated
// in forward time order, so one forward pass over each chunk yields its map; a per-channel pass over the chunks then gives the exact
// adjoints entering each chunk, and a last pass walks each chunk backward with those
// adjoints to produce gw, gp and the logit partials. Both chunk passes replay the forward
// recurrence over their chunk from its checkpoint for the values around each step.

// Per-step coefficients of M_t from the forward values around step t.
struct StepMap {
  float m00, m10, m11, m20, m21, m22;
};

__device__ __forceinline__ StepMap step_map(const Coef& k, float wt, float pt, float Lp, float Ep,
                                            float pe, float eff) {
  const float kap = (1.0f - k.ret) * k.rs;
  const float sal = pt * pe;
  const float a = Lp - sal * wt;
  const float sgn = (1.0f - pe * pe) * signf_(wt - Ep);
  StepMap m;
  m.m00 = eff;
  m.m10 = k.rd * kap * a;
  m.m11 = k.rd;
  m.m20 = sgn * ((1.0f - k.rd) * kap * a - (1.0f - eff) * wt * pt);
  m.m21 = sgn * (1.0f - k.rd);
  m.m22 = k.er;
  return m;
}

// Chunk maps: A (lower triangular, 6 entries) and v (3 entries), stored component-major
// in `maps` [9][nseg][B*H]. The forward values around each step are replayed from the
// chunk's checkpoint.
template <typename E>
__global__ void __launch_bounds__(NT) long_bwd_map(int B, int T, int H, int64_t ldx,
                                                   const E* w, const E* p, Logits lg,
                                                   const float* ckpt, const E* gout,
                                                   float* maps) {
  ChunkIdx c;
  if (!chunk_idx(B, T, H, ldx, c)) return;
  const Coef k = load_coef(lg.p);
  float wv[CK], pv[CK], gv[CK];
#pragma unroll
  for (int i = 0; i < CK; ++i) {
    // Clamped, unconditional loads so all requests are in flight at once (steps past the
    // chunk end are never used).
    const size_t t = static_cast<size_t>(c.t0 + min(i, c.len - 1)) * H;
    wv[i] = ld(w, c.ibase + t);
    pv[i] = ld(p, c.ibase + t);
    gv[i] = ld(gout, c.base + t);
  }
  float L = ckpt[c.cbase], Ev = ckpt[c.cbase + H], R = ckpt[c.cbase + 2 * H];
  float p00 = 1.f, p10 = 0.f, p11 = 1.f, p20 = 0.f, p21 = 0.f, p22 = 1.f;
  float v0 = 0.f, v1 = 0.f, v2 = 0.f;
#pragma unroll
  for (int i = 0; i < CK; ++i) {
    if (i < c.len) {
      const float Lp = L, Ep = Ev;
      float pe, eff;
      advance(k, wv[i], pv[i], L, Ev, R, pe, eff);
      const StepMap m = step_map(k, wv[i], pv[i], Lp, Ep, pe, eff);
      // v += P (M_i g_i e0)
      const float u0 = m.m00 * gv[i], u1 = m.m10 * gv[i], u2 = m.m20 * gv[i];
      v0 += p00 * u0;
      v1 += p10 * u0 + p11 * u1;
      v2 += p20 * u0 + p21 * u1 + p22 * u2;
      // P = P M_i
      const float n20 = p20 * m.m00 + p21 * m.m10 + p22 * m.m20;
      const float n21 = p21 * m.m11 + p22 * m.m21;
      const float n10 = p10 * m.m00 + p11 * m.m10;
      p00 *= m.m00;
      p10 = n10;
      p11 *= m.m11;
      p20 = n20;
      p21 = n21;
      p22 *= m.m22;
    }
  }
  const size_t stride = static_cast<size_t>(c.nseg) * B * H;
  const size_t li = static_cast<size_t>(c.k) * B * H + c.ch;
  maps[li] = p00;
  maps[li + stride] = p10;
  maps[li + 2 * stride] = p11;
  maps[li + 3 * stride] = p20;
  maps[li + 4 * stride] = p21;
  maps[li + 5 * stride] = p22;
  maps[li + 6 * stride] = v0;
  maps[li + 7 * stride] = v1;
  maps[li + 8 * stride] = v2;
}

// Per-channel reverse pass over the chunk maps: x_in(k) = adjoints entering chunk k (from
// chunk k + 1), written over the map's first three components; x leaving chunk 0 goes to
// gL0, gR0, gE0.
__global__ void __launch_bounds__(NT) long_bwd_carry(int B, int T, int H, const float* gLF,
                                                     const float* gRF, const float* gEF,
                                                     float* maps, float* gL0, float* gR0,
                                                     float* gE0) {
  const int64_t ch = static_cast<int64_t>(blockIdx.x) * NT + threadIdx.x;
  if (ch >= static_cast<int64_t>(B) * H) return;
  const int nseg = (T + CK - 1) / CK;
  const size_t stride = static_cast<size_t>(nseg) * B * H;
  float x0 = gLF ? gLF[ch] : 0.0f, x1 = gRF ? gRF[ch] : 0.0f, x2 = gEF ? gEF[ch] : 0.0f;
  for (int kk = nseg - 1; kk >= 0; --kk) {
    float* m = maps + static_cast<size_t>(kk) * B * H + ch;
    const float a00 = m[0], a10 = m[stride], a11 = m[2 * stride], a20 = m[3 * stride],
                a21 = m[4 * stride], a22 = m[5 * stride], v0 = m[6 * stride],
                v1 = m[7 * stride], v2 = m[8 * stride];
    m[0] = x0;
    m[stride] = x1;
    m[2 * stride] = x2;
    const float y0 = a00 * x0 + v0;
    const float y1 = a10 * x0 + a11 * x1 + v1;
    const float y2 = a20 * x0 + a21 * x1 + a22 * x2 + v2;
    x0 = y0;
    x1 = y1;
    x2 = y2;
  }
  gL0[ch] = x0;
  gR0[ch] = x1;
  gE0[ch] = x2;
}

// Final pass: walk the chunk backward from the exact entering adjoints (maps components
// 0..2), in sub-blocks of SB steps from the last: each sub-block replays its forward steps
// from its entering states (found by one replay of the chunk from its checkpoint) and keeps
// them in registers for its backward walk, so a thread holds SB steps of states instead of
// CK (the replays call `advance`, so every state equals the forward's bit for bit). Writes
// gw, gp (batch rows ldo apart) and reduces the logit gradients per block (fixed order).
// ACC: gw += the gradient rounded to E, the sum formed in fp32 and rounded once (an add of
// the rounded gradient into an existing gradient buffer).
constexpr int SB = 8;
static_assert(CK % SB == 0, "whole sub-blocks per chunk");

template <typename E, bool ACC>
__global__ void __launch_bounds__(NT) long_bwd_final(int B, int T, int H, int64_t ldx,
                                                     int64_t ldo, const E* w, const E* p,
                                                     Logits lg, const float* ckpt,
                                                     const E* gout, const float* maps, E* gw,
                                                     E* gp, float* part) {
  constexpr int NSB = CK / SB;
  __shared__ float red[4][NT];
  ChunkIdx c;
  const bool ok = chunk_idx(B, T, H, ldx, c);
  const Coef k = load_coef(lg.p);
  float d_er = 0.f, d_rd = 0.f, d_ret = 0.f, d_rs = 0.f;
  if (ok) {
    const size_t obase = static_cast<size_t>(c.b) * ldo + c.h;
    float wv[CK], pv[CK];
#pragma unroll
    for (int i = 0; i < CK; ++i) {
      // Clamped, unconditional loads (steps past the chunk end are never used).
      const size_t t = static_cast<size_t>(c.t0 + min(i, c.len - 1)) * H;
      wv[i] = ld(w, c.ibase + t);
      pv[i] = ld(p, c.ibase + t);
    }
    float Ls[NSB], Es[NSB], Rs[NSB];
    {
      float L = ckpt[c.cbase], Ev = ckpt[c.cbase + H], R = ckpt[c.cbase + 2 * H];
#pragma unroll
      for (int i = 0; i < CK; ++i) {
        if (i % SB == 0) {
          Ls[i / SB] = L;
          Es[i / SB] = Ev;
          Rs[i / SB] = R;
        }
        if (i < c.len) {
          float pe, eff;
          advance(k, wv[i], pv[i], L, Ev, R, pe, eff);
        }
      }
    }
    const size_t stride = static_cast<size_t>(c.nseg) * B * H;
    const size_t li = static_cast<size_t>(c.k) * B * H + c.ch;
    float gLc = maps[li], gRc = maps[li + stride], gEc = maps[li + 2 * stride];
#pragma unroll
    for (int sb = NSB - 1; sb >= 0; --sb) {
      float gv[SB], sv[ACC ? SB : 1], Lv[SB], Ev[SB], Rv[SB];
#pragma unroll
      for (int j = 0; j < SB; ++j) {
        const size_t t = static_cast<size_t>(c.t0 + min(sb * SB + j, c.len - 1)) * H;
        gv[j] = ld(gout, c.base + t);
        if constexpr (ACC) sv[j] = ld(gw, obase + t);
      }
      float L = Ls[sb], Es_ = Es[sb], R = Rs[sb];
#pragma unroll
      for (int j = 0; j < SB; ++j) {
        const int i = sb * SB + j;
        Lv[j] = L;
        Ev[j] = Es_;
        Rv[j] = R;
        if (i < c.len) {
          float pe, eff;
          advance(k, wv[i], pv[i], L, Es_, R, pe, eff);
        }
      }
#pragma unroll
      for (int j = SB - 1; j >= 0; --j) {
        const int i = sb * SB + j;
        if (i < c.len) {
          const float wt = wv[i], pt = pv[i];
          const float diff = wt - Ev[j];
          const float pe = tanhf(fabsf(diff));
          const float sal = pt * pe;
          const float Rcur = k.rd * Rv[j] + (1.0f - k.rd) * (1.0f - pe);
          const float eff = k.ret + (1.0f - k.ret) * k.rs * Rcur;
          const float gL = gv[j] + gLc;
          const float deff = gL * (Lv[j] - sal * wt);
          const float dsal = gL * (1.0f - eff) * wt;
          gLc = gL * eff;
          const float dR = gRc + deff * (1.0f - k.ret) * k.rs;
          gRc = dR * k.rd;
          const float dpe = dsal * pt - dR * (1.0f - k.rd);
          const float darg = dpe * (1.0f - pe * pe) * signf_(diff);
          const float dE = gEc;
          gEc = k.er * dE - darg;
          const size_t o = obase + static_cast<size_t>(c.t0 + i) * H;
          st(gp, o, dsal * pe);
          const float gwv = gL * (1.0f - eff) * sal + darg + (1.0f - k.er) * dE;
          if constexpr (ACC)
            st(gw, o, sv[j] + round_to<E>(gwv));
          else
            st(gw, o, gwv);
          d_er += dE * (Ev[j] - wt);
          d_rd += dR * (Rv[j] - (1.0f - pe));
          d_ret += deff * (1.0f - k.rs * Rcur);
          d_rs += deff * (1.0f - k.ret) * Rcur;
        }
      }
    }
  }
  // d logit = d coef * sigmoid'(logit), reduced per block in a fixed order.
  red[0][threadIdx.x] = d_er * k.er * (1.0f - k.er);
  red[1][threadIdx.x] = d_rd * k.rd * (1.0f - k.rd);
  red[2][threadIdx.x] = d_ret * k.ret * (1.0f - k.ret);
  red[3][threadIdx.x] = d_rs * k.rs * (1.0f - k.rs);
  __syncthreads();
  if (threadIdx.x < 4) {
    float s = 0.0f;
    for (int i = 0; i < NT; ++i) s += red[threadIdx.x][i];
    part[(static_cast<size_t>(blockIdx.y) * gridDim.x + blockIdx.x) * 4 + threadIdx.x] = s;
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

template <typename E>
static int long_fwd_impl(int B, int T, int H, int64_t ldx, const E* w, const E* p, Logits lg,
                         const float* L0,
                         const float* E0, const float* R0, E* out, float* LF, float* EF, float* RF,
                         float* keep, float* ws, hipStream_t stream) {
  const int gx = grid_for(B, H);
  const int nseg = (T + CK - 1) / CK;
  float* loc0 = ws;
  float* loc1 = ws + static_cast<size_t>(nseg) * B * H;
  // [B][nseg][3][H]: the caller's buffer when it keeps the checkpoint, else the workspace.
  float* ckpt = keep ? keep : ws + 2 * static_cast<size_t>(nseg) * B * H;
  const dim3 cg(gx, nseg), blk(NT);
  if (nseg == 1) {  // one chunk: a single walk, no chunk-parallel passes
    hipLaunchKernelGGL((long_fwd_single<E>), dim3(gx), blk, 0, stream, B, T, H, ldx, w, p, lg, L0, E0,
                       R0, out, LF, EF, RF, keep);
    DABSN_HIP_CHECK(hipGetLastError());
    return DABSN_OK;
  }
  if (nseg > 0) hipLaunchKernelGGL((long_fwd_chunk<E, 0>), cg, blk, 0, stream, B, T, H, ldx, w, p, lg, ckpt, loc0, loc1, out);
  hipLaunchKernelGGL(long_fwd_carry<1>, dim3(gx), blk, 0, stream, B, T, H, lg, E0, loc0, loc1, ckpt, EF);
  if (nseg > 0) hipLaunchKernelGGL((long_fwd_chunk<E, 1>), cg, blk, 0, stream, B, T, H, ldx, w, p, lg, ckpt, loc0, loc1, out);
  hipLaunchKernelGGL(long_fwd_carry<2>, dim3(gx), blk, 0, stream, B, T, H, lg, R0, loc0, loc1, ckpt, RF);
  if (nseg > 0) hipLaunchKernelGGL((long_fwd_chunk<E, 2>), cg, blk, 0, stream, B, T, H, ldx, w, p, lg, ckpt, loc0, loc1, out);
  hipLaunchKernelGGL(long_fwd_carry<0>, dim3(gx), blk, 0, stream, B, T, H, lg, L0, loc0, loc1, ckpt, LF);
  if (nseg > 0) hipLaunchKernelGGL((long_fwd_chunk<E, 3>), cg, blk, 0, stream, B, T, H, ldx, w, p, lg, ckpt, loc0, loc1, out);
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

template <typename E>
static int long_bwd_impl(int B, int T, int H, int64_t ldx, const E* w, const E* p, Logits lg,
                         const float* ckpt, const E* gout, const float* gLF, const float* gEF,
                         const float* gRF, E* gw, E* gp, int64_t ldo, bool acc, float* gL0,
                         float* gE0, float* gR0, float* part, float* ws, hipStream_t stream) {
  const int gx = grid_for(B, H);
  const int nseg = (T + CK - 1) / CK;
  const dim3 cg(gx, nseg), blk(NT);
  if (nseg > 0)
    hipLaunchKernelGGL(long_bwd_map<E>, cg, blk, 0, stream, B, T, H, ldx, w, p, lg, ckpt, gout,
                       ws);
  hipLaunchKernelGGL(long_bwd_carry, dim3(gx), blk, 0, stream, B, T, H, gLF, gRF, gEF, ws, gL0,
                     gR0, gE0);
  auto final_pass = acc ? long_bwd_final<E, true> : long_bwd_final<E, false>;
  if (nseg > 0)
    hipLaunchKernelGGL(final_pass, cg, blk, 0, stream, B, T, H, ldx, ldo, w, p, lg, ckpt, gout,
                       ws, gw, gp, part);
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

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

size_t dabsn_hip_long_workspace_bytes(int64_t B, int64_t T, int64_t H, int backward) {
  const int64_t nseg = (T + CK - 1) / CK;
  // forward: two chunk-end arrays + the chunk-start checkpoint (3 per chunk; used when the
  // caller passes no checkpoint buffer of its own);
  // backward: the 9-component chunk maps.
  return static_cast<size_t>(backward ? 9 : 5) * static_cast<size_t>(nseg) * B * H * sizeof(float);
}

// Batch stride of [B, T, H] operands: ldx elements (0: T H, the contiguous layout); at least
// T H, so a time window of longer [B, T', H] tapes can be passed in place; -1 if invalid.
static int64_t batch_stride(int64_t B, int64_t T, int64_t H, int64_t ldx) {
  if (ldx == 0) return T * H;
  if (ldx < T * H || (B - 1) * ldx + T * H >= (1ll << 46)) return -1;
  return ldx;
}

int dabsn_hip_long_fwd(int dtype, int64_t B, int64_t T, int64_t H, int64_t ldx, const void* w,
                       const void* p, const float* const* logits, const float* L0,
                       const float* E0, const float* R0, void* out, float* LF, float* EF,
                       float* RF, float* ckpt, void* workspace, size_t workspace_bytes,
                       hipStream_t stream) {
  DABSN_SHAPE_CHECK(B, T, H);
  const int64_t lx = batch_stride(B, T, H, ldx);
  DABSN_REQUIRE(lx >= 0, "long scan: bad input batch stride %lld for T=%lld H=%lld",
                (long long)ldx, (long long)T, (long long)H);
  DABSN_REQUIRE(w && p && logits && L0 && E0 && R0 && (out || T == 0) && LF && EF && RF &&
                    (workspace || T == 0),
                "long scan: null pointer");
  for (int i = 0; i < 4; ++i) DABSN_REQUIRE(logits[i], "long scan: null logit %d", i);
  DABSN_REQUIRE(workspace_bytes >= dabsn_hip_long_workspace_bytes(B, T, H, 0),
                "long scan: workspace %zu B < required %zu B", workspace_bytes,
                dabsn_hip_long_workspace_bytes(B, T, H, 0));
  DABSN_REQUIRE((T + CK - 1) / CK < 65536, "long scan: T too long");
  Logits lg{{logits[0], logits[1], logits[2], logits[3]}};
  if (dtype == kBF16)
    return long_fwd_impl<bf16>((int)B, (int)T, (int)H, lx, (const bf16*)w, (const bf16*)p, lg,
                               L0, E0, R0, (bf16*)out, LF, EF, RF, ckpt, (float*)workspace,
                               stream);
  if (dtype == kF32)
    return long_fwd_impl<float>((int)B, (int)T, (int)H, lx, (const float*)w, (const float*)p, lg,
                                L0, E0, R0, (float*)out, LF, EF, RF, ckpt, (float*)workspace,
                                stream);
  DABSN_REQUIRE(false, "long scan: bad dtype %d", dtype);
  return DABSN_OK;
}

int64_t dabsn_hip_long_partials(int64_t B, int64_t T, int64_t H) {
  return static_cast<int64_t>(grid_for(B, H)) * ((T + CK - 1) / CK);
}

int dabsn_hip_long_bwd(int dtype, int64_t B, int64_t T, int64_t H, int64_t ldx, const void* w,
                       const void* p, const float* const* logits, const float* ckpt,
                       const void* gout, const float* gLF, const float* gEF, const float* gRF,
                       void* gw, void* gp, int64_t ldo, int gw_accumulate, float* gL0,
                       float* gE0, float* gR0, float* part_logit, void* workspace,
                       size_t workspace_bytes, hipStream_t stream) {
  DABSN_SHAPE_CHECK(B, T, H);
  const int64_t lx = batch_stride(B, T, H, ldx), lo = batch_stride(B, T, H, ldo);
  DABSN_REQUIRE(lx >= 0 && lo >= 0,
                "long scan backward: bad batch stride (inputs %lld, outputs %lld) for T=%lld "
                "H=%lld", (long long)ldx, (long long)ldo, (long long)T, (long long)H);
  DABSN_REQUIRE(w && p && logits && (ckpt || T == 0) && (gout || T == 0) && gL0 && gE0 && gR0 &&
                    (part_logit || T == 0) && (workspace || T == 0) && ((gw && gp) || T == 0),
                "long scan backward: null pointer");
  for (int i = 0; i < 4; ++i) DABSN_REQUIRE(logits[i], "long scan backward: null logit %d", i);
  DABSN_REQUIRE(workspace_bytes >= dabsn_hip_long_workspace_bytes(B, T, H, 1),
                "long scan backward: workspace %zu B < required %zu B", workspace_bytes,
                dabsn_hip_long_workspace_bytes(B, T, H, 1));
  DABSN_REQUIRE((T + CK - 1) / CK < 65536, "long scan backward: T too long");
  Logits lg{{logits[0], logits[1], logits[2], logits[3]}};
  if (dtype == kBF16)
    return long_bwd_impl<bf16>((int)B, (int)T, (int)H, lx, (const bf16*)w, (const bf16*)p, lg,
                               ckpt, (const bf16*)gout, gLF, gEF, gRF, (bf16*)gw, (bf16*)gp, lo,
                               gw_accumulate != 0, gL0, gE0, gR0, part_logit, (float*)workspace,
                               stream);
  if (dtype == kF32)
    return long_bwd_impl<float>((int)B, (int)T, (int)H, lx, (const float*)w, (const float*)p, lg,
                                ckpt, (const float*)gout, gLF, gEF, gRF, (float*)gw, (float*)gp,
                                lo, gw_accumulate != 0, gL0, gE0, gR0, part_logit,
                                (float*)workspace, stream);
  DABSN_REQUIRE(false, "long scan backward: bad dtype %d", dtype);
  return DABSN_OK;
}

}  // extern "C"
