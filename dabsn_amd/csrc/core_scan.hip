// DABSN core recurrence: forward and reverse scans as persistent cooperative kernels.
//
// Math: reference src/dabsn/core.py:171-221 (forward) and the registered reverse
// recurrence src/dabsn/kernels/batched_runtime.py:299-466 (backward).
//
// Decomposition (one step = one time index):
//   * Channels are split into tiles of CH units; batch rows are split into groups of 16
//     (the MFMA N dimension). One workgroup owns (channel tile, batch group) and keeps
//     its slice of the recurrent matrix [Ug; A] in VGPRs for the whole scan.
//   * Every step needs the full y_t (forward) or the full [dgate; dexpr] vector
//     (backward) of its batch group. Workgroups publish their slice into a small
//     exchange buffer laid out exactly as the MFMA B operand, then meet at a
//     device-wide step barrier (a monotonic counter). Exchange traffic and the
//     counter use device-coherent (sc1) accesses so no L2 writeback/invalidate is
//     needed between XCDs.
//   * The recurrent product runs on v_mfma_f32_16x16x32_bf16 (bf16) or
//     v_mfma_f32_16x16x4_f32 (fp32) with K split across the 4 waves; partial tiles
//     are reduced through LDS in a fixed order (deterministic).
//   * State (b, e, c) and the per-unit parameters live in registers of the thread that
//     owns a (unit, batch row) pair; tapes are written once per step.
//   * Barrier waits are bounded: a wait that exceeds kSpinLimit polls sets the error
//     word and every workgroup exits.
#include "../../include/dabsn_hip.h"
#include "capi.hpp"
#include "common.hpp"

namespace dabsn {
namespace core {

constexpr int NW = 4;         // waves per workgroup
constexpr int NT = NW * 64;   // threads per workgroup
constexpr int NB = 16;        // batch rows per group (MFMA N)

template <typename E>
struct Mf;
template <>
struct Mf<bf16> {
  static constexpr int KSTEP = 32;
  static constexpr int UNIT = 16;  // bytes per lane per k-step in the exchange buffer
  using Reg = bf16x8;
  __device__ static f32x4 mma(Reg a, Reg b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  __device__ static Reg load_x(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, kCoherent);
    return __builtin_bit_cast(Reg, v);
  }
};
template <>
struct Mf<float> {
  static constexpr int KSTEP = 4;
  static constexpr int UNIT = 4;
  using Reg = float;
  __device__ static f32x4 mma(Reg a, Reg b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
  __device__ static Reg load_x(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    uint32_t v = __builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(off), 0, kCoherent);
    return __builtin_bit_cast(float, v);
  }
};

// Element offset of (k, n) inside one exchange slot, in units of E.
template <typename E>
__device__ __forceinline__ uint32_t xoff(int k, int n);
template <>
__device__ __forceinline__ uint32_t xoff<bf16>(int k, int n) {
  return static_cast<uint32_t>((((k >> 5) * 64 + ((k & 31) >> 3) * 16 + n) * 8) + (k & 7));
}
template <>
__device__ __forceinline__ uint32_t xoff<float>(int k, int n) {
  return static_cast<uint32_t>((k >> 2) * 64 + (k & 3) * 16 + n);
}

// Workspace layout: [0,4) error word, [4, 4 + 4*nbg) step counters, exchange slots
// from kXOff (2 slots per batch group).
constexpr size_t kXOff = 4096;

struct Params {
  const float* vec[16];
  const float* scal[3];
};

enum {
  V_BETA = 0, V_LOG_KAPPA, V_LOGIT_RECOVER, V_KS, V_KY, V_KB, V_KN, V_KBIAS,
  V_RS, V_RY, V_RB, V_RN, V_RBIAS, V_LOGIT_CDECAY, V_KC, V_RC
};

struct UnitParams {
  float beta, kappa, recover, ks, ky, kb, kn, kbias, rs, ry, rb, rn, rbias, decay, kc, rc;
  float lk_sig;  // sigmoid(log_kappa), used by the log_kappa gradient
};

__device__ __forceinline__ UnitParams load_unit(const Params& P, int c, bool ok) {
  UnitParams u;
  auto g = [&](int k) { return ok ? P.vec[k][c] : 0.0f; };
  u.beta = g(V_BETA);
  const float lk = g(V_LOG_KAPPA);
  u.kappa = softplusf_(lk);
  u.lk_sig = sigmoidf_(lk);
  u.recover = sigmoidf_(g(V_LOGIT_RECOVER));
  u.ks = g(V_KS); u.ky = g(V_KY); u.kb = g(V_KB); u.kn = g(V_KN); u.kbias = g(V_KBIAS);
  u.rs = g(V_RS); u.ry = g(V_RY); u.rb = g(V_RB); u.rn = g(V_RN); u.rbias = g(V_RBIAS);
  u.decay = sigmoidf_(g(V_LOGIT_CDECAY));
  u.kc = g(V_KC); u.rc = g(V_RC);
  return u;
}

// Thread 0 of a workgroup waits until the step counter reaches `target`.
// Returns false (and raises the error word) if the wait exceeded the spin bound.
__device__ __forceinline__ bool wait_counter(uint32_t* counter, uint32_t target, uint32_t* err) {
  uint32_t spins = 0;
  while (__hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
    if ((++spins & 1023u) == 0u) {
      if (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) return false;
      if (spins > kSpinLimit) {
        __hip_atomic_fetch_or(err, kErrBarrierTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
      }
    }
    __builtin_amdgcn_s_sleep(1);
  }
  return true;
}

__device__ __forceinline__ void arrive(uint32_t* counter) {
  __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wait for every outstanding vector memory operation of this wave (the exchange stores
// must be complete before the workgroup announces them on the counter).
__device__ __forceinline__ void drain_vmem() { __builtin_amdgcn_s_waitcnt(0); }

// Publishes `nvals` values per (unit, batch) pair into slot `xs` of the exchange
// buffer at k = kbase[i] + cl. bf16 stages through LDS so each lane stores one 16-byte
// unit (8 consecutive k for one batch column); fp32 stores one word per value.
template <typename E, int CH, int NV>
__device__ __forceinline__ void publish(__amdgpu_buffer_rsrc_t xr, uint32_t slot_bytes, int xs,
                                        const int (&kbase)[NV], const float (&vals)[NV],
                                        bool is_pair, int cl, int bl, bf16 (*stage)[NB][CH]) {
  const int tid = threadIdx.x;
  if constexpr (is_bf16<E>::value) {
    if (is_pair) {
#pragma unroll
      for (int i = 0; i < NV; ++i) stage[i][bl][cl] = f2bf(vals[i]);
    }
    __syncthreads();
    constexpr int GROUPS = CH / 8;
    constexpr int UNITS = NV * GROUPS * NB;
    for (int u = tid; u < UNITS; u += NT) {
      const int i = u / (GROUPS * NB);
      const int rem = u % (GROUPS * NB);
      const int g = rem / NB, n = rem % NB;
      const int k0 = kbase[i] + g * 8;
      uint32_t w[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        w[q] = static_cast<uint32_t>(stage[i][n][g * 8 + 2 * q]) |
               (static_cast<uint32_t>(stage[i][n][g * 8 + 2 * q + 1]) << 16);
      u32x4 v = {w[0], w[1], w[2], w[3]};
      const uint32_t off = xs * slot_bytes + xoff<bf16>(k0, n) * 2u;
      __builtin_amdgcn_raw_buffer_store_b128(v, xr, static_cast<int>(off), 0, kCoherent);
    }
  } else {
    (void)stage;
    if (is_pair) {
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const uint32_t off = xs * slot_bytes + xoff<float>(kbase[i] + cl, bl) * 4u;
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, vals[i]), xr,
                                              static_cast<int>(off), 0, kCoherent);
      }
    }
  }
  drain_vmem();
  __syncthreads();
}

// ---------------------------------------------------------------------------
// Forward scan.
// ---------------------------------------------------------------------------
template <typename E>
struct FwdArgs {
  int B, T, H, nct;
  const E* Wx;
  const E* Wgx;
  const E* GA;  // [2H][H]: Ug rows then A rows
  Params P;
  const float* b0;
  const float* e0;
  const float* c0;
  E* U;
  E* nov;
  E* pl;
  E* ay;
  E* wr;
  E* et;
  E* ctp;
  E* st;
  float* bF;
  float* eF;
  float* cF;
  uint8_t* ws;
  uint32_t slot_bytes;
};

// The reverse scan reads the hard-sigmoid gradient mask (0 < s < 1) back from the gate
// tape. A gate strictly inside (0, 1) whose nearest bf16 is exactly 0 or 1 is stored one
// ulp inside instead, so the mask survives the tape's rounding (the stored value is
// still within one bf16 ulp of the true gate).
template <typename E>
__device__ __forceinline__ float gate_tape_value(float s) {
  if constexpr (is_bf16<E>::value) {
    const float r = bf2f(f2bf(s));
    if (s > 0.0f && s < 1.0f && r >= 1.0f) return 0.99609375f;  // largest bf16 below 1
    if (s > 0.0f && s < 1.0f && r <= 0.0f) return bf2f(static_cast<bf16>(1));  // smallest positive
    return s;
  } else {
    return s;
  }
}

__device__ __forceinline__ void tile_of(int nct, int& ct, int& bg) {
  // Consecutive channel tiles go to the same XCD (workgroups are dealt round-robin over
  // the 8 XCDs), so the tape rows a step writes are merged in one L2.
  const int bid = blockIdx.x;
  bg = bid / nct;
  const int i = bid % nct;
  ct = (nct % 8 == 0) ? (i % 8) * (nct / 8) + i / 8 : i;
}

template <typename E, int CH, int KSTEPS>
__global__ void __launch_bounds__(NT, 1) core_fwd_kernel(FwdArgs<E> a) {
  using M = Mf<E>;
  constexpr int KSTEP = M::KSTEP;
  constexpr int KW = KSTEPS * KSTEP;
  constexpr int ROWS = 2 * CH;
  constexpr int MT = ROWS / 16;
  constexpr int PAIRS = CH * NB;
  static_assert(ROWS % 16 == 0, "CH must be a multiple of 8");
  static_assert(PAIRS <= NT, "one thread per (unit, batch) pair");

  __shared__ float red[NW][MT][16][16];
  __shared__ bf16 stage[1][NB][CH];
  __shared__ int s_abort;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int ct, bg;
  tile_of(a.nct, ct, bg);
  const int H = a.H, T = a.T, B = a.B;
  const uint32_t nct = static_cast<uint32_t>(a.nct);
  uint32_t* err = reinterpret_cast<uint32_t*>(a.ws);
  uint32_t* counter = reinterpret_cast<uint32_t*>(a.ws + 4) + bg;
  uint8_t* xbase = a.ws + kXOff + static_cast<size_t>(bg) * 2 * a.slot_bytes;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(xbase, 2 * a.slot_bytes);
  if (tid == 0) s_abort = 0;

  // Recurrent weights for this wave's K range, as MFMA A operands.
  typename M::Reg wreg[MT][KSTEPS];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int r = mt * 16 + (lane & 15);
    const int c = ct * CH + (r < CH ? r : r - CH);
    const size_t grow = static_cast<size_t>(r < CH ? c : H + c) * H;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      const int k0 = wave * KW + s * KSTEP;
      if constexpr (is_bf16<E>::value) {
        bf16 v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int k = k0 + (lane >> 4) * 8 + e;
          v[e] = (c < H && k < H) ? a.GA[grow + k] : static_cast<bf16>(0);
        }
        wreg[mt][s] = __builtin_bit_cast(bf16x8, v);
      } else {
        const int k = k0 + (lane >> 4);
        wreg[mt][s] = (c < H && k < H) ? a.GA[grow + k] : 0.0f;
      }
    }
  }

  const bool is_pair = tid < PAIRS;
  const int cl = tid % CH, bl = tid / CH;
  const int c = ct * CH + cl, b = bg * NB + bl;
  const bool act = is_pair && c < H && b < B;
  const UnitParams up = load_unit(a.P, c, is_pair && c < H);
  const float gate_alpha = sigmoidf_(a.P.scal[0][0]);
  const float lam = softplusf_(a.P.scal[1][0]);
  const float c_sup = sigmoidf_(a.P.scal[2][0]);
  float sb = act ? a.b0[static_cast<size_t>(b) * H + c] : 0.0f;
  float se = act ? a.e0[static_cast<size_t>(b) * H + c] : 0.0f;
  float sc = act ? a.c0[static_cast<size_t>(b) * H + c] : 0.0f;
  const size_t row0 = static_cast<size_t>(b) * T;

  float ycur = (act && T > 0) ? tanhf(ld(a.Wx, row0 * H + c) + sb) : 0.0f;
  const int kb_y[1] = {ct * CH};
  if (T > 0) {
    const float v[1] = {ycur};
    publish<E, CH, 1>(xr, a.slot_bytes, 0, kb_y, v, is_pair, cl, bl, stage);
    if (tid == 0) arrive(counter);
  }

  for (int t = 0; t < T; ++t) {
    const size_t rt = (row0 + t) * H + c;
    const float wgx = act ? ld(a.Wgx, rt) : 0.0f;
    const float wxn = (act && t + 1 < T) ? ld(a.Wx, rt + H) : 0.0f;
    if (tid == 0) {
      if (!wait_counter(counter, nct * static_cast<uint32_t>(t + 1), err)) s_abort = 1;
    }
    __syncthreads();
    if (s_abort) return;

    const uint32_t sbase = static_cast<uint32_t>(t & 1) * a.slot_bytes;
    typename M::Reg breg[KSTEPS];
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s)
      breg[s] = M::load_x(xr, sbase + static_cast<uint32_t>((wave * KSTEPS + s) * 64 + lane) * M::UNIT);
    f32x4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] = M::mma(wreg[mt][s], breg[s], acc[mt]);
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int j = 0; j < 4; ++j) red[wave][mt][(lane >> 4) * 4 + j][lane & 15] = acc[mt][j];
    }
    __syncthreads();

    float ynext = 0.0f, bn = 0.f, en = 0.f, cpost = 0.f, nov = 0.f, p = 0.f, s_g = 0.f, ay = 0.f;
    if (is_pair) {
      float ug = 0.0f;
      const int ra = CH + cl;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        ug += red[w][cl >> 4][cl & 15][bl];
        ay += red[w][ra >> 4][ra & 15][bl];
      }
      // The reference's recurrent GEMM returns the activation dtype.
      ug = round_to<E>(ug);
      ay = round_to<E>(ay);
      s_g = hardsigmoidf_(wgx + ug);
      nov = tanhf(fabsf(ay - sb));
      const float stress = nov * (1.0f - se);
      cpost = up.decay * sc + (1.0f - up.decay) * stress;
      const float nov_eff = nov * (1.0f - c_sup * cpost);
      const float tb = tanhf(sb);
      float k_sig = up.ks * s_g + up.ky * ycur + up.kb * tb + up.kn * nov_eff + up.kbias;
      float r_sig = up.rs * s_g + up.ry * ycur + up.rb * tb + up.rn * nov_eff + up.rbias;
      k_sig += up.kc * cpost;
      r_sig += up.rc * cpost;
      const float k_t = up.kappa * expf(0.5f * tanhf(k_sig));
      const float r_t = clamp01(up.recover * expf(0.5f * tanhf(r_sig)));
      p = s_g * se;
      bn = (1.0f - gate_alpha) * sb + up.beta + lam * (p * ay);
      en = clamp01(se + r_t * (1.0f - se) - k_t * p);
      if (act && t + 1 < T) ynext = tanhf(wxn + bn);
    }
    if (t + 1 < T) {
      const float v[1] = {ynext};
      publish<E, CH, 1>(xr, a.slot_bytes, (t + 1) & 1, kb_y, v, is_pair, cl, bl, stage);
      if (tid == 0) arrive(counter);
    }
    if (act) {
      const size_t ru = (row0 + t) * 2 * H + c;
      st(a.U, ru, ycur);
      st(a.U, ru + H, bn);
      st(a.nov, rt, nov);
      st(a.pl, rt, p);
      st(a.ay, rt, ay);
      st(a.wr, rt, p * ay);
      st(a.et, rt, se);
      st(a.ctp, rt, cpost);
      st(a.st, rt, gate_tape_value<E>(s_g));
    }
    sb = bn;
    se = en;
    sc = cpost;
    ycur = ynext;
  }
  if (act) {
    const size_t i = static_cast<size_t>(b) * H + c;
    a.bF[i] = sb;
    a.eF[i] = se;
    a.cF[i] = sc;
  }
}

// ---------------------------------------------------------------------------
// Reverse scan.
// ---------------------------------------------------------------------------
template <typename E>
struct BwdArgs {
  int B, T, H, nct, kp;
  const E* GAT;  // [H][2H]: transpose of [Ug; A]
  Params P;
  const float* b0;
  const float* c0;
  const E* U;
  const E* pl;
  const E* ay;
  const E* et;
  const E* ctp;
  const E* st;
  const E* gU;
  const E* gN;
  const E* gP;
  const E* gA;
  const E* gW;
  const E* gE;
  const E* gC;
  const float* gbF;
  const float* geF;
  const float* gcF;
  E* gWx;
  E* gWgx;
  E* day;
  float* part_vec;   // [nbg][16][H]
  float* part_scal;  // [nbg * nct][3]
  float* gb0;
  float* ge0;
  float* gc0;
  uint8_t* ws;
  uint32_t slot_bytes;
};

template <typename E, int CH, int KSTEPS>
__global__ void __launch_bounds__(NT, 1) core_bwd_kernel(BwdArgs<E> a) {
  using M = Mf<E>;
  constexpr int KSTEP = M::KSTEP;
  constexpr int KB = 2 * KSTEPS;  // per-wave k-steps over the 2*KP adjoint input
  constexpr int PAIRS = CH * NB;
  constexpr int NACC = 19;
  static_assert(CH <= 16, "one M tile of output units");

  __shared__ float red[NW][16][16];
  __shared__ bf16 stage[2][NB][CH];
  __shared__ float accs[NB][CH][NACC];
  __shared__ int s_abort;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int ct, bg;
  tile_of(a.nct, ct, bg);
  const int H = a.H, T = a.T, B = a.B, KP = a.kp;
  const uint32_t nct = static_cast<uint32_t>(a.nct);
  uint32_t* err = reinterpret_cast<uint32_t*>(a.ws);
  uint32_t* counter = reinterpret_cast<uint32_t*>(a.ws + 4) + bg;
  uint8_t* xbase = a.ws + kXOff + static_cast<size_t>(bg) * 2 * a.slot_bytes;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(xbase, 2 * a.slot_bytes);
  if (tid == 0) s_abort = 0;

  // A operand: rows = output units j of this tile, k = adjoint input index
  // (k < KP: gate-preactivation grad of unit k; k >= KP: expression grad of unit k-KP).
  typename M::Reg wreg[KB];
  {
    const int j = ct * CH + (lane & 15);
    const bool jok = (lane & 15) < CH && j < H;
    const size_t jrow = static_cast<size_t>(j) * 2 * H;
#pragma unroll
    for (int s = 0; s < KB; ++s) {
      const int k0 = (wave * KB + s) * KSTEP;
      if constexpr (is_bf16<E>::value) {
        bf16 v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int k = k0 + (lane >> 4) * 8 + e;
          const int r = k < KP ? k : H + (k - KP);
          const bool ok = jok && (k < KP ? k < H : (k - KP) < H);
          v[e] = ok ? a.GAT[jrow + r] : static_cast<bf16>(0);
        }
        wreg[s] = __builtin_bit_cast(bf16x8, v);
      } else {
        const int k = k0 + (lane >> 4);
        const int r = k < KP ? k : H + (k - KP);
        const bool ok = jok && (k < KP ? k < H : (k - KP) < H);
        wreg[s] = ok ? a.GAT[jrow + r] : 0.0f;
      }
    }
  }

  const bool is_pair = tid < PAIRS;
  const int cl = tid % CH, bl = tid / CH;
  const int c = ct * CH + cl, b = bg * NB + bl;
  const bool act = is_pair && c < H && b < B;
  const UnitParams up = load_unit(a.P, c, is_pair && c < H);
  const float alpha = sigmoidf_(a.P.scal[0][0]);
  const float lam = softplusf_(a.P.scal[1][0]);
  const float sig_lam = sigmoidf_(a.P.scal[1][0]);
  const float sup = sigmoidf_(a.P.scal[2][0]);
  const size_t bh = static_cast<size_t>(b) * H + c;
  float gbn = (act && a.gbF) ? a.gbF[bh] : 0.0f;
  float gen = (act && a.geF) ? a.geF[bh] : 0.0f;
  float gcn = (act && a.gcF) ? a.gcF[bh] : 0.0f;
  float acc[NACC];
#pragma unroll
  for (int i = 0; i < NACC; ++i) acc[i] = 0.0f;
  const size_t row0 = static_cast<size_t>(b) * T;
  const int kb2[2] = {ct * CH, KP + ct * CH};

  for (int n = 0; n < T; ++n) {
    const int t = T - 1 - n;
    const size_t rt = (row0 + t) * H + c;
    const size_t ru = (row0 + t) * 2 * H + c;
    float y = 0.f, dgate = 0.f, dexpr = 0.f, keep_b = 0.f, keep_e = 0.f, keep_c = 0.f, gyx = 0.f;
    if (act) {
      y = ld(a.U, ru);
      const float b_prev = t > 0 ? ld(a.U, ru - 2 * static_cast<size_t>(H) + H) : a.b0[bh];
      const float e_prev = ld(a.et, rt);
      const float c_prev = t > 0 ? ld(a.ctp, rt - H) : a.c0[bh];
      const float gate = ld(a.st, rt);
      const float p = ld(a.pl, rt);
      const float ay = ld(a.ay, rt);
      const float nov = tanhf(fabsf(ay - b_prev));
      const float c_t = ld(a.ctp, rt);
      const float gy0 = a.gU ? ld(a.gU, ru) : 0.0f;
      const float gb_new = (a.gU ? ld(a.gU, ru + H) : 0.0f) + gbn;
      const float gc_new = gcn + (a.gC ? ld(a.gC, rt) : 0.0f);
      const float gnov0 = a.gN ? ld(a.gN, rt) : 0.0f;
      const float gp0 = a.gP ? ld(a.gP, rt) : 0.0f;
      const float gay0 = a.gA ? ld(a.gA, rt) : 0.0f;
      const float gwrite = a.gW ? ld(a.gW, rt) : 0.0f;
      const float geo = a.gE ? ld(a.gE, rt) : 0.0f;

      const float tanh_b = tanhf(b_prev);
      const float nov_eff = nov * (1.0f - sup * c_t);
      const float k_signal = up.ks * gate + up.ky * y + up.kb * tanh_b + up.kn * nov_eff +
                             up.kbias + up.kc * c_t;
      const float r_signal = up.rs * gate + up.ry * y + up.rb * tanh_b + up.rn * nov_eff +
                             up.rbias + up.rc * c_t;
      const float tanh_k = tanhf(k_signal), tanh_r = tanhf(r_signal);
      const float exp_k = expf(0.5f * tanh_k), exp_r = expf(0.5f * tanh_r);
      const float write_cost = up.kappa * exp_k;
      const float recovery_pre = up.recover * exp_r;
      const float recovery = clamp01(recovery_pre);
      const float rclamp = (recovery_pre >= 0.0f && recovery_pre <= 1.0f) ? 1.0f : 0.0f;
      const float energy_pre = e_prev + recovery * (1.0f - e_prev) - write_cost * p;
      const float ge_pre = gen * ((energy_pre >= 0.0f && energy_pre <= 1.0f) ? 1.0f : 0.0f);
      const float g_bprev_state = gb_new * (1.0f - alpha);
      const float g_eprev_state = ge_pre * (1.0f - recovery);
      float gp = gp0 + gb_new * lam * ay - ge_pre * write_cost;
      const float gay = gay0 + gb_new * lam * p;
      const float g_write_cost = -ge_pre * p;
      const float g_recovery = ge_pre * (1.0f - e_prev);
      const float d_expr_main = gay + gwrite * p;
      gp = gp + gwrite * ay;
      const float g_k = g_write_cost * write_cost * 0.5f * (1.0f - tanh_k * tanh_k);
      const float g_rpre = g_recovery * rclamp;
      const float g_r = g_rpre * recovery_pre * 0.5f * (1.0f - tanh_r * tanh_r);
      const float g_gate_energy = g_k * up.ks + g_r * up.rs;
      const float gy_energy = g_k * up.ky + g_r * up.ry;
      const float gb_energy = (g_k * up.kb + g_r * up.rb) * (1.0f - tanh_b * tanh_b);
      const float gnov_eff = g_k * up.kn + g_r * up.rn;
      const float gc_energy = g_k * up.kc + g_r * up.rc;
      dgate = (gp * e_prev + g_gate_energy) *
              (((gate > 0.0f) && (gate < 1.0f)) ? (1.0f / 6.0f) : 0.0f);
      const float ge_gate = gp * gate;
      const float stress = nov * (1.0f - e_prev);
      const float c_new = up.decay * c_prev + (1.0f - up.decay) * stress;
      const float g_c_new = gc_new + gc_energy - gnov_eff * nov * sup;
      const float g_stress = g_c_new * (1.0f - up.decay);
      const float g_nov = gnov_eff * (1.0f - sup * c_new) + g_stress * (1.0f - e_prev);
      const float g_e_prev_cort = -g_stress * nov;
      const float diff = ay - b_prev;
      const float d_nov = (gnov0 + g_nov) * (1.0f - nov * nov) * signf_(diff);
      dexpr = d_expr_main + d_nov;
      keep_b = g_bprev_state + gb_energy - d_nov;
      keep_e = g_eprev_state + ge_gate + g_e_prev_cort + geo;
      keep_c = g_c_new * up.decay;
      gyx = gy0 + gy_energy;

      acc[0] += gb_new;
      acc[1] += g_write_cost * exp_k * up.lk_sig;
      acc[2] += g_rpre * exp_r * up.recover * (1.0f - up.recover);
      acc[3] += g_k * gate;
      acc[4] += g_k * y;
      acc[5] += g_k * tanh_b;
      acc[6] += g_k * nov_eff;
      acc[7] += g_k;
      acc[8] += g_r * gate;
      acc[9] += g_r * y;
      acc[10] += g_r * tanh_b;
      acc[11] += g_r * nov_eff;
      acc[12] += g_r;
      acc[13] += g_c_new * (c_prev - stress) * up.decay * (1.0f - up.decay);
      acc[14] += g_k * c_t;
      acc[15] += g_r * c_t;
      acc[16] += gb_new * (-b_prev) * alpha * (1.0f - alpha);
      acc[17] += gb_new * (p * ay) * sig_lam;
      acc[18] += gnov_eff * nov * (-c_new) * sup * (1.0f - sup);
    }
    {
      const float v[2] = {dgate, dexpr};
      publish<E, CH, 2>(xr, a.slot_bytes, n & 1, kb2, v, is_pair, cl, bl, stage);
      if (tid == 0) arrive(counter);
    }
    if (tid == 0) {
      if (!wait_counter(counter, nct * static_cast<uint32_t>(n + 1), err)) s_abort = 1;
    }
    __syncthreads();
    if (s_abort) return;

    const uint32_t sbase = static_cast<uint32_t>(n & 1) * a.slot_bytes;
    typename M::Reg breg[KB];
#pragma unroll
    for (int s = 0; s < KB; ++s)
      breg[s] = M::load_x(xr, sbase + static_cast<uint32_t>((wave * KB + s) * 64 + lane) * M::UNIT);
    f32x4 accm = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KB; ++s) accm = M::mma(wreg[s], breg[s], accm);
#pragma unroll
    for (int j = 0; j < 4; ++j) red[wave][(lane >> 4) * 4 + j][lane & 15] = accm[j];
    __syncthreads();
    if (act) {
      float adj = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; ++w) adj += red[w][cl][bl];
      adj = round_to<E>(adj);
      const float gy = gyx + adj;
      const float gpre = gy * (1.0f - y * y);
      st(a.gWx, rt, gpre);
      st(a.gWgx, rt, dgate);
      st(a.day, rt, dexpr);
      gbn = keep_b + gpre;
      gen = keep_e;
      gcn = keep_c;
    }
  }

  if (act) {
    a.gb0[bh] = gbn;
    a.ge0[bh] = gen;
    a.gc0[bh] = gcn;
  }
  // Per-unit parameter gradients: reduce the 16 batch rows of this tile in a fixed order.
  if (is_pair) {
#pragma unroll
    for (int i = 0; i < NACC; ++i) accs[bl][cl][i] = act ? acc[i] : 0.0f;
  }
  __syncthreads();
  for (int q = tid; q < 16 * CH; q += NT) {
    const int k = q / CH, u = q % CH;
    const int cu = ct * CH + u;
    float s = 0.0f;
    for (int r = 0; r < NB; ++r) s += accs[r][u][k];
    if (cu < H) a.part_vec[(static_cast<size_t>(bg) * 16 + k) * H + cu] = s;
  }
  if (tid < 3) {
    float s = 0.0f;
    for (int u = 0; u < CH; ++u)
      for (int r = 0; r < NB; ++r) s += accs[r][u][16 + tid];
    a.part_scal[static_cast<size_t>(blockIdx.x) * 3 + tid] = s;
  }
}

// ---------------------------------------------------------------------------
// Host side: configuration, workspace and launch.
// ---------------------------------------------------------------------------
struct Cfg {
  int ch = 0, ksteps = 0, kp = 0, nct = 0, nbg = 0;
};

static Cfg pick(int dtype, int64_t B, int64_t H) {
  Cfg c;
  const int kstep = dtype == kBF16 ? 32 : 4;
  const int need = static_cast<int>((H + NW * kstep - 1) / (NW * kstep));
  static const int bf_steps[] = {1, 2, 4, 8, 16};
  static const int f_steps[] = {1, 2, 4, 8, 16, 32, 64};
  const int* list = dtype == kBF16 ? bf_steps : f_steps;
  const int nlist = dtype == kBF16 ? 5 : 7;
  for (int i = 0; i < nlist; ++i) {
    if (list[i] >= need) {
      c.ksteps = list[i];
      break;
    }
  }
  if (c.ksteps == 0) return c;
  c.kp = NW * c.ksteps * kstep;
  c.ch = (dtype == kBF16 && H >= 1024) ? 16 : 8;
  c.nct = static_cast<int>((H + c.ch - 1) / c.ch);
  c.nbg = static_cast<int>((B + NB - 1) / NB);
  return c;
}

static size_t slot_bytes(int dtype, const Cfg& c, bool backward) {
  const size_t e = dtype == kBF16 ? 2 : 4;
  return (backward ? 2 : 1) * static_cast<size_t>(c.kp) * NB * e;
}

static size_t workspace_bytes(int dtype, const Cfg& c, bool backward) {
  return kXOff + static_cast<size_t>(c.nbg) * 2 * slot_bytes(dtype, c, backward);
}

template <typename K, typename A>
static int launch_coop(K kernel, int grid, const A& args, hipStream_t stream) {
  int dev = 0;
  DABSN_HIP_CHECK(hipGetDevice(&dev));
  int cus = 0, per_cu = 0, coop = 0;
  DABSN_HIP_CHECK(hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev));
  DABSN_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  DABSN_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, NT, 0));
  if (!coop || per_cu * cus < grid) {
    dabsn::set_error(
        "core scan needs %d co-resident workgroups but the device holds %d (%d per CU x %d CUs,"
        " cooperative=%d)",
        grid, per_cu * cus, per_cu, cus, coop);
    return DABSN_ERR_UNSUPPORTED;
  }
  void* kargs[] = {const_cast<A*>(&args)};
  DABSN_HIP_CHECK(hipLaunchCooperativeKernel(reinterpret_cast<const void*>(kernel), dim3(grid),
                                             dim3(NT), kargs, 0, stream));
  return DABSN_OK;
}

template <typename E>
static int fwd_dispatch(const Cfg& c, const FwdArgs<E>& args, hipStream_t stream) {
  const int grid = c.nct * c.nbg;
#define DABSN_CASE(CHV, KS)                                                    \
  if (c.ch == CHV && c.ksteps == KS)                                           \
    return launch_coop(core_fwd_kernel<E, CHV, KS>, grid, args, stream);
  if constexpr (is_bf16<E>::value) {
    DABSN_CASE(8, 1) DABSN_CASE(8, 2) DABSN_CASE(8, 4) DABSN_CASE(8, 8) DABSN_CASE(8, 16)
    DABSN_CASE(16, 8) DABSN_CASE(16, 16)
  } else {
    DABSN_CASE(8, 1) DABSN_CASE(8, 2) DABSN_CASE(8, 4) DABSN_CASE(8, 8) DABSN_CASE(8, 16)
    DABSN_CASE(8, 32) DABSN_CASE(8, 64)
  }
#undef DABSN_CASE
  dabsn::set_error("core scan: no kernel for CH=%d KSTEPS=%d", c.ch, c.ksteps);
  return DABSN_ERR_UNSUPPORTED;
}

template <typename E>
static int bwd_dispatch(const Cfg& c, const BwdArgs<E>& args, hipStream_t stream) {
  const int grid = c.nct * c.nbg;
#define DABSN_CASE(CHV, KS)                                                    \
  if (c.ch == CHV && c.ksteps == KS)                                           \
    return launch_coop(core_bwd_kernel<E, CHV, KS>, grid, args, stream);
  if constexpr (is_bf16<E>::value) {
    DABSN_CASE(8, 1) DABSN_CASE(8, 2) DABSN_CASE(8, 4) DABSN_CASE(8, 8) DABSN_CASE(8, 16)
    DABSN_CASE(16, 8) DABSN_CASE(16, 16)
  } else {
    DABSN_CASE(8, 1) DABSN_CASE(8, 2) DABSN_CASE(8, 4) DABSN_CASE(8, 8) DABSN_CASE(8, 16)
    DABSN_CASE(8, 32) DABSN_CASE(8, 64)
  }
#undef DABSN_CASE
  dabsn::set_error("core scan backward: no kernel for CH=%d KSTEPS=%d", c.ch, c.ksteps);
  return DABSN_ERR_UNSUPPORTED;
}

static Params to_params(const dabsn_core_params* p) {
  Params q;
  for (int i = 0; i < 16; ++i) q.vec[i] = p->vec[i];
  for (int i = 0; i < 3; ++i) q.scal[i] = p->scal[i];
  return q;
}

static int check_common(int dtype, int64_t B, int64_t T, int64_t H, const dabsn_core_params* p,
                        const Cfg& c, size_t ws_bytes, size_t need) {
  DABSN_REQUIRE(dtype == kF32 || dtype == kBF16, "core scan: dtype %d is not fp32(0)/bf16(1)", dtype);
  DABSN_REQUIRE(B > 0 && T >= 0 && H > 0, "core scan: bad shape B=%lld T=%lld H=%lld",
                (long long)B, (long long)T, (long long)H);
  DABSN_REQUIRE(T < (1ll << 30) && B * T * 2 * H < (1ll << 46), "core scan: shape too large");
  DABSN_REQUIRE(p != nullptr, "core scan: null parameter table");
  for (int i = 0; i < 16; ++i) DABSN_REQUIRE(p->vec[i] != nullptr, "core scan: null vector %d", i);
  for (int i = 0; i < 3; ++i) DABSN_REQUIRE(p->scal[i] != nullptr, "core scan: null scalar %d", i);
  if (c.ksteps == 0) {
    dabsn::set_error("core scan: H=%lld exceeds the supported width for dtype %d", (long long)H,
                     dtype);
    return DABSN_ERR_UNSUPPORTED;
  }
  DABSN_REQUIRE(ws_bytes >= need, "core scan: workspace %zu B < required %zu B", ws_bytes, need);
  return DABSN_OK;
}

}  // namespace core
}  // namespace dabsn

using namespace dabsn;
using namespace dabsn::core;

extern "C" {

size_t dabsn_hip_core_scan_workspace_bytes(int dtype, int64_t B, int64_t H, int backward) {
  const Cfg c = pick(dtype, B, H);
  if (c.ksteps == 0) return 0;
  return workspace_bytes(dtype, c, backward != 0);
}

int dabsn_hip_core_scan_layout(int dtype, int64_t B, int64_t H, int64_t* nbg, int64_t* nwg) {
  const Cfg c = pick(dtype, B, H);
  if (c.ksteps == 0) {
    dabsn::set_error("core scan: unsupported H=%lld", (long long)H);
    return DABSN_ERR_UNSUPPORTED;
  }
  if (nbg) *nbg = c.nbg;
  if (nwg) *nwg = static_cast<int64_t>(c.nbg) * c.nct;
  return DABSN_OK;
}

int dabsn_hip_core_scan_fwd(int dtype, int64_t B, int64_t T, int64_t H, const void* Wx,
                            const void* Wgx, const void* GA, const dabsn_core_params* params,
                            const float* b0, const float* e0, const float* c0, void* U, void* nov,
                            void* plast, void* expr, void* write, void* energy, void* sat,
                            void* gate, float* bF, float* eF, float* cF, void* workspace,
                            size_t workspace_bytes_, hipStream_t stream) {
  const Cfg c = pick(dtype, B, H);
  const int rc = check_common(dtype, B, T, H, params, c, workspace_bytes_,
                              c.ksteps ? workspace_bytes(dtype, c, false) : 0);
  if (rc != DABSN_OK) return rc;
  DABSN_REQUIRE(Wx && Wgx && GA && b0 && e0 && c0 && bF && eF && cF && workspace,
                "core scan: null pointer argument");
  DABSN_REQUIRE(T == 0 || (U && nov && plast && expr && write && energy && sat && gate),
                "core scan: null tape pointer");
  int zr = dabsn_hip_zero(workspace, workspace_bytes(dtype, c, false), stream);
  if (zr != DABSN_OK) return zr;
  if (dtype == kBF16) {
    FwdArgs<bf16> a{static_cast<int>(B), static_cast<int>(T), static_cast<int>(H), c.nct,
                    static_cast<const bf16*>(Wx), static_cast<const bf16*>(Wgx),
                    static_cast<const bf16*>(GA), to_params(params), b0, e0, c0,
                    static_cast<bf16*>(U), static_cast<bf16*>(nov), static_cast<bf16*>(plast),
                    static_cast<bf16*>(expr), static_cast<bf16*>(write),
                    static_cast<bf16*>(energy), static_cast<bf16*>(sat), static_cast<bf16*>(gate),
                    bF, eF, cF, static_cast<uint8_t*>(workspace),
                    static_cast<uint32_t>(slot_bytes(dtype, c, false))};
    return fwd_dispatch(c, a, stream);
  }
  FwdArgs<float> a{static_cast<int>(B), static_cast<int>(T), static_cast<int>(H), c.nct,
                   static_cast<const float*>(Wx), static_cast<const float*>(Wgx),
                   static_cast<const float*>(GA), to_params(params), b0, e0, c0,
                   static_cast<float*>(U), static_cast<float*>(nov), static_cast<float*>(plast),
                   static_cast<float*>(expr), static_cast<float*>(write),
                   static_cast<float*>(energy), static_cast<float*>(sat), static_cast<float*>(gate),
                   bF, eF, cF, static_cast<uint8_t*>(workspace),
                   static_cast<uint32_t>(slot_bytes(dtype, c, false))};
  return fwd_dispatch(c, a, stream);
}

int dabsn_hip_core_scan_bwd(int dtype, int64_t B, int64_t T, int64_t H, const void* GAT,
                            const dabsn_core_params* params, const float* b0, const float* c0,
                            const void* U, const void* plast, const void* expr, const void* energy,
                            const void* sat, const void* gate, const void* gU, const void* gNov,
                            const void* gP, const void* gAy, const void* gW, const void* gE,
                            const void* gC, const float* gbF, const float* geF, const float* gcF,
                            void* gWx, void* gWgx, void* day, float* part_vec, float* part_scal,
                            float* gb0, float* ge0, float* gc0, void* workspace,
                            size_t workspace_bytes_, hipStream_t stream) {
  const Cfg c = pick(dtype, B, H);
  const int rc = check_common(dtype, B, T, H, params, c, workspace_bytes_,
                              c.ksteps ? workspace_bytes(dtype, c, true) : 0);
  if (rc != DABSN_OK) return rc;
  DABSN_REQUIRE(GAT && b0 && c0 && part_vec && part_scal && gb0 && ge0 && gc0 && workspace,
                "core scan backward: null pointer argument");
  DABSN_REQUIRE(T == 0 || (U && plast && expr && energy && sat && gate && gWx && gWgx && day),
                "core scan backward: null tape pointer");
  if (dtype == kF32 && c.ksteps > 32) {
    dabsn::set_error("core scan backward: fp32 supports H <= 512 per workgroup register budget");
    return DABSN_ERR_UNSUPPORTED;
  }
  int zr = dabsn_hip_zero(workspace, workspace_bytes(dtype, c, true), stream);
  if (zr != DABSN_OK) return zr;
  if (dtype == kBF16) {
    using E = bf16;
    BwdArgs<E> a{static_cast<int>(B), static_cast<int>(T), static_cast<int>(H), c.nct, c.kp,
                 static_cast<const E*>(GAT), to_params(params), b0, c0,
                 static_cast<const E*>(U), static_cast<const E*>(plast),
                 static_cast<const E*>(expr), static_cast<const E*>(energy),
                 static_cast<const E*>(sat), static_cast<const E*>(gate),
                 static_cast<const E*>(gU), static_cast<const E*>(gNov),
                 static_cast<const E*>(gP), static_cast<const E*>(gAy),
                 static_cast<const E*>(gW), static_cast<const E*>(gE),
                 static_cast<const E*>(gC), gbF, geF, gcF, static_cast<E*>(gWx),
                 static_cast<E*>(gWgx), static_cast<E*>(day), part_vec, part_scal, gb0, ge0, gc0,
                 static_cast<uint8_t*>(workspace),
                 static_cast<uint32_t>(slot_bytes(dtype, c, true))};
    return bwd_dispatch(c, a, stream);
  }
  using E = float;
  BwdArgs<E> a{static_cast<int>(B), static_cast<int>(T), static_cast<int>(H), c.nct, c.kp,
               static_cast<const E*>(GAT), to_params(params), b0, c0,
               static_cast<const E*>(U), static_cast<const E*>(plast),
               static_cast<const E*>(expr), static_cast<const E*>(energy),
               static_cast<const E*>(sat), static_cast<const E*>(gate),
               static_cast<const E*>(gU), static_cast<const E*>(gNov),
               static_cast<const E*>(gP), static_cast<const E*>(gAy),
               static_cast<const E*>(gW), static_cast<const E*>(gE),
               static_cast<const E*>(gC), gbF, geF, gcF, static_cast<E*>(gWx),
               static_cast<E*>(gWgx), static_cast<E*>(day), part_vec, part_scal, gb0, ge0, gc0,
               static_cast<uint8_t*>(workspace),
               static_cast<uint32_t>(slot_bytes(dtype, c, true))};
  return bwd_dispatch(c, a, stream);
}

}  // extern "C"
