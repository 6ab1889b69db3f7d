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
//     device-wide step barrier: monotonic step counters split kSplit ways (one 64-byte
//     line each) so arrivals do not serialise on one address. Exchange traffic and the
//     counters use device-coherent (sc1) accesses so no L2 writeback/invalidate is
//     needed between XCDs.
//   * The recurrent product runs on v_mfma_f32_16x16x32_bf16 (bf16) or
//     v_mfma_f32_16x16x4_f32 (fp32) with K split across the NW waves; partial tiles
//     are reduced through LDS in a fixed order (deterministic).
//   * State (b, e, c) and the per-unit parameters live in registers of the thread that
//     owns a (unit, batch row) pair; tapes are written once per step.
//   * Only what the next exchange needs sits between two barriers: the forward
//     publishes y_{t+1} before it updates energy/cortisol and writes tapes, and the
//     backward prefetches its tapes two steps ahead and evaluates each reverse step as
//     base + X * slope, where X (the tanh pre-activation grad, the one quantity that
//     waits for the exchange) enters every output affinely through the budget grad.
//   * Barrier waits are bounded: a wait that exceeds kSpinLimit polls sets the error
//     word and every workgroup exits.
#include <algorithm>
#include <initializer_list>
#include <type_traits>

#include "../../include/dabsn_hip.h"
#include "capi.hpp"
#include "common.hpp"
#include "gemm.hpp"

namespace dabsn {
namespace core {

constexpr int NB = 16;  // batch rows per group (MFMA N)

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

// Workspace layout: [0,4) error word; from kCtrOff, kSplit step counters per batch
// group, kCtrStride bytes apart; exchange slots (2 per batch group) from
// xchg_offset(nbg).
constexpr int kSplit = 8;
constexpr size_t kCtrOff = 64;
constexpr size_t kCtrStride = 64;
__host__ __device__ inline size_t xchg_offset(int nbg) {
  const size_t end = kCtrOff + static_cast<size_t>(nbg) * kSplit * kCtrStride;
  return (end + 4095) / 4096 * 4096;
}

// Arrivals one split counter receives per step: workgroup i of a batch group (0 <= i <
// nct) arrives on counter i % kSplit.
__host__ __device__ inline uint32_t split_arrivals(int nct, int s) {
  return s < nct ? static_cast<uint32_t>((nct - s + kSplit - 1) / kSplit) : 0u;
}

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

// Scalar gains shared by every unit: gate mixing, budget write gain, cortisol suppression.
struct StepGains {
  float gate_alpha, lam, c_sup;
};
__device__ __forceinline__ StepGains load_gains(const Params& P) {
  return StepGains{sigmoidf_(P.scal[0][0]), softplusf_(P.scal[1][0]), sigmoidf_(P.scal[2][0])};
}

// One step of a unit after the recurrent products ug (gate rows) and ay (A rows), both
// already rounded to the activation dtype: the gate s_g, plasticity p and next budget bn.
__device__ __forceinline__ float budget_next(const UnitParams& up, const StepGains& sg, float sb,
                                             float se, float wgx, float ug, float ay, float& s_g,
                                             float& p) {
  s_g = hardsigmoidf_(wgx + ug);
  p = s_g * se;
  return (1.0f - sg.gate_alpha) * sb + up.beta + sg.lam * (p * ay);
}

// The rest of the step from the same inputs: novelty, cortisol after the step (cpost) and
// the next energy.
__device__ __forceinline__ float energy_next(const UnitParams& up, const StepGains& sg, float sb,
                                             float se, float sc, float y, float s_g, float p,
                                             float ay, float& nov, float& cpost) {
  nov = tanhf(fabsf(ay - sb));
  const float stress = nov * (1.0f - se);
  cpost = up.decay * sc + (1.0f - up.decay) * stress;
  const float nov_eff = nov * (1.0f - sg.c_sup * cpost);
  const float tb = tanhf(sb);
  float k_sig = up.ks * s_g + up.ky * y + up.kb * tb + up.kn * nov_eff + up.kbias;
  float r_sig = up.rs * s_g + up.ry * y + up.rb * tb + up.rn * nov_eff + up.rbias;
  k_sig += up.kc * cpost;
  r_sig += up.rc * cpost;
  const float k_t = up.kappa * expf(0.5f * tanhf(k_sig));
  const float r_t = clamp01(up.recover * expf(0.5f * tanhf(r_sig)));
  return clamp01(se + r_t * (1.0f - se) - k_t * p);
}

// Called by all 64 lanes of wave 0: waits until every split counter of the batch group
// (base `ctr`) has received `step1` rounds of arrivals. Lane s < kSplit polls counter s
// (the other lanes read counter 0 against a zero target, so the load needs no branch).
// One poll is in flight at a time: a load left pending at return would hold up the
// workgroup's next store drain. Returns false if the error word is raised or the wait
// exceeded the spin bound; lane 0 then raises the error word itself on a timeout.
__device__ __forceinline__ bool wait_step(const uint32_t* ctr, int nct, uint32_t step1,
                                          uint32_t* err) {
  const int lane = threadIdx.x & 63;
  const int s = lane < kSplit ? lane : 0;
  const uint32_t target = (lane < kSplit ? split_arrivals(nct, s) : 0u) * step1;
  const uint32_t* mine = ctr + s * (kCtrStride / 4);
  uint32_t spins = 0;
  while (true) {
    if (__all(__hip_atomic_load(mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= target))
      return true;
    if ((++spins & 1023u) == 0u) {
      if (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) return false;
      if (spins > kSpinLimit) {
        if (lane == 0)
          __hip_atomic_fetch_or(err, kErrBarrierTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
      }
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

__device__ __forceinline__ void arrive(uint32_t* counter) {
  __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Step counters of batch group bg, and the counter this workgroup arrives on.
__device__ __forceinline__ uint32_t* group_counters(uint8_t* ws, int bg) {
  return reinterpret_cast<uint32_t*>(ws + kCtrOff + static_cast<size_t>(bg) * kSplit * kCtrStride);
}
__device__ __forceinline__ uint32_t* my_counter(uint32_t* ctr, int nct, int bid) {
  return ctr + (bid % nct % kSplit) * (kCtrStride / 4);
}

// Wait for every outstanding vector memory operation of this wave (the exchange stores
// must be complete before the workgroup announces them on the counter).
__device__ __forceinline__ void drain_vmem() { __builtin_amdgcn_s_waitcnt(0); }

// Publishes `nvals` values per (unit, batch) pair into slot `xs` of the exchange
// buffer at k = kbase[i] + cl; every thread of the workgroup calls it. bf16: the 8
// consecutive lanes that hold units 8g..8g+7 of one batch row pack their values with
// lane shuffles and the first of them stores the 16-byte unit; fp32 stores one word per
// value. Returns once every store of the workgroup is complete.
template <typename E, int CH, int NV>
__device__ __forceinline__ void publish(__amdgpu_buffer_rsrc_t xr, uint32_t slot_bytes, int xs,
                                        const int (&kbase)[NV], const float (&vals)[NV],
                                        bool is_pair, int cl, int bl) {
  if constexpr (is_bf16<E>::value) {
    // Pair threads fill whole waves (tid = bl * CH + cl), so `is_pair` is wave-uniform
    // and lane & 7 == cl & 7.
    static_assert(CH % 8 == 0 && (CH * NB) % 64 == 0, "pair threads must fill whole waves");
    if (is_pair) {
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        // Groups of 8 lanes lie inside 16-lane rows, so in-row DPP shifts gather the
        // group for its first lane (the lanes whose shifts leave the row are not stored).
        const int h = static_cast<int>(f2bf(vals[i]));
        const int w0 = h | (row_shl<1>(h) << 16);
        const int w1 = row_shl<2>(w0);
        const int w2 = row_shl<4>(w0);
        const int w3 = row_shl<6>(w0);
        if ((cl & 7) == 0) {
          const u32x4 v = {static_cast<uint32_t>(w0), static_cast<uint32_t>(w1),
                           static_cast<uint32_t>(w2), static_cast<uint32_t>(w3)};
          const uint32_t off = xs * slot_bytes + xoff<bf16>(kbase[i] + cl, bl) * 2u;
          __builtin_amdgcn_raw_buffer_store_b128(v, xr, static_cast<int>(off), 0, kCoherent);
        }
      }
    }
  } else {
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
  int64_t ldt;  // time steps between consecutive batch rows of every [B, *, .] tensor (>= T)
  int64_t ldx;  // elements between consecutive time steps of Wx and Wgx (>= H)
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
  int sbf;  // initial and final states are bf16 (else fp32), addressed through ld/st_state
};

// Carried-state elements: fp32, or bf16 when the state is carried in the activation dtype
// (the final state rounded to nearest even, as a dtype conversion of the fp32 value).
__device__ __forceinline__ float ld_state(const float* p, size_t i, int sbf) {
  return sbf ? bf2f(reinterpret_cast<const bf16*>(p)[i]) : p[i];
}
__device__ __forceinline__ void st_state(float* p, size_t i, float v, int sbf) {
  if (sbf)
    reinterpret_cast<bf16*>(p)[i] = f2bf(v);
  else
    p[i] = v;
}

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

__device__ __forceinline__ void tile_of(int bid, int nct, int& ct, int& bg) {
  // Consecutive channel tiles go to the same XCD (workgroups are dealt round-robin over
  // the 8 XCDs), so the tape rows a step writes are merged in one L2.
  bg = bid / nct;
  const int i = bid % nct;
  ct = (nct % 8 == 0) ? (i % 8) * (nct / 8) + i / 8 : i;
}

// Forward scan of one workgroup: `bid` is its index among the `grid` workgroups of this
// scan (the kernel may host another scan in its other workgroups).
template <typename E, int CH, int KSTEPS, int NW>
__device__ __forceinline__ void fwd_body(const FwdArgs<E>& a, int bid, int grid) {
  using M = Mf<E>;
  constexpr int NT = NW * 64;
  constexpr int KSTEP = M::KSTEP;
  constexpr int KW = KSTEPS * KSTEP;
  constexpr int ROWS = 2 * CH;
  constexpr int MT = ROWS / 16;
  constexpr int PAIRS = CH * NB;
  static_assert(ROWS % 16 == 0, "CH must be a multiple of 8");
  static_assert(PAIRS <= NT, "one thread per (unit, batch) pair");

  // Partial products of the NW waves, [wave][tile][batch column][row]: each lane writes
  // its 4 accumulator rows as one 16-byte vector and each pair thread reads 64
  // consecutive words per wave, so neither side has LDS bank conflicts.
  __shared__ __attribute__((aligned(16))) float red[NW][MT][16][16];
  __shared__ int s_abort;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int ct, bg;
  tile_of(bid, a.nct, ct, bg);
  const int H = a.H, T = a.T, B = a.B;
  uint32_t* err = reinterpret_cast<uint32_t*>(a.ws);
  uint32_t* ctr = group_counters(a.ws, bg);
  uint32_t* counter = my_counter(ctr, a.nct, bid);
  const int nbg = grid / a.nct;
  uint8_t* xbase = a.ws + xchg_offset(nbg) + static_cast<size_t>(bg) * 2 * a.slot_bytes;
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

  // Staged tape stores (bf16, 16-unit tiles, H % 16 == 0). A step's 9 outputs per pair
  // are parked in LDS as [stream][row][unit] (two buffers, alternating by step) and
  // written out during the next step's shadow as 16-byte chunks (8 units of one batch
  // row) by the threads of waves 1.. -- never by the polling wave 0, whose counter loads
  // would otherwise queue behind the stores.
  constexpr bool OSTAGE = is_bf16<E>::value && CH == 16;
  constexpr int OSN = 9;                       // U (y), U (budget), n, p, ay, w, e, c, s
  constexpr int OCH = OSN * NB * 2;            // chunks per step
  constexpr int OCPT = OSTAGE ? (OCH + NT - 65) / (NT - 64) : 1;  // chunks per thread
  __shared__ __attribute__((aligned(16))) bf16 otape[OSTAGE ? 2 : 1][OSTAGE ? OSN : 1][NB][16];
  E* o_ptr[OCPT];
  uint32_t o_rs[OCPT];
  int o_q[OCPT];
  if constexpr (OSTAGE) {
#pragma unroll
    for (int i = 0; i < OCPT; ++i) {
      const int q = tid - 64 + i * (NT - 64);
      const int sidx = q / (NB * 2), r = (q / 2) % NB, hh = q & 1;
      const int bb = bg * NB + r;
      E* const dst[OSN] = {a.U, a.U, a.nov, a.pl, a.ay, a.wr, a.et, a.ctp, a.st};
      const bool ok = tid >= 64 && q < OCH && bb < B;
      o_q[i] = ok ? q : -1;
      o_rs[i] = static_cast<uint32_t>((sidx < 2 ? 2 : 1) * H);
      o_ptr[i] = ok ? dst[sidx] + static_cast<size_t>(bb) * static_cast<size_t>(a.ldt) * o_rs[i] +
                          (sidx == 1 ? H : 0) + ct * 16 + hh * 8
                    : nullptr;
    }
  }
  // Write out the chunks parked for step t.
  auto flush = [&](int t) {
#pragma unroll
    for (int i = 0; i < OCPT; ++i) {
      const int q = o_q[i];
      if (q >= 0)
        gstore16(o_ptr[i] + static_cast<size_t>(t) * o_rs[i],
                 *reinterpret_cast<const u32x4*>(&otape[t & 1][q / (NB * 2)][(q / 2) % NB][(q & 1) * 8]));
    }
  };

  const UnitParams up = load_unit(a.P, c, is_pair && c < H);
  const StepGains sg = load_gains(a.P);
  float sb = act ? ld_state(a.b0, static_cast<size_t>(b) * H + c, a.sbf) : 0.0f;
  float se = act ? ld_state(a.e0, static_cast<size_t>(b) * H + c, a.sbf) : 0.0f;
  float sc = act ? ld_state(a.c0, static_cast<size_t>(b) * H + c, a.sbf) : 0.0f;
  const size_t row0 = static_cast<size_t>(b) * static_cast<size_t>(a.ldt);

  float ycur = (act && T > 0) ? tanhf(ld(a.Wx, row0 * a.ldx + c) + sb) : 0.0f;
  const int kb_y[1] = {ct * CH};
  if (T > 0) {
    const float v[1] = {ycur};
    publish<E, CH, 1>(xr, a.slot_bytes, 0, kb_y, v, is_pair, cl, bl);
    if (tid == 0) arrive(counter);
  }

  // Wgx_t and Wx_{t+1} are requested one step ahead, unconditionally (threads without a
  // pair read element 0; the last step rereads its own row), so no select waits on them.
  const size_t lrow0 = act ? row0 : 0;
  const int lc = act ? c : 0;
  auto in_row = [&](int t) { return (lrow0 + static_cast<size_t>(t)) * a.ldx + lc; };
  // With 8 waves (16-unit bf16 tiles), wave 4 -- no pairs, no polling -- fetches the next
  // step's Wgx_t and Wx_{t+1} for the tile as 16-byte chunks (2 streams x 16 rows x 2)
  // during the shadow and parks them in LDS after the step barrier; the polling wave 0 then
  // has no loads queued ahead of its counter polls.
  constexpr bool INSTAGE = OSTAGE && NW == 8;
  __shared__ __attribute__((aligned(16))) bf16 inbuf[INSTAGE ? 2 : 1][NB][16];
  const bool in_loader = INSTAGE && wave == 4;
  const int iq = lane;  // chunk of a loader lane: stream iq / 32, row (iq / 2) % 16, half iq & 1
  const E* in_src = iq < 32 ? a.Wgx : a.Wx;
  const int in_bb = bg * NB + (iq / 2) % NB;
  const size_t in_base = static_cast<size_t>(in_bb < B ? in_bb : 0) * static_cast<size_t>(a.ldt) *
                             static_cast<size_t>(a.ldx) + ct * 16 + (iq & 1) * 8;
  // Chunk of step t: Wgx_t or Wx_{t+1} (clamped to the last row).
  auto in_load = [&](int t) {
    const int tr = min(iq < 32 ? t : t + 1, T - 1);
    return gload16(in_src + in_base + static_cast<size_t>(tr) * a.ldx);
  };
  u32x4 in_chunk = {0u, 0u, 0u, 0u};
  if (in_loader && T > 0) in_chunk = in_load(0);
  E wgx_next = INSTAGE ? static_cast<E>(0) : a.Wgx[in_row(0)];
  E wxn_next = INSTAGE ? static_cast<E>(0) : a.Wx[in_row(T > 1 ? 1 : 0)];
  for (int t = 0; t < T; ++t) {
    const size_t rt = (row0 + t) * H + c;
    if (wave == 0) {
      if (!wait_step(ctr, a.nct, static_cast<uint32_t>(t + 1), err) && tid == 0) s_abort = 1;
    }
    __syncthreads();
    if (s_abort) return;
    if constexpr (INSTAGE) {
      // Visible to the pairs after the reduction barrier below.
      if (in_loader)
        *reinterpret_cast<u32x4*>(&inbuf[iq / 32][(iq / 2) % NB][(iq & 1) * 8]) = in_chunk;
    }

    const uint32_t sbase = static_cast<uint32_t>(t & 1) * a.slot_bytes;
    typename M::Reg breg[KSTEPS];
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s)
      breg[s] = M::load_x(xr, sbase + static_cast<uint32_t>((wave * KSTEPS + s) * 64 + lane) * M::UNIT);
    // Keep every exchange load ahead of the first MFMA (all in flight at once).
    __builtin_amdgcn_sched_barrier(0);
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
      *reinterpret_cast<f32x4*>(&red[wave][mt][lane & 15][(lane >> 4) * 4]) = acc[mt];
    }
    __syncthreads();

    // Critical path: the budget update and y_{t+1}.
    float ynext = 0.0f, bn = 0.f, s_g = 0.f, ay = 0.f, p = 0.f;
    if (is_pair) {
      float ug = 0.0f;
      const int ra = CH + cl;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        ug += red[w][cl >> 4][bl][cl & 15];
        ay += red[w][ra >> 4][bl][ra & 15];
      }
      // The reference's recurrent GEMM returns the activation dtype.
      ug = round_to<E>(ug);
      ay = round_to<E>(ay);
      // The prefetched inputs are first read here, so their loads need not land before the
      // next barrier wait starts.
      if constexpr (INSTAGE) {
        wgx_next = inbuf[0][bl][cl];
        wxn_next = inbuf[1][bl][cl];
      }
      bn = budget_next(up, sg, sb, se, to_f(wgx_next), ug, ay, s_g, p);
      if (act && t + 1 < T) ynext = tanhf(to_f(wxn_next) + bn);
    }
    if (t + 1 < T) {
      const float v[1] = {ynext};
      publish<E, CH, 1>(xr, a.slot_bytes, (t + 1) & 1, kb_y, v, is_pair, cl, bl);
      if (tid == 0) arrive(counter);
    }
    // Off the critical path (overlaps the next barrier): energy and cortisol, tapes.
    float en = 0.f, cpost = 0.f, nov = 0.f;
    if (is_pair) en = energy_next(up, sg, sb, se, sc, ycur, s_g, p, ay, nov, cpost);
    if constexpr (OSTAGE) {
      if (t > 0) flush(t - 1);
      if (act) {
        const float v[OSN] = {ycur, bn, nov, p, ay, p * ay, se, cpost, gate_tape_value<E>(s_g)};
#pragma unroll
        for (int k = 0; k < OSN; ++k) otape[t & 1][k][bl][cl] = f2bf(v[k]);
      }
    } else if (act) {
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
    if constexpr (INSTAGE) {
      if (in_loader) in_chunk = in_load(t + 1 < T ? t + 1 : t);
    } else {
      wgx_next = a.Wgx[in_row(t + 1 < T ? t + 1 : t)];
      wxn_next = a.Wx[in_row(t + 2 < T ? t + 2 : (t + 1 < T ? t + 1 : t))];
    }
    sb = bn;
    se = en;
    sc = cpost;
    ycur = ynext;
  }
  if constexpr (OSTAGE) {
    if (T > 0) {
      __syncthreads();
      flush(T - 1);
    }
  }
  if (act) {
    const size_t i = static_cast<size_t>(b) * H + c;
    st_state(a.bF, i, sb, a.sbf);
    st_state(a.eF, i, se, a.sbf);
    st_state(a.cF, i, sc, a.sbf);
  }
}

// ---------------------------------------------------------------------------
// Reverse scan.
// ---------------------------------------------------------------------------
template <typename E>
struct BwdArgs {
  int B, T, H, nct, kp;
  int64_t ldt;  // as in FwdArgs
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

// Raw tape words of one time index, kept unconverted so the loads stay in flight across
// the step barrier (bf16: the 16 storage bits; fp32: the float bits).
struct TapeRaw {
  uint32_t y, b_prev, e_prev, c_prev, gate, p, ay, c_t;
  uint32_t gy0, gub, gc, gnov, gp, gay, gw, ge;
};

template <typename E>
__device__ __forceinline__ uint32_t ldraw(const E* p, size_t i) {
  if constexpr (is_bf16<E>::value) {
    return static_cast<uint32_t>(p[i]);
  } else {
    return __builtin_bit_cast(uint32_t, p[i]);
  }
}

template <typename E>
__device__ __forceinline__ float cvt(uint32_t w) {
  if constexpr (is_bf16<E>::value) {
    return __builtin_bit_cast(float, w << 16);
  } else {
    return __builtin_bit_cast(float, w);
  }
}

// Issue the loads of time index t (tapes and upstream grads). Every load is issued
// unconditionally: t is clamped to 0, the t - 1 neighbours of t = 0 read row t itself,
// and an absent grad reads a stand-in tensor of the same layout. reverse_step masks those
// values at use (Scal::gpresent, t > 0), so no select on a pending load forces a wait.
template <typename E>
__device__ __forceinline__ void load_tape(const BwdArgs<E>& a, size_t row0, int c, int t,
                                          TapeRaw& r) {
  const size_t H = static_cast<size_t>(a.H);
  const int tc = t > 0 ? t : 0;
  const size_t rt = (row0 + tc) * H + c;
  const size_t ru = (row0 + tc) * 2 * H + c;
  const size_t rtp = tc > 0 ? rt - H : rt;  // row t - 1 (cortisol)
  const size_t rup = tc > 0 ? ru - H : ru;  // budget half of U at t - 1
  r.y = ldraw(a.U, ru);
  r.b_prev = ldraw(a.U, rup);
  r.e_prev = ldraw(a.et, rt);
  r.c_prev = ldraw(a.ctp, rtp);
  r.gate = ldraw(a.st, rt);
  r.p = ldraw(a.pl, rt);
  r.ay = ldraw(a.ay, rt);
  r.c_t = ldraw(a.ctp, rt);
  r.gy0 = ldraw(a.gU ? a.gU : a.U, ru);
  r.gub = ldraw(a.gU ? a.gU : a.U, ru + H);
  r.gc = ldraw(a.gC ? a.gC : a.pl, rt);
  r.gnov = ldraw(a.gN ? a.gN : a.pl, rt);
  r.gp = ldraw(a.gP ? a.gP : a.pl, rt);
  r.gay = ldraw(a.gA ? a.gA : a.pl, rt);
  r.gw = ldraw(a.gW ? a.gW : a.pl, rt);
  r.ge = ldraw(a.gE ? a.gE : a.pl, rt);
}

// Bits of Scal::gpresent: which upstream grads the call provides.
enum : uint32_t { G_U = 1, G_C = 2, G_N = 4, G_P = 8, G_A = 16, G_W = 32, G_E = 64 };

struct Scal {
  float alpha, lam, sig_lam, sup;
  uint32_t gpresent;  // G_* bits
};

// One reverse step at time t, evaluated with the carried budget grad `gbn` without the
// pending pre-activation grad X of step t + 1, the carried energy grad `gen` and the
// cortisol grad `gcn`. The budget grad enters every output affinely, so the outputs
// are returned as (value at X = 0, slope in X); the per-unit parameter accumulators
// receive the X = 0 part here and the X part when X is known.
struct Pending {
  float dgate0, cg, dexpr0, cx, keep_b0, keep_e0, ce, keep_c, gyx, y, a16, a17;
};

template <typename E>
__device__ __forceinline__ Pending reverse_step(const TapeRaw& r, int t, float b0v, float c0v,
                                                const UnitParams& up, const Scal& sc, float gbn,
                                                float gen, float gcn, float (&acc)[19]) {
  const float y = cvt<E>(r.y);
  const float b_prev = t > 0 ? cvt<E>(r.b_prev) : b0v;
  const float e_prev = cvt<E>(r.e_prev);
  const float c_prev = t > 0 ? cvt<E>(r.c_prev) : c0v;
  const float gate = cvt<E>(r.gate);
  const float p = cvt<E>(r.p);
  const float ay = cvt<E>(r.ay);
  const float c_t = cvt<E>(r.c_t);
  auto gin = [&](uint32_t w, uint32_t bit) { return (sc.gpresent & bit) ? cvt<E>(w) : 0.0f; };
  const float gy0 = gin(r.gy0, G_U);
  const float gb_new = gin(r.gub, G_U) + gbn;
  const float gc_new = gcn + gin(r.gc, G_C);
  const float gnov0 = gin(r.gnov, G_N);
  const float gp0 = gin(r.gp, G_P);
  const float gay0 = gin(r.gay, G_A);
  const float gwrite = gin(r.gw, G_W);
  const float geo = gin(r.ge, G_E);

  const float nov = tanhf(fabsf(ay - b_prev));
  const float tanh_b = tanhf(b_prev);
  const float nov_eff = nov * (1.0f - sc.sup * c_t);
  const float k_signal = up.ks * gate + up.ky * y + up.kb * tanh_b + up.kn * nov_eff + up.kbias +
                         up.kc * c_t;
  const float r_signal = up.rs * gate + up.ry * y + up.rb * tanh_b + up.rn * nov_eff + up.rbias +
                         up.rc * c_t;
  const float tanh_k = tanhf(k_signal), tanh_r = tanhf(r_signal);
  const float exp_k = expf(0.5f * tanh_k), exp_r = expf(0.5f * tanh_r);
  const float write_cost = up.kappa * exp_k;
  const float recovery_pre = up.recover * exp_r;
  const float recovery = clamp01(recovery_pre);
  const float rclamp = (recovery_pre >= 0.0f && recovery_pre <= 1.0f) ? 1.0f : 0.0f;
  const float energy_pre = e_prev + recovery * (1.0f - e_prev) - write_cost * p;
  const float ge_pre = gen * ((energy_pre >= 0.0f && energy_pre <= 1.0f) ? 1.0f : 0.0f);
  const float g_bprev_state = gb_new * (1.0f - sc.alpha);
  const float g_eprev_state = ge_pre * (1.0f - recovery);
  float gp = gp0 + gb_new * sc.lam * ay - ge_pre * write_cost;
  const float gay = gay0 + gb_new * sc.lam * p;
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
  const float gmask = ((gate > 0.0f) && (gate < 1.0f)) ? (1.0f / 6.0f) : 0.0f;
  const float ge_gate = gp * gate;
  const float stress = nov * (1.0f - e_prev);
  const float c_new = up.decay * c_prev + (1.0f - up.decay) * stress;
  const float g_c_new = gc_new + gc_energy - gnov_eff * nov * sc.sup;
  const float g_stress = g_c_new * (1.0f - up.decay);
  const float g_nov = gnov_eff * (1.0f - sc.sup * c_new) + g_stress * (1.0f - e_prev);
  const float g_e_prev_cort = -g_stress * nov;
  const float diff = ay - b_prev;
  const float d_nov = (gnov0 + g_nov) * (1.0f - nov * nov) * signf_(diff);

  Pending o;
  o.dgate0 = (gp * e_prev + g_gate_energy) * gmask;
  o.cg = sc.lam * ay * e_prev * gmask;
  o.dexpr0 = d_expr_main + d_nov;
  o.cx = sc.lam * p;
  o.keep_b0 = g_bprev_state + gb_energy - d_nov;
  o.keep_e0 = g_eprev_state + ge_gate + g_e_prev_cort + geo;
  o.ce = sc.lam * ay * gate;
  o.keep_c = g_c_new * up.decay;
  o.gyx = gy0 + gy_energy;
  o.y = y;
  o.a16 = (-b_prev) * sc.alpha * (1.0f - sc.alpha);
  o.a17 = (p * ay) * sc.sig_lam;

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
  acc[16] += gb_new * o.a16;
  acc[17] += gb_new * o.a17;
  acc[18] += gnov_eff * nov * (-c_new) * sc.sup * (1.0f - sc.sup);
  return o;
}

// Staged tape prefetch (bf16, 16-unit tiles, H % 16 == 0). The 16 values a reverse step
// reads per (unit, batch) pair come from 16 streams (TapeRaw order). For one tile and
// time they are 16 streams x 16 batch rows x 32 bytes = 512 chunks of 16 bytes, fetched
// with one vector load per chunk by all threads, parked in LDS as [stream][row][unit]
// and read back per pair. Per stream: source tensor (a stand-in of the same layout for an
// absent grad), row stride in units of H, column offset, and whether it reads row t - 1.
constexpr int kTapeStreams = 16;
constexpr int kTapeChunks = kTapeStreams * NB * 2;

template <typename E>
struct TapeStream {
  const E* src;
  int mul;   // row stride in units of H (2 for U and its grad)
  int col;   // column offset (H for the budget half)
  int prev;  // 1: the row of t - 1 (t = 0 reads row 0)
};

template <typename E>
__device__ __forceinline__ TapeStream<E> tape_stream(const BwdArgs<E>& a, int s) {
  const E* gu = a.gU ? a.gU : a.U;
  switch (s) {
    case 0: return {a.U, 2, 0, 0};
    case 1: return {a.U, 2, a.H, 1};
    case 2: return {a.et, 1, 0, 0};
    case 3: return {a.ctp, 1, 0, 1};
    case 4: return {a.st, 1, 0, 0};
    case 5: return {a.pl, 1, 0, 0};
    case 6: return {a.ay, 1, 0, 0};
    case 7: return {a.ctp, 1, 0, 0};
    case 8: return {gu, 2, 0, 0};
    case 9: return {gu, 2, a.H, 0};
    case 10: return {a.gC ? a.gC : a.pl, 1, 0, 0};
    case 11: return {a.gN ? a.gN : a.pl, 1, 0, 0};
    case 12: return {a.gP ? a.gP : a.pl, 1, 0, 0};
    case 13: return {a.gA ? a.gA : a.pl, 1, 0, 0};
    case 14: return {a.gW ? a.gW : a.pl, 1, 0, 0};
    default: return {a.gE ? a.gE : a.pl, 1, 0, 0};
  }
}

// Reverse scan of one workgroup (`bid` among `grid`, as fwd_body).
template <typename E, int CH, int KSTEPS, int NW>
__device__ __forceinline__ void bwd_body(const BwdArgs<E>& a, int bid, int grid) {
  using M = Mf<E>;
  constexpr int NT = NW * 64;
  constexpr int KSTEP = M::KSTEP;
  constexpr int KB = 2 * KSTEPS;  // per-wave k-steps over the 2*KP adjoint input
  // Exchange operands held at once: all KB k-steps, or groups of KC when the weights of a
  // wide tile leave no room (64 fp32 / 16 bf16 k-steps: 64 registers per lane).
  constexpr int KC = KB <= (is_bf16<E>::value ? 16 : 64) ? KB : (is_bf16<E>::value ? 8 : 32);
  static_assert(KB % KC == 0, "exchange groups must divide the k-steps");
  constexpr int MTB = (CH + 15) / 16;
  constexpr int PAIRS = CH * NB;
  constexpr int NACC = 19;
  static_assert(PAIRS <= NT, "one thread per (unit, batch) pair");

  __shared__ __attribute__((aligned(16))) float red[NW][MTB][16][16];  // as in the forward
  __shared__ float accs[NB][CH][NACC];
  __shared__ int s_abort;
  constexpr bool STAGE = is_bf16<E>::value && CH == 16;
  // Staged prefetch: waves 1.. load the chunks (wave 0 polls the step barrier, and a poll
  // waits for every earlier load of its wave).
  constexpr int NL = NT - 64;                                   // loading threads
  constexpr int CPT = STAGE ? (kTapeChunks + NL - 1) / NL : 1;  // chunks per loading thread
  __shared__ __attribute__((aligned(16))) bf16 tape[STAGE ? kTapeStreams : 1][NB][16];
  // Per-unit parameters of the tile, shared by its 16 batch rows: read from LDS at each
  // reverse step instead of holding 17 registers per thread for the whole scan.
  __shared__ UnitParams upar[CH];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int ct, bg;
  tile_of(bid, a.nct, ct, bg);
  const int H = a.H, T = a.T, B = a.B, KP = a.kp;
  uint32_t* err = reinterpret_cast<uint32_t*>(a.ws);
  uint32_t* ctr = group_counters(a.ws, bg);
  uint32_t* counter = my_counter(ctr, a.nct, bid);
  const int nbg = grid / a.nct;
  uint8_t* xbase = a.ws + xchg_offset(nbg) + static_cast<size_t>(bg) * 2 * a.slot_bytes;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(xbase, 2 * a.slot_bytes);
  if (tid == 0) s_abort = 0;

  // A operand: rows = output units j of this tile, k = adjoint input index
  // (k < KP: gate-preactivation grad of unit k; k >= KP: expression grad of unit k-KP).
  typename M::Reg wreg[MTB][KB];
#pragma unroll
  for (int mt = 0; mt < MTB; ++mt) {
    const int jr = mt * 16 + (lane & 15);
    const int j = ct * CH + jr;
    const bool jok = jr < CH && j < H;
    const size_t jrow = static_cast<size_t>(jok ? j : 0) * 2 * H;
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
        wreg[mt][s] = __builtin_bit_cast(bf16x8, v);
      } else {
        const int k = k0 + (lane >> 4);
        const int r = k < KP ? k : H + (k - KP);
        const bool ok = jok && (k < KP ? k < H : (k - KP) < H);
        wreg[mt][s] = ok ? a.GAT[jrow + r] : 0.0f;
      }
    }
  }

  const bool is_pair = tid < PAIRS;
  const int cl = tid % CH, bl = tid / CH;
  const int c = ct * CH + cl, b = bg * NB + bl;
  const bool act = is_pair && c < H && b < B;
  const UnitParams up = load_unit(a.P, c, is_pair && c < H);
  if (is_pair && bl == 0) upar[cl] = up;
  Scal sc;
  sc.alpha = sigmoidf_(a.P.scal[0][0]);
  sc.lam = softplusf_(a.P.scal[1][0]);
  sc.sig_lam = sigmoidf_(a.P.scal[1][0]);
  sc.sup = sigmoidf_(a.P.scal[2][0]);
  sc.gpresent = (a.gU ? G_U : 0u) | (a.gC ? G_C : 0u) | (a.gN ? G_N : 0u) | (a.gP ? G_P : 0u) |
                (a.gA ? G_A : 0u) | (a.gW ? G_W : 0u) | (a.gE ? G_E : 0u);
  const size_t bh = static_cast<size_t>(b) * H + c;
  const float b0v = act ? a.b0[bh] : 0.0f;
  const float c0v = act ? a.c0[bh] : 0.0f;
  float acc[NACC];
#pragma unroll
  for (int i = 0; i < NACC; ++i) acc[i] = 0.0f;
  const size_t row0 = static_cast<size_t>(b) * static_cast<size_t>(a.ldt);
  // Load coordinates: threads without a (unit, batch) pair read row 0, unit 0 (values
  // unused), so the tape loads need no branch.
  const size_t lrow0 = act ? row0 : 0;
  const int lc = act ? c : 0;
  const int kb2[2] = {ct * CH, KP + ct * CH};

  // Staged prefetch: per chunk, its stream and the element offset of its time-0 row
  // (batch rows beyond B read batch 0; their values are never used).
  // Per chunk: the address of its time-0 element, its row stride (elements) and whether
  // it reads the row of t - 1.
  const E* ch_ptr[CPT];
  uint32_t ch_rs[CPT];
  bool ch_prev[CPT];
  const int lt = tid - 64;  // loading thread index (waves 1..)
  if constexpr (STAGE) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int q = min(max(lt, 0) + i * NL, kTapeChunks - 1);
      const int sidx = q / (NB * 2), r = (q / 2) % NB, hh = q & 1;
      const TapeStream<E> ts = tape_stream(a, sidx);
      const int bb = bg * NB + r;
      const size_t brow = static_cast<size_t>(bb < B ? bb : 0) * static_cast<size_t>(a.ldt);
      ch_rs[i] = static_cast<uint32_t>(ts.mul * H);
      ch_ptr[i] = ts.src + brow * ch_rs[i] + ts.col + ct * 16 + hh * 8;
      ch_prev[i] = ts.prev != 0;
    }
  }
  // 16-byte chunk loads of time t (clamped to 0; a t - 1 stream at t = 0 reads row 0).
  auto load_chunks = [&](int t, u32x4 (&v)[CPT]) {
    const int tc = t > 0 ? t : 0;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int tr = ch_prev[i] && tc > 0 ? tc - 1 : tc;
      v[i] = gload16(ch_ptr[i] + static_cast<size_t>(tr) * ch_rs[i]);
    }
  };
  auto park_chunks = [&](const u32x4 (&v)[CPT]) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int q = lt + i * NL;
      if (lt >= 0 && q < kTapeChunks)
        *reinterpret_cast<u32x4*>(&tape[q / (NB * 2)][(q / 2) % NB][(q & 1) * 8]) = v[i];
    }
  };
  auto read_parked = [&]() {
    uint32_t w[kTapeStreams];
#pragma unroll
    for (int k = 0; k < kTapeStreams; ++k) w[k] = tape[STAGE ? k : 0][bl % NB][cl % 16];
    TapeRaw r;
    r.y = w[0]; r.b_prev = w[1]; r.e_prev = w[2]; r.c_prev = w[3];
    r.gate = w[4]; r.p = w[5]; r.ay = w[6]; r.c_t = w[7];
    r.gy0 = w[8]; r.gub = w[9]; r.gc = w[10]; r.gnov = w[11];
    r.gp = w[12]; r.gay = w[13]; r.gw = w[14]; r.ge = w[15];
    return r;
  };
  u32x4 chunk[CPT];

  // Staged output stores (as the forward's tapes): a step's three outputs per pair -- gWgx
  // and da_y of t, gWx of t + 1 -- are parked in LDS (two buffers, alternating by step) and
  // written out as 16-byte chunks during the next step by waves 1.., so the polling wave 0
  // has no stores queued ahead of its counter polls.
  constexpr int GSN = 3;
  constexpr int GCH = GSN * NB * 2;                     // chunks per step
  constexpr int GCPT = STAGE ? (GCH + NL - 1) / NL : 1;  // chunks per loading thread
  __shared__ __attribute__((aligned(16))) bf16 gpark[STAGE ? 2 : 1][STAGE ? GSN : 1][NB][16];
  E* g_ptr[GCPT];
  int g_q[GCPT];
  if constexpr (STAGE) {
#pragma unroll
    for (int i = 0; i < GCPT; ++i) {
      const int q = lt + i * NL;
      const int sidx = q / (NB * 2), r = (q / 2) % NB, hh = q & 1;
      const int bb = bg * NB + r;
      const bool ok = lt >= 0 && q < GCH && bb < B;
      E* const dst[GSN] = {a.gWgx, a.day, a.gWx};
      g_q[i] = ok ? q : -1;
      g_ptr[i] = ok ? dst[sidx] + static_cast<size_t>(bb) * static_cast<size_t>(a.ldt) * H +
                          ct * 16 + hh * 8
                    : nullptr;
    }
  }
  // Write out the outputs parked at step n (time t): gWx of t + 1 only for n > 0.
  auto gflush = [&](int n, int t) {
#pragma unroll
    for (int i = 0; i < GCPT; ++i) {
      const int q = g_q[i];
      const int sidx = q / (NB * 2);
      if (q >= 0 && (sidx < 2 || n > 0))
        gstore16(g_ptr[i] + static_cast<size_t>(sidx < 2 ? t : t + 1) * H,
                 *reinterpret_cast<const u32x4*>(&gpark[n & 1][sidx][(q / 2) % NB][(q & 1) * 8]));
    }
  };

  // Pipeline state at the top of the step for time t: dg/dx are the final adjoint inputs
  // of t, keep_* the final carried grads towards t - 1 (budget without the pre-activation
  // grad of t), gyx/yv the pieces of the pre-activation grad of t, xprev the
  // pre-activation grad of t + 1 (not yet stored), nxt the raw tapes of t - 1.
  float dg = 0.f, dx = 0.f, keep_b = 0.f, keep_e = 0.f, keep_c = 0.f, gyx = 0.f, yv = 0.f;
  float xprev = 0.f;
  TapeRaw nxt = {};
  if (T > 0 && act) {
    TapeRaw cur = {};
    load_tape(a, row0, c, T - 1, cur);
    if (T > 1) load_tape(a, row0, c, T - 2, nxt);
    const float gbF = a.gbF ? a.gbF[bh] : 0.0f;
    const float geF = a.geF ? a.geF[bh] : 0.0f;
    const float gcF = a.gcF ? a.gcF[bh] : 0.0f;
    const Pending pd = reverse_step<E>(cur, T - 1, b0v, c0v, up, sc, gbF, geF, gcF, acc);
    if constexpr (STAGE) {
      // The tapes of T - 2 go where the staged prefetch parks later steps' tapes.
      const uint32_t w[kTapeStreams] = {nxt.y, nxt.b_prev, nxt.e_prev, nxt.c_prev, nxt.gate,
                                        nxt.p, nxt.ay, nxt.c_t, nxt.gy0, nxt.gub, nxt.gc,
                                        nxt.gnov, nxt.gp, nxt.gay, nxt.gw, nxt.ge};
#pragma unroll
      for (int k = 0; k < kTapeStreams; ++k) tape[k][bl][cl] = static_cast<bf16>(w[k]);
    }
    dg = pd.dgate0;
    dx = pd.dexpr0;
    keep_b = pd.keep_b0;
    keep_e = pd.keep_e0;
    keep_c = pd.keep_c;
    gyx = pd.gyx;
    yv = pd.y;
  }

  for (int n = 0; n < T; ++n) {
    const int t = T - 1 - n;
    // Staged: the tapes of t - 1, fetched during the previous step, go to LDS; the barrier
    // inside the publish makes them visible (step 0 uses the tapes loaded before the loop).
    if constexpr (STAGE) {
      if (n > 0) park_chunks(chunk);
    }
    {
      const float v[2] = {dg, dx};
      publish<E, CH, 2>(xr, a.slot_bytes, n & 1, kb2, v, is_pair, cl, bl);
      if (tid == 0) arrive(counter);
    }
    // Staged: the tapes of t - 2 are requested right after the exchange stores drained, so
    // they have the whole step to land before the next step parks them (the next drain
    // waits for every load of the wave).
    if constexpr (STAGE) {
      if (wave > 0) load_chunks(t - 2, chunk);
    }
    // Off the critical path: outputs of t (and the pre-activation grad of t + 1) and the
    // X = 0 part of the reverse step at t - 1.
    if constexpr (STAGE) {
      if (n > 0) gflush(n - 1, t + 1);
      if (is_pair) {
        gpark[n & 1][0][bl][cl] = f2bf(dg);
        gpark[n & 1][1][bl][cl] = f2bf(dx);
        gpark[n & 1][2][bl][cl] = f2bf(xprev);
      }
    }
    Pending pd = {};
    if (act) {
      if constexpr (!STAGE) {
        const size_t rt = (row0 + t) * H + c;
        st(a.gWgx, rt, dg);
        st(a.day, rt, dx);
        if (n > 0) st(a.gWx, rt + H, xprev);
      }
      if (t >= 1) {
        const UnitParams upl = upar[cl];
        if constexpr (STAGE) {
          pd = reverse_step<E>(read_parked(), t - 1, b0v, c0v, upl, sc, keep_b, keep_e, keep_c, acc);
        } else {
          pd = reverse_step<E>(nxt, t - 1, b0v, c0v, upl, sc, keep_b, keep_e, keep_c, acc);
        }
      }
    }
    if (wave == 0) {
      if (!wait_step(ctr, a.nct, static_cast<uint32_t>(n + 1), err) && tid == 0) s_abort = 1;
    }
    __syncthreads();
    if (s_abort) return;

    const uint32_t sbase = static_cast<uint32_t>(n & 1) * a.slot_bytes;
    f32x4 accm[MTB];
#pragma unroll
    for (int mt = 0; mt < MTB; ++mt) accm[mt] = (f32x4){0.f, 0.f, 0.f, 0.f};
    if constexpr (KC == KB) {
      typename M::Reg breg[KB];
#pragma unroll
      for (int s = 0; s < KB; ++s)
        breg[s] = M::load_x(xr, sbase + static_cast<uint32_t>((wave * KB + s) * 64 + lane) * M::UNIT);
      // Keep every exchange load ahead of the first MFMA (all in flight at once).
      __builtin_amdgcn_sched_barrier(0);
      // Unstaged: tapes of t - 2 are requested after the exchange loads. Completions are
      // counted in issue order and the loads are unconditional in every wave (clamped
      // indices), so the waits before the MFMAs count the exchange loads exactly and do not
      // wait for these.
      if constexpr (!STAGE) load_tape(a, lrow0, lc, t - 2, nxt);
#pragma unroll
      for (int s = 0; s < KB; ++s) {
#pragma unroll
        for (int mt = 0; mt < MTB; ++mt) accm[mt] = M::mma(wreg[mt][s], breg[s], accm[mt]);
      }
    } else {
      // Wide tiles: the exchange operands come in groups of KC k-steps (the weights already
      // fill most of the registers), the products in the same order as above.
      if constexpr (!STAGE) load_tape(a, lrow0, lc, t - 2, nxt);
#pragma unroll
      for (int s0 = 0; s0 < KB; s0 += KC) {
        typename M::Reg breg[KC];
#pragma unroll
        for (int s = 0; s < KC; ++s)
          breg[s] = M::load_x(
              xr, sbase + static_cast<uint32_t>((wave * KB + s0 + s) * 64 + lane) * M::UNIT);
#pragma unroll
        for (int s = 0; s < KC; ++s) {
#pragma unroll
          for (int mt = 0; mt < MTB; ++mt)
            accm[mt] = M::mma(wreg[mt][s0 + s], breg[s], accm[mt]);
        }
      }
    }
#pragma unroll
    for (int mt = 0; mt < MTB; ++mt) {
      *reinterpret_cast<f32x4*>(&red[wave][mt][lane & 15][(lane >> 4) * 4]) = accm[mt];
    }
    __syncthreads();
    if (act) {
      float adj = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; ++w) adj += red[w][cl >> 4][bl][cl & 15];
      adj = round_to<E>(adj);
      const float gy = gyx + adj;
      const float x = gy * (1.0f - yv * yv);  // pre-activation grad of t (gWx)
      if (t >= 1) {
        dg = pd.dgate0 + x * pd.cg;
        dx = pd.dexpr0 + x * pd.cx;
        keep_b = pd.keep_b0 + x * (1.0f - sc.alpha);
        keep_e = pd.keep_e0 + x * pd.ce;
        keep_c = pd.keep_c;
        acc[0] += x;
        acc[16] += x * pd.a16;
        acc[17] += x * pd.a17;
        gyx = pd.gyx;
        yv = pd.y;
      } else {
        keep_b += x;
      }
      xprev = x;
    }
  }

  if constexpr (STAGE) {
    // The last step's parked outputs (made visible by that step's barriers).
    if (T > 0) gflush(T - 1, 0);
  }
  if (act) {
    if (T > 0) st(a.gWx, row0 * H + c, xprev);
    a.gb0[bh] = T > 0 ? keep_b : (a.gbF ? a.gbF[bh] : 0.0f);
    a.ge0[bh] = T > 0 ? keep_e : (a.geF ? a.geF[bh] : 0.0f);
    a.gc0[bh] = T > 0 ? keep_c : (a.gcF ? a.gcF[bh] : 0.0f);
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
    a.part_scal[static_cast<size_t>(bid) * 3 + tid] = s;
  }
}

template <typename E, int CH, int KSTEPS, int NW>
__global__ void __launch_bounds__(NW * 64, 1) core_fwd_kernel(FwdArgs<E> a) {
  fwd_body<E, CH, KSTEPS, NW>(a, blockIdx.x, gridDim.x);
}

// One-step scans (T == 1) have no exchange: y_0 = E(tanh(Wx_0 + b_0)) for every (batch
// row, unit) (y0_kernel), the recurrent products of all rows at once as one GEMM
// [B, H] x [2H, H]^T (gemm.hpp), then every unit's step from them (step1_kernel) through
// the same budget_next / energy_next as the scan.
template <typename E>
__global__ void __launch_bounds__(256) y0_kernel(FwdArgs<E> a, E* y0) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i == 0) *reinterpret_cast<uint32_t*>(a.ws) = 0u;  // error word: no barriers to time out
  if (i >= static_cast<int64_t>(a.B) * a.H) return;
  const int b = static_cast<int>(i / a.H), c = static_cast<int>(i % a.H);
  st(y0, static_cast<size_t>(i),
     tanhf(ld(a.Wx, static_cast<size_t>(b) * static_cast<size_t>(a.ldt) * a.ldx + c) +
           ld_state(a.b0, static_cast<size_t>(i), a.sbf)));
}

template <typename E>
__global__ void __launch_bounds__(256) step1_kernel(FwdArgs<E> a, const float* G) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int H = a.H;
  if (i >= static_cast<int64_t>(a.B) * H) return;
  const int b = static_cast<int>(i / H), c = static_cast<int>(i % H);
  const UnitParams up = load_unit(a.P, c, true);
  const StepGains sg = load_gains(a.P);
  const float sb = ld_state(a.b0, i, a.sbf), se = ld_state(a.e0, i, a.sbf),
              sc = ld_state(a.c0, i, a.sbf);
  const size_t row0 = static_cast<size_t>(b) * static_cast<size_t>(a.ldt);
  const size_t rt = row0 * H + c;
  const size_t rx = row0 * a.ldx + c;
  const float y = tanhf(ld(a.Wx, rx) + sb);
  // The reference's recurrent GEMM returns the activation dtype.
  const float ug = round_to<E>(G[static_cast<size_t>(b) * 2 * H + c]);
  const float ay = round_to<E>(G[static_cast<size_t>(b) * 2 * H + H + c]);
  float s_g, p, nov, cpost;
  const float bn = budget_next(up, sg, sb, se, ld(a.Wgx, rx), ug, ay, s_g, p);
  const float en = energy_next(up, sg, sb, se, sc, y, s_g, p, ay, nov, cpost);
  const size_t ru = row0 * 2 * H + c;
  st(a.U, ru, y);
  st(a.U, ru + H, bn);
  st(a.nov, rt, nov);
  st(a.pl, rt, p);
  st(a.ay, rt, ay);
  st(a.wr, rt, p * ay);
  st(a.et, rt, se);
  st(a.ctp, rt, cpost);
  st(a.st, rt, gate_tape_value<E>(s_g));
  st_state(a.bF, i, bn, a.sbf);
  st_state(a.eF, i, en, a.sbf);
  st_state(a.cF, i, cpost, a.sbf);
}

template <typename E, int CH, int KSTEPS, int NW>
__global__ void __launch_bounds__(NW * 64, 1) core_bwd_kernel(BwdArgs<E> a) {
  bwd_body<E, CH, KSTEPS, NW>(a, blockIdx.x, gridDim.x);
}

// ---------------------------------------------------------------------------
// Host side: configuration, workspace and launch.
// ---------------------------------------------------------------------------
struct Cfg {
  int ch = 0, ksteps = 0, kp = 0, nct = 0, nbg = 0, nw = 0;
  int plain_cus = 0;  // > 0: plain launches on a stream owning that many CUs (see the header)
};

// Channel tile width for bf16 beyond H = 1024 (channels per workgroup).
#ifndef DABSN_CORE_CH_WIDE
#define DABSN_CORE_CH_WIDE 16
#endif

static Cfg pick(int dtype, int64_t B, int64_t H) {
  Cfg c;
  const int kstep = dtype == kBF16 ? 32 : 4;
  // Beyond H = 1024, 8 waves, each holding half as many weights (bf16 up to H = 4096 with
  // 16 k-steps of 32 per wave, fp32 up to H = 2048 with 64 k-steps of 4).
  c.nw = H > 1024 ? 8 : 4;
  const int need = static_cast<int>((H + c.nw * kstep - 1) / (c.nw * kstep));
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
  c.kp = c.nw * c.ksteps * kstep;
  c.ch = (dtype == kBF16 && H >= 1024) ? (H > 1024 ? DABSN_CORE_CH_WIDE : 16) : 8;
  c.nct = static_cast<int>((H + c.ch - 1) / c.ch);
  c.nbg = static_cast<int>((B + NB - 1) / NB);
  return c;
}

static size_t slot_bytes(int dtype, const Cfg& c, bool backward) {
  const size_t e = dtype == kBF16 ? 2 : 4;
  return (backward ? 2 : 1) * static_cast<size_t>(c.kp) * NB * e;
}

// Counters and exchange slots of the scan kernels (cleared before every scan).
static size_t scan_bytes(int dtype, const Cfg& c, bool backward) {
  return xchg_offset(c.nbg) + static_cast<size_t>(c.nbg) * 2 * slot_bytes(dtype, c, backward);
}

static size_t align4k(size_t x) { return (x + 4095) / 4096 * 4096; }

// One-step forward scans: y_0 [B][H] in E, then the recurrent products [B][2H] in fp32,
// after the scan region (B rounded up to whole batch groups).
static size_t y0_offset(int dtype, const Cfg& c) { return align4k(scan_bytes(dtype, c, false)); }
static size_t g_offset(int dtype, const Cfg& c, int64_t H) {
  return y0_offset(dtype, c) +
         align4k(static_cast<size_t>(c.nbg) * NB * H * (dtype == kBF16 ? 2 : 4));
}

static size_t workspace_bytes(int dtype, const Cfg& c, bool backward, int64_t H) {
  if (backward) return scan_bytes(dtype, c, true);
  return g_offset(dtype, c, H) + static_cast<size_t>(c.nbg) * NB * 2 * H * 4;
}

// The persistent kernels need every workgroup resident at once. A cooperative launch
// guarantees it (and the runtime then runs nothing beside it). With plain_cus > 0 the
// caller guarantees it instead: the stream owns plain_cus CUs (a CU-masked stream) on which
// nothing else runs while the scan does, so work on the other CUs can overlap the scan.
// Either way every barrier wait is bounded, so a misplaced launch ends with the error word
// set rather than a hang.
template <typename K, typename A>
static int launch_coop(K kernel, int grid, int threads, const A& args, int plain_cus,
                       hipStream_t stream) {
  int dev = 0;
  DABSN_HIP_CHECK(hipGetDevice(&dev));
  int cus = 0, per_cu = 0, coop = 0;
  DABSN_HIP_CHECK(hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev));
  DABSN_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  DABSN_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0));
  void* kargs[] = {const_cast<A*>(&args)};
  if (plain_cus > 0) {
    if (per_cu * std::min(plain_cus, cus) < grid) {
      dabsn::set_error("core scan needs %d co-resident workgroups but the stream's %d CUs hold %d",
                       grid, plain_cus, per_cu * std::min(plain_cus, cus));
      return DABSN_ERR_UNSUPPORTED;
    }
    DABSN_HIP_CHECK(hipLaunchKernel(reinterpret_cast<const void*>(kernel), dim3(grid),
                                    dim3(threads), kargs, 0, stream));
    return DABSN_OK;
  }
  if (!coop || per_cu * cus < grid) {
    dabsn::set_error(
        "core scan needs %d co-resident workgroups but the device holds %d (%d per CU x %d CUs,"
        " cooperative=%d)",
        grid, per_cu * cus, per_cu, cus, coop);
    return DABSN_ERR_UNSUPPORTED;
  }
  DABSN_HIP_CHECK(hipLaunchCooperativeKernel(reinterpret_cast<const void*>(kernel), dim3(grid),
                                             dim3(threads), kargs, 0, stream));
  return DABSN_OK;
}

// Batch rows are independent, so a batch whose workgroups cannot all be resident at once is
// scanned in slabs of whole batch groups, one cooperative launch per slab, each on the
// rows of its slab (pointer offsets) and the same workspace with its step counters
// cleared in between (the error word at its start is kept).
template <typename P>
static P* adv(P* p, size_t n) {
  return p ? p + n : p;
}

// A carried-state pointer advanced by n elements of the state's type (bf16 when sbf).
template <typename P>
static P* adv_state(P* p, size_t n, int sbf) {
  if (!p || !sbf) return adv(p, n);
  using B = std::conditional_t<std::is_const_v<P>, const uint16_t, uint16_t>;
  return reinterpret_cast<P*>(reinterpret_cast<B*>(p) + n);
}

template <typename E>
static FwdArgs<E> slab_of(const FwdArgs<E>& a, int g0, int ng) {
  FwdArgs<E> s = a;
  const size_t b0 = static_cast<size_t>(g0) * NB, row = static_cast<size_t>(a.ldt) * a.H;
  s.B = static_cast<int>(std::min<size_t>(static_cast<size_t>(ng) * NB, a.B - b0));
  s.Wx = adv(a.Wx, b0 * static_cast<size_t>(a.ldt) * a.ldx);
  s.Wgx = adv(a.Wgx, b0 * static_cast<size_t>(a.ldt) * a.ldx);
  s.b0 = adv_state(a.b0, b0 * a.H, a.sbf);
  s.e0 = adv_state(a.e0, b0 * a.H, a.sbf);
  s.c0 = adv_state(a.c0, b0 * a.H, a.sbf);
  s.U = adv(a.U, b0 * 2 * row);
  for (E** t : {&s.nov, &s.pl, &s.ay, &s.wr, &s.et, &s.ctp, &s.st}) *t = adv(*t, b0 * row);
  s.bF = adv_state(a.bF, b0 * a.H, a.sbf);
  s.eF = adv_state(a.eF, b0 * a.H, a.sbf);
  s.cF = adv_state(a.cF, b0 * a.H, a.sbf);
  return s;
}

template <typename E>
static BwdArgs<E> slab_of(const BwdArgs<E>& a, int g0, int ng) {
  BwdArgs<E> s = a;
  const size_t b0 = static_cast<size_t>(g0) * NB, row = static_cast<size_t>(a.ldt) * a.H;
  s.B = static_cast<int>(std::min<size_t>(static_cast<size_t>(ng) * NB, a.B - b0));
  s.b0 = adv(a.b0, b0 * a.H);
  s.c0 = adv(a.c0, b0 * a.H);
  s.U = adv(a.U, b0 * 2 * row);
  s.gU = adv(a.gU, b0 * 2 * row);
  for (const E** t : {&s.pl, &s.ay, &s.et, &s.ctp, &s.st, &s.gN, &s.gP, &s.gA, &s.gW, &s.gE,
                      &s.gC})
    *t = adv(*t, b0 * row);
  s.gbF = adv(a.gbF, b0 * a.H);
  s.geF = adv(a.geF, b0 * a.H);
  s.gcF = adv(a.gcF, b0 * a.H);
  for (E** t : {&s.gWx, &s.gWgx, &s.day}) *t = adv(*t, b0 * row);
  s.part_vec = adv(a.part_vec, static_cast<size_t>(g0) * 16 * a.H);
  s.part_scal = adv(a.part_scal, static_cast<size_t>(g0) * a.nct * 3);
  s.gb0 = adv(a.gb0, b0 * a.H);
  s.ge0 = adv(a.ge0, b0 * a.H);
  s.gc0 = adv(a.gc0, b0 * a.H);
  return s;
}

template <typename K, typename A>
static int launch_slabs(K kernel, int threads, const Cfg& c, const A& args, hipStream_t stream) {
  int dev = 0, cus = 0, per_cu = 0;
  DABSN_HIP_CHECK(hipGetDevice(&dev));
  DABSN_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  DABSN_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0));
  if (c.plain_cus > 0) cus = std::min(cus, c.plain_cus);
  const int per_launch = per_cu * cus / c.nct;  // batch groups one launch can hold
  if (per_launch < 1 || c.nbg <= per_launch)  // (reports a misfit)
    return launch_coop(kernel, c.nct * c.nbg, threads, args, c.plain_cus, stream);
  for (int g0 = 0; g0 < c.nbg; g0 += per_launch) {
    const int ng = std::min(per_launch, c.nbg - g0);
    if (g0 > 0) {
      const int rc = dabsn_hip_zero(args.ws + kCtrOff, xchg_offset(ng) - kCtrOff, stream);
      if (rc != DABSN_OK) return rc;
    }
    const int rc =
        launch_coop(kernel, c.nct * ng, threads, slab_of(args, g0, ng), c.plain_cus, stream);
    if (rc != DABSN_OK) return rc;
  }
  return DABSN_OK;
}

// Number of cooperative launches launch_slabs makes for this configuration on the
// current device (1 when every batch group fits one launch).
template <typename K>
static int slab_count(K kernel, int threads, const Cfg& c, int64_t* launches) {
  int dev = 0, cus = 0, per_cu = 0;
  DABSN_HIP_CHECK(hipGetDevice(&dev));
  DABSN_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  DABSN_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0));
  const int per_launch = per_cu * cus / c.nct;
  *launches = (per_launch < 1 || c.nbg <= per_launch) ? 1 : (c.nbg + per_launch - 1) / per_launch;
  return DABSN_OK;
}

// (CH, KSTEPS, NW) combinations compiled per dtype.
#define DABSN_CORE_CASES_BF16(X) \
  X(8, 1, 4) X(8, 2, 4) X(8, 4, 4) X(8, 8, 4) X(16, 8, 4) X(16, 8, 8) X(16, 16, 8)
#define DABSN_CORE_CASES_F32(X) \
  X(8, 1, 4) X(8, 2, 4) X(8, 4, 4) X(8, 8, 4) X(8, 16, 4) X(8, 32, 4) X(8, 64, 4) X(8, 64, 8)

// One-step scans: y_0, the recurrent products as one GEMM, the step. Decode batches of a
// few hundred rows give only tens of 128 x 128 tiles (B=256, H=2048: 64 workgroups on 256
// CUs), so such GEMMs take 64 x 64 tiles (256 workgroups); the tile shape does not change
// any output's summation order over K.
template <typename E>
static int launch_one_step(const Cfg& c, const FwdArgs<E>& args, hipStream_t stream) {
  const int dtype = is_bf16<E>::value ? kBF16 : kF32;
  const int64_t H = args.H, n = static_cast<int64_t>(args.B) * H;
  E* y0 = reinterpret_cast<E*>(args.ws + y0_offset(dtype, c));
  float* G = reinterpret_cast<float*>(args.ws + g_offset(dtype, c, H));
  const dim3 grid(static_cast<unsigned>((n + 255) / 256));
  hipLaunchKernelGGL(y0_kernel<E>, grid, dim3(256), 0, stream, args, y0);
  DABSN_HIP_CHECK(hipGetLastError());
  gemm::Args<E, float> g{};
  g.M = args.B; g.N = static_cast<int>(2 * H); g.K = static_cast<int>(H);
  g.A = y0; g.lda = H; g.sA = n;
  g.B = args.GA; g.ldb = H; g.sB = 2 * H * H;
  g.C = G; g.ldc = 2 * H; g.sC = 2 * n;
  g.alpha = 1.0f;
  const int64_t big_tiles = ((g.M + 127) / 128) * ((static_cast<int64_t>(g.N) + 127) / 128);
  if (big_tiles >= 1024)  // four 128 x 128 tiles per CU of MI355X's 256
    DABSN_HIP_CHECK((gemm::launch_shape<E, float, 128, 128, 2, 2>(g, 1, stream)));
  else
    DABSN_HIP_CHECK((gemm::launch_shape<E, float, 64, 64, 2, 2>(g, 1, stream)));
  hipLaunchKernelGGL(step1_kernel<E>, grid, dim3(256), 0, stream, args, G);
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

template <typename E>
static int fwd_dispatch(const Cfg& c, const FwdArgs<E>& args, hipStream_t stream) {
  if (args.T == 1) return launch_one_step(c, args, stream);
#define DABSN_CASE(CHV, KS, NWV)                                                           \
  if (c.ch == CHV && c.ksteps == KS && c.nw == NWV)                                        \
    return launch_slabs(core_fwd_kernel<E, CHV, KS, NWV>, NWV * 64, c, args, stream);
  if constexpr (is_bf16<E>::value) {
    DABSN_CORE_CASES_BF16(DABSN_CASE)
  } else {
    DABSN_CORE_CASES_F32(DABSN_CASE)
  }
#undef DABSN_CASE
  dabsn::set_error("core scan: no kernel for CH=%d KSTEPS=%d NW=%d", c.ch, c.ksteps, c.nw);
  return DABSN_ERR_UNSUPPORTED;
}

template <typename E>
static int bwd_dispatch(const Cfg& c, const BwdArgs<E>& args, hipStream_t stream) {
#define DABSN_CASE(CHV, KS, NWV)                                   \
  if (c.ch == CHV && c.ksteps == KS && c.nw == NWV)                \
    return launch_slabs(core_bwd_kernel<E, CHV, KS, NWV>, NWV * 64, c, args, stream);
  if constexpr (is_bf16<E>::value) {
    DABSN_CORE_CASES_BF16(DABSN_CASE)
  } else {
    DABSN_CORE_CASES_F32(DABSN_CASE)
  }
#undef DABSN_CASE
  dabsn::set_error("core scan backward: no kernel for CH=%d KSTEPS=%d NW=%d", c.ch, c.ksteps,
                   c.nw);
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
  // Step counters are 32-bit: arrivals per counter times steps must not wrap.
  DABSN_REQUIRE(static_cast<uint64_t>(split_arrivals(c.nct, 0)) * static_cast<uint64_t>(T + 1) <
                    (1ull << 32),
                "core scan: T=%lld too long for the 32-bit step counters", (long long)T);
  return DABSN_OK;
}

static int check_fwd(const dabsn_core_fwd_call& f, Cfg& c) {
  c = pick(f.dtype, f.B, f.H);
  DABSN_REQUIRE(f.coresident_cus >= 0, "core scan: coresident_cus must be >= 0");
  c.plain_cus = f.coresident_cus;
  const int rc = check_common(f.dtype, f.B, f.T, f.H, f.params, c, f.workspace_bytes,
                              c.ksteps ? workspace_bytes(f.dtype, c, false, f.H) : 0);
  if (rc != DABSN_OK) return rc;
  DABSN_REQUIRE(f.ldt == 0 || (f.ldt >= f.T && f.B * f.ldt * 2 * f.H < (1ll << 46)),
                "core scan: bad time stride ldt=%lld for T=%lld", (long long)f.ldt,
                (long long)f.T);
  DABSN_REQUIRE(f.ldx == 0 || f.ldx == f.H ||
                    (f.ldx > f.H && f.ldx % 8 == 0 &&
                     f.B * (f.ldt > 0 ? f.ldt : f.T) * f.ldx < (1ll << 46)),
                "core scan: bad input row stride ldx=%lld for H=%lld (H, or above H and a "
                "multiple of 8)", (long long)f.ldx, (long long)f.H);
  DABSN_REQUIRE(f.Wx && f.Wgx && f.GA && f.b0 && f.e0 && f.c0 && f.bF && f.eF && f.cF &&
                    f.workspace,
                "core scan: null pointer argument");
  DABSN_REQUIRE(f.state_dtype == kF32 || f.state_dtype == kBF16,
                "core scan: bad state dtype %d (0 = fp32, 1 = bf16)", f.state_dtype);
  DABSN_REQUIRE(f.T == 0 || (f.U && f.nov && f.plast && f.expr && f.write && f.energy && f.sat &&
                             f.gate),
                "core scan: null tape pointer");
  if (f.dtype == kBF16 && c.ch == 16 && f.T > 0) {
    // The 16-unit bf16 kernels write tapes (and, with 8 waves, read Wx/Wgx) as 16-byte
    // chunks of 8 units.
    DABSN_REQUIRE(f.H % 16 == 0, "core scan: bf16 with H >= 1024 needs H %% 16 == 0 (H=%lld)",
                  (long long)f.H);
    const void* outs[] = {f.U, f.nov, f.plast, f.expr, f.write, f.energy, f.sat, f.gate,
                          f.Wx, f.Wgx};
    for (const void* q : outs)
      DABSN_REQUIRE((reinterpret_cast<uintptr_t>(q) & 15u) == 0,
                    "core scan: bf16 input and tape pointers must be 16-byte aligned");
  }
  return DABSN_OK;
}

static int check_bwd(const dabsn_core_bwd_call& b, Cfg& c) {
  c = pick(b.dtype, b.B, b.H);
  DABSN_REQUIRE(b.coresident_cus >= 0, "core scan backward: coresident_cus must be >= 0");
  c.plain_cus = b.coresident_cus;
  const int rc = check_common(b.dtype, b.B, b.T, b.H, b.params, c, b.workspace_bytes,
                              c.ksteps ? workspace_bytes(b.dtype, c, true, b.H) : 0);
  if (rc != DABSN_OK) return rc;
  DABSN_REQUIRE(b.ldt == 0 || (b.ldt >= b.T && b.B * b.ldt * 2 * b.H < (1ll << 46)),
                "core scan backward: bad time stride ldt=%lld for T=%lld", (long long)b.ldt,
                (long long)b.T);
  DABSN_REQUIRE(b.GAT && b.b0 && b.c0 && b.part_vec && b.part_scal && b.gb0 && b.ge0 && b.gc0 &&
                    b.workspace,
                "core scan backward: null pointer argument");
  DABSN_REQUIRE(b.T == 0 || (b.U && b.plast && b.expr && b.energy && b.sat && b.gate && b.gWx &&
                             b.gWgx && b.day),
                "core scan backward: null tape pointer");
  if (b.dtype == kBF16 && c.ch == 16 && b.T > 0) {
    // The 16-unit bf16 kernels fetch tapes and grads as 16-byte chunks of 8 units.
    DABSN_REQUIRE(b.H % 16 == 0, "core scan backward: bf16 with H >= 1024 needs H %% 16 == 0 (H=%lld)",
                  (long long)b.H);
    const void* streams[] = {b.U, b.plast, b.expr, b.energy, b.sat, b.gate, b.gU, b.gNov,
                             b.gP, b.gAy, b.gW, b.gE, b.gC, b.gWx, b.gWgx, b.day};
    for (const void* q : streams)
      DABSN_REQUIRE(q == nullptr || (reinterpret_cast<uintptr_t>(q) & 15u) == 0,
                    "core scan backward: bf16 tape and grad pointers must be 16-byte aligned");
  }
  return DABSN_OK;
}

static int prepare_fwd(const dabsn_core_fwd_call& f, Cfg& c, hipStream_t stream) {
  const int rc = check_fwd(f, c);
  if (rc != DABSN_OK) return rc;
  if (f.T == 1) return DABSN_OK;  // no counters or exchange; y0_kernel clears the error word
  return dabsn_hip_zero(f.workspace, scan_bytes(f.dtype, c, false), stream);
}

static int prepare_bwd(const dabsn_core_bwd_call& b, Cfg& c, hipStream_t stream) {
  const int rc = check_bwd(b, c);
  if (rc != DABSN_OK) return rc;
  return dabsn_hip_zero(b.workspace, scan_bytes(b.dtype, c, true), stream);
}

template <typename E>
static FwdArgs<E> fwd_args(const dabsn_core_fwd_call& f, const Cfg& c) {
  return FwdArgs<E>{static_cast<int>(f.B), static_cast<int>(f.T), static_cast<int>(f.H), c.nct,
                    f.ldt > 0 ? f.ldt : f.T, f.ldx > 0 ? f.ldx : f.H, static_cast<const E*>(f.Wx),
                    static_cast<const E*>(f.Wgx),
                    static_cast<const E*>(f.GA), to_params(f.params), f.b0, f.e0, f.c0,
                    static_cast<E*>(f.U), static_cast<E*>(f.nov), static_cast<E*>(f.plast),
                    static_cast<E*>(f.expr), static_cast<E*>(f.write), static_cast<E*>(f.energy),
                    static_cast<E*>(f.sat), static_cast<E*>(f.gate), f.bF, f.eF, f.cF,
                    static_cast<uint8_t*>(f.workspace),
                    static_cast<uint32_t>(slot_bytes(f.dtype, c, false)),
                    f.state_dtype == kBF16 ? 1 : 0};
}

template <typename E>
static BwdArgs<E> bwd_args(const dabsn_core_bwd_call& b, const Cfg& c) {
  return BwdArgs<E>{static_cast<int>(b.B), static_cast<int>(b.T), static_cast<int>(b.H), c.nct,
                    c.kp, b.ldt > 0 ? b.ldt : b.T, static_cast<const E*>(b.GAT), to_params(b.params), b.b0, b.c0,
                    static_cast<const E*>(b.U), static_cast<const E*>(b.plast),
                    static_cast<const E*>(b.expr), static_cast<const E*>(b.energy),
                    static_cast<const E*>(b.sat), static_cast<const E*>(b.gate),
                    static_cast<const E*>(b.gU), static_cast<const E*>(b.gNov),
                    static_cast<const E*>(b.gP), static_cast<const E*>(b.gAy),
                    static_cast<const E*>(b.gW), static_cast<const E*>(b.gE),
                    static_cast<const E*>(b.gC), b.gbF, b.geF, b.gcF, static_cast<E*>(b.gWx),
                    static_cast<E*>(b.gWgx), static_cast<E*>(b.day), b.part_vec, b.part_scal,
                    b.gb0, b.ge0, b.gc0, static_cast<uint8_t*>(b.workspace),
                    static_cast<uint32_t>(slot_bytes(b.dtype, c, true))};
}

}  // namespace core
}  // namespace dabsn

using namespace dabsn;
using namespace dabsn::core;

extern "C" {

size_t dabsn_hip_core_scan_workspace_bytes(int dtype, int64_t B, int64_t H, int backward) {
  const Cfg c = pick(dtype, B, H);
  if (c.ksteps == 0) return 0;
  return workspace_bytes(dtype, c, backward != 0, H);
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

int dabsn_hip_core_scan_launches(int dtype, int64_t B, int64_t T, int64_t H, int backward,
                                 int64_t* launches) {
  DABSN_REQUIRE(launches, "core scan launches: null pointer");
  DABSN_REQUIRE(dtype == kF32 || dtype == kBF16, "core scan launches: bad dtype");
  const Cfg c = pick(dtype, B, H);
  if (c.ksteps == 0) {
    dabsn::set_error("core scan: unsupported H=%lld", (long long)H);
    return DABSN_ERR_UNSUPPORTED;
  }
  if (T <= 0 || (T == 1 && !backward)) {
    *launches = 0;  // nothing to scan, or the one-step path (no cooperative launch)
    return DABSN_OK;
  }
#define DABSN_CASE(CHV, KS, NWV)                                                      \
  if (c.ch == CHV && c.ksteps == KS && c.nw == NWV) {                                 \
    if (dtype == kBF16)                                                               \
      return backward ? slab_count(core_bwd_kernel<bf16, CHV, KS, NWV>, NWV * 64, c, launches) \
                      : slab_count(core_fwd_kernel<bf16, CHV, KS, NWV>, NWV * 64, c, launches); \
  }
  DABSN_CORE_CASES_BF16(DABSN_CASE)
#undef DABSN_CASE
#define DABSN_CASE(CHV, KS, NWV)                                                      \
  if (c.ch == CHV && c.ksteps == KS && c.nw == NWV) {                                 \
    if (dtype == kF32)                                                                \
      return backward ? slab_count(core_bwd_kernel<float, CHV, KS, NWV>, NWV * 64, c, launches) \
                      : slab_count(core_fwd_kernel<float, CHV, KS, NWV>, NWV * 64, c, launches); \
  }
  DABSN_CORE_CASES_F32(DABSN_CASE)
#undef DABSN_CASE
  dabsn::set_error("core scan: no kernel for CH=%d KSTEPS=%d NW=%d", c.ch, c.ksteps, c.nw);
  return DABSN_ERR_UNSUPPORTED;
}

int dabsn_hip_core_scan_config(int dtype, int64_t B, int64_t H, int* ch, int* ksteps, int* waves) {
  const Cfg c = pick(dtype, B, H);
  if (c.ksteps == 0) {
    dabsn::set_error("core scan: unsupported H=%lld", (long long)H);
    return DABSN_ERR_UNSUPPORTED;
  }
  if (ch) *ch = c.ch;
  if (ksteps) *ksteps = c.ksteps;
  if (waves) *waves = c.nw;
  return DABSN_OK;
}

int dabsn_hip_core_scan_fwd(int dtype, int64_t B, int64_t T, int64_t H, const void* Wx,
                            const void* Wgx, const void* GA, const dabsn_core_params* params,
                            const float* b0, const float* e0, const float* c0, void* U, void* nov,
                            void* plast, void* expr, void* write, void* energy, void* sat,
                            void* gate, float* bF, float* eF, float* cF, void* workspace,
                            size_t workspace_bytes_, hipStream_t stream) {
  const dabsn_core_fwd_call f{dtype, B, T, H, 0, 0, Wx, Wgx, GA, params, b0, e0, c0, U, nov,
                              plast, expr, write, energy, sat, gate, bF, eF, cF, workspace,
                              workspace_bytes_, kF32, 0};
  return dabsn_hip_core_scan_fwd_call(&f, stream);
}

int dabsn_hip_core_scan_fwd_call(const dabsn_core_fwd_call* f, hipStream_t stream) {
  DABSN_REQUIRE(f, "core scan: null call");
  Cfg c;
  int rc = prepare_fwd(*f, c, stream);
  if (rc != DABSN_OK) return rc;
  if (f->dtype == kBF16) return fwd_dispatch(c, fwd_args<bf16>(*f, c), stream);
  return fwd_dispatch(c, fwd_args<float>(*f, c), stream);
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
  const dabsn_core_bwd_call b{dtype, B, T, H, 0, GAT, params, b0, c0, U, plast, expr, energy,
                              sat, gate, gU, gNov, gP, gAy, gW, gE, gC, gbF, geF, gcF, gWx, gWgx,
                              day, part_vec, part_scal, gb0, ge0, gc0, workspace,
                              workspace_bytes_, 0};
  return dabsn_hip_core_scan_bwd_call(&b, stream);
}

int dabsn_hip_core_scan_bwd_call(const dabsn_core_bwd_call* b, hipStream_t stream) {
  DABSN_REQUIRE(b, "core scan backward: null call");
  Cfg c;
  int rc = prepare_bwd(*b, c, stream);
  if (rc != DABSN_OK) return rc;
  if (b->dtype == kBF16) return bwd_dispatch(c, bwd_args<bf16>(*b, c), stream);
  return bwd_dispatch(c, bwd_args<float>(*b, c), stream);
}

}  // extern "C"
