// Three-way admitted read (short, permanent, induction) over the compact bank ABI.
//
// Reference math: src/dabsn/kernels/admitted.py:9-65 (forward) and 116-239 (analytic
// backward); compact masks compact_admitted.py:176-198; CPU kernels
// cpu_runtime.cpp:321-438 and 479-662. Op boundary: dabsn::admitted_three_way_read_
// compact_flash and its backward op (compact_flash.py:71-107, 181-224).
//
// Structure (per batch row, queries t, bank slots j, width H):
//   S = Q K^T                        MFMA GEMM, fp32, only tiles with an allowed entry
//   softmax rows                     three masked softmaxes from S, key bias, admission,
//                                    cocktail term; writes P_V = sg Ps + pg Pp and
//                                    P_Vn = ig Pi (short and permanent share the values)
//   out = P_V V + P_Vn Vn            one MFMA GEMM over both products
// Backward recomputes S and the row statistics, forms dP = gO V^T, gO Vn^T, the score
// gradient G row by row, then gQ = G K, gK = G^T Q, gV = P_V^T gO, gVn = P_Vn^T gO.
// Every GEMM runs with both operands K-contiguous: operands whose natural layout is not
// (V, Vn, K for the products over slots; G, P_V, P_Vn, Q, gO for the products over
// queries) are first transposed into the workspace, which costs one extra read and write
// of each instead of transposing element by element inside every GEMM tile.
// Tile ranges follow the causal staircase: a query tile only visits bank slots that
// any of its queries may read; a bank tile only visits queries at or after its
// earliest admitted index.
#include <algorithm>
#include <mutex>

#include "../../include/dabsn_hip.h"
#include "capi.hpp"
#include "common.hpp"
#include "gemm.hpp"
#include "transpose.hpp"

namespace dabsn {
namespace read3 {

constexpr int TILE = 128;   // GEMM tile rows (query tiles and bank tiles)
constexpr int RT = 32;      // rows per workgroup in the gradient kernel
constexpr int CC = 1024;    // columns per workgroup in the gradient kernel
constexpr int NTH = 256;

struct Gains {
  const float* p[4];  // short, pad, induct, cocktail
};

__device__ __forceinline__ bool allow_at(int mode, int64_t idx, bool valid, int t) {
  return valid && (mode != 0 || idx <= t);
}
__device__ __forceinline__ bool induct_at(int mode, int64_t idx, bool valid, int t, int T) {
  return valid && (mode != 0 ? idx < T - 1 : idx < t);
}

// Per query tile: nhi = 1 + max allowed slot of the tile's last query; per bank tile:
// tlo = earliest query that may read any slot of the tile. One workgroup per tile, the
// slots split over its threads and combined with a wave/LDS max (min) reduction.
__global__ void __launch_bounds__(256) ranges_kernel(int T, int N, int H, int mode,
                                                     const int64_t* idx, const uint8_t* valid,
                                                     int32_t* rs, int32_t* ro, int32_t* rb) {
  __shared__ int sh[4];
  const int b = blockIdx.y;
  const int QT = (T + TILE - 1) / TILE, BT = (N + TILE - 1) / TILE;
  const int item = blockIdx.x;
  const int64_t* ib = idx + static_cast<size_t>(b) * N;
  const uint8_t* vb = valid + static_cast<size_t>(b) * N;
  const bool query_tile = item < QT;
  int v;
  if (query_tile) {
    const int tl = min(T - 1, item * TILE + TILE - 1);
    v = 0;
    for (int j = threadIdx.x; j < N; j += blockDim.x)
      if (allow_at(mode, ib[j], vb[j] != 0, tl)) v = j + 1;
  } else {
    const int bt = item - QT;
    v = T;
    for (int j = bt * TILE + threadIdx.x; j < min(N, bt * TILE + TILE); j += blockDim.x) {
      if (!vb[j]) continue;
      const int64_t first = mode != 0 ? 0 : (ib[j] < 0 ? 0 : ib[j]);
      v = first < v ? static_cast<int>(first) : v;
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const int o = __shfl_xor(v, m, 64);
    v = query_tile ? max(v, o) : min(v, o);
  }
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  if (threadIdx.x != 0) return;
  v = sh[0];
  for (int w = 1; w < static_cast<int>(blockDim.x >> 6); ++w) v = query_tile ? max(v, sh[w]) : min(v, sh[w]);
  if (query_tile) {
    int32_t* s = rs + (static_cast<size_t>(b) * QT + item) * 3;
    s[0] = 0; s[1] = H; s[2] = v;
    int32_t* o = ro + (static_cast<size_t>(b) * QT + item) * 3;
    o[0] = 0; o[1] = v; o[2] = H;
  } else {
    int32_t* r = rb + (static_cast<size_t>(b) * BT + (item - QT)) * 3;
    r[0] = v; r[1] = T; r[2] = H;
  }
}

// Waves per workgroup of the row kernels; per-row partials of the score gradient are
// kept per (column chunk, wave) and summed by reduce_rows_kernel.
constexpr int NWV = NTH / 64;

__device__ __forceinline__ float block_sum(float v, float* sh) {
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  return (sh[0] + sh[1]) + (sh[2] + sh[3]);
}

struct RowCtx {
  int T, N, mode;
  const float* S;
  const float* kb;
  const float* adm;
  const float* cb;
  const float* ck;
  const int64_t* idx;
  const uint8_t* valid;
  float scale, sg, pg, ig, cg;
};

// Scores of slot j for query t: short = scale*S + kb + adm; perm = short + cg*(ck . cb).
__device__ __forceinline__ void scores(const RowCtx& c, int b, int t, int j, const float* ckt,
                                       float& s_short, float& s_perm, float& cc, float& sraw) {
  const size_t bj = static_cast<size_t>(b) * c.N + j;
  sraw = c.S[(static_cast<size_t>(b) * c.T + t) * c.N + j];
  const float content = sraw * c.scale + c.kb[bj];
  const float* cbj = c.cb + bj * 4;
  cc = ckt[0] * cbj[0] + ckt[1] * cbj[1] + ckt[2] * cbj[2] + ckt[3] * cbj[3];
  s_short = content + c.adm[bj];
  s_perm = content + cc * c.cg + c.adm[bj];
}

// Online (max, sum) update of one softmax with score x.
__device__ __forceinline__ void online_add(float x, float& m, float& l) {
  if (x > m) {
    l = l * __expf(m - x) + 1.0f;  // m = -inf gives l * 0 + 1
    m = x;
  } else {
    l += __expf(x - m);
  }
}

// Online (max, sum) update of one softmax with UC scores at once (-inf for masked ones):
// one rescale to the group's new maximum, then the group's terms, so a lane evaluates
// UC + 1 exponentials per group (and no branch that diverges whenever some lane's maximum
// grows).
template <int U>
__device__ __forceinline__ void online_add_group(const float (&x)[U], float& m, float& l) {
  float g = x[0];
#pragma unroll
  for (int u = 1; u < U; ++u) g = fmaxf(g, x[u]);
  const float mn = fmaxf(m, g);
  if (mn == -INFINITY) return;  // every score so far masked: l stays 0
  float acc = l * __expf(m - mn);  // m = -inf: l = 0 and exp(-inf) = 0
#pragma unroll
  for (int u = 0; u < U; ++u) acc += __expf(x[u] - mn);
  l = acc;
  m = mn;
}

// Combine the per-lane (max, sum) of one softmax across the wave.
__device__ __forceinline__ void wave_softmax_stats(float& m, float& l) {
  const float M = wave_max(m);
  l = (m == -INFINITY) ? 0.0f : l * __expf(m - M);
  l = wave_sum(l);
  m = M;
}

// Row statistics (max and sum of each masked softmax), one wave per query row.
// stats[row] = (m_s, l_s, m_p, l_p, m_i, l_i); l = 0 marks an empty pathway.
// When P_V is non-null also writes P_V / P_Vn for j < nhi of the row's tile. With a
// successor fold (`fold` non-null; see SuccFold) the induction weight of slot j is added to
// P_V at column j + fold[j] instead of being written to P_Vn (not written).
template <typename E>
__global__ void __launch_bounds__(NTH) softmax_fwd_kernel(int64_t rows, RowCtx c, Gains g,
                                                          const float* scale_p, const int32_t* rs,
                                                          const int8_t* fold, float* stats, E* PV,
                                                          E* PVn) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * NWV + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int b = static_cast<int>(row / c.T), t = static_cast<int>(row % c.T);
  c.scale = scale_p[0];
  c.sg = g.p[0][0]; c.pg = g.p[1][0]; c.ig = g.p[2][0]; c.cg = g.p[3][0];
  const int QT = (c.T + TILE - 1) / TILE;
  const int nhi = rs[(static_cast<size_t>(b) * QT + t / TILE) * 3 + 2];
  const float* ckt = c.ck + static_cast<size_t>(row) * 4;
  const int64_t* ib = c.idx + static_cast<size_t>(b) * c.N;
  const uint8_t* vb = c.valid + static_cast<size_t>(b) * c.N;
  float ms = -INFINITY, mp = -INFINITY, mi = -INFINITY, ls = 0.f, lp = 0.f, li = 0.f;
  for (int j = lane; j < nhi; j += 64) {
    float ss, sp, cc, sr;
    scores(c, b, t, j, ckt, ss, sp, cc, sr);
    if (allow_at(c.mode, ib[j], vb[j] != 0, t)) {
      online_add(ss, ms, ls);
      online_add(sp, mp, lp);
    }
    if (induct_at(c.mode, ib[j], vb[j] != 0, t, c.T)) online_add(ss, mi, li);
  }
  wave_softmax_stats(ms, ls);
  wave_softmax_stats(mp, lp);
  wave_softmax_stats(mi, li);
  if (lane == 0) {
    float* o = stats + static_cast<size_t>(row) * 6;
    o[0] = ms; o[1] = ls; o[2] = mp; o[3] = lp; o[4] = mi; o[5] = li;
  }
  if (PV == nullptr) return;
  const float is = ls > 0.f ? 1.0f / ls : 0.f, ip = lp > 0.f ? 1.0f / lp : 0.f,
              ii = li > 0.f ? 1.0f / li : 0.f;
  const int8_t* fb = fold ? fold + static_cast<size_t>(b) * c.N : nullptr;
  // Folded: the weight slot j hands to column j + 1 reaches lane + 1 by a shuffle, and
  // lane 63's to lane 0 of the next 64 columns through `carry`. A weight is non-zero only
  // when slot j's induction is allowed, which makes slot j + 1 readable by this query, so
  // column j + 1 < nhi and nothing is carried past the row's last column.
  float carry = 0.f;
  for (int j0 = 0; j0 < nhi; j0 += 64) {
    const int j = j0 + lane;
    float pv = 0.f, pn = 0.f;
    int fj = 0;
    if (j < nhi) {
      float ss, sp, cc, sr;
      scores(c, b, t, j, ckt, ss, sp, cc, sr);
      if (allow_at(c.mode, ib[j], vb[j] != 0, t)) pv = c.sg * (__expf(ss - ms) * is) + c.pg * (__expf(sp - mp) * ip);
      if (induct_at(c.mode, ib[j], vb[j] != 0, t, c.T)) pn = c.ig * (__expf(ss - mi) * ii);
      if (fb) fj = fb[j];
    }
    const size_t o = static_cast<size_t>(row) * c.N + j;
    if (fb) {
      const float ahead = fj == 1 ? pn : 0.f;
      float from_prev = __shfl_up(ahead, 1, 64);
      if (lane == 0) from_prev = carry;
      carry = __shfl(ahead, 63, 64);
      if (j < nhi) st(PV, o, (pv + (fj == 0 ? pn : 0.f)) + from_prev);
    } else if (j < nhi) {
      st(PV, o, pv);
      st(PVn, o, pn);
    }
  }
}

// Per-slot operands of the row kernels, packed once per read (32 bytes, two 16-byte loads):
// key bias + admission, the bank cocktail, and the two mask limits -- slot j is readable by
// query t when alim <= t and enters the induction softmax when ilim < t (INT_MAX: never,
// INT_MIN: always), which is allow_at / induct_at of its index and validity.
struct alignas(16) SlotPack {
  float kbadm, c0, c1, c2, c3;
  int alim, ilim, pad;
};

__global__ void __launch_bounds__(256) pack_kernel(int T, int N, int mode, const float* kb,
                                                   const float* adm, const float* cb,
                                                   const int64_t* idx, const uint8_t* valid,
                                                   SlotPack* pk) {
  const int b = blockIdx.y;
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= N) return;
  const size_t bj = static_cast<size_t>(b) * N + j;
  SlotPack s;
  s.kbadm = kb[bj] + adm[bj];
  s.c0 = cb[bj * 4 + 0];
  s.c1 = cb[bj * 4 + 1];
  s.c2 = cb[bj * 4 + 2];
  s.c3 = cb[bj * 4 + 3];
  const int64_t i = idx[bj];
  const int ii = static_cast<int>(i < INT_MIN ? INT_MIN : (i > INT_MAX ? INT_MAX : i));
  if (valid[bj] == 0) {
    s.alim = s.ilim = INT_MAX;
  } else if (mode != 0) {
    s.alim = INT_MIN;
    s.ilim = i < T - 1 ? INT_MIN : INT_MAX;
  } else {
    s.alim = ii;
    s.ilim = ii;
  }
  s.pad = 0;
  pk[bj] = s;
}

// Query rows per wave of the grouped row kernels: RW consecutive rows of one batch row share
// the slot loads and the slot limit of their 128-row tile (RW divides TILE). Measured at
// config 4 with the grouped loads below: 2 rows per wave for both (4 slowed the softmax).
constexpr int RW_SOFTMAX = 2, RW_GRAD = 2;
static_assert(TILE % RW_SOFTMAX == 0 && TILE % RW_GRAD == 0,
              "row groups must not straddle a query tile");
// 64-column groups a row kernel loads together: every load of UC groups is issued (at
// clamped, in-row addresses) before any of them is used, so a wave waits for one memory
// round trip per UC groups instead of one per dependent load of every group. Each lane
// still visits its columns in increasing order, so the sums are the same as one group at
// a time.
constexpr int UC = 4;

// softmax_fwd_kernel for RW rows per wave: the row statistics and (PV non-null) P_V / P_Vn,
// with the slot operands read once per RW rows from the pack. P_V and P_Vn are written up
// to the row's write limit jlim = min(N, roundup(nhi, TILE)), zeros in [nhi, jlim): the
// backward's transposed GEMMs read whole 128-slot tiles of the P_V this call leaves.
template <typename E, int RW, bool FOLD>
__global__ void __launch_bounds__(NTH) softmax_fwd_rows_kernel(int B, RowCtx c, Gains g,
                                                               const float* scale_p,
                                                               const int32_t* rs,
                                                               const SlotPack* pk,
                                                               const int8_t* fold, float* stats,
                                                               E* PV, E* PVn) {
  const int lane = threadIdx.x & 63;
  const int groups = (c.T + RW - 1) / RW;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * NWV + (threadIdx.x >> 6);
  if (gid >= static_cast<int64_t>(B) * groups) return;
  const int b = static_cast<int>(gid / groups), t0 = static_cast<int>(gid % groups) * RW;
  const int nr = min(RW, c.T - t0);
  const float scale = scale_p[0], sg = g.p[0][0], pg = g.p[1][0], ig = g.p[2][0], cg = g.p[3][0];
  const int QT = (c.T + TILE - 1) / TILE;
  const int nhi = rs[(static_cast<size_t>(b) * QT + t0 / TILE) * 3 + 2];
  const size_t row0 = static_cast<size_t>(b) * c.T + t0;
  float ck[RW][4], ms[RW], ls[RW], mp[RW], lp[RW], mi[RW], li[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
#pragma unroll
    for (int k = 0; k < 4; ++k) ck[r][k] = r < nr ? c.ck[(row0 + r) * 4 + k] : 0.f;
    ms[r] = mp[r] = mi[r] = -INFINITY;
    ls[r] = lp[r] = li[r] = 0.f;
  }
  const SlotPack* pb = pk + static_cast<size_t>(b) * c.N;
  const float* Sr = c.S + row0 * c.N;
  for (int j0 = lane; j0 < nhi; j0 += 64 * UC) {
    SlotPack spu[UC];
    float sv[UC][RW];
#pragma unroll
    for (int u = 0; u < UC; ++u) {
      const int j = min(j0 + 64 * u, nhi - 1);
      spu[u] = pb[j];
#pragma unroll
      for (int r = 0; r < RW; ++r) sv[u][r] = Sr[static_cast<size_t>(min(r, nr - 1)) * c.N + j];
    }
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      if (r >= nr) continue;
      const int t = t0 + r;
      float xs[UC], xp[UC], xi[UC];
#pragma unroll
      for (int u = 0; u < UC; ++u) {
        const SlotPack& sp = spu[u];
        const bool in = j0 + 64 * u < nhi;
        const float ss = sv[u][r] * scale + sp.kbadm;
        const float cc = ck[r][0] * sp.c0 + ck[r][1] * sp.c1 + ck[r][2] * sp.c2 + ck[r][3] * sp.c3;
        const bool al = in && sp.alim <= t, il = in && sp.ilim < t;
        xs[u] = al ? ss : -INFINITY;
        xp[u] = al ? ss + cc * cg : -INFINITY;
        xi[u] = il ? ss : -INFINITY;
      }
      online_add_group(xs, ms[r], ls[r]);
      online_add_group(xp, mp[r], lp[r]);
      online_add_group(xi, mi[r], li[r]);
    }
  }
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    wave_softmax_stats(ms[r], ls[r]);
    wave_softmax_stats(mp[r], lp[r]);
    wave_softmax_stats(mi[r], li[r]);
    if (lane == 0 && r < nr) {
      float* o = stats + (row0 + r) * 6;
      o[0] = ms[r]; o[1] = ls[r]; o[2] = mp[r]; o[3] = lp[r]; o[4] = mi[r]; o[5] = li[r];
    }
  }
  if (PV == nullptr) return;
  float is[RW], ip[RW], ii[RW], carry[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    is[r] = ls[r] > 0.f ? 1.0f / ls[r] : 0.f;
    ip[r] = lp[r] > 0.f ? 1.0f / lp[r] : 0.f;
    ii[r] = li[r] > 0.f ? 1.0f / li[r] : 0.f;
    carry[r] = 0.f;
  }
  const int8_t* fb = FOLD ? fold + static_cast<size_t>(b) * c.N : nullptr;
  const int jlim = min(c.N, ((nhi + TILE - 1) / TILE) * TILE);
  // Folded: as softmax_fwd_kernel, per row (the induction weight of slot j moves to column
  // j + 1 through a lane shuffle, lane 63's to the next 64 columns through carry[r]).
  for (int g0 = 0; g0 < jlim; g0 += 64 * UC) {
    SlotPack spu[UC];
    int fju[UC];
    float sv[UC][RW];
#pragma unroll
    for (int u = 0; u < UC; ++u) {
      const int j = g0 + 64 * u + lane;
      const int jc = j < nhi ? j : 0;
      spu[u] = pb[jc];
      fju[u] = FOLD ? fb[jc] : 0;
#pragma unroll
      for (int r = 0; r < RW; ++r) sv[u][r] = Sr[static_cast<size_t>(min(r, nr - 1)) * c.N + jc];
    }
#pragma unroll
    for (int u = 0; u < UC; ++u) {
      const int j0 = g0 + 64 * u;
      if (j0 >= jlim) break;
      const int j = j0 + lane;
      const bool in = j < nhi, out = j < jlim;
      const SlotPack& sp = spu[u];
      const int fj = in ? fju[u] : 0;
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        if (r >= nr) continue;
        const int t = t0 + r;
        float pv = 0.f, pn = 0.f;
        if (in) {
          const float ss = sv[u][r] * scale + sp.kbadm;
          const float cc = ck[r][0] * sp.c0 + ck[r][1] * sp.c1 + ck[r][2] * sp.c2 + ck[r][3] * sp.c3;
          if (sp.alim <= t)
            pv = sg * (__expf(ss - ms[r]) * is[r]) + pg * (__expf(ss + cc * cg - mp[r]) * ip[r]);
          if (sp.ilim < t) pn = ig * (__expf(ss - mi[r]) * ii[r]);
        }
        const size_t o = (row0 + r) * c.N + j;
        if constexpr (FOLD) {
          const float ahead = fj == 1 ? pn : 0.f;
          float from_prev = __shfl_up(ahead, 1, 64);
          if (lane == 0) from_prev = carry[r];
          carry[r] = __shfl(ahead, 63, 64);
          if (out) st(PV, o, (pv + (fj == 0 ? pn : 0.f)) + from_prev);
        } else if (out) {
          st(PV, o, pv);
          st(PVn, o, pn);
        }
      }
    }
  }
}

// Per-row reductions needed by the score gradient, rowA = (sum Ps dPV, sum Pp dPV,
// sum Pi dPVn) unscaled by the gains, for RW rows per wave with the packed slot operands
// (with a successor fold the induction term reads column j + fold[j] of dP_V).
template <int RW, bool FOLD>
__global__ void __launch_bounds__(NTH) grad_rows_grouped_kernel(int B, RowCtx c, Gains g,
                                                                const float* scale_p,
                                                                const int32_t* rs_rng,
                                                                const SlotPack* pk,
                                                                const float* stats,
                                                                const int8_t* fold,
                                                                const float* dPV,
                                                                const float* dPVn, float* rowA) {
  const int lane = threadIdx.x & 63;
  const int groups = (c.T + RW - 1) / RW;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * NWV + (threadIdx.x >> 6);
  if (gid >= static_cast<int64_t>(B) * groups) return;
  const int b = static_cast<int>(gid / groups), t0 = static_cast<int>(gid % groups) * RW;
  const int nr = min(RW, c.T - t0);
  const float scale = scale_p[0], cg = g.p[3][0];
  const int QT = (c.T + TILE - 1) / TILE;
  const int nhi = rs_rng[(static_cast<size_t>(b) * QT + t0 / TILE) * 3 + 2];
  const size_t row0 = static_cast<size_t>(b) * c.T + t0;
  float ck[RW][4], m[RW][3], inv[RW][3], acc[RW][3];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const float* st6 = stats + (row0 + min(r, nr - 1)) * 6;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      m[r][k] = st6[2 * k];
      inv[r][k] = st6[2 * k + 1] > 0.f ? 1.0f / st6[2 * k + 1] : 0.f;
      acc[r][k] = 0.f;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) ck[r][k] = c.ck[(row0 + min(r, nr - 1)) * 4 + k];
  }
  const SlotPack* pb = pk + static_cast<size_t>(b) * c.N;
  const int8_t* fb = FOLD ? fold + static_cast<size_t>(b) * c.N : nullptr;
  for (int j0 = lane; j0 < nhi; j0 += 64 * UC) {
    // The induction term reads dP_Vn[:, j], which with a successor fold is dP_V[:, j + 1]
    // (fold code 1) or dP_V[:, j] (code 0): both candidates are loaded, the code selects.
    SlotPack spu[UC];
    int dn[UC];
    float sv[UC][RW], dv[UC][RW], nv[UC][RW];
#pragma unroll
    for (int u = 0; u < UC; ++u) {
      const int j = min(j0 + 64 * u, nhi - 1);
      const int jn = FOLD ? min(j + 1, c.N - 1) : j;
      spu[u] = pb[j];
      dn[u] = FOLD ? fb[j] : 0;
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        const size_t o = (row0 + min(r, nr - 1)) * c.N;
        sv[u][r] = c.S[o + j];
        dv[u][r] = dPV[o + j];
        nv[u][r] = FOLD ? dPV[o + jn] : dPVn[o + j];
      }
    }
#pragma unroll
    for (int u = 0; u < UC; ++u) {
      if (j0 + 64 * u >= nhi) continue;
      const SlotPack& sp = spu[u];
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        if (r >= nr) continue;
        const int t = t0 + r;
        const float ss = sv[u][r] * scale + sp.kbadm;
        if (sp.alim <= t) {
          const float cc = ck[r][0] * sp.c0 + ck[r][1] * sp.c1 + ck[r][2] * sp.c2 + ck[r][3] * sp.c3;
          const float d = dv[u][r];
          acc[r][0] += __expf(ss - m[r][0]) * inv[r][0] * d;
          acc[r][1] += __expf(ss + cc * cg - m[r][1]) * inv[r][1] * d;
        }
        if (sp.ilim < t)
          acc[r][2] += __expf(ss - m[r][2]) * inv[r][2] * (FOLD && dn[u] == 0 ? dv[u][r] : nv[u][r]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const float a0 = wave_sum(acc[r][0]), a1 = wave_sum(acc[r][1]), a2 = wave_sum(acc[r][2]);
    if (lane == 0 && r < nr) {
      float* o = rowA + (row0 + r) * 3;
      o[0] = a0; o[1] = a1; o[2] = a2;
    }
  }
}

// Four consecutive values of E stored with one 8-byte (bf16) or 16-byte (fp32) store.
template <typename E>
__device__ __forceinline__ void st4(E* p, float a, float b, float c, float d);
template <>
__device__ __forceinline__ void st4<bf16>(bf16* p, float a, float b, float c, float d) {
  const uint32_t lo = static_cast<uint32_t>(f2bf(a)) | (static_cast<uint32_t>(f2bf(b)) << 16);
  const uint32_t hi = static_cast<uint32_t>(f2bf(c)) | (static_cast<uint32_t>(f2bf(d)) << 16);
  *reinterpret_cast<uint2*>(p) = make_uint2(lo, hi);
}
template <>
__device__ __forceinline__ void st4<float>(float* p, float a, float b, float c, float d) {
  *reinterpret_cast<float4*>(p) = make_float4(a, b, c, d);
}

// Score gradient for a tile of RT rows x CC columns. Writes Gs = scale*G, and P_V / P_Vn
// where those pointers are non-null;
// per-(row, column chunk, wave) partials rowB = (G.S, dSp.cc, cg dSp cb[0..3]) and
// per-(row tile, column) partials colp = (sum G, cg sum dSp ck[0..3]).
// Each thread owns CJ = 4 consecutive columns: their per-slot operands (key bias +
// admission, bank cocktail, index, validity) are loaded once; a row's S / dP_V / dP_Vn
// come as 16-byte loads and its Gs / P_V / P_Vn go out as one vector store each when the
// rows are 16-byte aligned (N % 4 == 0); and the next row's loads are issued before the
// current row is evaluated, so a wave always has a row of loads in flight.
template <typename E>
__global__ void __launch_bounds__(NTH) grad_tile_kernel(RowCtx c, Gains g, const float* scale_p,
                                                        const int32_t* rs_rng, const float* stats,
                                                        const float* rowA, const int8_t* fold,
                                                        const float* dPV, const float* dPVn, E* Gs,
                                                        E* PV, E* PVn, float* rowB, float* colp) {
  constexpr int CJ = CC / NTH;
  static_assert(CJ == 4, "a thread owns one 4-column group");
  const int b = blockIdx.z, rt = blockIdx.y, cch = blockIdx.x;
  const int NCC = (c.N + CC - 1) / CC;
  const int RTILES = (c.T + RT - 1) / RT;
  c.scale = scale_p[0];
  c.sg = g.p[0][0]; c.pg = g.p[1][0]; c.ig = g.p[2][0]; c.cg = g.p[3][0];
  const int QT = (c.T + TILE - 1) / TILE;
  const int t0 = rt * RT, t1 = min(c.T, t0 + RT);
  const int wave = threadIdx.x >> 6;
  const int jb = cch * CC + threadIdx.x * CJ;  // this thread's first column
  // 16-byte rows: the workspace bases are 256-byte aligned, so N % 4 == 0 suffices; the
  // write limits (multiples of 128, or N) then never split a thread's group.
  const bool vec = (c.N & 3) == 0;
  auto jlim_of = [&](int t) {
    const int nhi = rs_rng[(static_cast<size_t>(b) * QT + t / TILE) * 3 + 2];
    // The transposed GEMMs read whole 128-wide slot tiles of any row inside their
    // k-range, so slots in [nhi, roundup(nhi, TILE)) are written as explicit zeros.
    return min(c.N, ((nhi + TILE - 1) / TILE) * TILE);
  };
  // Slot ranges grow with t, so a chunk beyond the last row's limit has nothing to write
  // but zero partials.
  if (cch * CC >= jlim_of(t1 - 1)) {
    for (int t = t0 + wave; t < t1; t += NWV) {
      if ((threadIdx.x & 63) < 6) {
        const size_t row = static_cast<size_t>(b) * c.T + t;
        for (int w = 0; w < NWV; ++w) rowB[((row * NCC + cch) * NWV + w) * 6 + (threadIdx.x & 63)] = 0.f;
      }
    }
#pragma unroll
    for (int q = 0; q < CJ; ++q) {
      const int j = jb + q;
      if (j >= c.N) continue;
      float* o = colp + ((static_cast<size_t>(b) * RTILES + rt) * c.N + j) * 5;
      o[0] = o[1] = o[2] = o[3] = o[4] = 0.f;
    }
    return;
  }
  // Per-row scalars of the tile, staged once: stats (6), row sums (3), cocktail (4), the
  // row's slot limit nhi and write limit jlim.
  __shared__ float rsc[RT][13];
  __shared__ int rlim[RT][2];
  for (int i = threadIdx.x; i < RT * 15; i += NTH) {
    const int r = i / 15, k = i % 15, t = t0 + r;
    if (t >= t1) continue;
    const size_t row = static_cast<size_t>(b) * c.T + t;
    if (k < 6) rsc[r][k] = stats[row * 6 + k];
    else if (k < 9) rsc[r][k] = rowA[row * 3 + (k - 6)];
    else if (k < 13) rsc[r][k] = c.ck[row * 4 + (k - 9)];
    else if (k == 13) rlim[r][0] = rs_rng[(static_cast<size_t>(b) * QT + t / TILE) * 3 + 2];
    else rlim[r][1] = jlim_of(t);
  }
  __syncthreads();
  const int64_t* ib = c.idx + static_cast<size_t>(b) * c.N;
  const uint8_t* vb = c.valid + static_cast<size_t>(b) * c.N;
  // Slot index per column, with invalid slots folded into INT_MAX (no query may read
  // them). Indices are sequence positions (|idx| < 2^31).
  // With a successor fold the induction product of slot j uses column j + fold[j] of dP_V
  // (dP_Vn is not formed).
  float kbadm[CJ], cbv[CJ][4];
  int slot[CJ], dnoff[CJ];
#pragma unroll
  for (int q = 0; q < CJ; ++q) {
    const int j = jb + q;
    const bool ok = j < c.N && vb[min(j, c.N - 1)] != 0;
    const size_t bj = static_cast<size_t>(b) * c.N + min(j, c.N - 1);
    kbadm[q] = c.kb[bj] + c.adm[bj];
    slot[q] = ok ? static_cast<int>(ib[min(j, c.N - 1)]) : INT_MAX;
    dnoff[q] = fold && ok ? fold[bj] : 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) cbv[q][k] = c.cb[bj * 4 + k];
  }
  float colG[CJ], colC[CJ][4];
#pragma unroll
  for (int q = 0; q < CJ; ++q) {
    colG[q] = 0.f;
    colC[q][0] = colC[q][1] = colC[q][2] = colC[q][3] = 0.f;
  }
  float nS[CJ], nD[CJ], nDn[CJ];
  int njl = 0;
  auto fetch = [&](int t) {
    njl = rlim[t - t0][1];
    const size_t rowoff = (static_cast<size_t>(b) * c.T + t) * c.N;
    if (vec && jb < njl) {
      // the whole group is inside the row's write limit (a multiple of 4)
      const float4 s4 = *reinterpret_cast<const float4*>(c.S + rowoff + jb);
      const float4 d4 = *reinterpret_cast<const float4*>(dPV + rowoff + jb);
      nS[0] = s4.x; nS[1] = s4.y; nS[2] = s4.z; nS[3] = s4.w;
      nD[0] = d4.x; nD[1] = d4.y; nD[2] = d4.z; nD[3] = d4.w;
      if (fold) {
        // column j + 1 of the last column: the next group's first (a code of 1 implies
        // that column exists)
        const float d5 = jb + CJ < c.N ? dPV[rowoff + jb + CJ] : 0.f;
        nDn[0] = dnoff[0] ? d4.y : d4.x;
        nDn[1] = dnoff[1] ? d4.z : d4.y;
        nDn[2] = dnoff[2] ? d4.w : d4.z;
        nDn[3] = dnoff[3] ? d5 : d4.w;
      } else {
        const float4 n4 = *reinterpret_cast<const float4*>(dPVn + rowoff + jb);
        nDn[0] = n4.x; nDn[1] = n4.y; nDn[2] = n4.z; nDn[3] = n4.w;
      }
      return;
    }
#pragma unroll
    for (int q = 0; q < CJ; ++q) {
      const int j = jb + q;
      const bool in = j < njl;
      nS[q] = in ? c.S[rowoff + j] : 0.f;
      nD[q] = in ? dPV[rowoff + j] : 0.f;
      nDn[q] = in ? (fold ? dPV[rowoff + j + dnoff[q]] : dPVn[rowoff + j]) : 0.f;
    }
  };
  fetch(t0);
  for (int t = t0; t < t1; ++t) {
    float cS[CJ], cD[CJ], cDn[CJ];
#pragma unroll
    for (int q = 0; q < CJ; ++q) {
      cS[q] = nS[q];
      cD[q] = nD[q];
      cDn[q] = nDn[q];
    }
    const int jlim = njl;
    if (t + 1 < t1) fetch(t + 1);
    const size_t row = static_cast<size_t>(b) * c.T + t;
    const float* sr = rsc[t - t0];
    const int nhi = rlim[t - t0][0];
    const float st6[6] = {sr[0], sr[1], sr[2], sr[3], sr[4], sr[5]};
    const float is = st6[1] > 0.f ? 1.0f / st6[1] : 0.f, ip = st6[3] > 0.f ? 1.0f / st6[3] : 0.f,
                ii = st6[5] > 0.f ? 1.0f / st6[5] : 0.f;
    const float ra = sr[6], rp = sr[7], ri = sr[8];
    const float ck0 = sr[9], ck1 = sr[10], ck2 = sr[11], ck3 = sr[12];
    float gsc = 0.f, gcg = 0.f, gk0 = 0.f, gk1 = 0.f, gk2 = 0.f, gk3 = 0.f;
    float oG[CJ], oV[CJ], oN[CJ];
#pragma unroll
    for (int q = 0; q < CJ; ++q) {
      const int j = jb + q;
      float ps = 0.f, pp = 0.f, pi = 0.f, G = 0.f, dsp = 0.f;
      if (j < nhi) {
        const float cc = ck0 * cbv[q][0] + ck1 * cbv[q][1] + ck2 * cbv[q][2] + ck3 * cbv[q][3];
        const float s_short = cS[q] * c.scale + kbadm[q];
        const float s_perm = s_short + cc * c.cg;
        float dss = 0.f, dsi = 0.f;
        if (allow_at(c.mode, slot[q], slot[q] != INT_MAX, t)) {
          ps = __expf(s_short - st6[0]) * is;
          pp = __expf(s_perm - st6[2]) * ip;
          dss = c.sg * ps * (cD[q] - ra);
          dsp = c.pg * pp * (cD[q] - rp);
        }
        if (induct_at(c.mode, slot[q], slot[q] != INT_MAX, t, c.T)) {
          pi = __expf(s_short - st6[4]) * ii;
          dsi = c.ig * pi * (cDn[q] - ri);
        }
        G = dss + dsp + dsi;
        gsc += G * cS[q];
        gcg += dsp * cc;
        const float w = dsp * c.cg;
        gk0 += w * cbv[q][0]; gk1 += w * cbv[q][1]; gk2 += w * cbv[q][2]; gk3 += w * cbv[q][3];
        colG[q] += G;
        colC[q][0] += w * ck0; colC[q][1] += w * ck1;
        colC[q][2] += w * ck2; colC[q][3] += w * ck3;
      }
      oG[q] = G * c.scale;
      oV[q] = c.sg * ps + c.pg * pp;
      oN[q] = c.ig * pi;
    }
    if (vec && jb < jlim) {
      const size_t o = row * c.N + jb;
      st4(Gs + o, oG[0], oG[1], oG[2], oG[3]);
      if (PV) st4(PV + o, oV[0], oV[1], oV[2], oV[3]);
      if (PVn) st4(PVn + o, oN[0], oN[1], oN[2], oN[3]);
    } else {
#pragma unroll
      for (int q = 0; q < CJ; ++q) {
        if (jb + q >= jlim) continue;
        const size_t o = row * c.N + jb + q;
        st(Gs, o, oG[q]);
        if (PV) st(PV, o, oV[q]);
        if (PVn) st(PVn, o, oN[q]);
      }
    }
    gsc = wave_sum(gsc);
    gcg = wave_sum(gcg);
    gk0 = wave_sum(gk0);
    gk1 = wave_sum(gk1);
    gk2 = wave_sum(gk2);
    gk3 = wave_sum(gk3);
    if ((threadIdx.x & 63) == 0) {
      float* o = rowB + ((row * NCC + cch) * NWV + wave) * 6;
      o[0] = gsc; o[1] = gcg; o[2] = gk0; o[3] = gk1; o[4] = gk2; o[5] = gk3;
    }
  }
#pragma unroll
  for (int q = 0; q < CJ; ++q) {
    const int j = jb + q;
    if (j >= c.N) continue;
    float* o = colp + ((static_cast<size_t>(b) * RTILES + rt) * c.N + j) * 5;
    o[0] = colG[q];
    o[1] = colC[q][0]; o[2] = colC[q][1]; o[3] = colC[q][2]; o[4] = colC[q][3];
  }
}

// Column reductions over row tiles: gkb = gadm = sum G; gcb = cg sum dSp ck.
__global__ void reduce_cols_kernel(int T, int N, const float* colp, float* gkb, float* gadm,
                                   float* gcb) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int b = blockIdx.y;
  if (i >= N) return;
  const int RTILES = (T + RT - 1) / RT;
  float s[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
  for (int r = 0; r < RTILES; ++r) {
    const float* p = colp + ((static_cast<size_t>(b) * RTILES + r) * N + i) * 5;
#pragma unroll
    for (int k = 0; k < 5; ++k) s[k] += p[k];
  }
  const size_t o = static_cast<size_t>(b) * N + i;
  gkb[o] = s[0];
  gadm[o] = s[0];
#pragma unroll
  for (int k = 0; k < 4; ++k) gcb[o * 4 + k] = s[1 + k];
}

// Row reductions: gck[row] = sum over column chunks; scalar partials per block.
__global__ void reduce_rows_kernel(int64_t rows, int NCC, const float* rowA, const float* rowB,
                                   float* gck, float* part) {
  __shared__ float sh[4];
  const int64_t row = static_cast<int64_t>(blockIdx.x) * NTH + threadIdx.x;
  float v[5] = {0.f, 0.f, 0.f, 0.f, 0.f};  // scale, short, pad, induct, cocktail
  if (row < rows) {
    float k4[4] = {0.f, 0.f, 0.f, 0.f};
    for (int cc = 0; cc < NCC * NWV; ++cc) {
      const float* p = rowB + (static_cast<size_t>(row) * NCC * NWV + cc) * 6;
      v[0] += p[0];
      v[4] += p[1];
#pragma unroll
      for (int k = 0; k < 4; ++k) k4[k] += p[2 + k];
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) gck[static_cast<size_t>(row) * 4 + k] = k4[k];
    v[1] = rowA[row * 3];
    v[2] = rowA[row * 3 + 1];
    v[3] = rowA[row * 3 + 2];
  }
#pragma unroll
  for (int k = 0; k < 5; ++k) {
    const float s = block_sum(v[k], sh);
    if (threadIdx.x == 0) part[static_cast<size_t>(blockIdx.x) * 5 + k] = s;
  }
}

// One wave per scalar (5 waves): lane l sums the partials of blocks l, l + 64, ... in
// order, then the wave's lanes are combined in a fixed tree order.
__global__ void __launch_bounds__(320) reduce_final_kernel(int nblocks, const float* part, float* out5) {
  const int k = threadIdx.x >> 6, lane = threadIdx.x & 63;
  float s = 0.f;
  for (int i = lane; i < nblocks; i += 64) s += part[static_cast<size_t>(i) * 5 + k];
  s = wave_sum(s);
  if (lane == 0) out5[k] = s;
}

// Successor fold. The read module's banks hold V[j] = write[idx[j]] and Vn[j] =
// write[next(idx[j])]. When next(idx[j]) is the position of slot j + 1 (consecutive admitted
// positions) Vn[j] is V[j + 1]; when next(idx[j]) = idx[j] (the clamped last position) it is
// V[j]. A fold array of one code per slot, fold[b][j] in {0, 1}, states Vn[j] = V[j +
// fold[j]] for every valid slot; then P_Vn Vn = P_V' V with the induction weights moved to
// column j + fold[j], so the reads and products over Vn disappear: one product in the output
// GEMM, no dP_Vn GEMM (dP_Vn[:, j] = dP_V[:, j + fold[j]]) and no gVn GEMM (its rows are
// part of gV).
//
// out[b][j][t] = PV[b][t][j] + (fold[j] == 0 ? PVn[b][t][j] : 0)
//                            + (fold[j - 1] == 1 ? PVn[b][t][j - 1] : 0),
// a transpose of the folded P_V for the gV GEMM (64 x 64 tiles as xpose::transpose_kernel,
// with the P_Vn tile staged one column wider on the left).
template <typename E>
__global__ void __launch_bounds__(xpose::TNT) fold_transpose_kernel(int R, int C, const E* PV,
                                                                   const E* PVn,
                                                                   const int8_t* fold, E* out,
                                                                   bool aligned) {
  constexpr int TT = xpose::TT, PITCH = TT + 2;
  constexpr int VEC = 16 / static_cast<int>(sizeof(E));  // elements per 16-byte vector
  constexpr int VPR = TT / VEC;                          // vectors per tile row
  // P_V and P_Vn tiles as stored (no rounding on the way in); the P_Vn tile is one column
  // wider on the left (index cc + 1 holds column c0 + cc).
  __shared__ E tpv[TT][PITCH];
  __shared__ E tpn[TT][PITCH];
  __shared__ int8_t fl[TT + 1];
  const int b = blockIdx.z;
  const int r0 = blockIdx.y * TT, c0 = blockIdx.x * TT;
  const E* pv = PV + static_cast<size_t>(b) * R * C;
  const E* pn = PVn + static_cast<size_t>(b) * R * C;
  const int8_t* fb = fold + static_cast<size_t>(b) * C;
  for (int i = threadIdx.x; i < TT + 1; i += xpose::TNT) {
    const int c = c0 - 1 + i;
    fl[i] = (c >= 0 && c < C) ? fb[c] : int8_t(2);  // 2: nothing folds from or into here
  }
  const bool full = aligned && r0 + TT <= R && c0 + TT <= C && (C % VEC) == 0 && (R % VEC) == 0;
  if (full) {
    for (int q = threadIdx.x; q < TT * VPR; q += xpose::TNT) {
      const int r = q / VPR, cv = (q % VPR) * VEC;
      const size_t o = static_cast<size_t>(r0 + r) * C + c0 + cv;
      E a[VEC], n[VEC];
      *reinterpret_cast<u32x4*>(a) = *reinterpret_cast<const u32x4*>(pv + o);
      *reinterpret_cast<u32x4*>(n) = *reinterpret_cast<const u32x4*>(pn + o);
#pragma unroll
      for (int k = 0; k < VEC; ++k) {
        tpv[r][cv + k] = a[k];
        tpn[r][cv + k + 1] = n[k];
      }
    }
    for (int r = threadIdx.x; r < TT; r += xpose::TNT)
      tpn[r][0] = c0 > 0 ? pn[static_cast<size_t>(r0 + r) * C + c0 - 1] : E(0);
  } else {
    for (int q = threadIdx.x; q < TT * (TT + 1); q += xpose::TNT) {
      const int r = q / (TT + 1), i = q % (TT + 1);
      const int rr = r0 + r, c = c0 - 1 + i;
      const bool in = rr < R && c >= 0 && c < C;
      const size_t o = static_cast<size_t>(rr) * C + c;
      tpn[r][i] = in ? pn[o] : E(0);
      if (i > 0) tpv[r][i - 1] = in ? pv[o] : E(0);
    }
  }
  __syncthreads();
  // out[c][r] = P_V[r][c] (+ P_Vn[r][c] when slot c keeps its own successor weight)
  // (+ P_Vn[r][c - 1] when slot c - 1 hands its weight on), summed in fp32 in that order.
  auto value = [&](int r, int c) {
    float v = to_f(tpv[r][c]);
    if (fl[c + 1] == 0) v += to_f(tpn[r][c + 1]);
    if (fl[c] == 1) v += to_f(tpn[r][c]);
    return v;
  };
  E* dst = out + static_cast<size_t>(b) * R * C;
  if (full) {
    for (int q = threadIdx.x; q < TT * VPR; q += xpose::TNT) {
      const int c = q / VPR, rv = (q % VPR) * VEC;
      E e[VEC];
#pragma unroll
      for (int k = 0; k < VEC; ++k) e[k] = from_f<E>(value(rv + k, c));
      *reinterpret_cast<u32x4*>(dst + static_cast<size_t>(c0 + c) * R + r0 + rv) =
          *reinterpret_cast<const u32x4*>(e);
    }
  } else {
    for (int q = threadIdx.x; q < TT * TT; q += xpose::TNT) {
      const int c = q / TT, r = q % TT;
      if (r0 + r < R && c0 + c < C) st(dst, static_cast<size_t>(c0 + c) * R + r0 + r, value(r, c));
    }
  }
}

// Workspace planning.
struct Plan {
  size_t off_S, off_rs, off_ro, off_rb, off_stats, off_PV, off_PVn, off_VT, off_VnT, off_pack,
      end_fwd;
  size_t split;  // end of the kept part: scores, tile ranges, row statistics and P_V
  size_t off_dPV, off_dPVn, off_Gs, off_rowA, off_rowB, off_colp, off_part, off_KT, off_QT,
      off_gOT, off_GsT, off_PVT, off_PVnT, end_bwd;
};

static size_t align_up(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

static Plan plan(int dtype, int64_t B, int64_t T, int64_t N, int64_t H) {
  Plan p{};
  const size_t e = dtype == kBF16 ? 2 : 4;
  const size_t QT = (T + TILE - 1) / TILE, BT = (N + TILE - 1) / TILE;
  const size_t TN = static_cast<size_t>(B) * T * N;
  size_t o = 0;
  p.off_S = o; o = align_up(o + TN * 4);
  p.off_rs = o; o = align_up(o + B * QT * 3 * 4);
  p.off_ro = o; o = align_up(o + B * QT * 3 * 4);
  p.off_rb = o; o = align_up(o + B * BT * 3 * 4);
  p.off_stats = o; o = align_up(o + static_cast<size_t>(B) * T * 6 * 4);
  p.off_PV = o; o = align_up(o + TN * e);
  p.split = o;
  p.off_PVn = o; o = align_up(o + TN * e);
  const size_t NH = static_cast<size_t>(B) * N * H, TH = static_cast<size_t>(B) * T * H;
  p.off_VT = o; o = align_up(o + NH * e);
  p.off_VnT = o; o = align_up(o + NH * e);
  p.off_pack = o; o = align_up(o + static_cast<size_t>(B) * N * sizeof(SlotPack));
  p.end_fwd = o;
  const size_t NCC = (N + CC - 1) / CC, RTILES = (T + RT - 1) / RT;
  p.off_dPV = o; o = align_up(o + TN * 4);
  p.off_dPVn = o; o = align_up(o + TN * 4);
  p.off_Gs = o; o = align_up(o + TN * e);
  p.off_rowA = o; o = align_up(o + static_cast<size_t>(B) * T * 3 * 4);
  p.off_rowB = o; o = align_up(o + static_cast<size_t>(B) * T * NCC * NWV * 6 * 4);
  p.off_colp = o; o = align_up(o + static_cast<size_t>(B) * RTILES * N * 5 * 4);
  p.off_part = o; o = align_up(o + ((static_cast<size_t>(B) * T + NTH - 1) / NTH) * 5 * 4);
  p.off_KT = o; o = align_up(o + NH * e);
  p.off_QT = o; o = align_up(o + TH * e);
  p.off_gOT = o; o = align_up(o + TH * e);
  p.off_GsT = o; o = align_up(o + TN * e);
  p.off_PVT = o; o = align_up(o + TN * e);
  p.off_PVnT = o; o = align_up(o + TN * e);
  p.end_bwd = o;
  return p;
}

// A workspace in two parts. `kept` holds the plan's regions below `split` -- the scores,
// the tile ranges, the row statistics and P_V (folded when the read folds), which a
// forward leaves for a later backward and which that backward only reads; `scratch` holds
// every region from `split` on. A single buffer is the case scratch = kept + split.
struct Ws {
  uint8_t* kept;
  uint8_t* scratch;
  size_t split;
  template <typename X>
  X* at(size_t off) const {
    return reinterpret_cast<X*>(off < split ? kept + off : scratch + (off - split));
  }
};

static Ws single_ws(void* ws, const Plan& p) {
  uint8_t* b = static_cast<uint8_t*>(ws);
  return Ws{b, b + p.split, p.split};
}

template <typename E>
static int forward_impl(int64_t B, int64_t T, int64_t N, int64_t H, const E* q, const E* K,
                        const E* V, const E* Vn, const float* ck, const float* cb, const float* kb,
                        const float* adm, const float* scale, const int64_t* idx,
                        const uint8_t* valid, const int8_t* fold, int mode, Gains g, E* out,
                        const Ws& ws, const Plan& p, bool write_p, hipStream_t stream) {
  const int QT = static_cast<int>((T + TILE - 1) / TILE), BT = static_cast<int>((N + TILE - 1) / TILE);
  float* S = ws.at<float>(p.off_S);
  int32_t* rs = ws.at<int32_t>(p.off_rs);
  int32_t* ro = ws.at<int32_t>(p.off_ro);
  int32_t* rb = ws.at<int32_t>(p.off_rb);
  float* stats = ws.at<float>(p.off_stats);
  E* PV = ws.at<E>(p.off_PV);
  E* PVn = ws.at<E>(p.off_PVn);
  hipLaunchKernelGGL(ranges_kernel, dim3((unsigned)(QT + BT), (unsigned)B), dim3(256), 0, stream,
                     (int)T, (int)N, (int)H, mode, idx, valid, rs, ro, rb);
  DABSN_HIP_CHECK(hipGetLastError());
  {
    gemm::Args<E, float> a{};
    a.M = (int)T; a.N = (int)N; a.K = (int)H;
    a.A = q; a.lda = H; a.sA = T * H;
    a.B = K; a.ldb = H; a.sB = N * H;
    a.C = S; a.ldc = N; a.sC = T * N;
    a.alpha = 1.0f;
    a.ranges = rs; a.mtiles = QT;
    DABSN_HIP_CHECK((gemm::launch<E, float>(a, (int)B, stream)));
  }
  RowCtx c{(int)T, (int)N, mode, S, kb, adm, cb, ck, idx, valid, 0.f, 0.f, 0.f, 0.f, 0.f};
  SlotPack* pk = ws.at<SlotPack>(p.off_pack);
  if (N > 0) {
    hipLaunchKernelGGL(pack_kernel, dim3((unsigned)((N + 255) / 256), (unsigned)B), dim3(256), 0,
                       stream, (int)T, (int)N, mode, kb, adm, cb, idx, valid, pk);
    DABSN_HIP_CHECK(hipGetLastError());
  }
  const int64_t groups = B * ((T + RW_SOFTMAX - 1) / RW_SOFTMAX);
  auto softmax_rows = fold ? softmax_fwd_rows_kernel<E, RW_SOFTMAX, true>
                          : softmax_fwd_rows_kernel<E, RW_SOFTMAX, false>;
  hipLaunchKernelGGL(softmax_rows, dim3((unsigned)((groups + NWV - 1) / NWV)),
                     dim3(NTH), 0, stream, (int)B, c, g, scale, rs, pk, fold, stats,
                     write_p ? PV : static_cast<E*>(nullptr),
                     write_p && !fold ? PVn : static_cast<E*>(nullptr));
  DABSN_HIP_CHECK(hipGetLastError());
  if (!write_p) return DABSN_OK;
  {
    E* VT = ws.at<E>(p.off_VT);
    E* VnT = ws.at<E>(p.off_VnT);
    DABSN_HIP_CHECK(xpose::transpose<E>(V, VT, (int)B, (int)N, (int)H, stream));
    if (!fold) DABSN_HIP_CHECK(xpose::transpose<E>(Vn, VnT, (int)B, (int)N, (int)H, stream));
    gemm::Args<E, E> a{};  // out = P_V V + P_Vn Vn (folded: P_V' V), B operands as V^T [H][N]
    a.M = (int)T; a.N = (int)H; a.K = (int)N;
    a.A = PV; a.lda = N; a.sA = T * N;
    a.B = VT; a.ldb = N; a.sB = H * N;
    if (!fold) {
      a.A2 = PVn;
      a.B2 = VnT;
    }
    a.C = out; a.ldc = H; a.sC = T * H;
    a.alpha = 1.0f;
    a.ranges = ro; a.mtiles = QT;
    DABSN_HIP_CHECK((gemm::launch<E, E>(a, (int)B, stream)));
  }
  return DABSN_OK;
}

template <typename E>
static int backward_impl(int64_t B, int64_t T, int64_t N, int64_t H, const E* gout, const E* q,
                         const E* K, const E* V, const E* Vn, const float* ck, const float* cb,
                         const float* kb, const float* adm, const float* scale, const int64_t* idx,
                         const uint8_t* valid, const int8_t* fold, int mode, Gains g, E* gq,
                         E* gK, E* gV, E* gVn,
                         float* gck, float* gcb, float* gkb, float* gadm, float* gscal5,
                         const Ws& ws, const Plan& p, bool recompute, hipStream_t stream) {
  // The tile ranges, S and the row statistics: recomputed here, or left in the workspace
  // by the forward call on the same inputs, which also left P_V there (folded when the read
  // folds, zeros up to each row's write limit). Recomputed, P_V and P_Vn are rebuilt below
  // by grad_tile_kernel; kept, only the unfolded read's P_Vn is.
  if (recompute) {
    const int rc = forward_impl<E>(B, T, N, H, q, K, V, Vn, ck, cb, kb, adm, scale, idx, valid,
                                   fold, mode, g, nullptr, ws, p, false, stream);
    if (rc != DABSN_OK) return rc;
  }
  const int QT = static_cast<int>((T + TILE - 1) / TILE), BT = static_cast<int>((N + TILE - 1) / TILE);
  const float* S = ws.at<const float>(p.off_S);
  const int32_t* rs = ws.at<const int32_t>(p.off_rs);
  const int32_t* ro = ws.at<const int32_t>(p.off_ro);
  const int32_t* rb = ws.at<const int32_t>(p.off_rb);
  const float* stats = ws.at<const float>(p.off_stats);
  E* PV = ws.at<E>(p.off_PV);
  E* PVn = ws.at<E>(p.off_PVn);
  float* dPV = ws.at<float>(p.off_dPV);
  float* dPVn = ws.at<float>(p.off_dPVn);
  E* Gs = ws.at<E>(p.off_Gs);
  float* rowA = ws.at<float>(p.off_rowA);
  float* rowB = ws.at<float>(p.off_rowB);
  float* colp = ws.at<float>(p.off_colp);
  float* part = ws.at<float>(p.off_part);
  for (int w = 0; w < (fold ? 1 : 2); ++w) {
    gemm::Args<E, float> a{};
    a.M = (int)T; a.N = (int)N; a.K = (int)H;
    a.A = gout; a.lda = H; a.sA = T * H;
    a.B = w == 0 ? V : Vn; a.ldb = H; a.sB = N * H;
    a.C = w == 0 ? dPV : dPVn; a.ldc = N; a.sC = T * N;
    a.alpha = 1.0f;
    a.ranges = rs; a.mtiles = QT;
    DABSN_HIP_CHECK((gemm::launch<E, float>(a, (int)B, stream)));
  }
  RowCtx c{(int)T, (int)N, mode, S, kb, adm, cb, ck, idx, valid, 0.f, 0.f, 0.f, 0.f, 0.f};
  // The slot pack lives in the forward's scratch, which a kept-workspace forward does not
  // hand over: rebuilt here (B N 32 bytes).
  SlotPack* pk = ws.at<SlotPack>(p.off_pack);
  if (N > 0) {
    hipLaunchKernelGGL(pack_kernel, dim3((unsigned)((N + 255) / 256), (unsigned)B), dim3(256), 0,
                       stream, (int)T, (int)N, mode, kb, adm, cb, idx, valid, pk);
    DABSN_HIP_CHECK(hipGetLastError());
  }
  const int64_t groups = B * ((T + RW_GRAD - 1) / RW_GRAD);
  auto grad_rows = fold ? grad_rows_grouped_kernel<RW_GRAD, true>
                       : grad_rows_grouped_kernel<RW_GRAD, false>;
  hipLaunchKernelGGL(grad_rows, dim3((unsigned)((groups + NWV - 1) / NWV)),
                     dim3(NTH), 0, stream, (int)B, c, g, scale, rs, pk, stats, fold, dPV, dPVn,
                     rowA);
  DABSN_HIP_CHECK(hipGetLastError());
  const int NCC = static_cast<int>((N + CC - 1) / CC), RTILES = static_cast<int>((T + RT - 1) / RT);
  if (N > 0) {
    hipLaunchKernelGGL(grad_tile_kernel<E>, dim3(NCC, RTILES, (unsigned)B), dim3(NTH), 0, stream, c,
                       g, scale, rs, stats, rowA, fold, dPV, dPVn, Gs,
                       recompute ? PV : static_cast<E*>(nullptr),
                       recompute || !fold ? PVn : static_cast<E*>(nullptr), rowB, colp);
    DABSN_HIP_CHECK(hipGetLastError());
  }
  E* KT = ws.at<E>(p.off_KT);
  E* QTr = ws.at<E>(p.off_QT);
  E* gOT = ws.at<E>(p.off_gOT);
  E* GsT = ws.at<E>(p.off_GsT);
  E* PVT = ws.at<E>(p.off_PVT);
  E* PVnT = ws.at<E>(p.off_PVnT);
  DABSN_HIP_CHECK(xpose::transpose<E>(K, KT, (int)B, (int)N, (int)H, stream));
  DABSN_HIP_CHECK(xpose::transpose<E>(q, QTr, (int)B, (int)T, (int)H, stream));
  DABSN_HIP_CHECK(xpose::transpose<E>(gout, gOT, (int)B, (int)T, (int)H, stream));
  DABSN_HIP_CHECK(xpose::transpose<E>(Gs, GsT, (int)B, (int)T, (int)N, stream));
  if (fold && recompute) {
    const dim3 grid((unsigned)((N + xpose::TT - 1) / xpose::TT),
                    (unsigned)((T + xpose::TT - 1) / xpose::TT), (unsigned)B);
    const bool aligned = ((reinterpret_cast<uintptr_t>(PV) | reinterpret_cast<uintptr_t>(PVn) |
                           reinterpret_cast<uintptr_t>(PVT)) & 15u) == 0;
    hipLaunchKernelGGL(fold_transpose_kernel<E>, grid, dim3(xpose::TNT), 0, stream, (int)T,
                       (int)N, PV, PVn, fold, PVT, aligned);
    DABSN_HIP_CHECK(hipGetLastError());
  } else {
    DABSN_HIP_CHECK(xpose::transpose<E>(PV, PVT, (int)B, (int)T, (int)N, stream));
    if (!fold) DABSN_HIP_CHECK(xpose::transpose<E>(PVn, PVnT, (int)B, (int)T, (int)N, stream));
  }
  {
    gemm::Args<E, E> a{};  // gQ = Gs K, B operand as K^T [H][N]
    a.M = (int)T; a.N = (int)H; a.K = (int)N;
    a.A = Gs; a.lda = N; a.sA = T * N;
    a.B = KT; a.ldb = N; a.sB = H * N;
    a.C = gq; a.ldc = H; a.sC = T * H;
    a.alpha = 1.0f;
    a.ranges = ro; a.mtiles = QT;
    DABSN_HIP_CHECK((gemm::launch<E, E>(a, (int)B, stream)));
  }
  // Entries of G, P_V, P_Vn the GEMMs read (rows t >= the bank tile's earliest query,
  // whole 128-slot tiles below roundup(nhi)) are all written, by grad_tile_kernel or the
  // forward's softmax_fwd_rows_kernel; the transposes copy them unchanged.
  const E* lhs[3] = {GsT, PVT, PVnT};
  const E* rhs[3] = {QTr, gOT, gOT};
  E* dst[3] = {gK, gV, gVn};
  for (int w = 0; w < (fold ? 2 : 3); ++w) {
    gemm::Args<E, E> a{};  // gK = Gs^T Q, gV = P_V^T gO, gVn = P_Vn^T gO over k = t
    a.M = (int)N; a.N = (int)H; a.K = (int)T;
    a.A = lhs[w]; a.lda = T; a.sA = N * T;
    a.B = rhs[w]; a.ldb = T; a.sB = H * T;
    a.C = dst[w]; a.ldc = H; a.sC = N * H;
    a.alpha = 1.0f;
    a.ranges = rb; a.mtiles = BT;
    DABSN_HIP_CHECK((gemm::launch<E, E>(a, (int)B, stream)));
  }
  if (N > 0) {
    hipLaunchKernelGGL(reduce_cols_kernel, dim3((unsigned)((N + NTH - 1) / NTH), (unsigned)B),
                       dim3(NTH), 0, stream, (int)T, (int)N, colp, gkb, gadm, gcb);
    DABSN_HIP_CHECK(hipGetLastError());
  }
  const int64_t rows = B * T;
  const int nblk = static_cast<int>((rows + NTH - 1) / NTH);
  hipLaunchKernelGGL(reduce_rows_kernel, dim3(nblk), dim3(NTH), 0, stream, rows, NCC, rowA, rowB,
                     gck, part);
  DABSN_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(reduce_final_kernel, dim3(1), dim3(320), 0, stream, nblk, part, gscal5);
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

}  // namespace read3
}  // namespace dabsn

using namespace dabsn;
using namespace dabsn::read3;

// ---------------------------------------------------------------------------
// Decode read: a few query rows (T <= kDecodeRows) against a long bank, reading the bank's
// write rows in place through an index list and a row stride, with no gathered K/V/Vn
// copies and no transposes. Same masks, softmaxes and dtype policy as forward_impl:
// K = E(write / max(norm, eps)) as bank_gather stores it (here as a product with the
// reciprocal, within one fp32 ulp before the rounding to E), scores in fp32, P_V / P_Vn
// stored in E, the output accumulated in fp32 (per slot split, then summed in split order)
// and stored in E. Inference only (no backward).
// ---------------------------------------------------------------------------
constexpr int kDecodeRows = 8;
constexpr int kDecodeSlotsPerBlock = 16;  // 4 waves x 4 slots
constexpr float kNormEps = 1e-12f;        // as bank_gather

// Bank row of slot index i of batch row b (indices are clamped into the bank).
template <typename E>
__device__ __forceinline__ const E* bank_row(const E* bank, int b, int64_t rowld, int64_t Nb,
                                             int64_t i, int H) {
  const int64_t r = i < 0 ? 0 : (i >= Nb ? Nb - 1 : i);
  return bank + (static_cast<size_t>(b) * rowld + r) * H;
}

// S[b, t, j] = q[b, t] . K_j for every slot j, K_j = E(write_j * (1 / norm_j)) (the
// gather's E(write_j / norm_j) up to one fp32 ulp before the rounding to E). One wave per
// slot; the T query rows of batch row b are staged in LDS (dynamic, T * H elements).
template <typename E>
__global__ void __launch_bounds__(256) decode_score_kernel(int T, int N, int H, int64_t Nb,
                                                           int64_t rowld, const E* q, const E* bank,
                                                           const float* norm_w,
                                                           const int64_t* idx, float* S) {
  extern __shared__ __attribute__((aligned(16))) unsigned char qraw[];
  E* qs = reinterpret_cast<E*>(qraw);
  const int b = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nch = H / 8;  // 8-element chunks per row
  for (int c = tid; c < T * nch; c += 256)
    *reinterpret_cast<u32x4*>(qs + c * 8) =
        *reinterpret_cast<const u32x4*>(q + static_cast<size_t>(b) * T * H + c * 8);
  if constexpr (sizeof(E) == 4) {
    for (int c = tid; c < T * nch; c += 256)
      *reinterpret_cast<u32x4*>(qs + c * 8 + 4) =
          *reinterpret_cast<const u32x4*>(q + static_cast<size_t>(b) * T * H + c * 8 + 4);
  }
  __syncthreads();
  // The wave's slots are processed together so their row loads are in flight at once;
  // slots past N read the last slot's row and are not stored.
  constexpr int KW = kDecodeSlotsPerBlock / 4;
  const int jw = blockIdx.x * kDecodeSlotsPerBlock + wave * KW;
  if (jw >= N) return;  // wave-uniform; no barrier follows
  const E* row[KW];
  float rn[KW];  // 1 / norm, once per slot (the gather divides per element: <= 1 ulp apart)
#pragma unroll
  for (int k = 0; k < KW; ++k) {
    const int j = min(jw + k, N - 1);
    const int64_t i = idx[static_cast<size_t>(b) * N + j];
    const int64_t ic = i < 0 ? 0 : (i >= Nb ? Nb - 1 : i);
    row[k] = bank_row(bank, b, rowld, Nb, i, H);
    rn[k] = 1.0f / fmaxf(norm_w[static_cast<size_t>(b) * Nb + ic], kNormEps);
  }
  float acc[KW][kDecodeRows];
#pragma unroll
  for (int k = 0; k < KW; ++k)
#pragma unroll
    for (int t = 0; t < kDecodeRows; ++t) acc[k][t] = 0.0f;
  for (int c = lane; c < nch; c += 64) {
    float v[KW][8];
#pragma unroll
    for (int k = 0; k < KW; ++k) ldv<E, 8>(row[k] + c * 8, v[k]);
#pragma unroll
    for (int k = 0; k < KW; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e) v[k][e] = round_to<E>(v[k][e] * rn[k]);  // K
#pragma unroll
    for (int t = 0; t < kDecodeRows; ++t) {
      if (t < T) {
        float qv[8];
        ldv<E, 8>(qs + (t * nch + c) * 8, qv);
#pragma unroll
        for (int k = 0; k < KW; ++k)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[k][t] += qv[e] * v[k][e];
      }
    }
  }
#pragma unroll
  for (int k = 0; k < KW; ++k) {
#pragma unroll
    for (int t = 0; t < kDecodeRows; ++t) {
      if (t < T) {
        const float sum = wave_sum(acc[k][t]);
        if (lane == 0 && jw + k < N) S[(static_cast<size_t>(b) * T + t) * N + jw + k] = sum;
      }
    }
  }
}

// part[s][b][t][h] = sum over the slots j < nhi of split s of P_V[t, j] V_j[h] +
// P_Vn[t, j] Vn_j[h], with V_j the bank row of idx[j] and Vn_j that of next_idx[j]. A
// thread owns 8 consecutive h; blocks: (h chunk, b, split).
template <typename E>
__global__ void __launch_bounds__(256) decode_out_kernel(int T, int N, int H, int64_t Nb,
                                                         int64_t rowld, int per_split,
                                                         const E* bank, const int64_t* idx,
                                                         const int64_t* next_idx, const E* PV,
                                                         const E* PVn, const int32_t* rs,
                                                         float* part) {
  const int b = blockIdx.y, s = blockIdx.z;
  const int h0 = (blockIdx.x * 256 + threadIdx.x) * 8;
  if (h0 >= H) return;
  const int QT = (T + TILE - 1) / TILE;
  const int nhi = min(N, rs[(static_cast<size_t>(b) * QT) * 3 + 2]);  // T <= TILE: one tile
  const int j0 = s * per_split, j1 = min(nhi, j0 + per_split);
  float acc[kDecodeRows][8];
#pragma unroll
  for (int t = 0; t < kDecodeRows; ++t)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[t][e] = 0.0f;
  const size_t prow = static_cast<size_t>(b) * T * N;
  // Slots are taken U at a time so their 2U row loads are in flight together; the slots
  // in a group are summed in order, as in the one-at-a-time loop.
  constexpr int U = 4;
  for (int jb = j0; jb < j1; jb += U) {
    float v[U][8], vn[U][8];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = min(jb + u, j1 - 1);
      ldv<E, 8>(bank_row(bank, b, rowld, Nb, idx[static_cast<size_t>(b) * N + j], H) + h0, v[u]);
      ldv<E, 8>(bank_row(bank, b, rowld, Nb, next_idx[static_cast<size_t>(b) * N + j], H) + h0,
                vn[u]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (jb + u < j1) {
        const int j = jb + u;
#pragma unroll
        for (int t = 0; t < kDecodeRows; ++t) {
          if (t < T) {
            const float pv = ld(PV, prow + static_cast<size_t>(t) * N + j);
            const float pn = ld(PVn, prow + static_cast<size_t>(t) * N + j);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[t][e] += pv * v[u][e] + pn * vn[u][e];
          }
        }
      }
    }
  }
#pragma unroll
  for (int t = 0; t < kDecodeRows; ++t) {
    if (t < T) {
      float* o = part + ((static_cast<size_t>(s) * gridDim.y + b) * T + t) * H + h0;
      *reinterpret_cast<f32x4*>(o) = (f32x4){acc[t][0], acc[t][1], acc[t][2], acc[t][3]};
      *reinterpret_cast<f32x4*>(o + 4) = (f32x4){acc[t][4], acc[t][5], acc[t][6], acc[t][7]};
    }
  }
}

// out = sum over splits of part, in split order; 8 elements per thread.
template <typename E>
__global__ void __launch_bounds__(256) decode_reduce_kernel(int64_t chunks, int splits,
                                                            int64_t stride, const float* part,
                                                            E* out) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (c >= chunks) return;
  float acc[8];
  ldv<float, 8>(part + c * 8, acc);
  for (int s = 1; s < splits; ++s) {
    float v[8];
    ldv<float, 8>(part + s * stride + c * 8, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] += v[e];
  }
  stv<E, 8>(out + c * 8, acc);
}

// ---------------------------------------------------------------------------
// One-query decode read in a single pass over the bank (T == 1, H <= 2048): one wave per
// (batch row, slot split) streams its slots' write rows once; each row gives the slot's
// score (K = E(write * 1/norm) as above) and, through online softmaxes, feeds the short,
// permanent and induction accumulators. The induction value of slot j is the row after
// idx[j]; when that row is slot j+1's row (consecutive admitted positions) it is taken
// from the registers that row is already in, one slot later. decode_combine_kernel merges
// the splits' (max, sum, accumulator) triples. Scores and sums are the softmaxes of
// softmax_fwd_kernel evaluated in one pass; the products with V run in fp32 from the
// exact softmax weights (the two-pass path rounds P_V / P_Vn to E first).
// ---------------------------------------------------------------------------
constexpr int kFusedMaxChunks = 4;  // 8-element chunks per lane: H <= 64 * 8 * 4
#ifndef DABSN_DECODE_DEPTH
#define DABSN_DECODE_DEPTH 2  // bf16 row buffers per wave (depth - 1 rows in flight)
#endif

// Per-slot inputs of the single-pass read (8 dwords, read with one scalar load).
struct SlotMeta {
  uint32_t row, nrow;  // bank rows (b * rowld + index) of V and of the induction value
  float rn;            // 1 / max(norm, eps) of the V row
  float kb, adm, ccg;  // key bias, admission, cocktail gain * (cocktail . bank cocktail)
  uint32_t flags;      // bit 0: short / permanent read allowed, bit 1: induction allowed
  uint32_t pad;
};

__global__ void __launch_bounds__(256) decode_meta_kernel(int N, int64_t Nb, int64_t rowld,
                                                          const float* norm_w, const int64_t* idx,
                                                          const int64_t* next_idx,
                                                          const int64_t* read_idx,
                                                          const uint8_t* valid, const float* ck,
                                                          const float* cb, const float* kb,
                                                          const float* adm, Gains g,
                                                          SlotMeta* meta) {
  const int b = blockIdx.y;
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= N) return;
  const size_t bj = static_cast<size_t>(b) * N + j;
  const int64_t i = idx[bj], n = next_idx[bj];
  const int64_t ic = i < 0 ? 0 : (i >= Nb ? Nb - 1 : i);
  const int64_t nc = n < 0 ? 0 : (n >= Nb ? Nb - 1 : n);
  const float* ckt = ck + static_cast<size_t>(b) * 4;
  const float* cbj = cb + bj * 4;
  const float cc = ckt[0] * cbj[0] + ckt[1] * cbj[1] + ckt[2] * cbj[2] + ckt[3] * cbj[3];
  const bool v = valid[bj] != 0;
  SlotMeta m;
  m.row = static_cast<uint32_t>(static_cast<int64_t>(b) * rowld + ic);
  m.nrow = static_cast<uint32_t>(static_cast<int64_t>(b) * rowld + nc);
  m.rn = 1.0f / fmaxf(norm_w[static_cast<size_t>(b) * Nb + ic], kNormEps);
  m.kb = kb[bj];
  m.adm = adm[bj];
  m.ccg = cc * g.p[3][0];
  m.flags = (allow_at(0, read_idx[bj], v, 0) ? 1u : 0u) | (induct_at(0, read_idx[bj], v, 0, 1) ? 2u : 0u);
  m.pad = 0u;
  meta[bj] = m;
}

// The same metadata read straight from a carried bank's kept glue and admitted-slot lists
// (one query row, the bank's last live position Nb - 1): slot j of batch row b is
// members[b, j], valid below max(count[b], 1); next_idx = min(idx + 1, Nb - 1), read_idx =
// idx - qstart, and the bank cocktail, key bias and admission are taken at idx. Every
// per-position array has row stride ld (stats: ld * 6, the write norm in column 5; cocktail:
// ld * 4). Thread 0 of each batch row also writes the row's slot bound nhi = min(N,
// max(count, 1)): every allowed slot is valid, so it bounds them, and slots below it that
// are not allowed carry flags 0.
__global__ void __launch_bounds__(256) decode_meta_members_kernel(
    int N, int64_t Nb, int64_t ld, int64_t qstart, const float* stats, const int64_t* members,
    const int64_t* counts, const float* cocktail, const float* key_bias, const float* admission,
    Gains g, SlotMeta* meta, int32_t* rs) {
  const int b = blockIdx.y;
  const int j = blockIdx.x * 256 + threadIdx.x;
  const int64_t cnt = counts[b] < 1 ? 1 : counts[b];
  if (j == 0) {
    int32_t* s = rs + static_cast<size_t>(b) * 3;
    s[0] = 0;
    s[1] = 0;
    s[2] = static_cast<int32_t>(cnt < N ? cnt : N);
  }
  if (j >= N) return;
  const size_t bl = static_cast<size_t>(b) * ld;
  const int64_t i = members[bl + j];
  const int64_t n = i + 1 < Nb - 1 ? i + 1 : Nb - 1;
  const int64_t ic = i < 0 ? 0 : (i >= Nb ? Nb - 1 : i);
  const int64_t nc = n < 0 ? 0 : n;
  const float* ckt = cocktail + (bl + Nb - 1) * 4;
  const float* cbj = cocktail + (bl + ic) * 4;
  const float cc = ckt[0] * cbj[0] + ckt[1] * cbj[1] + ckt[2] * cbj[2] + ckt[3] * cbj[3];
  const bool v = j < cnt;
  const int64_t ri = i - qstart;
  SlotMeta m;
  m.row = static_cast<uint32_t>(bl + ic);
  m.nrow = static_cast<uint32_t>(bl + nc);
  m.rn = 1.0f / fmaxf(stats[(bl + ic) * 6 + 5], kNormEps);
  m.kb = key_bias[bl + ic];
  m.adm = admission[bl + ic];
  m.ccg = cc * g.p[3][0];
  m.flags = (allow_at(0, ri, v, 0) ? 1u : 0u) | (induct_at(0, ri, v, 0, 1) ? 2u : 0u);
  m.pad = 0u;
  meta[static_cast<size_t>(b) * N + j] = m;
}

// NC chunks of 8 elements of one bank row, chunk k at element 8 * (lane + 64 k) (clamped
// to the row's last chunk; lanes past the row hold a copy and a zero query).
template <typename E, int NC>
struct RowChunks {
  static constexpr int W = sizeof(E) == 2 ? 1 : 2;  // 16-byte words per chunk
  u32x4 d[NC * W];
  __device__ __forceinline__ void load(const E* row, int lane, int nch) {
#pragma unroll
    for (int k = 0; k < NC; ++k) {
      const E* p = row + static_cast<size_t>(min(lane + 64 * k, nch - 1)) * 8;
#pragma unroll
      for (int w = 0; w < W; ++w) d[k * W + w] = gload16(p + w * 4);
    }
  }
  __device__ __forceinline__ void unpack(int k, float (&v)[8]) const {
    if constexpr (W == 1) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[2 * e] = __builtin_bit_cast(float, d[k][e] << 16);
        v[2 * e + 1] = __builtin_bit_cast(float, d[k][e] & 0xffff0000u);
      }
    } else {
      // Whole-vector casts: hipcc's __builtin_bit_cast of a single vector element (an
      // lvalue) reads element 0.
#pragma unroll
      for (int w = 0; w < 2; ++w) {
        const f32x4 f = __builtin_bit_cast(f32x4, d[2 * k + w]);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[4 * w + e] = f[e];
      }
    }
  }
};

// Online softmax step with score x: updates (m, l), returns x's weight and sets `alpha`,
// the factor the accumulator must be scaled by first (1 unless x is a new maximum).
__device__ __forceinline__ float online_weight(float x, float& m, float& l, float& alpha) {
  if (x > m) {
    alpha = __expf(m - x);  // m = -inf: 0
    l = l * alpha + 1.0f;
    m = x;
    return 1.0f;
  }
  alpha = 1.0f;
  const float w = __expf(x - m);
  l += w;
  return w;
}

template <typename E, int NC>
__device__ __forceinline__ void acc_add(float (&acc)[NC][8], const RowChunks<E, NC>& r, float w) {
#pragma unroll
  for (int k = 0; k < NC; ++k) {
    float v[8];
    r.unpack(k, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[k][e] = fmaf(w, v[e], acc[k][e]);
  }
}

template <int NC>
__device__ __forceinline__ void acc_scale(float (&acc)[NC][8], float a) {
#pragma unroll
  for (int k = 0; k < NC; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[k][e] *= a;
}

template <typename E>
struct FusedArgs {
  int N, H, splits, per_split;
  const E* q;
  const E* bank;
  const SlotMeta* meta;
  const int32_t* rs;
  const float* scale;
  float* pacc;    // [waves][3][H]: short, permanent, induction accumulators
  float* pstats;  // [waves][6]: (m, l) of the three softmaxes
};

// Query row b, lane's chunks: bf16 as packed pairs (the score uses v_dot2_f32_bf16 on the
// packed K pairs), fp32 as floats. Chunks past the row are zero.
template <typename E, int NC>
struct QueryChunks {
  static constexpr bool BF = sizeof(E) == 2;
  uint32_t w[BF ? NC * 4 : 1];
  float f[BF ? 1 : NC * 8];
  __device__ __forceinline__ void load(const E* q, int lane, int nch) {
#pragma unroll
    for (int k = 0; k < NC; ++k) {
      const int c = lane + 64 * k;
      if constexpr (BF) {
        const u32x4 u = c < nch ? gload16(q + c * 8) : (u32x4){0u, 0u, 0u, 0u};
#pragma unroll
        for (int e = 0; e < 4; ++e) w[k * 4 + e] = u[e];
      } else {
        float v[8];
        if (c < nch) {
          ldv<E, 8>(q + c * 8, v);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = 0.0f;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) f[k * 8 + e] = v[e];
      }
    }
  }
};

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Lane's part of q . K with K = E(row * rn).
template <typename E, int NC>
__device__ __forceinline__ float row_dot(const RowChunks<E, NC>& r, const QueryChunks<E, NC>& q,
                                         float rn) {
  float dot = 0.0f;
#pragma unroll
  for (int k = 0; k < NC; ++k) {
    if constexpr (sizeof(E) == 2) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t u = r.d[k][e];
        const float lo = __builtin_bit_cast(float, u << 16) * rn;
        const float hi = __builtin_bit_cast(float, u & 0xffff0000u) * rn;
        const bf16x2 kp = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};  // RTNE
        dot = __builtin_amdgcn_fdot2_f32_bf16(kp, __builtin_bit_cast(bf16x2, q.w[k * 4 + e]), dot,
                                              false);
      }
    } else {
      float v[8];
      r.unpack(k, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) dot = fmaf(q.f[k * 8 + e], v[e] * rn, dot);
    }
  }
  return dot;
}

// One wave (= one workgroup) per (batch row b, split s); slots [s * per_split, ...) below
// the row's nhi. Rows stream through D register buffers (D - 1 rows in flight ahead of
// the one in use); the loop is unrolled D times so every buffer keeps a fixed role and no
// in-flight register is copied. Slot metadata comes through scalar loads D slots ahead.
template <typename E, int NC>
__global__ void __launch_bounds__(64) decode_fused_kernel(FusedArgs<E> a) {
  constexpr int D = sizeof(E) == 2 ? DABSN_DECODE_DEPTH : 2;
  static_assert(D == 2 || D == 3 || D == 4, "row buffer depth");
  using Row = RowChunks<E, NC>;
  const int lane = threadIdx.x;
  const int w = blockIdx.x;
  const int b = w / a.splits, s = w % a.splits;
  const int H = a.H, nch = H / 8;
  const int nhi = min(a.N, a.rs[static_cast<size_t>(b) * 3 + 2]);
  const int j0 = s * a.per_split, j1 = min(nhi, j0 + a.per_split);
  const float scale = a.scale[0];
  QueryChunks<E, NC> qc;
  qc.load(a.q + static_cast<size_t>(b) * H, lane, nch);
  float acc[3][NC][8];
#pragma unroll
  for (int p = 0; p < 3; ++p)
#pragma unroll
    for (int k = 0; k < NC; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[p][k][e] = 0.0f;
  float m[3] = {-INFINITY, -INFINITY, -INFINITY}, l[3] = {0.f, 0.f, 0.f};
  const SlotMeta* mb = a.meta + static_cast<size_t>(b) * a.N;
  const size_t rowH = static_cast<size_t>(H);
  float pend_w = 0.0f;     // induction weight of the previous slot, not yet added
  uint32_t pend_row = 0u;  // its induction row
  if (j0 < j1) {
    SlotMeta ring[D];  // metadata of slots j .. j + D - 1
#pragma unroll
    for (int d = 0; d < D; ++d) ring[d] = mb[min(j0 + d, j1 - 1)];
    Row r[D];
#pragma unroll
    for (int d = 0; d < D - 1; ++d) r[d].load(a.bank + ring[d].row * rowH, lane, nch);
    // Slot j with its row in `cur`; requests slot j + D - 1's row into `pf`.
    auto step = [&](Row& cur, Row& pf, int j) __attribute__((always_inline)) {
      const SlotMeta mc = ring[0];
#pragma unroll
      for (int d = 0; d + 1 < D; ++d) ring[d] = ring[d + 1];
      ring[D - 1] = mb[min(j + D, j1 - 1)];
      pf.load(a.bank + ring[D - 2].row * rowH, lane, nch);  // the last slots reread theirs
      // The previous slot's induction value is this slot's row when it is that row (added
      // in the update below); otherwise it is loaded and added here.
      float wi = pend_w;
      if (pend_w != 0.0f && pend_row != mc.row) {
        Row vn;
        vn.load(a.bank + pend_row * rowH, lane, nch);
        acc_add<E, NC>(acc[2], vn, pend_w);
        wi = 0.0f;
      }
      pend_w = 0.0f;
      float ws = 0.0f, wp = 0.0f, as = 1.0f, ap = 1.0f, ai = 1.0f;
      if (mc.flags != 0u) {
        const float sraw = wave_sum(row_dot<E, NC>(cur, qc, mc.rn));
        const float content = sraw * scale + mc.kb;
        const float ss = content + mc.adm;
        const float sp = content + mc.ccg + mc.adm;
        if (mc.flags & 1u) {
          ws = online_weight(ss, m[0], l[0], as);
          wp = online_weight(sp, m[1], l[1], ap);
        }
        if (mc.flags & 2u) {
          pend_w = online_weight(ss, m[2], l[2], ai);
          pend_row = mc.nrow;
        }
      }
      // One pass over the row for the three accumulators: the short and permanent ones
      // rescaled to a new maximum before their term is added, the induction one after the
      // previous slot's term (weighted against the old maximum) is in.
      if (ws != 0.0f || wp != 0.0f || wi != 0.0f) {
        if (as != 1.0f) acc_scale<NC>(acc[0], as);
        if (ap != 1.0f) acc_scale<NC>(acc[1], ap);
#pragma unroll
        for (int k = 0; k < NC; ++k) {
          float v[8];
          cur.unpack(k, v);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            acc[0][k][e] = fmaf(ws, v[e], acc[0][k][e]);
            acc[1][k][e] = fmaf(wp, v[e], acc[1][k][e]);
            acc[2][k][e] = fmaf(wi, v[e], acc[2][k][e]);
          }
        }
      } else {
        if (as != 1.0f) acc_scale<NC>(acc[0], as);
        if (ap != 1.0f) acc_scale<NC>(acc[1], ap);
      }
      if (ai != 1.0f) acc_scale<NC>(acc[2], ai);
    };
    // Whole groups of D slots in a loop with one exit (an exit between the steps would
    // leave the next group's requests in flight on the loop's back edge, and the wait
    // placement would then drain them at the top of every group), the rest after it.
    const int full = j0 + (j1 - j0) / D * D;
    int j = j0;
    if constexpr (D == 4) {
      for (; j < full; j += 4) {
        step(r[0], r[3], j);
        step(r[1], r[0], j + 1);
        step(r[2], r[1], j + 2);
        step(r[3], r[2], j + 3);
      }
      if (j < j1) step(r[0], r[3], j);
      if (j + 1 < j1) step(r[1], r[0], j + 1);
      if (j + 2 < j1) step(r[2], r[1], j + 2);
    } else if constexpr (D == 3) {
      for (; j < full; j += 3) {
        step(r[0], r[2], j);
        step(r[1], r[0], j + 1);
        step(r[2], r[1], j + 2);
      }
      if (j < j1) step(r[0], r[2], j);
      if (j + 1 < j1) step(r[1], r[0], j + 1);
    } else {
      for (; j < full; j += 2) {
        step(r[0], r[1], j);
        step(r[1], r[0], j + 1);
      }
      if (j < j1) step(r[0], r[1], j);
    }
    if (pend_w != 0.0f) {
      Row vn;
      vn.load(a.bank + pend_row * rowH, lane, nch);
      acc_add<E, NC>(acc[2], vn, pend_w);
    }
  }
  float* pa = a.pacc + static_cast<size_t>(w) * 3 * H;
#pragma unroll
  for (int p = 0; p < 3; ++p)
#pragma unroll
    for (int k = 0; k < NC; ++k) {
      const int c = lane + 64 * k;
      if (c < nch) stv<float, 8>(pa + static_cast<size_t>(p) * H + c * 8, acc[p][k]);
    }
  if (lane == 0) {
    float* ps = a.pstats + static_cast<size_t>(w) * 6;
#pragma unroll
    for (int p = 0; p < 3; ++p) {
      ps[2 * p] = m[p];
      ps[2 * p + 1] = l[p];
    }
  }
}

// out[b] = sg * Ps V + pg * Pp V + ig * Pi Vn from the splits' partial softmaxes: each
// split's accumulator is rescaled to the row maximum and divided by the row sum.
// Four columns per thread (B * H / 4 threads: twice the waves of an 8-wide split, for a
// loop that waits on one partial load per split and pathway).
template <typename E>
__global__ void __launch_bounds__(256) decode_combine_kernel(int H, int splits, const float* pacc,
                                                             const float* pstats, Gains g, E* out) {
  const int b = blockIdx.y;
  const int h0 = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (h0 >= H) return;
  const float* st6 = pstats + static_cast<size_t>(b) * splits * 6;
  float M[3] = {-INFINITY, -INFINITY, -INFINITY}, L[3] = {0.f, 0.f, 0.f};
  for (int s = 0; s < splits; ++s)
#pragma unroll
    for (int p = 0; p < 3; ++p)
      if (st6[s * 6 + 2 * p + 1] > 0.f) M[p] = fmaxf(M[p], st6[s * 6 + 2 * p]);
  for (int s = 0; s < splits; ++s)
#pragma unroll
    for (int p = 0; p < 3; ++p) {
      const float ls = st6[s * 6 + 2 * p + 1];
      if (ls > 0.f) L[p] += ls * __expf(st6[s * 6 + 2 * p] - M[p]);
    }
  const float gain[3] = {g.p[0][0], g.p[1][0], g.p[2][0]};
  float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int s = 0; s < splits; ++s) {
#pragma unroll
    for (int p = 0; p < 3; ++p) {
      const float ls = st6[s * 6 + 2 * p + 1];
      if (ls > 0.f) {
        const float c = gain[p] * (__expf(st6[s * 6 + 2 * p] - M[p]) / L[p]);
        const f32x4 v = *reinterpret_cast<const f32x4*>(
            pacc + ((static_cast<size_t>(b) * splits + s) * 3 + p) * H + h0);
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] += c * v[e];
      }
    }
  }
  E* dst = out + static_cast<size_t>(b) * H + h0;
#pragma unroll
  for (int e = 0; e < 4; ++e) st(dst, e, o[e]);
}

struct DecodePlan {
  size_t off_S, off_rs, off_ro, off_rb, off_stats, off_PV, off_PVn, off_part, end;
  int splits, per_split;
  bool fused;
  size_t off_meta, off_pacc, off_pstats;
};

// Workgroups (one wave each) per CU the single-pass read aims for: two waves per SIMD.
constexpr int kFusedWavesPerCU = 8;

static int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return 256;
  return cus;
}

static DecodePlan decode_plan(int dtype, int64_t B, int64_t T, int64_t N, int64_t H) {
  DecodePlan p{};
  const size_t e = dtype == kBF16 ? 2 : 4;
  const size_t QT = (T + TILE - 1) / TILE, BT = (N + TILE - 1) / TILE;
  const size_t TN = static_cast<size_t>(B) * T * N;
  if (T == 1 && H <= 64 * 8 * kFusedMaxChunks) {
    // Single pass: enough (b, split) waves to fill the CUs, at least 16 slots per split.
    p.fused = true;
    const int64_t want = (static_cast<int64_t>(kFusedWavesPerCU) * device_cus() + B - 1) / B;
    const int64_t splits = std::max<int64_t>(1, std::min<int64_t>(want, (N + 15) / 16));
    p.splits = static_cast<int>(splits);
    p.per_split = static_cast<int>((N + splits - 1) / splits);
    size_t o = 0;
    p.off_rs = o; o = align_up(o + B * QT * 3 * 4);
    p.off_ro = o; o = align_up(o + B * QT * 3 * 4);
    p.off_meta = o; o = align_up(o + static_cast<size_t>(B) * N * sizeof(SlotMeta));
    p.off_pacc = o; o = align_up(o + static_cast<size_t>(B) * splits * 3 * H * 4);
    p.off_pstats = o; o = align_up(o + static_cast<size_t>(B) * splits * 6 * 4);
    p.end = o;
    return p;
  }
  const int64_t hblocks = (H + 2047) / 2048;
  // Enough (h chunk, b, split) blocks to keep about 8 per CU with loads in flight, at
  // least 64 slots per split.
  int64_t splits = (2048 + hblocks * B - 1) / (hblocks * B);
  splits = std::max<int64_t>(1, std::min<int64_t>(splits, (N + 63) / 64));
  p.splits = static_cast<int>(splits);
  p.per_split = static_cast<int>((N + splits - 1) / splits);
  size_t o = 0;
  p.off_S = o; o = align_up(o + TN * 4);
  p.off_rs = o; o = align_up(o + B * QT * 3 * 4);
  p.off_ro = o; o = align_up(o + B * QT * 3 * 4);
  p.off_rb = o; o = align_up(o + B * BT * 3 * 4);
  p.off_stats = o; o = align_up(o + static_cast<size_t>(B) * T * 6 * 4);
  p.off_PV = o; o = align_up(o + TN * e);
  p.off_PVn = o; o = align_up(o + TN * e);
  p.off_part = o; o = align_up(o + static_cast<size_t>(splits) * B * T * H * 4);
  p.end = o;
  return p;
}

// The single pass and the split combine, from slot metadata and row bounds already in the
// workspace (decode_meta_kernel after ranges_kernel, or decode_meta_members_kernel).
template <typename E>
static int decode_pass(int64_t B, int64_t N, int64_t H, const E* q, const E* bank,
                       const SlotMeta* meta, const int32_t* rs, const float* scale, Gains g, E* out,
                       uint8_t* ws, const DecodePlan& p, hipStream_t stream) {
  float* pacc = reinterpret_cast<float*>(ws + p.off_pacc);
  float* pstats = reinterpret_cast<float*>(ws + p.off_pstats);
  FusedArgs<E> fa{(int)N, (int)H, p.splits, p.per_split, q, bank, meta, rs, scale, pacc, pstats};
  const dim3 grid((unsigned)(B * p.splits));
  if (H <= 512)
    hipLaunchKernelGGL((decode_fused_kernel<E, 1>), grid, dim3(64), 0, stream, fa);
  else if (H <= 1024)
    hipLaunchKernelGGL((decode_fused_kernel<E, 2>), grid, dim3(64), 0, stream, fa);
  else
    hipLaunchKernelGGL((decode_fused_kernel<E, 4>), grid, dim3(64), 0, stream, fa);
  DABSN_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(decode_combine_kernel<E>, dim3((unsigned)((H + 1023) / 1024), (unsigned)B),
                     dim3(256), 0, stream, (int)H, p.splits, pacc, pstats, g, out);
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

template <typename E>
static int decode_impl(int64_t B, int64_t T, int64_t N, int64_t H, int64_t Nb, int64_t rowld,
                       const E* q, const E* bank, const float* norm_w, const int64_t* idx,
                       const int64_t* next_idx, const int64_t* read_idx, const uint8_t* valid,
                       const float* ck, const float* cb, const float* kb, const float* adm,
                       const float* scale, Gains g, E* out, uint8_t* ws, const DecodePlan& p,
                       hipStream_t stream) {
  const int QT = static_cast<int>((T + TILE - 1) / TILE), BT = static_cast<int>((N + TILE - 1) / TILE);
  if (p.fused) {
    int32_t* rs = reinterpret_cast<int32_t*>(ws + p.off_rs);
    int32_t* ro = reinterpret_cast<int32_t*>(ws + p.off_ro);
    SlotMeta* meta = reinterpret_cast<SlotMeta*>(ws + p.off_meta);
    // Query tiles only (grid QT): nhi per batch row; no bank-tile ranges are needed.
    hipLaunchKernelGGL(ranges_kernel, dim3((unsigned)QT, (unsigned)B), dim3(256), 0, stream,
                       (int)T, (int)N, (int)H, 0, read_idx, valid, rs, ro, nullptr);
    DABSN_HIP_CHECK(hipGetLastError());
    hipLaunchKernelGGL(decode_meta_kernel, dim3((unsigned)((N + 255) / 256), (unsigned)B), dim3(256),
                       0, stream, (int)N, Nb, rowld, norm_w, idx, next_idx, read_idx, valid, ck, cb,
                       kb, adm, g, meta);
    DABSN_HIP_CHECK(hipGetLastError());
    return decode_pass<E>(B, N, H, q, bank, meta, rs, scale, g, out, ws, p, stream);
  }
  float* S = reinterpret_cast<float*>(ws + p.off_S);
  int32_t* rs = reinterpret_cast<int32_t*>(ws + p.off_rs);
  int32_t* ro = reinterpret_cast<int32_t*>(ws + p.off_ro);
  int32_t* rb = reinterpret_cast<int32_t*>(ws + p.off_rb);
  float* stats = reinterpret_cast<float*>(ws + p.off_stats);
  E* PV = reinterpret_cast<E*>(ws + p.off_PV);
  E* PVn = reinterpret_cast<E*>(ws + p.off_PVn);
  float* part = reinterpret_cast<float*>(ws + p.off_part);
  hipLaunchKernelGGL(ranges_kernel, dim3((unsigned)(QT + BT), (unsigned)B), dim3(256), 0, stream,
                     (int)T, (int)N, (int)H, 0, read_idx, valid, rs, ro, rb);
  DABSN_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(decode_score_kernel<E>,
                     dim3((unsigned)((N + kDecodeSlotsPerBlock - 1) / kDecodeSlotsPerBlock), (unsigned)B),
                     dim3(256), static_cast<unsigned>(T * H * sizeof(E)), stream, (int)T, (int)N,
                     (int)H, Nb, rowld, q, bank, norm_w, idx, S);
  DABSN_HIP_CHECK(hipGetLastError());
  RowCtx c{(int)T, (int)N, 0, S, kb, adm, cb, ck, read_idx, valid, 0.f, 0.f, 0.f, 0.f, 0.f};
  hipLaunchKernelGGL(softmax_fwd_kernel<E>, dim3((unsigned)((B * T + NWV - 1) / NWV)), dim3(NTH), 0,
                     stream, B * T, c, g, scale, rs, static_cast<const int8_t*>(nullptr), stats,
                     PV, PVn);
  DABSN_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(decode_out_kernel<E>,
                     dim3((unsigned)((H + 2047) / 2048), (unsigned)B, (unsigned)p.splits), dim3(256), 0,
                     stream, (int)T, (int)N, (int)H, Nb, rowld, p.per_split, bank, idx, next_idx, PV,
                     PVn, rs, part);
  DABSN_HIP_CHECK(hipGetLastError());
  const int64_t chunks = B * T * H / 8;
  hipLaunchKernelGGL(decode_reduce_kernel<E>, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0,
                     stream, chunks, p.splits, B * T * H, part, out);
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

static int read3_checks(int dtype, int64_t B, int64_t T, int64_t N, int64_t H, int mode) {
  DABSN_REQUIRE(dtype == kF32 || dtype == kBF16, "read3: bad dtype %d", dtype);
  DABSN_REQUIRE(mode == 0 || mode == 1, "read3: mode must be 0 (seq) or 1 (field)");
  DABSN_REQUIRE(B > 0 && T > 0 && N >= 0 && H > 0, "read3: bad shape");
  DABSN_REQUIRE(T < (1 << 30) && N < (1 << 30) && H < (1 << 30) && B < 65536,
                "read3: dimension too large");
  DABSN_REQUIRE(B * T * N < (1ll << 40), "read3: score matrix too large");
  return DABSN_OK;
}

extern "C" {

size_t dabsn_hip_read3_workspace_bytes(int dtype, int64_t B, int64_t T, int64_t N, int64_t H,
                                       int part) {
  const Plan p = plan(dtype, B, T, N, H);
  switch (part) {
    case 0: return p.end_fwd;
    case 1: return p.end_bwd;
    case 2: return p.split;
    case 3: return p.end_fwd - p.split;
    case 4: return p.end_bwd - p.split;
    default: return 0;
  }
}

static int read3_fwd_entry(int dtype, int64_t B, int64_t T, int64_t N, int64_t H, const void* q,
                           const void* K, const void* V, const void* Vn, const float* cocktail,
                           const float* bank_cocktail, const float* key_bias,
                           const float* admission, const float* scale, const int64_t* idx,
                           const uint8_t* valid, const int8_t* fold, int mode,
                           const float* const* gains, void* out, void* kept, size_t kept_bytes,
                           void* scratch, size_t scratch_bytes, bool single, hipStream_t stream) {
  const int rc = read3_checks(dtype, B, T, N, H, mode);
  if (rc != DABSN_OK) return rc;
  DABSN_REQUIRE(q && out && cocktail && scale && gains, "read3: null pointer");
  for (int i = 0; i < 4; ++i) DABSN_REQUIRE(gains[i], "read3: null gain %d", i);
  if (N == 0) return dabsn_hip_zero(out, static_cast<size_t>(B * T * H) * (dtype == kBF16 ? 2 : 4), stream);
  DABSN_REQUIRE(K && V && (Vn || fold) && bank_cocktail && key_bias && admission && idx && valid &&
                    kept && (single || scratch),
                "read3: null bank or workspace pointer");
  const Plan p = plan(dtype, B, T, N, H);
  Ws w;
  if (single) {
    DABSN_REQUIRE(kept_bytes >= p.end_fwd, "read3: workspace %zu < %zu", kept_bytes, p.end_fwd);
    w = single_ws(kept, p);
  } else {
    DABSN_REQUIRE(kept_bytes >= p.split && scratch_bytes >= p.end_fwd - p.split,
                  "read3: kept %zu < %zu or scratch %zu < %zu", kept_bytes, p.split,
                  scratch_bytes, p.end_fwd - p.split);
    w = Ws{static_cast<uint8_t*>(kept), static_cast<uint8_t*>(scratch), p.split};
  }
  Gains g{{gains[0], gains[1], gains[2], gains[3]}};
  if (dtype == kBF16)
    return forward_impl<bf16>(B, T, N, H, (const bf16*)q, (const bf16*)K, (const bf16*)V,
                              (const bf16*)Vn, cocktail, bank_cocktail, key_bias, admission, scale,
                              idx, valid, fold, mode, g, (bf16*)out, w, p, true, stream);
  return forward_impl<float>(B, T, N, H, (const float*)q, (const float*)K, (const float*)V,
                             (const float*)Vn, cocktail, bank_cocktail, key_bias, admission, scale,
                             idx, valid, fold, mode, g, (float*)out, w, p, true, stream);
}

int dabsn_hip_read3_fwd(int dtype, int64_t B, int64_t T, int64_t N, int64_t H, const void* q,
                        const void* K, const void* V, const void* Vn, const float* cocktail,
                        const float* bank_cocktail, const float* key_bias, const float* admission,
                        const float* scale, const int64_t* idx, const uint8_t* valid, int mode,
                        const float* const* gains, void* out, void* workspace,
                        size_t workspace_bytes, hipStream_t stream) {
  return read3_fwd_entry(dtype, B, T, N, H, q, K, V, Vn, cocktail, bank_cocktail, key_bias,
                         admission, scale, idx, valid, nullptr, mode, gains, out, workspace,
                         workspace_bytes, nullptr, 0, true, stream);
}

int dabsn_hip_read3_fwd_keep(int dtype, int64_t B, int64_t T, int64_t N, int64_t H,
                             const void* q, const void* K, const void* V, const void* Vn,
                             const float* cocktail, const float* bank_cocktail,
                             const float* key_bias, const float* admission, const float* scale,
                             const int64_t* idx, const uint8_t* valid, const int8_t* fold,
                             int mode, const float* const* gains, void* out, void* kept,
                             size_t kept_bytes, void* scratch, size_t scratch_bytes,
                             hipStream_t stream) {
  return read3_fwd_entry(dtype, B, T, N, H, q, K, V, Vn, cocktail, bank_cocktail, key_bias,
                         admission, scale, idx, valid, fold, mode, gains, out, kept, kept_bytes,
                         scratch, scratch_bytes, false, stream);
}

// The backward entry points: with recompute, from the inputs alone (one workspace); without,
// on the kept part a forward call with the same inputs filled, which is only read, plus a
// scratch buffer.
static int read3_bwd_entry(bool recompute, int dtype, int64_t B, int64_t T, int64_t N,
                           int64_t H, const void* gout, const void* q, const void* K,
                           const void* V, const void* Vn, const float* cocktail,
                           const float* bank_cocktail, const float* key_bias,
                           const float* admission, const float* scale, const int64_t* idx,
                           const uint8_t* valid, const int8_t* fold, int mode,
                           const float* const* gains, void* gq, void* gK, void* gV, void* gVn,
                           float* gcocktail,
                           float* gbank_cocktail, float* gkey_bias, float* gadmission,
                           float* gscalars5, void* kept, size_t kept_bytes, void* scratch,
                           size_t scratch_bytes, hipStream_t stream) {
  const int rc = read3_checks(dtype, B, T, N, H, mode);
  if (rc != DABSN_OK) return rc;
  DABSN_REQUIRE(gout && q && gq && cocktail && gcocktail && scale && gains && gscalars5,
                "read3 backward: null pointer");
  for (int i = 0; i < 4; ++i) DABSN_REQUIRE(gains[i], "read3 backward: null gain %d", i);
  const size_t e = dtype == kBF16 ? 2 : 4;
  if (N == 0) {
    int z = dabsn_hip_zero(gq, static_cast<size_t>(B * T * H) * e, stream);
    if (z == DABSN_OK) z = dabsn_hip_zero(gcocktail, static_cast<size_t>(B * T * 4) * 4, stream);
    if (z == DABSN_OK) z = dabsn_hip_zero(gscalars5, 5 * 4, stream);
    return z;
  }
  DABSN_REQUIRE(K && V && (Vn || fold) && bank_cocktail && key_bias && admission && idx && valid &&
                    gK && gV && (gVn || fold) && gbank_cocktail && gkey_bias && gadmission &&
                    kept && (recompute || scratch),
                "read3 backward: null bank or workspace pointer");
  const Plan p = plan(dtype, B, T, N, H);
  Ws w;
  if (recompute) {
    DABSN_REQUIRE(kept_bytes >= p.end_bwd, "read3 backward: workspace %zu < %zu", kept_bytes,
                  p.end_bwd);
    w = single_ws(kept, p);
  } else {
    DABSN_REQUIRE(kept_bytes >= p.split && scratch_bytes >= p.end_bwd - p.split,
                  "read3 backward: kept %zu < %zu or scratch %zu < %zu", kept_bytes, p.split,
                  scratch_bytes, p.end_bwd - p.split);
    w = Ws{static_cast<uint8_t*>(kept), static_cast<uint8_t*>(scratch), p.split};
  }
  Gains g{{gains[0], gains[1], gains[2], gains[3]}};
  if (dtype == kBF16)
    return backward_impl<bf16>(B, T, N, H, (const bf16*)gout, (const bf16*)q, (const bf16*)K,
                               (const bf16*)V, (const bf16*)Vn, cocktail, bank_cocktail, key_bias,
                               admission, scale, idx, valid, fold, mode, g, (bf16*)gq, (bf16*)gK,
                               (bf16*)gV, (bf16*)gVn, gcocktail, gbank_cocktail, gkey_bias,
                               gadmission, gscalars5, w, p, recompute, stream);
  return backward_impl<float>(B, T, N, H, (const float*)gout, (const float*)q, (const float*)K,
                              (const float*)V, (const float*)Vn, cocktail, bank_cocktail, key_bias,
                              admission, scale, idx, valid, fold, mode, g, (float*)gq, (float*)gK,
                              (float*)gV, (float*)gVn, gcocktail, gbank_cocktail, gkey_bias,
                              gadmission, gscalars5, w, p, recompute, stream);
}

int dabsn_hip_read3_bwd(int dtype, int64_t B, int64_t T, int64_t N, int64_t H, const void* gout,
                        const void* q, const void* K, const void* V, const void* Vn,
                        const float* cocktail, const float* bank_cocktail, const float* key_bias,
                        const float* admission, const float* scale, const int64_t* idx,
                        const uint8_t* valid, int mode, const float* const* gains, void* gq,
                        void* gK, void* gV, void* gVn, float* gcocktail, float* gbank_cocktail,
                        float* gkey_bias, float* gadmission, float* gscalars5, void* workspace,
                        size_t workspace_bytes, hipStream_t stream) {
  return read3_bwd_entry(true, dtype, B, T, N, H, gout, q, K, V, Vn, cocktail, bank_cocktail,
                         key_bias, admission, scale, idx, valid, nullptr, mode, gains, gq, gK, gV,
                         gVn,
                         gcocktail, gbank_cocktail, gkey_bias, gadmission, gscalars5, workspace,
                         workspace_bytes, nullptr, 0, stream);
}

int dabsn_hip_read3_bwd_after_fwd(int dtype, int64_t B, int64_t T, int64_t N, int64_t H,
                                  const void* gout, const void* q, const void* K, const void* V,
                                  const void* Vn, const float* cocktail,
                                  const float* bank_cocktail, const float* key_bias,
                                  const float* admission, const float* scale,
                                  const int64_t* idx, const uint8_t* valid,
                                  const int8_t* fold, int mode, const float* const* gains,
                                  void* gq, void* gK, void* gV, void* gVn, float* gcocktail,
                                  float* gbank_cocktail, float* gkey_bias, float* gadmission,
                                  float* gscalars5, const void* kept, size_t kept_bytes,
                                  void* scratch, size_t scratch_bytes, hipStream_t stream) {
  return read3_bwd_entry(false, dtype, B, T, N, H, gout, q, K, V, Vn, cocktail, bank_cocktail,
                         key_bias, admission, scale, idx, valid, fold, mode, gains, gq, gK, gV,
                         gVn,
                         gcocktail, gbank_cocktail, gkey_bias, gadmission, gscalars5,
                         const_cast<void*>(kept), kept_bytes, scratch, scratch_bytes, stream);
}


size_t dabsn_hip_read3_decode_workspace_bytes(int dtype, int64_t B, int64_t T, int64_t N,
                                              int64_t H) {
  return decode_plan(dtype, B, T, N, H).end;
}

int dabsn_hip_read3_decode(int dtype, int64_t B, int64_t T, int64_t N, int64_t H, const void* q,
                           const void* bank, int64_t bank_len, int64_t bank_ld,
                           const float* norm_w, const int64_t* idx, const int64_t* next_idx,
                           const int64_t* read_idx, const uint8_t* valid, const float* cocktail,
                           const float* bank_cocktail, const float* key_bias,
                           const float* admission, const float* scale,
                           const float* const* gains, void* out, void* workspace,
                           size_t workspace_bytes, hipStream_t stream) {
  const int rc = read3_checks(dtype, B, T, N, H, 0);
  if (rc != DABSN_OK) return rc;
  DABSN_REQUIRE(T <= kDecodeRows, "read3 decode: T=%lld query rows > %d", (long long)T, kDecodeRows);
  DABSN_REQUIRE(N > 0 && bank_len > 0 && bank_ld >= bank_len, "read3 decode: bad bank shape");
  DABSN_REQUIRE(B * bank_ld <= static_cast<int64_t>(UINT32_MAX),
                "read3 decode: B * bank_ld = %lld bank rows exceeds 2^32 - 1", (long long)(B * bank_ld));
  DABSN_REQUIRE(H % 8 == 0, "read3 decode: H=%lld must be a multiple of 8", (long long)H);
  DABSN_REQUIRE(T * H * (dtype == kBF16 ? 2 : 4) <= 65536,
                "read3 decode: T*H too large for the query staging");
  DABSN_REQUIRE(q && bank && norm_w && idx && next_idx && read_idx && valid && cocktail &&
                    bank_cocktail && key_bias && admission && scale && gains && out && workspace,
                "read3 decode: null pointer");
  for (int i = 0; i < 4; ++i) DABSN_REQUIRE(gains[i], "read3 decode: null gain %d", i);
  const void* vec[] = {q, bank, out};
  for (const void* v : vec)
    DABSN_REQUIRE((reinterpret_cast<uintptr_t>(v) & 15u) == 0,
                  "read3 decode: q, bank and out must be 16-byte aligned");
  const DecodePlan p = decode_plan(dtype, B, T, N, H);
  DABSN_REQUIRE(workspace_bytes >= p.end, "read3 decode: workspace %zu < %zu", workspace_bytes,
                p.end);
  Gains g{{gains[0], gains[1], gains[2], gains[3]}};
  if (dtype == kBF16)
    return decode_impl<bf16>(B, T, N, H, bank_len, bank_ld, (const bf16*)q, (const bf16*)bank,
                             norm_w, idx, next_idx, read_idx, valid, cocktail, bank_cocktail,
                             key_bias, admission, scale, g, (bf16*)out, (uint8_t*)workspace, p,
                             stream);
  return decode_impl<float>(B, T, N, H, bank_len, bank_ld, (const float*)q, (const float*)bank,
                            norm_w, idx, next_idx, read_idx, valid, cocktail, bank_cocktail,
                            key_bias, admission, scale, g, (float*)out, (uint8_t*)workspace, p,
                            stream);
}

int dabsn_hip_read3_decode_members(int dtype, int64_t B, int64_t N, int64_t H, const void* q,
                                   const void* bank, int64_t bank_len, int64_t bank_ld,
                                   const float* stats, const int64_t* members,
                                   const int64_t* counts, int64_t query_start,
                                   const float* cocktail, const float* key_bias,
                                   const float* admission, const float* scale,
                                   const float* const* gains, void* out, void* workspace,
                                   size_t workspace_bytes, hipStream_t stream) {
  const int rc = read3_checks(dtype, B, 1, N, H, 0);
  if (rc != DABSN_OK) return rc;
  DABSN_REQUIRE(H % 8 == 0 && H <= 64 * 8 * kFusedMaxChunks,
                "read3 decode (members): H=%lld must be a multiple of 8 and at most %d",
                (long long)H, 64 * 8 * kFusedMaxChunks);
  DABSN_REQUIRE(N > 0 && N <= bank_ld && bank_len > 0 && bank_ld >= bank_len,
                "read3 decode (members): bad bank shape");
  DABSN_REQUIRE(B * bank_ld <= static_cast<int64_t>(UINT32_MAX),
                "read3 decode (members): B * bank_ld = %lld bank rows exceeds 2^32 - 1",
                (long long)(B * bank_ld));
  DABSN_REQUIRE(q && bank && stats && members && counts && cocktail && key_bias && admission &&
                    scale && gains && out && workspace,
                "read3 decode (members): null pointer");
  for (int i = 0; i < 4; ++i) DABSN_REQUIRE(gains[i], "read3 decode (members): null gain %d", i);
  const void* vec[] = {q, bank, out};
  for (const void* v : vec)
    DABSN_REQUIRE((reinterpret_cast<uintptr_t>(v) & 15u) == 0,
                  "read3 decode (members): q, bank and out must be 16-byte aligned");
  const DecodePlan p = decode_plan(dtype, B, 1, N, H);
  DABSN_REQUIRE(p.fused, "read3 decode (members): no single-pass plan");
  DABSN_REQUIRE(workspace_bytes >= p.end, "read3 decode (members): workspace %zu < %zu",
                workspace_bytes, p.end);
  Gains g{{gains[0], gains[1], gains[2], gains[3]}};
  int32_t* rs = reinterpret_cast<int32_t*>(static_cast<uint8_t*>(workspace) + p.off_rs);
  SlotMeta* meta = reinterpret_cast<SlotMeta*>(static_cast<uint8_t*>(workspace) + p.off_meta);
  hipLaunchKernelGGL(decode_meta_members_kernel, dim3((unsigned)((N + 255) / 256), (unsigned)B),
                     dim3(256), 0, stream, (int)N, bank_len, bank_ld, query_start, stats, members,
                     counts, cocktail, key_bias, admission, g, meta, rs);
  DABSN_HIP_CHECK(hipGetLastError());
  if (dtype == kBF16)
    return decode_pass<bf16>(B, N, H, (const bf16*)q, (const bf16*)bank, meta, rs, scale, g,
                             (bf16*)out, (uint8_t*)workspace, p, stream);
  return decode_pass<float>(B, N, H, (const float*)q, (const float*)bank, meta, rs, scale, g,
                            (float*)out, (uint8_t*)workspace, p, stream);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// The decode read without a workspace argument, for callers that cannot allocate device
// memory: code under HIP graph capture, serving loops whose buffers are all planned ahead.
// The scratch is a file-scope device array, so every device the library runs on holds its
// own kNoAllocScratchBytes from module load until the process ends. Every call on a device
// uses that device's copy: calls that overlap on one device (other streams, other threads)
// race. Nothing needs clearing between calls -- each kernel of the decode read writes every
// scratch element it or a later kernel of the same call reads.
// ---------------------------------------------------------------------------
constexpr size_t kNoAllocScratchBytes = DABSN_READ3_DECODE_NOALLOC_MAX_BYTES;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) uint8_t decode_scratch[kNoAllocScratchBytes];

static std::mutex g_scratch_mutex;
static uint8_t* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's copy of decode_scratch, looked up once per device
// (the array's host-side name is not a device address).
static int scratch_of_current_device(uint8_t** out) {
  int dev = 0;
  DABSN_HIP_CHECK(hipGetDevice(&dev));
  DABSN_REQUIRE(dev >= 0 && dev < kMaxDevices, "read3 decode (no allocation): device %d", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    DABSN_HIP_CHECK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(decode_scratch)));
    DABSN_REQUIRE(ptr != nullptr, "read3 decode (no allocation): no scratch on device %d", dev);
    g_scratch_ptr[dev] = static_cast<uint8_t*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return DABSN_OK;
}

extern "C" {

int dabsn_hip_read3_decode_noalloc(int dtype, int64_t B, int64_t T, int64_t N, int64_t H,
                                   const void* q, const void* bank, int64_t bank_len,
                                   int64_t bank_ld, const float* norm_w, const int64_t* idx,
                                   const int64_t* next_idx, const int64_t* read_idx,
                                   const uint8_t* valid, const float* cocktail,
                                   const float* bank_cocktail, const float* key_bias,
                                   const float* admission, const float* scale,
                                   const float* const* gains, void* out, hipStream_t stream) {
  const int rc = read3_checks(dtype, B, T, N, H, 0);
  if (rc != DABSN_OK) return rc;
  DABSN_REQUIRE(T <= kDecodeRows, "read3 decode: T=%lld query rows > %d", (long long)T, kDecodeRows);
  const DecodePlan p = decode_plan(dtype, B, T, N, H);
  DABSN_REQUIRE(p.end <= kNoAllocScratchBytes,
                "read3 decode (no allocation): B=%lld, T=%lld, N=%lld, H=%lld needs %zu bytes of "
                "scratch, more than the %zu bytes the library holds per device; call "
                "dabsn_hip_read3_decode with a workspace instead",
                (long long)B, (long long)T, (long long)N, (long long)H, p.end,
                kNoAllocScratchBytes);
  uint8_t* ws = nullptr;
  const int sc = scratch_of_current_device(&ws);
  if (sc != DABSN_OK) return sc;
  return dabsn_hip_read3_decode(dtype, B, T, N, H, q, bank, bank_len, bank_ld, norm_w, idx,
                                next_idx, read_idx, valid, cocktail, bank_cocktail, key_bias,
                                admission, scale, gains, out, ws, kNoAllocScratchBytes, stream);
}

}  // extern "C"
