// Read glue: per-position tape statistics, query normalisation, admitted-slot
// selection and the bank gather (with their backward passes).
//
// Reference: src/dabsn/read.py:58-72 (admission), 154-183 (query, key bias, cocktail; the
// same on a bank 680-700),
// 185-239 (cummax floor, member, stable partition, bank width), 241-256 and 298-303
// (bank gather, next-write gather).
#include "../../include/dabsn_hip.h"
#include "capi.hpp"
#include "common.hpp"

#include <initializer_list>

namespace dabsn {
namespace glue {

constexpr float kEps = 1e-12f;

struct Ptr8 {
  const float* p[8];
};

// Element kernels take V = 8 (16-byte vector accesses, H % 8 == 0 and aligned operands) or
// V = 1. Elementwise kernels index V-element chunks with 32-bit arithmetic; row kernels put
// one wave on a (b, t) row.

// One wave per (b, t) row.
// Rows (b, t), t < T, of tapes whose batch rows are ldt time steps apart (a time window of
// longer sequences); statistics rows lds apart per batch row.
template <typename E, int V>
__global__ void __launch_bounds__(256) stats_kernel(int64_t rows, int T, int64_t ldt, int64_t lds,
                                                    int H, const E* nov, const E* pl, const E* en,
                                                    const E* sat, const E* ay, const E* wr,
                                                    float* stats) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const int64_t b = row / T, t = row % T;
  const size_t base = static_cast<size_t>(b * ldt + t) * H;
  float se = 0.f, sc = 0.f, sn = 0.f, sp = 0.f, sa = 0.f, sw = 0.f;
  for (int h = lane * V; h < H; h += 64 * V) {
    const size_t o = base + h;
    float e[V], c[V], n[V], q[V], a[V], w[V];
    ldv<E, V>(en + o, e);
    ldv<E, V>(sat + o, c);
    ldv<E, V>(nov + o, n);
    ldv<E, V>(pl + o, q);
    ldv<E, V>(ay + o, a);
    ldv<E, V>(wr + o, w);
#pragma unroll
    for (int k = 0; k < V; ++k) {
      se += e[k];
      sc += c[k];
      sn += n[k];
      sp += q[k];
      sa += a[k] * a[k];
      sw += w[k] * w[k];
    }
  }
  se = wave_sum(se);
  sc = wave_sum(sc);
  sn = wave_sum(sn);
  sp = wave_sum(sp);
  sa = wave_sum(sa);
  sw = wave_sum(sw);
  if (lane == 0) {
    const float inv = 1.0f / static_cast<float>(H);
    float* o = stats + static_cast<size_t>(b * lds + t) * 6;
    o[0] = se * inv;
    o[1] = sc * inv;
    o[2] = sn * inv;
    o[3] = sp * inv;
    o[4] = sqrtf(sa);
    o[5] = sqrtf(sw);
  }
}

// g_tape[b,t,h] += g_mean[b,t] / H for the four averaged tapes; one thread per V elements.
// Mean gradients broadcast over H: g = gstats / H, written (accumulate = 0) or added to
// what the buffers hold (accumulate = 1).
template <typename E, int V>
__global__ void __launch_bounds__(256) stats_bwd_kernel(uint32_t chunks, uint32_t cpr, int H, int T,
                                                        int64_t ldt, int64_t lds,
                                                        const float* gstats, int accumulate,
                                                        E* gen, E* gsat, E* gnov, E* gpl) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i >= chunks) return;
  const uint32_t row = i / cpr;
  const int64_t b = row / T, t = row % T;
  const size_t o = static_cast<size_t>(b * ldt + t) * H + static_cast<size_t>(i % cpr) * V;
  const float inv = 1.0f / static_cast<float>(H);
  const float* g = gstats + static_cast<size_t>(b * lds + t) * 6;
  E* dst[4] = {gen, gsat, gnov, gpl};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    if (!dst[k]) continue;
    float v[V];
    const float add = g[k] * inv;
    if (accumulate) {
      ldv<E, V>(dst[k] + o, v);
#pragma unroll
      for (int e = 0; e < V; ++e) v[e] += add;
    } else {
#pragma unroll
      for (int e = 0; e < V; ++e) v[e] = add;
    }
    stv<E, V>(dst[k] + o, v);
  }
}

template <typename E, int V>
__global__ void __launch_bounds__(256) normalize_kernel(uint32_t chunks, uint32_t cpr, const E* x,
                                                        const float* norms, E* q) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i >= chunks) return;
  const float n = fmaxf(norms[i / cpr], kEps);
  const size_t o = static_cast<size_t>(i) * V;
  float v[V];
  ldv<E, V>(x + o, v);
#pragma unroll
  for (int e = 0; e < V; ++e) v[e] = v[e] / n;
  stv<E, V>(q + o, v);
}

// One wave per row: gx += (gq - q (q.gq)) / |x| if |x| > eps, else gq / eps.
template <typename E, int V>
__global__ void __launch_bounds__(256) normalize_bwd_kernel(int64_t rows, int H, const E* q,
                                                            const float* norms, const E* gq,
                                                            E* gx) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const size_t base = static_cast<size_t>(row) * H;
  const float nrm = norms[row];
  float dot = 0.0f;
  if (nrm > kEps) {
    for (int h = lane * V; h < H; h += 64 * V) {
      float a[V], g[V];
      ldv<E, V>(q + base + h, a);
      ldv<E, V>(gq + base + h, g);
#pragma unroll
      for (int e = 0; e < V; ++e) dot += a[e] * g[e];
    }
    dot = wave_sum(dot);
  }
  const float n = fmaxf(nrm, kEps);
  for (int h = lane * V; h < H; h += 64 * V) {
    const size_t o = base + h;
    float a[V], g[V], acc[V];
    ldv<E, V>(q + o, a);
    ldv<E, V>(gq + o, g);
    ldv<E, V>(gx + o, acc);
#pragma unroll
    for (int e = 0; e < V; ++e) acc[e] += nrm > kEps ? (g[e] - a[e] * dot) / n : g[e] / n;
    stv<E, V>(gx + o, acc);
  }
}

// Admitted-slot selection, one workgroup per batch row. Each thread owns a contiguous
// chunk of time steps; block scans combine the per-chunk running max and member counts.
constexpr int SEL_T = 256;

// With floor_bf16 the floor cummax - window is rounded to bf16, as the reference evaluates
// it when the admission values are bf16 (read.py:185-188 in the tapes' dtype). With `whole`
// the floor is the whole row's max - window (field and hybrid geometry, read.py:189-191).
__global__ void __launch_bounds__(SEL_T) select_kernel(int T, const float* adm, const float* window,
                                                       int floor_bf16, int whole, int64_t* order,
                                                       int64_t* counts, int32_t* rank) {
  __shared__ float smax[SEL_T];
  __shared__ int scnt[SEL_T];
  const int b = blockIdx.x, tid = threadIdx.x;
  const float* a = adm + static_cast<size_t>(b) * T;
  const int chunk = (T + SEL_T - 1) / SEL_T;
  const int t0 = min(T, tid * chunk), t1 = min(T, t0 + chunk);
  const float win = window[0];
  float m = -INFINITY;
  for (int t = t0; t < t1; ++t) m = fmaxf(m, a[t]);
  smax[tid] = m;
  __syncthreads();
  // Inclusive prefix max over chunk maxima (Hillis-Steele).
  for (int off = 1; off < SEL_T; off <<= 1) {
    const float v = tid >= off ? smax[tid - off] : -INFINITY;
    __syncthreads();
    smax[tid] = fmaxf(smax[tid], v);
    __syncthreads();
  }
  const float before = tid > 0 ? smax[tid - 1] : -INFINITY;
  const float row_max = smax[SEL_T - 1];
  int cnt = 0;
  float run = before;
  auto floor_of = [&](float m) { return floor_bf16 ? round_to<bf16>(m - win) : m - win; };
  for (int t = t0; t < t1; ++t) {
    run = whole ? row_max : ((t == 0 || a[t] > run) ? a[t] : run);
    cnt += (a[t] >= floor_of(run)) ? 1 : 0;
  }
  scnt[tid] = cnt;
  __syncthreads();
  for (int off = 1; off < SEL_T; off <<= 1) {
    const int v = tid >= off ? scnt[tid - off] : 0;
    __syncthreads();
    scnt[tid] += v;
    __syncthreads();
  }
  const int total = scnt[SEL_T - 1];
  int mpos = tid > 0 ? scnt[tid - 1] : 0;  // members before this chunk
  run = before;
  int64_t* o = order + static_cast<size_t>(b) * T;
  int32_t* rk = rank + static_cast<size_t>(b) * T;
  for (int t = t0; t < t1; ++t) {
    run = whole ? row_max : ((t == 0 || a[t] > run) ? a[t] : run);
    int r;
    if (a[t] >= floor_of(run)) {
      r = mpos++;
    } else {
      r = total + (t - mpos);
    }
    o[r] = t;
    rk[t] = r;
  }
  if (tid == 0) counts[b] = total;
}

// Gather K (normalised), V and Vn rows of the bank; one thread per V elements.
template <typename E, int V>
__global__ void __launch_bounds__(256) gather_kernel(int T, int N, int H, int hblocks, const E* w,
                                                     const float* norm_w, const int64_t* idx,
                                                     const int64_t* nidx, E* K, E* Vv, E* Vn) {
  const int64_t row = blockIdx.x / hblocks;  // b * N + j
  const int h = ((blockIdx.x % hblocks) * 256 + threadIdx.x) * V;
  if (h >= H) return;
  const int64_t b = row / N;
  int64_t t = idx[row];
  t = t < 0 ? 0 : (t >= T ? T - 1 : t);
  float v[V], k[V];
  ldv<E, V>(w + (static_cast<size_t>(b) * T + t) * H + h, v);
  const float n = fmaxf(norm_w[static_cast<size_t>(b) * T + t], kEps);
#pragma unroll
  for (int e = 0; e < V; ++e) k[e] = v[e] / n;
  const size_t o = static_cast<size_t>(row) * H + h;
  stv<E, V>(K + o, k);
  stv<E, V>(Vv + o, v);
  if (Vn) {  // absent when the read folds successor rows into V (no next rows needed)
    int64_t tn = nidx[row];
    tn = tn < 0 ? 0 : (tn >= T ? T - 1 : tn);
    float vn[V];
    ldv<E, V>(w + (static_cast<size_t>(b) * T + tn) * H + h, vn);
    stv<E, V>(Vn + o, vn);
  }
}

// One workgroup per (b, t) position of the write tape; writes gw[t] (zero where no slot
// maps to t). gVn may be null (no successor-row gradients).
template <typename E, int V>
__global__ void __launch_bounds__(256) gather_bwd_kernel(int T, int ldg, int N, int H,
                                                         const float* norm_w,
                                                         const int32_t* rank, const E* K,
                                                         const E* gK, const E* gV, const E* gVn,
                                                         int accumulate, E* gw) {
  __shared__ float part[4];
  const int64_t bt = blockIdx.x;
  const int64_t b = bt / T;
  const int t = static_cast<int>(bt % T);
  const int64_t pos = b * ldg + t;  // row of norm_w and gw (rows ldg positions apart)
  const int32_t* rk = rank + static_cast<size_t>(b) * T;
  const int r0 = rk[t];
  const int r1 = gVn && t >= 1 ? rk[t - 1] : N;
  const int r2 = gVn && t == T - 1 ? rk[T - 1] : N;
  const bool in0 = r0 < N, in1 = r1 < N, in2 = r2 < N;
  const float nrm = norm_w[pos];
  const float n = fmaxf(nrm, kEps);
  float dot = 0.0f;
  // The slot's K and gK rows are read once: the first RC vectors of each thread stay in
  // registers from the dot product to the update (H <= 256 V RC, e.g. 4096 in bf16).
  constexpr int RC = 2;
  float kc[RC][V], gc[RC][V];
  if (in0 && nrm > kEps) {
    const size_t kb = (static_cast<size_t>(b) * N + r0) * H;
    float s = 0.0f;
    int i = 0;
    for (int h = threadIdx.x * V; h < H; h += 256 * V, ++i) {
      float k[V], g[V];
      ldv<E, V>(K + kb + h, k);
      ldv<E, V>(gK + kb + h, g);
#pragma unroll
      for (int e = 0; e < V; ++e) s += k[e] * g[e];
#pragma unroll
      for (int c = 0; c < RC; ++c) {
        if (c == i) {
#pragma unroll
          for (int e = 0; e < V; ++e) {
            kc[c][e] = k[e];
            gc[c][e] = g[e];
          }
        }
      }
    }
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    dot = part[0] + part[1] + part[2] + part[3];
  }
  const bool cached = in0 && nrm > kEps;
  int i = 0;
  for (int h = threadIdx.x * V; h < H; h += 256 * V, ++i) {
    const size_t o = static_cast<size_t>(pos) * H + h;
    float acc[V];
    if (accumulate) {
      ldv<E, V>(gw + o, acc);
    } else {
#pragma unroll
      for (int e = 0; e < V; ++e) acc[e] = 0.0f;
    }
    if (in0) {
      const size_t kb = (static_cast<size_t>(b) * N + r0) * H + h;
      float gk[V], gv[V], k[V];
      ldv<E, V>(gV + kb, gv);
      if (cached && i < RC) {
#pragma unroll
        for (int c = 0; c < RC; ++c) {
          if (c == i) {
#pragma unroll
            for (int e = 0; e < V; ++e) {
              k[e] = kc[c][e];
              gk[e] = gc[c][e];
            }
          }
        }
      } else {
        ldv<E, V>(gK + kb, gk);
        ldv<E, V>(K + kb, k);
      }
#pragma unroll
      for (int e = 0; e < V; ++e)
        acc[e] += gv[e] + (nrm > kEps ? (gk[e] - k[e] * dot) / n : gk[e] / n);
    }
    if (in1) {
      float g[V];
      ldv<E, V>(gVn + (static_cast<size_t>(b) * N + r1) * H + h, g);
#pragma unroll
      for (int e = 0; e < V; ++e) acc[e] += g[e];
    }
    if (in2) {
      float g[V];
      ldv<E, V>(gVn + (static_cast<size_t>(b) * N + r2) * H + h, g);
#pragma unroll
      for (int e = 0; e < V; ++e) acc[e] += g[e];
    }
    stv<E, V>(gw + o, acc);
  }
}

// Successor-fold codes of a bank selected by select_kernel (slot order = admitted positions
// ascending; next position = min(idx + 1, T - 1), as the read builds it): for slot j of row
// b, 1 when its next position is the position of slot j + 1, 0 when the next position is
// its own (the clamped last position) or the slot is past the row's count, 2 otherwise (no
// fold). One thread per slot; `codes` (width N) and `unfoldable` (set to 1 when any valid
// slot codes 2, never cleared here) are each optional.
__global__ void __launch_bounds__(256) fold_kernel(int T, int N, const int64_t* order,
                                                   const int64_t* counts, int8_t* codes,
                                                   uint32_t* unfoldable) {
  const int b = blockIdx.y;
  const int j = blockIdx.x * 256 + threadIdx.x;
  const int64_t cnt = counts[b];
  int code = 0;
  if (j < T && j < cnt) {
    const int64_t* ob = order + static_cast<size_t>(b) * T;
    const int64_t i = ob[j];
    const int64_t nx = i + 1 < T ? i + 1 : T - 1;
    code = nx == i ? 0 : (j + 1 < cnt && ob[j + 1] == nx ? 1 : 2);
  }
  if (codes && j < N) codes[static_cast<size_t>(b) * N + j] = static_cast<int8_t>(code);
  if (unfoldable && __any(code == 2) && (threadIdx.x & 63) == 0)
    __hip_atomic_fetch_or(unfoldable, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// out = a (+ x) over a [B, R, C] box whose operands each have their own batch and row
// strides (elements; the columns are contiguous): a time window of [B, T, H] tensors, a
// column block of a wider row, or a dense buffer. One thread per V elements of a row; V = 8
// moves 16 bytes per access (bf16) and needs C and every stride a multiple of 8 and 16-byte
// aligned bases. bf16 sums are formed in fp32 and rounded once, as torch's add rounds them.
template <typename E, int V>
__global__ void __launch_bounds__(256) window_add_kernel(uint32_t chunks, uint32_t cpr, uint32_t R,
                                                         const E* a, int64_t a_sb, int64_t a_sr,
                                                         const E* x, int64_t x_sb, int64_t x_sr,
                                                         E* out, int64_t o_sb, int64_t o_sr) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i >= chunks) return;
  const int64_t c = static_cast<int64_t>(i % cpr) * V;
  const uint32_t rr = i / cpr;
  const int64_t r = rr % R, b = rr / R;
  float va[V];
  ldv<E, V>(a + b * a_sb + r * a_sr + c, va);
  if (x != nullptr) {
    float vx[V];
    ldv<E, V>(x + b * x_sb + r * x_sr + c, vx);
#pragma unroll
    for (int e = 0; e < V; ++e) va[e] += vx[e];
  }
  stv<E, V>(out + b * o_sb + r * o_sr + c, va);
}

// The bank width a read needs and whether its successor rows fold (one host read of two
// int64 values instead of a reduction, a flag kernel and their stacking): out[0] = the
// largest admitted count over the rows, out[1] = 1 when some admitted slot's successor is
// neither the next slot's position nor its own (fold_kernel's code 2). out is zeroed first.
__global__ void __launch_bounds__(256) width_kernel(int T, const int64_t* order,
                                                    const int64_t* counts, int check_fold,
                                                    unsigned long long* out) {
  const int b = blockIdx.y;
  const int j = blockIdx.x * 256 + threadIdx.x;
  const int64_t cnt = counts[b];
  if (j == 0) atomicMax(out, static_cast<unsigned long long>(cnt > 0 ? cnt : 0));
  if (!check_fold) return;
  bool bad = false;
  if (j < T && j < cnt) {
    const int64_t* ob = order + static_cast<size_t>(b) * T;
    const int64_t i = ob[j];
    const int64_t nx = i + 1 < T ? i + 1 : T - 1;
    bad = nx != i && !(j + 1 < cnt && ob[j + 1] == nx);
  }
  if (__any(bad) && (threadIdx.x & 63) == 0) atomicOr(out + 1, 1ull);
}

// The slot arrays of a read of width N from a bank_select result (read.py:233-239 after the
// host read of the width): idx = order[:, :N], valid = j < max(count, 1), next_idx =
// min(idx + 1, T - 1), read_idx = idx - query_start and, optionally, the fold codes of
// fold_kernel. One thread per slot.
__global__ void __launch_bounds__(256) slots_kernel(int T, int N, int64_t query_start,
                                                    const int64_t* order, const int64_t* counts,
                                                    int64_t* idx, uint8_t* valid,
                                                    int64_t* next_idx, int64_t* read_idx,
                                                    int8_t* codes) {
  const int b = blockIdx.y;
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= N) return;
  const int64_t cnt = counts[b];
  const int64_t* ob = order + static_cast<size_t>(b) * T;
  const int64_t i = ob[j];
  const int64_t nx = i + 1 < T ? i + 1 : T - 1;
  const size_t o = static_cast<size_t>(b) * N + j;
  idx[o] = i;
  valid[o] = j < (cnt > 1 ? cnt : 1) ? 1 : 0;
  next_idx[o] = nx;
  read_idx[o] = i - query_start;
  if (codes) {
    int code = 0;
    if (j < cnt) code = nx == i ? 0 : (j + 1 < cnt && ob[j + 1] == nx ? 1 : 2);
    codes[o] = static_cast<int8_t>(code);
  }
}

}  // namespace glue
}  // namespace dabsn

using namespace dabsn;
using namespace dabsn::glue;

static inline unsigned blocks_for(int64_t n, int per) {
  return static_cast<unsigned>((n + per - 1) / per);
}

// 16-byte vector accesses need H % 8 == 0 and 16-byte aligned row bases.
static inline bool vec_ok(int64_t H, std::initializer_list<const void*> ptrs) {
  if (H % 8 != 0) return false;
  for (const void* q : ptrs)
    if (q && (reinterpret_cast<uintptr_t>(q) & 15u) != 0) return false;
  return true;
}

// Read output (read.py:435-438, 821-823): out = proj + gain * long, evaluated as the
// reference's two tensor operations under type promotion -- the product in the dtype of
// (gain, long), rounded to bf16 when prod_bf16, then the sum in the dtype of (proj, product),
// rounded by the store to O. No contraction into a fused multiply-add.
// Elements are addressed as segments: chunk i of V elements lies in segment i / seg (seg
// chunks each), and each tensor has its own segment stride (in chunks), so a time window
// [t0, t1) of [B, T, H] tensors is B segments of (t1 - t0) H elements, T H apart, and a
// contiguous [B, t1 - t0, H] block the same segments (t1 - t0) H apart. A flat array is one
// segment.
struct SegLd {
  uint64_t ld[4];
};

__device__ __forceinline__ size_t seg_offset(uint32_t s, uint32_t r, uint64_t ld) {
  return static_cast<size_t>(s) * ld + r;
}

template <typename P, typename L, typename O, int V>
__global__ void __launch_bounds__(256) read_out_kernel(uint32_t chunks, uint32_t seg, SegLd ld,
                                                       const P* proj, const L* lng,
                                                       const float* gain, int prod_bf16, O* out) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i >= chunks) return;
  const uint32_t s = i / seg, r = i % seg;
  const float g = gain[0];
  float a[V], l[V];
  ldv<P, V>(proj + seg_offset(s, r, ld.ld[0]) * V, a);
  ldv<L, V>(lng + seg_offset(s, r, ld.ld[1]) * V, l);
#pragma unroll
  for (int e = 0; e < V; ++e) {
    float prod = g * l[e];
    if (prod_bf16) prod = round_to<bf16>(prod);
    a[e] = a[e] + prod;
  }
  stv<O, V>(out + seg_offset(s, r, ld.ld[2]) * V, a);
}

// Its backward, as autograd evaluates it: gproj = gout cast to P; the product's gradient
// gp = gout cast to the product dtype; glong = gp * gain in that dtype, cast to L; the gain's
// gradient sums gp * long (each term in the product dtype, the sum in fp32), one partial per
// workgroup, reduced in a fixed order by read_out_reduce_kernel.
template <typename O, typename P, typename L, int V>
__global__ void __launch_bounds__(256) read_out_bwd_kernel(uint32_t chunks, uint32_t seg,
                                                           SegLd ld, const O* gout,
                                                           const L* lng, const float* gain,
                                                           int prod_bf16, P* gproj, L* glong,
                                                           float* partial) {
  __shared__ float sh[4];
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  float acc = 0.0f;
  if (i < chunks) {
    const uint32_t s = i / seg, r = i % seg;
    const float g = gain[0];
    float go[V], l[V], gl[V];
    ldv<O, V>(gout + seg_offset(s, r, ld.ld[0]) * V, go);
    ldv<L, V>(lng + seg_offset(s, r, ld.ld[1]) * V, l);
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const float gp = prod_bf16 ? round_to<bf16>(go[e]) : go[e];
      float x = gp * g;
      if (prod_bf16) x = round_to<bf16>(x);
      gl[e] = x;
      float t = gp * l[e];
      if (prod_bf16) t = round_to<bf16>(t);
      acc += t;
    }
    stv<P, V>(gproj + seg_offset(s, r, ld.ld[2]) * V, go);
    stv<L, V>(glong + seg_offset(s, r, ld.ld[3]) * V, gl);
  }
  acc = wave_sum(acc);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) partial[blockIdx.x] = (sh[0] + sh[1]) + (sh[2] + sh[3]);
}

// One workgroup: strided partial sums per thread, then the wave/LDS tree; fixed order.
// One workgroup of 1024 threads: thread i sums partials i, i + 1024, ... in order (four
// loads in flight), then the waves' sums are combined in a fixed tree order.
__global__ void __launch_bounds__(1024) read_out_reduce_kernel(uint32_t n, const float* partial,
                                                               float* out) {
  __shared__ float sh[16];
  float acc = 0.0f;
  uint32_t k = threadIdx.x;
  for (; k + 3u * 1024u < n; k += 4u * 1024u) {
    const float a = partial[k], b = partial[k + 1024u], c = partial[k + 2048u],
                d = partial[k + 3072u];
    acc = acc + a + b + c + d;
  }
  for (; k < n; k += 1024u) acc += partial[k];
  acc = wave_sum(acc);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float s8[8];
#pragma unroll
    for (int w = 0; w < 8; ++w) s8[w] = sh[2 * w] + sh[2 * w + 1];
    out[0] = ((s8[0] + s8[1]) + (s8[2] + s8[3])) + ((s8[4] + s8[5]) + (s8[6] + s8[7]));
  }
}

// Runs LAUNCH(E, V) for the dtype code, with V = 8 when `vec` holds and V = 1 otherwise.
#define GLUE_DISPATCH(what, dtype, vec, LAUNCH)                       \
  do {                                                                \
    if ((dtype) == kBF16) {                                           \
      if (vec) { LAUNCH(bf16, 8); } else { LAUNCH(bf16, 1); }         \
    } else if ((dtype) == kF32) {                                     \
      if (vec) { LAUNCH(float, 8); } else { LAUNCH(float, 1); }       \
    } else {                                                          \
      DABSN_REQUIRE(false, what ": bad dtype %d", dtype);             \
    }                                                                 \
  } while (0)

// Key bias, admission and cocktail from rows of tape statistics (mean energy, saturation,
// novelty, plasticity, ...; 6 floats per row, rows of batch b `ld` floats apart): the
// expressions of read.py:58-72 and 155-180 / 680-700 on the means, with the same operation
// order (products of gains and means added left to right, no contraction), so the results
// match the torch expressions up to the last-bit rounding of log1p and the norm.
// prm = 8 fp32 scalars: p_gain, novelty_gain, null_bias, adm_p_gain, adm_novelty_gain,
// adm_saturation_gain, adm_energy_gain, adm_bias. One thread per row.
// `mode` reproduces the dtype the reference evaluates these expressions in: bit 0 = the
// tapes are bf16, so the means and every tape-dtype intermediate (mean_p * H, its log1p,
// the cocktail's norm and quotients) are rounded to bf16; bit 1 = the gains are bf16
// too, so every product and sum is rounded as well (with fp32 gains, type promotion makes
// them fp32). Operation order is that of read.py:58-72, 161-183.
// Key bias, admission and cocktail of one statistics row s (6 floats).
__device__ __forceinline__ void glue_row(const float* s, float hidden, const Ptr8& prm, int mode,
                                         float* kb, float* adm, float* ck) {
  const bool tb = mode & 1, pb = (mode & 2) && tb;
  auto rt = [tb](float v) { return tb ? round_to<bf16>(v) : v; };
  auto rp = [pb](float v) { return pb ? round_to<bf16>(v) : v; };
  const float me = rt(s[0]), mc = rt(s[1]), mn = rt(s[2]), mp = rt(s[3]);
  const float lp = rt(log1pf(rt(mp * hidden)));
  float P[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) P[k] = prm.p[k][0];
  if (kb) *kb = rp(rp(rp(P[0] * lp) + rp(P[1] * mn)) + P[2]);
  if (adm)
    *adm = rp(rp(rp(rp(rp(P[3] * lp) + rp(P[4] * mn)) + rp(P[5] * mc)) + rp(P[6] * me)) + P[7]);
  const float d = rt(fmaxf(rt(sqrtf(me * me + mc * mc + mn * mn + mp * mp)), kEps));
  *reinterpret_cast<float4*>(ck) = make_float4(rt(me / d), rt(mc / d), rt(mn / d), rt(mp / d));
}

__global__ void __launch_bounds__(256) means_glue_kernel(int64_t rows, int N, int64_t ld,
                                                         const float* __restrict__ stats,
                                                         float hidden, Ptr8 prm, int mode,
                                                         float* kb, float* adm, float* ck) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= rows) return;
  glue_row(stats + (i / N) * ld + (i % N) * 6, hidden, prm, mode, kb ? kb + i : nullptr,
           adm ? adm + i : nullptr, ck + i * 4);
}

// Per-slot glue of the training read: key bias, admission and cocktail of bank row idx[b][j]
// for every slot j (glue_row, gathered inside the kernel). One thread per (b, j).
__global__ void __launch_bounds__(256) glue_slots_kernel(int64_t n, int N, int L, int64_t ld,
                                                         const float* __restrict__ stats,
                                                         const int64_t* __restrict__ idx,
                                                         float hidden, Ptr8 prm, int mode,
                                                         float* kb, float* adm, float* cb) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  const int64_t b = i / N;
  int64_t pos = idx[i];
  pos = pos < 0 ? 0 : (pos >= L ? L - 1 : pos);
  glue_row(stats + b * ld + pos * 6, hidden, prm, mode, kb + i, adm + i, cb + i * 4);
}

// Gradient of one row's glue with respect to its four means (g4 = mean e, c, n, p) and the
// eight parameters (added to gp), given the gradients of key bias, admission and cocktail
// (gkb, gadm; gc4 may be null). Evaluated in fp32 from the means and intermediates of the
// forward (rounded as the forward rounds them): the chain rule of the expressions in
// glue_row, i.e. of read.py:58-72, 161-183.
__device__ __forceinline__ void glue_row_bwd(const float* s, float hidden, const float* P,
                                             int mode, float gkb, float gadm, const float* gc4,
                                             float* g4, float* gp) {
  const bool tb = mode & 1;
  auto rt = [tb](float v) { return tb ? round_to<bf16>(v) : v; };
  const float m[4] = {rt(s[0]), rt(s[1]), rt(s[2]), rt(s[3])};  // e, c, n, p
  const float x = rt(m[3] * hidden);
  const float lp = rt(log1pf(x));
  gp[0] += gkb * lp;
  gp[1] += gkb * m[2];
  gp[2] += gkb;
  gp[3] += gadm * lp;
  gp[4] += gadm * m[2];
  gp[5] += gadm * m[1];
  gp[6] += gadm * m[0];
  gp[7] += gadm;
  const float glp = gkb * P[0] + gadm * P[3];
  float g[4] = {gadm * P[6], gadm * P[5], gkb * P[1] + gadm * P[4], glp * hidden / (1.0f + x)};
  if (gc4) {
    // c = m / max(|m|, eps): dc/dm = (I - c c^T) / |m| above eps, I / eps below.
    const float nrm = sqrtf(m[0] * m[0] + m[1] * m[1] + m[2] * m[2] + m[3] * m[3]);
    if (nrm > kEps) {
      const float inv = 1.0f / nrm;
      float c[4], dot = 0.0f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        c[k] = m[k] * inv;
        dot += c[k] * gc4[k];
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) g[k] += (gc4[k] - c[k] * dot) * inv;
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) g[k] += gc4[k] / kEps;
    }
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) g4[k] = g[k];
}

// Backward of glue_slots_kernel: the means gradient of each slot's bank row is written to
// gstats[b][idx[b][j]][0..3] (slots of a row are distinct positions; the caller zeroes the
// other rows), and per-workgroup partial sums of the eight parameter gradients go to
// partial[block][8] (summed in a fixed order by glue_params_reduce_kernel).
__global__ void __launch_bounds__(256) glue_slots_bwd_kernel(
    int64_t n, int N, int L, int64_t ld, const float* __restrict__ stats,
    const int64_t* __restrict__ idx, float hidden, Ptr8 prm, int mode, const float* gkb,
    const float* gadm, const float* gcb, float* gstats, int64_t ldg, float* partial) {
  __shared__ float sh[4][8];
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  float gp[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (i < n) {
    const int64_t b = i / N;
    int64_t pos = idx[i];
    pos = pos < 0 ? 0 : (pos >= L ? L - 1 : pos);
    float P[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) P[k] = prm.p[k][0];
    float g4[4];
    glue_row_bwd(stats + b * ld + pos * 6, hidden, P, mode, gkb[i], gadm[i], gcb + i * 4, g4, gp);
    float* o = gstats + b * ldg + pos * 6;
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = g4[k];
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const float v = wave_sum(gp[k]);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6][k] = v;
  }
  __syncthreads();
  if (threadIdx.x < 8) {
    const int k = threadIdx.x;
    partial[static_cast<size_t>(blockIdx.x) * 8 + k] = (sh[0][k] + sh[1][k]) + (sh[2][k] + sh[3][k]);
  }
}

// One wave per parameter (8 waves): lane l sums the partials of blocks l, l + 64, ... in
// order, then the wave's lanes are combined in a fixed tree order.
__global__ void __launch_bounds__(512) glue_params_reduce_kernel(int nblocks, const float* partial,
                                                                 float* gparams) {
  const int k = threadIdx.x >> 6, lane = threadIdx.x & 63;
  float acc = 0.0f;
  for (int i = lane; i < nblocks; i += 64) acc += partial[static_cast<size_t>(i) * 8 + k];
  acc = wave_sum(acc);
  if (lane == 0) gparams[k] = acc;
}

// Backward of the query cocktails (means_glue rows with only the cocktail output): rows
// (b, t), t < T, ld floats apart per batch row; gstats rows ldg apart.
__global__ void __launch_bounds__(256) glue_rows_bwd_kernel(int64_t n, int T, int64_t ld,
                                                            const float* __restrict__ stats,
                                                            int mode, const float* gck,
                                                            float* gstats, int64_t ldg) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  const int64_t b = i / T, t = i % T;
  const float P[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float gp[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float g4[4];
  glue_row_bwd(stats + b * ld + t * 6, 1.0f, P, mode, 0.0f, 0.0f, gck + i * 4, g4, gp);
  float* o = gstats + b * ldg + t * 6;
#pragma unroll
  for (int k = 0; k < 4; ++k) o[k] = g4[k];
}

// Incremental admission of the positions base .. base + n - 1 appended to a carried bank
// (streaming decode). One workgroup per batch row: its threads compute the new positions'
// glue into the bank's glue arrays (unless `stats` is null: the admission values are then
// already there), then thread 0 walks them in order, keeping the running prefix max, and
// appends each member position to the row's slot list. In seq geometry the floor of a
// position depends only on the positions before it, so this equals bank_select over the
// whole bank: the same floor, comparison and order.
__global__ void __launch_bounds__(256) admit_step_kernel(int64_t n, int64_t base, int64_t cap,
                                                         const float* __restrict__ stats,
                                                         float hidden, Ptr8 prm, int mode,
                                                         const float* window, int floor_bf16,
                                                         float* kb, float* adm, float* ck,
                                                         float* amax, int64_t* mcount,
                                                         int64_t* members) {
  const int64_t b = blockIdx.x;
  const size_t row0 = static_cast<size_t>(b) * cap + base;
  if (stats) {
    for (int64_t t = threadIdx.x; t < n; t += 256)
      glue_row(stats + (row0 + t) * 6, hidden, prm, mode, kb + row0 + t, adm + row0 + t,
               ck + (row0 + t) * 4);
  }
  __syncthreads();  // the glue rows of this batch row, visible to thread 0
  if (threadIdx.x != 0) return;
  const float win = window[0];
  const float* a = adm + row0;
  int64_t* mem = members + static_cast<size_t>(b) * cap;
  float run = amax[b];
  int64_t c = base == 0 ? 0 : mcount[b];
  for (int64_t t = 0; t < n; ++t) {
    const float v = a[t];
    run = (base + t == 0 || v > run) ? v : run;
    const float fl = floor_bf16 ? round_to<bf16>(run - win) : run - win;
    if (v >= fl) mem[c++] = base + t;
  }
  amax[b] = run;
  mcount[b] = c;
}

extern "C" {

int dabsn_hip_tape_stats_window(int dtype, int64_t B, int64_t T, int64_t H, int64_t ldt,
                                const void* nov, const void* plast, const void* energy,
                                const void* sat, const void* expr, const void* write,
                                float* stats, int64_t lds, hipStream_t stream) {
  DABSN_REQUIRE(B > 0 && T >= 0 && H > 0 && H < (1 << 30) && T < (1ll << 31), "tape_stats: bad shape");
  DABSN_REQUIRE(ldt >= T && lds >= T, "tape_stats: row strides ldt=%lld, lds=%lld below T=%lld",
                (long long)ldt, (long long)lds, (long long)T);
  const int64_t rows = B * T;
  if (rows == 0) return DABSN_OK;
  DABSN_REQUIRE(nov && plast && energy && sat && expr && write && stats, "tape_stats: null pointer");
  const dim3 grid(blocks_for(rows, 4)), block(256);
  const bool vec = vec_ok(H, {nov, plast, energy, sat, expr, write});
#define L(E, V)                                                                                  \
  hipLaunchKernelGGL((stats_kernel<E, V>), grid, block, 0, stream, rows, (int)T, ldt, lds, (int)H, \
                     (const E*)nov, (const E*)plast, (const E*)energy, (const E*)sat,           \
                     (const E*)expr, (const E*)write, stats)
  GLUE_DISPATCH("tape_stats", dtype, vec, L);
#undef L
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

int dabsn_hip_tape_stats(int dtype, int64_t B, int64_t T, int64_t H, const void* nov,
                         const void* plast, const void* energy, const void* sat, const void* expr,
                         const void* write, float* stats, hipStream_t stream) {
  return dabsn_hip_tape_stats_window(dtype, B, T, H, T, nov, plast, energy, sat, expr, write,
                                     stats, T, stream);
}

int dabsn_hip_tape_stats_bwd_window(int dtype, int64_t B, int64_t T, int64_t H, int64_t ldt,
                                    const float* gstats, int64_t lds, int accumulate, void* gnov,
                                    void* gplast, void* genergy, void* gsat, hipStream_t stream) {
  DABSN_REQUIRE(B > 0 && T >= 0 && H > 0 && T < (1ll << 31), "tape_stats backward: bad shape");
  DABSN_REQUIRE(ldt >= T && lds >= T, "tape_stats backward: row strides below T");
  const int64_t rows = B * T;
  if (rows == 0) return DABSN_OK;
  DABSN_REQUIRE(gstats, "tape_stats backward: null gstats");
  const bool vec = vec_ok(H, {gnov, gplast, genergy, gsat});
  const int64_t V = vec ? 8 : 1;
  const int64_t chunks = rows * (H / V);
  DABSN_REQUIRE(chunks < (1ll << 32), "tape_stats backward: too many elements");
  const dim3 grid(blocks_for(chunks, 256)), block(256);
#define L(E, VV)                                                                                \
  hipLaunchKernelGGL((stats_bwd_kernel<E, VV>), grid, block, 0, stream, (uint32_t)chunks,      \
                     (uint32_t)(H / VV), (int)H, (int)T, ldt, lds, gstats, accumulate ? 1 : 0, \
                     (E*)genergy, (E*)gsat, (E*)gnov, (E*)gplast)
  GLUE_DISPATCH("tape_stats backward", dtype, vec, L);
#undef L
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

int dabsn_hip_tape_stats_bwd(int dtype, int64_t B, int64_t T, int64_t H, const float* gstats,
                             int accumulate, void* gnov, void* gplast, void* genergy, void* gsat,
                             hipStream_t stream) {
  return dabsn_hip_tape_stats_bwd_window(dtype, B, T, H, T, gstats, T, accumulate, gnov, gplast,
                                         genergy, gsat, stream);
}

int dabsn_hip_normalize_rows(int dtype, int64_t rows, int64_t H, const void* x, const float* norms,
                             void* q, hipStream_t stream) {
  if (rows == 0) return DABSN_OK;
  DABSN_REQUIRE(x && norms && q && H > 0 && rows > 0, "normalize_rows: bad arguments");
  const bool vec = vec_ok(H, {x, q});
  const int64_t V = vec ? 8 : 1;
  const int64_t chunks = rows * (H / V);
  DABSN_REQUIRE(chunks < (1ll << 32), "normalize_rows: too many elements");
  const dim3 grid(blocks_for(chunks, 256)), block(256);
#define L(E, VV)                                                                                \
  hipLaunchKernelGGL((normalize_kernel<E, VV>), grid, block, 0, stream, (uint32_t)chunks,      \
                     (uint32_t)(H / VV), (const E*)x, norms, (E*)q)
  GLUE_DISPATCH("normalize_rows", dtype, vec, L);
#undef L
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

int dabsn_hip_normalize_rows_bwd(int dtype, int64_t rows, int64_t H, const void* q,
                                 const float* norms, const void* gq, void* gx, hipStream_t stream) {
  if (rows == 0) return DABSN_OK;
  DABSN_REQUIRE(q && norms && gq && gx && H > 0, "normalize_rows backward: bad arguments");
  const dim3 grid(blocks_for(rows, 4)), block(256);
  const bool vec = vec_ok(H, {q, gq, gx});
#define L(E, V)                                                                                 \
  hipLaunchKernelGGL((normalize_bwd_kernel<E, V>), grid, block, 0, stream, rows, (int)H,       \
                     (const E*)q, norms, (const E*)gq, (E*)gx)
  GLUE_DISPATCH("normalize_rows backward", dtype, vec, L);
#undef L
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

int dabsn_hip_bank_select(int adm_dtype, int whole, int64_t B, int64_t T, const float* adm,
                          const float* window, int64_t* order, int64_t* counts, int32_t* rank,
                          hipStream_t stream) {
  DABSN_REQUIRE(B > 0 && T > 0 && T < (1ll << 30) && B < (1ll << 31), "bank_select: bad shape");
  DABSN_REQUIRE(adm_dtype == 0 || adm_dtype == 1, "bank_select: adm_dtype must be 0 or 1");
  DABSN_REQUIRE(whole == 0 || whole == 1, "bank_select: whole must be 0 or 1");
  DABSN_REQUIRE(adm && window && order && counts && rank, "bank_select: null pointer");
  hipLaunchKernelGGL(select_kernel, dim3((unsigned)B), dim3(SEL_T), 0, stream, (int)T, adm, window,
                     adm_dtype, whole, order, counts, rank);
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

int dabsn_hip_bank_fold(int64_t B, int64_t T, int64_t N, const int64_t* order,
                        const int64_t* counts, int8_t* codes, uint32_t* unfoldable,
                        hipStream_t stream) {
  DABSN_REQUIRE(B > 0 && B < 65536 && T > 0 && N >= 0 && N <= T && T < (1ll << 31),
                "bank_fold: bad shape");
  DABSN_REQUIRE(order && counts && (codes || unfoldable), "bank_fold: null pointer");
  if (unfoldable) {
    const int rc = dabsn_hip_zero(unfoldable, 4, stream);
    if (rc != DABSN_OK) return rc;
  }
  const int64_t width = unfoldable ? T : N;  // the flag covers every admitted slot
  if (width == 0) return DABSN_OK;
  hipLaunchKernelGGL(fold_kernel, dim3(blocks_for(width, 256), (unsigned)B), dim3(256), 0, stream,
                     (int)T, (int)N, order, counts, codes, unfoldable);
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

int dabsn_hip_window_add(int dtype, int64_t B, int64_t R, int64_t C, const void* a, int64_t a_sb,
                         int64_t a_sr, const void* x, int64_t x_sb, int64_t x_sr, void* out,
                         int64_t o_sb, int64_t o_sr, hipStream_t stream) {
  DABSN_REQUIRE(B >= 0 && R >= 0 && C >= 0, "window_add: bad shape");
  if (B == 0 || R == 0 || C == 0) return DABSN_OK;
  DABSN_REQUIRE(a && out, "window_add: null pointer");
  bool vec = C % 8 == 0 && a_sb % 8 == 0 && a_sr % 8 == 0 && o_sb % 8 == 0 && o_sr % 8 == 0;
  for (const void* q : {a, x, static_cast<const void*>(out)})
    if (q && (reinterpret_cast<uintptr_t>(q) & 15u) != 0) vec = false;
  if (x && (x_sb % 8 != 0 || x_sr % 8 != 0)) vec = false;
  const int64_t cpr = C / (vec ? 8 : 1);
  const int64_t chunks = B * R * cpr;
  DABSN_REQUIRE(chunks < (1ll << 32) && R < (1ll << 32), "window_add: too many elements");
  const dim3 grid(blocks_for(chunks, 256)), block(256);
#define L(E, VV)                                                                              \
  hipLaunchKernelGGL((window_add_kernel<E, VV>), grid, block, 0, stream, (uint32_t)chunks,      \
                     (uint32_t)cpr, (uint32_t)R, (const E*)a, a_sb, a_sr, (const E*)x, x_sb,    \
                     x_sr, (E*)out, o_sb, o_sr)
  GLUE_DISPATCH("window_add", dtype, vec, L);
#undef L
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

int dabsn_hip_bank_width(int64_t B, int64_t T, const int64_t* order, const int64_t* counts,
                         int check_fold, int64_t* out, hipStream_t stream) {
  DABSN_REQUIRE(B > 0 && B < 65536 && T > 0 && T < (1ll << 31), "bank_width: bad shape");
  DABSN_REQUIRE(counts && out && (order || !check_fold), "bank_width: null pointer");
  const int rc = dabsn_hip_zero(out, 2 * sizeof(int64_t), stream);
  if (rc != DABSN_OK) return rc;
  const unsigned xb = check_fold ? blocks_for(T, 256) : 1u;
  hipLaunchKernelGGL(width_kernel, dim3(xb, (unsigned)B), dim3(256), 0, stream, (int)T, order,
                     counts, check_fold ? 1 : 0, reinterpret_cast<unsigned long long*>(out));
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

int dabsn_hip_bank_slots(int64_t B, int64_t T, int64_t N, const int64_t* order,
                         const int64_t* counts, int64_t query_start, int64_t* idx,
                         uint8_t* valid, int64_t* next_idx, int64_t* read_idx, int8_t* codes,
                         hipStream_t stream) {
  DABSN_REQUIRE(B > 0 && B < 65536 && T > 0 && N >= 0 && N <= T && T < (1ll << 31),
                "bank_slots: bad shape");
  if (N == 0) return DABSN_OK;
  DABSN_REQUIRE(order && counts && idx && valid && next_idx && read_idx,
                "bank_slots: null pointer");
  hipLaunchKernelGGL(slots_kernel, dim3(blocks_for(N, 256), (unsigned)B), dim3(256), 0, stream,
                     (int)T, (int)N, query_start, order, counts, idx, valid, next_idx, read_idx,
                     codes);
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

int dabsn_hip_bank_gather(int dtype, int64_t B, int64_t T, int64_t N, int64_t H, const void* w,
                          const float* norm_w, const int64_t* idx, const int64_t* next_idx,
                          void* K, void* V, void* Vn, hipStream_t stream) {
  DABSN_REQUIRE(B > 0 && T > 0 && N >= 0 && H > 0, "bank_gather: bad shape");
  if (N == 0) return DABSN_OK;
  DABSN_REQUIRE(w && norm_w && idx && K && V && (next_idx || !Vn), "bank_gather: null pointer");
  const bool vec = vec_ok(H, {w, K, V, Vn});
  const int hblocks = static_cast<int>(blocks_for(H, 256 * (vec ? 8 : 1)));
  DABSN_REQUIRE(B * N * hblocks <= 2147483647ll, "bank_gather: too many bank rows");
  const dim3 grid(static_cast<unsigned>(B * N * hblocks)), block(256);
#define L(E, VV)                                                                                \
  hipLaunchKernelGGL((gather_kernel<E, VV>), grid, block, 0, stream, (int)T, (int)N, (int)H,   \
                     hblocks, (const E*)w, norm_w, idx, next_idx, (E*)K, (E*)V, (E*)Vn)
  GLUE_DISPATCH("bank_gather", dtype, vec, L);
#undef L
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

int dabsn_hip_bank_gather_bwd(int dtype, int64_t B, int64_t T, int64_t N, int64_t H,
                              const void* w, const float* norm_w, const int32_t* rank,
                              const void* K, const void* gK, const void* gV, const void* gVn,
                              void* gw, hipStream_t stream) {
  (void)w;
  DABSN_REQUIRE(B > 0 && T > 0 && N >= 0 && H > 0, "bank_gather backward: bad shape");
  // Every position is written (zero where no slot maps to it), N == 0 included.
  DABSN_REQUIRE(gw && norm_w && rank && (N == 0 || (K && gK && gV)),
                "bank_gather backward: null pointer");
  return dabsn_hip_bank_gather_bwd_prefix(dtype, B, T, T, N, H, norm_w, rank, K, gK, gV, gVn, 0,
                                          gw, stream);
}

int dabsn_hip_bank_gather_bwd_prefix(int dtype, int64_t B, int64_t T, int64_t ldg, int64_t N,
                                     int64_t H, const float* norm_w, const int32_t* rank,
                                     const void* K, const void* gK, const void* gV,
                                     const void* gVn, int accumulate, void* gw,
                                     hipStream_t stream) {
  DABSN_REQUIRE(B > 0 && T > 0 && ldg >= T && N >= 0 && H > 0, "bank_gather backward: bad shape");
  DABSN_REQUIRE(gw && norm_w && rank && (N == 0 || (K && gK && gV)),
                "bank_gather backward: null pointer");
  DABSN_REQUIRE(B * T <= 2147483647ll && B * ldg < (1ll << 40),
                "bank_gather backward: too many positions");
  const dim3 grid((unsigned)(B * T)), block(256);
  const bool vec = vec_ok(H, {K, gK, gV, gVn, gw});
#define L(E, VV)                                                                                \
  hipLaunchKernelGGL((gather_bwd_kernel<E, VV>), grid, block, 0, stream, (int)T, (int)ldg,     \
                     (int)N, (int)H, norm_w, rank, (const E*)K, (const E*)gK, (const E*)gV,     \
                     (const E*)gVn, accumulate ? 1 : 0, (E*)gw)
  GLUE_DISPATCH("bank_gather backward", dtype, vec, L);
#undef L
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

static bool read_out_vec(int64_t n, std::initializer_list<const void*> ptrs) {
  if (n % 8 != 0) return false;
  for (const void* p : ptrs)
    if (reinterpret_cast<uintptr_t>(p) & 15u) return false;
  return true;
}

// Calls LAUNCH(A, B, C, V) with A, B, C the element types of three dtype codes.
#define READ_OUT_TYPES(what, da, db, dc, vec, LAUNCH)                                     \
  do {                                                                                    \
    DABSN_REQUIRE((da == kF32 || da == kBF16) && (db == kF32 || db == kBF16) &&           \
                      (dc == kF32 || dc == kBF16),                                        \
                  "%s: dtype codes must be 0 (fp32) or 1 (bf16)", what);                  \
    const int code = (da == kBF16 ? 4 : 0) | (db == kBF16 ? 2 : 0) | (dc == kBF16 ? 1 : 0); \
    switch (code * 2 + (vec ? 1 : 0)) {                                                   \
      case 0: LAUNCH(float, float, float, 1); break;                                      \
      case 1: LAUNCH(float, float, float, 8); break;                                      \
      case 2: LAUNCH(float, float, bf16, 1); break;                                       \
      case 3: LAUNCH(float, float, bf16, 8); break;                                       \
      case 4: LAUNCH(float, bf16, float, 1); break;                                       \
      case 5: LAUNCH(float, bf16, float, 8); break;                                       \
      case 6: LAUNCH(float, bf16, bf16, 1); break;                                        \
      case 7: LAUNCH(float, bf16, bf16, 8); break;                                        \
      case 8: LAUNCH(bf16, float, float, 1); break;                                       \
      case 9: LAUNCH(bf16, float, float, 8); break;                                       \
      case 10: LAUNCH(bf16, float, bf16, 1); break;                                       \
      case 11: LAUNCH(bf16, float, bf16, 8); break;                                       \
      case 12: LAUNCH(bf16, bf16, float, 1); break;                                       \
      case 13: LAUNCH(bf16, bf16, float, 8); break;                                       \
      case 14: LAUNCH(bf16, bf16, bf16, 1); break;                                        \
      default: LAUNCH(bf16, bf16, bf16, 8); break;                                        \
    }                                                                                     \
  } while (0)

// Segment strides of `n` tensors in V-element chunks (one segment: the row length); false
// when a stride is shorter than a row or, on the vector path, not a multiple of 8.
static bool seg_strides(int64_t rows, int64_t row_len, const int64_t* ld, int n, int64_t V,
                        SegLd& out) {
  for (int k = 0; k < n; ++k) {
    if (rows > 1 && (ld[k] < row_len || ld[k] % V != 0)) return false;
    out.ld[k] = static_cast<uint64_t>((rows <= 1 ? row_len : ld[k]) / V);
  }
  return true;
}

// read_output over `rows` segments of row_len elements, ld[k] elements apart in tensor k
// (proj, long, out; a flat array: one row). The vector path needs row_len and every ld
// multiples of 8 and 16-byte aligned bases.
static int read_output_rows(const char* what, int proj_dtype, int long_dtype, int prod_dtype,
                            int out_dtype, int64_t rows, int64_t row_len, const int64_t ld[3],
                            const void* proj, const void* lng, const float* gain, void* out,
                            hipStream_t stream) {
  SegLd sl{};
  DABSN_REQUIRE(rows >= 0 && row_len >= 0 && seg_strides(rows, row_len, ld, 3, 1, sl),
                "%s: bad size", what);
  const int64_t n = rows * row_len;
  if (n == 0) return DABSN_OK;
  DABSN_REQUIRE(proj && lng && gain && out, "%s: null pointer", what);
  DABSN_REQUIRE(prod_dtype == kF32 || prod_dtype == kBF16, "%s: bad product dtype", what);
  const bool vec =
      read_out_vec(row_len, {proj, lng, out}) && seg_strides(rows, row_len, ld, 3, 8, sl);
  if (!vec) seg_strides(rows, row_len, ld, 3, 1, sl);
  const int64_t V = vec ? 8 : 1;
  const int64_t chunks = n / V, seg = row_len / V;
  DABSN_REQUIRE(chunks < (1ll << 32), "%s: too many elements", what);
  const dim3 grid(blocks_for(chunks, 256)), block(256);
#define L(P, Lt, O, VV)                                                                        \
  hipLaunchKernelGGL((read_out_kernel<P, Lt, O, VV>), grid, block, 0, stream, (uint32_t)chunks,  \
                     (uint32_t)seg, sl, (const P*)proj, (const Lt*)lng, gain,                   \
                     prod_dtype == kBF16 ? 1 : 0, (O*)out)
  READ_OUT_TYPES(what, proj_dtype, long_dtype, out_dtype, vec, L);
#undef L
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

// Its backward; ld[k] for gout, long, gproj, glong.
static int read_output_bwd_rows(const char* what, int out_dtype, int proj_dtype, int long_dtype,
                                int prod_dtype, int64_t rows, int64_t row_len,
                                const int64_t ld[4], const void* gout, const void* lng,
                                const float* gain, void* gproj, void* glong, float* ggain,
                                float* partials, size_t partial_count, hipStream_t stream) {
  SegLd sl{};
  DABSN_REQUIRE(rows >= 0 && row_len >= 0 && seg_strides(rows, row_len, ld, 4, 1, sl),
                "%s: bad size", what);
  DABSN_REQUIRE(ggain && partials, "%s: null pointer", what);
  const int64_t n = rows * row_len;
  if (n == 0) return dabsn_hip_zero(ggain, 4, stream);
  DABSN_REQUIRE(gout && lng && gain && gproj && glong, "%s: null pointer", what);
  DABSN_REQUIRE(prod_dtype == kF32 || prod_dtype == kBF16, "%s: bad product dtype", what);
  const bool vec = read_out_vec(row_len, {gout, lng, gproj, glong}) &&
                   seg_strides(rows, row_len, ld, 4, 8, sl);
  if (!vec) seg_strides(rows, row_len, ld, 4, 1, sl);
  const int64_t V = vec ? 8 : 1;
  const int64_t chunks = n / V, seg = row_len / V;
  DABSN_REQUIRE(chunks < (1ll << 32), "%s: too many elements", what);
  const unsigned nblk = blocks_for(chunks, 256);
  DABSN_REQUIRE(partial_count >= nblk, "%s: %zu partials < %u", what, partial_count, nblk);
  const dim3 grid(nblk), block(256);
#define L(O, P, Lt, VV)                                                                        \
  hipLaunchKernelGGL((read_out_bwd_kernel<O, P, Lt, VV>), grid, block, 0, stream,              \
                     (uint32_t)chunks, (uint32_t)seg, sl, (const O*)gout,                       \
                     (const Lt*)lng, gain, prod_dtype == kBF16 ? 1 : 0, (P*)gproj, (Lt*)glong,  \
                     partials)
  READ_OUT_TYPES(what, out_dtype, proj_dtype, long_dtype, vec, L);
#undef L
  DABSN_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(read_out_reduce_kernel, dim3(1), dim3(1024), 0, stream, nblk, partials, ggain);
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

int dabsn_hip_read_output(int proj_dtype, int long_dtype, int prod_dtype, int out_dtype,
                          int64_t n, const void* proj, const void* lng, const float* gain,
                          void* out, hipStream_t stream) {
  DABSN_REQUIRE(n >= 0, "read_output: bad size");
  const int64_t ld[3] = {n, n, n};
  return read_output_rows("read_output", proj_dtype, long_dtype, prod_dtype, out_dtype, 1, n, ld,
                          proj, lng, gain, out, stream);
}

int dabsn_hip_read_output_window(int proj_dtype, int long_dtype, int prod_dtype, int out_dtype,
                                 int64_t rows, int64_t row_len, int64_t ld_proj,
                                 int64_t ld_long, int64_t ld_out, const void* proj,
                                 const void* lng, const float* gain, void* out,
                                 hipStream_t stream) {
  const int64_t ld[3] = {ld_proj, ld_long, ld_out};
  return read_output_rows("read_output window", proj_dtype, long_dtype, prod_dtype, out_dtype,
                          rows, row_len, ld, proj, lng, gain, out, stream);
}

size_t dabsn_hip_read_output_partials(int64_t n) {
  // One partial per workgroup of 256 threads; the unvectorised count bounds both cases.
  return static_cast<size_t>(blocks_for(n > 0 ? n : 1, 256));
}

int dabsn_hip_read_output_bwd(int out_dtype, int proj_dtype, int long_dtype, int prod_dtype,
                              int64_t n, const void* gout, const void* lng, const float* gain,
                              void* gproj, void* glong, float* ggain, float* partials,
                              size_t partial_count, hipStream_t stream) {
  DABSN_REQUIRE(n >= 0, "read_output backward: bad size");
  const int64_t ld[4] = {n, n, n, n};
  return read_output_bwd_rows("read_output backward", out_dtype, proj_dtype, long_dtype,
                              prod_dtype, 1, n, ld, gout, lng, gain, gproj, glong, ggain,
                              partials, partial_count, stream);
}

int dabsn_hip_read_output_bwd_window(int out_dtype, int proj_dtype, int long_dtype,
                                     int prod_dtype, int64_t rows, int64_t row_len,
                                     int64_t ld_gout, int64_t ld_long, int64_t ld_gproj,
                                     int64_t ld_glong, const void* gout, const void* lng,
                                     const float* gain, void* gproj, void* glong, float* ggain,
                                     float* partials, size_t partial_count, hipStream_t stream) {
  const int64_t ld[4] = {ld_gout, ld_long, ld_gproj, ld_glong};
  return read_output_bwd_rows("read_output window backward", out_dtype, proj_dtype, long_dtype,
                              prod_dtype, rows, row_len, ld, gout, lng, gain, gproj, glong,
                              ggain, partials, partial_count, stream);
}

int dabsn_hip_admit_step(int mode, int64_t B, int64_t n, int64_t base, int64_t cap,
                         const float* stats, int64_t hidden, const float* const* params,
                         const float* window, int adm_dtype, float* key_bias, float* admission,
                         float* cocktail, float* amax, int64_t* mcount, int64_t* members,
                         hipStream_t stream) {
  DABSN_REQUIRE(mode >= 0 && mode <= 3, "admit_step: mode must be 0..3");
  DABSN_REQUIRE(adm_dtype == 0 || adm_dtype == 1, "admit_step: adm_dtype must be 0 or 1");
  DABSN_REQUIRE(B > 0 && B < (1ll << 31) && n >= 0 && base >= 0 && base + n <= cap && hidden > 0,
                "admit_step: bad shape (B %lld, n %lld, base %lld, cap %lld)", (long long)B,
                (long long)n, (long long)base, (long long)cap);
  if (n == 0) return DABSN_OK;
  DABSN_REQUIRE(window && admission && amax && mcount && members, "admit_step: null pointer");
  Ptr8 prm{};
  if (stats) {
    DABSN_REQUIRE(params && key_bias && cocktail, "admit_step: null glue pointer");
    DABSN_REQUIRE((reinterpret_cast<uintptr_t>(cocktail) & 15u) == 0,
                  "admit_step: cocktail must be 16-byte aligned");
    for (int k = 0; k < 8; ++k) {
      DABSN_REQUIRE(params[k], "admit_step: null parameter %d", k);
      prm.p[k] = params[k];
    }
  }
  hipLaunchKernelGGL(admit_step_kernel, dim3(static_cast<unsigned>(B)), dim3(256), 0, stream, n,
                     base, cap, stats, static_cast<float>(hidden), prm, mode, window, adm_dtype,
                     key_bias, admission, cocktail, amax, mcount, members);
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

static int ptr8_of(const float* const* params, Ptr8& prm, const char* what) {
  for (int k = 0; k < 8; ++k) {
    DABSN_REQUIRE(params[k], "%s: null parameter %d", what, k);
    prm.p[k] = params[k];
  }
  return DABSN_OK;
}

int dabsn_hip_glue_slots(int64_t B, int64_t N, int64_t L, int64_t ld, const float* stats,
                         const int64_t* idx, int64_t hidden, const float* const* params, int mode,
                         float* key_bias, float* admission, float* cocktail, hipStream_t stream) {
  DABSN_REQUIRE(mode >= 0 && mode <= 3, "glue_slots: mode must be 0..3");
  DABSN_REQUIRE(B > 0 && N >= 0 && L > 0 && ld >= 6 * L && hidden > 0 && B * N < (1ll << 40),
                "glue_slots: bad shape");
  if (N == 0) return DABSN_OK;
  DABSN_REQUIRE(stats && idx && params && key_bias && admission && cocktail,
                "glue_slots: null pointer");
  DABSN_REQUIRE((reinterpret_cast<uintptr_t>(cocktail) & 15u) == 0,
                "glue_slots: cocktail must be 16-byte aligned");
  Ptr8 prm;
  if (ptr8_of(params, prm, "glue_slots") != DABSN_OK) return DABSN_ERR_ARG;
  const int64_t n = B * N;
  hipLaunchKernelGGL(glue_slots_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, stream, n, (int)N,
                     (int)L, ld, stats, idx, static_cast<float>(hidden), prm, mode, key_bias,
                     admission, cocktail);
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

size_t dabsn_hip_glue_slots_partials(int64_t B, int64_t N) {
  return static_cast<size_t>(blocks_for(B * N, 256)) * 8 * sizeof(float);
}

int dabsn_hip_glue_slots_bwd(int64_t B, int64_t N, int64_t L, int64_t ld, const float* stats,
                             const int64_t* idx, int64_t hidden, const float* const* params,
                             int mode, const float* gkey_bias, const float* gadmission,
                             const float* gcocktail, float* gstats, int64_t ldg, float* partial,
                             float* gparams, hipStream_t stream) {
  DABSN_REQUIRE(mode >= 0 && mode <= 3, "glue_slots backward: mode must be 0..3");
  DABSN_REQUIRE(B > 0 && N >= 0 && L > 0 && ld >= 6 * L && ldg >= 6 * L && hidden > 0 &&
                    B * N < (1ll << 40),
                "glue_slots backward: bad shape");
  DABSN_REQUIRE(gparams, "glue_slots backward: null gparams");
  if (N == 0) return dabsn_hip_zero(gparams, 8 * sizeof(float), stream);
  DABSN_REQUIRE(stats && idx && params && gkey_bias && gadmission && gcocktail && gstats && partial,
                "glue_slots backward: null pointer");
  Ptr8 prm;
  if (ptr8_of(params, prm, "glue_slots backward") != DABSN_OK) return DABSN_ERR_ARG;
  const int64_t n = B * N;
  const unsigned nblk = blocks_for(n, 256);
  hipLaunchKernelGGL(glue_slots_bwd_kernel, dim3(nblk), dim3(256), 0, stream, n, (int)N, (int)L,
                     ld, stats, idx, static_cast<float>(hidden), prm, mode, gkey_bias, gadmission,
                     gcocktail, gstats, ldg, partial);
  DABSN_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(glue_params_reduce_kernel, dim3(1), dim3(512), 0, stream, (int)nblk, partial,
                     gparams);
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

int dabsn_hip_glue_rows_bwd(int64_t B, int64_t T, int64_t ld, const float* stats, int mode,
                            const float* gcocktail, float* gstats, int64_t ldg,
                            hipStream_t stream) {
  DABSN_REQUIRE(mode >= 0 && mode <= 3, "glue_rows backward: mode must be 0..3");
  DABSN_REQUIRE(B > 0 && T >= 0 && ld >= 6 * T && ldg >= 6 * T && T < (1ll << 31),
                "glue_rows backward: bad shape");
  if (T == 0) return DABSN_OK;
  DABSN_REQUIRE(stats && gcocktail && gstats, "glue_rows backward: null pointer");
  const int64_t n = B * T;
  hipLaunchKernelGGL(glue_rows_bwd_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, stream, n,
                     (int)T, ld, stats, mode, gcocktail, gstats, ldg);
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

int dabsn_hip_means_glue(int64_t B, int64_t N, int64_t ld, const float* stats, int64_t hidden,
                         const float* const* params, int mode, float* key_bias, float* admission,
                         float* cocktail, hipStream_t stream) {
  DABSN_REQUIRE(mode >= 0 && mode <= 3, "means_glue: mode must be 0..3");
  DABSN_REQUIRE(B > 0 && N >= 0 && N < (1 << 30) && ld >= 6 * N && hidden > 0,
                "means_glue: bad shape");
  const int64_t rows = B * N;
  if (rows == 0) return DABSN_OK;
  DABSN_REQUIRE(stats && params && cocktail, "means_glue: null pointer");
  DABSN_REQUIRE((reinterpret_cast<uintptr_t>(cocktail) & 15u) == 0,
                "means_glue: cocktail must be 16-byte aligned");
  Ptr8 prm;
  for (int k = 0; k < 8; ++k) {
    DABSN_REQUIRE(params[k], "means_glue: null parameter %d", k);
    prm.p[k] = params[k];
  }
  hipLaunchKernelGGL(means_glue_kernel, dim3(static_cast<unsigned>((rows + 255) / 256)), dim3(256),
                     0, stream, rows, (int)N, ld, stats, static_cast<float>(hidden), prm, mode,
                     key_bias, admission, cocktail);
  DABSN_HIP_CHECK(hipGetLastError());
  return DABSN_OK;
}

}  // extern "C"
