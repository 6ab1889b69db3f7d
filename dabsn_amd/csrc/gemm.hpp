// Batched MFMA GEMM with per-tile work ranges, used by the three-way read.
//
//   C[b](m, n) = alpha * sum_k A[b](m, k) B[b](n, k)  (+ A2[b](m, k) B2[b](n, k))
//
// Both operands are K-contiguous: A(m, k) = A[m*lda + k], B(n, k) = B[n*ldb + k] (callers
// hand M- or N-contiguous operands over as transposed copies). Causal structure is
// expressed per (batch, 128-row tile) as a k-range [klo, khi) and a column limit nhi:
// tiles at or beyond nhi are skipped and only k-tiles that intersect [klo, khi) are
// visited (the operands are zero outside that range by construction of the callers, and
// elements outside it are read as zero).
//
// Block tile BM x BN with WM x WN waves, each wave a (BM/WM) x (BN/WN) grid of 16x16
// MFMA tiles (v_mfma_f32_16x16x32_bf16, or 16x16x4 fp32). K advances BK at a time
// through two LDS buffers: the 16-byte global loads of k-tile kt + 2 are in flight while
// the MFMAs consume k-tile kt, and one barrier per k-tile separates the buffers.
//
// Blocks are mapped XCD-aware: hardware deals consecutive workgroups round-robin over the
// 8 XCDs, so workgroup L runs logical tile (L % 8) * C + L / 8 (C = tiles per XCD). Each
// XCD walks a contiguous range of the logical order, which is batch-major and, within a
// batch, made of 8 x 8-tile patches: the ~64 blocks an XCD runs at once share A and B
// k-slices in its L2.
#pragma once

#include "common.hpp"

namespace dabsn {
namespace gemm {

constexpr int RANGE_ROWS = 128;  // rows per entry of the k-range table
constexpr int PATCH = 8;         // patch edge (tiles) of the XCD-local block order

template <typename E>
struct G;
template <>
struct G<bf16> {
  // LDS rows are 64 elements (8 chunks of 16 bytes) with no padding; chunk c of row r is
  // stored at position c ^ ((r >> 1) & 7). The 16 lanes of one b128 read (rows r..r+15,
  // one logical chunk) and the 16 lanes of one b128 write (two rows) then touch 16
  // distinct 16-byte bank groups.
  static constexpr int BK = 64, PAD = 0, VEC = 8, KSTEP = 32;
  using R = bf16x8;
  __device__ static int pos(int c, int r) { return c ^ ((r >> 1) & 7); }
  // Fragment of k-step ks for the lane's row (row & 15 == lane & 15).
  __device__ static R frag(const bf16* row, int ks, int lane) {
    return __builtin_bit_cast(
        R, *reinterpret_cast<const u32x4*>(row + pos(ks * 4 + (lane >> 4), lane & 15) * 8));
  }
  __device__ static f32x4 mma(R a, R b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct G<float> {
  static constexpr int BK = 32, PAD = 4, VEC = 4, KSTEP = 4;
  using R = float;
  __device__ static int pos(int c, int) { return c; }
  __device__ static R frag(const float* row, int ks, int lane) { return row[ks * KSTEP + (lane >> 4)]; }
  __device__ static f32x4 mma(R a, R b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
};

template <typename E, typename OUT>
struct Args {
  int M, N, K;
  const E* A;
  int64_t lda, sA;
  const E* B;
  int64_t ldb, sB;
  const E* A2;  // optional second product (same layout and strides as A, B)
  const E* B2;
  OUT* C;
  int64_t ldc, sC;
  float alpha;
  const int32_t* ranges;  // optional [batch][ceil(M / 128)][3] = (klo, khi, nhi)
  int mtiles;             // entries per batch of `ranges`
};

template <typename OUT>
__device__ __forceinline__ void put(OUT* p, float v);
template <>
__device__ __forceinline__ void put<float>(float* p, float v) { *p = v; }
template <>
__device__ __forceinline__ void put<bf16>(bf16* p, float v) { *p = f2bf(v); }

// Stores 4 consecutive values (p aligned to 4 elements).
template <typename OUT>
__device__ __forceinline__ void store4(OUT* p, f32x4 v);
template <>
__device__ __forceinline__ void store4<float>(float* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }
template <>
__device__ __forceinline__ void store4<bf16>(bf16* p, f32x4 v) {
  const uint32_t lo = static_cast<uint32_t>(f2bf(v[0])) | (static_cast<uint32_t>(f2bf(v[1])) << 16);
  const uint32_t hi = static_cast<uint32_t>(f2bf(v[2])) | (static_cast<uint32_t>(f2bf(v[3])) << 16);
  *reinterpret_cast<uint2*>(p) = make_uint2(lo, hi);
}

template <int BM, int BN, int WM, int WN>
struct Shape {
  static constexpr int NTH = WM * WN * 64;
  static constexpr int TM = BM / WM / 16, TN = BN / WN / 16;
  static_assert(BM % (WM * 16) == 0 && BN % (WN * 16) == 0, "wave tiles must be whole MFMA tiles");
  static_assert(BM % RANGE_ROWS == 0 || RANGE_ROWS % BM == 0, "row tiles must nest with the ranges");
};

// Logical tile of workgroup L (see the header comment); false for padding workgroups.
__device__ __forceinline__ bool tile_of(int L, int nblk, int batch, int mt_n, int nt_n, int& bz,
                                        int& mt, int& nt) {
  const int per_xcd = nblk / 8;
  const int g = (L % 8) * per_xcd + L / 8;
  const int per_batch = mt_n * nt_n;
  if (g >= batch * per_batch) return false;
  bz = g / per_batch;
  int r = g % per_batch;
  // Patches of PATCH x PATCH tiles, row-major; a partial last patch row/column is
  // narrower.
  const int prow = PATCH * nt_n;  // tiles per band of PATCH tile rows
  const int band = r / prow;
  r %= prow;
  const int rows = min(PATCH, mt_n - band * PATCH);
  const int pcol = r / (rows * PATCH);
  r %= rows * PATCH;
  const int cols = min(PATCH, nt_n - pcol * PATCH);
  mt = band * PATCH + r / cols;
  nt = pcol * PATCH + r % cols;
  return true;
}

template <typename E, typename OUT, int BM, int BN, int WM, int WN, bool VECOK>
__global__ void __launch_bounds__(WM * WN * 64) gemm_kernel(Args<E, OUT> a, int batch, int nblk) {
  using S = Shape<BM, BN, WM, WN>;
  constexpr int NTH = S::NTH, TM = S::TM, TN = S::TN;
  constexpr int BK = G<E>::BK, PAD = G<E>::PAD, VEC = G<E>::VEC, KSTEP = G<E>::KSTEP;
  constexpr int LDR = BK + PAD;                         // LDS row pitch (elements)
  constexpr int CPR = BK / VEC;                         // 16-byte chunks per row
  constexpr int NV = (BM + BN) * CPR / NTH;             // chunks per thread per k-tile
  static_assert((BM + BN) * CPR % NTH == 0, "staging must divide evenly");
  __shared__ __attribute__((aligned(16))) E lds[2][BM + BN][LDR];

  const int mt_n = (a.M + BM - 1) / BM, nt_n = (a.N + BN - 1) / BN;
  int bz, mt, nt;
  if (!tile_of(blockIdx.x, nblk, batch, mt_n, nt_n, bz, mt, nt)) return;
  const int m0 = mt * BM, n0 = nt * BN;
  // k-range of each 128-row range entry this row tile covers (A rows are zero outside
  // their own entry's range and may be unwritten there), and their union.
  constexpr int NSUB = BM >= RANGE_ROWS ? BM / RANGE_ROWS : 1;
  int sklo[NSUB], skhi[NSUB];
  int klo = a.K, khi = 0, nhi = 0;
#pragma unroll
  for (int u = 0; u < NSUB; ++u) {
    sklo[u] = 0;
    skhi[u] = a.K;
    int sn = a.N;
    const int r = m0 / RANGE_ROWS + u;
    if (a.ranges) {
      if (r < a.mtiles) {
        const int32_t* e = a.ranges + (static_cast<int64_t>(bz) * a.mtiles + r) * 3;
        sklo[u] = max(0, e[0]);
        skhi[u] = min(a.K, e[1]);
        sn = min(a.N, e[2]);
      } else {
        sklo[u] = skhi[u] = 0;
        sn = 0;
      }
    }
    if (skhi[u] > sklo[u]) {
      klo = min(klo, sklo[u]);
      khi = max(khi, skhi[u]);
    }
    nhi = max(nhi, sn);
  }
  if (n0 >= nhi) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

  if (khi > klo) {
    const int kt0 = klo / BK, kt1 = (khi + BK - 1) / BK;
    const int nprod = a.A2 ? 2 : 1;
    const int nk = kt1 - kt0;
    const int total = nprod * nk;  // k-tiles over both products
    // Operands are read through buffer resources over this batch's slice: rows beyond M
    // (N) lie beyond the resource and read as zero. Chunk i of a thread covers row
    // tid / CPR + i * RPI of the stacked [A rows; B rows] tile, so its offset is one
    // per-thread base plus a per-chunk scalar stride, and its k-range entry is fixed at
    // compile time: A rows use their own 128-row entry (they are zero outside it and may
    // be unwritten there), B rows the union. k-tiles inside every non-empty range take
    // the 16-byte path, decided once per k-tile for the whole block.
    constexpr int RPI = NTH / CPR;  // rows per chunk index
    constexpr int NVA = BM / RPI;   // chunk indices that hold A rows
    static_assert(BM % RPI == 0 && (RPI % RANGE_ROWS == 0 || RANGE_ROWS % RPI == 0),
                  "chunk rows must nest with the A rows and the range entries");
    constexpr uint32_t ES = sizeof(E);
    const __amdgpu_buffer_rsrc_t rA = make_rsrc(a.A + static_cast<int64_t>(bz) * a.sA,
                                                static_cast<uint32_t>(a.M * a.lda * ES));
    const __amdgpu_buffer_rsrc_t rB = make_rsrc(a.B + static_cast<int64_t>(bz) * a.sB,
                                                static_cast<uint32_t>(a.N * a.ldb * ES));
    const __amdgpu_buffer_rsrc_t rA2 =
        a.A2 ? make_rsrc(a.A2 + static_cast<int64_t>(bz) * a.sA, static_cast<uint32_t>(a.M * a.lda * ES)) : rA;
    const __amdgpu_buffer_rsrc_t rB2 =
        a.B2 ? make_rsrc(a.B2 + static_cast<int64_t>(bz) * a.sB, static_cast<uint32_t>(a.N * a.ldb * ES)) : rB;
    const int trow = tid / CPR, tk = (tid % CPR) * VEC;
    const uint32_t voffA = static_cast<uint32_t>(((m0 + trow) * a.lda + tk) * ES);
    const uint32_t voffB = static_cast<uint32_t>(((n0 + trow) * a.ldb + tk) * ES);
    const uint32_t strideA = static_cast<uint32_t>(RPI * a.lda * ES);
    const uint32_t strideB = static_cast<uint32_t>(RPI * a.ldb * ES);
    int lo_max = klo, hi_min = khi;
#pragma unroll
    for (int u = 0; u < NSUB; ++u) {
      if (skhi[u] > sklo[u]) {
        lo_max = max(lo_max, sklo[u]);
        hi_min = min(hi_min, skhi[u]);
      }
    }
    u32x4 stage[NV];
    auto load = [&](int it) {
      const int pr = it / nk;
      const int k0 = (kt0 + it % nk) * BK;
      const __amdgpu_buffer_rsrc_t ra = pr == 0 ? rA : rA2;
      const __amdgpu_buffer_rsrc_t rb = pr == 0 ? rB : rB2;
      const bool fast = VECOK && k0 >= lo_max && k0 + BK <= hi_min;
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const bool isA = i < NVA;
        const int u = isA && NSUB > 1 ? (i * RPI) / RANGE_ROWS : 0;
        const int lo = isA ? sklo[u] : klo, hi = isA ? skhi[u] : khi;
        const __amdgpu_buffer_rsrc_t r = isA ? ra : rb;
        // The whole offset goes in the VGPR operand: the range check applies to it.
        const int off = static_cast<int>((isA ? voffA + i * strideA : voffB + (i - NVA) * strideB) + k0 * ES);
        if (fast) {
          stage[i] = hi > lo ? __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0) : (u32x4){0u, 0u, 0u, 0u};
        } else {
          const int k = k0 + tk;
          E v[VEC];
          if constexpr (VECOK) {
            *reinterpret_cast<u32x4*>(v) = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
#pragma unroll
            for (int e = 0; e < VEC; ++e)
              if (k + e < lo || k + e >= hi) v[e] = static_cast<E>(0);
          } else {
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
              const int o = off + e * static_cast<int>(ES);
              if constexpr (sizeof(E) == 2) {
                const uint16_t w = __builtin_amdgcn_raw_buffer_load_b16(r, o, 0, 0);
                v[e] = __builtin_bit_cast(E, w);
              } else {
                const uint32_t w = __builtin_amdgcn_raw_buffer_load_b32(r, o, 0, 0);
                v[e] = __builtin_bit_cast(E, w);
              }
              if (k + e < lo || k + e >= hi) v[e] = static_cast<E>(0);
            }
          }
          stage[i] = *reinterpret_cast<const u32x4*>(v);
        }
      }
    };
    auto store = [&](int buf) {
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int q = tid + i * NTH;
        const int row = q / CPR;
        *reinterpret_cast<u32x4*>(&lds[buf][row][G<E>::pos(q % CPR, row) * VEC]) = stage[i];
      }
    };

    load(0);
    store(0);
    if (total > 1) load(1);
    __syncthreads();
    for (int it = 0; it < total; ++it) {
      const int buf = it & 1;
      if (it + 1 < total) {
        store(buf ^ 1);  // buffer buf ^ 1 was released by the barrier ending step it - 1
        if (it + 2 < total) load(it + 2);
      }
      const E* arow = &lds[buf][wm * (BM / WM) + (lane & 15)][0];
      const E* brow = &lds[buf][BM + wn * (BN / WN) + (lane & 15)][0];
#pragma unroll
      for (int ks = 0; ks < BK / KSTEP; ++ks) {
        typename G<E>::R af[TM];
#pragma unroll
        for (int i = 0; i < TM; ++i) af[i] = G<E>::frag(arow + i * 16 * LDR, ks, lane);
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const typename G<E>::R bf = G<E>::frag(brow + j * 16 * LDR, ks, lane);
#pragma unroll
          for (int i = 0; i < TM; ++i) acc[i][j] = G<E>::mma(bf, af[i], acc[i][j]);
        }
      }
      __syncthreads();
    }
  }

  // The products are computed as C^T tiles (B fragments in the MFMA A slot), so each lane
  // holds 4 consecutive columns of one row and stores them as one vector.
  OUT* Cb = a.C + static_cast<int64_t>(bz) * a.sC;
  const bool cvec = (reinterpret_cast<uintptr_t>(Cb) % (4 * sizeof(OUT))) == 0 && a.ldc % 4 == 0;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int m = m0 + wm * (BM / WM) + i * 16 + (lane & 15);
    if (m >= a.M) continue;
    OUT* crow = Cb + static_cast<int64_t>(m) * a.ldc;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + wn * (BN / WN) + j * 16 + (lane >> 4) * 4;
      const f32x4 v = acc[i][j] * a.alpha;
      if (cvec && n + 4 <= a.N) {
        store4<OUT>(crow + n, v);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (n + r < a.N) put<OUT>(crow + n + r, v[r]);
      }
    }
  }
}

// Host-side launcher for one block shape. The vector path needs 16-byte aligned operand
// bases and leading dimensions / batch strides that keep every row 16-byte aligned.
template <typename E, typename OUT, int BM, int BN, int WM, int WN>
inline hipError_t launch_shape(const Args<E, OUT>& a, int batch, hipStream_t stream) {
  constexpr int VEC = G<E>::VEC;
  if (batch <= 0 || a.M <= 0 || a.N <= 0) return hipSuccess;
  auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  bool vec = al(a.A) && al(a.B) && (a.lda % VEC == 0) && (a.ldb % VEC == 0) &&
             (a.sA % VEC == 0) && (a.sB % VEC == 0);
  if (a.A2) vec = vec && al(a.A2) && al(a.B2);
  // Buffer offsets are 32-bit: every row a tile may address must stay below 2^31 bytes.
  if ((static_cast<int64_t>(a.M) + BM) * a.lda * static_cast<int64_t>(sizeof(E)) >= (1ll << 31) ||
      (static_cast<int64_t>(a.N) + BN) * a.ldb * static_cast<int64_t>(sizeof(E)) >= (1ll << 31))
    return hipErrorInvalidValue;
  const int64_t tiles = static_cast<int64_t>(batch) * ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  const int nblk = static_cast<int>((tiles + 7) / 8 * 8);
  constexpr int NTH = Shape<BM, BN, WM, WN>::NTH;
  if (vec)
    hipLaunchKernelGGL((gemm_kernel<E, OUT, BM, BN, WM, WN, true>), dim3(nblk), dim3(NTH), 0,
                       stream, a, batch, nblk);
  else
    hipLaunchKernelGGL((gemm_kernel<E, OUT, BM, BN, WM, WN, false>), dim3(nblk), dim3(NTH), 0,
                       stream, a, batch, nblk);
  return hipGetLastError();
}

// bf16: 256 x 256 blocks of 8 waves (64 x 128 per wave; 147 KB of LDS, one block per CU).
// fp32: 128 x 128 blocks of 4 waves.
template <typename E, typename OUT>
inline hipError_t launch(const Args<E, OUT>& a, int batch, hipStream_t stream) {
  if constexpr (is_bf16<E>::value) {
    return launch_shape<E, OUT, 256, 256, 4, 2>(a, batch, stream);
  } else {
    return launch_shape<E, OUT, 128, 128, 2, 2>(a, batch, stream);
  }
}

}  // namespace gemm
}  // namespace dabsn
