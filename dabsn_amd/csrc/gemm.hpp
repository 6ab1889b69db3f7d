// Batched MFMA GEMM with per-tile work ranges, used by the three-way read.
//
//   C[b](m, n) = alpha * sum_k A[b](m, k) B[b](k, n)  (+ A2[b](m, k) B2[b](k, n))
//                (+ beta * Cin[b](m, n))
//
// A(m, k) is A[m*lda + k] (K-contiguous) or, with TA, A[k*lda + m]; B(k, n) is
// B[k*ldb + n] or, with TB, B[n*ldb + k]. Causal structure is expressed per
// (batch, 128-row tile) as a k-range [klo, khi) and a column limit nhi: tiles beyond
// nhi are skipped, and only k-tiles that intersect [klo, khi) are visited (the operands
// are zero outside that range by construction of the callers).
//
// Tile 128x128, 256 threads = 4 waves in a 2x2 arrangement, each wave 64x64 as 4x4
// MFMA 16x16 tiles. Operands are staged through LDS K-contiguous; M/N-contiguous
// sources are transposed while being written to LDS.
#pragma once

#include "common.hpp"

namespace dabsn {
namespace gemm {

constexpr int BM = 128, BN = 128, NTH = 256;

template <typename E>
struct G;
template <>
struct G<bf16> {
  static constexpr int BK = 32, PAD = 8, VEC = 8, KSUB = 1;
};
template <>
struct G<float> {
  static constexpr int BK = 16, PAD = 4, VEC = 4, KSUB = 4;
};

template <typename E, typename OUT>
struct Args {
  int M, N, K;
  const E* A;
  int64_t lda, sA;
  const E* B;
  int64_t ldb, sB;
  const E* A2;  // optional second product (same layout/strides as A, B)
  const E* B2;
  OUT* C;
  int64_t ldc, sC;
  const float* Cin;  // optional accumulate input (fp32), same ld/stride as C
  float alpha, beta;
  const int32_t* ranges;  // optional [batch][mtiles][3] = (klo, khi, nhi)
  int mtiles;
};

template <typename E>
__device__ __forceinline__ E zero_e() { return static_cast<E>(0); }

// Loads one BK-wide slab of rows [r0, r0+128) of a K-contiguous (kc=true) or
// row-contiguous (kc=false) operand into registers; vector path when `vec`.
template <typename E, bool KC, bool VECOK>
struct Stage {
  static constexpr int BK = G<E>::BK, VEC = G<E>::VEC;
  static constexpr int NV = (128 * BK) / (VEC * NTH);  // vectors per thread (=2)
  E v[NV][VEC];

  __device__ void load(const E* src, int64_t ld, int r0, int rlim, int k0, int klo, int khi) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int q = tid + i * NTH;
      if constexpr (KC) {
        // q -> (row, k-chunk)
        const int row = q / (BK / VEC), kc = (q % (BK / VEC)) * VEC;
        const int r = r0 + row, k = k0 + kc;
        if constexpr (VECOK) {
          if (r < rlim && k >= klo && k + VEC <= khi) {
            const E* p = src + static_cast<int64_t>(r) * ld + k;
            const u32x4 x = *reinterpret_cast<const u32x4*>(p);
            *reinterpret_cast<u32x4*>(v[i]) = x;
          } else {
            // Outside the k-range the operand is defined as zero (it may be unwritten).
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
              const int kk = k + e;
              v[i][e] = (r < rlim && kk >= klo && kk < khi)
                            ? src[static_cast<int64_t>(r) * ld + kk]
                            : zero_e<E>();
            }
          }
        } else {
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            const int kk = k + e;
            v[i][e] = (r < rlim && kk >= klo && kk < khi) ? src[static_cast<int64_t>(r) * ld + kk]
                                                           : zero_e<E>();
          }
        }
      } else {
        // q -> (k-row, row-chunk); element (r, k) at src[k*ld + r]
        const int kr = q / (128 / VEC), rc = (q % (128 / VEC)) * VEC;
        const int k = k0 + kr, r = r0 + rc;
        const bool kok = k >= klo && k < khi;
        if constexpr (VECOK) {
          if (kok && r + VEC <= rlim) {
            const E* p = src + static_cast<int64_t>(k) * ld + r;
            const u32x4 x = *reinterpret_cast<const u32x4*>(p);
            *reinterpret_cast<u32x4*>(v[i]) = x;
          } else {
#pragma unroll
            for (int e = 0; e < VEC; ++e)
              v[i][e] = (kok && r + e < rlim) ? src[static_cast<int64_t>(k) * ld + r + e] : zero_e<E>();
          }
        } else {
#pragma unroll
          for (int e = 0; e < VEC; ++e)
            v[i][e] = (kok && r + e < rlim) ? src[static_cast<int64_t>(k) * ld + r + e] : zero_e<E>();
        }
      }
    }
  }

  __device__ void store(E (*lds)[G<E>::BK + G<E>::PAD]) const {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int q = tid + i * NTH;
      if constexpr (KC) {
        const int row = q / (BK / VEC), kc = (q % (BK / VEC)) * VEC;
#pragma unroll
        for (int e = 0; e < VEC; ++e) lds[row][kc + e] = v[i][e];
      } else {
        const int kr = q / (128 / VEC), rc = (q % (128 / VEC)) * VEC;
#pragma unroll
        for (int e = 0; e < VEC; ++e) lds[rc + e][kr] = v[i][e];
      }
    }
  }
};

template <typename E>
struct Frag;
template <>
struct Frag<bf16> {
  using R = bf16x8;
  __device__ static R load(const bf16 (*lds)[G<bf16>::BK + G<bf16>::PAD], int row, int ks, int lane) {
    (void)ks;
    const bf16* p = &lds[row][(lane >> 4) * 8];
    return __builtin_bit_cast(R, *reinterpret_cast<const u32x4*>(p));
  }
  __device__ static f32x4 mma(R a, R b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Frag<float> {
  using R = float;
  __device__ static R load(const float (*lds)[G<float>::BK + G<float>::PAD], int row, int ks, int lane) {
    return lds[row][ks * 4 + (lane >> 4)];
  }
  __device__ static f32x4 mma(R a, R b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
};

template <typename OUT>
__device__ __forceinline__ void put(OUT* p, float v);
template <>
__device__ __forceinline__ void put<float>(float* p, float v) { *p = v; }
template <>
__device__ __forceinline__ void put<bf16>(bf16* p, float v) { *p = f2bf(v); }

template <typename E, typename OUT, bool TA, bool TB, bool VECOK>
__global__ void __launch_bounds__(NTH) gemm_kernel(Args<E, OUT> a) {
  constexpr int BK = G<E>::BK, PAD = G<E>::PAD, KSUB = G<E>::KSUB;
  __shared__ __attribute__((aligned(16))) E As[BM][BK + PAD];
  __shared__ __attribute__((aligned(16))) E Bs[BN][BK + PAD];

  const int nt = blockIdx.x, mt = blockIdx.y, bz = blockIdx.z;
  const int m0 = mt * BM, n0 = nt * BN;
  int klo = 0, khi = a.K, nhi = a.N;
  if (a.ranges) {
    const int32_t* r = a.ranges + (static_cast<int64_t>(bz) * a.mtiles + mt) * 3;
    klo = max(0, r[0]);
    khi = min(a.K, r[1]);
    nhi = min(a.N, r[2]);
  }
  if (n0 >= nhi) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

  const int nprod = a.A2 ? 2 : 1;
  if (khi > klo) {
    const int kt0 = klo / BK, kt1 = (khi + BK - 1) / BK;
    for (int pr = 0; pr < nprod; ++pr) {
      const E* Ab = (pr == 0 ? a.A : a.A2) + static_cast<int64_t>(bz) * a.sA;
      const E* Bb = (pr == 0 ? a.B : a.B2) + static_cast<int64_t>(bz) * a.sB;
      Stage<E, !TA, VECOK> sa;
      Stage<E, TB, VECOK> sb;
      sa.load(Ab, a.lda, m0, a.M, kt0 * BK, klo, khi);
      sb.load(Bb, a.ldb, n0, a.N, kt0 * BK, klo, khi);
      for (int kt = kt0; kt < kt1; ++kt) {
        __syncthreads();
        sa.store(As);
        sb.store(Bs);
        __syncthreads();
        if (kt + 1 < kt1) {
          sa.load(Ab, a.lda, m0, a.M, (kt + 1) * BK, klo, khi);
          sb.load(Bb, a.ldb, n0, a.N, (kt + 1) * BK, klo, khi);
        }
#pragma unroll
        for (int ks = 0; ks < KSUB; ++ks) {
          typename Frag<E>::R af[4], bfr[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) af[i] = Frag<E>::load(As, wm * 64 + i * 16 + (lane & 15), ks, lane);
#pragma unroll
          for (int j = 0; j < 4; ++j) bfr[j] = Frag<E>::load(Bs, wn * 64 + j * 16 + (lane & 15), ks, lane);
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = Frag<E>::mma(af[i], bfr[j], acc[i][j]);
        }
      }
    }
  }

  OUT* Cb = a.C + static_cast<int64_t>(bz) * a.sC;
  const float* Ci = a.Cin ? a.Cin + static_cast<int64_t>(bz) * a.sC : nullptr;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + wn * 64 + j * 16 + (lane & 15);
      if (n >= a.N) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * 64 + i * 16 + (lane >> 4) * 4 + r;
        if (m >= a.M) continue;
        const int64_t o = static_cast<int64_t>(m) * a.ldc + n;
        float v = a.alpha * acc[i][j][r];
        if (Ci) v += a.beta * Ci[o];
        put<OUT>(Cb + o, v);
      }
    }
  }
}

// Host-side launcher. Chooses the vector path when every operand is 16-byte aligned
// and the contiguous extents are multiples of the vector width.
template <typename E, typename OUT, bool TA, bool TB>
inline hipError_t launch(const Args<E, OUT>& a, int batch, hipStream_t stream) {
  constexpr int VEC = G<E>::VEC;
  auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  bool vec = al(a.A) && al(a.B) && (a.lda % VEC == 0) && (a.ldb % VEC == 0) &&
             (a.sA % VEC == 0) && (a.sB % VEC == 0);
  if (a.A2) vec = vec && al(a.A2) && al(a.B2);
  // Contiguous extents must be multiples of VEC so vectors never straddle a boundary.
  vec = vec && (TA ? (a.M % VEC == 0) : (a.K % VEC == 0)) && (TB ? (a.K % VEC == 0) : (a.N % VEC == 0));
  const dim3 grid((a.N + BN - 1) / BN, (a.M + BM - 1) / BM, batch);
  if (vec)
    hipLaunchKernelGGL((gemm_kernel<E, OUT, TA, TB, true>), grid, dim3(NTH), 0, stream, a);
  else
    hipLaunchKernelGGL((gemm_kernel<E, OUT, TA, TB, false>), grid, dim3(NTH), 0, stream, a);
  return hipGetLastError();
}

}  // namespace gemm
}  // namespace dabsn
