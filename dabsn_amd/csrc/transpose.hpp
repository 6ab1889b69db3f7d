// Batched 2-D transpose through LDS: out[b][c][r] = in[b][r][c] for [batch][R][C] inputs.
//
// Used to hand the GEMMs K-contiguous copies of operands whose natural layout is
// M- or N-contiguous (their MFMA fragments need 8 consecutive k per lane). A 64x64 tile
// is read with 16-byte row vectors, staged in LDS with a padded pitch, and written back
// as 16-byte vectors of the transposed rows; edge tiles fall back to element accesses.
#pragma once

#include "common.hpp"

namespace dabsn {
namespace xpose {

constexpr int TT = 64;    // tile edge
constexpr int TNT = 256;  // threads per tile

template <typename E>
__global__ void __launch_bounds__(TNT) transpose_kernel(int R, int C, const E* __restrict__ in,
                                                        E* __restrict__ out, bool aligned) {
  constexpr int VEC = 16 / static_cast<int>(sizeof(E));  // elements per 16-byte vector
  constexpr int PITCH = TT + 2;
  __shared__ E tile[TT][PITCH];
  const int b = blockIdx.z;
  const int r0 = blockIdx.y * TT, c0 = blockIdx.x * TT;
  const E* src = in + static_cast<size_t>(b) * R * C;
  E* dst = out + static_cast<size_t>(b) * R * C;
  const bool full =
      aligned && r0 + TT <= R && c0 + TT <= C && (C % VEC) == 0 && (R % VEC) == 0;
  constexpr int VPR = TT / VEC;  // vectors per tile row
  if (full) {
    for (int q = threadIdx.x; q < TT * VPR; q += TNT) {
      const int r = q / VPR, cv = (q % VPR) * VEC;
      const u32x4 v = *reinterpret_cast<const u32x4*>(src + static_cast<size_t>(r0 + r) * C + c0 + cv);
      E e[VEC];
      *reinterpret_cast<u32x4*>(e) = v;
#pragma unroll
      for (int k = 0; k < VEC; ++k) tile[r][cv + k] = e[k];
    }
  } else {
    for (int q = threadIdx.x; q < TT * TT; q += TNT) {
      const int r = q / TT, c = q % TT;
      if (r0 + r < R && c0 + c < C) tile[r][c] = src[static_cast<size_t>(r0 + r) * C + c0 + c];
    }
  }
  __syncthreads();
  if (full) {
    for (int q = threadIdx.x; q < TT * VPR; q += TNT) {
      const int c = q / VPR, rv = (q % VPR) * VEC;
      E e[VEC];
#pragma unroll
      for (int k = 0; k < VEC; ++k) e[k] = tile[rv + k][c];
      *reinterpret_cast<u32x4*>(dst + static_cast<size_t>(c0 + c) * R + r0 + rv) =
          *reinterpret_cast<const u32x4*>(e);
    }
  } else {
    for (int q = threadIdx.x; q < TT * TT; q += TNT) {
      const int c = q / TT, r = q % TT;
      if (r0 + r < R && c0 + c < C) dst[static_cast<size_t>(c0 + c) * R + r0 + r] = tile[r][c];
    }
  }
}

// The vector path needs 16-byte aligned bases (and row lengths that keep rows aligned).
template <typename E>
inline hipError_t transpose(const E* in, E* out, int batch, int R, int C, hipStream_t stream) {
  if (batch <= 0 || R <= 0 || C <= 0) return hipSuccess;
  const bool aligned = ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) & 15u) == 0;
  const dim3 grid((C + TT - 1) / TT, (R + TT - 1) / TT, batch);
  hipLaunchKernelGGL(transpose_kernel<E>, grid, dim3(TNT), 0, stream, R, C, in, out, aligned);
  return hipGetLastError();
}

}  // namespace xpose
}  // namespace dabsn
