// Shared device helpers for the DABSN gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace dabsn {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Storage types: fp32 tapes are `float`, bf16 tapes are raw `uint16_t` bits.
using bf16 = uint16_t;

enum DType : int { kF32 = 0, kBF16 = 1 };

__device__ __forceinline__ float bf2f(bf16 h) {
  return __builtin_bit_cast(float, static_cast<uint32_t>(h) << 16);
}

// Round-to-nearest-even fp32 -> bf16 (matches torch's .to(torch.bfloat16)); one
// v_cvt_pk_bf16_f32 on gfx950.
__device__ __forceinline__ bf16 f2bf(float f) { return __builtin_bit_cast(bf16, static_cast<__bf16>(f)); }

template <typename E>
struct is_bf16 { static constexpr bool value = false; };
template <>
struct is_bf16<bf16> { static constexpr bool value = true; };

template <typename E>
__device__ __forceinline__ float ld(const E* p, size_t i);
template <>
__device__ __forceinline__ float ld<float>(const float* p, size_t i) { return p[i]; }
template <>
__device__ __forceinline__ float ld<bf16>(const bf16* p, size_t i) { return bf2f(p[i]); }

__device__ __forceinline__ float to_f(float v) { return v; }
__device__ __forceinline__ float to_f(bf16 v) { return bf2f(v); }
// The element of type E that st() stores for v.
template <typename E>
__device__ __forceinline__ E from_f(float v);
template <>
__device__ __forceinline__ float from_f<float>(float v) { return v; }
template <>
__device__ __forceinline__ bf16 from_f<bf16>(float v) { return f2bf(v); }

template <typename E>
__device__ __forceinline__ void st(E* p, size_t i, float v);
template <>
__device__ __forceinline__ void st<float>(float* p, size_t i, float v) { p[i] = v; }
template <>
__device__ __forceinline__ void st<bf16>(bf16* p, size_t i, float v) { p[i] = f2bf(v); }

// 16-byte global load / store through an explicit global-address-space pointer. Pointers
// picked at run time from a table of tensors lose their address space in the compiler and
// would become FLAT accesses, which also count against the LDS wait counter.
__device__ __forceinline__ u32x4 gload16(const void* p) {
  return *(const __attribute__((address_space(1))) u32x4*)p;  // address-space cast
}
__device__ __forceinline__ void gstore16(void* p, u32x4 v) {
  *(__attribute__((address_space(1))) u32x4*)p = v;  // address-space cast
}

// V consecutive elements at p as floats (V = 1, or 8: one 16-byte access for bf16, two for
// fp32; p must then be 16-byte aligned).
template <typename E, int V>
__device__ __forceinline__ void ldv(const E* p, float (&v)[V]) {
  if constexpr (V == 1) {
    v[0] = ld(p, 0);
  } else if constexpr (is_bf16<E>::value) {
    static_assert(V == 8, "bf16 vectors are 8 wide");
    const u32x4 u = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[2 * k] = __builtin_bit_cast(float, u[k] << 16);
      v[2 * k + 1] = __builtin_bit_cast(float, u[k] & 0xffff0000u);
    }
  } else {
    static_assert(V == 8, "fp32 vectors are 8 wide");
    const f32x4 a = *reinterpret_cast<const f32x4*>(p), b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[k] = a[k];
      v[4 + k] = b[k];
    }
  }
}
template <typename E, int V>
__device__ __forceinline__ void stv(E* p, const float (&v)[V]) {
  if constexpr (V == 1) {
    st(p, 0, v[0]);
  } else if constexpr (is_bf16<E>::value) {
    static_assert(V == 8, "bf16 vectors are 8 wide");
    u32x4 u;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      u[k] = static_cast<uint32_t>(f2bf(v[2 * k])) | (static_cast<uint32_t>(f2bf(v[2 * k + 1])) << 16);
    *reinterpret_cast<u32x4*>(p) = u;
  } else {
    static_assert(V == 8, "fp32 vectors are 8 wide");
    *reinterpret_cast<f32x4*>(p) = (f32x4){v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4*>(p + 4) = (f32x4){v[4], v[5], v[6], v[7]};
  }
}

// Value as it would be stored in E (identity for fp32, RTNE round trip for bf16).
template <typename E>
__device__ __forceinline__ float round_to(float v);
template <>
__device__ __forceinline__ float round_to<float>(float v) { return v; }
template <>
__device__ __forceinline__ float round_to<bf16>(float v) { return bf2f(f2bf(v)); }


// Buffer resource over [base, base + bytes); out-of-range accesses are dropped (stores)
// or return zero (loads). Third dword per the gfx9 buffer descriptor format.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                           static_cast<int>(bytes), 0x00020000);
}

// Cache-policy bit for device-coherent (cross-XCD) vector memory accesses.
constexpr int kCoherent = 16;  // sc1

// Wave-wide reductions over 64 lanes on DPP: butterflies inside quads and rows of 16
// lanes (quad_perm, row_half_mirror, row_mirror), then row_bcast15 / row_bcast31 fold
// the four rows into lane 63, whose value every lane receives through v_readlane.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_mov(float x, float old) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old),
                                                               __builtin_bit_cast(int, x), CTRL,
                                                               ROW_MASK, 0xF, false));
}
// Lane i receives lane i + N of its 16-lane row (DPP row_shl); lanes past the row's end
// keep their own value. A VALU move: no LDS round trip, unlike ds_bpermute.
template <int N>
__device__ __forceinline__ int row_shl(int x) {
  return __builtin_amdgcn_update_dpp(x, x, 0x100 + N, 0xF, 0xF, false);
}
template <typename Op>
__device__ __forceinline__ float wave_reduce(float v, float identity, Op op) {
  v = op(v, dpp_mov<0xB1, 0xF>(v, identity));   // quad_perm [1,0,3,2]
  v = op(v, dpp_mov<0x4E, 0xF>(v, identity));   // quad_perm [2,3,0,1]
  v = op(v, dpp_mov<0x141, 0xF>(v, identity));  // row_half_mirror
  v = op(v, dpp_mov<0x140, 0xF>(v, identity));  // row_mirror
  v = op(v, dpp_mov<0x142, 0xA>(v, identity));  // row_bcast15 into rows 1, 3
  v = op(v, dpp_mov<0x143, 0xC>(v, identity));  // row_bcast31 into rows 2, 3
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
__device__ __forceinline__ float wave_sum(float v) {
  return wave_reduce(v, 0.0f, [](float a, float b) { return a + b; });
}
__device__ __forceinline__ float wave_max(float v) {
  return wave_reduce(v, -INFINITY, [](float a, float b) { return fmaxf(a, b); });
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float softplusf_(float x) {
  return fmaxf(x, 0.0f) + log1pf(expf(-fabsf(x)));
}
__device__ __forceinline__ float hardsigmoidf_(float x) {
  return fminf(fmaxf(x + 3.0f, 0.0f), 6.0f) * (1.0f / 6.0f);
}
__device__ __forceinline__ float clamp01(float x) { return fminf(fmaxf(x, 0.0f), 1.0f); }
__device__ __forceinline__ float signf_(float x) {
  return static_cast<float>((x > 0.0f) - (x < 0.0f));
}

// Spin bound for device-wide step barriers: any wait longer than this (seconds of
// polling) sets the error flag and the kernel exits instead of hanging.
constexpr uint32_t kSpinLimit = 1u << 22;

// Error bits reported through the workspace error word.
constexpr uint32_t kErrBarrierTimeout = 1u;

}  // namespace dabsn
