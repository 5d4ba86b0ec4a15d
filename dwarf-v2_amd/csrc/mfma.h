// Thin wrappers over the gfx950 MFMA instructions used by the DSQG kernels.
//
// Lane layouts (wave64, lane l; verified on gfx950):
//   v_mfma_f32_16x16x4_f32    A[i = l%16][k = l/16]          (1 fp32 per lane)
//                             B[k = l/16][j = l%16]
//   v_mfma_f32_16x16x32_bf16  A[i = l%16][k = 8*(l/16) + e]  (8 bf16 per lane, e = 0..7)
//                             B[k = 8*(l/16) + e][j = l%16]
//   both                      C[i = 4*(l/16) + r][j = l%16]  (4 fp32 per lane, r = 0..3)
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dwarf {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x4 mfma16_f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma16_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// Eight fp32 values split into bf16 high and low parts: x ~= hi + lo with
// about 16 significant bits, so an MFMA pair (hi, lo) reproduces fp32
// products to ~2^-17 relative.
__device__ __forceinline__ void split_bf16x8(const float* x, bf16x8& hi, bf16x8& lo) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const __bf16 h = static_cast<__bf16>(x[e]);
    hi[e] = h;
    lo[e] = static_cast<__bf16>(x[e] - static_cast<float>(h));
  }
}

__device__ __forceinline__ bf16x8 bf16x8_from_bits(uint4 w) { return __builtin_bit_cast(bf16x8, w); }

__device__ __forceinline__ bf16x8 bf16x8_zero() { return __builtin_bit_cast(bf16x8, uint4{0u, 0u, 0u, 0u}); }

}  // namespace dwarf
