// Thin wrappers over the gfx950 MFMA instructions used by the DSQG kernels.
//
// Lane layouts (wave64, lane l; verified on gfx950):
//   v_mfma_f32_16x16x4_f32    A[i = l%16][k = l/16]          (1 fp32 per lane)
//                             B[k = l/16][j = l%16]
//   v_mfma_f32_16x16x16_bf16  A[i = l%16][k = 4*(l/16) + e]  (4 bf16 per lane, e = 0..3)
//                             B[k = 4*(l/16) + e][j = l%16]
//   v_mfma_f32_16x16x32_bf16  A[i = l%16][k = 8*(l/16) + e]  (8 bf16 per lane, e = 0..7)
//                             B[k = 8*(l/16) + e][j = l%16]
//   all                       C[i = 4*(l/16) + r][j = l%16]  (4 fp32 per lane, r = 0..3)
//
// ds_read_b64_tr_b16 (gfx950), per group of 16 lanes: lane j supplies the
// address of 4 consecutive 16-bit elements chunk[j][0..3]; lane i receives
// element e = chunk[4e + i/4][i%4].  With lane j pointing at row r0 + j/4,
// column c0 + 4*(j%4) of a row-major matrix X, lane i receives
// X[r0 + e][c0 + i] for e = 0..3: a 4 x 16 tile transposed, which is the
// B operand of the 16x16x16 MFMA (rows = k, column = j).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dwarf {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mfma16_f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma16_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma16k16_bf16(i16x4 a, i16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

// Transposing LDS read (see the layout note above); p is a generic pointer into LDS.
__device__ __forceinline__ i16x4 lds_read_tr16(const void* p) {
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(const_cast<void*>(p)));
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
