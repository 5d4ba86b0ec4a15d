// Device helpers shared by the DSQG, EMA and q6 kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dwarf_dsqg.h"

namespace dwarf {

constexpr int kWave = 64;
constexpr int kPlanes = DWARF_R_PLANES;

// ---------------------------------------------------------------------------
// bf16 <-> fp32.  bf16 is carried as raw 16-bit storage; widening is exact.
// ---------------------------------------------------------------------------
struct bf16 {
  uint16_t bits;
};

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Round-to-nearest-even fp32 -> bf16 (the hardware conversion on gfx950).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  __bf16 h = static_cast<__bf16>(f);
  return __builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ float round_bf16(float f) {
  return __uint_as_float(static_cast<uint32_t>(f32_to_bf16_bits(f)) << 16);
}
// Two values in one v_cvt_pk_bf16_f32 (round to nearest even), lo in bits 0-15.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2v));
}

// ---------------------------------------------------------------------------
// Row chunks: CNT consecutive elements (CNT a multiple of 8) loaded with
// 16-byte vector loads and widened to fp32, or narrowed and stored.
// ---------------------------------------------------------------------------
template <typename T, int CNT>
__device__ __forceinline__ void load_f32(const T* __restrict__ p, float* __restrict__ dst);

template <int CNT>
__device__ __forceinline__ void load_f32_bf16(const uint16_t* __restrict__ p, float* __restrict__ dst) {
  static_assert(CNT % 8 == 0, "chunk must be whole 16-byte vectors");
  const uint4* v = reinterpret_cast<const uint4*>(p);
#pragma unroll
  for (int i = 0; i < CNT / 8; ++i) {
    const uint4 w = v[i];
    dst[8 * i + 0] = bf16_lo(w.x); dst[8 * i + 1] = bf16_hi(w.x);
    dst[8 * i + 2] = bf16_lo(w.y); dst[8 * i + 3] = bf16_hi(w.y);
    dst[8 * i + 4] = bf16_lo(w.z); dst[8 * i + 5] = bf16_hi(w.z);
    dst[8 * i + 6] = bf16_lo(w.w); dst[8 * i + 7] = bf16_hi(w.w);
  }
}

template <>
__device__ __forceinline__ void load_f32<bf16, 64>(const bf16* p, float* dst) {
  load_f32_bf16<64>(reinterpret_cast<const uint16_t*>(p), dst);
}
template <>
__device__ __forceinline__ void load_f32<bf16, 32>(const bf16* p, float* dst) {
  load_f32_bf16<32>(reinterpret_cast<const uint16_t*>(p), dst);
}
template <>
__device__ __forceinline__ void load_f32<bf16, 16>(const bf16* p, float* dst) {
  load_f32_bf16<16>(reinterpret_cast<const uint16_t*>(p), dst);
}
template <>
__device__ __forceinline__ void load_f32<bf16, 8>(const bf16* p, float* dst) {
  load_f32_bf16<8>(reinterpret_cast<const uint16_t*>(p), dst);
}

template <int CNT>
__device__ __forceinline__ void load_f32_f32(const float* __restrict__ p, float* __restrict__ dst) {
  static_assert(CNT % 4 == 0, "chunk must be whole 16-byte vectors");
  const float4* v = reinterpret_cast<const float4*>(p);
#pragma unroll
  for (int i = 0; i < CNT / 4; ++i) {
    const float4 w = v[i];
    dst[4 * i + 0] = w.x; dst[4 * i + 1] = w.y; dst[4 * i + 2] = w.z; dst[4 * i + 3] = w.w;
  }
}
template <>
__device__ __forceinline__ void load_f32<float, 64>(const float* p, float* dst) { load_f32_f32<64>(p, dst); }
template <>
__device__ __forceinline__ void load_f32<float, 32>(const float* p, float* dst) { load_f32_f32<32>(p, dst); }
template <>
__device__ __forceinline__ void load_f32<float, 16>(const float* p, float* dst) { load_f32_f32<16>(p, dst); }
template <>
__device__ __forceinline__ void load_f32<float, 8>(const float* p, float* dst) { load_f32_f32<8>(p, dst); }

// 16 consecutive values as raw 16-byte vectors, so that a later step's row
// can be requested before the current one is used (software prefetch).
template <typename T>
struct RawSlice16 {
  uint4 w[16 * sizeof(T) / 16];
};

template <typename T>
__device__ __forceinline__ void load_raw(const T* p, RawSlice16<T>& r) {
  const uint4* v = reinterpret_cast<const uint4*>(p);
#pragma unroll
  for (int i = 0; i < 16 * static_cast<int>(sizeof(T)) / 16; ++i) r.w[i] = v[i];
}

__device__ __forceinline__ void widen(const RawSlice16<bf16>& r, float* x) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    x[8 * i + 0] = bf16_lo(r.w[i].x); x[8 * i + 1] = bf16_hi(r.w[i].x);
    x[8 * i + 2] = bf16_lo(r.w[i].y); x[8 * i + 3] = bf16_hi(r.w[i].y);
    x[8 * i + 4] = bf16_lo(r.w[i].z); x[8 * i + 5] = bf16_hi(r.w[i].z);
    x[8 * i + 6] = bf16_lo(r.w[i].w); x[8 * i + 7] = bf16_hi(r.w[i].w);
  }
}
__device__ __forceinline__ void widen(const RawSlice16<float>& r, float* x) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[4 * i + 0] = __uint_as_float(r.w[i].x); x[4 * i + 1] = __uint_as_float(r.w[i].y);
    x[4 * i + 2] = __uint_as_float(r.w[i].z); x[4 * i + 3] = __uint_as_float(r.w[i].w);
  }
}

template <typename T, int CNT>
__device__ __forceinline__ void store_from_f32(T* __restrict__ p, const float* __restrict__ src);

template <int CNT>
__device__ __forceinline__ void store_bf16(uint16_t* __restrict__ p, const float* __restrict__ src) {
  uint4* v = reinterpret_cast<uint4*>(p);
#pragma unroll
  for (int i = 0; i < CNT / 8; ++i) {
    uint4 w;
    w.x = pack_bf16x2(src[8 * i + 0], src[8 * i + 1]);
    w.y = pack_bf16x2(src[8 * i + 2], src[8 * i + 3]);
    w.z = pack_bf16x2(src[8 * i + 4], src[8 * i + 5]);
    w.w = pack_bf16x2(src[8 * i + 6], src[8 * i + 7]);
    v[i] = w;
  }
}
template <>
__device__ __forceinline__ void store_from_f32<bf16, 64>(bf16* p, const float* src) {
  store_bf16<64>(reinterpret_cast<uint16_t*>(p), src);
}
template <>
__device__ __forceinline__ void store_from_f32<bf16, 32>(bf16* p, const float* src) {
  store_bf16<32>(reinterpret_cast<uint16_t*>(p), src);
}

template <int CNT>
__device__ __forceinline__ void store_f32(float* __restrict__ p, const float* __restrict__ src) {
  float4* v = reinterpret_cast<float4*>(p);
#pragma unroll
  for (int i = 0; i < CNT / 4; ++i) v[i] = make_float4(src[4 * i], src[4 * i + 1], src[4 * i + 2], src[4 * i + 3]);
}
template <>
__device__ __forceinline__ void store_from_f32<float, 64>(float* p, const float* src) { store_f32<64>(p, src); }
template <>
__device__ __forceinline__ void store_from_f32<float, 32>(float* p, const float* src) { store_f32<32>(p, src); }

// ---------------------------------------------------------------------------
// Math.  FAST selects the hardware transcendental instructions (bf16 paths,
// where results are rounded to bf16 anyway); otherwise the correctly
// range-reduced device-library routines are called (fp32 parity paths).
// ---------------------------------------------------------------------------
template <bool FAST>
__device__ __forceinline__ float dexp(float x) {
  if constexpr (FAST) return __expf(x);
  else return expf(x);
}
template <bool FAST>
__device__ __forceinline__ float dlog(float x) {
  if constexpr (FAST) return __logf(x);
  else return logf(x);
}
template <bool FAST>
__device__ __forceinline__ void dsincos(float x, float* s, float* c) {
  if constexpr (FAST) {
    *s = __sinf(x);
    *c = __cosf(x);
  } else {
    sincosf(x, s, c);
  }
}

// ---------------------------------------------------------------------------
// Wave64 reductions on DPP.  wave_sum_to_last leaves the full sum in lane 63.
// ---------------------------------------------------------------------------
template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf, bool BOUND_CTRL = true>
__device__ __forceinline__ float dpp_f(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, ROW_MASK, BANK_MASK, BOUND_CTRL));
}

__device__ __forceinline__ float wave_sum_to_last(float x) {
  x += dpp_f<0x111>(x);  // row_shr:1
  x += dpp_f<0x112>(x);  // row_shr:2
  x += dpp_f<0x114>(x);  // row_shr:4  (lanes 4..15 of each row now hold 4..8-lane sums)
  x += dpp_f<0x118>(x);  // row_shr:8  (lane 15 of each row holds the row sum)
  x += dpp_f<0x142, 0xa>(x);  // row_bcast:15 into rows 1 and 3
  x += dpp_f<0x143, 0xc>(x);  // row_bcast:31 into rows 2 and 3
  return x;                   // lane 63 holds the wave sum
}

// Sum across groups of L adjacent lanes (L = 1, 2 or 4); every lane of the
// group receives the total.
template <int L>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (L >= 2) x += dpp_f<0xB1>(x);  // quad_perm [1,0,3,2]
  if constexpr (L >= 4) x += dpp_f<0x4E>(x);  // quad_perm [2,3,0,1]
  return x;
}

__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

}  // namespace dwarf
