// Pieces shared by the causal EMA scan (ema.hip) and the InterferencePacket
// pool (packet.hip): element loads and stores, the chunk geometry, the carry
// stage that joins the chunks and the fixed-order dalpha reductions.  The
// kernels are in an unnamed namespace: each translation unit that launches
// them holds its own copy.
#pragma once

#include "common.h"
#include "gather.h"

namespace dwarf {

constexpr int kChunkT = 16;
constexpr int kEmaBlock = 256;

namespace {


template <typename T>
__device__ __forceinline__ float ld1(const T* p);
template <>
__device__ __forceinline__ float ld1<bf16>(const bf16* p) {
  return __uint_as_float(static_cast<uint32_t>(reinterpret_cast<const uint16_t*>(p)[0]) << 16);
}
template <>
__device__ __forceinline__ float ld1<float>(const float* p) { return *p; }

template <typename T>
__device__ __forceinline__ void st1(T* p, float v);
template <>
__device__ __forceinline__ void st1<bf16>(bf16* p, float v) { reinterpret_cast<uint16_t*>(p)[0] = f32_to_bf16_bits(v); }
template <>
__device__ __forceinline__ void st1<float>(float* p, float v) { *p = v; }

// VEC adjacent channels.
template <typename T, int VEC>
__device__ __forceinline__ void ldv(const T* p, float* v) {
  if constexpr (VEC == 4 && sizeof(T) == 2) {
    const uint2 w = *reinterpret_cast<const uint2*>(p);
    v[0] = bf16_lo(w.x); v[1] = bf16_hi(w.x); v[2] = bf16_lo(w.y); v[3] = bf16_hi(w.y);
  } else if constexpr (VEC == 4 && sizeof(T) == 4) {
    const float4 w = *reinterpret_cast<const float4*>(p);
    v[0] = w.x; v[1] = w.y; v[2] = w.z; v[3] = w.w;
  } else if constexpr (VEC == 2 && sizeof(T) == 2) {
    const uint32_t w = *reinterpret_cast<const uint32_t*>(p);
    v[0] = bf16_lo(w); v[1] = bf16_hi(w);
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) v[i] = ld1<T>(p + i);
  }
}
template <typename T, int VEC>
__device__ __forceinline__ void stv(T* p, const float* v) {
  if constexpr (VEC == 4 && sizeof(T) == 2) {
    uint2 w;
    w.x = pack_bf16x2(v[0], v[1]);
    w.y = pack_bf16x2(v[2], v[3]);
    *reinterpret_cast<uint2*>(p) = w;
  } else if constexpr (VEC == 4 && sizeof(T) == 4) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  } else if constexpr (VEC == 2 && sizeof(T) == 2) {
    *reinterpret_cast<uint32_t*>(p) = pack_bf16x2(v[0], v[1]);
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) st1<T>(p + i, v[i]);
  }
}

struct EmaGeom {
  int B, N, D, NC, DV;  // DV = D / VEC lanes per row
  int per_channel;
  int alpha_div;          // channels per factor when per_channel (see clamp_alpha)
  float lo, hi;
  const uint8_t* reset;   // [B,N] reset flags (RESET kernels only)
  int64_t srb, srn;
  uint8_t* cut;           // [B][NC]: the chunk cuts the carry (a reset inside, see ema_carry)
};

// The state is zeroed before a token whose reset flag is set (ema:533-535).
__device__ __forceinline__ bool reset_at(const EmaGeom& g, int b, int t) {
  return g.reset[b * g.srb + static_cast<int64_t>(t) * g.srn] != 0;
}

// The clamped factor of channel d: one factor for all channels, or one per
// run of alpha_div channels (1: per channel; D: one per scale of the packet
// pool, whose channels are scale-major).
__device__ __forceinline__ float clamp_alpha(const float* alpha, const EmaGeom& g, int d) {
  const float a = alpha[g.per_channel ? d / g.alpha_div : 0];
  return fminf(fmaxf(a, g.lo), g.hi);
}

// Rows of one chunk are loaded in blocks of kRows<T> (all loads of a block
// are issued before the recurrence consumes them), so a lane keeps a block of
// rows in flight instead of one.
template <typename T>
constexpr int kRows = sizeof(T) == 2 ? 16 : 8;

// Carry stage, one workgroup of kCarryWaves waves per (b, block of CH
// channels): carries[c] = state entering chunk c (REVERSE: the adjoint
// entering chunk c from the future).  Lane l takes channel l % CH and segment
// p = (64 / CH) w + l / CH of the chunks in scan order (1024 / CH segments),
// so each access reads a CH-wide run of a [B][NC][D] row.  CH = 16 suits few
// (b, channel block) pairs and many chunks; a wider CH gives fewer, longer
// segments and 4*CH-byte runs.  With A = decay^kChunkT the
// chunks compose as s(next) = A s + ends[c]: each lane folds its segment into
// (A_seg, B_seg), the lane folds the earlier segments' pairs from LDS in order
// into its incoming state, and rescans its segment writing each chunk's
// incoming state.  With resets a chunk whose cut flag is set has A = 0: its
// end state does not depend on the state entering it.
constexpr int kCarryWaves = 16;
constexpr int kCarryChannels = 16;
constexpr int kCarrySegs = kCarryWaves * (kWave / kCarryChannels);
constexpr int kCarrySeg = 32;   // chunk states a lane holds in registers per pass
constexpr int kDaRows = 16;     // dalpha partials loaded per block

template <bool REVERSE, bool RESET, int CH = kCarryChannels>
__global__ __launch_bounds__(kWave * kCarryWaves) void ema_carry(const float* __restrict__ ends,
                                                                 float* __restrict__ carries,
                                                                 const float* __restrict__ alpha, EmaGeom g) {
  constexpr int kSegs = kCarryWaves * (kWave / CH);
  __shared__ float2 sAB[kSegs][CH];
  const int w = threadIdx.x / kWave, l = threadIdx.x % kWave;
  const int ch = l % CH;
  const int p = w * (kWave / CH) + l / CH;
  const int nblk = (g.D + CH - 1) / CH;
  const int b = blockIdx.x / nblk;
  const int d = (blockIdx.x - b * nblk) * CH + ch;
  const bool live = d < g.D;
  const float decay = live ? 1.f - clamp_alpha(alpha, g, d) : 0.f;
  float full = 1.f;  // decay^kChunkT, by repeated multiplication as a serial scan applies it
  for (int i = 0; i < kChunkT; ++i) full *= decay;
  const int seg = (g.NC + kSegs - 1) / kSegs;
  const int k0 = p * seg, k1 = min(k0 + seg, g.NC);
  auto chunk = [&](int k) { return REVERSE ? g.NC - 1 - k : k; };
  const float* e = ends + static_cast<int64_t>(b) * g.NC * g.D + d;
  float* cr = carries + static_cast<int64_t>(b) * g.NC * g.D + d;
  auto factor = [&](int k) { return RESET && g.cut[b * g.NC + chunk(k)] ? 0.f : full; };
  // fold the segment: s_out = A s_in + Bv
  float A = 1.f, Bv = 0.f;
  float ev[kCarrySeg];   // the segment's first kCarrySeg chunk states, kept for the second pass
  if (live) {
    for (int kb = k0; kb < k1; kb += kCarrySeg) {
#pragma unroll
      for (int r = 0; r < kCarrySeg; ++r) ev[r] = kb + r < k1 ? e[static_cast<int64_t>(chunk(kb + r)) * g.D] : 0.f;
#pragma unroll
      for (int r = 0; r < kCarrySeg; ++r)
        if (kb + r < k1) {
          const float f = factor(kb + r);
          Bv = fmaf(f, Bv, ev[r]);
          A *= f;
        }
    }
  }
  sAB[p][ch] = make_float2(A, Bv);
  __syncthreads();
  float s = 0.f;   // state entering this lane's segment: the earlier segments in order
  for (int v = 0; v < p; ++v) {
    const float2 ab = sAB[v][ch];
    s = fmaf(ab.x, s, ab.y);
  }
  if (live) {
    for (int kb = k0; kb < k1; kb += kCarrySeg) {
      if (kb != k0 || seg > kCarrySeg) {   // reload unless the whole segment is still in registers
#pragma unroll
        for (int r = 0; r < kCarrySeg; ++r) ev[r] = kb + r < k1 ? e[static_cast<int64_t>(chunk(kb + r)) * g.D] : 0.f;
      }
#pragma unroll
      for (int r = 0; r < kCarrySeg; ++r)
        if (kb + r < k1) {
          cr[static_cast<int64_t>(chunk(kb + r)) * g.D] = s;
          s = fmaf(factor(kb + r), s, ev[r]);
        }
    }
  }
}

// Launches the carry stage over DK channels of B rows with the widest channel
// run that still gives every CU a workgroup (64 or 32 channels), else 16.
template <bool REVERSE, bool RESET>
void launch_carry(const float* in, float* out, const float* alpha, const EmaGeom& g, int B, int DK,
                  hipStream_t stream) {
  constexpr int kCus = 256;
  const dim3 block(kWave * kCarryWaves);
  if (static_cast<int64_t>(B) * ((DK + 63) / 64) >= kCus)
    hipLaunchKernelGGL((ema_carry<REVERSE, RESET, 64>), dim3(B * ((DK + 63) / 64)), block, 0, stream, in, out, alpha,
                       g);
  else if (static_cast<int64_t>(B) * ((DK + 31) / 32) >= kCus)
    hipLaunchKernelGGL((ema_carry<REVERSE, RESET, 32>), dim3(B * ((DK + 31) / 32)), block, 0, stream, in, out, alpha,
                       g);
  else
    hipLaunchKernelGGL((ema_carry<REVERSE, RESET, 16>), dim3(B * ((DK + 15) / 16)), block, 0, stream, in, out, alpha,
                       g);
}

// dalpha, one workgroup of kCarryWaves waves per block of kDaChannels
// channels: lane l takes channel l % kDaChannels and row phase
// p = 4 w + l / kDaChannels, and sums rows p, p + 64, ... of the [B * NC][D]
// partials in row order; the four phases of a wave are added by lane swaps
// and the waves in wave order.  For a per-channel alpha the projected-clamp
// rule is applied per channel; for a single alpha the channel sums go to
// `out` and a second pass adds them in order.
constexpr int kDaChannels = 16;
constexpr int kDaPhases = kCarryWaves * (kWave / kDaChannels);

__global__ __launch_bounds__(kWave * kCarryWaves) void ema_dalpha_channels(const float* __restrict__ da_part,
                                                                           const float* __restrict__ alpha,
                                                                           float* __restrict__ out, EmaGeom g) {
  __shared__ float sS[kCarryWaves][kDaChannels];
  const int w = threadIdx.x / kWave, l = threadIdx.x % kWave;
  const int ch = l % kDaChannels;
  const int phase = w * (kWave / kDaChannels) + l / kDaChannels;
  const int d = blockIdx.x * kDaChannels + ch;
  const bool live = d < g.D;
  const int rows = g.B * g.NC;
  float s = 0.f;
  if (live) {
    for (int r0 = phase; r0 < rows; r0 += kDaPhases * kDaRows) {
      float v[kDaRows];
#pragma unroll
      for (int i = 0; i < kDaRows; ++i) {
        const int r = r0 + i * kDaPhases;
        v[i] = r < rows ? da_part[static_cast<int64_t>(r) * g.D + d] : 0.f;
      }
#pragma unroll
      for (int i = 0; i < kDaRows; ++i) s += v[i];
    }
  }
  s = add_xor32(add_xor16(s));   // the wave's four phases, fixed order
  if (l < kDaChannels) sS[w][l] = s;
  __syncthreads();
  if (w == 0 && l < kDaChannels && live) {
    float t = 0.f;
    for (int v = 0; v < kCarryWaves; ++v) t += sS[v][l];
    if (g.per_channel) {
      const float ai = alpha[d];
      const bool blocked = (ai <= g.lo && t > 0.f) || (ai >= g.hi && t < 0.f);
      out[d] = blocked ? 0.f : t;
    } else {
      out[d] = t;
    }
  }
}

__global__ __launch_bounds__(kWave) void ema_dalpha_scalar(const float* __restrict__ chan, const float* __restrict__ alpha,
                                                          float* __restrict__ dalpha, EmaGeom g) {
  const int l = threadIdx.x;
  float s = 0.f;
  for (int d = l; d < g.D; d += kWave) s += chan[d];
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) s += __shfl_xor(s, o);
  if (l == 0) {
    const float ai = alpha[0];
    const bool blocked = (ai <= g.lo && s > 0.f) || (ai >= g.hi && s < 0.f);
    dalpha[0] = blocked ? 0.f : s;
  }
}

inline size_t ws_floats(int B, int N, int D) {
  const int NC = (N + kChunkT - 1) / kChunkT;
  return static_cast<size_t>(B) * NC * D;
}

// the per-chunk cut flags, after the float arrays
inline size_t ws_cut_bytes(int B, int N) {
  const int NC = (N + kChunkT - 1) / kChunkT;
  return (static_cast<size_t>(B) * NC + 255) / 256 * 256;
}

inline EmaGeom make_geom(int B, int N, int D, int vec, int per_channel, float lo, float hi, const uint8_t* reset,
                         const int64_t* reset_stride, void* workspace, size_t nfloats) {
  EmaGeom g;
  g.B = B; g.N = N; g.D = D;
  g.NC = (N + kChunkT - 1) / kChunkT;
  g.DV = D / vec;
  g.per_channel = per_channel;
  g.alpha_div = 1;
  g.lo = lo; g.hi = hi;
  g.reset = reset;
  g.srb = reset ? reset_stride[0] : 0;
  g.srn = reset ? reset_stride[1] : 0;
  g.cut = static_cast<uint8_t*>(workspace) + nfloats * sizeof(float);
  return g;
}

}  // namespace
}  // namespace dwarf
