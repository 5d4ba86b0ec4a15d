// Pieces shared by the causal EMA scan (ema.hip) and the InterferencePacket
// pool (packet.hip): element loads and stores, the chunk geometry, the carry
// stage that joins the chunks and the fixed-order dalpha reductions.  The
// kernels are in an unnamed namespace: each translation unit that launches
// them holds its own copy.
#pragma once

#include <algorithm>

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


// ---------------------------------------------------------------------------
// Single-pass scans with decoupled look-back over [N][D] slabs (the causal EMA
// in ema.hip, the InterferencePacket pool in packet.hip; ema.hip describes the
// scheme).  A workgroup of kLbWaves waves takes that many consecutive
// 128-token tiles of one (b, channel block); the helpers below publish and
// walk the workgroups' packed (value, tag) words.
// ---------------------------------------------------------------------------
constexpr int kLbGroups = 16;   // channel groups of a tile (lanes cg)
constexpr int kLbSegs = 4;      // token segments of a tile (lanes ts)
constexpr int kLbSeg = 32;                         // tokens per segment (the lane's registers)
constexpr int kLbWaitLimit = 1 << 22;              // default polls before a wait gives up
constexpr size_t kLbHead = 256;                    // bytes ahead of the words (unused, kept zero)
constexpr int kLbWaves = 4;                        // tiles (one wave each) per workgroup, consecutive in scan order
constexpr int kLbRun = 32;                         // workgroup tiles per run (one inclusive state per run)
constexpr int kLbBatch = 8;                        // aggregates loaded together by a carry walk

struct LbGeom {
  int B, N, D;
  int CB;    // channel blocks of 16 VEC channels
  int NCH;   // tiles along time per (b, channel block)
  int NWG;   // workgroup tiles along time, ceil(NCH / kLbWaves)
  int S;     // (b, channel block) slices, B * CB
  int per_channel;
  float lo, hi;
  const uint8_t* reset;
  int64_t srb, srn;
  unsigned long long* words;   // [NWG * S][16 VEC]: workgroup aggregates, (value bits, tag << 32)
  unsigned long long* runs;    // [(ceil(NWG / kLbRun) - 1) * S][16 VEC]: inclusive states of all runs but the last
  int64_t kw, kr;              // words and runs of one scale (scale k at words + k kw, runs + k kr)
  float* da_part;              // backward: [NWG][B][D] dalpha partials (row widx * B + b)
  int wait_limit;
};

__device__ __forceinline__ float lb_alpha(const float* alpha, const LbGeom& g, int d) {
  const float a = alpha[g.per_channel ? d : 0];
  return fminf(fmaxf(a, g.lo), g.hi);
}

// The reset flags of tokens s0 .. s0 + kLbSeg of batch row b as bits 0 ..
// kLbSeg (a token outside [0, N) reads 0), for lane (cg = lane & 15,
// ts = lane >> 4) of a tile whose segment ts starts at s0: the segment's 16
// lanes read two flags each and two wave ballots hand every lane its 32,
// and each lane reads the flag of the token after its segment.  The scans
// then test bits instead of loading a flag at each use.  Every lane of the
// wave calls it.
__device__ __forceinline__ uint64_t lb_reset_bits(const LbGeom& g, int b, int s0) {
  static_assert(kLbSeg == 32 && kLbGroups == 16 && kLbSegs * kLbGroups == kWave, "16 lanes per 32-token segment");
  const int lane = threadIdx.x & (kWave - 1), cg = lane & 15, ts = lane >> 4;
  const uint8_t* p = g.reset + b * g.srb;
  auto flag = [&](int tt) {
    const uint8_t f = p[static_cast<int64_t>(min(max(tt, 0), g.N - 1)) * g.srn];   // an address inside the row
    return tt >= 0 && tt < g.N && f != 0;
  };
  const uint64_t lo = __ballot(flag(s0 + cg)), hi = __ballot(flag(s0 + 16 + cg));
  const bool nx = flag(s0 + kLbSeg);
  return ((lo >> (16 * ts)) & 0xffffu) | (((hi >> (16 * ts)) & 0xffffu) << 16) | (static_cast<uint64_t>(nx) << 32);
}

__device__ __forceinline__ bool lb_bit(uint64_t m, int t) { return (m >> t) & 1u; }

// Raw VEC channels of one token in registers, loaded and stored through
// buffer resources (an out-of-range offset reads zeros / drops the store).
template <typename T, int VEC>
struct LbRaw {
  static constexpr int kWords = (VEC * sizeof(T) + 3) / 4;
  uint32_t w[kWords];
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    if constexpr (VEC * sizeof(T) == 16) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
      w[0] = v[0]; w[1] = v[1]; w[2] = v[2]; w[3] = v[3];
    } else if constexpr (VEC * sizeof(T) == 8) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
      w[0] = v[0]; w[1] = v[1];
    } else if constexpr (VEC * sizeof(T) == 4) {
      w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
    } else {
      w[0] = __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
    }
  }
  __device__ __forceinline__ void widen(float* v) const {
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int i = 0; i < VEC; ++i) v[i] = (i & 1) ? bf16_hi(w[i / 2]) : bf16_lo(w[i / 2]);
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) v[i] = __uint_as_float(w[i]);
    }
  }
};

template <typename T, int VEC>
__device__ __forceinline__ void lb_store(__amdgpu_buffer_rsrc_t r, uint32_t off, const float* v) {
  if constexpr (sizeof(T) == 2 && VEC == 4) {
    __builtin_amdgcn_raw_buffer_store_b64(
        __builtin_bit_cast(__attribute__((ext_vector_type(2))) unsigned, make_uint2(pack_bf16x2(v[0], v[1]),
                                                                                    pack_bf16x2(v[2], v[3]))),
        r, off, 0, 0);
  } else if constexpr (sizeof(T) == 4 && VEC == 4) {
    __builtin_amdgcn_raw_buffer_store_b128(
        __builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned,
                           make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                                      __float_as_uint(v[3]))),
        r, off, 0, 0);
  } else if constexpr (sizeof(T) == 2) {
    __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16_bits(v[0]), r, off, 0, 0);
  } else {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v[0]), r, off, 0, 0);
  }
}

// One [N][D] slab of batch row b (the host bounds its span below 2 GiB).
template <typename T>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t lb_rsrc(const T* base, int64_t sb, int64_t sn, int b, int N) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(base + b * sb), 0,
                                           static_cast<int>(static_cast<int64_t>(N) * sn * sizeof(T)), 0x00020000);
}

__device__ __forceinline__ void lb_publish(unsigned long long* w, float v, unsigned tag) {
  const unsigned long long x = (static_cast<unsigned long long>(tag) << 32) | __float_as_uint(v);
  __hip_atomic_store(w, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The published word, or 0 when the wait gives up.
__device__ __forceinline__ unsigned long long lb_wait(const unsigned long long* w, int limit) {
  for (int it = 0; it < limit; ++it) {
    const unsigned long long x = __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (x >> 32) return x;
    __builtin_amdgcn_s_sleep(2);
  }
  return 0;
}

// The state entering the workgroup tile at scan-order index idx of its slice:
// the aggregates of the run's tiles before it composed in order into
// (Pa, Qa) (P_p = full for tag 1, 0 for tag 3), loaded kLbBatch at a time,
// then applied to the previous run's inclusive state (none in the first run):
// C = Pa C_run + Qa.  The run's state is waited on last, so the walk over the
// aggregates overlaps the previous run's.  NaN when a wait gives up.
__device__ __forceinline__ float lb_carry(const LbGeom& g, const unsigned long long* words,
                                         const unsigned long long* runs, int slice, int ch, int ct, int idx,
                                         float full) {
  const int run = idx / kLbRun, first = run * kLbRun;
  float Pa = 1.f, Qa = 0.f;
  for (int p0 = first; p0 < idx; p0 += kLbBatch) {
    unsigned long long w[kLbBatch];
#pragma unroll
    for (int k = 0; k < kLbBatch; ++k) {   // a slot past idx - 1 reloads the last one (unused)
      const int p = min(p0 + k, idx - 1);
      w[k] = __hip_atomic_load(words + (static_cast<int64_t>(p) * g.S + slice) * ct + ch, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int k = 0; k < kLbBatch; ++k) {
      const int p = p0 + k;
      if (p < idx) {
        unsigned long long x = w[k];
        if (!(x >> 32)) {
          x = lb_wait(words + (static_cast<int64_t>(p) * g.S + slice) * ct + ch, g.wait_limit);
          if (!x) return __builtin_nanf("");
        }
        const float Pp = (x >> 32) == 3u ? 0.f : full;
        Qa = fmaf(Pp, Qa, __uint_as_float(static_cast<uint32_t>(x)));
        Pa *= Pp;
      }
    }
  }
  if (run == 0) return Qa;
  const unsigned long long x = lb_wait(runs + (static_cast<int64_t>(run - 1) * g.S + slice) * ct + ch,
                                       g.wait_limit);
  if (!x) return __builtin_nanf("");
  return fmaf(Pa, __uint_as_float(static_cast<uint32_t>(x)), Qa);
}

// LDS of a workgroup: each wave's tile maps (P, Q) per channel and scale,
// and the states entering the workgroup.
template <int K>
struct LbShared {
  float P[K][kLbWaves][kWave];
  float Q[K][kLbWaves][kWave];
  float C[K][kWave];
};

// Steps 3-4 for channel ch of wave w's tile, for each of K scans of the same
// tiles (owner lanes only take part): the tiles' maps meet in LDS; wave 0
// composes them in scan order into the workgroup's (P, Q) of each scale and
// publishes every scale's Q tagged with its factor before it waits on
// anything, then forms the states entering the workgroup from the earlier
// workgroups (lb_carry; full_wg is a full workgroup's factor per scale) and,
// in a run's last workgroup, publishes the runs' inclusive states; each wave
// then composes the states entering its own tile from those and the earlier
// tiles of its workgroup, in order.  Every lane of the workgroup reaches both
// barriers.
template <int K>
__device__ __forceinline__ void lb_join(const LbGeom& g, LbShared<K>& sh, int slice, int ch, bool owner, int ct,
                                        int widx, int w, const float* Po, const float* Qo, const float* full_wg,
                                        float* C) {
  if (owner) {
#pragma unroll
    for (int k = 0; k < K; ++k) {
      sh.P[k][w][ch] = Po[k];
      sh.Q[k][w][ch] = Qo[k];
    }
  }
  __syncthreads();
  if (w == 0 && owner) {
    float P[K], Q[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      P[k] = 1.f;
      Q[k] = 0.f;
#pragma unroll
      for (int j = 0; j < kLbWaves; ++j) {
        Q[k] = fmaf(sh.P[k][j][ch], Q[k], sh.Q[k][j][ch]);
        P[k] *= sh.P[k][j][ch];
      }
      lb_publish(g.words + k * g.kw + (static_cast<int64_t>(widx) * g.S + slice) * ct + ch, Q[k],
                 P[k] == 0.f ? 3u : 1u);
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const float Ck = widx > 0 ? lb_carry(g, g.words + k * g.kw, g.runs + k * g.kr, slice, ch, ct, widx, full_wg[k])
                                : 0.f;
      if (widx % kLbRun == kLbRun - 1 && widx + 1 < g.NWG)
        lb_publish(g.runs + k * g.kr + (static_cast<int64_t>(widx / kLbRun) * g.S + slice) * ct + ch,
                   fmaf(P[k], Ck, Q[k]), 2u);
      sh.C[k][ch] = Ck;
    }
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < K; ++k) {
    float Ck = 0.f;
    if (owner) {
      Ck = sh.C[k][ch];
      for (int j = 0; j < w; ++j) Ck = fmaf(sh.P[k][j][ch], Ck, sh.Q[k][j][ch]);
    }
    C[k] = Ck;
  }
}

// Clears the look-back words of the next scan.
__global__ __launch_bounds__(kEmaBlock) void ema_lb_zero(uint4* __restrict__ p, int64_t n16) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kEmaBlock + threadIdx.x; i < n16;
       i += static_cast<int64_t>(gridDim.x) * kEmaBlock)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// Look-back plan: channel blocks, tiles along time, words of one scale and
// bytes of the words of K scales (each scale's aggregates, then each scale's
// runs' inclusive states).
struct LbPlan {
  int CB, NCH, NWG, S;
  int64_t kw, kr;       // aggregate words and run words of one scale
  size_t words_bytes;
};

inline LbPlan lb_plan(int B, int N, int D, int vec, int seg, int K = 1) {
  LbPlan p;
  const int ct = kLbGroups * vec;
  p.CB = (D + ct - 1) / ct;
  p.NCH = (N + kLbSegs * seg - 1) / (kLbSegs * seg);
  p.NWG = (p.NCH + kLbWaves - 1) / kLbWaves;
  p.S = B * p.CB;
  const int runs = (p.NWG + kLbRun - 1) / kLbRun;   // the last run publishes no inclusive state
  p.kw = static_cast<int64_t>(p.NWG) * p.S * ct;
  p.kr = static_cast<int64_t>(std::max(runs - 1, 0)) * p.S * ct;
  p.words_bytes = static_cast<size_t>(K) * (p.kw + p.kr) * 8;
  return p;
}

// Every [N][D] slab of these tensors within 32-bit buffer offsets.
inline bool lb_fits(int N, int64_t sn, size_t elem) {
  return static_cast<int64_t>(N) * sn * static_cast<int64_t>(elem) < (int64_t(1) << 31);
}

// The zeroing launch ahead of a scan: the words.
inline void lb_zero(const LbGeom& g, const LbPlan& p, hipStream_t stream) {
  const int64_t n16 = static_cast<int64_t>(p.words_bytes / 16);
  const int blocks = static_cast<int>(std::min<int64_t>(std::max<int64_t>((n16 + kEmaBlock - 1) / kEmaBlock, 1), 1024));
  hipLaunchKernelGGL(ema_lb_zero, dim3(blocks), dim3(kEmaBlock), 0, stream, reinterpret_cast<uint4*>(g.words), n16);
}


}  // namespace
}  // namespace dwarf
