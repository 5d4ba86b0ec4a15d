// Causal EMA scan, y[t] = a x[t] + (1 - a) y[t-1], y[-1] = 0, fp32 state
// (reference: _CausalEMAFn ema:263-364 with kernels ema:73-260).
//
// Time is cut into chunks of kChunkT tokens.  Each lane owns VEC adjacent
// channels of one (b, chunk), so a wave reads 64*VEC consecutive channels of
// one token per load.
//   forward:  local  - chunk end state with zero carry-in (reads x)
//             carry  - one workgroup per (b, 16 channels) scans the chunk
//                      ends and writes each chunk's carry-in (tiny)
//             apply  - rescans the chunk from its carry-in, writes y
//   backward: the same three stages run in reverse time on dy for the
//             adjoint lambda[t] = dy[t] + (1 - a) lambda[t+1]; the apply
//             stage writes dx = a * lambda and a per-lane partial of
//             dalpha = sum lambda[t] (x[t] - y[t-1]); one workgroup per 16
//             channels sums the partials in a fixed order and applies the
//             projected-clamp rule of ema:357-364.
// The carry and dalpha stages read the [B][NC][D] per-chunk arrays in runs of
// 16 channels (lane = channel within the run) and combine in a fixed order.
// Alpha may be one value (the reference contract, ema:557-558) or one per
// channel; the clamp to [floor, ceiling] happens in-kernel (ema:274-277).
// Optional reset flags [B,N] zero the state before the tokens they mark
// (the reset-aware scan, ema:368-509): the local and apply stages apply them
// inside the chunk, the local stage records whether a chunk contains one, and
// the carry stage gives such a chunk a zero transfer factor.  In reverse
// time a reset at token t + 1 cuts the adjoint flowing into t, and y[t-1]
// does not enter dalpha at a reset token.
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
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) st1<T>(p + i, v[i]);
  }
}

struct EmaGeom {
  int B, N, D, NC, DV;  // DV = D / VEC lanes per row
  int per_channel;
  float lo, hi;
  const uint8_t* reset;   // [B,N] reset flags (RESET kernels only)
  int64_t srb, srn;
  uint8_t* cut;           // [B][NC]: the chunk cuts the carry (a reset inside, see ema_carry)
};

// The state is zeroed before a token whose reset flag is set (ema:533-535).
__device__ __forceinline__ bool reset_at(const EmaGeom& g, int b, int t) {
  return g.reset[b * g.srb + static_cast<int64_t>(t) * g.srn] != 0;
}

__device__ __forceinline__ float clamp_alpha(const float* alpha, int per_channel, int d, float lo, float hi) {
  const float a = alpha[per_channel ? d : 0];
  return fminf(fmaxf(a, lo), hi);
}

// Rows of one chunk are loaded in blocks of kRows<T> (all loads of a block
// are issued before the recurrence consumes them), so a lane keeps a block of
// rows in flight instead of one.
template <typename T>
constexpr int kRows = sizeof(T) == 2 ? 16 : 8;

// ---- forward --------------------------------------------------------------
template <typename T, int VEC, bool RESET>
__global__ __launch_bounds__(kEmaBlock) void ema_fwd_local(const T* __restrict__ x, int64_t sxb, int64_t sxn,
                                                          const float* __restrict__ alpha, float* __restrict__ ends,
                                                          EmaGeom g) {
  constexpr int R = kRows<T>;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * kEmaBlock + threadIdx.x;
  const int dv = tid % g.DV;
  const int c = (tid / g.DV) % g.NC;
  const int b = tid / (static_cast<int64_t>(g.DV) * g.NC);
  if (b >= g.B) return;
  const int d0 = dv * VEC;
  float a[VEC], st[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) { a[i] = clamp_alpha(alpha, g.per_channel, d0 + i, g.lo, g.hi); st[i] = 0.f; }
  const int t0 = c * kChunkT;
  const int len = min(kChunkT, g.N - t0);
  const T* p = x + b * sxb + static_cast<int64_t>(t0) * sxn + d0;
  bool cut = false;
  for (int tb = 0; tb < len; tb += R) {
    float xv[R][VEC];
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (tb + r < len) ldv<T, VEC>(p + static_cast<int64_t>(tb + r) * sxn, xv[r]);
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (tb + r < len) {
        if constexpr (RESET) {
          if (reset_at(g, b, t0 + tb + r)) {
            cut = true;
#pragma unroll
            for (int i = 0; i < VEC; ++i) st[i] = 0.f;
          }
        }
#pragma unroll
        for (int i = 0; i < VEC; ++i) st[i] = fmaf(a[i], xv[r][i], (1.f - a[i]) * st[i]);
      }
  }
  float* e = ends + (static_cast<int64_t>(b) * g.NC + c) * g.D + d0;
#pragma unroll
  for (int i = 0; i < VEC; ++i) e[i] = st[i];
  if (RESET && dv == 0) g.cut[b * g.NC + c] = cut;   // a reset in [t0, t0 + len)
}

// Carry stage, one workgroup of kCarryWaves waves per (b, block of
// kCarryChannels channels): carries[c] = state entering chunk c (REVERSE: the
// adjoint entering chunk c from the future).  Lane l takes channel
// l % kCarryChannels and segment p = 4 w + l / kCarryChannels of the chunks
// in scan order (kCarrySegs segments), so each access reads a
// kCarryChannels-wide run of a [B][NC][D] row.  With A = decay^kChunkT the
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

template <bool REVERSE, bool RESET>
__global__ __launch_bounds__(kWave * kCarryWaves) void ema_carry(const float* __restrict__ ends,
                                                                 float* __restrict__ carries,
                                                                 const float* __restrict__ alpha, EmaGeom g) {
  __shared__ float2 sAB[kCarrySegs][kCarryChannels];
  const int w = threadIdx.x / kWave, l = threadIdx.x % kWave;
  const int ch = l % kCarryChannels;
  const int p = w * (kWave / kCarryChannels) + l / kCarryChannels;
  const int nblk = (g.D + kCarryChannels - 1) / kCarryChannels;
  const int b = blockIdx.x / nblk;
  const int d = (blockIdx.x - b * nblk) * kCarryChannels + ch;
  const bool live = d < g.D;
  const float decay = live ? 1.f - clamp_alpha(alpha, g.per_channel, d, g.lo, g.hi) : 0.f;
  float full = 1.f;  // decay^kChunkT, by repeated multiplication as a serial scan applies it
  for (int i = 0; i < kChunkT; ++i) full *= decay;
  const int seg = (g.NC + kCarrySegs - 1) / kCarrySegs;
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

template <typename T, int VEC, bool RESET>
__global__ __launch_bounds__(kEmaBlock) void ema_fwd_apply(const T* __restrict__ x, int64_t sxb, int64_t sxn,
                                                          T* __restrict__ y, int64_t syb, int64_t syn,
                                                          const float* __restrict__ alpha,
                                                          const float* __restrict__ carries, EmaGeom g) {
  constexpr int R = kRows<T>;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * kEmaBlock + threadIdx.x;
  const int dv = tid % g.DV;
  const int c = (tid / g.DV) % g.NC;
  const int b = tid / (static_cast<int64_t>(g.DV) * g.NC);
  if (b >= g.B) return;
  const int d0 = dv * VEC;
  float a[VEC], st[VEC];
  const float* cr = carries + (static_cast<int64_t>(b) * g.NC + c) * g.D + d0;
#pragma unroll
  for (int i = 0; i < VEC; ++i) { a[i] = clamp_alpha(alpha, g.per_channel, d0 + i, g.lo, g.hi); st[i] = cr[i]; }
  const int t0 = c * kChunkT;
  const int len = min(kChunkT, g.N - t0);
  const T* px = x + b * sxb + static_cast<int64_t>(t0) * sxn + d0;
  T* py = y + b * syb + static_cast<int64_t>(t0) * syn + d0;
  for (int tb = 0; tb < len; tb += R) {
    float xv[R][VEC];
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (tb + r < len) ldv<T, VEC>(px + static_cast<int64_t>(tb + r) * sxn, xv[r]);
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (tb + r < len) {
        if constexpr (RESET) {
          if (reset_at(g, b, t0 + tb + r)) {
#pragma unroll
            for (int i = 0; i < VEC; ++i) st[i] = 0.f;
          }
        }
#pragma unroll
        for (int i = 0; i < VEC; ++i) st[i] = fmaf(a[i], xv[r][i], (1.f - a[i]) * st[i]);
        stv<T, VEC>(py + static_cast<int64_t>(tb + r) * syn, st);
      }
  }
}

// ---- backward -------------------------------------------------------------
template <typename T, int VEC, bool RESET>
__global__ __launch_bounds__(kEmaBlock) void ema_bwd_local(const T* __restrict__ dy, int64_t sgb, int64_t sgn,
                                                          const float* __restrict__ alpha, float* __restrict__ starts,
                                                          EmaGeom g) {
  constexpr int R = kRows<T>;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * kEmaBlock + threadIdx.x;
  const int dv = tid % g.DV;
  const int c = (tid / g.DV) % g.NC;
  const int b = tid / (static_cast<int64_t>(g.DV) * g.NC);
  if (b >= g.B) return;
  const int d0 = dv * VEC;
  float dec[VEC], st[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) { dec[i] = 1.f - clamp_alpha(alpha, g.per_channel, d0 + i, g.lo, g.hi); st[i] = 0.f; }
  const int t0 = c * kChunkT;
  const int len = min(kChunkT, g.N - t0);
  const T* p = dy + b * sgb + static_cast<int64_t>(t0) * sgn + d0;
  for (int tb = len - 1; tb >= 0; tb -= R) {   // rows tb, tb-1, ..., tb-R+1
    float gv[R][VEC];
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (tb - r >= 0) ldv<T, VEC>(p + static_cast<int64_t>(tb - r) * sgn, gv[r]);
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (tb - r >= 0) {
        if constexpr (RESET) {   // a reset at token t + 1 cuts the adjoint flowing back into t
          if (tb - r + 1 < len && reset_at(g, b, t0 + tb - r + 1)) {
#pragma unroll
            for (int i = 0; i < VEC; ++i) st[i] = 0.f;
          }
        }
#pragma unroll
        for (int i = 0; i < VEC; ++i) st[i] = fmaf(dec[i], st[i], gv[r][i]);
      }
  }
  float* e = starts + (static_cast<int64_t>(b) * g.NC + c) * g.D + d0;
#pragma unroll
  for (int i = 0; i < VEC; ++i) e[i] = st[i];
  if (RESET && dv == 0) {   // a reset in [t0 + 1, t0 + len] (tokens inside the sequence)
    bool cut = false;
    for (int t = t0 + 1; t <= t0 + len && t < g.N; ++t) cut = cut || reset_at(g, b, t);
    g.cut[b * g.NC + c] = cut;
  }
}

template <typename T, int VEC, bool RESET>
__global__ __launch_bounds__(kEmaBlock) void ema_bwd_apply(const T* __restrict__ x, int64_t sxb, int64_t sxn,
                                                          const T* __restrict__ y, int64_t syb, int64_t syn,
                                                          const T* __restrict__ dy, int64_t sgb, int64_t sgn,
                                                          T* __restrict__ dx, int64_t sdb, int64_t sdn,
                                                          const float* __restrict__ alpha,
                                                          const float* __restrict__ carries,
                                                          float* __restrict__ da_part, EmaGeom g) {
  constexpr int R = kRows<T> / 2;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * kEmaBlock + threadIdx.x;
  const int dv = tid % g.DV;
  const int c = (tid / g.DV) % g.NC;
  const int b = tid / (static_cast<int64_t>(g.DV) * g.NC);
  if (b >= g.B) return;
  const int d0 = dv * VEC;
  float a[VEC], st[VEC], da[VEC];
  const float* cr = carries + (static_cast<int64_t>(b) * g.NC + c) * g.D + d0;
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    a[i] = clamp_alpha(alpha, g.per_channel, d0 + i, g.lo, g.hi);
    st[i] = cr[i];
    da[i] = 0.f;
  }
  const int t0 = c * kChunkT;
  const int len = min(kChunkT, g.N - t0);
  const T* pg = dy + b * sgb + static_cast<int64_t>(t0) * sgn + d0;
  const T* pxx = x + b * sxb + static_cast<int64_t>(t0) * sxn + d0;
  const T* pyy = y + b * syb + static_cast<int64_t>(t0) * syn + d0;
  T* pd = dx + b * sdb + static_cast<int64_t>(t0) * sdn + d0;
  for (int tb = len - 1; tb >= 0; tb -= R) {
    float gv[R][VEC], xv[R][VEC], yp[R][VEC];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int t = tb - r;
      if (t >= 0) {
        ldv<T, VEC>(pg + static_cast<int64_t>(t) * sgn, gv[r]);
        ldv<T, VEC>(pxx + static_cast<int64_t>(t) * sxn, xv[r]);
        if (t0 + t > 0) {
          ldv<T, VEC>(pyy + static_cast<int64_t>(t - 1) * syn, yp[r]);
        } else {
#pragma unroll
          for (int i = 0; i < VEC; ++i) yp[r][i] = 0.f;
        }
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int t = tb - r;
      if (t >= 0) {
        if constexpr (RESET) {
          if (t0 + t + 1 < g.N && reset_at(g, b, t0 + t + 1)) {   // cut from the future (or the carry)
#pragma unroll
            for (int i = 0; i < VEC; ++i) st[i] = 0.f;
          }
          if (reset_at(g, b, t0 + t)) {   // y[t-1] does not feed token t (ema:445-448)
#pragma unroll
            for (int i = 0; i < VEC; ++i) yp[r][i] = 0.f;
          }
        }
        float out[VEC];
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          st[i] = fmaf(1.f - a[i], st[i], gv[r][i]);
          out[i] = a[i] * st[i];
          da[i] = fmaf(st[i], xv[r][i] - yp[r][i], da[i]);
        }
        stv<T, VEC>(pd + static_cast<int64_t>(t) * sdn, out);
      }
    }
  }
  float* dp = da_part + (static_cast<int64_t>(b) * g.NC + c) * g.D + d0;
#pragma unroll
  for (int i = 0; i < VEC; ++i) dp[i] = da[i];
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
  g.lo = lo; g.hi = hi;
  g.reset = reset;
  g.srb = reset ? reset_stride[0] : 0;
  g.srn = reset ? reset_stride[1] : 0;
  g.cut = static_cast<uint8_t*>(workspace) + nfloats * sizeof(float);
  return g;
}

template <typename T, int VEC, bool RESET>
hipError_t ema_fwd_typed(const dwarf_ema_fwd_args& a, hipStream_t stream) {
  const size_t nf = ws_floats(a.B, a.N, a.D);
  const EmaGeom g = make_geom(a.B, a.N, a.D, VEC, a.alpha_per_channel, a.floor_, a.ceiling, a.reset,
                              a.reset_stride, a.workspace, 2 * nf);
  float* ends = static_cast<float*>(a.workspace);
  float* carries = ends + nf;
  const int64_t lanes = static_cast<int64_t>(a.B) * g.NC * g.DV;
  const int blocks = static_cast<int>((lanes + kEmaBlock - 1) / kEmaBlock);
  const T* x = static_cast<const T*>(a.x);
  T* y = static_cast<T*>(a.y);
  hipLaunchKernelGGL((ema_fwd_local<T, VEC, RESET>), dim3(blocks), dim3(kEmaBlock), 0, stream, x, a.x_stride[0],
                     a.x_stride[1], a.alpha, ends, g);
  const int cblocks = a.B * ((a.D + kCarryChannels - 1) / kCarryChannels);
  hipLaunchKernelGGL((ema_carry<false, RESET>), dim3(cblocks), dim3(kWave * kCarryWaves), 0, stream, ends, carries,
                     a.alpha, g);
  hipLaunchKernelGGL((ema_fwd_apply<T, VEC, RESET>), dim3(blocks), dim3(kEmaBlock), 0, stream, x, a.x_stride[0],
                     a.x_stride[1], y, a.y_stride[0], a.y_stride[1], a.alpha, carries, g);
  return hipGetLastError();
}

template <typename T, int VEC, bool RESET>
hipError_t ema_bwd_typed(const dwarf_ema_bwd_args& a, hipStream_t stream) {
  const size_t nf = ws_floats(a.B, a.N, a.D);
  const EmaGeom g = make_geom(a.B, a.N, a.D, VEC, a.alpha_per_channel, a.floor_, a.ceiling, a.reset,
                              a.reset_stride, a.workspace, 3 * nf);
  float* starts = static_cast<float*>(a.workspace);
  float* carries = starts + nf;
  float* da_part = carries + nf;
  const int64_t lanes = static_cast<int64_t>(a.B) * g.NC * g.DV;
  const int blocks = static_cast<int>((lanes + kEmaBlock - 1) / kEmaBlock);
  hipLaunchKernelGGL((ema_bwd_local<T, VEC, RESET>), dim3(blocks), dim3(kEmaBlock), 0, stream,
                     static_cast<const T*>(a.dy), a.dy_stride[0], a.dy_stride[1], a.alpha, starts, g);
  const int cblocks = a.B * ((a.D + kCarryChannels - 1) / kCarryChannels);
  hipLaunchKernelGGL((ema_carry<true, RESET>), dim3(cblocks), dim3(kWave * kCarryWaves), 0, stream, starts, carries,
                     a.alpha, g);
  hipLaunchKernelGGL((ema_bwd_apply<T, VEC, RESET>), dim3(blocks), dim3(kEmaBlock), 0, stream,
                     static_cast<const T*>(a.x), a.x_stride[0], a.x_stride[1], static_cast<const T*>(a.y),
                     a.y_stride[0], a.y_stride[1], static_cast<const T*>(a.dy), a.dy_stride[0], a.dy_stride[1],
                     static_cast<T*>(a.dx), a.dx_stride[0], a.dx_stride[1], a.alpha, carries, da_part, g);
  if (a.dalpha) {
    const int rb = (a.D + kDaChannels - 1) / kDaChannels;
    if (a.alpha_per_channel) {
      hipLaunchKernelGGL(ema_dalpha_channels, dim3(rb), dim3(kWave * kCarryWaves), 0, stream, da_part, a.alpha,
                         a.dalpha, g);
    } else {
      float* chan = starts;   // free after the apply stage; D <= B * NC * D floats
      hipLaunchKernelGGL(ema_dalpha_channels, dim3(rb), dim3(kWave * kCarryWaves), 0, stream, da_part, a.alpha,
                         chan, g);
      hipLaunchKernelGGL(ema_dalpha_scalar, dim3(1), dim3(kWave), 0, stream, chan, a.alpha, a.dalpha, g);
    }
  }
  return hipGetLastError();
}

}  // namespace

size_t ema_fwd_workspace(int B, int N, int D) {
  return 2 * ws_floats(B, N, D) * sizeof(float) + ws_cut_bytes(B, N);
}
size_t ema_bwd_workspace(int B, int N, int D) {
  return 3 * ws_floats(B, N, D) * sizeof(float) + ws_cut_bytes(B, N);
}

template <bool RESET>
hipError_t launch_ema_fwd_r(const dwarf_ema_fwd_args& a, hipStream_t stream) {
  const bool vec4 = (a.D % 4) == 0;
  if (a.dtype == DWARF_BF16)
    return vec4 ? ema_fwd_typed<bf16, 4, RESET>(a, stream) : ema_fwd_typed<bf16, 1, RESET>(a, stream);
  return vec4 ? ema_fwd_typed<float, 4, RESET>(a, stream) : ema_fwd_typed<float, 1, RESET>(a, stream);
}

template <bool RESET>
hipError_t launch_ema_bwd_r(const dwarf_ema_bwd_args& a, hipStream_t stream) {
  const bool vec4 = (a.D % 4) == 0;
  if (a.dtype == DWARF_BF16)
    return vec4 ? ema_bwd_typed<bf16, 4, RESET>(a, stream) : ema_bwd_typed<bf16, 1, RESET>(a, stream);
  return vec4 ? ema_bwd_typed<float, 4, RESET>(a, stream) : ema_bwd_typed<float, 1, RESET>(a, stream);
}

hipError_t launch_ema_fwd(const dwarf_ema_fwd_args& a, hipStream_t stream) {
  return a.reset ? launch_ema_fwd_r<true>(a, stream) : launch_ema_fwd_r<false>(a, stream);
}

hipError_t launch_ema_bwd(const dwarf_ema_bwd_args& a, hipStream_t stream) {
  return a.reset ? launch_ema_bwd_r<true>(a, stream) : launch_ema_bwd_r<false>(a, stream);
}

}  // namespace dwarf
