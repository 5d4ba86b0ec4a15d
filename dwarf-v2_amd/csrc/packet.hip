// InterferencePacket pool (reference: InterferencePacket.forward,
// train:260-267): K causal EMA scans of one input x at scalar factors a_k and
// their mix
//   scan_k = EMA(x, a_k) stored in T,   pooled = ((w_0 scan_0 + w_1 scan_1) + ...)
// with w_k = softmax(mix_logits)_k cast to T and every product and partial
// sum rounded to T, as the reference's bf16 tensor arithmetic rounds them.
// The reference runs K separate scans (each reading x and writing its scan)
// and K products and K - 1 sums; here the forward reads x once and writes
// pooled once.
//
// Forward and backward are each one pass with the EMA's decoupled look-back
// (packet_fwd_lb, packet_bwd_lb; the backward's parameter sums then take one
// reduction launch) wherever every [N][D] slab of the operands spans less
// than 2 GiB.  Larger slabs take three stages on the EMA's 16-token chunks
// (ema_common.h), the forward then reading x twice:
//   forward:  local - the K chunk-end states with zero carry-in (reads x)
//             carry - the EMA carry stage over K*D scale-major channels,
//                     writing each chunk's incoming states to `state`
//             apply - rescans the chunk for the K scales, writes pooled
//   backward: local - the K chunk-start adjoints of the scan gradients
//                     dscan_k = T(dpooled w_k) (reads dpooled)
//             carry - the reverse carry stage over K*D channels
//             apply - recomputes the chunk's scans from `state` (forward in
//                     time, kept in registers), then runs the adjoints back
//                     in time: dx = sum_k a_k lambda_k, and per workgroup
//                     the sums of lambda_k (x[t] - scan_k[t-1]) (dalpha) and
//                     of T(dpooled scan_k) (dweight)
//             reduce - the workgroup sums in a fixed order: dalpha with the
//                      projected-clamp rule of ema:357-364, dweight in T.
#include <algorithm>

#include "ema_common.h"
#include "dwarf_dsqg.h"

namespace dwarf {
namespace {

constexpr int kMaxScales = 4;
constexpr int kPkRedThreads = 1024;
// Rows a lane keeps per block of the look-back backward's reverse pass with
// four channels per lane (bf16 8, fp32 4: its kept scans take a register
// each); one channel per lane keeps a whole chunk.
template <typename T>
constexpr int pk_lb_keep() { return sizeof(T) == 2 ? 8 : 4; }
// Tokens per lane segment of the look-back backward (16-token segments, twice
// the waves, measured 2 us slower at [15, 2048, 512]).
constexpr int kPkLbSeg = kLbSeg;

// The value a T tensor holds for v.
template <typename T>
__device__ __forceinline__ float rnd(float v);
template <>
__device__ __forceinline__ float rnd<float>(float v) { return v; }
template <>
__device__ __forceinline__ float rnd<bf16>(float v) { return round_bf16(v); }

// rnd<T> of VEC values in place, bf16 two to a conversion (v_cvt_pk_bf16_f32
// rounds both halves to nearest even, as the single conversion does).
template <typename T, int VEC>
__device__ __forceinline__ void rnd_vec(float* v) {
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int i = 0; i + 1 < VEC; i += 2) {
      const uint32_t w = pack_bf16x2(v[i], v[i + 1]);
      v[i] = bf16_lo(w);
      v[i + 1] = bf16_hi(w);
    }
    if constexpr (VEC & 1) v[VEC - 1] = round_bf16(v[VEC - 1]);
  }
}

// One token of the pool for VEC channels: each scan advanced over x, then
// pooled = T(...T(T(w_0 T(scan_0)) + T(w_1 T(scan_1)))...), every value's
// operations in the reference's order.
template <typename T, int VEC, int K>
__device__ __forceinline__ void pool_token(const float* xv, const float* a, const float* dec, const float* wk,
                                           float (&st)[K][VEC], float* out) {
#pragma unroll
  for (int k = 0; k < K; ++k) {
    float term[VEC];
#pragma unroll
    for (int i = 0; i < VEC; ++i) term[i] = st[k][i] = fmaf(a[k], xv[i], dec[k] * st[k][i]);
    rnd_vec<T, VEC>(term);
#pragma unroll
    for (int i = 0; i < VEC; ++i) term[i] *= wk[k];
    rnd_vec<T, VEC>(term);
    if (k == 0) {
#pragma unroll
      for (int i = 0; i < VEC; ++i) out[i] = term[i];
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) out[i] += term[i];
      rnd_vec<T, VEC>(out);
    }
  }
}

// Factor k clamped to [lo, hi] (one scalar EMA factor per scale, ema:274-277).
__device__ __forceinline__ float pk_alpha(const float* alpha, int k, const EmaGeom& g) {
  return fminf(fmaxf(alpha[k], g.lo), g.hi);
}

// ---- forward --------------------------------------------------------------
template <typename T, int VEC, int K>
__global__ __launch_bounds__(kEmaBlock) void packet_fwd_local(const T* __restrict__ x, int64_t sxb, int64_t sxn,
                                                             const float* __restrict__ alpha, float* __restrict__ ends,
                                                             EmaGeom g) {
  constexpr int R = kRows<T>;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * kEmaBlock + threadIdx.x;
  const int dv = tid % g.DV;
  const int c = (tid / g.DV) % g.NC;
  const int b = tid / (static_cast<int64_t>(g.DV) * g.NC);
  if (b >= g.B) return;
  const int d0 = dv * VEC;
  float a[K], st[K][VEC];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    a[k] = pk_alpha(alpha, k, g);
#pragma unroll
    for (int i = 0; i < VEC; ++i) st[k][i] = 0.f;
  }
  const int t0 = c * kChunkT;
  const int len = min(kChunkT, g.N - t0);
  const T* p = x + b * sxb + static_cast<int64_t>(t0) * sxn + d0;
  for (int tb = 0; tb < len; tb += R) {
    float xv[R][VEC];
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (tb + r < len) ldv<T, VEC>(p + static_cast<int64_t>(tb + r) * sxn, xv[r]);
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (tb + r < len) {
#pragma unroll
        for (int k = 0; k < K; ++k)
#pragma unroll
          for (int i = 0; i < VEC; ++i) st[k][i] = fmaf(a[k], xv[r][i], (1.f - a[k]) * st[k][i]);
      }
  }
  float* e = ends + (static_cast<int64_t>(b) * g.NC + c) * (K * g.D) + d0;
#pragma unroll
  for (int k = 0; k < K; ++k)
#pragma unroll
    for (int i = 0; i < VEC; ++i) e[k * g.D + i] = st[k][i];
}

template <typename T, int VEC, int K>
__global__ __launch_bounds__(kEmaBlock) void packet_fwd_apply(const T* __restrict__ x, int64_t sxb, int64_t sxn,
                                                             T* __restrict__ pooled, int64_t spb, int64_t spn,
                                                             const float* __restrict__ alpha,
                                                             const float* __restrict__ weight,
                                                             const float* __restrict__ state, EmaGeom g) {
  constexpr int R = kRows<T>;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * kEmaBlock + threadIdx.x;
  const int dv = tid % g.DV;
  const int c = (tid / g.DV) % g.NC;
  const int b = tid / (static_cast<int64_t>(g.DV) * g.NC);
  if (b >= g.B) return;
  const int d0 = dv * VEC;
  float a[K], wk[K], st[K][VEC];
  const float* cr = state + (static_cast<int64_t>(b) * g.NC + c) * (K * g.D) + d0;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    a[k] = pk_alpha(alpha, k, g);
    wk[k] = rnd<T>(weight[k]);
#pragma unroll
    for (int i = 0; i < VEC; ++i) st[k][i] = cr[k * g.D + i];
  }
  const int t0 = c * kChunkT;
  const int len = min(kChunkT, g.N - t0);
  const T* px = x + b * sxb + static_cast<int64_t>(t0) * sxn + d0;
  T* po = pooled + b * spb + static_cast<int64_t>(t0) * spn + d0;
  for (int tb = 0; tb < len; tb += R) {
    float xv[R][VEC];
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (tb + r < len) ldv<T, VEC>(px + static_cast<int64_t>(tb + r) * sxn, xv[r]);
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (tb + r < len) {
        float out[VEC];
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          float acc = 0.f;
#pragma unroll
          for (int k = 0; k < K; ++k) {
            st[k][i] = fmaf(a[k], xv[r][i], (1.f - a[k]) * st[k][i]);
            const float term = rnd<T>(wk[k] * rnd<T>(st[k][i]));
            acc = k == 0 ? term : rnd<T>(acc + term);
          }
          out[i] = acc;
        }
        stv<T, VEC>(po + static_cast<int64_t>(tb + r) * spn, out);
      }
  }
}

// ---- forward in one pass (decoupled look-back, ema_common.h) -------------
// The K scans of the pool in one pass over x with the EMA's look-back (its
// tiles, run walk and bounded waits; ema.hip describes them): a wave takes
// (b, 16 VEC channels, 128 tokens), lane (cg, ts) VEC channels of a 32-token
// segment held in registers; the segment scans of every scale compose into
// the tile's maps, and the workgroup's four tiles publish K aggregates per
// channel.  The rescan writes, at every 16-token chunk start, the K incoming
// states for the backward (state [B][NC][K][D], as the three-stage forward
// does) and, with POOLED, the pool with the reference's rounding of each
// scan, product and partial sum to T.  Every factor is one scalar per scale,
// so a tile's factor P_k is the same for all its channels.
template <typename T, int VEC, int K, bool POOLED>
__global__ __launch_bounds__(kWave * kLbWaves) void packet_fwd_lb(const T* __restrict__ x, int64_t sxb, int64_t sxn,
                                                                  T* __restrict__ pooled, int64_t spb, int64_t spn,
                                                                  const float* __restrict__ alpha,
                                                                  const float* __restrict__ weight,
                                                                  float* __restrict__ state, LbGeom g, int NC) {
  constexpr int SEG = kLbSeg;
  constexpr int CT = kLbGroups * VEC;
  __shared__ LbShared<K> sh;
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  const int cg = lane & 15, ts = lane >> 4;
  const int id = blockIdx.x;   // workgroups of lower index are dispatched first
  const int widx = id / g.S, slice = id - widx * g.S;
  const int chunk = widx * kLbWaves + w;   // a chunk past the last holds no tokens
  const int b = slice / g.CB, cb = slice - b * g.CB;
  const int d0 = (cb * kLbGroups + cg) * VEC;
  const bool dlive = d0 < g.D;
  const int s0 = (chunk * kLbSegs + ts) * SEG;
  const int len = max(0, min(SEG, g.N - s0));
  float a[K], dec[K], wk[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    a[k] = fminf(fmaxf(alpha[k], g.lo), g.hi);
    dec[k] = 1.f - a[k];
    wk[k] = rnd<T>(weight[k]);
  }
  const __amdgpu_buffer_rsrc_t rx = lb_rsrc(x, sxb, sxn, b, g.N);
  const uint32_t rsx = static_cast<uint32_t>(sxn * sizeof(T)), cox = static_cast<uint32_t>(d0 * sizeof(T));
  LbRaw<T, VEC> raw[SEG];
#pragma unroll
  for (int t = 0; t < SEG; ++t)
    raw[t].load(rx, t < len && dlive ? static_cast<uint32_t>(s0 + t) * rsx + cox : kOutOfRange);

  // 1. the segment from a zero state, every scale
  float L[K][VEC], A[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    A[k] = 1.f;
#pragma unroll
    for (int i = 0; i < VEC; ++i) L[k][i] = 0.f;
  }
#pragma unroll
  for (int t = 0; t < SEG; ++t) {
    if (t < len) {
      float v[VEC];
      raw[t].widen(v);
#pragma unroll
      for (int k = 0; k < K; ++k) {
#pragma unroll
        for (int i = 0; i < VEC; ++i) L[k][i] = fmaf(a[k], v[i], dec[k] * L[k][i]);
        A[k] *= dec[k];
      }
    }
  }
  // 2. the four segments of each channel in time order: the tile's (P, Q) and this lane's prefix
  float P[K], Q[K][VEC], Pp[K], Qp[K][VEC];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    P[k] = 1.f;
    Pp[k] = 1.f;
#pragma unroll
    for (int i = 0; i < VEC; ++i) { Q[k][i] = 0.f; Qp[k][i] = 0.f; }
  }
#pragma unroll
  for (int s = 0; s < kLbSegs; ++s) {
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const float As = __shfl(A[k], cg + 16 * s);
      Pp[k] = s == ts ? P[k] : Pp[k];
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        const float Ls = __shfl(L[k][i], cg + 16 * s);
        Qp[k][i] = s == ts ? Q[k][i] : Qp[k][i];
        Q[k][i] = fmaf(As, Q[k][i], Ls);
      }
      P[k] *= As;
    }
  }
  // 3-4. the channel this lane publishes (VEC 4: channel ts of the group; VEC 1: lanes ts = 0)
  const int io = VEC == 4 ? ts : 0;
  const bool owner = (VEC == 4 || ts == 0) && dlive && d0 + io < g.D;
  float Qo[K], full_wg[K], C[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    Qo[k] = VEC == 4 ? pick4(io, Q[k][0], Q[k][VEC > 1 ? 1 : 0], Q[k][VEC > 2 ? 2 : 0], Q[k][VEC > 3 ? 3 : 0])
                     : Q[k][0];
    float seg = 1.f, full = 1.f;   // a full tile's factor, composed as a tile composes its segments
    for (int t = 0; t < SEG; ++t) seg *= dec[k];
#pragma unroll
    for (int s = 0; s < kLbSegs; ++s) full *= seg;
    full_wg[k] = 1.f;
#pragma unroll
    for (int j = 0; j < kLbWaves; ++j) full_wg[k] *= full;
  }
  lb_join<K>(g, sh, slice, cg * VEC + io, owner, CT, widx, w, P, Qo, full_wg, C);
  // 5. incoming state of each channel of this lane's segment, then the rescan
  float st[K][VEC];
#pragma unroll
  for (int k = 0; k < K; ++k)
#pragma unroll
    for (int i = 0; i < VEC; ++i) st[k][i] = fmaf(Pp[k], __shfl(C[k], VEC == 4 ? cg + 16 * i : cg), Qp[k][i]);
  const __amdgpu_buffer_rsrc_t rp = lb_rsrc(pooled, spb, spn, b, g.N);
  const uint32_t rsp = static_cast<uint32_t>(spn * sizeof(T)), cop = static_cast<uint32_t>(d0 * sizeof(T));
#pragma unroll
  for (int t = 0; t < SEG; ++t) {
    if (t < len) {
      if ((t % kChunkT) == 0 && dlive) {   // the states entering chunk (s0 + t) / 16
        float* sr = state + ((static_cast<int64_t>(b) * NC + (s0 + t) / kChunkT) * K) * g.D + d0;
#pragma unroll
        for (int k = 0; k < K; ++k) {
          if constexpr (VEC == 4) {
            *reinterpret_cast<float4*>(sr + k * g.D) = make_float4(st[k][0], st[k][VEC > 1 ? 1 : 0],
                                                                   st[k][VEC > 2 ? 2 : 0], st[k][VEC > 3 ? 3 : 0]);
          } else {
            sr[k * g.D] = st[k][0];
          }
        }
      }
      float v[VEC];
      raw[t].widen(v);
      float out[VEC];
      pool_token<T, VEC, K>(v, a, dec, wk, st, out);
      if constexpr (POOLED) lb_store<T, VEC>(rp, dlive ? static_cast<uint32_t>(s0 + t) * rsp + cop : kOutOfRange, out);
    }
  }
}

// ---- backward -------------------------------------------------------------
template <typename T, int VEC, int K>
__global__ __launch_bounds__(kEmaBlock) void packet_bwd_local(const T* __restrict__ dp, int64_t sgb, int64_t sgn,
                                                             const float* __restrict__ alpha,
                                                             const float* __restrict__ weight,
                                                             float* __restrict__ starts, EmaGeom g) {
  constexpr int R = kRows<T>;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * kEmaBlock + threadIdx.x;
  const int dv = tid % g.DV;
  const int c = (tid / g.DV) % g.NC;
  const int b = tid / (static_cast<int64_t>(g.DV) * g.NC);
  if (b >= g.B) return;
  const int d0 = dv * VEC;
  float dec[K], wk[K], st[K][VEC];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    dec[k] = 1.f - pk_alpha(alpha, k, g);
    wk[k] = rnd<T>(weight[k]);
#pragma unroll
    for (int i = 0; i < VEC; ++i) st[k][i] = 0.f;
  }
  const int t0 = c * kChunkT;
  const int len = min(kChunkT, g.N - t0);
  const T* p = dp + b * sgb + static_cast<int64_t>(t0) * sgn + d0;
  for (int tb = len - 1; tb >= 0; tb -= R) {   // rows tb, tb-1, ..., tb-R+1
    float gv[R][VEC];
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (tb - r >= 0) ldv<T, VEC>(p + static_cast<int64_t>(tb - r) * sgn, gv[r]);
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (tb - r >= 0) {
#pragma unroll
        for (int k = 0; k < K; ++k)
#pragma unroll
          for (int i = 0; i < VEC; ++i) st[k][i] = fmaf(dec[k], st[k][i], rnd<T>(gv[r][i] * wk[k]));
      }
  }
  float* e = starts + (static_cast<int64_t>(b) * g.NC + c) * (K * g.D) + d0;
#pragma unroll
  for (int k = 0; k < K; ++k)
#pragma unroll
    for (int i = 0; i < VEC; ++i) e[k * g.D + i] = st[k][i];
}

// The chunk's scans kept between the forward recompute and the reverse pass:
// bf16 values two to a register, fp32 values one to a register.
template <typename T, int VEC>
struct ScanKeep;
template <>
struct ScanKeep<bf16, 2> {
  uint32_t w;
  __device__ __forceinline__ void put(const float* v) { w = pack_bf16x2(v[0], v[1]); }
  __device__ __forceinline__ float get(int i) const { return i == 0 ? bf16_lo(w) : bf16_hi(w); }
};
template <>
struct ScanKeep<bf16, 1> {
  float v0;
  __device__ __forceinline__ void put(const float* v) { v0 = v[0]; }
  __device__ __forceinline__ float get(int) const { return v0; }
};
template <>
struct ScanKeep<float, 1> {
  float v0;
  __device__ __forceinline__ void put(const float* v) { v0 = v[0]; }
  __device__ __forceinline__ float get(int) const { return v0; }
};

template <typename T, int VEC, int K>
__device__ __forceinline__ void packet_bwd_lane(
    const T* __restrict__ x, int64_t sxb, int64_t sxn, const T* __restrict__ dp, int64_t sgb, int64_t sgn,
    T* __restrict__ dx, int64_t sdb, int64_t sdn, const float* __restrict__ alpha, const float* __restrict__ weight,
    const float* __restrict__ state, const float* __restrict__ carries, const EmaGeom& g, int b, int c, int dv,
    float (&dw)[K], float (&dsum)[K]) {
  const int d0 = dv * VEC;
  const int t0 = c * kChunkT;
  const int len = min(kChunkT, g.N - t0);
  float a[K], wk[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    a[k] = pk_alpha(alpha, k, g);
    wk[k] = rnd<T>(weight[k]);
  }
  float xv[kChunkT][VEC], gv[kChunkT][VEC];
  const T* px = x + b * sxb + static_cast<int64_t>(t0) * sxn + d0;
  const T* pg = dp + b * sgb + static_cast<int64_t>(t0) * sgn + d0;
#pragma unroll
  for (int t = 0; t < kChunkT; ++t)
    if (t < len) {
      ldv<T, VEC>(px + static_cast<int64_t>(t) * sxn, xv[t]);
      ldv<T, VEC>(pg + static_cast<int64_t>(t) * sgn, gv[t]);
    }
  const int64_t srow = (static_cast<int64_t>(b) * g.NC + c) * (K * g.D) + d0;
  // forward in time: scan_k[t] of the chunk from its incoming state, and the
  // dweight partials
  float y[K][VEC], prev0[K][VEC];
  ScanKeep<T, VEC> keep[kChunkT][K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      y[k][i] = state[srow + k * g.D + i];
      prev0[k][i] = t0 > 0 ? rnd<T>(y[k][i]) : 0.f;   // scan_k[t0 - 1] as stored
    }
  }
#pragma unroll
  for (int t = 0; t < kChunkT; ++t)
    if (t < len) {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        float s[VEC];
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          y[k][i] = fmaf(a[k], xv[t][i], (1.f - a[k]) * y[k][i]);
          s[i] = rnd<T>(y[k][i]);
          dw[k] += rnd<T>(gv[t][i] * s[i]);
        }
        keep[t][k].put(s);
      }
    }
  // back in time: the adjoints, dx and the dalpha partials
  float lam[K][VEC], da[K][VEC];
#pragma unroll
  for (int k = 0; k < K; ++k)
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      lam[k][i] = carries[srow + k * g.D + i];
      da[k][i] = 0.f;
    }
  T* pd = dx + b * sdb + static_cast<int64_t>(t0) * sdn + d0;
#pragma unroll
  for (int t = kChunkT - 1; t >= 0; --t)
    if (t < len) {
      float out[VEC];
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < K; ++k) {
          lam[k][i] = fmaf(1.f - a[k], lam[k][i], rnd<T>(gv[t][i] * wk[k]));
          acc = fmaf(a[k], lam[k][i], acc);
          const float sprev = t > 0 ? keep[t > 0 ? t - 1 : 0][k].get(i) : prev0[k][i];
          da[k][i] = fmaf(lam[k][i], xv[t][i] - sprev, da[k][i]);
        }
        out[i] = acc;
      }
      stv<T, VEC>(pd + static_cast<int64_t>(t) * sdn, out);
    }
#pragma unroll
  for (int k = 0; k < K; ++k) {
    dsum[k] = da[k][0];
#pragma unroll
    for (int i = 1; i < VEC; ++i) dsum[k] += da[k][i];
  }
}

// One lane: VEC channels of one chunk, all of its rows in registers.  The
// lane's dweight and dalpha partials (every factor and weight is one scalar)
// are summed over the workgroup (wave butterflies, then the waves in order)
// into one slot per (quantity, workgroup): part[k] for dweight_k, part[K + k]
// for dalpha_k, each a row of gridDim.x slots.
template <typename T, int VEC, int K>
__global__ __launch_bounds__(kEmaBlock) void packet_bwd_apply(
    const T* __restrict__ x, int64_t sxb, int64_t sxn, const T* __restrict__ dp, int64_t sgb, int64_t sgn,
    T* __restrict__ dx, int64_t sdb, int64_t sdn, const float* __restrict__ alpha, const float* __restrict__ weight,
    const float* __restrict__ state, const float* __restrict__ carries, float* __restrict__ part, EmaGeom g) {
  __shared__ float s_p[kEmaBlock / kWave][2 * K];
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * kEmaBlock + threadIdx.x;
  const int dv = tid % g.DV;
  const int c = (tid / g.DV) % g.NC;
  const int b = tid / (static_cast<int64_t>(g.DV) * g.NC);
  float dw[K], dsum[K];
#pragma unroll
  for (int k = 0; k < K; ++k) dw[k] = dsum[k] = 0.f;
  if (b < g.B)
    packet_bwd_lane<T, VEC, K>(x, sxb, sxn, dp, sgb, sgn, dx, sdb, sdn, alpha, weight, state, carries, g, b, c, dv,
                               dw, dsum);
  const int w = threadIdx.x / kWave, l = threadIdx.x % kWave;
#pragma unroll
  for (int q = 0; q < 2 * K; ++q) {
    float v = q < K ? dw[q] : dsum[q - K];
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) v += __shfl_xor(v, o);
    if (l == 0) s_p[w][q] = v;
  }
  __syncthreads();
  if (threadIdx.x < 2 * K) {
    float t = 0.f;
    for (int v = 0; v < kEmaBlock / kWave; ++v) t += s_p[v][threadIdx.x];
    part[static_cast<int64_t>(threadIdx.x) * gridDim.x + blockIdx.x] = t;
  }
}

// Rounded scan values of VEC channels kept between the backward look-back's
// forward recompute and its reverse pass: bf16 four to two registers.
template <typename T, int VEC>
struct LbKeep {
  float v[VEC];
  __device__ __forceinline__ void put(const float* y, float* s) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) s[i] = v[i] = rnd<T>(y[i]);
  }
  __device__ __forceinline__ float get(int i) const { return v[i]; }
};
template <>
struct LbKeep<bf16, 4> {
  uint32_t w[2];
  __device__ __forceinline__ void put(const float* y, float* s) {
    w[0] = pack_bf16x2(y[0], y[1]);
    w[1] = pack_bf16x2(y[2], y[3]);
    s[0] = bf16_lo(w[0]); s[1] = bf16_hi(w[0]); s[2] = bf16_lo(w[1]); s[3] = bf16_hi(w[1]);
  }
  __device__ __forceinline__ float get(int i) const { return (i & 1) ? bf16_hi(w[i / 2]) : bf16_lo(w[i / 2]); }
};

// The pool's backward in one pass with the decoupled look-back, in reverse
// time (workgroup tile 0 holds the last tokens), where every [N][D] slab of
// x, dpooled and dx spans less than 2 GiB.  Lane (cg, ts) holds VEC channels
// of a 32-token segment:
//   1. the adjoints of the K scans over the segment from zero, on
//      dscan_k = T(dpooled w_k), and the segment's factor (1 - a_k)^len;
//   2-4. the segments' and tiles' maps composed as in the forward, K
//      aggregates per channel published and walked (lb_join), giving the
//      adjoint entering each segment from the tokens after it;
//   5. the segment again, KT tokens at a time from its end: the scans of
//      the KT tokens recomputed forward from the state entering their
//      16-token chunk (`state`, as the forward wrote it; a block that starts
//      inside a chunk recomputes from the chunk's start), each rounded to T
//      as the pool stored it and kept in registers, the dweight terms
//      T(dpooled scan_k) summed on the way, then the adjoints run back over
//      the block: dx = sum_k a_k lambda_k and the dalpha terms
//      lambda_k (x[t] - scan_k[t-1]).
// Each workgroup's dweight and dalpha sums (wave butterflies, then the waves
// in order) go to one slot per (quantity, workgroup): part[q * slots + id].
template <typename T, int VEC, int K, int KT, int SEG>
__global__ __launch_bounds__(kWave * kLbWaves) void packet_bwd_lb(
    const T* __restrict__ x, int64_t sxb, int64_t sxn, const T* __restrict__ dp, int64_t sgb, int64_t sgn,
    T* __restrict__ dx, int64_t sdb, int64_t sdn, const float* __restrict__ alpha, const float* __restrict__ weight,
    const float* __restrict__ state, float* __restrict__ part, LbGeom g, int NC) {
  constexpr int CT = kLbGroups * VEC;
  static_assert(kChunkT % KT == 0 && SEG % kChunkT == 0, "blocks tile the chunks");
  __shared__ LbShared<K> sh;
  __shared__ float s_p[kLbWaves][2 * K];
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  const int cg = lane & 15, ts = lane >> 4;
  const int id = blockIdx.x;   // workgroups of lower index are dispatched first
  const int widx = id / g.S, slice = id - widx * g.S;
  const int chunk = g.NCH - 1 - (widx * kLbWaves + w);   // a chunk below 0 holds no tokens
  const int b = slice / g.CB, cb = slice - b * g.CB;
  const int d0 = (cb * kLbGroups + cg) * VEC;
  const bool dlive = d0 < g.D;
  const int s0 = (chunk * kLbSegs + ts) * SEG;
  const int len = chunk < 0 ? 0 : max(0, min(SEG, g.N - s0));
  float a[K], dec[K], wk[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    a[k] = fminf(fmaxf(alpha[k], g.lo), g.hi);
    dec[k] = 1.f - a[k];
    wk[k] = rnd<T>(weight[k]);
  }
  const __amdgpu_buffer_rsrc_t rg = lb_rsrc(dp, sgb, sgn, b, g.N);
  const uint32_t rsg = static_cast<uint32_t>(sgn * sizeof(T)), cog = static_cast<uint32_t>(d0 * sizeof(T));

  // 1. the segment in reverse time from zero adjoints, every scale
  float L[K][VEC], A[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    A[k] = 1.f;
#pragma unroll
    for (int i = 0; i < VEC; ++i) L[k][i] = 0.f;
  }
  {
    LbRaw<T, VEC> raw[SEG];
#pragma unroll
    for (int t = 0; t < SEG; ++t)
      raw[t].load(rg, t < len && dlive ? static_cast<uint32_t>(s0 + t) * rsg + cog : kOutOfRange);
#pragma unroll
    for (int t = SEG - 1; t >= 0; --t) {
      if (t < len) {
        float v[VEC];
        raw[t].widen(v);
#pragma unroll
        for (int k = 0; k < K; ++k) {
          float gk[VEC];
#pragma unroll
          for (int i = 0; i < VEC; ++i) gk[i] = v[i] * wk[k];
          rnd_vec<T, VEC>(gk);
#pragma unroll
          for (int i = 0; i < VEC; ++i) L[k][i] = fmaf(dec[k], L[k][i], gk[i]);
          A[k] *= dec[k];
        }
      }
    }
  }
  // 2. the segments composed in reverse time order (3, 2, 1, 0): the tile's (P, Q) and this lane's prefix
  float P[K], Q[K][VEC], Pp[K], Qp[K][VEC];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    P[k] = 1.f;
    Pp[k] = 1.f;
#pragma unroll
    for (int i = 0; i < VEC; ++i) { Q[k][i] = 0.f; Qp[k][i] = 0.f; }
  }
#pragma unroll
  for (int s = kLbSegs - 1; s >= 0; --s) {
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const float As = __shfl(A[k], cg + 16 * s);
      Pp[k] = s == ts ? P[k] : Pp[k];
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        const float Ls = __shfl(L[k][i], cg + 16 * s);
        Qp[k][i] = s == ts ? Q[k][i] : Qp[k][i];
        Q[k][i] = fmaf(As, Q[k][i], Ls);
      }
      P[k] *= As;
    }
  }
  // 3-4. publish and walk back over the workgroups of later tokens
  const int io = VEC == 4 ? ts : 0;
  const bool owner = (VEC == 4 || ts == 0) && dlive && d0 + io < g.D;
  float Qo[K], full_wg[K], C[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    Qo[k] = VEC == 4 ? pick4(io, Q[k][0], Q[k][VEC > 1 ? 1 : 0], Q[k][VEC > 2 ? 2 : 0], Q[k][VEC > 3 ? 3 : 0])
                     : Q[k][0];
    float seg = 1.f, full = 1.f;   // a full tile's factor, composed as a tile composes its segments
    for (int t = 0; t < SEG; ++t) seg *= dec[k];
#pragma unroll
    for (int s = 0; s < kLbSegs; ++s) full *= seg;
    full_wg[k] = 1.f;
#pragma unroll
    for (int j = 0; j < kLbWaves; ++j) full_wg[k] *= full;
  }
  lb_join<K>(g, sh, slice, cg * VEC + io, owner, CT, widx, w, P, Qo, full_wg, C);
  // 5. the adjoints entering the segment from the tokens after it, then the blocks from the segment's end
  float lam[K][VEC], da[K][VEC], dw[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    dw[k] = 0.f;
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      lam[k][i] = fmaf(Pp[k], __shfl(C[k], VEC == 4 ? cg + 16 * i : cg), Qp[k][i]);
      da[k][i] = 0.f;
    }
  }
  const __amdgpu_buffer_rsrc_t rx = lb_rsrc(x, sxb, sxn, b, g.N);
  const __amdgpu_buffer_rsrc_t rd = lb_rsrc(dx, sdb, sdn, b, g.N);
  const uint32_t rsx = static_cast<uint32_t>(sxn * sizeof(T)), cox = static_cast<uint32_t>(d0 * sizeof(T));
  const uint32_t rsd = static_cast<uint32_t>(sdn * sizeof(T)), cod = static_cast<uint32_t>(d0 * sizeof(T));
#pragma unroll
  for (int u0 = SEG - KT; u0 >= 0; u0 -= KT) {
    if (u0 < len) {
      const int c0 = u0 / kChunkT * kChunkT;   // the block's chunk starts at token s0 + c0
      constexpr int R = kChunkT;               // rows c0 .. u0 + KT - 1 (at most one chunk)
      LbRaw<T, VEC> xr[R], gr[KT];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int t = c0 + r;
        if (t < u0 + KT)
          xr[r].load(rx, t < len && dlive ? static_cast<uint32_t>(s0 + t) * rsx + cox : kOutOfRange);
      }
#pragma unroll
      for (int r = 0; r < KT; ++r) {
        const int t = u0 + r;
        gr[r].load(rg, t < len && dlive ? static_cast<uint32_t>(s0 + t) * rsg + cog : kOutOfRange);
      }
      // the scans entering the chunk, as the forward kept them
      float y[K][VEC], prev[K][VEC];
      const int64_t srow = ((static_cast<int64_t>(b) * NC + (s0 + c0) / kChunkT) * K) * g.D + d0;
#pragma unroll
      for (int k = 0; k < K; ++k) {
        if constexpr (VEC == 4) {
          const float4 v = dlive ? *reinterpret_cast<const float4*>(state + srow + k * g.D) : make_float4(0, 0, 0, 0);
          y[k][0] = v.x; y[k][VEC > 1 ? 1 : 0] = v.y; y[k][VEC > 2 ? 2 : 0] = v.z; y[k][VEC > 3 ? 3 : 0] = v.w;
        } else {
          y[k][0] = dlive ? state[srow + k * g.D] : 0.f;
        }
#pragma unroll
        for (int i = 0; i < VEC; ++i) prev[k][i] = s0 + c0 > 0 ? rnd<T>(y[k][i]) : 0.f;   // scan_k[t - 1] as stored
      }
      // forward over rows c0 .. u0 + KT - 1, keeping the block's rounded scans
      LbKeep<T, VEC> keep[KT][K];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int t = c0 + r;
        if (t < u0 + KT && t < len) {
          float xv[VEC];
          xr[r].widen(xv);
#pragma unroll
          for (int k = 0; k < K; ++k) {
#pragma unroll
            for (int i = 0; i < VEC; ++i) y[k][i] = fmaf(a[k], xv[i], dec[k] * y[k][i]);
            if (t >= u0) {
              float sv[VEC];
              keep[t - u0 < 0 ? 0 : t - u0][k].put(y[k], sv);
            } else if (t == u0 - 1) {
#pragma unroll
              for (int i = 0; i < VEC; ++i) prev[k][i] = rnd<T>(y[k][i]);
            }
          }
        }
      }
      // back over the block: the dweight terms, the adjoints, dx and the dalpha terms
#pragma unroll
      for (int r = KT - 1; r >= 0; --r) {
        const int t = u0 + r;
        if (t < len) {
          float xv[VEC], gv[VEC], out[VEC], gk[K][VEC];
          xr[t - c0].widen(xv);
          gr[r].widen(gv);
#pragma unroll
          for (int k = 0; k < K; ++k) {
            float pr[VEC];
#pragma unroll
            for (int i = 0; i < VEC; ++i) {
              gk[k][i] = gv[i] * wk[k];
              pr[i] = gv[i] * keep[r][k].get(i);
            }
            rnd_vec<T, VEC>(gk[k]);
            rnd_vec<T, VEC>(pr);
#pragma unroll
            for (int i = 0; i < VEC; ++i) dw[k] += pr[i];
          }
#pragma unroll
          for (int i = 0; i < VEC; ++i) {
            float acc = 0.f;
#pragma unroll
            for (int k = 0; k < K; ++k) {
              lam[k][i] = fmaf(dec[k], lam[k][i], gk[k][i]);
              acc = fmaf(a[k], lam[k][i], acc);
              const float sprev = r > 0 ? keep[r > 0 ? r - 1 : 0][k].get(i) : prev[k][i];
              da[k][i] = fmaf(lam[k][i], xv[i] - sprev, da[k][i]);
            }
            out[i] = acc;
          }
          lb_store<T, VEC>(rd, dlive ? static_cast<uint32_t>(s0 + t) * rsd + cod : kOutOfRange, out);
        }
      }
    }
  }
  // the workgroup's sums: dweight_k (q = k) and dalpha_k (q = K + k)
#pragma unroll
  for (int q = 0; q < 2 * K; ++q) {
    float v;
    if (q < K) {
      v = dw[q];
    } else {
      v = da[q - K][0];
#pragma unroll
      for (int i = 1; i < VEC; ++i) v += da[q - K][i];
    }
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) v += __shfl_xor(v, o);
    if (lane == 0) s_p[w][q] = v;
  }
  __syncthreads();
  if (threadIdx.x < 2 * K) {
    float t = 0.f;
#pragma unroll
    for (int j = 0; j < kLbWaves; ++j) t += s_p[j][threadIdx.x];
    part[static_cast<int64_t>(threadIdx.x) * gridDim.x + id] = t;
  }
}

// Row q of the per-workgroup partials, summed in a fixed order (thread i adds
// slots i, i + 1024, ... in order, the wave by a fixed butterfly, the waves in
// wave order): dweight_k = T(row k), as a sum-reduction in T returns it;
// dalpha_k = row K + k with the projected-clamp rule of ema:357-364.
template <typename T>
__global__ __launch_bounds__(kPkRedThreads) void packet_param_reduce(const float* __restrict__ part, int64_t slots,
                                                                    int K, const float* __restrict__ alpha,
                                                                    float* __restrict__ dweight,
                                                                    float* __restrict__ dalpha, EmaGeom g) {
  constexpr int kWaves = kPkRedThreads / kWave;
  __shared__ float s_w[kWaves];
  const int q = blockIdx.x;
  const float* src = part + q * slots;
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < slots; i += kPkRedThreads) s += src[i];
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) s += __shfl_xor(s, o);
  if (threadIdx.x % kWave == 0) s_w[threadIdx.x / kWave] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.f;
    for (int v = 0; v < kWaves; ++v) t += s_w[v];
    if (q < K) {
      if (dweight) dweight[q] = rnd<T>(t);
    } else if (dalpha) {
      const float ai = alpha[q - K];
      const bool blocked = (ai <= g.lo && t > 0.f) || (ai >= g.hi && t < 0.f);
      dalpha[q - K] = blocked ? 0.f : t;
    }
  }
}

// ---- packet: RMS direction, confidence and gate (train:268-273) -----------
// Per token, with u the stored pooled values and s = sigmoid(gate logit):
//   ms = mean_d u^2,   r = rsqrt(ms + 1e-6),   conf = tanh(sqrt(ms) / 0.25)
//   packet = G(((u r) conf) s)                 (G: the packet's dtype)
// packet_fwd_rows takes one workgroup per (batch row, 16-token chunk) with
// its lanes over all D channels (VEC each): it reads the chunk's pooled rows
// as the look-back forward stored them (or, with RESCAN, rescans the chunk
// from its incoming states as the pool's apply stage and stores pooled), so
// the 16 tokens' ms are one two-level LDS sum (fixed order) away.
constexpr int kPkRowMaxThreads = 1024;
constexpr float kPkEps = 1e-6f;
constexpr float kPkConfScale = 0.25f;

// sigmoid(z) = 1 / (1 + e^-z) with the hardware reciprocal (v_rcp_f32, about
// one ulp): a few fp32 ulps in all, against the ten-instruction correctly
// rounded division.  e^-z = inf gives 0 and e^-z = 0 gives 1.
__device__ __forceinline__ float pk_sigmoid(float z) { return __builtin_amdgcn_rcpf(1.f + __expf(-z)); }

// Sum of row r of s_red ([16][nt + 1]: rows padded by one word, so the
// sixteen rows a wave's level-1 reads span sit in different banks) in a
// fixed order: level 1 adds 16 entries per (row, quarter-block), level 2
// adds the nt / 16 partials of each row.  Every thread of the block calls
// it; returns the 16 sums in s_out.
__device__ __forceinline__ void pk_rows_sum(float* s_red, float* s_mid, float* s_out) {
  const int nt = blockDim.x, q = nt / 16;
  __syncthreads();
  {
    const int r = threadIdx.x & 15, part = threadIdx.x >> 4;
    const float* src = s_red + r * (nt + 1) + part * 16;
    float sum = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) sum += src[e];
    s_mid[r * q + part] = sum;
  }
  __syncthreads();
  if (threadIdx.x < 16) {
    float sum = 0.f;
    for (int part = 0; part < q; ++part) sum += s_mid[threadIdx.x * q + part];
    s_out[threadIdx.x] = sum;
  }
  __syncthreads();
}

template <typename T, typename G, int VEC, int K, bool RESCAN>
__global__ __launch_bounds__(kPkRowMaxThreads) void packet_fwd_rows(
    const T* __restrict__ x, int64_t sxb, int64_t sxn, T* __restrict__ pooled, int64_t spb, int64_t spn,
    const G* __restrict__ gate, int64_t sgb, int64_t sgn, G* __restrict__ packet, int64_t sqb, int64_t sqn,
    float* __restrict__ ms, const float* __restrict__ alpha, const float* __restrict__ weight,
    const float* __restrict__ state, EmaGeom g) {
  extern __shared__ float s_pk[];
  float* s_red = s_pk;                                // [16][nt + 1]
  float* s_mid = s_red + kChunkT * (blockDim.x + 1);  // [16][nt / 16]
  float* s_ms = s_mid + blockDim.x;             // [16]
  const int c = blockIdx.x % g.NC, b = blockIdx.x / g.NC;
  const int dv = threadIdx.x;
  const bool live = dv < g.DV;
  const int d0 = dv * VEC;
  const int t0 = c * kChunkT;
  const int len = min(kChunkT, g.N - t0);
  float u[kChunkT][VEC];
#pragma unroll
  for (int t = 0; t < kChunkT; ++t)
#pragma unroll
    for (int i = 0; i < VEC; ++i) u[t][i] = 0.f;
  if (live && !RESCAN) {   // pooled as the look-back forward stored it
    const T* po = pooled + b * spb + static_cast<int64_t>(t0) * spn + d0;
#pragma unroll
    for (int t = 0; t < kChunkT; ++t)
      if (t < len) ldv<T, VEC>(po + static_cast<int64_t>(t) * spn, u[t]);
  }
  if (live && RESCAN) {
    float a[K], dec[K], wk[K], st[K][VEC];
    const float* cr = state + (static_cast<int64_t>(b) * g.NC + c) * (K * g.D) + d0;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      a[k] = pk_alpha(alpha, k, g);
      dec[k] = 1.f - a[k];
      wk[k] = rnd<T>(weight[k]);
#pragma unroll
      for (int i = 0; i < VEC; ++i) st[k][i] = cr[k * g.D + i];
    }
    const T* px = x + b * sxb + static_cast<int64_t>(t0) * sxn + d0;
    T* po = pooled + b * spb + static_cast<int64_t>(t0) * spn + d0;
    float xv[kChunkT][VEC];
#pragma unroll
    for (int t = 0; t < kChunkT; ++t)
      if (t < len) ldv<T, VEC>(px + static_cast<int64_t>(t) * sxn, xv[t]);
#pragma unroll
    for (int t = 0; t < kChunkT; ++t)
      if (t < len) {
        pool_token<T, VEC, K>(xv[t], a, dec, wk, st, u[t]);
        stv<T, VEC>(po + static_cast<int64_t>(t) * spn, u[t]);
      }
  }
#pragma unroll
  for (int t = 0; t < kChunkT; ++t) {
    float sq = 0.f;
#pragma unroll
    for (int i = 0; i < VEC; ++i) sq = fmaf(u[t][i], u[t][i], sq);
    s_red[t * (blockDim.x + 1) + threadIdx.x] = sq;
  }
  pk_rows_sum(s_red, s_mid, s_ms);
  const float inv_d = 1.f / static_cast<float>(g.D);
  if (threadIdx.x < 16 && threadIdx.x < len) ms[static_cast<int64_t>(b) * g.N + t0 + threadIdx.x] = s_ms[threadIdx.x] * inv_d;
  if (!live) return;
  const G* pg = gate + b * sgb + static_cast<int64_t>(t0) * sgn + d0;
  G* pq = packet + b * sqb + static_cast<int64_t>(t0) * sqn + d0;
#pragma unroll
  for (int t = 0; t < kChunkT; ++t)
    if (t < len) {
      const float m = s_ms[t] * inv_d;
      const float r = rsqrtf(m + kPkEps);
      const float conf = tanhf(sqrtf(m) / kPkConfScale);
      float gl[VEC], out[VEC];
      ldv<G, VEC>(pg + static_cast<int64_t>(t) * sgn, gl);
#pragma unroll
      for (int i = 0; i < VEC; ++i) out[i] = ((u[t][i] * r) * conf) * pk_sigmoid(gl[i]);
      stv<G, VEC>(pq + static_cast<int64_t>(t) * sqn, out);
    }
}

// Backward of the packet for KPB tokens per workgroup, lanes over channels.
// With A = u r conf and S = sum_d G_d s_d u_d (G = dpacket):
//   dgate = G(dpacket A s (1 - s))
//   dms   = -0.5 r^3 conf S  +  r S (1 - conf^2) / 0.25 / (2 sqrt(ms))
//   dpooled = T(dpacket s r conf + dms 2 u / D)
// (the chain autograd forms for train:268-273; sqrt(ms) = 0 gives NaN there
// as it does in the reference).  dpooled goes to the pool's backward.
constexpr int kPkBwdTokens = 4;

template <typename T, typename G, int VEC>
__global__ __launch_bounds__(kPkRowMaxThreads) void packet_bwd_rows(
    const T* __restrict__ pooled, int64_t spb, int64_t spn, const float* __restrict__ ms,
    const G* __restrict__ gate, int64_t sgb, int64_t sgn, const G* __restrict__ dpacket, int64_t sdb, int64_t sdn,
    T* __restrict__ dpooled, int64_t sab, int64_t san, G* __restrict__ dgate, int64_t seb, int64_t sen, EmaGeom g) {
  __shared__ float s_red[kPkBwdTokens][kPkRowMaxThreads / kWave];
  __shared__ float s_sum[kPkBwdTokens];
  const int groups = (g.N + kPkBwdTokens - 1) / kPkBwdTokens;
  const int tg = blockIdx.x % groups, b = blockIdx.x / groups;
  const int t0 = tg * kPkBwdTokens;
  const int len = min(kPkBwdTokens, g.N - t0);
  const int dv = threadIdx.x;
  const bool live = dv < g.DV;
  const int d0 = dv * VEC;
  float u[kPkBwdTokens][VEC], dp[kPkBwdTokens][VEC], sg[kPkBwdTokens][VEC];
  float part[kPkBwdTokens];
#pragma unroll
  for (int t = 0; t < kPkBwdTokens; ++t) {
    part[t] = 0.f;
#pragma unroll
    for (int i = 0; i < VEC; ++i) u[t][i] = dp[t][i] = sg[t][i] = 0.f;
    if (live && t < len) {
      const int64_t n = t0 + t;
      float gl[VEC];
      ldv<T, VEC>(pooled + b * spb + n * spn + d0, u[t]);
      ldv<G, VEC>(gate + b * sgb + n * sgn + d0, gl);
      ldv<G, VEC>(dpacket + b * sdb + n * sdn + d0, dp[t]);
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        sg[t][i] = pk_sigmoid(gl[i]);
        part[t] = fmaf(dp[t][i] * sg[t][i], u[t][i], part[t]);
      }
    }
  }
  // S per token: wave sums (fixed butterfly), then the waves in order
  const int w = threadIdx.x / kWave, l = threadIdx.x % kWave;
#pragma unroll
  for (int t = 0; t < kPkBwdTokens; ++t) {
    float v = part[t];
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) v += __shfl_xor(v, o);
    if (l == 0) s_red[t][w] = v;
  }
  __syncthreads();
  if (threadIdx.x < kPkBwdTokens) {
    float sum = 0.f;
    for (int v = 0; v < static_cast<int>(blockDim.x) / kWave; ++v) sum += s_red[threadIdx.x][v];
    s_sum[threadIdx.x] = sum;
  }
  __syncthreads();
  if (!live) return;
  const float two_over_d = 2.f / static_cast<float>(g.D);
#pragma unroll
  for (int t = 0; t < kPkBwdTokens; ++t)
    if (t < len) {
      const int64_t n = t0 + t;
      const float m = ms[static_cast<int64_t>(b) * g.N + n];
      const float r = rsqrtf(m + kPkEps);
      const float rms = sqrtf(m);
      const float conf = tanhf(rms / kPkConfScale);
      const float S = s_sum[t];
      const float dconf = r * S, dr = conf * S;
      const float dms = dr * (-0.5f * r * r * r) + (dconf * (1.f - conf * conf) / kPkConfScale) / (2.f * rms);
      float du[VEC], dgl[VEC];
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        const float A = (u[t][i] * r) * conf;
        du[i] = ((dp[t][i] * sg[t][i]) * conf) * r + dms * two_over_d * u[t][i];
        dgl[i] = ((dp[t][i] * A) * (1.f - sg[t][i])) * sg[t][i];
      }
      stv<T, VEC>(dpooled + b * sab + n * san + d0, du);
      stv<G, VEC>(dgate + b * seb + n * sen + d0, dgl);
    }
}

inline int pk_nc(int N) { return (N + kChunkT - 1) / kChunkT; }

inline size_t pk_state_floats(int B, int N, int D, int K) {
  return static_cast<size_t>(B) * pk_nc(N) * D * K;
}

inline size_t pk_round256(size_t n) { return (n + 255) / 256 * 256; }

// The look-back backward's workspace: the head, the words of K scales, then
// 2K slots per workgroup.
inline size_t pk_lb_bwd_ws(int B, int N, int D, int K, int vec, int seg) {
  const LbPlan p = lb_plan(B, N, D, vec, seg, K);
  return kLbHead + pk_round256(p.words_bytes) + 2 * static_cast<size_t>(K) * p.NWG * p.S * sizeof(float);
}

// The pool backward's workspace: the three-stage backward's starts and
// carries (K*D per chunk each) and 2K slots per apply workgroup (a lane
// takes at least one (chunk, channel) pair, so at most ceil(B*NC*D / 256)
// workgroups), or the look-back's (four channels or one per lane), whichever
// is largest.
inline size_t pk_pool_bwd_ws(int B, int N, int D, int K) {
  const size_t pairs = static_cast<size_t>(B) * pk_nc(N) * D;
  size_t n = (2 * pk_state_floats(B, N, D, K) + 2 * static_cast<size_t>(K) * ((pairs + kEmaBlock - 1) / kEmaBlock)) *
             sizeof(float);
  n = std::max(n, pk_lb_bwd_ws(B, N, D, K, 1, kPkLbSeg));
  return std::max(n, pk_lb_bwd_ws(B, N, D, K, 4, kPkLbSeg));
}

// The look-back geometry of a pool scan (K scales' words after the head of ws).
inline LbGeom pk_lb_geom(int B, int N, int D, int K, float lo, float hi, void* ws, const LbPlan& p) {
  LbGeom g{};
  g.B = B; g.N = N; g.D = D;
  g.CB = p.CB; g.NCH = p.NCH; g.NWG = p.NWG; g.S = p.S;
  g.lo = lo; g.hi = hi;
  g.words = reinterpret_cast<unsigned long long*>(static_cast<char*>(ws) + kLbHead);
  g.runs = g.words + K * p.kw;
  g.kw = p.kw;
  g.kr = p.kr;
  g.wait_limit = kLbWaitLimit;
  return g;
}

// The geometry of the x-shaped stages (D channels, VEC per lane).
inline EmaGeom pk_geom(int B, int N, int D, int vec, float lo, float hi) {
  EmaGeom g = make_geom(B, N, D, vec, 0, lo, hi, nullptr, nullptr, nullptr, 0);
  g.cut = nullptr;
  return g;
}

// The carry stage's geometry: K*D scale-major channels, factor k for
// channels [k D, (k + 1) D).
inline EmaGeom pk_carry_geom(int B, int N, int D, int K, float lo, float hi) {
  EmaGeom g = make_geom(B, N, K * D, 1, 1, lo, hi, nullptr, nullptr, nullptr, 0);
  g.alpha_div = D;
  g.cut = nullptr;
  return g;
}

// The forward in one pass where every [N][D] slab of x and pooled spans less
// than 2 GiB (32-bit buffer offsets): the words' zeroing launch, then
// packet_fwd_lb (states, and with POOLED the pool).  False: the three-stage
// forward runs instead.
template <typename T, int VEC, int K, bool POOLED>
bool pk_fwd_lookback(const dwarf_packet_pool_fwd_args& a, hipStream_t stream) {
  if (!lb_fits(a.N, a.x_stride[1], sizeof(T)) || (POOLED && !lb_fits(a.N, a.pooled_stride[1], sizeof(T))))
    return false;
  const LbPlan p = lb_plan(a.B, a.N, a.D, VEC, kLbSeg, K);
  const LbGeom g = pk_lb_geom(a.B, a.N, a.D, K, a.floor_, a.ceiling, a.workspace, p);
  lb_zero(g, p, stream);
  hipLaunchKernelGGL((packet_fwd_lb<T, VEC, K, POOLED>), dim3(p.NWG * p.S), dim3(kWave * kLbWaves), 0, stream,
                     static_cast<const T*>(a.x), a.x_stride[0], a.x_stride[1], static_cast<T*>(a.pooled),
                     POOLED ? a.pooled_stride[0] : 0, POOLED ? a.pooled_stride[1] : 0, a.alpha, a.weight, a.state, g,
                     pk_nc(a.N));
  return true;
}

// The forward's local and carry stages: each chunk's incoming scan states in `state`.
template <typename T, int VEC, int K>
void pk_fwd_states(const dwarf_packet_pool_fwd_args& a, const EmaGeom& g, hipStream_t stream) {
  if (pk_fwd_lookback<T, VEC, K, false>(a, stream)) return;
  float* ends = static_cast<float*>(a.workspace);
  const int64_t lanes = static_cast<int64_t>(a.B) * g.NC * g.DV;
  const int blocks = static_cast<int>((lanes + kEmaBlock - 1) / kEmaBlock);
  hipLaunchKernelGGL((packet_fwd_local<T, VEC, K>), dim3(blocks), dim3(kEmaBlock), 0, stream,
                     static_cast<const T*>(a.x), a.x_stride[0], a.x_stride[1], a.alpha, ends, g);
  const EmaGeom gc = pk_carry_geom(a.B, a.N, a.D, K, a.floor_, a.ceiling);
  launch_carry<false, false>(ends, a.state, a.alpha, gc, a.B, K * a.D, stream);
}

template <typename T, int VEC, int K>
void pk_fwd_typed(const dwarf_packet_pool_fwd_args& a, hipStream_t stream) {
  if (pk_fwd_lookback<T, VEC, K, true>(a, stream)) return;
  const EmaGeom g = pk_geom(a.B, a.N, a.D, VEC, a.floor_, a.ceiling);
  pk_fwd_states<T, VEC, K>(a, g, stream);
  const int64_t lanes = static_cast<int64_t>(a.B) * g.NC * g.DV;
  const int blocks = static_cast<int>((lanes + kEmaBlock - 1) / kEmaBlock);
  hipLaunchKernelGGL((packet_fwd_apply<T, VEC, K>), dim3(blocks), dim3(kEmaBlock), 0, stream,
                     static_cast<const T*>(a.x), a.x_stride[0], a.x_stride[1], static_cast<T*>(a.pooled),
                     a.pooled_stride[0], a.pooled_stride[1], a.alpha, a.weight, a.state, g);
}

inline int pk_row_threads(int DV) { return (DV + kWave - 1) / kWave * kWave; }

// The packet's forward: the pool by the look-back pass (pooled and the chunk
// states), then packet_fwd_rows on the stored pooled; for slabs over 2 GiB
// the three-stage chunk states, then packet_fwd_rows rescanning each chunk.
template <typename T, typename G, int VEC, int K>
void pkt_fwd_typed(const dwarf_packet_fwd_args& p, hipStream_t stream) {
  const dwarf_packet_pool_fwd_args& a = p.pool;
  const EmaGeom g = pk_geom(a.B, a.N, a.D, VEC, a.floor_, a.ceiling);
  const bool pooled_done = pk_fwd_lookback<T, VEC, K, true>(a, stream);
  if (!pooled_done) pk_fwd_states<T, VEC, K>(a, g, stream);
  const int nt = pk_row_threads(g.DV);
  const size_t lds = static_cast<size_t>(kChunkT * (nt + 1) + nt + 16) * sizeof(float);
  auto rows = pooled_done ? packet_fwd_rows<T, G, VEC, K, false> : packet_fwd_rows<T, G, VEC, K, true>;
  hipLaunchKernelGGL(rows, dim3(a.B * g.NC), dim3(nt), lds, stream,
                     static_cast<const T*>(a.x), a.x_stride[0], a.x_stride[1], static_cast<T*>(a.pooled),
                     a.pooled_stride[0], a.pooled_stride[1], static_cast<const G*>(p.gate), p.gate_stride[0],
                     p.gate_stride[1], static_cast<G*>(p.packet), p.packet_stride[0], p.packet_stride[1], p.ms,
                     a.alpha, a.weight, a.state, g);
}

// The backward in one pass where every [N][D] slab of x, dpooled and dx spans
// less than 2 GiB: the words' zeroing launch, packet_bwd_lb, then the
// parameter sums over its workgroups' slots.  False: the three-stage
// backward runs instead.
template <typename T, int VEC, int K, int KT, int SEG>
bool pk_bwd_lookback(const dwarf_packet_pool_bwd_args& a, hipStream_t stream) {
  const dwarf_packet_pool_fwd_args& f = a.fwd;
  if (!lb_fits(f.N, f.x_stride[1], sizeof(T)) || !lb_fits(f.N, a.dpooled_stride[1], sizeof(T)) ||
      !lb_fits(f.N, a.dx_stride[1], sizeof(T)))
    return false;
  const LbPlan p = lb_plan(f.B, f.N, f.D, VEC, SEG, K);
  const LbGeom g = pk_lb_geom(f.B, f.N, f.D, K, f.floor_, f.ceiling, a.workspace, p);
  float* part = reinterpret_cast<float*>(static_cast<char*>(a.workspace) + kLbHead + pk_round256(p.words_bytes));
  const int slots = p.NWG * p.S;
  lb_zero(g, p, stream);
  hipLaunchKernelGGL((packet_bwd_lb<T, VEC, K, KT, SEG>), dim3(slots), dim3(kWave * kLbWaves), 0, stream,
                     static_cast<const T*>(f.x), f.x_stride[0], f.x_stride[1], static_cast<const T*>(a.dpooled),
                     a.dpooled_stride[0], a.dpooled_stride[1], static_cast<T*>(a.dx), a.dx_stride[0], a.dx_stride[1],
                     f.alpha, f.weight, f.state, part, g, pk_nc(f.N));
  if (a.dalpha || a.dweight) {
    const EmaGeom ga = pk_geom(f.B, f.N, f.D, 1, f.floor_, f.ceiling);
    hipLaunchKernelGGL((packet_param_reduce<T>), dim3(2 * K), dim3(kPkRedThreads), 0, stream, part,
                       static_cast<int64_t>(slots), K, f.alpha, a.dweight, a.dalpha, ga);
  }
  return true;
}


template <typename T, int VEC, int VA, int K>
void pk_bwd_typed(const dwarf_packet_pool_bwd_args& a, hipStream_t stream) {
  // four channels per lane up to three scales (four scales there overflow the registers into scratch
  // memory), else one
  constexpr int LBV = VEC == 4 && K <= 3 ? 4 : 1;
  if (pk_bwd_lookback<T, LBV, K, LBV == 4 ? pk_lb_keep<T>() : kChunkT, kPkLbSeg>(a, stream)) return;
  const dwarf_packet_pool_fwd_args& f = a.fwd;
  const size_t nf = pk_state_floats(f.B, f.N, f.D, K);
  float* starts = static_cast<float*>(a.workspace);
  float* carries = starts + nf;
  float* part = carries + nf;   // 2K rows of one slot per apply workgroup
  const EmaGeom g = pk_geom(f.B, f.N, f.D, VEC, f.floor_, f.ceiling);
  const int64_t lanes = static_cast<int64_t>(f.B) * g.NC * g.DV;
  const int blocks = static_cast<int>((lanes + kEmaBlock - 1) / kEmaBlock);
  hipLaunchKernelGGL((packet_bwd_local<T, VEC, K>), dim3(blocks), dim3(kEmaBlock), 0, stream,
                     static_cast<const T*>(a.dpooled), a.dpooled_stride[0], a.dpooled_stride[1], f.alpha, f.weight,
                     starts, g);
  const EmaGeom gc = pk_carry_geom(f.B, f.N, f.D, K, f.floor_, f.ceiling);
  launch_carry<true, false>(starts, carries, f.alpha, gc, f.B, K * f.D, stream);
  const EmaGeom ga = pk_geom(f.B, f.N, f.D, VA, f.floor_, f.ceiling);
  const int64_t alanes = static_cast<int64_t>(f.B) * ga.NC * ga.DV;
  const int ablocks = static_cast<int>((alanes + kEmaBlock - 1) / kEmaBlock);
  hipLaunchKernelGGL((packet_bwd_apply<T, VA, K>), dim3(ablocks), dim3(kEmaBlock), 0, stream,
                     static_cast<const T*>(f.x), f.x_stride[0], f.x_stride[1], static_cast<const T*>(a.dpooled),
                     a.dpooled_stride[0], a.dpooled_stride[1], static_cast<T*>(a.dx), a.dx_stride[0], a.dx_stride[1],
                     f.alpha, f.weight, f.state, carries, part, ga);
  if (a.dalpha || a.dweight)
    hipLaunchKernelGGL((packet_param_reduce<T>), dim3(2 * K), dim3(kPkRedThreads), 0, stream, part,
                       static_cast<int64_t>(ablocks), K, f.alpha, a.dweight, a.dalpha, ga);
}

template <typename T, int VEC, int VA>
void pk_fwd_k(const dwarf_packet_pool_fwd_args& a, hipStream_t s) {
  switch (a.K) {
    case 1: pk_fwd_typed<T, VEC, 1>(a, s); break;
    case 2: pk_fwd_typed<T, VEC, 2>(a, s); break;
    case 3: pk_fwd_typed<T, VEC, 3>(a, s); break;
    default: pk_fwd_typed<T, VEC, 4>(a, s); break;
  }
}

template <typename T, int VEC, int VA>
void pk_bwd_k(const dwarf_packet_pool_bwd_args& a, hipStream_t s) {
  switch (a.fwd.K) {
    case 1: pk_bwd_typed<T, VEC, VA, 1>(a, s); break;
    case 2: pk_bwd_typed<T, VEC, VA, 2>(a, s); break;
    case 3: pk_bwd_typed<T, VEC, VA, 3>(a, s); break;
    default: pk_bwd_typed<T, VEC, VA, 4>(a, s); break;
  }
}

template <typename T, typename G, int VEC, int VA>
void pkt_fwd_k(const dwarf_packet_fwd_args& a, hipStream_t s) {
  switch (a.pool.K) {
    case 1: pkt_fwd_typed<T, G, VEC, 1>(a, s); break;
    case 2: pkt_fwd_typed<T, G, VEC, 2>(a, s); break;
    case 3: pkt_fwd_typed<T, G, VEC, 3>(a, s); break;
    default: pkt_fwd_typed<T, G, VEC, 4>(a, s); break;
  }
}

// The packet's backward: dpooled (into the workspace after the pool's part)
// and dgate from the rows kernel, then the pool's backward on that dpooled.
template <typename T, typename G, int VEC, int VA>
void pkt_bwd_k(const dwarf_packet_bwd_args& p, hipStream_t s) {
  const dwarf_packet_pool_fwd_args& f = p.fwd.pool;
  const EmaGeom g = pk_geom(f.B, f.N, f.D, VEC, f.floor_, f.ceiling);
  const size_t pool_ws = (pk_pool_bwd_ws(f.B, f.N, f.D, f.K) + 255) / 256 * 256;
  T* dpooled = reinterpret_cast<T*>(static_cast<char*>(p.workspace) + pool_ws);
  const int64_t dsn = f.D, dsb = static_cast<int64_t>(f.N) * f.D;
  const int nt = pk_row_threads(g.DV);
  const int groups = (f.N + kPkBwdTokens - 1) / kPkBwdTokens;
  hipLaunchKernelGGL((packet_bwd_rows<T, G, VEC>), dim3(f.B * groups), dim3(nt), 0, s,
                     static_cast<const T*>(f.pooled), f.pooled_stride[0], f.pooled_stride[1], p.fwd.ms,
                     static_cast<const G*>(p.fwd.gate), p.fwd.gate_stride[0], p.fwd.gate_stride[1],
                     static_cast<const G*>(p.dpacket), p.dpacket_stride[0], p.dpacket_stride[1], dpooled, dsb, dsn,
                     static_cast<G*>(p.dgate), p.dgate_stride[0], p.dgate_stride[1], g);
  dwarf_packet_pool_bwd_args pb{};
  pb.fwd = f;
  pb.dpooled = dpooled;
  pb.dpooled_stride[0] = dsb; pb.dpooled_stride[1] = dsn; pb.dpooled_stride[2] = 1;
  pb.dx = p.dx;
  for (int i = 0; i < 3; ++i) pb.dx_stride[i] = p.dx_stride[i];
  pb.dalpha = p.dalpha;
  pb.dweight = p.dweight;
  pb.workspace = p.workspace;
  pb.workspace_bytes = pool_ws;
  pk_bwd_k<T, VEC, VA>(pb, s);
}

}  // namespace

size_t packet_state_bytes(int B, int N, int D, int K) { return pk_state_floats(B, N, D, K) * sizeof(float); }
// The three-stage forward's chunk ends, or the look-back's words, whichever is larger.
size_t packet_fwd_workspace(int B, int N, int D, int K) {
  const size_t chunked = pk_state_floats(B, N, D, K) * sizeof(float);
  const size_t lb = kLbHead + lb_plan(B, N, D, D % 4 == 0 ? 4 : 1, kLbSeg, K).words_bytes;
  return chunked > lb ? chunked : lb;
}
size_t packet_bwd_workspace(int B, int N, int D, int K) { return pk_pool_bwd_ws(B, N, D, K); }
// The pool's backward workspace, then dpooled [B,N,D] of the pool dtype.
size_t interference_packet_bwd_workspace(int B, int N, int D, int K, int dtype) {
  return (pk_pool_bwd_ws(B, N, D, K) + 255) / 256 * 256 +
         static_cast<size_t>(B) * N * D * (dtype == DWARF_BF16 ? 2 : 4);
}
// A row's channels are the lanes of one workgroup: 4 per lane when D % 4 == 0.
int packet_max_row_channels(int D) { return D % 4 == 0 ? kPkRowMaxThreads * 4 : kPkRowMaxThreads; }
int packet_max_scales() { return kMaxScales; }

// Lanes take 4 channels in the streaming stages when D % 4 == 0 (rows are
// then 8- or 16-byte aligned, checked on the host); the backward apply keeps
// a whole chunk per lane and takes 2 bf16 or 1 fp32 channel.
hipError_t launch_packet_fwd(const dwarf_packet_pool_fwd_args& a, hipStream_t stream) {
  const bool vec4 = (a.D % 4) == 0;
  if (a.dtype == DWARF_BF16) {
    if (vec4) pk_fwd_k<bf16, 4, 2>(a, stream);
    else pk_fwd_k<bf16, 1, 1>(a, stream);
  } else {
    if (vec4) pk_fwd_k<float, 4, 1>(a, stream);
    else pk_fwd_k<float, 1, 1>(a, stream);
  }
  return hipGetLastError();
}

hipError_t launch_packet_bwd(const dwarf_packet_pool_bwd_args& a, hipStream_t stream) {
  const bool vec4 = (a.fwd.D % 4) == 0;
  if (a.fwd.dtype == DWARF_BF16) {
    if (vec4) pk_bwd_k<bf16, 4, 2>(a, stream);
    else pk_bwd_k<bf16, 1, 1>(a, stream);
  } else {
    if (vec4) pk_bwd_k<float, 4, 1>(a, stream);
    else pk_bwd_k<float, 1, 1>(a, stream);
  }
  return hipGetLastError();
}

// The packet kernels take 4 channels per lane when D % 4 == 0, else 1; the
// pool's backward as above.
template <typename G>
void ipk_fwd_pool(const dwarf_packet_fwd_args& a, hipStream_t stream) {
  const bool vec4 = (a.pool.D % 4) == 0;
  if (a.pool.dtype == DWARF_BF16) {
    if (vec4) pkt_fwd_k<bf16, G, 4, 2>(a, stream);
    else pkt_fwd_k<bf16, G, 1, 1>(a, stream);
  } else {
    if (vec4) pkt_fwd_k<float, G, 4, 1>(a, stream);
    else pkt_fwd_k<float, G, 1, 1>(a, stream);
  }
}

template <typename G>
void ipk_bwd_pool(const dwarf_packet_bwd_args& a, hipStream_t stream) {
  const bool vec4 = (a.fwd.pool.D % 4) == 0;
  if (a.fwd.pool.dtype == DWARF_BF16) {
    if (vec4) pkt_bwd_k<bf16, G, 4, 2>(a, stream);
    else pkt_bwd_k<bf16, G, 1, 1>(a, stream);
  } else {
    if (vec4) pkt_bwd_k<float, G, 4, 1>(a, stream);
    else pkt_bwd_k<float, G, 1, 1>(a, stream);
  }
}

hipError_t launch_interference_packet_fwd(const dwarf_packet_fwd_args& a, hipStream_t stream) {
  if (a.packet_dtype == DWARF_BF16) ipk_fwd_pool<bf16>(a, stream);
  else ipk_fwd_pool<float>(a, stream);
  return hipGetLastError();
}

hipError_t launch_interference_packet_bwd(const dwarf_packet_bwd_args& a, hipStream_t stream) {
  if (a.fwd.packet_dtype == DWARF_BF16) ipk_bwd_pool<bf16>(a, stream);
  else ipk_bwd_pool<float>(a, stream);
  return hipGetLastError();
}

}  // namespace dwarf
