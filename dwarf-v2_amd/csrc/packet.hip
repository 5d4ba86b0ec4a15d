// InterferencePacket pool (reference: InterferencePacket.forward,
// train:260-267): K causal EMA scans of one input x at scalar factors a_k and
// their mix
//   scan_k = EMA(x, a_k) stored in T,   pooled = ((w_0 scan_0 + w_1 scan_1) + ...)
// with w_k = softmax(mix_logits)_k cast to T and every product and partial
// sum rounded to T, as the reference's bf16 tensor arithmetic rounds them.
// The reference runs K separate scans (each reading x and writing its scan)
// and K products and K - 1 sums; here x is read twice and pooled written
// once.
//
// Stages, on the EMA's 16-token chunks (ema_common.h):
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
#include "ema_common.h"
#include "dwarf_dsqg.h"

namespace dwarf {
namespace {

constexpr int kMaxScales = 4;
constexpr int kPkRedThreads = 1024;

// The value a T tensor holds for v.
template <typename T>
__device__ __forceinline__ float rnd(float v);
template <>
__device__ __forceinline__ float rnd<float>(float v) { return v; }
template <>
__device__ __forceinline__ float rnd<bf16>(float v) { return round_bf16(v); }

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

inline int pk_nc(int N) { return (N + kChunkT - 1) / kChunkT; }

inline size_t pk_state_floats(int B, int N, int D, int K) {
  return static_cast<size_t>(B) * pk_nc(N) * D * K;
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

template <typename T, int VEC, int K>
void pk_fwd_typed(const dwarf_packet_pool_fwd_args& a, hipStream_t stream) {
  const EmaGeom g = pk_geom(a.B, a.N, a.D, VEC, a.floor_, a.ceiling);
  float* ends = static_cast<float*>(a.workspace);
  const int64_t lanes = static_cast<int64_t>(a.B) * g.NC * g.DV;
  const int blocks = static_cast<int>((lanes + kEmaBlock - 1) / kEmaBlock);
  const T* x = static_cast<const T*>(a.x);
  hipLaunchKernelGGL((packet_fwd_local<T, VEC, K>), dim3(blocks), dim3(kEmaBlock), 0, stream, x, a.x_stride[0],
                     a.x_stride[1], a.alpha, ends, g);
  const EmaGeom gc = pk_carry_geom(a.B, a.N, a.D, K, a.floor_, a.ceiling);
  launch_carry<false, false>(ends, a.state, a.alpha, gc, a.B, K * a.D, stream);
  hipLaunchKernelGGL((packet_fwd_apply<T, VEC, K>), dim3(blocks), dim3(kEmaBlock), 0, stream, x, a.x_stride[0],
                     a.x_stride[1], static_cast<T*>(a.pooled), a.pooled_stride[0], a.pooled_stride[1], a.alpha,
                     a.weight, a.state, g);
}

template <typename T, int VEC, int VA, int K>
void pk_bwd_typed(const dwarf_packet_pool_bwd_args& a, hipStream_t stream) {
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

}  // namespace

size_t packet_state_bytes(int B, int N, int D, int K) { return pk_state_floats(B, N, D, K) * sizeof(float); }
size_t packet_fwd_workspace(int B, int N, int D, int K) { return pk_state_floats(B, N, D, K) * sizeof(float); }
// starts and carries (K*D per chunk each), then 2K slots per apply workgroup
// (a lane takes at least one (chunk, channel) pair, so at most
// ceil(B*NC*D / 256) workgroups).
size_t packet_bwd_workspace(int B, int N, int D, int K) {
  const size_t pairs = static_cast<size_t>(B) * pk_nc(N) * D;
  return (2 * pk_state_floats(B, N, D, K) + 2 * static_cast<size_t>(K) * ((pairs + kEmaBlock - 1) / kEmaBlock)) *
         sizeof(float);
}
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

}  // namespace dwarf
