// Causal EMA scan, y[t] = a x[t] + (1 - a) y[t-1], y[-1] = 0, fp32 state
// (reference: _CausalEMAFn ema:263-364 with kernels ema:73-260).
//
// Time is cut into chunks of kChunkT tokens.  Each lane owns VEC adjacent
// channels of one (b, chunk), so a wave reads 64*VEC consecutive channels of
// one token per load.
//   forward:  local  - chunk end state with zero carry-in (reads x)
//             carry  - one lane per (b, channel) walks the chunk ends and
//                      writes each chunk's carry-in (tiny)
//             apply  - rescans the chunk from its carry-in, writes y
//   backward: the same three stages run in reverse time on dy for the
//             adjoint lambda[t] = dy[t] + (1 - a) lambda[t+1]; the apply
//             stage writes dx = a * lambda and a per-lane partial of
//             dalpha = sum lambda[t] (x[t] - y[t-1]); a final kernel sums the
//             partials in a fixed order and applies the projected-clamp rule
//             of ema:357-364.
// Alpha may be one value (the reference contract, ema:557-558) or one per
// channel; the clamp to [floor, ceiling] happens in-kernel (ema:274-277).
#include "common.h"

namespace dwarf {

constexpr int kChunkT = 64;
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
};

__device__ __forceinline__ float clamp_alpha(const float* alpha, int per_channel, int d, float lo, float hi) {
  const float a = alpha[per_channel ? d : 0];
  return fminf(fmaxf(a, lo), hi);
}

// ---- forward --------------------------------------------------------------
template <typename T, int VEC>
__global__ __launch_bounds__(kEmaBlock) void ema_fwd_local(const T* __restrict__ x, int64_t sxb, int64_t sxn,
                                                          const float* __restrict__ alpha, float* __restrict__ ends,
                                                          EmaGeom g) {
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
  const int t1 = min(t0 + kChunkT, g.N);
  const T* p = x + b * sxb + static_cast<int64_t>(t0) * sxn + d0;
  for (int t = t0; t < t1; ++t, p += sxn) {
    float xv[VEC];
    ldv<T, VEC>(p, xv);
#pragma unroll
    for (int i = 0; i < VEC; ++i) st[i] = fmaf(a[i], xv[i], (1.f - a[i]) * st[i]);
  }
  float* e = ends + (static_cast<int64_t>(b) * g.NC + c) * g.D + d0;
#pragma unroll
  for (int i = 0; i < VEC; ++i) e[i] = st[i];
}

// One lane per (b, channel): carries[c] = state entering chunk c.  When
// REVERSE, chunks are walked from the last and carries[c] is the adjoint
// entering chunk c from the future.
template <bool REVERSE>
__global__ __launch_bounds__(kEmaBlock) void ema_carry(const float* __restrict__ ends, float* __restrict__ carries,
                                                      const float* __restrict__ alpha, EmaGeom g) {
  const int tid = blockIdx.x * kEmaBlock + threadIdx.x;
  if (tid >= g.B * g.D) return;
  const int b = tid / g.D, d = tid - b * g.D;
  const float a = clamp_alpha(alpha, g.per_channel, d, g.lo, g.hi);
  const float decay = 1.f - a;
  float full = 1.f;  // decay^kChunkT, by repeated multiplication as the serial scan applies it
  for (int i = 0; i < kChunkT; ++i) full *= decay;
  const int last_len = g.N - (g.NC - 1) * kChunkT;
  float last = 1.f;
  for (int i = 0; i < last_len; ++i) last *= decay;
  const float* e = ends + static_cast<int64_t>(b) * g.NC * g.D + d;
  float* cr = carries + static_cast<int64_t>(b) * g.NC * g.D + d;
  float carry = 0.f;
  for (int k = 0; k < g.NC; ++k) {
    const int c = REVERSE ? g.NC - 1 - k : k;
    cr[static_cast<int64_t>(c) * g.D] = carry;
    const float pw = (c == g.NC - 1) ? last : full;
    carry = fmaf(pw, carry, e[static_cast<int64_t>(c) * g.D]);
  }
}

template <typename T, int VEC>
__global__ __launch_bounds__(kEmaBlock) void ema_fwd_apply(const T* __restrict__ x, int64_t sxb, int64_t sxn,
                                                          T* __restrict__ y, int64_t syb, int64_t syn,
                                                          const float* __restrict__ alpha,
                                                          const float* __restrict__ carries, EmaGeom g) {
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
  const int t1 = min(t0 + kChunkT, g.N);
  const T* px = x + b * sxb + static_cast<int64_t>(t0) * sxn + d0;
  T* py = y + b * syb + static_cast<int64_t>(t0) * syn + d0;
  for (int t = t0; t < t1; ++t, px += sxn, py += syn) {
    float xv[VEC];
    ldv<T, VEC>(px, xv);
#pragma unroll
    for (int i = 0; i < VEC; ++i) st[i] = fmaf(a[i], xv[i], (1.f - a[i]) * st[i]);
    stv<T, VEC>(py, st);
  }
}

// ---- backward -------------------------------------------------------------
template <typename T, int VEC>
__global__ __launch_bounds__(kEmaBlock) void ema_bwd_local(const T* __restrict__ dy, int64_t sgb, int64_t sgn,
                                                          const float* __restrict__ alpha, float* __restrict__ starts,
                                                          EmaGeom g) {
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
  const int t1 = min(t0 + kChunkT, g.N);
  const T* p = dy + b * sgb + static_cast<int64_t>(t1 - 1) * sgn + d0;
  for (int t = t1 - 1; t >= t0; --t, p -= sgn) {
    float gv[VEC];
    ldv<T, VEC>(p, gv);
#pragma unroll
    for (int i = 0; i < VEC; ++i) st[i] = fmaf(dec[i], st[i], gv[i]);
  }
  float* e = starts + (static_cast<int64_t>(b) * g.NC + c) * g.D + d0;
#pragma unroll
  for (int i = 0; i < VEC; ++i) e[i] = st[i];
}

template <typename T, int VEC>
__global__ __launch_bounds__(kEmaBlock) void ema_bwd_apply(const T* __restrict__ x, int64_t sxb, int64_t sxn,
                                                          const T* __restrict__ y, int64_t syb, int64_t syn,
                                                          const T* __restrict__ dy, int64_t sgb, int64_t sgn,
                                                          T* __restrict__ dx, int64_t sdb, int64_t sdn,
                                                          const float* __restrict__ alpha,
                                                          const float* __restrict__ carries,
                                                          float* __restrict__ da_part, EmaGeom g) {
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
  const int t1 = min(t0 + kChunkT, g.N);
  for (int t = t1 - 1; t >= t0; --t) {
    float gv[VEC], xv[VEC], yp[VEC];
    ldv<T, VEC>(dy + b * sgb + static_cast<int64_t>(t) * sgn + d0, gv);
    ldv<T, VEC>(x + b * sxb + static_cast<int64_t>(t) * sxn + d0, xv);
    if (t > 0) {
      ldv<T, VEC>(y + b * syb + static_cast<int64_t>(t - 1) * syn + d0, yp);
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) yp[i] = 0.f;
    }
    float out[VEC];
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      st[i] = fmaf(1.f - a[i], st[i], gv[i]);
      out[i] = a[i] * st[i];
      da[i] = fmaf(st[i], xv[i] - yp[i], da[i]);
    }
    stv<T, VEC>(dx + b * sdb + static_cast<int64_t>(t) * sdn + d0, out);
  }
  float* dp = da_part + (static_cast<int64_t>(b) * g.NC + c) * g.D + d0;
#pragma unroll
  for (int i = 0; i < VEC; ++i) dp[i] = da[i];
}

// dalpha[d] (or the single dalpha) = sum over (b, chunk) of the partials, in
// order; then the projected-clamp rule.
__global__ __launch_bounds__(kEmaBlock) void ema_dalpha_reduce(const float* __restrict__ da_part,
                                                              const float* __restrict__ alpha,
                                                              float* __restrict__ dalpha, EmaGeom g) {
  __shared__ float s_red[kEmaBlock];
  const int rows = g.B * g.NC;
  if (g.per_channel) {
    const int d = blockIdx.x * kEmaBlock + threadIdx.x;
    if (d >= g.D) return;
    float s = 0.f;
    for (int r = 0; r < rows; ++r) s += da_part[static_cast<int64_t>(r) * g.D + d];
    const float ai = alpha[d];
    const bool blocked = (ai <= g.lo && s > 0.f) || (ai >= g.hi && s < 0.f);
    dalpha[d] = blocked ? 0.f : s;
    return;
  }
  // Scalar alpha: one workgroup; each lane sums a fixed set of channels
  // over all rows, then a fixed-shape tree over the lanes.
  float s = 0.f;
  for (int d = threadIdx.x; d < g.D; d += kEmaBlock)
    for (int r = 0; r < rows; ++r) s += da_part[static_cast<int64_t>(r) * g.D + d];
  s_red[threadIdx.x] = s;
  __syncthreads();
  for (int w = kEmaBlock / 2; w > 0; w >>= 1) {
    if (threadIdx.x < w) s_red[threadIdx.x] += s_red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const float tot = s_red[0];
    const float ai = alpha[0];
    const bool blocked = (ai <= g.lo && tot > 0.f) || (ai >= g.hi && tot < 0.f);
    dalpha[0] = blocked ? 0.f : tot;
  }
}

inline size_t ws_floats(int B, int N, int D) {
  const int NC = (N + kChunkT - 1) / kChunkT;
  return static_cast<size_t>(B) * NC * D;
}

inline EmaGeom make_geom(int B, int N, int D, int vec, int per_channel, float lo, float hi) {
  EmaGeom g;
  g.B = B; g.N = N; g.D = D;
  g.NC = (N + kChunkT - 1) / kChunkT;
  g.DV = D / vec;
  g.per_channel = per_channel;
  g.lo = lo; g.hi = hi;
  return g;
}

template <typename T, int VEC>
hipError_t ema_fwd_typed(const dwarf_ema_fwd_args& a, hipStream_t stream) {
  const EmaGeom g = make_geom(a.B, a.N, a.D, VEC, a.alpha_per_channel, a.floor_, a.ceiling);
  float* ends = static_cast<float*>(a.workspace);
  float* carries = ends + ws_floats(a.B, a.N, a.D);
  const int64_t lanes = static_cast<int64_t>(a.B) * g.NC * g.DV;
  const int blocks = static_cast<int>((lanes + kEmaBlock - 1) / kEmaBlock);
  const T* x = static_cast<const T*>(a.x);
  T* y = static_cast<T*>(a.y);
  hipLaunchKernelGGL((ema_fwd_local<T, VEC>), dim3(blocks), dim3(kEmaBlock), 0, stream, x, a.x_stride[0],
                     a.x_stride[1], a.alpha, ends, g);
  hipLaunchKernelGGL((ema_carry<false>), dim3((a.B * a.D + kEmaBlock - 1) / kEmaBlock), dim3(kEmaBlock), 0, stream,
                     ends, carries, a.alpha, g);
  hipLaunchKernelGGL((ema_fwd_apply<T, VEC>), dim3(blocks), dim3(kEmaBlock), 0, stream, x, a.x_stride[0],
                     a.x_stride[1], y, a.y_stride[0], a.y_stride[1], a.alpha, carries, g);
  return hipGetLastError();
}

template <typename T, int VEC>
hipError_t ema_bwd_typed(const dwarf_ema_bwd_args& a, hipStream_t stream) {
  const EmaGeom g = make_geom(a.B, a.N, a.D, VEC, a.alpha_per_channel, a.floor_, a.ceiling);
  const size_t nf = ws_floats(a.B, a.N, a.D);
  float* starts = static_cast<float*>(a.workspace);
  float* carries = starts + nf;
  float* da_part = carries + nf;
  const int64_t lanes = static_cast<int64_t>(a.B) * g.NC * g.DV;
  const int blocks = static_cast<int>((lanes + kEmaBlock - 1) / kEmaBlock);
  hipLaunchKernelGGL((ema_bwd_local<T, VEC>), dim3(blocks), dim3(kEmaBlock), 0, stream,
                     static_cast<const T*>(a.dy), a.dy_stride[0], a.dy_stride[1], a.alpha, starts, g);
  hipLaunchKernelGGL((ema_carry<true>), dim3((a.B * a.D + kEmaBlock - 1) / kEmaBlock), dim3(kEmaBlock), 0, stream,
                     starts, carries, a.alpha, g);
  hipLaunchKernelGGL((ema_bwd_apply<T, VEC>), dim3(blocks), dim3(kEmaBlock), 0, stream,
                     static_cast<const T*>(a.x), a.x_stride[0], a.x_stride[1], static_cast<const T*>(a.y),
                     a.y_stride[0], a.y_stride[1], static_cast<const T*>(a.dy), a.dy_stride[0], a.dy_stride[1],
                     static_cast<T*>(a.dx), a.dx_stride[0], a.dx_stride[1], a.alpha, carries, da_part, g);
  if (a.dalpha) {
    const int rb = a.alpha_per_channel ? (a.D + kEmaBlock - 1) / kEmaBlock : 1;
    hipLaunchKernelGGL(ema_dalpha_reduce, dim3(rb), dim3(kEmaBlock), 0, stream, da_part, a.alpha, a.dalpha, g);
  }
  return hipGetLastError();
}

}  // namespace

size_t ema_fwd_workspace(int B, int N, int D) { return 2 * ws_floats(B, N, D) * sizeof(float); }
size_t ema_bwd_workspace(int B, int N, int D) { return 3 * ws_floats(B, N, D) * sizeof(float); }

hipError_t launch_ema_fwd(const dwarf_ema_fwd_args& a, hipStream_t stream) {
  const bool vec4 = (a.D % 4) == 0;
  if (a.dtype == DWARF_BF16) return vec4 ? ema_fwd_typed<bf16, 4>(a, stream) : ema_fwd_typed<bf16, 1>(a, stream);
  return vec4 ? ema_fwd_typed<float, 4>(a, stream) : ema_fwd_typed<float, 1>(a, stream);
}

hipError_t launch_ema_bwd(const dwarf_ema_bwd_args& a, hipStream_t stream) {
  const bool vec4 = (a.D % 4) == 0;
  if (a.dtype == DWARF_BF16) return vec4 ? ema_bwd_typed<bf16, 4>(a, stream) : ema_bwd_typed<bf16, 1>(a, stream);
  return vec4 ? ema_bwd_typed<float, 4>(a, stream) : ema_bwd_typed<float, 1>(a, stream);
}

}  // namespace dwarf
