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
#include "ema_common.h"

namespace dwarf {

namespace {

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
  for (int i = 0; i < VEC; ++i) { a[i] = clamp_alpha(alpha, g, d0 + i); st[i] = 0.f; }
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
  for (int i = 0; i < VEC; ++i) { a[i] = clamp_alpha(alpha, g, d0 + i); st[i] = cr[i]; }
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
  for (int i = 0; i < VEC; ++i) { dec[i] = 1.f - clamp_alpha(alpha, g, d0 + i); st[i] = 0.f; }
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
    a[i] = clamp_alpha(alpha, g, d0 + i);
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
  launch_carry<false, RESET>(ends, carries, a.alpha, g, a.B, a.D, stream);
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
  launch_carry<true, RESET>(starts, carries, a.alpha, g, a.B, a.D, stream);
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
