// NPCI rotation of K or V rows toward an injected delta (reference:
// npci_rotate, dsqg:221-254; applied to the kv_inject deltas at
// dsqg:3196-3229).  Per row x of [B,H,T,hd] with delta d and the head's
// angle theta_h:
//   n = max(|x|, 1e-12), u = x / n, p = d - (d.u) u, m = |p|,
//   active = m > 1e-7 n, e = p / m, s = tanh(m / (tau n + 1e-12)),
//   a = theta_h s, r = cos(a) x + sin(a) n e   (r = x where not active).
// The backward forms the vector-Jacobian products of that expression for x,
// d and theta (the reference leaves them to autograd); dtheta goes through a
// per-row buffer and a fixed-order sum per head.
//
// Four lanes per row (lane g holds dims [16g, 16g+16)), 16 rows per wave, 64
// rows per workgroup step, persistent workgroups; each row's dot products are
// quarter-row partials summed over the lane quad.
#include "common.h"
#include "dsqg_internal.h"
#include "gather.h"

namespace dwarf {
namespace {

constexpr int kNpRows = 64;        // rows per workgroup step
constexpr int kNpWgsPerCu = 4;
constexpr int kNpCus = 256;        // CUs of an MI355X
constexpr int kNpDims = 16;        // head dims per lane
constexpr int kNpRedWaves = 16;    // waves of the dtheta reduction workgroup

struct NpGeom {
  int B, H, T;
  int64_t rows;   // B * H * T
  float tau;
};

struct NpRow {
  int b, h, t;
};

// Row wave_row + i (i < 16): the wave's first row is uniform and divided on
// the scalar unit; with T >= 16 the 16 rows cross at most one (b, h) boundary.
// rows < 2^31 (checked on the host).
__device__ __forceinline__ NpRow np_row(const NpGeom& gm, int64_t wave_row, int i) {
  NpRow r;
  if (gm.T < 16) {
    const uint32_t rw = static_cast<uint32_t>(wave_row + i);
    const uint32_t bh = rw / static_cast<uint32_t>(gm.T);
    r.t = static_cast<int>(rw - bh * static_cast<uint32_t>(gm.T));
    r.b = static_cast<int>(bh / static_cast<uint32_t>(gm.H));
    r.h = static_cast<int>(bh) - r.b * gm.H;
    return r;
  }
  const uint32_t w0 = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(wave_row)));
  const uint32_t bh0 = w0 / static_cast<uint32_t>(gm.T);
  r.t = static_cast<int>(w0 - bh0 * static_cast<uint32_t>(gm.T)) + i;
  r.b = static_cast<int>(bh0 / static_cast<uint32_t>(gm.H));
  r.h = static_cast<int>(bh0) - r.b * gm.H;
  if (r.t >= gm.T) {
    r.t -= gm.T;
    if (++r.h == gm.H) {
      r.h = 0;
      ++r.b;
    }
  }
  return r;
}

template <typename T>
__device__ __forceinline__ void store16(T* p, const float* v);
template <>
__device__ __forceinline__ void store16<bf16>(bf16* p, const float* v) {
  store_bf16<kNpDims>(reinterpret_cast<uint16_t*>(p), v);
}
template <>
__device__ __forceinline__ void store16<float>(float* p, const float* v) {
  store_f32<kNpDims>(p, v);
}

__device__ __forceinline__ float quad_sum(float v) { return group_sum<4>(v); }

// Forward quantities of one row from the lane's slices of x and d.
struct NpFwd {
  float u[kNpDims], p[kNpDims];
  float norm, c1, m, s, sa, ca, theta;
  bool active, clamped;
};

__device__ __forceinline__ void np_forward(const float* xv, const float* dv, float theta, float tau, NpFwd& f) {
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < kNpDims; ++k) ss = fmaf(xv[k], xv[k], ss);
  const float raw = sqrtf(quad_sum(ss));
  f.clamped = raw < 1e-12f;
  f.norm = fmaxf(raw, 1e-12f);
  float c1 = 0.f;
#pragma unroll
  for (int k = 0; k < kNpDims; ++k) {
    f.u[k] = xv[k] / f.norm;
    c1 = fmaf(dv[k], f.u[k], c1);
  }
  f.c1 = quad_sum(c1);
  float m2 = 0.f;
#pragma unroll
  for (int k = 0; k < kNpDims; ++k) {
    f.p[k] = fmaf(-f.c1, f.u[k], dv[k]);
    m2 = fmaf(f.p[k], f.p[k], m2);
  }
  f.m = sqrtf(quad_sum(m2));
  f.active = f.m > f.norm * 1e-7f;
  f.s = tanhf(f.m / (tau * f.norm + 1e-12f));
  f.theta = theta;
  sincosf(theta * f.s, &f.sa, &f.ca);
}

template <typename TX, typename TD>
__global__ __launch_bounds__(kBlock, kNpWgsPerCu) void npci_fwd_kernel(
    const TX* __restrict__ x, int64_t sx0, int64_t sx1, int64_t sx2, const TD* __restrict__ d, int64_t sd0,
    int64_t sd1, int64_t sd2, const float* __restrict__ theta, TX* __restrict__ r, int64_t sr0, int64_t sr1,
    int64_t sr2, NpGeom gm) {
  const int l = threadIdx.x % kWave, w = threadIdx.x / kWave;
  const int g = l & 3;
  for (int64_t r0 = static_cast<int64_t>(blockIdx.x) * kNpRows; r0 < gm.rows;
       r0 += static_cast<int64_t>(gridDim.x) * kNpRows) {
    const int64_t row = r0 + w * 16 + (l >> 2);   // the same in the four lanes of a quad
    if (row >= gm.rows) continue;
    const NpRow rw = np_row(gm, r0 + w * 16, l >> 2);
    float xv[kNpDims], dv[kNpDims];
    load_f32<TX, kNpDims>(x + rw.b * sx0 + rw.h * sx1 + static_cast<int64_t>(rw.t) * sx2 + kNpDims * g, xv);
    load_f32<TD, kNpDims>(d + rw.b * sd0 + rw.h * sd1 + static_cast<int64_t>(rw.t) * sd2 + kNpDims * g, dv);
    NpFwd f;
    np_forward(xv, dv, theta[rw.h], gm.tau, f);
    float out[kNpDims];
    const float sn = f.sa * f.norm / fmaxf(f.m, 1e-20f);
#pragma unroll
    for (int k = 0; k < kNpDims; ++k) out[k] = f.active ? fmaf(f.ca, xv[k], sn * f.p[k]) : xv[k];
    store16<TX>(r + rw.b * sr0 + rw.h * sr1 + static_cast<int64_t>(rw.t) * sr2 + kNpDims * g, out);
  }
}

template <typename TX, typename TD>
__global__ __launch_bounds__(kBlock, kNpWgsPerCu) void npci_bwd_kernel(
    const TX* __restrict__ x, int64_t sx0, int64_t sx1, int64_t sx2, const TD* __restrict__ d, int64_t sd0,
    int64_t sd1, int64_t sd2, const float* __restrict__ theta, const TX* __restrict__ gr, int64_t sg0, int64_t sg1,
    int64_t sg2, TX* __restrict__ dx, int64_t sdx0, int64_t sdx1, int64_t sdx2, TD* __restrict__ dd, int64_t sdd0,
    int64_t sdd1, int64_t sdd2, float* __restrict__ trow, NpGeom gm) {
  const int l = threadIdx.x % kWave, w = threadIdx.x / kWave;
  const int g = l & 3;
  const float tau = gm.tau;
  for (int64_t r0 = static_cast<int64_t>(blockIdx.x) * kNpRows; r0 < gm.rows;
       r0 += static_cast<int64_t>(gridDim.x) * kNpRows) {
    const int64_t row = r0 + w * 16 + (l >> 2);
    if (row >= gm.rows) continue;
    const NpRow rw = np_row(gm, r0 + w * 16, l >> 2);
    float xv[kNpDims], dv[kNpDims], gv[kNpDims];
    load_f32<TX, kNpDims>(x + rw.b * sx0 + rw.h * sx1 + static_cast<int64_t>(rw.t) * sx2 + kNpDims * g, xv);
    load_f32<TD, kNpDims>(d + rw.b * sd0 + rw.h * sd1 + static_cast<int64_t>(rw.t) * sd2 + kNpDims * g, dv);
    load_f32<TX, kNpDims>(gr + rw.b * sg0 + rw.h * sg1 + static_cast<int64_t>(rw.t) * sg2 + kNpDims * g, gv);
    NpFwd f;
    np_forward(xv, dv, theta[rw.h], tau, f);
    const float inv_m = 1.f / fmaxf(f.m, 1e-20f);
    float sgx = 0.f, sge = 0.f;
#pragma unroll
    for (int k = 0; k < kNpDims; ++k) {
      sgx = fmaf(gv[k], xv[k], sgx);
      sge = fmaf(gv[k], f.p[k] * inv_m, sge);
    }
    sgx = quad_sum(sgx);
    sge = quad_sum(sge);
    const float ga = fmaf(-f.sa, sgx, f.ca * f.norm * sge);
    const float den = tau * f.norm + 1e-12f;
    const float gw = ga * f.theta * (1.f - f.s * f.s);
    const float gm_ = gw / den;
    const float gn = fmaf(f.sa, sge, -gw * f.m * tau / (den * den));
    // gp = (ge - e (e.ge)) / m + gm e with ge = sin(a) n g and e.ge = sin(a) n sge
    const float san = f.sa * f.norm;
    float gp[kNpDims];
    float ugp = 0.f;
#pragma unroll
    for (int k = 0; k < kNpDims; ++k) {
      const float e = f.p[k] * inv_m;
      gp[k] = fmaf(san * inv_m, fmaf(-e, sge, gv[k]), gm_ * e);
      ugp = fmaf(f.u[k], gp[k], ugp);
    }
    ugp = quad_sum(ugp);
    float gd[kNpDims], gu[kNpDims];
    float ugu = 0.f;
#pragma unroll
    for (int k = 0; k < kNpDims; ++k) {
      gd[k] = fmaf(-f.u[k], ugp, gp[k]);
      gu[k] = fmaf(-f.c1, gp[k], -dv[k] * ugp);
      ugu = fmaf(f.u[k], gu[k], ugu);
    }
    ugu = quad_sum(ugu);
    float gxo[kNpDims], gdo[kNpDims];
    const float inv_n = 1.f / f.norm;
#pragma unroll
    for (int k = 0; k < kNpDims; ++k) {
      const float gxu = f.clamped ? gu[k] * inv_n : fmaf(-f.u[k], ugu, gu[k]) * inv_n;
      const float gxn = f.clamped ? 0.f : gn * f.u[k];
      gxo[k] = f.active ? fmaf(f.ca, gv[k], gxu + gxn) : gv[k];
      gdo[k] = f.active ? gd[k] : 0.f;
    }
    store16<TX>(dx + rw.b * sdx0 + rw.h * sdx1 + static_cast<int64_t>(rw.t) * sdx2 + kNpDims * g, gxo);
    store16<TD>(dd + rw.b * sdd0 + rw.h * sdd1 + static_cast<int64_t>(rw.t) * sdd2 + kNpDims * g, gdo);
    if (g == 0) trow[(static_cast<int64_t>(rw.b) * gm.H + rw.h) * gm.T + rw.t] = f.active ? ga * f.s : 0.f;
  }
}

// dtheta[h] = sum over (b, t) of trow[b][h][t]: one workgroup per head; thread
// i adds entries i, i + 1024, ... of the head's B*T values in order, the wave
// sums by a fixed butterfly, the waves in wave order.
__global__ __launch_bounds__(kWave * kNpRedWaves) void npci_dtheta_reduce(const float* __restrict__ trow,
                                                                        float* __restrict__ dtheta, NpGeom gm) {
  __shared__ float s_w[kNpRedWaves];
  const int h = blockIdx.x;
  const int64_t per_head = static_cast<int64_t>(gm.B) * gm.T;
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < per_head; i += kWave * kNpRedWaves) {
    const int b = static_cast<int>(i / gm.T), t = static_cast<int>(i - static_cast<int64_t>(b) * gm.T);
    s += trow[(static_cast<int64_t>(b) * gm.H + h) * gm.T + t];
  }
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) s += __shfl_xor(s, o);
  if (threadIdx.x % kWave == 0) s_w[threadIdx.x / kWave] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.f;
    for (int v = 0; v < kNpRedWaves; ++v) t += s_w[v];
    dtheta[h] = t;
  }
}

NpGeom np_geom(const dwarf_npci_fwd_args& a) {
  NpGeom gm;
  gm.B = a.B; gm.H = a.H; gm.T = a.T;
  gm.rows = static_cast<int64_t>(a.B) * a.H * a.T;
  gm.tau = a.strength_tau;
  return gm;
}

int np_wgs(int64_t rows) {
  const int64_t steps = (rows + kNpRows - 1) / kNpRows;
  return static_cast<int>(steps < kNpCus * kNpWgsPerCu ? steps : kNpCus * kNpWgsPerCu);
}

template <typename TX, typename TD>
void np_fwd_typed(const dwarf_npci_fwd_args& a, const NpGeom& gm, hipStream_t stream) {
  hipLaunchKernelGGL((npci_fwd_kernel<TX, TD>), dim3(np_wgs(gm.rows)), dim3(kBlock), 0, stream,
                     static_cast<const TX*>(a.x), a.x_stride[0], a.x_stride[1], a.x_stride[2],
                     static_cast<const TD*>(a.delta), a.delta_stride[0], a.delta_stride[1], a.delta_stride[2], a.theta,
                     static_cast<TX*>(a.out), a.out_stride[0], a.out_stride[1], a.out_stride[2], gm);
}

template <typename TX, typename TD>
void np_bwd_typed(const dwarf_npci_bwd_args& a, const NpGeom& gm, float* trow, hipStream_t stream) {
  const dwarf_npci_fwd_args& f = a.fwd;
  hipLaunchKernelGGL((npci_bwd_kernel<TX, TD>), dim3(np_wgs(gm.rows)), dim3(kBlock), 0, stream,
                     static_cast<const TX*>(f.x), f.x_stride[0], f.x_stride[1], f.x_stride[2],
                     static_cast<const TD*>(f.delta), f.delta_stride[0], f.delta_stride[1], f.delta_stride[2], f.theta,
                     static_cast<const TX*>(a.grad), a.grad_stride[0], a.grad_stride[1], a.grad_stride[2],
                     static_cast<TX*>(a.dx), a.dx_stride[0], a.dx_stride[1], a.dx_stride[2],
                     static_cast<TD*>(a.ddelta), a.ddelta_stride[0], a.ddelta_stride[1], a.ddelta_stride[2], trow, gm);
}

}  // namespace

size_t npci_bwd_workspace(const dwarf_npci_bwd_args& a) {
  return static_cast<size_t>(a.fwd.B) * a.fwd.H * a.fwd.T * sizeof(float);
}

hipError_t launch_npci_fwd(const dwarf_npci_fwd_args& a, hipStream_t stream) {
  const NpGeom gm = np_geom(a);
  if (gm.rows == 0) return hipSuccess;
  const bool xb = a.x_dtype == DWARF_BF16, db = a.delta_dtype == DWARF_BF16;
  if (xb && db) np_fwd_typed<bf16, bf16>(a, gm, stream);
  else if (xb) np_fwd_typed<bf16, float>(a, gm, stream);
  else if (db) np_fwd_typed<float, bf16>(a, gm, stream);
  else np_fwd_typed<float, float>(a, gm, stream);
  return hipGetLastError();
}

hipError_t launch_npci_bwd(const dwarf_npci_bwd_args& a, hipStream_t stream) {
  const NpGeom gm = np_geom(a.fwd);
  if (gm.rows == 0) return hipSuccess;
  float* trow = static_cast<float*>(a.workspace);
  const bool xb = a.fwd.x_dtype == DWARF_BF16, db = a.fwd.delta_dtype == DWARF_BF16;
  if (xb && db) np_bwd_typed<bf16, bf16>(a, gm, trow, stream);
  else if (xb) np_bwd_typed<bf16, float>(a, gm, trow, stream);
  else if (db) np_bwd_typed<float, bf16>(a, gm, trow, stream);
  else np_bwd_typed<float, float>(a, gm, trow, stream);
  hipLaunchKernelGGL(npci_dtheta_reduce, dim3(gm.H), dim3(kWave * kNpRedWaves), 0, stream, trow, a.dtheta, gm);
  return hipGetLastError();
}

}  // namespace dwarf
