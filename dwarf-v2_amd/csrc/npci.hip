// NPCI rotation of K or V rows toward an injected delta (reference:
// npci_rotate, dsqg:221-254; applied to the kv_inject deltas at
// dsqg:3196-3229).  Per row x of [B,H,T,hd] with delta d and the head's
// angle theta_h:
//   n = max(|x|, 1e-12), u = x / n, p = d - (d.u) u, m = |p|,
//   active = m > 1e-7 n, e = p / m, s = tanh(m / (tau n + 1e-12)),
//   a = theta_h s, r = cos(a) x + sin(a) n e   (r = x where not active).
// The backward forms the vector-Jacobian products of that expression for x,
// d and theta (the reference leaves them to autograd) as per-row
// combinations of g, p and x; dtheta goes through a per-row buffer (head
// major) and a fixed-order sum per head.
//
// Four lanes per row (lane g holds dims [16g, 16g+16)), 16 rows per wave, 64
// rows per workgroup step, persistent workgroups; each row's dot products are
// quarter-row partials summed over the lane quad.  (Requesting the next step's
// rows before computing the current one measured slower here.)
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

// Forward scalars of one row from the lane's slices of x and d; p (the part
// of d orthogonal to x) is left in the lane's slice.  c1 = d.u with u = x / n,
// and p = d - c1 u = d - (c1 / n) x.
struct NpRowFwd {
  float ss, norm, inv_n, c1, m, s, sa, ca, den;
  bool active, clamped;
};

__device__ __forceinline__ NpRowFwd np_forward(const float* xv, const float* dv, float theta, float tau, float* p) {
  NpRowFwd f;
  float ss = 0.f, dx = 0.f;
#pragma unroll
  for (int k = 0; k < kNpDims; ++k) {
    ss = fmaf(xv[k], xv[k], ss);
    dx = fmaf(dv[k], xv[k], dx);
  }
  f.ss = quad_sum(ss);
  const float raw = sqrtf(f.ss);
  f.clamped = raw < 1e-12f;
  f.norm = fmaxf(raw, 1e-12f);
  f.inv_n = 1.f / f.norm;
  f.c1 = quad_sum(dx) * f.inv_n;
  const float cu = f.c1 * f.inv_n;
  float m2 = 0.f;
#pragma unroll
  for (int k = 0; k < kNpDims; ++k) {
    p[k] = fmaf(-cu, xv[k], dv[k]);
    m2 = fmaf(p[k], p[k], m2);
  }
  f.m = sqrtf(quad_sum(m2));
  f.active = f.m > f.norm * 1e-7f;
  f.den = fmaf(tau, f.norm, 1e-12f);
  f.s = tanhf(f.m / f.den);
  sincosf(theta * f.s, &f.sa, &f.ca);
  return f;
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
    float xv[kNpDims], dv[kNpDims], p[kNpDims];
    load_f32<TX, kNpDims>(x + rw.b * sx0 + rw.h * sx1 + static_cast<int64_t>(rw.t) * sx2 + kNpDims * g, xv);
    load_f32<TD, kNpDims>(d + rw.b * sd0 + rw.h * sd1 + static_cast<int64_t>(rw.t) * sd2 + kNpDims * g, dv);
    const NpRowFwd f = np_forward(xv, dv, theta[rw.h], gm.tau, p);
    // r = cos(a) x + sin(a) n p / m on active rows, x elsewhere
    const float cx = f.active ? f.ca : 1.f;
    const float cp = f.active ? f.sa * f.norm / fmaxf(f.m, 1e-20f) : 0.f;
    float out[kNpDims];
#pragma unroll
    for (int k = 0; k < kNpDims; ++k) out[k] = fmaf(cx, xv[k], cp * p[k]);
    store16<TX>(r + rw.b * sr0 + rw.h * sr1 + static_cast<int64_t>(rw.t) * sr2 + kNpDims * g, out);
  }
}

// The vector-Jacobian products of one row, with e = p / m, u = x / n:
//   ga = -sin(a) (g.x) + cos(a) n (g.e)          (dL/da; dtheta += ga s)
//   gw = ga theta (1 - s^2),  gm = gw / den,  gn = sin(a) (g.e) - gw m tau / den^2
//   gp = A g + B p  with A = sin(a) n / m,  B = (gm - A (g.e)) / m
//   gd = gp - (u.gp) u
//   gx = cos(a) g + (gu - (u.gu) u) / n + gn u,  gu = -c1 gp - (u.gp) d
// and u.gp = A (g.x) / n + B (u.p), u.p = 0 (c1 (1 - |u|^2) when |x| < 1e-12
// clamps n; then gx = cos(a) g + gu / n, as n no longer depends on x).  With
// d = p + c1 u and u.gu = -2 c1 (u.gp) for a unit u, both products are
// combinations of the row's g, p and x, formed per row on the scalar values:
//   gd = A g + B p - (u.gp) / n x
//   gx = (cos(a) - c1 A / n) g - (c1 B + u.gp) / n p + cx x,
//   cx = (c1 (u.gp) / n + gn) / n, or -c1 (u.gp) / n^2 when n is clamped.
// Inactive rows pass g through to x and give d and theta nothing.
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
    float xv[kNpDims], dv[kNpDims], gv[kNpDims], p[kNpDims];
    load_f32<TX, kNpDims>(x + rw.b * sx0 + rw.h * sx1 + static_cast<int64_t>(rw.t) * sx2 + kNpDims * g, xv);
    load_f32<TD, kNpDims>(d + rw.b * sd0 + rw.h * sd1 + static_cast<int64_t>(rw.t) * sd2 + kNpDims * g, dv);
    load_f32<TX, kNpDims>(gr + rw.b * sg0 + rw.h * sg1 + static_cast<int64_t>(rw.t) * sg2 + kNpDims * g, gv);
    const float th = theta[rw.h];
    const NpRowFwd f = np_forward(xv, dv, th, tau, p);
    float sgx = 0.f, sgp = 0.f;
#pragma unroll
    for (int k = 0; k < kNpDims; ++k) {
      sgx = fmaf(gv[k], xv[k], sgx);
      sgp = fmaf(gv[k], p[k], sgp);
    }
    sgx = quad_sum(sgx);
    const float inv_m = 1.f / fmaxf(f.m, 1e-20f);
    const float sge = quad_sum(sgp) * inv_m;
    const float ga = fmaf(-f.sa, sgx, f.ca * f.norm * sge);
    const float inv_den = 1.f / f.den;
    const float gw = ga * th * (1.f - f.s * f.s);
    const float gn = fmaf(f.sa, sge, -gw * f.m * tau * inv_den * inv_den);
    const float A = f.sa * f.norm * inv_m;
    const float Bc = fmaf(-A, sge, gw * inv_den) * inv_m;
    const float up = f.clamped ? f.c1 * (1.f - f.ss * f.inv_n * f.inv_n) : 0.f;
    const float ugp = fmaf(A * f.inv_n, sgx, Bc * up);
    const float c1n = f.c1 * f.inv_n;
    const float cx_n = f.clamped ? -c1n * ugp * f.inv_n : fmaf(c1n, ugp, gn) * f.inv_n;
    // gx = xg g + xp p + xx x, gd = dg g + dp p + dx_ x
    const float xg = f.active ? fmaf(-c1n, A, f.ca) : 1.f;
    const float xp = f.active ? -fmaf(f.c1, Bc, ugp) * f.inv_n : 0.f;
    const float xx = f.active ? cx_n : 0.f;
    const float dg = f.active ? A : 0.f;
    const float dp = f.active ? Bc : 0.f;
    const float dx_ = f.active ? -ugp * f.inv_n : 0.f;
    float gxo[kNpDims], gdo[kNpDims];
#pragma unroll
    for (int k = 0; k < kNpDims; ++k) {
      gxo[k] = fmaf(xg, gv[k], fmaf(xp, p[k], xx * xv[k]));
      gdo[k] = fmaf(dg, gv[k], fmaf(dp, p[k], dx_ * xv[k]));
    }
    store16<TX>(dx + rw.b * sdx0 + rw.h * sdx1 + static_cast<int64_t>(rw.t) * sdx2 + kNpDims * g, gxo);
    store16<TD>(dd + rw.b * sdd0 + rw.h * sdd1 + static_cast<int64_t>(rw.t) * sdd2 + kNpDims * g, gdo);
    if (g == 0) trow[(static_cast<int64_t>(rw.h) * gm.B + rw.b) * gm.T + rw.t] = f.active ? ga * f.s : 0.f;
  }
}

// dtheta[h] = sum of the head's B*T entries of trow (stored head-major): one
// workgroup per head; thread i adds the entries of 16-byte vectors i, i + 1024,
// ... in order (eight vectors in flight; single entries when B*T is not a
// multiple of 4 or the buffer not 16-byte aligned), the wave sums by a fixed butterfly, the waves in wave order.
__global__ __launch_bounds__(kWave * kNpRedWaves) void npci_dtheta_reduce(const float* __restrict__ trow,
                                                                        float* __restrict__ dtheta, NpGeom gm) {
  constexpr int kThreads = kWave * kNpRedWaves;
  constexpr int kInFlight = 8;
  __shared__ float s_w[kNpRedWaves];
  const int64_t per_head = static_cast<int64_t>(gm.B) * gm.T;
  const float* src = trow + static_cast<int64_t>(blockIdx.x) * per_head;
  float s = 0.f;
  if ((per_head & 3) == 0 && (reinterpret_cast<uintptr_t>(trow) & 15) == 0) {
    const float4* v = reinterpret_cast<const float4*>(src);
    const int64_t nv = per_head >> 2;
    int64_t i = threadIdx.x;
    for (; i + (kInFlight - 1) * kThreads < nv; i += kInFlight * kThreads) {
      float4 a[kInFlight];
#pragma unroll
      for (int j = 0; j < kInFlight; ++j) a[j] = v[i + j * kThreads];
#pragma unroll
      for (int j = 0; j < kInFlight; ++j) s = (((s + a[j].x) + a[j].y) + a[j].z) + a[j].w;
    }
    for (; i < nv; i += kThreads) {
      const float4 a = v[i];
      s = (((s + a.x) + a.y) + a.z) + a.w;
    }
  } else {
    for (int64_t i = threadIdx.x; i < per_head; i += kThreads) s += src[i];
  }
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) s += __shfl_xor(s, o);
  if (threadIdx.x % kWave == 0) s_w[threadIdx.x / kWave] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.f;
    for (int v = 0; v < kNpRedWaves; ++v) t += s_w[v];
    dtheta[blockIdx.x] = t;
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
