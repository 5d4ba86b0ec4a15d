// Phase-probe features of the DSQG block (reference: _PhaseProbeFn dsqg:371-419
// with its kernels dsqg:275-369; phase_probe_features dsqg:422-451):
//   y[b,h,n,r] = <x[b,h,n], p_r> / sqrt(|x[b,h,n]|^2 + 1e-6 hd)   for n in [start, end)
// and 0 for every other row; the backward, with inv = 1/sqrt(|x|^2 + 1e-6 hd)
// and raw_r = <x, p_r>:
//   dx = inv sum_r g_r p_r - x inv^3 sum_r g_r raw_r        (0 outside [start, end))
//   dprobes[r] = sum over rows of g_r inv x.
//
// Four lanes per row (lane g holds dims [16g, 16g+16)), 16 rows per wave, 64
// rows per workgroup step.  Workgroups are persistent, so each lane loads
// its 4 planes x 16 dims of the probes once.  |x|^2 and the four projections
// are quarter-row partials summed over the lane quad.  The forward's lane g
// stores plane g (a 16-byte row of the output per quad).  The backward keeps
// per-lane dprobes partials in registers, sums them over the wave's 16 rows
// (lane swaps, then DPP row rotations), then over the workgroup's 4 waves in
// wave order into the workgroup's slot; a second launch adds the slots in a
// fixed order, so dprobes has a fixed summation order (the reference adds
// with atomics, dsqg:358-363).
#include "common.h"
#include "dsqg_internal.h"
#include "gather.h"

namespace dwarf {
namespace {

constexpr int kPrRows = 64;        // rows per workgroup step
constexpr int kPrWgsPerCu = 4;
constexpr int kPrCus = 256;        // CUs of an MI355X
constexpr int kPrDims = 16;        // head dims per lane
constexpr int kPrSlot = kPlanes * kHeadDim;   // floats per dprobes slot

struct PrGeom {
  int B, H, N, start, end;
  int64_t rows;   // B * H * N
};

struct PrRow {
  int b, h, n;
  bool live;      // n in [start, end)
};

// rows < 2^31 (checked on the host): 32-bit division.
__device__ __forceinline__ PrRow pr_row(const PrGeom& gm, int64_t row) {
  PrRow r;
  const uint32_t rw = static_cast<uint32_t>(row);
  const uint32_t bh = rw / static_cast<uint32_t>(gm.N);
  r.n = static_cast<int>(rw - bh * static_cast<uint32_t>(gm.N));
  r.b = static_cast<int>(bh / static_cast<uint32_t>(gm.H));
  r.h = static_cast<int>(bh) - r.b * gm.H;
  r.live = r.n >= gm.start && r.n < gm.end;
  return r;
}

// Row wave_row + i (i < 16) from the decomposition of the wave's first row,
// which is uniform and so divided on the scalar unit; with N >= 16 the 16
// rows cross at most one (b, h) boundary.
__device__ __forceinline__ PrRow pr_row_wave(const PrGeom& gm, int64_t wave_row, int i) {
  if (gm.N < 16) return pr_row(gm, wave_row + i);
  const uint32_t w0 = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(wave_row)));
  const uint32_t bh0 = w0 / static_cast<uint32_t>(gm.N);
  const int n0 = static_cast<int>(w0 - bh0 * static_cast<uint32_t>(gm.N));
  const int b0 = static_cast<int>(bh0 / static_cast<uint32_t>(gm.H));
  const int h0 = static_cast<int>(bh0) - b0 * gm.H;
  PrRow r;
  r.n = n0 + i;
  r.h = h0;
  r.b = b0;
  if (r.n >= gm.N) {
    r.n -= gm.N;
    if (++r.h == gm.H) {
      r.h = 0;
      ++r.b;
    }
  }
  r.live = r.n >= gm.start && r.n < gm.end;
  return r;
}

template <typename T>
__device__ __forceinline__ void store16(T* p, const float* v);
template <>
__device__ __forceinline__ void store16<bf16>(bf16* p, const float* v) {
  store_bf16<kPrDims>(reinterpret_cast<uint16_t*>(p), v);
}
template <>
__device__ __forceinline__ void store16<float>(float* p, const float* v) {
  store_f32<kPrDims>(p, v);
}

// One workgroup step of a lane: its row (the same in the four lanes of a
// quad), whether it exists, and the loads issued for it.
template <typename T>
struct PrStep {
  PrRow rw;
  bool ok;
  RawSlice16<T> x;
  float gown;   // backward: dout[row][plane g]
};

// Lane g's 16 dims of the four probes.
__device__ __forceinline__ void load_probe_slice(const float* __restrict__ probes, int g, float (&p)[kPlanes][kPrDims]) {
#pragma unroll
  for (int r = 0; r < kPlanes; ++r) load_f32<float, kPrDims>(probes + r * kHeadDim + kPrDims * g, p[r]);
}

// |x|^2 and <x, p_r> of the row, summed over the lane quad (every lane of the
// quad holds the full sums).
__device__ __forceinline__ void row_sums(const float* xv, const float (&p)[kPlanes][kPrDims], float& ss,
                                         float (&raw)[kPlanes]) {
  ss = 0.f;
#pragma unroll
  for (int r = 0; r < kPlanes; ++r) raw[r] = 0.f;
#pragma unroll
  for (int d = 0; d < kPrDims; ++d) {
    ss = fmaf(xv[d], xv[d], ss);
#pragma unroll
    for (int r = 0; r < kPlanes; ++r) raw[r] = fmaf(xv[d], p[r][d], raw[r]);
  }
  ss = group_sum<4>(ss);
#pragma unroll
  for (int r = 0; r < kPlanes; ++r) raw[r] = group_sum<4>(raw[r]);
}

template <typename T>
__global__ __launch_bounds__(kBlock, kPrWgsPerCu) void phase_probe_fwd_kernel(
    const T* __restrict__ x, int64_t sx0, int64_t sx1, int64_t sx2, const float* __restrict__ probes,
    float* __restrict__ out, int64_t so0, int64_t so1, int64_t so2, int64_t so3, PrGeom gm) {
  const int l = threadIdx.x % kWave, w = threadIdx.x / kWave;
  const int g = l & 3;
  float p[kPlanes][kPrDims];
  load_probe_slice(probes, g, p);
  const float eps = 1e-6f * kHeadDim;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kPrRows;
  auto fetch = [&](int64_t r0, PrStep<T>& st) {
    const int64_t row = r0 + w * 16 + (l >> 2);
    st.ok = row < gm.rows;
    if (st.ok) {
      st.rw = pr_row_wave(gm, r0 + w * 16, l >> 2);
      if (st.rw.live) load_raw(x + st.rw.b * sx0 + st.rw.h * sx1 + static_cast<int64_t>(st.rw.n) * sx2 + kPrDims * g, st.x);
    }
  };
  auto process = [&](const PrStep<T>& cur) {
    if (!cur.ok) return;
    float y = 0.f;
    if (cur.rw.live) {
      float xv[kPrDims];
      widen(cur.x, xv);
      float ss, raw[kPlanes];
      row_sums(xv, p, ss, raw);
      y = pick4(g, raw[0], raw[1], raw[2], raw[3]) * rsqrtf(ss + eps);
    }
    out[cur.rw.b * so0 + cur.rw.h * so1 + static_cast<int64_t>(cur.rw.n) * so2 + g * so3] = y;
  };
  // two step buffers in turn, the next step's loads in flight while one is consumed (a copy of a
  // prefetch buffer into a current one would wait for its loads at every step)
  PrStep<T> s0, s1;
  int64_t r0 = static_cast<int64_t>(blockIdx.x) * kPrRows;
  if (r0 < gm.rows) fetch(r0, s0);
  for (; r0 < gm.rows; r0 += 2 * stride) {
    if (r0 + stride < gm.rows) fetch(r0 + stride, s1);
    process(s0);
    if (r0 + stride >= gm.rows) break;
    if (r0 + 2 * stride < gm.rows) fetch(r0 + 2 * stride, s0);
    process(s1);
  }
}

// The backward holds x, dx and (with dprobes) 64 partials per lane: three or
// two workgroups per CU.
__host__ __device__ constexpr int pr_bwd_wgs_per_cu(bool dprobes) { return dprobes ? 2 : 3; }

template <typename T, bool DPROBES>
__global__ __launch_bounds__(kBlock, pr_bwd_wgs_per_cu(DPROBES)) void phase_probe_bwd_kernel(
    const T* __restrict__ x, int64_t sx0, int64_t sx1, int64_t sx2, const float* __restrict__ probes,
    const float* __restrict__ dout, int64_t sg0, int64_t sg1, int64_t sg2, int64_t sg3, T* __restrict__ dx,
    int64_t sd0, int64_t sd1, int64_t sd2, float* __restrict__ part, PrGeom gm) {
  __shared__ float s_part[DPROBES ? 4 : 1][kPrSlot];
  const int l = threadIdx.x % kWave, w = threadIdx.x / kWave;
  const int g = l & 3;
  float p[kPlanes][kPrDims];
  load_probe_slice(probes, g, p);
  float dp[kPlanes * kPrDims];   // dprobes partial, [plane][dim of the lane's slice]
#pragma unroll
  for (int i = 0; i < kPlanes * kPrDims; ++i) dp[i] = 0.f;
  const float eps = 1e-6f * kHeadDim;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kPrRows;
  auto fetch = [&](int64_t r0, PrStep<T>& st) {
    const int64_t row = r0 + w * 16 + (l >> 2);
    st.ok = row < gm.rows;
    if (st.ok) {
      st.rw = pr_row_wave(gm, r0 + w * 16, l >> 2);
      if (st.rw.live) {
        load_raw(x + st.rw.b * sx0 + st.rw.h * sx1 + static_cast<int64_t>(st.rw.n) * sx2 + kPrDims * g, st.x);
        st.gown = dout[st.rw.b * sg0 + st.rw.h * sg1 + static_cast<int64_t>(st.rw.n) * sg2 + g * sg3];
      }
    }
  };
  auto process = [&](const PrStep<T>& cur) {
    if (!cur.ok) return;
    const PrRow& rw = cur.rw;
    float dxv[kPrDims];
#pragma unroll
    for (int d = 0; d < kPrDims; ++d) dxv[d] = 0.f;
    if (rw.live) {
      float xv[kPrDims];
      widen(cur.x, xv);
      // lane g fetched g_g; the quad shares the four
      const float gown = cur.gown;
      float gr[kPlanes];
      gr[0] = dpp_f<0x00>(gown);   // quad_perm [0,0,0,0]
      gr[1] = dpp_f<0x55>(gown);   // quad_perm [1,1,1,1]
      gr[2] = dpp_f<0xaa>(gown);   // quad_perm [2,2,2,2]
      gr[3] = dpp_f<0xff>(gown);   // quad_perm [3,3,3,3]
      float ss, raw[kPlanes];
      row_sums(xv, p, ss, raw);
      const float inv = rsqrtf(ss + eps);
      float graw = 0.f;
#pragma unroll
      for (int r = 0; r < kPlanes; ++r) graw = fmaf(gr[r], raw[r], graw);
      const float a = inv * inv * inv * graw;
#pragma unroll
      for (int d = 0; d < kPrDims; ++d) {
        float s = 0.f;
#pragma unroll
        for (int r = 0; r < kPlanes; ++r) s = fmaf(gr[r], p[r][d], s);
        dxv[d] = fmaf(s, inv, -a * xv[d]);
      }
      if constexpr (DPROBES) {
#pragma unroll
        for (int r = 0; r < kPlanes; ++r) {
          const float gi = gr[r] * inv;
#pragma unroll
          for (int d = 0; d < kPrDims; ++d) dp[r * kPrDims + d] = fmaf(gi, xv[d], dp[r * kPrDims + d]);
        }
      }
    }
    store16<T>(dx + rw.b * sd0 + rw.h * sd1 + static_cast<int64_t>(rw.n) * sd2 + kPrDims * g, dxv);
  };
  // two step buffers in turn (as in the forward)
  PrStep<T> s0, s1;
  int64_t r0 = static_cast<int64_t>(blockIdx.x) * kPrRows;
  if (r0 < gm.rows) fetch(r0, s0);
  for (; r0 < gm.rows; r0 += 2 * stride) {
    if (r0 + stride < gm.rows) fetch(r0 + stride, s1);
    process(s0);
    if (r0 + stride >= gm.rows) break;
    if (r0 + 2 * stride < gm.rows) fetch(r0 + 2 * stride, s0);
    process(s1);
  }
  if constexpr (DPROBES) {
    // Sum over the wave's 16 rows (lanes sharing g), reduce-scattered: after
    // the two swaps lane l holds plane l >> 4, dims 16g + [0, 16), of four
    // rows; two row rotations add the other twelve.
    float r32[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) r32[i] = add_swap32(dp[i], dp[i + 32]);
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float s = add_swap16(r32[i], r32[i + 16]);
      s += dpp_f<0x124>(s);   // row_ror:4
      s += dpp_f<0x128>(s);   // row_ror:8
      v[i] = s;
    }
    if (((l >> 2) & 3) == 0) {
      float* dst = s_part[w] + (l >> 4) * kHeadDim + kPrDims * g;
#pragma unroll
      for (int i = 0; i < 16; ++i) dst[i] = v[i];
    }
    __syncthreads();
    for (int t = threadIdx.x; t < kPrSlot; t += kBlock)
      part[static_cast<int64_t>(blockIdx.x) * kPrSlot + t] = ((s_part[0][t] + s_part[1][t]) + s_part[2][t]) + s_part[3][t];
  }
}

// dprobes[t] = sum of the slots' entry t.  Workgroup k takes entries
// [64k, 64k + 64); thread (t, q) adds slots q, q + 16, ... in order (loads
// issued kPrRedBatch at a time), then the 16 phases are added in phase order.
constexpr int kPrRedCols = 64;
constexpr int kPrRedPhases = 16;
constexpr int kPrRedBatch = 32;

__global__ __launch_bounds__(kPrRedCols * kPrRedPhases) void phase_probe_dprobes_reduce(const float* __restrict__ part,
                                                                                        int slots,
                                                                                        float* __restrict__ dprobes) {
  __shared__ float s_q[kPrRedPhases][kPrRedCols];
  const int c = threadIdx.x % kPrRedCols, q = threadIdx.x / kPrRedCols;
  const int t = blockIdx.x * kPrRedCols + c;
  float s = 0.f;
  for (int k0 = q; k0 < slots; k0 += kPrRedPhases * kPrRedBatch) {
    float v[kPrRedBatch];
#pragma unroll
    for (int i = 0; i < kPrRedBatch; ++i) {
      const int k = k0 + i * kPrRedPhases;
      v[i] = k < slots ? part[static_cast<int64_t>(k) * kPrSlot + t] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < kPrRedBatch; ++i) s += v[i];
  }
  s_q[q][c] = s;
  __syncthreads();
  if (q == 0) {
    float u = 0.f;
    for (int i = 0; i < kPrRedPhases; ++i) u += s_q[i][c];
    dprobes[t] = u;
  }
}

PrGeom pr_geom(const dwarf_phase_probe_fwd_args& a) {
  PrGeom gm;
  gm.B = a.B; gm.H = a.H; gm.N = a.N;
  gm.start = a.start < 0 ? 0 : (a.start > a.N ? a.N : a.start);
  gm.end = a.end < gm.start ? gm.start : (a.end > a.N ? a.N : a.end);
  gm.rows = static_cast<int64_t>(a.B) * a.H * a.N;
  return gm;
}

int pr_wgs(int64_t rows, int per_cu) {
  const int64_t steps = (rows + kPrRows - 1) / kPrRows;
  return static_cast<int>(steps < kPrCus * per_cu ? steps : kPrCus * per_cu);
}

}  // namespace

size_t phase_probe_bwd_workspace(const dwarf_phase_probe_bwd_args& a) {
  const int64_t rows = static_cast<int64_t>(a.fwd.B) * a.fwd.H * a.fwd.N;
  return rows > 0 ? static_cast<size_t>(pr_wgs(rows, pr_bwd_wgs_per_cu(true))) * kPrSlot * sizeof(float) : 0;
}

hipError_t launch_phase_probe_fwd(const dwarf_phase_probe_fwd_args& a, hipStream_t stream) {
  const PrGeom gm = pr_geom(a);
  if (gm.rows == 0) return hipSuccess;
  const int wgs = pr_wgs(gm.rows, kPrWgsPerCu);
  if (a.dtype == DWARF_BF16)
    hipLaunchKernelGGL(phase_probe_fwd_kernel<bf16>, dim3(wgs), dim3(kBlock), 0, stream,
                       static_cast<const bf16*>(a.x), a.x_stride[0], a.x_stride[1], a.x_stride[2], a.probes, a.out,
                       a.out_stride[0], a.out_stride[1], a.out_stride[2], a.out_stride[3], gm);
  else
    hipLaunchKernelGGL(phase_probe_fwd_kernel<float>, dim3(wgs), dim3(kBlock), 0, stream,
                       static_cast<const float*>(a.x), a.x_stride[0], a.x_stride[1], a.x_stride[2], a.probes, a.out,
                       a.out_stride[0], a.out_stride[1], a.out_stride[2], a.out_stride[3], gm);
  return hipGetLastError();
}

hipError_t launch_phase_probe_bwd(const dwarf_phase_probe_bwd_args& a, hipStream_t stream) {
  const dwarf_phase_probe_fwd_args& f = a.fwd;
  const PrGeom gm = pr_geom(f);
  if (gm.rows == 0) return hipSuccess;
  const bool dp = a.dprobes != nullptr;
  const int wgs = pr_wgs(gm.rows, pr_bwd_wgs_per_cu(dp));
  float* part = static_cast<float*>(a.workspace);
#define DWARF_PR_BWD(T, DP)                                                                                          \
  hipLaunchKernelGGL((phase_probe_bwd_kernel<T, DP>), dim3(wgs), dim3(kBlock), 0, stream,                           \
                     static_cast<const T*>(f.x), f.x_stride[0], f.x_stride[1], f.x_stride[2], f.probes, a.dout,      \
                     a.dout_stride[0], a.dout_stride[1], a.dout_stride[2], a.dout_stride[3], static_cast<T*>(a.dx),  \
                     a.dx_stride[0], a.dx_stride[1], a.dx_stride[2], part, gm)
  if (f.dtype == DWARF_BF16) {
    if (dp) DWARF_PR_BWD(bf16, true); else DWARF_PR_BWD(bf16, false);
  } else {
    if (dp) DWARF_PR_BWD(float, true); else DWARF_PR_BWD(float, false);
  }
#undef DWARF_PR_BWD
  if (dp)
    hipLaunchKernelGGL(phase_probe_dprobes_reduce, dim3(kPrSlot / kPrRedCols), dim3(kPrRedCols * kPrRedPhases), 0,
                       stream, part, wgs, a.dprobes);
  return hipGetLastError();
}

}  // namespace dwarf
