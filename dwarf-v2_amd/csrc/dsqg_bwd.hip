// DSQG backward (reference: _DSQGV18GroupedFn.backward dsqg:2354-2552 and
// the kernels _compute_D_v18_grouped dsqg:1263-1289, _bwd_dq_v18_grouped
// dsqg:1296-1488, _bwd_dkdv_v18_grouped dsqg:1734-1955).
//
// Launches on the caller's stream:
//  1. dq kernel (dsqg_bwd_dq.hip), query-centric: delta, dQ, dY and one
//     partial of dPB / dSE / dPhaseBase / dPhaseGain per workgroup.
//  2. two reduce kernels: fixed-order sums of those partials (stage 1 over
//     groups of 16 rows, stage 2 over the groups), so the parameter gradients
//     are bitwise reproducible.
//  3. dkdv kernel, key-centric.  For each key row m and each query head of
//     its KV group, the pairs n = m + delta are revisited to accumulate dK,
//     dV and dZ in registers; the GQA head sum happens in-kernel.
#include "common.h"
#include "dsqg_internal.h"

namespace dwarf {
namespace {


__host__ __device__ constexpr size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

template <typename T, int SHIFT, int L, bool FAST>
__global__ __launch_bounds__(kBlock) void dsqg_bwd_dkdv_kernel(const dwarf_dsqg_bwd_args a,
                                                              const float* __restrict__ delta_ws, int tiles, int total) {
  constexpr int HD = kHeadDim;
  constexpr int DPL = HD / L;
  constexpr int KPB = kBlock / L;
  constexpr int SEG = HD / kPlanes;
  const dwarf_dsqg_fwd_args& f = a.fwd;

  extern __shared__ float smem[];
  float* s_se = smem;                               // [J][64]
  int* s_off = reinterpret_cast<int*>(s_se + f.J * HD);

  const int work = xcd_remap(blockIdx.x, total);
  const int bhk = work / tiles;
  const int tile = work - bhk * tiles;
  const int b = bhk / f.H_kv;
  const int hk = bhk - b * f.H_kv;
  const int group = f.H / f.H_kv;

  for (int i = threadIdx.x; i < f.J * HD; i += kBlock) {
    const int j = i / HD, d = i - j * HD;
    const float e = f.scale_embed[j * f.se_stride[0] + d * f.se_stride[1]];
    s_se[i] = f.se_round_bf16 ? round_bf16(e) : e;
  }
  for (int j = threadIdx.x; j < f.J; j += kBlock) s_off[j] = f.offsets[j];
  __syncthreads();

  const int lane = threadIdx.x;
  const int g = lane % L;
  const int m = tile * KPB + lane / L;
  if (m >= f.N) return;  // no barriers below
  const int wave_m_first = uniform(tile * KPB + (lane / kWave) * (kWave / L));
  const int wave_m_last = wave_m_first + kWave / L - 1;
  const int64_t mm = m;

  float kv[DPL], vv[DPL], dk[DPL], dv[DPL];
  load_f32<T, DPL>(reinterpret_cast<const T*>(f.k) + b * f.k_stride[0] + hk * f.k_stride[1] + mm * f.k_stride[2] + g * DPL, kv);
  load_f32<T, DPL>(reinterpret_cast<const T*>(f.v) + b * f.v_stride[0] + hk * f.v_stride[1] + mm * f.v_stride[2] + g * DPL, vv);
#pragma unroll
  for (int d = 0; d < DPL; ++d) { dk[d] = 0.f; dv[d] = 0.f; }
  const float4 z4 = *reinterpret_cast<const float4*>(f.z_pre + b * f.z_stride[0] + hk * f.z_stride[1] + mm * f.z_stride[2]);
  const float zs[4] = {z4.x, z4.y, z4.z, z4.w};
  float dz[4] = {0.f, 0.f, 0.f, 0.f};
  constexpr float scale = 0.125f;

  for (int hh = 0; hh < group; ++hh) {
    const int h = hk * group + hh;
    const int bh = b * f.H + h;
    const T* qbase = reinterpret_cast<const T*>(f.q) + b * f.q_stride[0] + h * f.q_stride[1] + g * DPL;
    const T* dobase = reinterpret_cast<const T*>(a.dout) + b * a.dout_stride[0] + h * a.dout_stride[1] + g * DPL;
    const float* lsebase = f.lse + b * f.lse_stride[0] + h * f.lse_stride[1];
    const float* dltbase = delta_ws + static_cast<int64_t>(bh) * f.N;
    const float* ybase = f.y_pre + b * f.y_stride[0] + h * f.y_stride[1];

    for (int j = 0; j < f.J; ++j) {
      const int delta = s_off[j];
      if (wave_m_first + delta >= f.N || wave_m_last + delta < f.query_start) continue;
      const int n = m + delta;
      if (n < 0 || n >= f.N) continue;
      const int64_t nn = n;
      const float lse = lsebase[nn * f.lse_stride[2]];
      if (!(lse > -INFINITY)) continue;
      float qn[DPL], don[DPL];
      load_f32<T, DPL>(qbase + nn * f.q_stride[2], qn);
      const float* e = s_se + j * HD + g * DPL;
      float dot = 0.f;
#pragma unroll
      for (int d = 0; d < DPL; ++d) dot = fmaf(qn[d], kv[d] + e[d], dot);
      dot = group_sum<L>(dot);
      const float P = dexp<FAST>(fmaf(dot, scale, f.pos_bias[j * f.pb_stride[0] + h * f.pb_stride[1]]) - lse);

      load_f32<T, DPL>(dobase + nn * a.dout_stride[2], don);
      float gd = 0.f;
#pragma unroll
      for (int d = 0; d < DPL; ++d) gd = fmaf(don[d], vv[d], gd);
      // dV contribution with rotated channels replaced below.
      float dva[4] = {0.f, 0.f, 0.f, 0.f}, dvb[4] = {0.f, 0.f, 0.f, 0.f};
      bool far = j >= f.J_small;
      if (far) {
        const int i = j - f.J_small;
        const float4 y4 = *reinterpret_cast<const float4*>(ybase + nn * f.y_stride[2]);
        const float ys[4] = {y4.x, y4.y, y4.z, y4.w};
#pragma unroll
        for (int r = 0; r < kPlanes; ++r) {
          const int ch = r * SEG + SHIFT;
          if (ch / DPL != g) continue;
          const int la = ch % DPL;
          const float pg = f.phase_gain[i * f.pgain_stride[0] + h * f.pgain_stride[1] + r];
          const float theta = f.phase_base[i * f.pbase_stride[0] + h * f.pbase_stride[1] + r] + pg * ys[r] * zs[r];
          float sn, cs;
          dsincos<FAST>(theta, &sn, &cs);
          const float va = vv[la], vb = vv[la + 1];
          const float da = don[la], db = don[la + 1];
          gd += da * (cs * va - sn * vb - va) + db * (sn * va + cs * vb - vb);
          const float t = P * (da * (-va * sn - vb * cs) + db * (va * cs - vb * sn));
          dz[r] = fmaf(t * pg, ys[r], dz[r]);
          dva[r] = cs * da + sn * db;   // (R^T dO)_a
          dvb[r] = -sn * da + cs * db;  // (R^T dO)_b
        }
      }
      gd = group_sum<L>(gd);
      const float dS = P * (gd - dltbase[nn]);
      const float cds = scale * dS;
#pragma unroll
      for (int d = 0; d < DPL; ++d) {
        dk[d] = fmaf(cds, qn[d], dk[d]);
        dv[d] = fmaf(P, don[d], dv[d]);
      }
      if (far) {
#pragma unroll
        for (int r = 0; r < kPlanes; ++r) {
          const int ch = r * SEG + SHIFT;
          if (ch / DPL != g) continue;
          const int la = ch % DPL;
          dv[la] = fmaf(P, dva[r] - don[la], dv[la]);
          dv[la + 1] = fmaf(P, dvb[r] - don[la + 1], dv[la + 1]);
        }
      }
    }
  }

  store_from_f32<T, DPL>(reinterpret_cast<T*>(a.dk) + b * a.dk_stride[0] + hk * a.dk_stride[1] + mm * a.dk_stride[2] + g * DPL, dk);
  store_from_f32<T, DPL>(reinterpret_cast<T*>(a.dv) + b * a.dv_stride[0] + hk * a.dv_stride[1] + mm * a.dv_stride[2] + g * DPL, dv);
  float dzo[4];
#pragma unroll
  for (int r = 0; r < kPlanes; ++r) dzo[r] = group_sum<L>(dz[r]);
  if (g == 0)
    *reinterpret_cast<float4*>(a.dz_pre + (static_cast<int64_t>(bhk) * f.N + m) * kPlanes) =
        make_float4(dzo[0], dzo[1], dzo[2], dzo[3]);
}

// ---- bf16 dkdv: packed rows and v_dot2 ------------------------------------
// Same mapping as dsqg_bwd_dkdv_kernel (two lanes per key, 32 dims each).
// <q, k>, <q, e_j> and <dO, v> are v_dot2_f32_bf16 on the packed rows (exact
// bf16 products, fp32 sums); the rank-1 updates dK += c dS q and dV += P dO
// stay fp32 FMAs on the widened rows, and the rotated MOVT channels of dV get
// an fp32 correction term.
constexpr int kERowDkdv = 72;  // bf16 E row stride (elements)

__device__ __forceinline__ float dot2b(uint32_t a, uint32_t b, float c) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
}

template <int SHIFT>
__global__ __launch_bounds__(kBlock) void dsqg_bwd_dkdv_bf16_v2(const dwarf_dsqg_bwd_args a,
                                                                const float* __restrict__ delta_ws, int tiles,
                                                                int total) {
  constexpr int HD = kHeadDim, DPL = 32, KPB = kBlock / 2, SEG = HD / kPlanes;
  constexpr float kScale = 0.125f;
  const dwarf_dsqg_fwd_args& f = a.fwd;
  extern __shared__ float smem[];
  int* s_off = reinterpret_cast<int*>(smem);
  uint16_t* sE = reinterpret_cast<uint16_t*>(smem + ((f.J + 3) & ~3));   // [J][kERowDkdv]

  const int work = xcd_remap(blockIdx.x, total);
  const int bhk = work / tiles;
  const int tile = work - bhk * tiles;
  const int b = bhk / f.H_kv;
  const int hk = bhk - b * f.H_kv;
  const int group = f.H / f.H_kv;
  for (int i = threadIdx.x; i < f.J * HD; i += kBlock) {
    const int j = i / HD, d = i - j * HD;
    float e = f.scale_embed[j * f.se_stride[0] + d * f.se_stride[1]];
    if (f.se_round_bf16) e = round_bf16(e);
    sE[j * kERowDkdv + d] = f32_to_bf16_bits(e);
  }
  for (int j = threadIdx.x; j < f.J; j += kBlock) s_off[j] = f.offsets[j];
  __syncthreads();

  const int lane = threadIdx.x;
  const int g = lane & 1;
  const int m = tile * KPB + lane / 2;
  if (m >= f.N) return;  // no barriers below
  const int wave_m_first = uniform(tile * KPB + (lane / kWave) * (kWave / 2));
  const int wave_m_last = wave_m_first + kWave / 2 - 1;
  const int64_t mm = m;

  uint32_t k32[16], v32[16];
  {
    const uint4* k4 = reinterpret_cast<const uint4*>(reinterpret_cast<const bf16*>(f.k) + b * f.k_stride[0] +
                                                     hk * f.k_stride[1] + mm * f.k_stride[2] + g * DPL);
    const uint4* v4 = reinterpret_cast<const uint4*>(reinterpret_cast<const bf16*>(f.v) + b * f.v_stride[0] +
                                                     hk * f.v_stride[1] + mm * f.v_stride[2] + g * DPL);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 x = k4[i], y = v4[i];
      k32[4 * i] = x.x; k32[4 * i + 1] = x.y; k32[4 * i + 2] = x.z; k32[4 * i + 3] = x.w;
      v32[4 * i] = y.x; v32[4 * i + 1] = y.y; v32[4 * i + 2] = y.z; v32[4 * i + 3] = y.w;
    }
  }
  float dk[DPL], dv[DPL];
#pragma unroll
  for (int d = 0; d < DPL; ++d) { dk[d] = 0.f; dv[d] = 0.f; }
  const float4 z4 = *reinterpret_cast<const float4*>(f.z_pre + b * f.z_stride[0] + hk * f.z_stride[1] + mm * f.z_stride[2]);
  const float zs[4] = {z4.x, z4.y, z4.z, z4.w};
  float dz[4] = {0.f, 0.f, 0.f, 0.f};

  for (int hh = 0; hh < group; ++hh) {
    const int h = hk * group + hh;
    const int bh = b * f.H + h;
    const bf16* qbase = reinterpret_cast<const bf16*>(f.q) + b * f.q_stride[0] + h * f.q_stride[1] + g * DPL;
    const bf16* dobase = reinterpret_cast<const bf16*>(a.dout) + b * a.dout_stride[0] + h * a.dout_stride[1] + g * DPL;
    const float* lsebase = f.lse + b * f.lse_stride[0] + h * f.lse_stride[1];
    const float* dltbase = delta_ws + static_cast<int64_t>(bh) * f.N;
    const float* ybase = f.y_pre + b * f.y_stride[0] + h * f.y_stride[1];
    for (int j = 0; j < f.J; ++j) {
      const int delta = s_off[j];
      if (wave_m_first + delta >= f.N || wave_m_last + delta < f.query_start) continue;
      const int n = m + delta;
      if (n < 0 || n >= f.N) continue;
      const int64_t nn = n;
      const float lse = lsebase[nn * f.lse_stride[2]];
      if (!(lse > -INFINITY)) continue;
      uint32_t q32[16], o32[16];
      const uint4* q4 = reinterpret_cast<const uint4*>(qbase + nn * f.q_stride[2]);
      const uint4* o4 = reinterpret_cast<const uint4*>(dobase + nn * a.dout_stride[2]);
      const uint4* e4 = reinterpret_cast<const uint4*>(sE + j * kERowDkdv + g * DPL);
      float dot = 0.f, gd = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint4 x = q4[i], e = e4[i], y = o4[i];
        q32[4 * i] = x.x; q32[4 * i + 1] = x.y; q32[4 * i + 2] = x.z; q32[4 * i + 3] = x.w;
        o32[4 * i] = y.x; o32[4 * i + 1] = y.y; o32[4 * i + 2] = y.z; o32[4 * i + 3] = y.w;
        dot = dot2b(x.x, k32[4 * i], dot); dot = dot2b(x.y, k32[4 * i + 1], dot);
        dot = dot2b(x.z, k32[4 * i + 2], dot); dot = dot2b(x.w, k32[4 * i + 3], dot);
        dot = dot2b(x.x, e.x, dot); dot = dot2b(x.y, e.y, dot);
        dot = dot2b(x.z, e.z, dot); dot = dot2b(x.w, e.w, dot);
        gd = dot2b(y.x, v32[4 * i], gd); gd = dot2b(y.y, v32[4 * i + 1], gd);
        gd = dot2b(y.z, v32[4 * i + 2], gd); gd = dot2b(y.w, v32[4 * i + 3], gd);
      }
      dot = group_sum<2>(dot);
      const float P = __expf(fmaf(dot, kScale, f.pos_bias[j * f.pb_stride[0] + h * f.pb_stride[1]]) - lse);
      float corr_a[4] = {0.f, 0.f, 0.f, 0.f}, corr_b[4] = {0.f, 0.f, 0.f, 0.f};
      const bool far = j >= f.J_small;
      if (far) {
        const int i = j - f.J_small;
        const float4 y4 = *reinterpret_cast<const float4*>(ybase + nn * f.y_stride[2]);
        const float ys[4] = {y4.x, y4.y, y4.z, y4.w};
#pragma unroll
        for (int r = 0; r < kPlanes; ++r) {
          const int ch = r * SEG + SHIFT;
          if (ch / DPL != g) continue;
          const int la = ch % DPL, lb = la + 1;
          const float va = (la & 1) ? bf16_hi(v32[la >> 1]) : bf16_lo(v32[la >> 1]);
          const float vb = (lb & 1) ? bf16_hi(v32[lb >> 1]) : bf16_lo(v32[lb >> 1]);
          const float da = (la & 1) ? bf16_hi(o32[la >> 1]) : bf16_lo(o32[la >> 1]);
          const float db = (lb & 1) ? bf16_hi(o32[lb >> 1]) : bf16_lo(o32[lb >> 1]);
          const float pg = f.phase_gain[i * f.pgain_stride[0] + h * f.pgain_stride[1] + r];
          const float theta = f.phase_base[i * f.pbase_stride[0] + h * f.pbase_stride[1] + r] + pg * ys[r] * zs[r];
          float sn, cs;
          dsincos<true>(theta, &sn, &cs);
          gd += da * (cs * va - sn * vb - va) + db * (sn * va + cs * vb - vb);
          const float t = P * (da * (-va * sn - vb * cs) + db * (va * cs - vb * sn));
          dz[r] = fmaf(t * pg, ys[r], dz[r]);
          corr_a[r] = (cs - 1.f) * da + sn * db;   // (R^T dO - dO)_a
          corr_b[r] = -sn * da + (cs - 1.f) * db;  // (R^T dO - dO)_b
        }
      }
      gd = group_sum<2>(gd);
      const float dS = P * (gd - dltbase[nn]);
      const float cdS = kScale * dS;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        dk[2 * i] = fmaf(cdS, bf16_lo(q32[i]), dk[2 * i]);
        dk[2 * i + 1] = fmaf(cdS, bf16_hi(q32[i]), dk[2 * i + 1]);
        dv[2 * i] = fmaf(P, bf16_lo(o32[i]), dv[2 * i]);
        dv[2 * i + 1] = fmaf(P, bf16_hi(o32[i]), dv[2 * i + 1]);
      }
      if (far) {
#pragma unroll
        for (int r = 0; r < kPlanes; ++r) {
          const int ch = r * SEG + SHIFT;
          if (ch / DPL != g) continue;
          const int la = ch % DPL;
          dv[la] = fmaf(P, corr_a[r], dv[la]);
          dv[la + 1] = fmaf(P, corr_b[r], dv[la + 1]);
        }
      }
    }
  }
  store_from_f32<bf16, DPL>(reinterpret_cast<bf16*>(a.dk) + b * a.dk_stride[0] + hk * a.dk_stride[1] + mm * a.dk_stride[2] + g * DPL, dk);
  store_from_f32<bf16, DPL>(reinterpret_cast<bf16*>(a.dv) + b * a.dv_stride[0] + hk * a.dv_stride[1] + mm * a.dv_stride[2] + g * DPL, dv);
  float dzo[4];
#pragma unroll
  for (int r = 0; r < kPlanes; ++r) dzo[r] = group_sum<2>(dz[r]);
  if (g == 0)
    *reinterpret_cast<float4*>(a.dz_pre + (static_cast<int64_t>(bhk) * f.N + m) * kPlanes) =
        make_float4(dzo[0], dzo[1], dzo[2], dzo[3]);
}

hipError_t launch_dkdv_bf16_v2(const dwarf_dsqg_bwd_args& a, const BwdWorkspace& ws, hipStream_t stream) {
  const dwarf_dsqg_fwd_args& f = a.fwd;
  constexpr int KPB = kBlock / 2;
  const float* delta = reinterpret_cast<const float*>(static_cast<char*>(a.workspace) + ws.delta_off);
  const int tiles = (f.N + KPB - 1) / KPB;
  const int total = tiles * f.B * f.H_kv;
  const size_t lds = static_cast<size_t>((f.J + 3) & ~3) * sizeof(int) + static_cast<size_t>(f.J) * kERowDkdv * 2;
#define DWARF_DKDV2_CASE(S) \
  case S: hipLaunchKernelGGL(dsqg_bwd_dkdv_bf16_v2<S>, dim3(total), dim3(kBlock), lds, stream, a, delta, tiles, total); break;
  switch (f.plane_shift) {
    DWARF_DKDV2_CASE(0) DWARF_DKDV2_CASE(1) DWARF_DKDV2_CASE(2) DWARF_DKDV2_CASE(3) DWARF_DKDV2_CASE(4)
    DWARF_DKDV2_CASE(5) DWARF_DKDV2_CASE(6) DWARF_DKDV2_CASE(7) DWARF_DKDV2_CASE(8) DWARF_DKDV2_CASE(9)
    DWARF_DKDV2_CASE(10) DWARF_DKDV2_CASE(11) DWARF_DKDV2_CASE(12) DWARF_DKDV2_CASE(13) DWARF_DKDV2_CASE(14)
    default: return hipErrorInvalidValue;
  }
#undef DWARF_DKDV2_CASE
  return hipGetLastError();
}

// ---- fixed-order reduction of the dq partials -----------------------------
constexpr int kRedRows = 16;  // rows summed per stage-1 group

struct RedArray {
  const float* in;   // [nseg * rows][cols]
  float* tmp;        // [nseg][groups][cols]
  int nseg, rows, cols, groups;
};

struct RedPlan {
  RedArray arr[3];   // 0: dSE, 1: dPB, 2: dPhase
  int blocks1[3];    // stage-1 blocks per array
  int outputs[3];    // stage-2 outputs per array
};

__global__ __launch_bounds__(kBlock) void dsqg_bwd_reduce1(RedPlan p) {
  int blk = blockIdx.x, ai = 0;
  while (ai < 2 && blk >= p.blocks1[ai]) blk -= p.blocks1[ai++];
  const RedArray& A = p.arr[ai];
  const int cblocks = (A.cols + kBlock - 1) / kBlock;
  const int cb = blk % cblocks;
  const int grp = (blk / cblocks) % A.groups;
  const int seg = blk / (cblocks * A.groups);
  const int col = cb * kBlock + threadIdx.x;
  if (seg >= A.nseg || col >= A.cols) return;
  const int r0 = grp * kRedRows;
  const int r1 = min(A.rows, r0 + kRedRows);
  const float* src = A.in + (static_cast<int64_t>(seg) * A.rows + r0) * A.cols + col;
  float sum = 0.f;
  for (int r = r0; r < r1; ++r, src += A.cols) sum += *src;
  A.tmp[(static_cast<int64_t>(seg) * A.groups + grp) * A.cols + col] = sum;
}

__global__ __launch_bounds__(kBlock) void dsqg_bwd_reduce2(RedPlan p, const dwarf_dsqg_bwd_args a) {
  int idx = blockIdx.x * kBlock + threadIdx.x, ai = 0;
  while (ai < 2 && idx >= p.outputs[ai]) idx -= p.outputs[ai++];
  if (idx >= p.outputs[ai]) return;
  const RedArray& A = p.arr[ai];
  const int seg = idx / A.cols, col = idx - seg * A.cols;
  const float* src = A.tmp + static_cast<int64_t>(seg) * A.groups * A.cols + col;
  float sum = 0.f;
  for (int gi = 0; gi < A.groups; ++gi, src += A.cols) sum += *src;
  const dwarf_dsqg_fwd_args& f = a.fwd;
  if (ai == 0) {
    a.dscale_embed[col] = sum;                          // [J][64]
  } else if (ai == 1) {
    a.dpos_bias[col * f.H + seg] = sum;                 // [J][H], seg = h
  } else {
    const int i = col / 8, rk = col % 8;                // col = i*8 + r*2 + kind
    float* dst = (rk & 1) ? a.dphase_gain : a.dphase_base;
    dst[(i * f.H + seg) * kPlanes + (rk >> 1)] = sum;   // [J_L][H][4]
  }
}

RedPlan make_red_plan(const dwarf_dsqg_bwd_args& a, const BwdWorkspace& ws) {
  const dwarf_dsqg_fwd_args& f = a.fwd;
  char* base = static_cast<char*>(a.workspace);
  float* red = reinterpret_cast<float*>(base + ws.red_off);
  const int R = f.B * ws.dq_ntg;
  RedPlan p;
  p.arr[0] = {reinterpret_cast<const float*>(base + ws.part_se_off), red, 1, ws.dq_wgs, f.J * kHeadDim,
              ws.red_groups_se};
  red += static_cast<size_t>(ws.red_groups_se) * f.J * kHeadDim;
  p.arr[1] = {reinterpret_cast<const float*>(base + ws.part_pb_off), red, f.H, R, f.J, ws.red_groups_pb};
  red += static_cast<size_t>(f.H) * ws.red_groups_pb * f.J;
  p.arr[2] = {reinterpret_cast<const float*>(base + ws.part_ph_off), red, f.H, 4 * R, f.J_large * 8,
              ws.red_groups_ph};
  for (int i = 0; i < 3; ++i) {
    const RedArray& A = p.arr[i];
    p.blocks1[i] = A.cols > 0 ? A.nseg * A.groups * ((A.cols + kBlock - 1) / kBlock) : 0;
    p.outputs[i] = A.nseg * A.cols;
  }
  return p;
}

template <typename T, int L, bool FAST>
hipError_t launch_dkdv_typed(const dwarf_dsqg_bwd_args& a, const BwdWorkspace& ws, hipStream_t stream) {
  const dwarf_dsqg_fwd_args& f = a.fwd;
  constexpr int KPB = kBlock / L;
  const float* delta = reinterpret_cast<const float*>(static_cast<char*>(a.workspace) + ws.delta_off);
  const int tiles = (f.N + KPB - 1) / KPB;
  const int total_k = tiles * f.B * f.H_kv;
  const size_t lds_k = static_cast<size_t>(f.J) * (kHeadDim + 1) * sizeof(float);
#define DWARF_DKDV_CASE(S)                                                                                    \
  case S:                                                                                                     \
    hipLaunchKernelGGL((dsqg_bwd_dkdv_kernel<T, S, L, FAST>), dim3(total_k), dim3(kBlock), lds_k, stream, a, \
                       delta, tiles, total_k);                                                                \
    break;
  switch (f.plane_shift) {
    DWARF_DKDV_CASE(0) DWARF_DKDV_CASE(1) DWARF_DKDV_CASE(2) DWARF_DKDV_CASE(3) DWARF_DKDV_CASE(4)
    DWARF_DKDV_CASE(5) DWARF_DKDV_CASE(6) DWARF_DKDV_CASE(7) DWARF_DKDV_CASE(8) DWARF_DKDV_CASE(9)
    DWARF_DKDV_CASE(10) DWARF_DKDV_CASE(11) DWARF_DKDV_CASE(12) DWARF_DKDV_CASE(13) DWARF_DKDV_CASE(14)
    default:
      return hipErrorInvalidValue;
  }
#undef DWARF_DKDV_CASE
  return hipGetLastError();
}

constexpr int kLanesBwd = 2;

}  // namespace

BwdWorkspace bwd_workspace_layout(const dwarf_dsqg_bwd_args& a) {
  const dwarf_dsqg_fwd_args& f = a.fwd;
  BwdWorkspace w{};
  constexpr int kTile = 128;
  w.dq_tiles = (f.N + kTile - 1) / kTile;
  const int total_tiles = w.dq_tiles * f.B * f.H;
  // Two 4-wave workgroups fit per CU (VGPR/LDS bound): size the tile groups so
  // every workgroup is resident at once (at most 512 on 256 CUs).
  w.dq_tpw = (total_tiles + 511) / 512;
  if (w.dq_tpw < 1) w.dq_tpw = 1;
  if (w.dq_tpw > 8) w.dq_tpw = 8;
  if (w.dq_tpw > w.dq_tiles) w.dq_tpw = w.dq_tiles > 0 ? w.dq_tiles : 1;
  w.dq_ntg = (w.dq_tiles + w.dq_tpw - 1) / w.dq_tpw;
  w.dq_wgs = f.B * f.H * w.dq_ntg;
  const int JL = f.J_large > 0 ? f.J_large : 1;
  const int R = f.B * w.dq_ntg;
  w.red_groups_se = (w.dq_wgs + kRedRows - 1) / kRedRows;
  w.red_groups_pb = (R + kRedRows - 1) / kRedRows;
  w.red_groups_ph = (4 * R + kRedRows - 1) / kRedRows;
  size_t off = 0;
  w.delta_off = off;
  w.delta_bytes = static_cast<size_t>(f.B) * f.H * f.N * sizeof(float);
  off += align256(w.delta_bytes);
  w.part_se_off = off;
  w.part_se_bytes = static_cast<size_t>(w.dq_wgs) * f.J * kHeadDim * sizeof(float);
  off += align256(w.part_se_bytes);
  w.part_pb_off = off;
  w.part_pb_bytes = static_cast<size_t>(w.dq_wgs) * f.J * sizeof(float);
  off += align256(w.part_pb_bytes);
  w.part_ph_off = off;
  w.part_ph_bytes = static_cast<size_t>(w.dq_wgs) * 4 * JL * 8 * sizeof(float);
  off += align256(w.part_ph_bytes);
  w.red_off = off;
  w.red_bytes = (static_cast<size_t>(w.red_groups_se) * f.J * kHeadDim +
                 static_cast<size_t>(f.H) * w.red_groups_pb * f.J +
                 static_cast<size_t>(f.H) * w.red_groups_ph * JL * 8) * sizeof(float);
  off += align256(w.red_bytes);
  w.total = off;
  return w;
}

hipError_t launch_dsqg_bwd(const dwarf_dsqg_bwd_args& a, const BwdWorkspace& ws, hipStream_t stream, bool do_dq,
                           bool do_dkdv) {
  if (do_dq) {
    hipError_t e = launch_dsqg_bwd_dq(a, ws, stream);
    if (e != hipSuccess) return e;
    const RedPlan p = make_red_plan(a, ws);
    const int b1 = p.blocks1[0] + p.blocks1[1] + p.blocks1[2];
    const int o2 = p.outputs[0] + p.outputs[1] + p.outputs[2];
    if (b1 > 0) hipLaunchKernelGGL(dsqg_bwd_reduce1, dim3(b1), dim3(kBlock), 0, stream, p);
    if (o2 > 0) hipLaunchKernelGGL(dsqg_bwd_reduce2, dim3((o2 + kBlock - 1) / kBlock), dim3(kBlock), 0, stream, p, a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (do_dkdv) {
    if (a.fwd.dtype == DWARF_BF16) return launch_dkdv_bf16_v2(a, ws, stream);
    return launch_dkdv_typed<float, kLanesBwd, false>(a, ws, stream);
  }
  return hipSuccess;
}

}  // namespace dwarf
