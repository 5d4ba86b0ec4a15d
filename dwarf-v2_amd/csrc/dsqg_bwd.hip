// DSQG backward (reference: _DSQGV18GroupedFn.backward dsqg:2354-2552 and
// the kernels _compute_D_v18_grouped dsqg:1263-1289, _bwd_dq_v18_grouped
// dsqg:1296-1488, _bwd_dkdv_v18_grouped dsqg:1734-1955).
//
// Three launches on the caller's stream:
//  1. dq kernel, query-centric.  Computes delta = <dO, O> for its rows
//     (writing it to the workspace for launch 2), then for every offset the
//     recomputed probability P, the value gradient g = <dO, R v>, dS, dQ and
//     dY.  Per-offset sums over its queries (dPB, dSE, dPhaseBase,
//     dPhaseGain) are formed in LDS and written as one partial per
//     workgroup; no atomics.
//  2. dkdv kernel, key-centric.  For each key row m and each query head of
//     its KV group, the pairs n = m + delta are revisited to accumulate dK,
//     dV and dZ in registers; the GQA head sum happens in-kernel.
//  3. reduce kernel: sums the workgroup partials in a fixed order, so the
//     parameter gradients are bitwise reproducible.
#include "common.h"
#include "dsqg_internal.h"

namespace dwarf {
namespace {

constexpr int kChunk = 8;  // offsets per LDS reduction round in the dq kernel

__host__ __device__ constexpr size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

template <typename T, int SHIFT, int L, bool FAST>
__global__ __launch_bounds__(kBlock) void dsqg_bwd_dq_kernel(const dwarf_dsqg_bwd_args a, float* __restrict__ delta_ws,
                                                            float* __restrict__ part_se, float* __restrict__ part_pb,
                                                            float* __restrict__ part_ph, int tiles, int total) {
  constexpr int HD = kHeadDim;
  constexpr int DPL = HD / L;
  constexpr int QPB = kBlock / L;
  constexpr int SEG = HD / kPlanes;
  const dwarf_dsqg_fwd_args& f = a.fwd;

  extern __shared__ float smem[];
  float* s_se = smem;                                // [J][64]
  float* s_q = s_se + f.J * HD;                      // [QPB][64]
  float* s_ds = s_q + QPB * HD;                      // [QPB][kChunk]
  float* s_dth = s_ds + QPB * kChunk;                // [QPB][kChunk][4]
  float* s_dthyz = s_dth + QPB * kChunk * kPlanes;   // [QPB][kChunk][4]
  float* s_pb = s_dthyz + QPB * kChunk * kPlanes;    // [J]
  int* s_off = reinterpret_cast<int*>(s_pb + f.J);   // [J]

  const int work = xcd_remap(blockIdx.x, total);
  const int bh = work / tiles;
  const int tile = work - bh * tiles;
  const int b = bh / f.H;
  const int h = bh - b * f.H;
  const int hk = h / (f.H / f.H_kv);

  for (int i = threadIdx.x; i < f.J * HD; i += kBlock) {
    const int j = i / HD, d = i - j * HD;
    const float e = f.scale_embed[j * f.se_stride[0] + d * f.se_stride[1]];
    s_se[i] = f.se_round_bf16 ? round_bf16(e) : e;
  }
  for (int j = threadIdx.x; j < f.J; j += kBlock) {
    s_pb[j] = f.pos_bias[j * f.pb_stride[0] + h * f.pb_stride[1]];
    s_off[j] = f.offsets[j];
  }

  const int lane = threadIdx.x;
  const int g = lane % L;
  const int qi = lane / L;
  const int n = tile * QPB + qi;
  const bool row_ok = n < f.N;
  const bool row_live = row_ok && n >= f.query_start;
  const int wave_n_last = uniform(tile * QPB + (lane / kWave) * (kWave / L)) + kWave / L - 1;

  float q[DPL], dO[DPL], dq[DPL];
  float ys[4] = {0.f, 0.f, 0.f, 0.f};
  float dy[4] = {0.f, 0.f, 0.f, 0.f};
  float lse = -INFINITY, dlt = 0.f;
#pragma unroll
  for (int d = 0; d < DPL; ++d) { q[d] = 0.f; dO[d] = 0.f; dq[d] = 0.f; }
  if (row_live) {
    const int64_t nn = n;
    load_f32<T, DPL>(reinterpret_cast<const T*>(f.q) + b * f.q_stride[0] + h * f.q_stride[1] + nn * f.q_stride[2] + g * DPL, q);
    load_f32<T, DPL>(reinterpret_cast<const T*>(a.dout) + b * a.dout_stride[0] + h * a.dout_stride[1] +
                         nn * a.dout_stride[2] + g * DPL, dO);
    float o[DPL];
    load_f32<T, DPL>(reinterpret_cast<const T*>(f.out) + b * f.out_stride[0] + h * f.out_stride[1] +
                         nn * f.out_stride[2] + g * DPL, o);
#pragma unroll
    for (int d = 0; d < DPL; ++d) dlt = fmaf(dO[d], o[d], dlt);
    lse = f.lse[b * f.lse_stride[0] + h * f.lse_stride[1] + nn * f.lse_stride[2]];
    const float4 y4 = *reinterpret_cast<const float4*>(f.y_pre + b * f.y_stride[0] + h * f.y_stride[1] + nn * f.y_stride[2]);
    ys[0] = y4.x; ys[1] = y4.y; ys[2] = y4.z; ys[3] = y4.w;
  }
  dlt = group_sum<L>(dlt);
  if (row_ok && g == 0) delta_ws[static_cast<int64_t>(bh) * f.N + n] = dlt;
#pragma unroll
  for (int d = 0; d < DPL; ++d) s_q[qi * HD + g * DPL + d] = q[d];
  const bool has_mass = row_live && lse > -INFINITY;

  const T* kbase = reinterpret_cast<const T*>(f.k) + b * f.k_stride[0] + hk * f.k_stride[1] + g * DPL;
  const T* vbase = reinterpret_cast<const T*>(f.v) + b * f.v_stride[0] + hk * f.v_stride[1] + g * DPL;
  const float* zbase = f.z_pre + b * f.z_stride[0] + hk * f.z_stride[1];
  constexpr float scale = 0.125f;

  for (int j0 = 0; j0 < f.J; j0 += kChunk) {
    __syncthreads();  // s_q / tables ready; previous round's readers done
    for (int jj = 0; jj < kChunk; ++jj) {
      const int j = j0 + jj;
      float dS = 0.f;
      float dth[4] = {0.f, 0.f, 0.f, 0.f};
      float dthyz[4] = {0.f, 0.f, 0.f, 0.f};
      if (j < f.J) {
        const int delta = s_off[j];
        const int s = n - delta;
        if (wave_n_last >= delta && has_mass && s >= 0 && s < f.N) {
          float kv[DPL], vv[DPL];
          load_f32<T, DPL>(kbase + static_cast<int64_t>(s) * f.k_stride[2], kv);
          const float* e = s_se + j * HD + g * DPL;
#pragma unroll
          for (int d = 0; d < DPL; ++d) kv[d] += e[d];
          float dot = 0.f;
#pragma unroll
          for (int d = 0; d < DPL; ++d) dot = fmaf(q[d], kv[d], dot);
          dot = group_sum<L>(dot);
          const float P = dexp<FAST>(fmaf(dot, scale, s_pb[j]) - lse);

          load_f32<T, DPL>(vbase + static_cast<int64_t>(s) * f.v_stride[2], vv);
          float gd = 0.f;
#pragma unroll
          for (int d = 0; d < DPL; ++d) gd = fmaf(dO[d], vv[d], gd);
          if (j >= f.J_small) {
            const int i = j - f.J_small;
            const float4 zk = *reinterpret_cast<const float4*>(zbase + static_cast<int64_t>(s) * f.z_stride[2]);
            const float zs[4] = {zk.x, zk.y, zk.z, zk.w};
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
              const float da = dO[la], db = dO[la + 1];
              gd += da * (cs * va - sn * vb - va) + db * (sn * va + cs * vb - vb);
              const float t = P * (da * (-va * sn - vb * cs) + db * (va * cs - vb * sn));
              dth[r] = t;
              dthyz[r] = t * ys[r] * zs[r];
              dy[r] = fmaf(t * pg, zs[r], dy[r]);
            }
          }
          gd = group_sum<L>(gd);
          dS = P * (gd - dlt);
          const float cds = scale * dS;
#pragma unroll
          for (int d = 0; d < DPL; ++d) dq[d] = fmaf(cds, kv[d], dq[d]);
        }
      }
      if (g == 0) s_ds[qi * kChunk + jj] = dS;
#pragma unroll
      for (int r = 0; r < kPlanes; ++r) {
        if ((r * SEG + SHIFT) / DPL != g) continue;
        s_dth[(qi * kChunk + jj) * kPlanes + r] = dth[r];
        s_dthyz[(qi * kChunk + jj) * kPlanes + r] = dthyz[r];
      }
    }
    __syncthreads();

    // Per-workgroup partial sums of this chunk, in a fixed order.
    {
      const int d = threadIdx.x % HD;
      const int jg = threadIdx.x / HD;  // 0..3 -> offsets 2*jg, 2*jg+1 of the chunk
      float a0 = 0.f, a1 = 0.f;
      for (int t = 0; t < QPB; ++t) {
        const float qv = s_q[t * HD + d];
        a0 = fmaf(s_ds[t * kChunk + 2 * jg], qv, a0);
        a1 = fmaf(s_ds[t * kChunk + 2 * jg + 1], qv, a1);
      }
      const int ja = j0 + 2 * jg;
      float* dst = part_se + static_cast<int64_t>(work) * f.J * HD;
      if (ja < f.J) dst[ja * HD + d] = a0 * scale;
      if (ja + 1 < f.J) dst[(ja + 1) * HD + d] = a1 * scale;
    }
    if (threadIdx.x < kChunk) {
      const int jj = threadIdx.x;
      float sum = 0.f;
      for (int t = 0; t < QPB; ++t) sum += s_ds[t * kChunk + jj];
      if (j0 + jj < f.J) part_pb[static_cast<int64_t>(work) * f.J + j0 + jj] = sum;
    } else if (threadIdx.x >= 64 && threadIdx.x < 64 + kChunk * kPlanes * 2) {
      const int k = threadIdx.x - 64;
      const int kind = k / (kChunk * kPlanes);
      const int jr = k % (kChunk * kPlanes);
      const float* src = kind == 0 ? s_dth : s_dthyz;
      float sum = 0.f;
      for (int t = 0; t < QPB; ++t) sum += src[t * kChunk * kPlanes + jr];
      const int j = j0 + jr / kPlanes;
      const int r = jr % kPlanes;
      if (j >= f.J_small && j < f.J) {
        const int i = j - f.J_small;
        part_ph[((static_cast<int64_t>(work) * f.J_large + i) * kPlanes + r) * 2 + kind] = sum;
      }
    }
  }

  if (row_ok) {
    const int64_t nn = n;
    T* dqp = reinterpret_cast<T*>(a.dq) + b * a.dq_stride[0] + h * a.dq_stride[1] + nn * a.dq_stride[2] + g * DPL;
    store_from_f32<T, DPL>(dqp, dq);
    float dyo[4];
#pragma unroll
    for (int r = 0; r < kPlanes; ++r) dyo[r] = group_sum<L>(dy[r]);
    if (g == 0)
      *reinterpret_cast<float4*>(a.dy_pre + (static_cast<int64_t>(bh) * f.N + n) * kPlanes) =
          make_float4(dyo[0], dyo[1], dyo[2], dyo[3]);
  }
}

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

// Fixed-order sums of the dq kernel's per-workgroup partials.
__global__ __launch_bounds__(kBlock) void dsqg_bwd_reduce_kernel(const dwarf_dsqg_bwd_args a, const float* __restrict__ part_se,
                                                                const float* __restrict__ part_pb,
                                                                const float* __restrict__ part_ph, int tiles) {
  const dwarf_dsqg_fwd_args& f = a.fwd;
  const int HD = kHeadDim;
  const int n_se = f.J * HD;
  const int n_pb = f.J * f.H;
  const int n_ph = f.J_large * f.H * kPlanes;
  const int idx = blockIdx.x * kBlock + threadIdx.x;
  const int works = tiles * f.B * f.H;
  if (idx < n_se) {
    float sum = 0.f;
    for (int w = 0; w < works; ++w) sum += part_se[static_cast<int64_t>(w) * n_se + idx];
    a.dscale_embed[idx] = sum;
    return;
  }
  int k = idx - n_se;
  if (k < n_pb) {
    const int j = k / f.H, h = k - j * f.H;
    float sum = 0.f;
    for (int b = 0; b < f.B; ++b)
      for (int t = 0; t < tiles; ++t) sum += part_pb[static_cast<int64_t>((b * f.H + h) * tiles + t) * f.J + j];
    a.dpos_bias[k] = sum;
    return;
  }
  k -= n_pb;
  if (k < 2 * n_ph) {
    const int kind = k / n_ph;
    const int e = k - kind * n_ph;  // (i, h, r)
    const int i = e / (f.H * kPlanes);
    const int h = (e / kPlanes) % f.H;
    const int r = e % kPlanes;
    float sum = 0.f;
    for (int b = 0; b < f.B; ++b)
      for (int t = 0; t < tiles; ++t)
        sum += part_ph[((static_cast<int64_t>((b * f.H + h) * tiles + t) * f.J_large + i) * kPlanes + r) * 2 + kind];
    (kind == 0 ? a.dphase_base : a.dphase_gain)[e] = sum;
  }
}

template <typename T, int L, bool FAST>
hipError_t launch_bwd_typed(const dwarf_dsqg_bwd_args& a, const BwdWorkspace& ws, hipStream_t stream, bool do_dq,
                            bool do_dkdv) {
  const dwarf_dsqg_fwd_args& f = a.fwd;
  constexpr int QPB = kBlock / L;
  char* base = static_cast<char*>(a.workspace);
  float* delta = reinterpret_cast<float*>(base + ws.delta_off);
  float* part_se = reinterpret_cast<float*>(base + ws.part_se_off);
  float* part_pb = reinterpret_cast<float*>(base + ws.part_pb_off);
  float* part_ph = reinterpret_cast<float*>(base + ws.part_ph_off);

  const int tiles = (f.N + QPB - 1) / QPB;
  const int total_q = tiles * f.B * f.H;
  const size_t lds_q = (static_cast<size_t>(f.J) * (kHeadDim + 2) + QPB * kHeadDim + QPB * kChunk * (1 + 2 * kPlanes)) * sizeof(float);
  const int total_k = tiles * f.B * f.H_kv;
  const size_t lds_k = static_cast<size_t>(f.J) * (kHeadDim + 1) * sizeof(float);

#define DWARF_BWD_CASE(S)                                                                                           \
  case S:                                                                                                           \
    if (do_dq)                                                                                                      \
      hipLaunchKernelGGL((dsqg_bwd_dq_kernel<T, S, L, FAST>), dim3(total_q), dim3(kBlock), lds_q, stream, a, delta, \
                         part_se, part_pb, part_ph, tiles, total_q);                                                \
    if (do_dkdv)                                                                                                    \
      hipLaunchKernelGGL((dsqg_bwd_dkdv_kernel<T, S, L, FAST>), dim3(total_k), dim3(kBlock), lds_k, stream, a,     \
                         delta, tiles, total_k);                                                                    \
    break;
  switch (f.plane_shift) {
    DWARF_BWD_CASE(0) DWARF_BWD_CASE(1) DWARF_BWD_CASE(2) DWARF_BWD_CASE(3) DWARF_BWD_CASE(4)
    DWARF_BWD_CASE(5) DWARF_BWD_CASE(6) DWARF_BWD_CASE(7) DWARF_BWD_CASE(8) DWARF_BWD_CASE(9)
    DWARF_BWD_CASE(10) DWARF_BWD_CASE(11) DWARF_BWD_CASE(12) DWARF_BWD_CASE(13) DWARF_BWD_CASE(14)
    default:
      return hipErrorInvalidValue;
  }
#undef DWARF_BWD_CASE
  if (do_dq) {
    const int outputs = f.J * kHeadDim + f.J * f.H + 2 * f.J_large * f.H * kPlanes;
    hipLaunchKernelGGL(dsqg_bwd_reduce_kernel, dim3((outputs + kBlock - 1) / kBlock), dim3(kBlock), 0, stream, a,
                       part_se, part_pb, part_ph, tiles);
  }
  return hipGetLastError();
}

constexpr int kLanesBwd = 2;

}  // namespace

BwdWorkspace bwd_workspace_layout(const dwarf_dsqg_bwd_args& a) {
  const dwarf_dsqg_fwd_args& f = a.fwd;
  constexpr int QPB = kBlock / kLanesBwd;
  BwdWorkspace w{};
  const int tiles = (f.N + QPB - 1) / QPB;
  w.blocks_q = tiles * f.B * f.H;
  size_t off = 0;
  w.delta_off = off;
  w.delta_bytes = static_cast<size_t>(f.B) * f.H * f.N * sizeof(float);
  off += align256(w.delta_bytes);
  w.part_se_off = off;
  w.part_se_bytes = static_cast<size_t>(w.blocks_q) * f.J * kHeadDim * sizeof(float);
  off += align256(w.part_se_bytes);
  w.part_pb_off = off;
  w.part_pb_bytes = static_cast<size_t>(w.blocks_q) * f.J * sizeof(float);
  off += align256(w.part_pb_bytes);
  w.part_ph_off = off;
  w.part_ph_bytes = static_cast<size_t>(w.blocks_q) * (f.J_large > 0 ? f.J_large : 1) * kPlanes * 2 * sizeof(float);
  off += align256(w.part_ph_bytes);
  w.total = off;
  return w;
}

hipError_t launch_dsqg_bwd(const dwarf_dsqg_bwd_args& a, const BwdWorkspace& ws, hipStream_t stream, bool do_dq,
                           bool do_dkdv) {
  if (a.fwd.dtype == DWARF_BF16) return launch_bwd_typed<bf16, kLanesBwd, true>(a, ws, stream, do_dq, do_dkdv);
  return launch_bwd_typed<float, kLanesBwd, false>(a, ws, stream, do_dq, do_dkdv);
}

}  // namespace dwarf
