// DSQG backward, query-centric launch: delta, dQ, dY and the per-workgroup
// partials of dPB, dSE, dPhaseBase, dPhaseGain (reference kernels
// _compute_D_v18_grouped dsqg:1263-1289 and _bwd_dq_v18_grouped
// dsqg:1296-1488; the reference sums the parameter gradients with fp32
// atomics, here they are reduced in a fixed order).
//
// Mapping.  A workgroup of 4 waves walks `tpw` consecutive 128-query tiles of
// one (b, h).  Two lanes share a query (32 head dims each); wave w owns
// queries 32w..32w+31 of the tile.  Offsets are processed in chunks of 16.
//
// Per chunk, the dense sub-products run on MFMA:
//   QE   = Q E^T          the <q, e_j> term of every score       (wave level)
//   dQe += dS E            the e_j part of dQ                      (wave level)
//   dSE  = dS^T Q, dPB = dS^T 1                                    (workgroup level)
// and the lanes do the gathered work: <q, k_s>, <dO, v_s>, the MOVT rotation
// of the 8 rotated channels, P, dS and dQ += c dS k_s.  For bf16 inputs the
// MFMAs are v_mfma_f32_16x16x32_bf16 with dS split into bf16 high and low
// parts (~2^-17 relative); for fp32 inputs they are v_mfma_f32_16x16x4_f32.
// dPhase sums are formed every 4 offsets by a padded per-wave LDS transpose.
// Workgroup partials are accumulated in their own global slots (each entry
// owned by one wave, so the update order is fixed) and summed by
// dsqg_bwd_reduce.
#include "common.h"
#include "dsqg_internal.h"
#include "mfma.h"
#include "gather.h"

namespace dwarf {
namespace {

constexpr int kWaves = 4;
constexpr int kQ = 128;       // queries per tile
constexpr int kCJ = 16;       // offsets per chunk
constexpr int kDsRow = kQ + 4;    // s_ds[jj][q] row (floats), 16-byte aligned, bank-staggered
constexpr int kQeRow = 33;        // s_qe[jj][qi]
constexpr int kDs2Row = 20;       // s_ds2[qi][jj]
constexpr int kPhRow = 36;        // s_ph[jj4 * 8 + r * 2 + kind][qi]
constexpr int kStageRow = 68;     // dQe staging [qi][d]
constexpr int kQeOff = 0;
constexpr int kDs2Off = kCJ * kQeRow;                 // 528
constexpr int kPhOff = kDs2Off + 32 * kDs2Row;        // 1168
constexpr int kWaveRegion = kPhOff + 32 * kPhRow;     // 2320 floats (>= 32 * kStageRow = 2176)
constexpr int kERowBf16 = 72;     // bf16 E row stride (elements)
constexpr int kERowF32 = 68;      // fp32 E row stride (floats)

__host__ __device__ constexpr int align4(int x) { return (x + 3) & ~3; }

struct DqLds {
  int e_words;     // words of the E table (bf16 pairs or fp32)
  int et_words;    // words of the bf16 E^T table
  int jp;          // E^T row length (bf16 elements)
  size_t bytes;
};

template <typename T>
__host__ __device__ DqLds dq_lds(int J) {
  DqLds s;
  if constexpr (sizeof(T) == 2) {
    s.e_words = J * kERowBf16 / 2;
    s.jp = ((J + 7) / 8) * 8 + 8;
    s.et_words = kHeadDim * s.jp / 2;
  } else {
    s.e_words = J * kERowF32;
    s.jp = 0;
    s.et_words = 0;
  }
  const int words = align4(s.e_words) + align4(s.et_words) + align4(J) * 2 + 2 * kCJ * kDsRow + kWaves * kWaveRegion;
  s.bytes = static_cast<size_t>(words) * 4;
  return s;
}

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
}

template <typename T, int SHIFT>
__global__ __launch_bounds__(kBlock, 2) void dsqg_bwd_dq_v2(const dwarf_dsqg_bwd_args a, float* __restrict__ delta_ws,
                                                            float* __restrict__ part_se, float* __restrict__ part_pb,
                                                            float* __restrict__ part_ph, int tiles, int tpw, int n_tg,
                                                            int total) {
  constexpr bool BF = sizeof(T) == 2;
  constexpr int HD = kHeadDim, DPL = 32, SEG = HD / kPlanes;
  constexpr float kScale = 0.125f;
  const dwarf_dsqg_fwd_args& f = a.fwd;
  const int J = f.J;
  const DqLds lay = dq_lds<T>(J);

  extern __shared__ float smem[];
  uint32_t* sE = reinterpret_cast<uint32_t*>(smem);                        // E rows
  uint32_t* sET = sE + align4(lay.e_words);                                // bf16 E^T rows (bf16 path)
  float* s_pb = reinterpret_cast<float*>(sET + align4(lay.et_words));      // [J]
  int* s_off = reinterpret_cast<int*>(s_pb + align4(J));                   // [J]
  float* s_ds = reinterpret_cast<float*>(s_off + align4(J));               // [2][kCJ][kDsRow]
  float* s_wave = s_ds + 2 * kCJ * kDsRow;                                 // [kWaves][kWaveRegion]

  const int work = xcd_remap(blockIdx.x, total);
  const int bh = work / n_tg;
  const int tg = work - bh * n_tg;
  const int b = bh / f.H;
  const int h = bh - b * f.H;
  const int hk = h / (f.H / f.H_kv);
  const int slot = (h * f.B + b) * n_tg + tg;   // head-major partial slot

  // ---- stage the offset tables -------------------------------------------
  for (int i = threadIdx.x; i < J * HD; i += kBlock) {
    const int j = i / HD, d = i - j * HD;
    float e = f.scale_embed[j * f.se_stride[0] + d * f.se_stride[1]];
    if (f.se_round_bf16) e = round_bf16(e);
    if constexpr (BF) {
      uint16_t* e16 = reinterpret_cast<uint16_t*>(sE);
      e16[j * kERowBf16 + d] = f32_to_bf16_bits(e);
    } else {
      reinterpret_cast<float*>(sE)[j * kERowF32 + d] = e;
    }
  }
  if constexpr (BF) {
    uint16_t* et16 = reinterpret_cast<uint16_t*>(sET);
    for (int i = threadIdx.x; i < HD * lay.jp; i += kBlock) {
      const int d = i / lay.jp, j = i - d * lay.jp;
      float e = 0.f;
      if (j < J) {
        e = f.scale_embed[j * f.se_stride[0] + d * f.se_stride[1]];
        if (f.se_round_bf16) e = round_bf16(e);
      }
      et16[d * lay.jp + j] = f32_to_bf16_bits(e);
    }
  }
  for (int j = threadIdx.x; j < J; j += kBlock) {
    s_pb[j] = f.pos_bias[j * f.pb_stride[0] + h * f.pb_stride[1]];
    s_off[j] = f.offsets[j];
  }
  __syncthreads();

  const int lane = threadIdx.x;
  const int w = lane / kWave;
  const int l = lane % kWave;       // MFMA lane
  const int g = lane & 1;           // head-dim half
  const int qi = l >> 1;            // query within the wave
  const int qw = 32 * w + qi;       // query within the tile
  const int lr = l & 15, lc = l >> 4;
  float* wreg = s_wave + w * kWaveRegion;
  float* s_qe = wreg + kQeOff;
  float* s_ds2 = wreg + kDs2Off;
  float* s_ph = wreg + kPhOff;
  float* s_stage = wreg;

  const T* qb = reinterpret_cast<const T*>(f.q) + b * f.q_stride[0] + h * f.q_stride[1];
  const T* kb = reinterpret_cast<const T*>(f.k) + b * f.k_stride[0] + hk * f.k_stride[1] + g * DPL;
  const T* vb = reinterpret_cast<const T*>(f.v) + b * f.v_stride[0] + hk * f.v_stride[1] + g * DPL;
  const float* zb = f.z_pre + b * f.z_stride[0] + hk * f.z_stride[1];
  const float* pbase_h = f.phase_base + h * f.pbase_stride[1];
  const float* pgain_h = f.phase_gain + h * f.pgain_stride[1];

  const int t_begin = tg * tpw;
  const int t_end = min(tiles, t_begin + tpw);
  int chunk_count = 0;  // s_ds buffer parity alternates across tiles too (one barrier per chunk)
  for (int t = t_begin; t < t_end; ++t) {
    const bool first = t == t_begin;
    const int n0 = t * kQ;
    const int n = n0 + qw;
    const bool row_ok = n < f.N;
    const bool row_live = row_ok && n >= f.query_start;
    const int wave_n_last = n0 + 32 * w + 31;
    const int64_t nn = n;

    // ---- this lane's query slice, dO slice, delta, lse, y ------------------
    uint32_t qw16[BF ? 16 : 1], dw16[BF ? 16 : 1];
    float qf[BF ? 1 : DPL], df[BF ? 1 : DPL];
    float dlt = 0.f, lse = -INFINITY;
    float ys[4] = {0.f, 0.f, 0.f, 0.f};
    if constexpr (BF) {
#pragma unroll
      for (int i = 0; i < 16; ++i) { qw16[i] = 0u; dw16[i] = 0u; }
    } else {
#pragma unroll
      for (int i = 0; i < DPL; ++i) { qf[i] = 0.f; df[i] = 0.f; }
    }
    if (row_live) {
      const T* qp = qb + nn * f.q_stride[2] + g * DPL;
      const T* dp = reinterpret_cast<const T*>(a.dout) + b * a.dout_stride[0] + h * a.dout_stride[1] +
                    nn * a.dout_stride[2] + g * DPL;
      const T* op = reinterpret_cast<const T*>(f.out) + b * f.out_stride[0] + h * f.out_stride[1] +
                    nn * f.out_stride[2] + g * DPL;
      if constexpr (BF) {
        const uint4* q4 = reinterpret_cast<const uint4*>(qp);
        const uint4* d4 = reinterpret_cast<const uint4*>(dp);
        const uint4* o4 = reinterpret_cast<const uint4*>(op);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint4 x = q4[i], y = d4[i], o = o4[i];
          qw16[4 * i] = x.x; qw16[4 * i + 1] = x.y; qw16[4 * i + 2] = x.z; qw16[4 * i + 3] = x.w;
          dw16[4 * i] = y.x; dw16[4 * i + 1] = y.y; dw16[4 * i + 2] = y.z; dw16[4 * i + 3] = y.w;
          dlt = dot2_bf16(y.x, o.x, dlt); dlt = dot2_bf16(y.y, o.y, dlt);
          dlt = dot2_bf16(y.z, o.z, dlt); dlt = dot2_bf16(y.w, o.w, dlt);
        }
      } else {
        float o[DPL];
        load_f32<float, DPL>(reinterpret_cast<const float*>(qp), qf);
        load_f32<float, DPL>(reinterpret_cast<const float*>(dp), df);
        load_f32<float, DPL>(reinterpret_cast<const float*>(op), o);
#pragma unroll
        for (int i = 0; i < DPL; ++i) dlt = fmaf(df[i], o[i], dlt);
      }
      lse = f.lse[b * f.lse_stride[0] + h * f.lse_stride[1] + nn * f.lse_stride[2]];
      const float4 y4 = *reinterpret_cast<const float4*>(f.y_pre + b * f.y_stride[0] + h * f.y_stride[1] + nn * f.y_stride[2]);
      ys[0] = y4.x; ys[1] = y4.y; ys[2] = y4.z; ys[3] = y4.w;
    }
    dlt = group_sum<2>(dlt);
    if (row_ok && g == 0) delta_ws[static_cast<int64_t>(bh) * f.N + n] = dlt;
    const bool has_mass = row_live && lse > -INFINITY;

    // ---- MFMA operands for this tile ----------------------------------------
    // QE:  A[i = query 16mt + lr][k = dim]   (wave's own queries)
    // dSE: B[k = query of the tile][j = dim 16w + lr]
    bf16x8 aq[BF ? 2 : 1][BF ? 2 : 1];
    bf16x8 bq[BF ? 4 : 1];
    if constexpr (BF) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const int na = n0 + 32 * w + 16 * mt + lr;
        const bool ok = na < f.N && na >= f.query_start;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          uint4 x = {0u, 0u, 0u, 0u};
          if (ok) x = *reinterpret_cast<const uint4*>(qb + static_cast<int64_t>(na) * f.q_stride[2] + 32 * ks + 8 * lc);
          aq[mt][ks] = bf16x8_from_bits(x);
        }
      }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int nq = n0 + 32 * ks + 8 * lc + e;
          uint16_t bits = 0;
          if (nq < f.N && nq >= f.query_start)
            bits = reinterpret_cast<const uint16_t*>(qb + static_cast<int64_t>(nq) * f.q_stride[2])[16 * w + lr];
          bq[ks][e] = __builtin_bit_cast(__bf16, bits);
        }
      }
    }
    // fp32 inputs: the MFMA operands are re-read from global (L1) per chunk.
    auto qf32_at = [&](int nq, int d) -> float {
      return (nq < f.N && nq >= f.query_start)
                 ? reinterpret_cast<const float*>(qb + static_cast<int64_t>(nq) * f.q_stride[2])[d]
                 : 0.f;
    };

    float dq[DPL];
#pragma unroll
    for (int i = 0; i < DPL; ++i) dq[i] = 0.f;
    float dy[4] = {0.f, 0.f, 0.f, 0.f};
    f32x4 dqe[2][4];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) dqe[mt][nt] = zero4();

    for (int j0 = 0; j0 < J; j0 += kCJ) {
      float* sdsb = s_ds + (chunk_count++ & 1) * kCJ * kDsRow;
      const int jrow = j0 + lr;  // this MFMA lane's offset row

      // ---- (a) QE for the wave's 32 queries x 16 offsets ---------------------
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        f32x4 c = zero4();
        if constexpr (BF) {
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            uint4 x = {0u, 0u, 0u, 0u};
            if (jrow < J)
              x = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(sE) + jrow * kERowBf16 + 32 * ks + 8 * lc);
            c = mfma16_bf16(aq[mt][ks], bf16x8_from_bits(x), c);
          }
        } else {
          const float* er = reinterpret_cast<const float*>(sE) + jrow * kERowF32;
          const int na = n0 + 32 * w + 16 * mt + lr;
#pragma unroll
          for (int st = 0; st < 16; ++st)
            c = mfma16_f32(qf32_at(na, 4 * st + lc), jrow < J ? er[4 * st + lc] : 0.f, c);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) s_qe[lr * kQeRow + 16 * mt + 4 * lc + r] = c[r];
      }
      __builtin_amdgcn_wave_barrier();

      // ---- (b) gathered pair work --------------------------------------------
      for (int jj = 0; jj < kCJ; ++jj) {
        const int j = j0 + jj;
        float dS = 0.f;
        float dth[4] = {0.f, 0.f, 0.f, 0.f}, dthyz[4] = {0.f, 0.f, 0.f, 0.f};
        if (j < J) {
          const int delta = s_off[j];
          const int s = n - delta;
          if (wave_n_last >= delta && has_mass && s >= 0 && s < f.N) {
            const int64_t ss = s;
            float dot = 0.f, gd = 0.f;
            uint32_t kw[BF ? 16 : 1], vw[BF ? 16 : 1];
            float kf[BF ? 1 : DPL], vf[BF ? 1 : DPL];
            if constexpr (BF) {
              const uint4* k4 = reinterpret_cast<const uint4*>(kb + ss * f.k_stride[2]);
              const uint4* v4 = reinterpret_cast<const uint4*>(vb + ss * f.v_stride[2]);
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                const uint4 x = k4[i], y = v4[i];
                kw[4 * i] = x.x; kw[4 * i + 1] = x.y; kw[4 * i + 2] = x.z; kw[4 * i + 3] = x.w;
                vw[4 * i] = y.x; vw[4 * i + 1] = y.y; vw[4 * i + 2] = y.z; vw[4 * i + 3] = y.w;
              }
#pragma unroll
              for (int i = 0; i < 16; ++i) {
                dot = dot2_bf16(qw16[i], kw[i], dot);
                gd = dot2_bf16(dw16[i], vw[i], gd);
              }
            } else {
              load_f32<float, DPL>(reinterpret_cast<const float*>(kb + ss * f.k_stride[2]), kf);
              load_f32<float, DPL>(reinterpret_cast<const float*>(vb + ss * f.v_stride[2]), vf);
#pragma unroll
              for (int i = 0; i < DPL; ++i) {
                dot = fmaf(qf[i], kf[i], dot);
                gd = fmaf(df[i], vf[i], gd);
              }
            }
            dot = group_sum<2>(dot) + s_qe[jj * kQeRow + qi];
            const float P = dexp<BF>(fmaf(dot, kScale, s_pb[j]) - lse);
            if (j >= f.J_small) {
              const int i = j - f.J_small;
              const float4 zk = *reinterpret_cast<const float4*>(zb + ss * f.z_stride[2]);
              const float zs[4] = {zk.x, zk.y, zk.z, zk.w};
#pragma unroll
              for (int r = 0; r < kPlanes; ++r) {
                const int ch = r * SEG + SHIFT;
                if (ch / DPL != g) continue;
                const int la = ch % DPL;
                float va, vb2, da, db;
                if constexpr (BF) {
                  va = (la & 1) ? bf16_hi(vw[la >> 1]) : bf16_lo(vw[la >> 1]);
                  vb2 = ((la + 1) & 1) ? bf16_hi(vw[(la + 1) >> 1]) : bf16_lo(vw[(la + 1) >> 1]);
                  da = (la & 1) ? bf16_hi(dw16[la >> 1]) : bf16_lo(dw16[la >> 1]);
                  db = ((la + 1) & 1) ? bf16_hi(dw16[(la + 1) >> 1]) : bf16_lo(dw16[(la + 1) >> 1]);
                } else {
                  va = vf[la]; vb2 = vf[la + 1]; da = df[la]; db = df[la + 1];
                }
                const float pg = pgain_h[i * f.pgain_stride[0] + r];
                const float theta = pbase_h[i * f.pbase_stride[0] + r] + pg * ys[r] * zs[r];
                float sn, cs;
                dsincos<BF>(theta, &sn, &cs);
                gd += da * (cs * va - sn * vb2 - va) + db * (sn * va + cs * vb2 - vb2);
                const float tq = P * (da * (-va * sn - vb2 * cs) + db * (va * cs - vb2 * sn));
                dth[r] = tq;
                dthyz[r] = tq * ys[r] * zs[r];
                dy[r] = fmaf(tq * pg, zs[r], dy[r]);
              }
            }
            gd = group_sum<2>(gd);
            dS = P * (gd - dlt);
            const float cds = kScale * dS;
            if constexpr (BF) {
#pragma unroll
              for (int i = 0; i < 16; ++i) {
                dq[2 * i] = fmaf(cds, bf16_lo(kw[i]), dq[2 * i]);
                dq[2 * i + 1] = fmaf(cds, bf16_hi(kw[i]), dq[2 * i + 1]);
              }
            } else {
#pragma unroll
              for (int i = 0; i < DPL; ++i) dq[i] = fmaf(cds, kf[i], dq[i]);
            }
          }
        }
        if (g == 0) {
          sdsb[jj * kDsRow + qw] = dS;
          s_ds2[qi * kDs2Row + jj] = dS;
        }
#pragma unroll
        for (int r = 0; r < kPlanes; ++r) {
          if ((r * SEG + SHIFT) / DPL != g) continue;
          s_ph[((jj & 3) * 8 + r * 2 + 0) * kPhRow + qi] = dth[r];
          s_ph[((jj & 3) * 8 + r * 2 + 1) * kPhRow + qi] = dthyz[r];
        }
        if ((jj & 3) == 3) {
          // dPhase sums of these 4 offsets over the wave's 32 queries.
          __builtin_amdgcn_wave_barrier();
          const int row = l >> 1;           // (jj4, r, kind)
          const int half = l & 1;
          const float* src = s_ph + row * kPhRow + 16 * half;
          float sum = 0.f;
#pragma unroll
          for (int x = 0; x < 16; ++x) sum += src[x];
          sum = group_sum<2>(sum);
          const int jq = j0 + (jj & ~3) + (row >> 3);
          if (half == 0 && jq >= f.J_small && jq < J) {
            const int i = jq - f.J_small;
            const int rk = row & 7;
            float* dst = part_ph + ((static_cast<int64_t>(slot) * kWaves + w) * f.J_large + i) * 8 + rk;
            *dst = first ? sum : *dst + sum;
          }
          __builtin_amdgcn_wave_barrier();
        }
      }
      __builtin_amdgcn_wave_barrier();

      // ---- (c) dQe += dS E over this chunk (wave's queries) -----------------
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        if constexpr (BF) {
          bf16x8 ahi = bf16x8_zero(), alo = bf16x8_zero();
          if (lc < 2) {
            float x[8];
            const float* src = s_ds2 + (16 * mt + lr) * kDs2Row + 8 * lc;
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = src[e];
            split_bf16x8(x, ahi, alo);
          }
#pragma unroll
          for (int nt = 0; nt < 4; ++nt) {
            uint4 xb = {0u, 0u, 0u, 0u};
            if (lc < 2)
              xb = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(sET) + (16 * nt + lr) * lay.jp + j0 + 8 * lc);
            const bf16x8 bb = bf16x8_from_bits(xb);
            dqe[mt][nt] = mfma16_bf16(ahi, bb, dqe[mt][nt]);
            dqe[mt][nt] = mfma16_bf16(alo, bb, dqe[mt][nt]);
          }
        } else {
#pragma unroll
          for (int st = 0; st < 4; ++st) {
            const float av = s_ds2[(16 * mt + lr) * kDs2Row + 4 * st + lc];
            const int je = j0 + 4 * st + lc;
            const float* er = reinterpret_cast<const float*>(sE) + je * kERowF32;
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) dqe[mt][nt] = mfma16_f32(av, je < J ? er[16 * nt + lr] : 0.f, dqe[mt][nt]);
          }
        }
      }

      __syncthreads();  // the tile's dS for this chunk is complete in sdsb

      // ---- (e) dSE (dims 16w..16w+15) and dPB (wave 0) over the 128 queries ----
      {
        f32x4 c = zero4(), c1 = zero4();
        if constexpr (BF) {
          bf16x8 one;
#pragma unroll
          for (int e = 0; e < 8; ++e) one[e] = static_cast<__bf16>(lr == 0 ? 1.f : 0.f);
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) {
            float x[8];
            const float* src = sdsb + lr * kDsRow + 32 * ks + 8 * lc;
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = src[e];
            bf16x8 ahi, alo;
            split_bf16x8(x, ahi, alo);
            c = mfma16_bf16(ahi, bq[ks], c);
            c = mfma16_bf16(alo, bq[ks], c);
            if (w == 0) {
              c1 = mfma16_bf16(ahi, one, c1);
              c1 = mfma16_bf16(alo, one, c1);
            }
          }
        } else {
#pragma unroll
          for (int st = 0; st < 32; ++st) {
            const float av = sdsb[lr * kDsRow + 4 * st + lc];
            c = mfma16_f32(av, qf32_at(n0 + 4 * st + lc, 16 * w + lr), c);
            if (w == 0) c1 = mfma16_f32(av, lr == 0 ? 1.f : 0.f, c1);
          }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = j0 + 4 * lc + r;
          if (j < J) {
            float* dst = part_se + (static_cast<int64_t>(slot) * J + j) * HD + 16 * w + lr;
            const float v = kScale * c[r];
            *dst = first ? v : *dst + v;
            if (w == 0 && lr == 0) {
              float* dp = part_pb + static_cast<int64_t>(slot) * J + j;
              *dp = first ? c1[r] : *dp + c1[r];
            }
          }
        }
      }
    }

    // ---- end of tile: dQ += c dQe, store dQ and dY ---------------------------
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int r = 0; r < 4; ++r) s_stage[(16 * mt + 4 * lc + r) * kStageRow + 16 * nt + lr] = dqe[mt][nt][r];
    __builtin_amdgcn_wave_barrier();
    {
      const float* src = s_stage + qi * kStageRow + g * DPL;
#pragma unroll
      for (int i = 0; i < DPL; ++i) dq[i] = fmaf(kScale, src[i], dq[i]);
    }
    __builtin_amdgcn_wave_barrier();
    if (row_ok) {
      T* dqp = reinterpret_cast<T*>(a.dq) + b * a.dq_stride[0] + h * a.dq_stride[1] + nn * a.dq_stride[2] + g * DPL;
      store_from_f32<T, DPL>(dqp, dq);
    }
    float dyo[4];
#pragma unroll
    for (int r = 0; r < kPlanes; ++r) dyo[r] = group_sum<2>(dy[r]);
    if (row_ok && g == 0)
      *reinterpret_cast<float4*>(a.dy_pre + (static_cast<int64_t>(bh) * f.N + n) * kPlanes) =
          make_float4(dyo[0], dyo[1], dyo[2], dyo[3]);
  }
}

// ---------------------------------------------------------------------------
// bf16 dQ launch, four lanes per query (the forward's mapping).
//
// dsqg_bwd_dq_bf16_g4: a persistent workgroup of 4 waves walks a sequence of
// 64-query tiles (the order is described at the tile loop); wave w owns
// queries 16w..16w+15 of a tile and lane g of a query holds head dims
// [16g, 16g+16).  Each wave walks its offset list (offsets that give one of
// its queries a source row) in chunks of CJ with the next chunk's K/V/z loads
// in flight; a lane without a source reads zeros (out-of-range buffer offset)
// and gets P = 0.  Per pair the lanes form <q, k_s> + <q, e_j> and <dO, v_s>
// with v_dot2_f32_bf16, the MOVT rotation of their one channel pair, P,
// dS = P (g - delta) and dQ += c dS k_s.  dS goes to the workspace matrix
// dS[b, h][j][n] (16 consecutive queries: one 64-byte store), and every four
// offsets one v_mfma_f32_16x16x4_f32 per 16 head dims adds their
// dS (16 queries x 4 offsets) times E (4 rows x 16 dims) into the wave's dQe
// accumulator, which joins dQ through a wave-local LDS transpose at the end of
// the tile.  dPhase sums over the wave's 16 queries are reduced per offset
// (DPP + permlane swaps) into a per-wave LDS table whose four waves are added
// in a fixed order into the tile's row.
//
// dsqg_bwd_dse_bf16: dSE = dS^T Q and dPB = dS^T 1 from the dS matrix, on
// v_mfma_f32_16x16x32_bf16 with dS split into bf16 high and low parts (~2^-17
// relative); a persistent workgroup accumulates dSE over its tiles in its own
// slot (wave w: dims 16w..16w+15), dPB goes to the tile's row.  Entries of the
// dS matrix that no wave wrote (offsets with no source for any query of a
// wave) are exactly those with n < offset_j and are masked.  Every sum has a
// fixed order.
// ---------------------------------------------------------------------------
constexpr int kQT = 64;           // queries per tile
constexpr int kQPW = 16;          // queries per wave
constexpr int kStepDq = 4;        // offsets per loop step (one dQe MFMA step); one in flight ahead
constexpr int kERowT = 72;        // bf16 E row stride (elements)
constexpr int kStRow = 36;        // dQe staging row (half a head row + padding), floats
constexpr int kGatherWgsPerCu = 3;
// dSE launch: 16-row dS blocks per wave (JE / 16 dealt to 4 waves) and the
// resident workgroups per CU its registers allow
__host__ __device__ constexpr int dse_blocks_per_wave(int J) { return (J + 1 + 15) / 16 <= 8 ? 2 : 5; }
__host__ __device__ constexpr int dse_wgs_per_cu(int mbw) { return mbw <= 2 ? 4 : 2; }

// Near band: the leading small offsets j < JB (ascending, unique, at most
// kBandMax) are served from a K window [n0 - kBandMax, n0 + 64) in LDS on the
// matrix cores (dsqg_bwd_dq_bf16_g4); the gather loop takes the others.
constexpr int kBandMax = 32;                    // largest band offset; the window's look-back
constexpr int kWinRows = kQT + kBandMax;        // 96 K rows of 128 bytes
constexpr int kBandSlots = 32;                  // band scratch columns per query
constexpr int kBandDummy = kQPW * kBandSlots;   // a scratch word that takes the band's masked-off stores

struct DqG4Layout {
  int JE, JL4, list_len, dphw;
  size_t off_ph, off_list, off_dph, off_e, off_jn, off_st, bytes;
};

// JE >= J + 1 keeps a sentinel row J of zeros in the E table.  A wave's dPhase
// table doubles as its band scratch [16][32] fp32 (and the word after it, which
// takes the band's masked-off stores) at the start of a tile (it is cleared
// after the band); the last region holds the K window [96][128 B]
// at the start of a tile and the dQe staging [4][16][36] fp32 at its end.
__host__ __device__ inline DqG4Layout dq_g4_layout(int J, int J_large) {
  DqG4Layout L;
  L.JE = (J + 1 + 15) / 16 * 16;
  L.JL4 = (J_large + 1) / 2 * 2;
  L.list_len = (L.JE + 2 * kStepDq + 1) / 2 * 2;   // list + padding for the last step and its prefetch
  L.dphw = L.JL4 * 8 > kBandDummy + 4 ? L.JL4 * 8 : kBandDummy + 4;
  L.off_ph = static_cast<size_t>(2 * L.JE) * 4;                       // s_pb2[JE], s_off[JE]
  L.off_list = L.off_ph + static_cast<size_t>(L.JL4) * 4 * 8;         // s_ph[JL4][4] float2
  L.off_dph = L.off_list + static_cast<size_t>(4 * L.list_len) * 8;   // s_list[4][list_len] int2
  L.off_e = L.off_dph + static_cast<size_t>(4 * L.dphw) * 4;          // s_dph[4][dphw]
  L.off_jn = L.off_e + static_cast<size_t>(L.JE) * kERowT * 2;        // sE[JE][72] bf16
  L.off_st = L.off_jn + kJnSize * 4;                                   // s_jn[kJnSize] int
  const size_t st = static_cast<size_t>(4 * kQPW * kStRow) * 4;
  const size_t win = static_cast<size_t>(kWinRows) * 128;
  L.bytes = L.off_st + (st > win ? st : win);
  return L;
}

template <int SHIFT, int CJ>
struct DqChunk {
  uint4 k[CJ][2], v[CJ][2];
  float z[CJ], pb2[CJ];
  bool ok[CJ];
  int j[CJ];
};

// Tile order of the persistent dQ launches.  Workgroups are dealt round-robin
// over the 8 XCDs; XCD x owns a contiguous range of the (b, h)-major tiles and
// its U workgroups take them in steps of U consecutive tiles (a few (b, h) at
// a time, so the K/V rows they gather stay in that XCD's L2).  Within a step
// the tiles are rotated by 7 per step, so each workgroup sees early (few
// valid offsets) and late positions of the sequence alike.
struct TileOrder {
  int Ux, u, T0, T1;
  __device__ TileOrder(int64_t total_tiles) {
    const int W = gridDim.x;
    const int x = blockIdx.x % kXcds;
    u = blockIdx.x / kXcds;
    Ux = (W - x + kXcds - 1) / kXcds;
    int cum_x = 0;
    for (int y = 0; y < x; ++y) cum_x += (W - y + kXcds - 1) / kXcds;
    T0 = static_cast<int>(total_tiles * cum_x / W);
    T1 = static_cast<int>(total_tiles * (cum_x + Ux) / W);
  }
  __device__ int steps() const { return (T1 - T0 + Ux - 1) / Ux; }
  __device__ int tile(int kstep) const {   // -1: none this step
    const int Lt = kstep * Ux + (u + 7 * kstep) % Ux;
    return Lt < T1 - T0 ? T0 + Lt : -1;
  }
};

template <int SHIFT>
__global__ __launch_bounds__(kBlock, kGatherWgsPerCu) void dsqg_bwd_dq_bf16_g4(
    const dwarf_dsqg_bwd_args a, float* __restrict__ delta_ws, float* __restrict__ ds_ws, float* __restrict__ part_ph,
    int tiles) {
  constexpr float kC = 0.125f * kLog2e;
  constexpr float kScale = 0.125f;
  static_assert(SHIFT + 1 < kHeadDim / kPlanes, "MOVT pair must stay inside one lane's slice");
  constexpr int CJ = 1;   // offsets per prefetch chunk
  const dwarf_dsqg_fwd_args& f = a.fwd;
  const int J = f.J, N = f.N, J_small = f.J_small, JL = f.J_large;
  const DqG4Layout lay = dq_g4_layout(J, JL);
  extern __shared__ float smem[];
  char* sm = reinterpret_cast<char*>(smem);
  float* s_pb2 = smem;                                        // log2(e) * pb_j of the tile's head
  int* s_off = reinterpret_cast<int*>(smem + lay.JE);
  float2* s_ph = reinterpret_cast<float2*>(sm + lay.off_ph);
  int2* s_list_all = reinterpret_cast<int2*>(sm + lay.off_list);
  float* s_dph_all = reinterpret_cast<float*>(sm + lay.off_dph);
  uint16_t* sE = reinterpret_cast<uint16_t*>(sm + lay.off_e);
  float* s_st_all = reinterpret_cast<float*>(sm + lay.off_st);
  int* s_jn = reinterpret_cast<int*>(sm + lay.off_jn);       // [0]: JB; [kJnBias + d]: band slot of delta d, or -1
  char* s_win = sm + lay.off_st;                              // K window [96][128 B] (aliases the dQe staging)

  stage_tables<true, false, true, false, true>(
      f, lay.JE, 0, 1, TableStage{sE, kERowT, nullptr, 0.f, s_off, nullptr, 0, s_jn, kBandMax, kBandSlots,
                                  (f.schedule & DWARF_SCHED_BAND) != 0});
  __syncthreads();   // s_jn is read in every tile's prologue

  const int lane = threadIdx.x;
  const int w = lane / kWave;
  const int l = lane % kWave;
  const int g = l & 3;
  const int qi = l >> 2;
  const int lr = l & 15, lc = l >> 4;
  int2* s_list = s_list_all + w * lay.list_len;
  float* s_dph = s_dph_all + w * lay.dphw;
  float* s_st = s_st_all + w * kQPW * kStRow;
  const int ks_b = static_cast<int>(f.k_stride[2]) * 2, vs_b = static_cast<int>(f.v_stride[2]) * 2;
  const int zs_b = static_cast<int>(f.z_stride[2]) * 4;

  const TileOrder order(static_cast<int64_t>(tiles) * f.B * f.H);
  int cur_h = -1;
  for (int kstep = 0; kstep < order.steps(); ++kstep) {
    const int T = order.tile(kstep);
    if (T < 0) continue;   // uniform over the workgroup
    const int bh = T / tiles;
    const int t = T - bh * tiles;
    const int b = bh / f.H;
    const int h = bh - b * f.H;
    const int hk = h / (f.H / f.H_kv);
    const int64_t prow = static_cast<int64_t>(h * f.B + b) * tiles + t;   // head-major partial row
    const bf16* qb = reinterpret_cast<const bf16*>(f.q) + b * f.q_stride[0] + h * f.q_stride[1];
    const bf16* dob = reinterpret_cast<const bf16*>(a.dout) + b * a.dout_stride[0] + h * a.dout_stride[1];
    const bf16* ob = reinterpret_cast<const bf16*>(f.out) + b * f.out_stride[0] + h * f.out_stride[1];
    const __amdgpu_buffer_rsrc_t rk =
        rows_rsrc(reinterpret_cast<const bf16*>(f.k) + b * f.k_stride[0] + hk * f.k_stride[1], ks_b, N, 128);
    const __amdgpu_buffer_rsrc_t rv =
        rows_rsrc(reinterpret_cast<const bf16*>(f.v) + b * f.v_stride[0] + hk * f.v_stride[1], vs_b, N, 128);
    const __amdgpu_buffer_rsrc_t rz = rows_rsrc(f.z_pre + b * f.z_stride[0] + hk * f.z_stride[1], zs_b, N, 16);
    // the (b, h) slab of the dS matrix, J rows of N fp32; this lane's query column
    const __amdgpu_buffer_rsrc_t rds = rows_rsrc(ds_ws + static_cast<int64_t>(bh) * J * N, 4 * N, J, 4 * N);

    const int n0w = t * kQT + kQPW * w;
    const int n = n0w + qi;
    const int n_hi = min(n0w + kQPW - 1, N - 1);
    const bool row_ok = n < N;
    const bool live = row_ok && n >= f.query_start;
    const int64_t nn = n;

    // ---- this lane's slices of q and dO, delta = <dO, O> (bf16 O), lse, y ----
    uint32_t q32[8], d32[8];
    float dlt = 0.f, lse2 = 0.f, yg = 0.f;
    bool mass = false;
#pragma unroll
    for (int i = 0; i < 8; ++i) { q32[i] = 0u; d32[i] = 0u; }
    if (live) {
      const uint4* q4 = reinterpret_cast<const uint4*>(qb + nn * f.q_stride[2] + 16 * g);
      const uint4* d4 = reinterpret_cast<const uint4*>(dob + nn * a.dout_stride[2] + 16 * g);
      const uint4* o4 = reinterpret_cast<const uint4*>(ob + nn * f.out_stride[2] + 16 * g);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const uint4 x = q4[i], y = d4[i], o = o4[i];
        q32[4 * i] = x.x; q32[4 * i + 1] = x.y; q32[4 * i + 2] = x.z; q32[4 * i + 3] = x.w;
        d32[4 * i] = y.x; d32[4 * i + 1] = y.y; d32[4 * i + 2] = y.z; d32[4 * i + 3] = y.w;
        dlt = dot2bf(y.x, o.x, dlt); dlt = dot2bf(y.y, o.y, dlt);
        dlt = dot2bf(y.z, o.z, dlt); dlt = dot2bf(y.w, o.w, dlt);
      }
      const float lse = f.lse[b * f.lse_stride[0] + h * f.lse_stride[1] + nn * f.lse_stride[2]];
      mass = lse > -INFINITY;
      lse2 = mass ? lse * kLog2e : 0.f;
      yg = f.y_pre[b * f.y_stride[0] + h * f.y_stride[1] + nn * f.y_stride[2] + g];
    }
    dlt = group_sum<4>(dlt);
    // (delta, lse in log2 units) for the dK/dV launch; +inf makes P = 0 for a
    // query without softmax mass or before query_start
    // (under DWARF_SCHED_DELTA_STAGE dsqg_bwd_delta_bf16 writes them, the same bits)
    if (row_ok && g == 0 && !(f.schedule & DWARF_SCHED_DELTA_STAGE))
      *reinterpret_cast<float2*>(delta_ws + 2 * (static_cast<int64_t>(bh) * N + n)) =
          make_float2(dlt, mass ? lse2 : INFINITY);
    // the wave's q rows as the B operand of the per-step <q, e_j> MFMA: lane
    // (lr, lc) holds dims 32 ks + 8 lc + [0, 8) of query n0w + lr
    uint4 xq[2] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
    if (n0w + lr < N) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        xq[ks] = *reinterpret_cast<const uint4*>(qb + static_cast<int64_t>(n0w + lr) * f.q_stride[2] + 32 * ks + 8 * lc);
    }
    const int n_eff = mass ? n : n0w - 2 * N;   // no source for queries without softmax mass
    const int kb_lane = n_eff * ks_b + 32 * g;
    const int vb_lane = n_eff * vs_b + 32 * g;
    const int zb_lane = n_eff * zs_b + 4 * g;
    const uint32_t ds_lane = row_ok ? static_cast<uint32_t>(4 * n) : kOutOfRange;

    __syncthreads();   // the previous tile's dPhase tables and dQe staging have been read
    const int JB = s_jn[0];
    if (JB > 0) {
      // K rows [n0 - kBandMax, n0 + 64) into the window: three 1 KB DMA loads per wave; LDS chunk
      // (i & 7) of row i >> 3 holds the row's 16-byte chunk (i & 7) ^ (row & 7) (bank spread)
      typedef __attribute__((address_space(3))) void lds_void;
#pragma unroll
      for (int u = 0; u < 3; ++u) {
        const int i = kBlock * u + lane;
        const int row = i >> 3, c = (i & 7) ^ (row & 7);
        const int key = t * kQT - kBandMax + row;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void*)(void*)(s_win + 4096 * u + 1024 * w), 16,
                                                 static_cast<uint32_t>(key * ks_b + 16 * c), 0, 0, 0);
      }
    }
    if (h != cur_h) {
      cur_h = h;
      for (int j = lane; j < lay.JE; j += kBlock)
        s_pb2[j] = j < J ? kLog2e * f.pos_bias[j * f.pb_stride[0] + h * f.pb_stride[1]] : 0.f;
      for (int i = lane; i < JL * kPlanes; i += kBlock) {
        const int ii = i / kPlanes, r = i - ii * kPlanes;
        s_ph[i] = make_float2(f.phase_base[ii * f.pbase_stride[0] + h * f.pbase_stride[1] + r],
                              f.phase_gain[ii * f.pgain_stride[0] + h * f.pgain_stride[1] + r]);
      }
    }
    int cnt = 0;
    // padded with the sentinel to a multiple of 4 plus 4: every step's reads and the next prefetch
    if (n0w < N)
      cnt = build_offset_list<kStepDq / 2>(s_list, s_off, J, n0w, n_hi, N, 1, make_int2(J, n0w - N), JB);
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): this wave's window loads have landed
    __syncthreads();   // tables and the K window staged

    // ---- near band (offsets j < JB) on the matrix cores ----
    // Band lane (lc, lr) serves query n0w + lr; in the MFMA C layout it holds
    // keys 16 t + 4 lc + r of the wave's key blocks t = 0..2 (keys
    // [n0w - 32, n0w + 16)), and its dQ result dims 16 lc + [0, 16).
    //   S^T  = K_win Q^T, dP^T = V dO^T     (v_mfma_f32_16x16x32_bf16)
    //   P = exp2(S' - lse), dS = P (dP - delta) on the band's diagonals
    //   dQ^T += K_win^T dS^T + E^T dS^T     (v_mfma_f32_16x16x16_bf16, dS as bf16 hi + lo)
    float* scr = s_dph;   // this wave's band scratch [16 queries][32 slots] (cleared below)
    float bandq[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) bandq[i] = 0.f;
    if (JB > 0 && n0w < N) {
      const int src4 = 4 * (4 * lr);                     // gather-layout lane of query n0w + lr
      const float dl_b = __int_as_float(__builtin_amdgcn_ds_bpermute(src4, __float_as_int(dlt)));
      const float ls_b = __int_as_float(
          __builtin_amdgcn_ds_bpermute(src4, __float_as_int(row_ok && mass ? lse2 : INFINITY)));
      uint4 xd[2] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
      if (n0w + lr < N) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
          xd[ks] = *reinterpret_cast<const uint4*>(dob + static_cast<int64_t>(n0w + lr) * a.dout_stride[2] + 32 * ks +
                                                   8 * lc);
      }
      auto win16 = [&](int row, int c) { return s_win + row * 128 + 16 * (c ^ (row & 7)); };
      // band slot of the pair (query n0w + lr, key n0w - 32 + 16 tb + 4 lc + r), or -1;
      // the delta lies in [-15, 47], inside the table
      auto band_slot = [&](int tb, int r) {
        const int slot = s_jn[kJnBias + lr + kBandMax - 16 * tb - 4 * lc - r];
        return n0w - kBandMax + 16 * tb + 4 * lc + r >= 0 ? slot : -1;
      };
      // <q, e_slot> of the band slots, into the scratch as [query][slot]
#pragma unroll
      for (int bb = 0; bb < 2; ++bb) {
        if (16 * bb < JB) {
          f32x4 qe = zero4();
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            const uint4 ea = *reinterpret_cast<const uint4*>(sE + (16 * bb + lr) * kERowT + 32 * ks + 8 * lc);
            qe = mfma16_bf16(bf16x8_from_bits(ea), bf16x8_from_bits(xq[ks]), qe);
          }
          *reinterpret_cast<f32x4*>(scr + lr * kBandSlots + 16 * bb + 4 * lc) = qe;
        }
      }
      float dsv[3][4];
#pragma unroll
      for (int tb = 0; tb < 3; ++tb) {
        const int wr = 16 * (w + tb) + lr;               // window row of key n0w - 32 + 16 tb + lr
        const uint4 ka0 = *reinterpret_cast<const uint4*>(win16(wr, lc));
        const uint4 ka1 = *reinterpret_cast<const uint4*>(win16(wr, 4 + lc));
        f32x4 S = mfma16_bf16(bf16x8_from_bits(ka0), bf16x8_from_bits(xq[0]), zero4());
        S = mfma16_bf16(bf16x8_from_bits(ka1), bf16x8_from_bits(xq[1]), S);
        const int key = n0w - kBandMax + 16 * tb + lr;   // before 0: out of range, zeros
        const uint32_t vo = static_cast<uint32_t>(key * vs_b + 16 * lc);
        const uint4 va0 = buf_load16(rv, vo), va1 = buf_load16(rv, vo + 64);
        f32x4 Dp = mfma16_bf16(bf16x8_from_bits(va0), bf16x8_from_bits(xd[0]), zero4());
        Dp = mfma16_bf16(bf16x8_from_bits(va1), bf16x8_from_bits(xd[1]), Dp);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          // computed for every lane (slot 0 stands in off the band) and masked, with no branch
          const int slot = band_slot(tb, r);
          const int sl = slot >= 0 ? slot : 0;
          const float p = __builtin_amdgcn_exp2f(fmaf(S[r] + scr[lr * kBandSlots + sl], kC, s_pb2[sl]) - ls_b);
          dsv[tb][r] = slot >= 0 ? p * (Dp[r] - dl_b) : 0.f;
        }
      }
      // dS of the band into the scratch as [query][slot] (zeros where no pair)
      __builtin_amdgcn_wave_barrier();
      *reinterpret_cast<f32x4*>(scr + lr * kBandSlots + 8 * lc) = zero4();
      *reinterpret_cast<f32x4*>(scr + lr * kBandSlots + 8 * lc + 4) = zero4();
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int tb = 0; tb < 3; ++tb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int slot = band_slot(tb, r);
          scr[slot >= 0 ? lr * kBandSlots + slot : kBandDummy] = dsv[tb][r];
        }
      __builtin_amdgcn_wave_barrier();
      f32x4 acch[4];
#pragma unroll
      for (int db = 0; db < 4; ++db) acch[db] = zero4();
      // dQ^T += K^T (c dS^T): K^T read transposed from the window (rows 16 (w + tb) + 4 lc + e, dims
      // 16 (lr / 4) + 4 db + lr % 4 of MFMA row lr), c dS^T from the C layout of S^T as bf16 hi + lo
#pragma unroll
      for (int tb = 0; tb < 3; ++tb) {
        float cd[4], cl[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          cd[r] = kScale * dsv[tb][r];
          cl[r] = cd[r] - round_bf16(cd[r]);
        }
        const i16x4 bh = __builtin_bit_cast(i16x4, make_uint2(pack_bf16x2(cd[0], cd[1]), pack_bf16x2(cd[2], cd[3])));
        const i16x4 bl = __builtin_bit_cast(i16x4, make_uint2(pack_bf16x2(cl[0], cl[1]), pack_bf16x2(cl[2], cl[3])));
        const int R = 16 * (w + tb) + 4 * lc + (lr >> 2);
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          const i16x4 ak = lds_read_tr16(win16(R, 2 * (lr & 3) + (db >> 1)) + 8 * (db & 1));
          acch[db] = mfma16k16_bf16(ak, bh, acch[db]);
          acch[db] = mfma16k16_bf16(ak, bl, acch[db]);
        }
      }
      // dQe of the band: E^T (c dS^T), E^T read transposed from the bf16 E table
#pragma unroll
      for (int bb = 0; bb < 2; ++bb) {
        if (16 * bb < JB) {
          const f32x4 dsr = *reinterpret_cast<const f32x4*>(scr + lr * kBandSlots + 16 * bb + 4 * lc);
          float cd[4], cl[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            cd[r] = kScale * dsr[r];
            cl[r] = cd[r] - round_bf16(cd[r]);
          }
          const i16x4 bh = __builtin_bit_cast(i16x4, make_uint2(pack_bf16x2(cd[0], cd[1]), pack_bf16x2(cd[2], cd[3])));
          const i16x4 bl = __builtin_bit_cast(i16x4, make_uint2(pack_bf16x2(cl[0], cl[1]), pack_bf16x2(cl[2], cl[3])));
#pragma unroll
          for (int db = 0; db < 4; ++db) {
            const i16x4 ae = lds_read_tr16(sE + (16 * bb + 4 * lc + (lr >> 2)) * kERowT + 16 * (lr & 3) + 4 * db);
            acch[db] = mfma16k16_bf16(ae, bh, acch[db]);
            acch[db] = mfma16k16_bf16(ae, bl, acch[db]);
          }
        }
      }
      // the band's dS into the workspace matrix (query column n0w + lr, rows j = lc + 4 k)
      for (int j = lc; j < JB; j += 4) {
        const uint32_t off = n0w + lr < N ? static_cast<uint32_t>(4 * (j * N + n0w + lr)) : kOutOfRange;
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(scr[lr * kBandSlots + j]), rds, off, 0, 0);
      }
      // into the gather layout: query qi, dims 16 g + i <- band lane (lc = g, lr = qi)
      const int srcq = 4 * (qi + 16 * g);
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          bandq[4 * db + r] = __int_as_float(
              __builtin_amdgcn_ds_bpermute(srcq, __float_as_int(acch[db][r])));
      __builtin_amdgcn_wave_barrier();
    }
    for (int i = l; i < lay.dphw; i += kWave) scr[i] = 0.f;   // this wave's dPhase table
    __builtin_amdgcn_wave_barrier();

    float dq[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) dq[i] = bandq[i];
    float dy = 0.f;
    f32x4 dqe[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) dqe[nb] = zero4();

    auto fetch = [&](int k0, DqChunk<SHIFT, CJ>& c) {
#pragma unroll
      for (int jj = 0; jj < CJ; ++jj) {
        const int2 e = s_list[k0 + jj];
        const int j = uniform(e.x), d = uniform(e.y);
        c.j[jj] = j;
        c.ok[jj] = static_cast<uint32_t>(n_eff - d) < static_cast<uint32_t>(N);
        const uint32_t ko = static_cast<uint32_t>(kb_lane - d * ks_b);
        const uint32_t vo = static_cast<uint32_t>(vb_lane - d * vs_b);
        const uint32_t zo = (j >= J_small && j < J) ? static_cast<uint32_t>(zb_lane - d * zs_b) : kOutOfRange;
        c.k[jj][0] = buf_load16(rk, ko);
        c.k[jj][1] = buf_load16(rk, ko + 16);
        c.v[jj][0] = buf_load16(rv, vo);
        c.v[jj][1] = buf_load16(rv, vo + 16);
        c.z[jj] = buf_load_f32(rz, zo);
        c.pb2[jj] = s_pb2[j];
      }
    };

    // per pair of the chunk (qe: <q, e_j> of the lane's query, from the step's
    // MFMA): returns dS in ds_out[jj] and the lane's dPhase terms (tq, tq y z)
    // in ph_out[2 jj], ph_out[2 jj + 1]
    auto consume = [&](const DqChunk<SHIFT, CJ>& c, float* ds_out, float* ph_out, float qe) {
#pragma unroll
      for (int jj = 0; jj < CJ; ++jj) {
        const int j = c.j[jj];
        const bool far = j >= J_small && j < J;
        const uint32_t* kw = reinterpret_cast<const uint32_t*>(&c.k[jj][0]);
        const uint32_t* vw = reinterpret_cast<const uint32_t*>(&c.v[jj][0]);
        float dot = 0.f, gd = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          dot = dot2bf(q32[i], kw[i], dot);
          gd = dot2bf(d32[i], vw[i], gd);
        }
        float tq_pre = 0.f, pg = 0.f;
        if (far) {
          const float2 ph = s_ph[(j - J_small) * kPlanes + g];
          pg = ph.y;
          float sn, cs;
          dsincos<true>(fmaf(ph.y * yg, c.z[jj], ph.x), &sn, &cs);
          const float va = (SHIFT & 1) ? bf16_hi(vw[SHIFT >> 1]) : bf16_lo(vw[SHIFT >> 1]);
          const float vb = ((SHIFT + 1) & 1) ? bf16_hi(vw[(SHIFT + 1) >> 1]) : bf16_lo(vw[(SHIFT + 1) >> 1]);
          const float da = (SHIFT & 1) ? bf16_hi(d32[SHIFT >> 1]) : bf16_lo(d32[SHIFT >> 1]);
          const float db = ((SHIFT + 1) & 1) ? bf16_hi(d32[(SHIFT + 1) >> 1]) : bf16_lo(d32[(SHIFT + 1) >> 1]);
          gd += da * (cs * va - sn * vb - va) + db * (sn * va + cs * vb - vb);
          tq_pre = da * (-va * sn - vb * cs) + db * (va * cs - vb * sn);
        }
        dot = group_sum<4>(dot) + qe;
        gd = group_sum<4>(gd);
        // exp2(-inf) = 0 without a source (no branch around the exponential)
        const float P = __builtin_amdgcn_exp2f(c.ok[jj] ? fmaf(dot, kC, c.pb2[jj]) - lse2 : -INFINITY);
        const float dS = P * (gd - dlt);
        const float cds = kScale * dS;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          dq[2 * i] = fmaf(cds, bf16_lo(kw[i]), dq[2 * i]);
          dq[2 * i + 1] = fmaf(cds, bf16_hi(kw[i]), dq[2 * i + 1]);
        }
        // keep the accumulation here: sunk to the loop latch it holds every
        // chunk's K registers live and the prefetch turns into register copies
        pin_regs<16>(dq);
        // the four lanes of a query store the same value; rows past N and the
        // sentinel go out of range (dropped)
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(dS), rds, j < J ? ds_lane + 4 * j * N : kOutOfRange, 0,
                                              0);
        ds_out[jj] = dS;
        const float tq = P * tq_pre;
        dy = fmaf(tq * pg, c.z[jj], dy);
        pin_regs<1>(&dy);
        ph_out[2 * jj] = tq;
        ph_out[2 * jj + 1] = tq * yg * c.z[jj];
      }
    };

    // dQe += dS (16 queries x the step's 4 offsets) E (4 rows x 64 dims):
    // lane (lr, lc) supplies dS of query lr at offset lc (from the lane of
    // query lr with g = lc) and E[j_lc][16 nb + lr].
    auto dqe_step = [&](const float* ds4, const int* j4) {
      const float sel = pick4(g, ds4[0], ds4[1], ds4[2], ds4[3]);
      const float av = __shfl(sel, 4 * lr + lc);
      const int jsel = pick4(lc, j4[0], j4[1], j4[2], j4[3]);
      const uint16_t* er = sE + jsel * kERowT + lr;
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
        dqe[nb] = mfma16_f32(av, __uint_as_float(static_cast<uint32_t>(er[16 * nb]) << 16), dqe[nb]);
    };

    // dPhase of the step's four offsets summed over the wave's 16 queries,
    // reduce-scattered: after the two lane swaps 16-lane row k holds offset k
    // (tq in u0, tq y z in u1) for four queries per plane, and two row
    // rotations add the other twelve.  Far offsets are stored (each appears
    // once in the list: a store, no accumulation).
    auto dphase_step = [&](const float* ph8, const int* j4) {
      float r[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) r[i] = add_swap32(ph8[i], ph8[i + 4]);
      float u0 = add_swap16(r[0], r[2]), u1 = add_swap16(r[1], r[3]);
      u0 += dpp_f<0x124>(u0);   // row_ror:4
      u1 += dpp_f<0x124>(u1);
      u0 += dpp_f<0x128>(u0);   // row_ror:8
      u1 += dpp_f<0x128>(u1);
      const int k = l >> 4;
      const int jk = pick4(k, j4[0], j4[1], j4[2], j4[3]);
      if (((l >> 2) & 3) == 0 && jk >= J_small && jk < J)
        *reinterpret_cast<float2*>(s_dph + (jk - J_small) * 8 + 2 * g) = make_float2(u0, u1);
    };

    if (cnt > 0) {
      DqChunk<SHIFT, CJ> c0, c1;
      fetch(0, c0);
      for (int k0 = 0; k0 < cnt; k0 += kStepDq) {
        float ds4[kStepDq], ph8[2 * kStepDq];
        int j4[kStepDq];
        // <q, e_j> of the wave's 16 queries for the step's four offsets:
        // A = the four E rows (rows 4..15 zero), B = q^T; lane q (< 16)
        // receives offset k in register k
        f32x4 qe = zero4();
        {
          uint4 ea[2] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
          if (lr < kStepDq) {
            const int jr = s_list[k0 + lr].x;
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
              ea[ks] = *reinterpret_cast<const uint4*>(sE + jr * kERowT + 32 * ks + 8 * lc);
          }
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) qe = mfma16_bf16(bf16x8_from_bits(ea[ks]), bf16x8_from_bits(xq[ks]), qe);
        }
        j4[0] = c0.j[0];
        fetch(k0 + 1, c1);
        consume(c0, ds4, ph8, __shfl(qe[0], qi));
        j4[1] = c1.j[0];
        fetch(k0 + 2, c0);
        consume(c1, ds4 + 1, ph8 + 2, __shfl(qe[1], qi));
        j4[2] = c0.j[0];
        fetch(k0 + 3, c1);
        consume(c0, ds4 + 2, ph8 + 4, __shfl(qe[2], qi));
        j4[3] = c1.j[0];
        fetch(k0 + 4, c0);
        consume(c1, ds4 + 3, ph8 + 6, __shfl(qe[3], qi));
        dqe_step(ds4, j4);
        dphase_step(ph8, j4);
      }
    }
    __syncthreads();   // every wave's dPhase table is complete
    // dPhase of this tile: the four waves' sums in a fixed order
    for (int i = lane; i < JL * 8; i += kBlock)
      part_ph[prow * JL * 8 + i] = ((s_dph_all[i] + s_dph_all[lay.dphw + i]) + s_dph_all[2 * lay.dphw + i]) +
                                   s_dph_all[3 * lay.dphw + i];
    // dQe rows move from the MFMA layout (query 4 lc + r, dim 16 nb + lr) to
    // the lane layout through the wave's staging area, half a row at a time
#pragma unroll
    for (int half = 0; half < 2; ++half) {
#pragma unroll
      for (int nb = 2 * half; nb < 2 * half + 2; ++nb)
#pragma unroll
        for (int r = 0; r < 4; ++r) s_st[(4 * lc + r) * kStRow + 16 * (nb - 2 * half) + lr] = dqe[nb][r];
      __builtin_amdgcn_wave_barrier();
      if ((g >> 1) == half) {
        const float4* src = reinterpret_cast<const float4*>(s_st + qi * kStRow + 16 * (g - 2 * half));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float4 x = src[i];
          dq[4 * i] = fmaf(kScale, x.x, dq[4 * i]);
          dq[4 * i + 1] = fmaf(kScale, x.y, dq[4 * i + 1]);
          dq[4 * i + 2] = fmaf(kScale, x.z, dq[4 * i + 2]);
          dq[4 * i + 3] = fmaf(kScale, x.w, dq[4 * i + 3]);
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
    // with query_probes y was formed from q in the forward: dy goes into dq through the probe
    // features (the block's einsum backward, dsqg:3231-3254) instead of out to dy_pre
    if (f.query_probes) fold_probe_grad(dq, q32, f.query_probes, g, yg, dy);
    if (row_ok) {
      uint4* o4 = reinterpret_cast<uint4*>(reinterpret_cast<bf16*>(a.dq) + b * a.dq_stride[0] + h * a.dq_stride[1] +
                                           nn * a.dq_stride[2] + 16 * g);
      uint4 x0, x1;
      x0.x = pack_bf16x2(dq[0], dq[1]);   x0.y = pack_bf16x2(dq[2], dq[3]);
      x0.z = pack_bf16x2(dq[4], dq[5]);   x0.w = pack_bf16x2(dq[6], dq[7]);
      x1.x = pack_bf16x2(dq[8], dq[9]);   x1.y = pack_bf16x2(dq[10], dq[11]);
      x1.z = pack_bf16x2(dq[12], dq[13]); x1.w = pack_bf16x2(dq[14], dq[15]);
      o4[0] = x0;
      o4[1] = x1;
      if (!f.query_probes) a.dy_pre[(static_cast<int64_t>(bh) * N + n) * kPlanes + g] = dy;
    }
  }
}

// The delta stage on its own (DWARF_SCHED_DELTA_STAGE): the (delta, lse in
// log2 units) pairs of the dQ prologue, with the same lane layout and the same
// arithmetic (delta = <dO, O_bf16> as v_dot2 over the lane's 16 dims, then the
// four lanes' sum by DPP), so the pairs equal bit for bit those the dQ launch
// forms (reference: _compute_D_v18_grouped, dsqg:1263-1289).  One 64-query
// tile per workgroup.
__global__ __launch_bounds__(kBlock) void dsqg_bwd_delta_bf16(const dwarf_dsqg_bwd_args a, float* __restrict__ delta_ws,
                                                             int tiles) {
  const dwarf_dsqg_fwd_args& f = a.fwd;
  const int N = f.N;
  const int T = xcd_remap(blockIdx.x, static_cast<int>(gridDim.x));
  const int bh = T / tiles;
  const int t = T - bh * tiles;
  const int b = bh / f.H;
  const int h = bh - b * f.H;
  const int lane = threadIdx.x;
  const int w = lane / kWave;
  const int l = lane % kWave;
  const int g = l & 3;
  const int qi = l >> 2;
  const int n = t * kQT + kQPW * w + qi;
  const bool row_ok = n < N;
  const bool live = row_ok && n >= f.query_start;
  const int64_t nn = n;
  float dlt = 0.f, lse2 = 0.f;
  bool mass = false;
  if (live) {
    const bf16* dob = reinterpret_cast<const bf16*>(a.dout) + b * a.dout_stride[0] + h * a.dout_stride[1];
    const bf16* ob = reinterpret_cast<const bf16*>(f.out) + b * f.out_stride[0] + h * f.out_stride[1];
    const uint4* d4 = reinterpret_cast<const uint4*>(dob + nn * a.dout_stride[2] + 16 * g);
    const uint4* o4 = reinterpret_cast<const uint4*>(ob + nn * f.out_stride[2] + 16 * g);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint4 y = d4[i], o = o4[i];
      dlt = dot2bf(y.x, o.x, dlt); dlt = dot2bf(y.y, o.y, dlt);
      dlt = dot2bf(y.z, o.z, dlt); dlt = dot2bf(y.w, o.w, dlt);
    }
    const float lse = f.lse[b * f.lse_stride[0] + h * f.lse_stride[1] + nn * f.lse_stride[2]];
    mass = lse > -INFINITY;
    lse2 = mass ? lse * kLog2e : 0.f;
  }
  dlt = group_sum<4>(dlt);
  if (row_ok && g == 0)
    *reinterpret_cast<float2*>(delta_ws + 2 * (static_cast<int64_t>(bh) * N + n)) =
        make_float2(dlt, mass ? lse2 : INFINITY);
}

template <int MBW>
__global__ __launch_bounds__(kBlock, dse_wgs_per_cu(MBW)) void dsqg_bwd_dse_bf16(const dwarf_dsqg_bwd_args a,
                                                               const float* __restrict__ ds_ws,
                                                               float* __restrict__ part_se,
                                                               float* __restrict__ part_pb, int tiles) {
  constexpr int kQRow = 72;   // bf16 row stride of the staged Q tile
  const dwarf_dsqg_fwd_args& f = a.fwd;
  const int J = f.J, N = f.N;
  const int JB = (J + 1 + 15) / 16;   // 16-row blocks of dS; wave w takes blocks w, w + 4, ...
  __shared__ int s_off[64 * MBW];
  __shared__ __attribute__((aligned(16))) uint16_t s_q[kQT * kQRow];
  for (int j = threadIdx.x; j < 64 * MBW; j += kBlock) s_off[j] = j < J ? f.offsets[j] : 0;
  __syncthreads();
  const int lane = threadIdx.x;
  const int w = lane / kWave;
  const int l = lane % kWave;
  const int lr = l & 15, lc = l >> 4;
  const int qs_b = static_cast<int>(f.q_stride[2]) * 2;
  // dSE[16 (w + 4 i) + 4 lc + r][16 nb + lr] of this workgroup, over all its tiles
  f32x4 dse[MBW][4];
#pragma unroll
  for (int i = 0; i < MBW; ++i)
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) dse[i][nb] = zero4();
  bf16x8 one;
#pragma unroll
  for (int e = 0; e < 8; ++e) one[e] = static_cast<__bf16>(lr == 0 ? 1.f : 0.f);

  const TileOrder order(static_cast<int64_t>(tiles) * f.B * f.H);
  for (int kstep = 0; kstep < order.steps(); ++kstep) {
    const int T = order.tile(kstep);
    if (T < 0) continue;   // uniform over the workgroup
    const int bh = T / tiles;
    const int t = T - bh * tiles;
    const int b = bh / f.H;
    const int h = bh - b * f.H;
    const int64_t prow = static_cast<int64_t>(h * f.B + b) * tiles + t;
    const int n0 = t * kQT;
    const __amdgpu_buffer_rsrc_t rq =
        rows_rsrc(reinterpret_cast<const bf16*>(f.q) + b * f.q_stride[0] + h * f.q_stride[1], qs_b, N, 128);
    // the (b, h) slab of the dS matrix: J rows of N fp32
    const __amdgpu_buffer_rsrc_t rds = rows_rsrc(ds_ws + static_cast<int64_t>(bh) * J * N, 4 * N, J, 4 * N);
    // this wave's dS blocks and this lane's Q chunks, loaded before the barrier
    uint4 xs[MBW][2][2], qv[2];
#pragma unroll
    for (int i = 0; i < MBW; ++i) {
      const int j = 16 * (w + 4 * i) + lr;
      const int dj = j < J ? s_off[j] : 0;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int nb0 = n0 + 32 * ks + 8 * lc;
        // eight entries that are all unwritten (n < offset_j) are not fetched
        const bool any = j < J && nb0 + 7 >= dj && nb0 < N;
        const uint32_t off = any ? static_cast<uint32_t>((j * N + nb0) * 4) : kOutOfRange;
        xs[i][ks][0] = buf_load16(rds, off);
        xs[i][ks][1] = buf_load16(rds, off + 16);
      }
    }
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const int i = lane + kBlock * s2;   // 64 rows x 8 chunks of 16 bytes
      const int nq = n0 + (i >> 3);
      qv[s2] = buf_load16(rq, nq < N ? static_cast<uint32_t>(nq * qs_b + 16 * (i & 7)) : kOutOfRange);
    }
    __syncthreads();   // the previous tile's Q reads are done
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const int i = lane + kBlock * s2;
      *reinterpret_cast<uint4*>(s_q + (i >> 3) * kQRow + 8 * (i & 7)) = qv[s2];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < MBW; ++i) {
      const int mb = w + 4 * i;
      if (mb >= JB) break;
      const int j = 16 * mb + lr;
      const int dj = s_off[j];
      f32x4 c1 = zero4();
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int nb0 = n0 + 32 * ks + 8 * lc;
        const uint32_t xw[8] = {xs[i][ks][0].x, xs[i][ks][0].y, xs[i][ks][0].z, xs[i][ks][0].w,
                                xs[i][ks][1].x, xs[i][ks][1].y, xs[i][ks][1].z, xs[i][ks][1].w};
        float x[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int nq = nb0 + e;
          // written entries only: n - offset_j >= 0 and n < N
          x[e] = (nq < N && nq >= dj) ? __uint_as_float(xw[e]) : 0.f;
        }
        bf16x8 ahi, alo;
        split_bf16x8(x, ahi, alo);
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
          // Q rows 32 ks + 8 lc + (0..7), dim 16 nb + lr, read transposed
          const uint16_t* src = s_q + (32 * ks + 8 * lc + (lr >> 2)) * kQRow + 16 * nb + 4 * (lr & 3);
          const i16x4 lo4 = lds_read_tr16(src), hi4 = lds_read_tr16(src + 4 * kQRow);
          const bf16x8 bq = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
          dse[i][nb] = mfma16_bf16(ahi, bq, dse[i][nb]);
          dse[i][nb] = mfma16_bf16(alo, bq, dse[i][nb]);
        }
        c1 = mfma16_bf16(ahi, one, c1);
        c1 = mfma16_bf16(alo, one, c1);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int jr = 16 * mb + 4 * lc + r;
        if (lr == 0 && jr < J) part_pb[prow * J + jr] = c1[r];
      }
    }
  }
  constexpr float kScale = 0.125f;
#pragma unroll
  for (int i = 0; i < MBW; ++i)
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = 16 * (w + 4 * i) + 4 * lc + r;
        if (j < J)
          part_se[(static_cast<int64_t>(blockIdx.x) * J + j) * kHeadDim + 16 * nb + lr] = kScale * dse[i][nb][r];
      }
}

hipError_t launch_dq_bf16_g4(const dwarf_dsqg_bwd_args& a, const BwdWorkspace& ws, hipStream_t stream) {
  const dwarf_dsqg_fwd_args& f = a.fwd;
  char* base = static_cast<char*>(a.workspace);
  float* delta = reinterpret_cast<float*>(base + ws.delta_off);
  float* ds = reinterpret_cast<float*>(base + ws.ds_off);
  float* part_ph = reinterpret_cast<float*>(base + ws.part_ph_off);
  if (ws.dq_gather_wgs == 0) return hipSuccess;
  const size_t lds = dq_g4_layout(f.J, f.J_large).bytes;
#define DWARF_DQG4_CASE(S)                                                                                     \
  case S:                                                                                                      \
    hipLaunchKernelGGL((dsqg_bwd_dq_bf16_g4<S>), dim3(ws.dq_gather_wgs), dim3(kBlock), lds, stream, a,     \
                       delta, ds, part_ph, ws.dq_tiles);                                                       \
    break;
  switch (f.plane_shift) {
    DWARF_DQG4_CASE(0) DWARF_DQG4_CASE(1) DWARF_DQG4_CASE(2) DWARF_DQG4_CASE(3) DWARF_DQG4_CASE(4)
    DWARF_DQG4_CASE(5) DWARF_DQG4_CASE(6) DWARF_DQG4_CASE(7) DWARF_DQG4_CASE(8) DWARF_DQG4_CASE(9)
    DWARF_DQG4_CASE(10) DWARF_DQG4_CASE(11) DWARF_DQG4_CASE(12) DWARF_DQG4_CASE(13) DWARF_DQG4_CASE(14)
    default: return hipErrorInvalidValue;
  }
#undef DWARF_DQG4_CASE
  return hipGetLastError();
}

template <int MBW>
hipError_t launch_dse_bf16(const dwarf_dsqg_bwd_args& a, const BwdWorkspace& ws, hipStream_t stream) {
  char* base = static_cast<char*>(a.workspace);
  const float* ds = reinterpret_cast<const float*>(base + ws.ds_off);
  float* part_se = reinterpret_cast<float*>(base + ws.part_se_off);
  float* part_pb = reinterpret_cast<float*>(base + ws.part_pb_off);
  hipLaunchKernelGGL((dsqg_bwd_dse_bf16<MBW>), dim3(ws.dq_wgs), dim3(kBlock), 0, stream, a, ds, part_se, part_pb,
                     ws.dq_tiles);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_dq_typed(const dwarf_dsqg_bwd_args& a, const BwdWorkspace& ws, hipStream_t stream) {
  const dwarf_dsqg_fwd_args& f = a.fwd;
  char* base = static_cast<char*>(a.workspace);
  float* delta = reinterpret_cast<float*>(base + ws.delta_off);
  float* part_se = reinterpret_cast<float*>(base + ws.part_se_off);
  float* part_pb = reinterpret_cast<float*>(base + ws.part_pb_off);
  float* part_ph = reinterpret_cast<float*>(base + ws.part_ph_off);
  const size_t lds = dq_lds<T>(f.J).bytes;
#define DWARF_DQ_CASE(S)                                                                                        \
  case S:                                                                                                       \
    hipLaunchKernelGGL((dsqg_bwd_dq_v2<T, S>), dim3(ws.dq_wgs), dim3(kBlock), lds, stream, a, delta, part_se,   \
                       part_pb, part_ph, ws.dq_tiles, ws.dq_tpw, ws.dq_ntg, ws.dq_wgs);                          \
    break;
  switch (f.plane_shift) {
    DWARF_DQ_CASE(0) DWARF_DQ_CASE(1) DWARF_DQ_CASE(2) DWARF_DQ_CASE(3) DWARF_DQ_CASE(4)
    DWARF_DQ_CASE(5) DWARF_DQ_CASE(6) DWARF_DQ_CASE(7) DWARF_DQ_CASE(8) DWARF_DQ_CASE(9)
    DWARF_DQ_CASE(10) DWARF_DQ_CASE(11) DWARF_DQ_CASE(12) DWARF_DQ_CASE(13) DWARF_DQ_CASE(14)
    default:
      return hipErrorInvalidValue;
  }
#undef DWARF_DQ_CASE
  return hipGetLastError();
}

}  // namespace

hipError_t launch_dsqg_bwd_delta(const dwarf_dsqg_bwd_args& a, const BwdWorkspace& ws, hipStream_t stream) {
  const dwarf_dsqg_fwd_args& f = a.fwd;
  const int total = ws.dq_tiles * f.B * f.H;
  if (total == 0) return hipSuccess;
  float* delta = reinterpret_cast<float*>(static_cast<char*>(a.workspace) + ws.delta_off);
  hipLaunchKernelGGL(dsqg_bwd_delta_bf16, dim3(total), dim3(kBlock), 0, stream, a, delta, ws.dq_tiles);
  return hipGetLastError();
}

size_t dq_lds_bytes(int J, int J_large, int dtype) {
  return dtype == DWARF_BF16 ? dq_g4_layout(J, J_large).bytes : dq_lds<float>(J).bytes;
}

int dq_gather_wgs_per_cu() { return kGatherWgsPerCu; }
int dq_dse_wgs_per_cu(int J) { return dse_wgs_per_cu(dse_blocks_per_wave(J)); }

int dq_tile_queries(int dtype) { return dtype == DWARF_BF16 ? kQT : kQ; }

hipError_t launch_dsqg_bwd_dq(const dwarf_dsqg_bwd_args& a, const BwdWorkspace& ws, hipStream_t stream) {
  if (a.fwd.dtype == DWARF_BF16) return launch_dq_bf16_g4(a, ws, stream);
  return launch_dq_typed<float>(a, ws, stream);
}

hipError_t launch_dsqg_bwd_dse(const dwarf_dsqg_bwd_args& a, const BwdWorkspace& ws, hipStream_t stream) {
  if (a.fwd.dtype != DWARF_BF16 || ws.dq_gather_wgs == 0) return hipSuccess;   // fp32: partials come with dQ
  if (dse_blocks_per_wave(a.fwd.J) == 2) return launch_dse_bf16<2>(a, ws, stream);
  return launch_dse_bf16<5>(a, ws, stream);
}

}  // namespace dwarf
