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
#include "gather.h"
#include "mfma.h"

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

// ---- bf16 dK/dV launch: four lanes per key ------------------------------
// A workgroup of 4 waves owns 64 consecutive keys of one (b, kv head); wave w
// owns keys 16w..16w+15 and lane g of a key holds head dims [16g, 16g+16) of
// its K and V rows and of the dK/dV accumulators.  Each wave lists the
// offsets that give one of its keys a query n = m + delta inside [0, N) and
// walks that list once per query head of the GQA group, in chunks of CJ with
// the next chunk's loads in flight: the lane gathers its slices of q_n and
// dO_n (16-byte buffer loads) plus lse_n, delta_n and y_n[g]; lanes without a
// query read zeros through an out-of-range offset and get P = 0.  Per pair:
// <q, k + e_j> and <dO, v> on v_dot2_f32_bf16 (summed over the 4 lanes by
// DPP), P, dS = P (g - delta), dK += c dS q_n and dV += P R^T dO_n in fp32; the
// MOVT pair of plane g lies in lane g's slice (plane_shift <= 14), so the
// lane also forms its dZ term.  Reference kernel: _bwd_dkdv_v18_grouped
// (dsqg:1734-1955).
constexpr int kKPW = 16;       // keys per wave
constexpr int kKPB = 64;       // keys per workgroup
constexpr int kChunkKv = 1;    // offsets per prefetch chunk
constexpr int kMinWgKv = 3;    // workgroups per CU the register budget is sized for
constexpr int kERowKv = 72;    // bf16 E row stride (elements)
// Near band: the leading small offsets j < JB (ascending, unique, at most
// kBandMaxKv) are served on the matrix cores from Q / dO windows of the
// queries [m0, m0 + 96) of the workgroup's 64 keys; the gather loop takes the
// other offsets.
constexpr int kBandMaxKv = 32;
constexpr int kWinRowsKv = kKPB + kBandMaxKv;   // 96 query rows of 128 bytes per window

struct KvLayout {
  int JE, JL4, list_len, group;
  size_t off_ph, off_list, off_e, off_jn, off_win, off_dl, bytes;
};

__host__ __device__ inline KvLayout kv_layout(int J, int J_large, int group, int CJ) {
  KvLayout L;
  L.JE = (J + 1 + 15) / 16 * 16;
  L.JL4 = (J_large + 1) / 2 * 2;
  L.group = group;
  L.list_len = (L.JE + 4 * CJ + 1) / 2 * 2;
  L.off_ph = static_cast<size_t>(group + 1) * L.JE * 4;                  // s_pb2[group][JE], s_off[JE]
  L.off_list = L.off_ph + static_cast<size_t>(group) * L.JL4 * 4 * 8;    // s_ph[group][JL4][4] float2
  L.off_e = L.off_list + static_cast<size_t>(4 * L.list_len) * 8;        // s_list[4][list_len] int2
  L.off_jn = L.off_e + static_cast<size_t>(L.JE) * kERowKv * 2;          // sE[JE][72] bf16
  L.off_win = L.off_jn + kJnSize * 4;                                    // s_jn[kJnSize] int
  L.off_dl = L.off_win + static_cast<size_t>(2 * kWinRowsKv) * 128;      // Q window, dO window [96][128 B]
  L.bytes = L.off_dl + static_cast<size_t>(kWinRowsKv) * 8;              // s_dl[96] (delta, log2 lse)
  return L;
}

template <int CJ>
struct KvChunk {
  uint4 q[CJ][2], d[CJ][2];
  float2 dl2[CJ];   // (delta, lse in log2 units; +inf without softmax mass)
  float y[CJ];
  int j[CJ];
};

template <int SHIFT, int CJ, int MINWG>
__global__ __launch_bounds__(kBlock, MINWG) void dsqg_bwd_dkdv_bf16_k4(const dwarf_dsqg_bwd_args a,
                                                                   const float* __restrict__ delta_ws, int tiles,
                                                                   int total, int whole, int nsplit,
                                                                   float* __restrict__ kvp) {
  constexpr float kC = 0.125f * kLog2e;
  constexpr float kScale = 0.125f;
  static_assert(SHIFT + 1 < kHeadDim / kPlanes, "MOVT pair must stay inside one lane's slice");
  const dwarf_dsqg_fwd_args& f = a.fwd;
  const int J = f.J, N = f.N, J_small = f.J_small, JL = f.J_large;
  const int group = f.H / f.H_kv;
  const KvLayout lay = kv_layout(J, JL, group, CJ);
  extern __shared__ float smem[];
  char* sm = reinterpret_cast<char*>(smem);
  float* s_pb2 = smem;                                   // [group][JE] log2(e) * pb
  int* s_off = reinterpret_cast<int*>(smem + group * lay.JE);
  float2* s_ph = reinterpret_cast<float2*>(sm + lay.off_ph);
  int2* s_list_all = reinterpret_cast<int2*>(sm + lay.off_list);
  uint16_t* sE = reinterpret_cast<uint16_t*>(sm + lay.off_e);
  int* s_jn = reinterpret_cast<int*>(sm + lay.off_jn);  // [0]: JB; [d]: band slot of offset d, or -1
  char* s_qw = sm + lay.off_win;                         // Q rows m0 .. m0 + 95 (16-byte chunks swizzled)
  char* s_dw = s_qw + kWinRowsKv * 128;                  // dO rows, same layout
  float2* s_dl = reinterpret_cast<float2*>(sm + lay.off_dl);

  // Work units are (b, kv head, key tile).  The first `whole` workgroups take units 0 .. whole - 1 with all
  // of the group's query heads; the others take the remaining units in subsets of group / nsplit query
  // heads, the subsets of a unit side by side, and leave fp32 partials for dsqg_bwd_dkdv_combine.
  const bool part = static_cast<int>(blockIdx.x) >= whole;   // uniform
  int unit, split = 0, ns = 1;
  if (!part) {
    unit = xcd_remap(blockIdx.x, whole);
  } else {
    const int t = xcd_remap(blockIdx.x - whole, total - whole);
    unit = whole + t / nsplit;
    split = t - (unit - whole) * nsplit;
    ns = nsplit;
  }
  const int bhk = unit / tiles;
  const int tile = unit - bhk * tiles;
  const int b = bhk / f.H_kv;
  const int hk = bhk - b * f.H_kv;
  const int hh0 = split * (group / ns), hh1 = hh0 + group / ns;   // the workgroup's query heads

  // this lane's key row (K, V slices and z) is requested first, so its latency
  // overlaps the table staging
  const int lane = threadIdx.x;
  const int w = lane / kWave;
  const int l = lane % kWave;
  const int g = l & 3;
  const int ki = l >> 2;
  const int lr = l & 15, lc = l >> 4;
  const int m0 = tile * kKPB;
  const int m0w = m0 + w * kKPW;
  const int m = m0w + ki;
  const bool key_ok = m < N;
  const int64_t mm = m;
  uint4 kx0 = {0u, 0u, 0u, 0u}, kx1 = {0u, 0u, 0u, 0u}, vx0 = {0u, 0u, 0u, 0u}, vx1 = {0u, 0u, 0u, 0u};
  float zg = 0.f;
  const bf16* kbase = reinterpret_cast<const bf16*>(f.k) + b * f.k_stride[0] + hk * f.k_stride[1];
  const bf16* vbase = reinterpret_cast<const bf16*>(f.v) + b * f.v_stride[0] + hk * f.v_stride[1];
  if (key_ok) {
    const uint4* k4 = reinterpret_cast<const uint4*>(kbase + mm * f.k_stride[2] + 16 * g);
    const uint4* v4 = reinterpret_cast<const uint4*>(vbase + mm * f.v_stride[2] + 16 * g);
    kx0 = k4[0]; kx1 = k4[1]; vx0 = v4[0]; vx1 = v4[1];
    zg = f.z_pre[b * f.z_stride[0] + hk * f.z_stride[1] + mm * f.z_stride[2] + g];
  }

  stage_tables<true, true, true, true, true>(
      f, lay.JE, hk * group, group,
      TableStage{sE, kERowKv, s_pb2, kLog2e, s_off, s_ph, lay.JL4 * kPlanes, s_jn, kBandMaxKv, kBandMaxKv,
                 (f.schedule & DWARF_SCHED_BAND) != 0});
  __syncthreads();
  const int JB = s_jn[0];
  const bool wave_live = m0w < N;   // waves past the end still reach every barrier

  const int m_hi = min(m0w + kKPW - 1, N - 1);
  int2* s_list = s_list_all + w * lay.list_len;
  // offsets giving some key m0w..m_hi a query m + delta in [0, N), the band's
  // left out; the sentinel offset N + 16 - m0w puts every key's query past the end.
  const int cnt = wave_live ? build_offset_list<CJ>(s_list, s_off, J, m0w, m_hi, N, -1, make_int2(J, N + 16 - m0w), JB)
                            : 0;
  const int cntp = (cnt + CJ - 1) / CJ * CJ;

  const uint32_t k32[8] = {kx0.x, kx0.y, kx0.z, kx0.w, kx1.x, kx1.y, kx1.z, kx1.w};
  const uint32_t v32[8] = {vx0.x, vx0.y, vx0.z, vx0.w, vx1.x, vx1.y, vx1.z, vx1.w};
  // own V pair of plane g (dims 16g + SHIFT, +1)
  const float va = (SHIFT & 1) ? bf16_hi(v32[SHIFT >> 1]) : bf16_lo(v32[SHIFT >> 1]);
  const float vb = ((SHIFT + 1) & 1) ? bf16_hi(v32[(SHIFT + 1) >> 1]) : bf16_lo(v32[(SHIFT + 1) >> 1]);
  // the wave's keys as MFMA B operands for the band: key m0w + lr, dims 32 ks + 8 lc + [0, 8)
  uint4 kB[2] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}}, vB[2] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
  if (JB > 0 && m0w + lr < N) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      kB[ks] = *reinterpret_cast<const uint4*>(kbase + static_cast<int64_t>(m0w + lr) * f.k_stride[2] + 32 * ks + 8 * lc);
      vB[ks] = *reinterpret_cast<const uint4*>(vbase + static_cast<int64_t>(m0w + lr) * f.v_stride[2] + 32 * ks + 8 * lc);
    }
  }

  float dk[16], dv[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) { dk[i] = 0.f; dv[i] = 0.f; }
  float dz = 0.f;

  // a key past the end uses m_eff = m0w - 2N - 64: m_eff + delta < 0 for every listed delta
  const int m_eff = key_ok ? m : m0w - 2 * N - 64;
  const int qs_b = static_cast<int>(f.q_stride[2]) * 2, ds_b = static_cast<int>(a.dout_stride[2]) * 2;
  const int ys_b = static_cast<int>(f.y_stride[2]) * 4;
  const int qb_lane = m_eff * qs_b + 32 * g, db_lane = m_eff * ds_b + 32 * g;
  const int yb_lane = m_eff * ys_b + 4 * g;

  for (int hh = hh0; hh < hh1; ++hh) {
    const int h = hk * group + hh;
    const int bh = b * f.H + h;
    const __amdgpu_buffer_rsrc_t rq =
        rows_rsrc(reinterpret_cast<const bf16*>(f.q) + b * f.q_stride[0] + h * f.q_stride[1], qs_b, N, 128);
    const __amdgpu_buffer_rsrc_t rd = rows_rsrc(
        reinterpret_cast<const bf16*>(a.dout) + b * a.dout_stride[0] + h * a.dout_stride[1], ds_b, N, 128);
    const __amdgpu_buffer_rsrc_t rdl = rows_rsrc(delta_ws + 2 * static_cast<int64_t>(bh) * N, 8, N, 8);
    const __amdgpu_buffer_rsrc_t ry = rows_rsrc(f.y_pre + b * f.y_stride[0] + h * f.y_stride[1], ys_b, N, 16);
    const float* pb2 = s_pb2 + hh * lay.JE;
    const float2* ph_h = s_ph + hh * lay.JL4 * kPlanes;

    // the near band's windows for this head: query rows m0 .. m0 + 95 of q and dO (three 1 KB DMA
    // loads per wave and window; LDS chunk (i & 7) of row i >> 3 holds the row's 16-byte chunk
    // (i & 7) ^ (row & 7), a bank spread) and their (delta, log2 lse) pairs (4-byte DMA loads).  They
    // land while the gather loop runs; the band follows it.
    typedef __attribute__((address_space(3))) void lds_void;
    if (JB > 0) {   // uniform over the workgroup
      if (hh > 0) __syncthreads();   // every wave is done with the previous head's windows
#pragma unroll
      for (int u = 0; u < 3; ++u) {
        const int i = kBlock * u + lane;
        const int row = i >> 3, c = (i & 7) ^ (row & 7);
        const int nq = m0 + row;   // past N: out of range, zeros
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, (lds_void*)(void*)(s_qw + 4096 * u + 1024 * w), 16,
                                                 static_cast<uint32_t>(nq * qs_b + 16 * c), 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rd, (lds_void*)(void*)(s_dw + 4096 * u + 1024 * w), 16,
                                                 static_cast<uint32_t>(nq * ds_b + 16 * c), 0, 0, 0);
      }
      if (w < 3)   // dwords 64 w + l of the (delta, log2 lse) rows m0 ..; past N: zeros (masked below)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rdl, (lds_void*)(void*)(reinterpret_cast<char*>(s_dl) + 256 * w), 4,
                                                 static_cast<uint32_t>(8 * m0 + 4 * lane), 0, 0, 0);
    }

    auto fetch = [&](int k0, KvChunk<CJ>& c) {
#pragma unroll
      for (int jj = 0; jj < CJ; ++jj) {
        const int2 e = s_list[k0 + jj];
        const int j = uniform(e.x), d = uniform(e.y);
        const int n = m_eff + d;
        c.j[jj] = j;
        // lane bases plus wave-uniform products (no per-lane multiplies).  A
        // query outside [0, N) reads zeros: its q and dO rows are 0, so the
        // pair adds nothing whatever P is.
        const uint32_t qo = static_cast<uint32_t>(qb_lane + d * qs_b);
        const uint32_t dof = static_cast<uint32_t>(db_lane + d * ds_b);
        c.q[jj][0] = buf_load16(rq, qo);
        c.q[jj][1] = buf_load16(rq, qo + 16);
        c.d[jj][0] = buf_load16(rd, dof);
        c.d[jj][1] = buf_load16(rd, dof + 16);
        // the elements are copied out before reinterpreting: this compiler
        // reads element 0 for __builtin_bit_cast of any element of the vector
        const auto x = __builtin_amdgcn_raw_buffer_load_b64(rdl, static_cast<uint32_t>(8 * n), 0, 0);
        const uint32_t x0 = x[0], x1 = x[1];
        c.dl2[jj] = make_float2(__uint_as_float(x0), __uint_as_float(x1));
        c.y[jj] = buf_load_f32(ry, (j >= J_small && j < J) ? static_cast<uint32_t>(yb_lane + d * ys_b) : kOutOfRange);
      }
    };

    auto consume = [&](const KvChunk<CJ>& c) {
#pragma unroll
      for (int jj = 0; jj < CJ; ++jj) {
        const int j = c.j[jj];
        const bool far = j >= J_small && j < J;
        const uint32_t* qw = reinterpret_cast<const uint32_t*>(&c.q[jj][0]);
        const uint32_t* dw = reinterpret_cast<const uint32_t*>(&c.d[jj][0]);
        const uint4* e4 = reinterpret_cast<const uint4*>(sE + j * kERowKv + 16 * g);
        const uint4 e0 = e4[0], e1 = e4[1];
        const uint32_t ew[8] = {e0.x, e0.y, e0.z, e0.w, e1.x, e1.y, e1.z, e1.w};
        float dot = 0.f, gd = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          dot = dot2bf(qw[i], k32[i], dot);
          dot = dot2bf(qw[i], ew[i], dot);
          gd = dot2bf(dw[i], v32[i], gd);
        }
        const float da = (SHIFT & 1) ? bf16_hi(dw[SHIFT >> 1]) : bf16_lo(dw[SHIFT >> 1]);
        const float db = ((SHIFT + 1) & 1) ? bf16_hi(dw[(SHIFT + 1) >> 1]) : bf16_lo(dw[(SHIFT + 1) >> 1]);
        float sn = 0.f, cs = 1.f, pg = 0.f;
        if (far) {
          const float2 ph = ph_h[(j - J_small) * kPlanes + g];
          pg = ph.y;
          dsincos<true>(fmaf(ph.y * c.y[jj], zg, ph.x), &sn, &cs);
          gd += da * (cs * va - sn * vb - va) + db * (sn * va + cs * vb - vb);
        }
        dot = group_sum<4>(dot);
        gd = group_sum<4>(gd);
        const float P = __builtin_amdgcn_exp2f(fmaf(dot, kC, pb2[j]) - c.dl2[jj].y);
        const float dS = P * (gd - c.dl2[jj].x);
        const float cds = kScale * dS;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          dk[2 * i] = fmaf(cds, bf16_lo(qw[i]), dk[2 * i]);
          dk[2 * i + 1] = fmaf(cds, bf16_hi(qw[i]), dk[2 * i + 1]);
          dv[2 * i] = fmaf(P, bf16_lo(dw[i]), dv[2 * i]);
          dv[2 * i + 1] = fmaf(P, bf16_hi(dw[i]), dv[2 * i + 1]);
        }
        // keep the accumulation here: sunk to the loop latch it holds every
        // chunk's q/dO registers live and the prefetch turns into register copies
        pin_regs<16>(dk);
        pin_regs<16>(dv);
        if (far) {
          // dV gets R^T dO on the rotated pair; dZ gets d(theta) * gain * y
          dv[SHIFT] = fmaf(P, (cs - 1.f) * da + sn * db, dv[SHIFT]);
          dv[SHIFT + 1] = fmaf(P, (cs - 1.f) * db - sn * da, dv[SHIFT + 1]);
          const float tq = P * (da * (-va * sn - vb * cs) + db * (va * cs - vb * sn));
          dz = fmaf(tq * pg, c.y[jj], dz);
        }
        pin_regs<1>(&dz);
      }
    };

    if (cnt > 0) {
      KvChunk<CJ> c0, c1;
      fetch(0, c0);
      for (int k0 = 0; k0 < cntp; k0 += 2 * CJ) {
        fetch(k0 + CJ, c1);
        consume(c0);
        fetch(k0 + 2 * CJ, c0);
        consume(c1);
      }
    }
    // ---- near band (offsets j < JB) on the matrix cores ----
    // Band lane (lc, lr) serves key m0w + lr; in the MFMA C layout it holds
    // queries m0w + 16 tb + 4 lc + r of the wave's query blocks tb = 0..2
    // (queries [m0w, m0w + 48)), and its dK / dV results dims 16 lc + [0, 16).
    //   S^T = Q K^T, dP^T = dO V^T, <q, e_slot> = Q E^T   (v_mfma_f32_16x16x32_bf16)
    //   P = exp2(S' - lse), dS = P (dP - delta) on the band's diagonals
    //   dK^T += Q^T (c dS^T), dV^T += dO^T P^T            (v_mfma_f32_16x16x16_bf16, bf16 hi + lo)
    if (JB > 0) {   // uniform over the workgroup
      __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): this wave's window loads have landed
      __syncthreads();
      auto win16 = [&](char* wb, int row, int c) { return wb + row * 128 + 16 * (c ^ (row & 7)); };
      const bool key_band = m0w + lr < N;
      f32x4 acck[4], accv[4];
#pragma unroll
      for (int db = 0; db < 4; ++db) { acck[db] = zero4(); accv[db] = zero4(); }
#pragma unroll
      for (int tb = 0; tb < 3; ++tb) {
        const int wr = 16 * (w + tb) + lr;   // window row of query m0w + 16 tb + lr
        const uint4 qa0 = *reinterpret_cast<const uint4*>(win16(s_qw, wr, lc));
        const uint4 qa1 = *reinterpret_cast<const uint4*>(win16(s_qw, wr, 4 + lc));
        const uint4 da0 = *reinterpret_cast<const uint4*>(win16(s_dw, wr, lc));
        const uint4 da1 = *reinterpret_cast<const uint4*>(win16(s_dw, wr, 4 + lc));
        f32x4 S = mfma16_bf16(bf16x8_from_bits(qa0), bf16x8_from_bits(kB[0]), zero4());
        S = mfma16_bf16(bf16x8_from_bits(qa1), bf16x8_from_bits(kB[1]), S);
        f32x4 Dp = mfma16_bf16(bf16x8_from_bits(da0), bf16x8_from_bits(vB[0]), zero4());
        Dp = mfma16_bf16(bf16x8_from_bits(da1), bf16x8_from_bits(vB[1]), Dp);
        // <q, e_slot> of this block's queries: C[query 4 lc + r][slot 16 bb + lr]
        f32x4 qe[2];
#pragma unroll
        for (int bb = 0; bb < 2; ++bb) {
          qe[bb] = zero4();
          if (16 * bb < JB) {
            const uint4 e0 = *reinterpret_cast<const uint4*>(sE + (16 * bb + lr) * kERowKv + 8 * lc);
            const uint4 e1 = *reinterpret_cast<const uint4*>(sE + (16 * bb + lr) * kERowKv + 32 + 8 * lc);
            qe[bb] = mfma16_bf16(bf16x8_from_bits(qa0), bf16x8_from_bits(e0), qe[bb]);
            qe[bb] = mfma16_bf16(bf16x8_from_bits(qa1), bf16x8_from_bits(e1), qe[bb]);
          }
        }
        float pv[4], cds[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int qq = 16 * tb + 4 * lc + r;   // query m0w + qq, key m0w + lr
          const int delta = qq - lr;
          const int slot = delta >= 1 && delta <= kBandMaxKv ? s_jn[kJnBias + delta] : -1;
          // <q, e_slot> of this lane's query lives in lane (slot % 16, lc), register r of block slot / 16
          const int src = 4 * ((slot & 15) + 16 * lc);
          const float q0 = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(qe[0][r])));
          const float q1 = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(qe[1][r])));
          float p = 0.f, ds = 0.f;
          if (slot >= 0 && key_band && m0w + qq < N) {
            const float2 dl = s_dl[16 * (w + tb) + 4 * lc + r];
            const float qev = slot < 16 ? q0 : q1;
            p = __builtin_amdgcn_exp2f(fmaf(S[r] + qev, kC, pb2[slot]) - dl.y);
            ds = p * (Dp[r] - dl.x);
          }
          pv[r] = p;
          cds[r] = kScale * ds;
        }
        float cl[4], pl[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          cl[r] = cds[r] - round_bf16(cds[r]);
          pl[r] = pv[r] - round_bf16(pv[r]);
        }
        const i16x4 dsh = __builtin_bit_cast(i16x4, make_uint2(pack_bf16x2(cds[0], cds[1]), pack_bf16x2(cds[2], cds[3])));
        const i16x4 dsl = __builtin_bit_cast(i16x4, make_uint2(pack_bf16x2(cl[0], cl[1]), pack_bf16x2(cl[2], cl[3])));
        const i16x4 ph = __builtin_bit_cast(i16x4, make_uint2(pack_bf16x2(pv[0], pv[1]), pack_bf16x2(pv[2], pv[3])));
        const i16x4 plo = __builtin_bit_cast(i16x4, make_uint2(pack_bf16x2(pl[0], pl[1]), pack_bf16x2(pl[2], pl[3])));
        // Q^T and dO^T read transposed from the windows: rows 16 (w + tb) + 4 lc + e, dims
        // 16 (lr / 4) + 4 db + lr % 4 of MFMA row lr
        const int R = 16 * (w + tb) + 4 * lc + (lr >> 2);
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          const i16x4 aq = lds_read_tr16(win16(s_qw, R, 2 * (lr & 3) + (db >> 1)) + 8 * (db & 1));
          const i16x4 ad = lds_read_tr16(win16(s_dw, R, 2 * (lr & 3) + (db >> 1)) + 8 * (db & 1));
          acck[db] = mfma16k16_bf16(aq, dsh, acck[db]);
          acck[db] = mfma16k16_bf16(aq, dsl, acck[db]);
          accv[db] = mfma16k16_bf16(ad, ph, accv[db]);
          accv[db] = mfma16k16_bf16(ad, plo, accv[db]);
        }
      }
      // into the gather layout: key ki, dims 16 g + i <- band lane (lc = g, lr = ki)
      const int srck = 4 * (ki + 16 * g);
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          dk[4 * db + r] += __int_as_float(__builtin_amdgcn_ds_bpermute(srck, __float_as_int(acck[db][r])));
          dv[4 * db + r] += __int_as_float(__builtin_amdgcn_ds_bpermute(srck, __float_as_int(accv[db][r])));
        }
    }

  }

  if (part) {   // a subset of the query heads: its partial sums, which dsqg_bwd_dkdv_combine adds up
    if (!key_ok) return;
    // rows of the split units, kKPB per unit: [split][unit - whole][key in tile]
    const int64_t rows = static_cast<int64_t>(total - whole) / nsplit * kKPB;
    const int64_t row = static_cast<int64_t>(unit - whole) * kKPB + (m - tile * kKPB);
    float4* pk = reinterpret_cast<float4*>(kvp + (split * rows + row) * kHeadDim + 16 * g);
    float4* pv = reinterpret_cast<float4*>(kvp + ((nsplit + split) * rows + row) * kHeadDim + 16 * g);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pk[i] = make_float4(dk[4 * i], dk[4 * i + 1], dk[4 * i + 2], dk[4 * i + 3]);
      pv[i] = make_float4(dv[4 * i], dv[4 * i + 1], dv[4 * i + 2], dv[4 * i + 3]);
    }
    kvp[2 * nsplit * rows * kHeadDim + (split * rows + row) * kPlanes + g] = dz;
    return;
  }
  // with key_probes z came from the key probes: dz goes into dk through the probe features (the
  // block's einsum backward, dsqg:3231-3254) instead of out to dz_pre
  if (f.key_probes) fold_probe_grad(dk, k32, f.key_probes, g, zg, dz);
  if (!key_ok) return;
  uint4* k4 = reinterpret_cast<uint4*>(reinterpret_cast<bf16*>(a.dk) + b * a.dk_stride[0] + hk * a.dk_stride[1] +
                                       mm * a.dk_stride[2] + 16 * g);
  uint4* v4 = reinterpret_cast<uint4*>(reinterpret_cast<bf16*>(a.dv) + b * a.dv_stride[0] + hk * a.dv_stride[1] +
                                       mm * a.dv_stride[2] + 16 * g);
  uint4 x;
  x.x = pack_bf16x2(dk[0], dk[1]);   x.y = pack_bf16x2(dk[2], dk[3]);
  x.z = pack_bf16x2(dk[4], dk[5]);   x.w = pack_bf16x2(dk[6], dk[7]);
  k4[0] = x;
  x.x = pack_bf16x2(dk[8], dk[9]);   x.y = pack_bf16x2(dk[10], dk[11]);
  x.z = pack_bf16x2(dk[12], dk[13]); x.w = pack_bf16x2(dk[14], dk[15]);
  k4[1] = x;
  x.x = pack_bf16x2(dv[0], dv[1]);   x.y = pack_bf16x2(dv[2], dv[3]);
  x.z = pack_bf16x2(dv[4], dv[5]);   x.w = pack_bf16x2(dv[6], dv[7]);
  v4[0] = x;
  x.x = pack_bf16x2(dv[8], dv[9]);   x.y = pack_bf16x2(dv[10], dv[11]);
  x.z = pack_bf16x2(dv[12], dv[13]); x.w = pack_bf16x2(dv[14], dv[15]);
  v4[1] = x;
  if (!f.key_probes) a.dz_pre[(static_cast<int64_t>(bhk) * N + m) * kPlanes + g] = dz;
}

// Sums the query-head subsets' partial dK, dV and dZ of each key in subset order, folds dZ into dK
// through the key probes when z came from them, and writes the bf16 gradients. Four lanes per key,
// lane g holding dims 16g .. 16g + 15 and plane g, as in dsqg_bwd_dkdv_bf16_k4.
__global__ __launch_bounds__(kBlock) void dsqg_bwd_dkdv_combine(const dwarf_dsqg_bwd_args a,
                                                                const float* __restrict__ kvp, int tiles,
                                                                int whole, int split_units, int nsplit) {
  const dwarf_dsqg_fwd_args& f = a.fwd;
  const int N = f.N;
  const int64_t rows = static_cast<int64_t>(split_units) * kKPB;   // the split units' key rows
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  const int64_t row = t >> 2;
  const int g = static_cast<int>(t & 3);
  if (row >= rows) return;   // rows * 4 threads: a key's four lanes leave together
  const int unit = whole + static_cast<int>(row / kKPB);
  const int bhk = unit / tiles, tile = unit - bhk * tiles;
  const int64_t mm = static_cast<int64_t>(tile) * kKPB + (row - static_cast<int64_t>(unit - whole) * kKPB);
  if (mm >= N) return;   // past the end of the last tile: a key's four lanes leave together
  const int b = bhk / f.H_kv, hk = bhk - b * f.H_kv;
  float dk[16], dv[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) { dk[i] = 0.f; dv[i] = 0.f; }
  float dz = 0.f;
  for (int s = 0; s < nsplit; ++s) {
    const float4* pk = reinterpret_cast<const float4*>(kvp + (s * rows + row) * kHeadDim + 16 * g);
    const float4* pv = reinterpret_cast<const float4*>(kvp + ((nsplit + s) * rows + row) * kHeadDim + 16 * g);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 x = pk[i], y = pv[i];
      dk[4 * i] += x.x; dk[4 * i + 1] += x.y; dk[4 * i + 2] += x.z; dk[4 * i + 3] += x.w;
      dv[4 * i] += y.x; dv[4 * i + 1] += y.y; dv[4 * i + 2] += y.z; dv[4 * i + 3] += y.w;
    }
    dz += kvp[2 * nsplit * rows * kHeadDim + (s * rows + row) * kPlanes + g];
  }
  if (f.key_probes) {
    const bf16* kb = reinterpret_cast<const bf16*>(f.k) + b * f.k_stride[0] + hk * f.k_stride[1];
    const uint4* k4 = reinterpret_cast<const uint4*>(kb + mm * f.k_stride[2] + 16 * g);
    const uint4 kx0 = k4[0], kx1 = k4[1];
    const uint32_t k32[8] = {kx0.x, kx0.y, kx0.z, kx0.w, kx1.x, kx1.y, kx1.z, kx1.w};
    const float zg = f.z_pre[b * f.z_stride[0] + hk * f.z_stride[1] + mm * f.z_stride[2] + g];
    fold_probe_grad(dk, k32, f.key_probes, g, zg, dz);
  }
  uint4* k4 = reinterpret_cast<uint4*>(reinterpret_cast<bf16*>(a.dk) + b * a.dk_stride[0] + hk * a.dk_stride[1] +
                                       mm * a.dk_stride[2] + 16 * g);
  uint4* v4 = reinterpret_cast<uint4*>(reinterpret_cast<bf16*>(a.dv) + b * a.dv_stride[0] + hk * a.dv_stride[1] +
                                       mm * a.dv_stride[2] + 16 * g);
  uint4 x;
  x.x = pack_bf16x2(dk[0], dk[1]);   x.y = pack_bf16x2(dk[2], dk[3]);
  x.z = pack_bf16x2(dk[4], dk[5]);   x.w = pack_bf16x2(dk[6], dk[7]);
  k4[0] = x;
  x.x = pack_bf16x2(dk[8], dk[9]);   x.y = pack_bf16x2(dk[10], dk[11]);
  x.z = pack_bf16x2(dk[12], dk[13]); x.w = pack_bf16x2(dk[14], dk[15]);
  k4[1] = x;
  x.x = pack_bf16x2(dv[0], dv[1]);   x.y = pack_bf16x2(dv[2], dv[3]);
  x.z = pack_bf16x2(dv[4], dv[5]);   x.w = pack_bf16x2(dv[6], dv[7]);
  v4[0] = x;
  x.x = pack_bf16x2(dv[8], dv[9]);   x.y = pack_bf16x2(dv[10], dv[11]);
  x.z = pack_bf16x2(dv[12], dv[13]); x.w = pack_bf16x2(dv[14], dv[15]);
  v4[1] = x;
  if (!f.key_probes) a.dz_pre[(static_cast<int64_t>(bhk) * N + mm) * kPlanes + g] = dz;
}

// Grouped-query heads: a KV head's workgroups walk all of its query heads, so the grid has 1 / group
// of the MHA grid's workgroups, each group-times as long.  Units (key tile, KV head) past what the
// resident slots (256 CUs x kMinWgKv) take in a whole round are split into subsets of the query heads,
// one workgroup per subset, the smallest divisor of the group size whose subsets fill a round (two rounds
// for a grid that fills none): the last round then runs shorter workgroups instead of a few whole-group
// ones alone on the chip.  The subsets' fp32 partials are summed by dsqg_bwd_dkdv_combine.  A grid of
// two or more rounds keeps whole groups.
constexpr int kKvResidentWgs = 256 * kMinWgKv;

KvSplit dkdv_split(const dwarf_dsqg_fwd_args& f) {
  const int group = f.H_kv > 0 ? f.H / f.H_kv : 1;
  const int64_t units = static_cast<int64_t>((f.N + kKPB - 1) / kKPB) * f.B * f.H_kv;
  KvSplit k{static_cast<int>(units), 1};
  if (group == 1 || units >= 2 * kKvResidentWgs) return k;
  int64_t target = kKvResidentWgs;
  if (units < kKvResidentWgs) {
    k.whole = 0;
    target = 2 * kKvResidentWgs;
  } else {
    k.whole = kKvResidentWgs;
  }
  const int64_t rest = units - k.whole;
  int s = 1;
  while (s < group && rest * s < target) {
    do ++s; while (group % s);
  }
  k.nsplit = s;
  if (s == 1) k.whole = static_cast<int>(units);
  return k;
}

hipError_t launch_dkdv_bf16_k4(const dwarf_dsqg_bwd_args& a, const BwdWorkspace& ws, hipStream_t stream) {
  const dwarf_dsqg_fwd_args& f = a.fwd;
  const float* delta = reinterpret_cast<const float*>(static_cast<char*>(a.workspace) + ws.delta_off);
  const int tiles = (f.N + kKPB - 1) / kKPB;
  const int units = tiles * f.B * f.H_kv;
  const int ns = ws.kv_split, whole = ws.kv_whole;
  float* kvp = ns > 1 ? reinterpret_cast<float*>(static_cast<char*>(a.workspace) + ws.kv_part_off) : nullptr;
  const int total = whole + (units - whole) * ns;
  if (total == 0) return hipSuccess;
  const size_t lds = kv_layout(f.J, f.J_large, f.H / f.H_kv, kChunkKv).bytes;
#define DWARF_KV4_CASE(S) \
  case S:                                                                                                     \
    hipLaunchKernelGGL((dsqg_bwd_dkdv_bf16_k4<S, kChunkKv, kMinWgKv>), dim3(total), dim3(kBlock), lds, stream, a, \
                       delta, tiles, total, whole, ns, kvp);                                                  \
    break;
  switch (f.plane_shift) {
    DWARF_KV4_CASE(0) DWARF_KV4_CASE(1) DWARF_KV4_CASE(2) DWARF_KV4_CASE(3) DWARF_KV4_CASE(4)
    DWARF_KV4_CASE(5) DWARF_KV4_CASE(6) DWARF_KV4_CASE(7) DWARF_KV4_CASE(8) DWARF_KV4_CASE(9)
    DWARF_KV4_CASE(10) DWARF_KV4_CASE(11) DWARF_KV4_CASE(12) DWARF_KV4_CASE(13) DWARF_KV4_CASE(14)
    default: return hipErrorInvalidValue;
  }
#undef DWARF_KV4_CASE
  if (ns > 1) {
    const int64_t threads = static_cast<int64_t>(units - whole) * kKPB * kPlanes;
    hipLaunchKernelGGL(dsqg_bwd_dkdv_combine, dim3(static_cast<unsigned>((threads + kBlock - 1) / kBlock)),
                       dim3(kBlock), 0, stream, a, kvp, tiles, whole, units - whole, ns);
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Fixed-order reduction of the parameter-gradient partials.
// ---------------------------------------------------------------------------
constexpr int kRedRows = 64;  // rows summed per stage-1 group (16 rows: the step 3-4 us longer at B15 H8 T2048)

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
  // the loads are independent; the adds keep row order
#pragma unroll 16
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
#pragma unroll 8
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
  RedPlan p;
  p.arr[0] = {reinterpret_cast<const float*>(base + ws.part_se_off), red, 1, ws.dq_wgs, f.J * kHeadDim,
              ws.red_groups_se};
  red += static_cast<size_t>(ws.red_groups_se) * f.J * kHeadDim;
  p.arr[1] = {reinterpret_cast<const float*>(base + ws.part_pb_off), red, f.H, ws.pb_rows, f.J, ws.red_groups_pb};
  red += static_cast<size_t>(f.H) * ws.red_groups_pb * f.J;
  p.arr[2] = {reinterpret_cast<const float*>(base + ws.part_ph_off), red, f.H, ws.ph_rows, f.J_large * 8,
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
  const int kTile = dq_tile_queries(f.dtype);
  w.dq_tiles = (f.N + kTile - 1) / kTile;
  const int total_tiles = w.dq_tiles * f.B * f.H;
  const int JL = f.J_large > 0 ? f.J_large : 1;
  if (f.dtype == DWARF_BF16) {
    // Persistent workgroups, all resident: the gather launch (dQ, dY, dS,
    // dPhase partials per tile) and the dSE launch, whose workgroups
    // accumulate dSE in their own slots (dPB partials per tile).
    w.dq_tpw = 0;
    w.dq_ntg = 0;
    // beside a concurrent dK/dV launch (the delta stage) the dQ launch takes 400 workgroups (50 per XCD,
    // about three per two CUs) and leaves the rest to dK/dV, so that the two streams end together: at
    // B15 H8 T2048 the step measured 0.550-0.552 ms with 400 workgroups, 0.556 with 384 and 0.572 with 512
    // (352: 0.578, 416: 0.557-0.561, 448: 0.565, 256: 0.626); at B4 H8 T8192 0.871-0.873 with 384 or 400
    // against 0.880
    const int gather_max = (f.schedule & DWARF_SCHED_DELTA_STAGE) ? 400 : 256 * dq_gather_wgs_per_cu();
    w.dq_gather_wgs = total_tiles < gather_max ? total_tiles : gather_max;
    const int dse_max = 256 * dq_dse_wgs_per_cu(f.J);
    w.dq_wgs = total_tiles < dse_max ? (total_tiles > 0 ? total_tiles : 1) : dse_max;
    w.pb_rows = f.B * w.dq_tiles;
    w.ph_rows = f.B * w.dq_tiles;
  } else {
    // Two 4-wave workgroups fit per CU: size the tile groups so every
    // workgroup is resident at once (at most 512 on 256 CUs).
    w.dq_tpw = (total_tiles + 511) / 512;
    if (w.dq_tpw < 1) w.dq_tpw = 1;
    if (w.dq_tpw > 16) w.dq_tpw = 16;
    if (w.dq_tpw > w.dq_tiles) w.dq_tpw = w.dq_tiles > 0 ? w.dq_tiles : 1;
    w.dq_ntg = (w.dq_tiles + w.dq_tpw - 1) / w.dq_tpw;
    w.dq_wgs = f.B * f.H * w.dq_ntg;
    w.pb_rows = f.B * w.dq_ntg;
    w.ph_rows = 4 * f.B * w.dq_ntg;   // one row per wave
  }
  w.red_groups_se = (w.dq_wgs + kRedRows - 1) / kRedRows;
  w.red_groups_pb = (w.pb_rows + kRedRows - 1) / kRedRows;
  w.red_groups_ph = (w.ph_rows + kRedRows - 1) / kRedRows;
  size_t off = 0;
  w.delta_off = off;   // bf16: (delta, log2 lse) pairs; fp32: delta
  w.delta_bytes = static_cast<size_t>(f.B) * f.H * f.N * 2 * sizeof(float);
  off += align256(w.delta_bytes);
  w.part_se_off = off;
  w.part_se_bytes = static_cast<size_t>(w.dq_wgs) * f.J * kHeadDim * sizeof(float);
  off += align256(w.part_se_bytes);
  w.part_pb_off = off;
  w.part_pb_bytes = static_cast<size_t>(f.H) * w.pb_rows * f.J * sizeof(float);
  off += align256(w.part_pb_bytes);
  w.part_ph_off = off;
  w.part_ph_bytes = static_cast<size_t>(f.H) * w.ph_rows * JL * 8 * sizeof(float);
  off += align256(w.part_ph_bytes);
  w.ds_off = off;
  w.ds_bytes = f.dtype == DWARF_BF16 ? static_cast<size_t>(f.B) * f.H * f.J * f.N * sizeof(float) : 0;
  off += align256(w.ds_bytes);
  w.red_off = off;
  w.red_bytes = (static_cast<size_t>(w.red_groups_se) * f.J * kHeadDim +
                 static_cast<size_t>(f.H) * w.red_groups_pb * f.J +
                 static_cast<size_t>(f.H) * w.red_groups_ph * JL * 8) * sizeof(float);
  off += align256(w.red_bytes);
  const int kv_units = (f.N + kKPB - 1) / kKPB * f.B * f.H_kv;
  const KvSplit ks = f.dtype == DWARF_BF16 ? dkdv_split(f) : KvSplit{kv_units, 1};
  w.kv_split = ks.nsplit;
  w.kv_whole = ks.whole;
  w.kv_part_off = off;
  w.kv_part_bytes = ks.nsplit > 1 ? static_cast<size_t>(ks.nsplit) * (kv_units - ks.whole) * kKPB *
                                        (2 * kHeadDim + kPlanes) * sizeof(float)
                                  : 0;
  off += align256(w.kv_part_bytes);
  w.total = off;
  return w;
}

size_t dkdv_lds_bytes(int J, int J_large, int group) { return kv_layout(J, J_large, group, kChunkKv).bytes; }

hipError_t launch_dsqg_bwd(const dwarf_dsqg_bwd_args& a, const BwdWorkspace& ws, hipStream_t stream, bool do_dq,
                           bool do_params, bool do_dkdv) {
  // all stages on one stream with the delta stage requested: the dQ launch then
  // skips the (delta, lse) pairs, so the delta launch writes them first
  if (do_dq && do_dkdv && a.fwd.dtype == DWARF_BF16 && (a.fwd.schedule & DWARF_SCHED_DELTA_STAGE)) {
    const hipError_t e = launch_dsqg_bwd_delta(a, ws, stream);
    if (e != hipSuccess) return e;
  }
  if (do_dq) {
    const hipError_t e = launch_dsqg_bwd_dq(a, ws, stream);
    if (e != hipSuccess) return e;
  }
  if (do_params) {
    hipError_t e = launch_dsqg_bwd_dse(a, ws, stream);
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
    if (a.fwd.dtype == DWARF_BF16) return launch_dkdv_bf16_k4(a, ws, stream);
    return launch_dkdv_typed<float, kLanesBwd, false>(a, ws, stream);
  }
  return hipSuccess;
}

}  // namespace dwarf
