// DSQG forward: one pass over the offset lattice per query with an fp32
// online softmax (reference kernel _fwd_v22_online, dsqg:698-860).
//
// Work mapping: a workgroup of 256 lanes owns 256/L consecutive queries of
// one (b, h); L lanes share a query and each holds 64/L head dimensions.
// For every offset the lane gathers its slice of the K and V source rows
// s = n - delta, so one wave reads 64/L consecutive K rows per offset.
// Offsets whose source lies before position 0 for the whole wave are skipped
// with a wave-uniform branch (about half of the lattice at T = 2048).
//
// The softmax keeps a running reference m that is only raised when a score
// exceeds it by more than kRescaleSlack (natural-log units).  Weights
// exp(s - m) then stay below e^kRescaleSlack, the rescale of the accumulator
// is skipped on almost every offset, and out = acc / l, lse = m + log(l) are
// unchanged mathematically.
#include "common.h"
#include "dsqg_internal.h"
#include "mfma.h"
#include "gather.h"

namespace dwarf {
namespace {

constexpr float kRescaleSlack = 8.0f;

template <typename T, int SHIFT, int L, bool FAST, bool TWO_PASS>
__global__ __launch_bounds__(kBlock) void dsqg_fwd_kernel(const dwarf_dsqg_fwd_args a, int tiles, int total) {
  constexpr int HD = kHeadDim;
  constexpr int DPL = HD / L;     // head dims held by one lane
  constexpr int QPB = kBlock / L; // queries per workgroup
  constexpr int SEG = HD / kPlanes;

  extern __shared__ float smem[];
  float* s_se = smem;                    // [J][64], bf16-rounded when asked
  float* s_pb = smem + a.J * HD;         // [J] pos_bias for this head
  int* s_off = reinterpret_cast<int*>(s_pb + a.J);  // [J]

  const int work = xcd_remap(blockIdx.x, total);
  const int bh = work / tiles;
  const int tile = work - bh * tiles;
  const int b = bh / a.H;
  const int h = bh - b * a.H;
  const int hk = h / (a.H / a.H_kv);

  for (int i = threadIdx.x; i < a.J * HD; i += kBlock) {
    const int j = i / HD, d = i - j * HD;
    float e = a.scale_embed[j * a.se_stride[0] + d * a.se_stride[1]];
    s_se[i] = a.se_round_bf16 ? round_bf16(e) : e;
  }
  for (int j = threadIdx.x; j < a.J; j += kBlock) {
    s_pb[j] = a.pos_bias[j * a.pb_stride[0] + h * a.pb_stride[1]];
    s_off[j] = a.offsets[j];
  }
  __syncthreads();

  const int lane = threadIdx.x;
  const int g = lane % L;                   // slice of the head dims
  const int n = tile * QPB + lane / L;      // query position
  const int wave_n_last = uniform(tile * QPB + (lane / kWave) * (kWave / L)) + kWave / L - 1;
  if (n >= a.N) return;

  T* orow = reinterpret_cast<T*>(a.out) + b * a.out_stride[0] + h * a.out_stride[1] +
            static_cast<int64_t>(n) * a.out_stride[2] + g * DPL;
  float* lse_p = a.lse + b * a.lse_stride[0] + h * a.lse_stride[1] + static_cast<int64_t>(n) * a.lse_stride[2];

  float acc[DPL];
#pragma unroll
  for (int d = 0; d < DPL; ++d) acc[d] = 0.f;
  float m = -INFINITY, l = 0.f;

  if (n >= a.query_start) {
    float q[DPL];
    load_f32<T, DPL>(reinterpret_cast<const T*>(a.q) + b * a.q_stride[0] + h * a.q_stride[1] +
                         static_cast<int64_t>(n) * a.q_stride[2] + g * DPL,
                     q);
    const float4 yq = *reinterpret_cast<const float4*>(a.y_pre + b * a.y_stride[0] + h * a.y_stride[1] +
                                                        static_cast<int64_t>(n) * a.y_stride[2]);
    const float ys[4] = {yq.x, yq.y, yq.z, yq.w};
    const T* kbase = reinterpret_cast<const T*>(a.k) + b * a.k_stride[0] + hk * a.k_stride[1] + g * DPL;
    const T* vbase = reinterpret_cast<const T*>(a.v) + b * a.v_stride[0] + hk * a.v_stride[1] + g * DPL;
    const float* zbase = a.z_pre + b * a.z_stride[0] + hk * a.z_stride[1];
    const float scale = 0.125f;  // 1/sqrt(64)

    if constexpr (TWO_PASS) {
      // offline softmax (dsqg:863-1044): the row maximum first, so the weighted sum never rescales
      for (int j = 0; j < a.J; ++j) {
        const int delta = s_off[j];
        if (wave_n_last < delta) continue;
        const int s = n - delta;
        if (s < 0 || s >= a.N) continue;
        float kv[DPL];
        load_f32<T, DPL>(kbase + static_cast<int64_t>(s) * a.k_stride[2], kv);
        const float* e = s_se + j * HD + g * DPL;
        float dot = 0.f;
#pragma unroll
        for (int d = 0; d < DPL; ++d) dot = fmaf(q[d], kv[d] + e[d], dot);
        dot = group_sum<L>(dot);
        const float score = fmaf(dot, scale, s_pb[j]);
        if (score > m) m = score;
      }
    }

    for (int j = 0; j < a.J; ++j) {
      const int delta = s_off[j];
      if (wave_n_last < delta) continue;  // no lane of this wave has a source
      const int s = n - delta;
      if (s < 0 || s >= a.N) continue;

      float kv[DPL];
      load_f32<T, DPL>(kbase + static_cast<int64_t>(s) * a.k_stride[2], kv);
      const float* e = s_se + j * HD + g * DPL;
      float dot = 0.f;
#pragma unroll
      for (int d = 0; d < DPL; ++d) dot = fmaf(q[d], kv[d] + e[d], dot);
      dot = group_sum<L>(dot);
      const float score = fmaf(dot, scale, s_pb[j]);

      load_f32<T, DPL>(vbase + static_cast<int64_t>(s) * a.v_stride[2], kv);
      if (j >= a.J_small) {
        const int i = j - a.J_small;
        const float4 zk = *reinterpret_cast<const float4*>(zbase + static_cast<int64_t>(s) * a.z_stride[2]);
        const float zs[4] = {zk.x, zk.y, zk.z, zk.w};
#pragma unroll
        for (int r = 0; r < kPlanes; ++r) {
          const int ch = r * SEG + SHIFT;  // compile-time after unrolling
          if (ch / DPL != g) continue;     // plane held by another lane of the group
          const int la = ch % DPL;
          const float theta = a.phase_base[i * a.pbase_stride[0] + h * a.pbase_stride[1] + r] +
                              a.phase_gain[i * a.pgain_stride[0] + h * a.pgain_stride[1] + r] * ys[r] * zs[r];
          float sn, cs;
          dsincos<FAST>(theta, &sn, &cs);
          const float va = kv[la], vb = kv[la + 1];
          kv[la] = cs * va - sn * vb;
          kv[la + 1] = sn * va + cs * vb;
        }
      }

      if (!TWO_PASS && score > m + kRescaleSlack) {
        const float c = dexp<FAST>(m - score);  // 0 on the first valid offset
#pragma unroll
        for (int d = 0; d < DPL; ++d) acc[d] *= c;
        l *= c;
        m = score;
      }
      const float p = dexp<FAST>(score - m);
      l += p;
#pragma unroll
      for (int d = 0; d < DPL; ++d) acc[d] = fmaf(p, kv[d], acc[d]);
    }
  }

  const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
  for (int d = 0; d < DPL; ++d) acc[d] *= inv;
  store_from_f32<T, DPL>(orow, acc);
  if (g == 0) *lse_p = l > 0.f ? m + dlog<FAST>(l) : -INFINITY;
}

// ---------------------------------------------------------------------------
// bf16 forward, four lanes per query.
//
// Lane g of a query holds head dims [16g, 16g+16): its slices of q, of the
// accumulator and of every gathered K/V row (two 16-byte loads each), so one
// wave load instruction covers 64 contiguous bytes of 16 consecutive source
// rows.
//
// Each wave first lists the offsets that give at least one of its 16 queries
// a source row (s_list, padded with a sentinel whose rows are out of range),
// then walks that list in chunks of CJ with the next chunk's loads already in
// flight (two register buffers).  The gathers are raw buffer loads with
// 32-bit offsets: a lane without a source gets an offset past the end of the
// tensor and reads zeros, so the loop has no per-lane branches.
//
// <q, e_j> for the wave's 16 queries and all offsets is one
// v_mfma_f32_16x16x32_bf16 pass at the start, stored pre-scaled together
// with pos_bias (s_qe = log2(e) * (<q,e_j>/8 + pb_j)); the softmax runs in
// base 2.  <q, k> is v_dot2_f32_bf16 on the packed rows summed over the 4
// lanes with DPP.  P.V stays fp32 (widened bf16 rows times the fp32 weight),
// as the reference accumulates it (dsqg:993-1013).  With plane_shift <= 14
// the MOVT pair of plane r (dims 16r+shift, 16r+shift+1) lies in lane r's
// slice, so each lane rotates exactly one pair of every far V row.
// ---------------------------------------------------------------------------
constexpr int kLanesQ = 4;                  // lanes per query
constexpr int kQPW = kWave / kLanesQ;       // 16 queries per wave
constexpr int kQPB = kBlock / kLanesQ;      // 64 queries per workgroup
constexpr int kChunkFwd = 1;                // offsets per prefetch chunk (the launch's choice)
constexpr int kERowFwd = 72;                // bf16 E row stride (elements)
// LDS: s_pb[JE] f32, s_off[JE] i32, s_ph[JL4][4] float2, s_list[4][list_len] int2,
// then one region that first holds the bf16 E rows (sE[JE][72]) and, after a
// barrier, the four waves' s_qe[16][qe_row] tables.
struct FwdLayout {
  int JE, JL4, qe_row, list_len, max_blocks;
  size_t off_ph, off_list, off_big, bytes;
};

constexpr int kMaxQeBlocks = 17;   // JE / 16 for J <= kMaxOffsets (256) plus the sentinel

// JE >= J + 1 keeps a sentinel slot (index J) with an unreachable offset.
__host__ __device__ inline FwdLayout fwd_layout(int J, int J_large, int CJ) {
  FwdLayout L;
  L.JE = (J + 1 + 15) / 16 * 16;
  L.JL4 = (J_large + 1) / 2 * 2;                       // keeps the float2 table a multiple of 16 bytes
  L.qe_row = L.JE + 4;
  L.list_len = (L.JE + 4 * CJ + 1) / 2 * 2;            // list + padding for the prefetch overrun
  L.off_ph = static_cast<size_t>(2 * L.JE) * 4;
  L.off_list = L.off_ph + static_cast<size_t>(L.JL4) * 4 * 8;
  L.off_big = L.off_list + static_cast<size_t>(4 * L.list_len) * 8;
  const size_t e_bytes = static_cast<size_t>(L.JE) * kERowFwd * 2;
  const size_t qe_bytes = static_cast<size_t>(4 * kQPW * L.qe_row) * 4;
  L.bytes = L.off_big + (e_bytes > qe_bytes ? e_bytes : qe_bytes);
  return L;
}

template <int CJ>
struct FwdChunk {
  uint4 k[CJ][2], v[CJ][2];
  float z[CJ];
  bool ok[CJ];
  int j[CJ];
};

template <int SHIFT, int CJ, bool TWO_PASS>
__global__ __launch_bounds__(kBlock, 2) void dsqg_fwd_bf16_q4(const dwarf_dsqg_fwd_args a, int tiles, int total) {
  constexpr float kC = 0.125f * kLog2e;           // 1/sqrt(64) in base-2 score units
  constexpr float kSlack2 = 8.0f * kLog2e;        // kRescaleSlack in base 2
  static_assert(SHIFT + 1 < kHeadDim / kPlanes, "MOVT pair must stay inside one lane's slice");
  const int J = a.J, N = a.N, J_small = a.J_small;
  const FwdLayout lay = fwd_layout(J, a.J_large, CJ);
  extern __shared__ float smem[];
  char* sm = reinterpret_cast<char*>(smem);
  float* s_pb = smem;
  int* s_off = reinterpret_cast<int*>(smem + lay.JE);
  float2* s_ph = reinterpret_cast<float2*>(sm + lay.off_ph);
  int2* s_list_all = reinterpret_cast<int2*>(sm + lay.off_list);
  uint16_t* sE = reinterpret_cast<uint16_t*>(sm + lay.off_big);
  float* s_qe_all = reinterpret_cast<float*>(sm + lay.off_big);   // replaces sE after the second barrier

  const int work = xcd_remap(blockIdx.x, total);
  const int bh = work / tiles;
  // late query tiles (more valid offsets) of each (b, h) are dispatched first
  const int tile = tiles - 1 - (work - bh * tiles);
  const int b = bh / a.H;
  const int h = bh - b * a.H;
  const int hk = h / (a.H / a.H_kv);

  const int lane = threadIdx.x;
  const int w = lane / kWave;
  const int l = lane % kWave;
  const int g = l & 3;
  const int qi = l >> 2;
  const int lr = l & 15, lc = l >> 4;
  const int n0w = tile * kQPB + w * kQPW;
  const int n = n0w + qi;
  const int n_hi = min(n0w + kQPW - 1, N - 1);
  const bool row_ok = n < N;
  const bool live = row_ok && n >= a.query_start;
  const int64_t nn = n;
  float* s_qe = s_qe_all + w * kQPW * lay.qe_row;
  int2* s_list = s_list_all + w * lay.list_len;

  // The wave's q rows (MFMA operand layout and this lane's slice) and y are
  // requested first, so their latency overlaps the table staging.
  const bf16* qbase = reinterpret_cast<const bf16*>(a.q) + b * a.q_stride[0] + h * a.q_stride[1];
  uint4 xa[2] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
  if (n0w + lr < N) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      xa[ks] = *reinterpret_cast<const uint4*>(qbase + static_cast<int64_t>(n0w + lr) * a.q_stride[2] + 32 * ks + 8 * lc);
  }
  // with query_probes y is formed below from the q row (every row < N) and written to y_out
  const bool probed = a.query_probes != nullptr;
  uint4 qx0 = {0u, 0u, 0u, 0u}, qx1 = {0u, 0u, 0u, 0u};
  float yg = 0.f;
  if (probed ? row_ok : live) {
    const uint4* q4 = reinterpret_cast<const uint4*>(qbase + nn * a.q_stride[2] + 16 * g);
    qx0 = q4[0];
    qx1 = q4[1];
    if (!probed) yg = a.y_pre[b * a.y_stride[0] + h * a.y_stride[1] + nn * a.y_stride[2] + g];
  }

  stage_tables<true, true, true, true, false>(
      a, lay.JE, h, 1, TableStage{sE, kERowFwd, s_pb, 1.0f, s_off, s_ph, 0, nullptr, 0, 0, false});
  __syncthreads();

  // s_qe[query][j] = log2(e) * (<q, e_j> / 8 + pb_j) for the wave's 16 queries:
  // products into registers, a barrier (every wave is done reading sE), then
  // the tables are written over sE.
  {
    f32x4 c[kMaxQeBlocks];
#pragma unroll
    for (int bi = 0; bi < kMaxQeBlocks; ++bi) {
      c[bi] = zero4();
      if (bi * 16 < lay.JE) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const uint4 xb = *reinterpret_cast<const uint4*>(sE + (bi * 16 + lr) * kERowFwd + 32 * ks + 8 * lc);
          c[bi] = mfma16_bf16(bf16x8_from_bits(xa[ks]), bf16x8_from_bits(xb), c[bi]);
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int bi = 0; bi < kMaxQeBlocks; ++bi) {
      if (bi * 16 < lay.JE) {
        const float pb8 = 8.0f * s_pb[bi * 16 + lr];
#pragma unroll
        for (int r = 0; r < 4; ++r) s_qe[(4 * lc + r) * lay.qe_row + bi * 16 + lr] = (c[bi][r] + pb8) * kC;
      }
    }
  }
  if (n0w >= N) return;                       // whole wave past the end (no block barriers below)
  // The wave's offset list: offsets giving some query n0w..n_hi a source row in [0, N).
  // The sentinel (index J) gets the offset n0w - N, out of range for every query.
  const int cnt = build_offset_list<CJ>(s_list, s_off, J, n0w, n_hi, N, 1, make_int2(J, n0w - N));
  const int cntp = (cnt + CJ - 1) / CJ * CJ;

  const uint32_t q32[8] = {qx0.x, qx0.y, qx0.z, qx0.w, qx1.x, qx1.y, qx1.z, qx1.w};
  if (probed) {   // y of plane g (dsqg:3231-3254); the four lanes of each query take part
    yg = probe_feature(q32, a.query_probes, g);
    if (row_ok) a.y_out[(static_cast<int64_t>(b * a.H + h) * N + n) * kPlanes + g] = yg;
  }
  // Per-lane byte offsets of row 0 shifted by the lane's query; a lane without
  // a live query uses n_eff = n0w - 2N, so n_eff - d < 0 for every listed d.
  const int n_eff = live ? n : n0w - 2 * N;
  const int ks_b = static_cast<int>(a.k_stride[2]) * 2, vs_b = static_cast<int>(a.v_stride[2]) * 2;
  const int zs_b = static_cast<int>(a.z_stride[2]) * 4;
  const __amdgpu_buffer_rsrc_t rk =
      rows_rsrc(reinterpret_cast<const bf16*>(a.k) + b * a.k_stride[0] + hk * a.k_stride[1], ks_b, N, 128);
  const __amdgpu_buffer_rsrc_t rv =
      rows_rsrc(reinterpret_cast<const bf16*>(a.v) + b * a.v_stride[0] + hk * a.v_stride[1], vs_b, N, 128);
  const __amdgpu_buffer_rsrc_t rz = rows_rsrc(a.z_pre + b * a.z_stride[0] + hk * a.z_stride[1], zs_b, N, 16);
  const int kb_lane = n_eff * ks_b + 32 * g;
  const int vb_lane = n_eff * vs_b + 32 * g;
  const int zb_lane = n_eff * zs_b + 4 * g;

  float acc[16];
#pragma unroll
  for (int d = 0; d < 16; ++d) acc[d] = 0.f;
  float m = -3.0e38f, lsum = 0.f;

  auto fetch = [&](int k0, FwdChunk<CJ>& c) {
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
      c.z[jj] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rz, zo, 0, 0));
    }
  };

  auto consume = [&](const FwdChunk<CJ>& c) {
    float sc[CJ];
    float cmax = -INFINITY;
#pragma unroll
    for (int jj = 0; jj < CJ; ++jj) {
      const uint32_t* kw = reinterpret_cast<const uint32_t*>(&c.k[jj][0]);
      float dot = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) dot = dot2bf(q32[i], kw[i], dot);
      dot = group_sum<4>(dot);
      const float s2 = fmaf(dot, kC, s_qe[qi * lay.qe_row + c.j[jj]]);
      sc[jj] = c.ok[jj] ? s2 : -INFINITY;
      cmax = fmaxf(cmax, sc[jj]);
    }
    if (!TWO_PASS && cmax > m + kSlack2) {
      const float f = __builtin_amdgcn_exp2f(m - cmax);   // 0 on the first valid chunk
#pragma unroll
      for (int d = 0; d < 16; ++d) acc[d] *= f;
      lsum *= f;
      m = cmax;
    }
#pragma unroll
    for (int jj = 0; jj < CJ; ++jj) {
      const float p = __builtin_amdgcn_exp2f(sc[jj] - m);  // m is finite: 0 without a source
      lsum += p;
      const uint32_t* vw = reinterpret_cast<const uint32_t*>(&c.v[jj][0]);
      float vf[16];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        vf[2 * i] = bf16_lo(vw[i]);
        vf[2 * i + 1] = bf16_hi(vw[i]);
      }
      const int j = c.j[jj];
      if (j >= J_small && j < J) {
        const float2 ph = s_ph[(j - J_small) * kPlanes + g];
        float sn, cs;
        dsincos<true>(fmaf(ph.y * yg, c.z[jj], ph.x), &sn, &cs);
        const float va = vf[SHIFT], vb = vf[SHIFT + 1];
        vf[SHIFT] = cs * va - sn * vb;
        vf[SHIFT + 1] = sn * va + cs * vb;
      }
#pragma unroll
      for (int d = 0; d < 16; ++d) acc[d] = fmaf(p, vf[d], acc[d]);
    }
  };

  if (TWO_PASS && cnt > 0) {
    // offline softmax (dsqg:863-1044): each row's score maximum over the list first, so the
    // weighted sum below never rescales (m stays the maximum; -3e38 for a row without sources)
    float mx = -3.0e38f;
    for (int k0 = 0; k0 < cnt; ++k0) {
      const int2 e = s_list[k0];
      const int j = uniform(e.x), d = uniform(e.y);
      const uint32_t ko = static_cast<uint32_t>(kb_lane - d * ks_b);
      const uint4 k0v = buf_load16(rk, ko), k1v = buf_load16(rk, ko + 16);
      const uint32_t kw[8] = {k0v.x, k0v.y, k0v.z, k0v.w, k1v.x, k1v.y, k1v.z, k1v.w};
      float dot = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) dot = dot2bf(q32[i], kw[i], dot);
      dot = group_sum<4>(dot);
      const float s2 = fmaf(dot, kC, s_qe[qi * lay.qe_row + j]);
      if (static_cast<uint32_t>(n_eff - d) < static_cast<uint32_t>(N)) mx = fmaxf(mx, s2);
    }
    m = mx;
  }
  if (cnt > 0) {
    FwdChunk<CJ> c0, c1;
    fetch(0, c0);
    for (int k0 = 0; k0 < cntp; k0 += 2 * CJ) {
      fetch(k0 + CJ, c1);        // past the list end this reads the sentinel: zeros
      consume(c0);
      fetch(k0 + 2 * CJ, c0);
      consume(c1);
    }
  }

  if (!row_ok) return;
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  uint4* o4 = reinterpret_cast<uint4*>(reinterpret_cast<bf16*>(a.out) + b * a.out_stride[0] + h * a.out_stride[1] +
                                       nn * a.out_stride[2] + 16 * g);
  uint4 x0, x1;
  x0.x = pack_bf16x2(acc[0] * inv, acc[1] * inv);
  x0.y = pack_bf16x2(acc[2] * inv, acc[3] * inv);
  x0.z = pack_bf16x2(acc[4] * inv, acc[5] * inv);
  x0.w = pack_bf16x2(acc[6] * inv, acc[7] * inv);
  x1.x = pack_bf16x2(acc[8] * inv, acc[9] * inv);
  x1.y = pack_bf16x2(acc[10] * inv, acc[11] * inv);
  x1.z = pack_bf16x2(acc[12] * inv, acc[13] * inv);
  x1.w = pack_bf16x2(acc[14] * inv, acc[15] * inv);
  o4[0] = x0;
  o4[1] = x1;
  if (g == 0)
    a.lse[b * a.lse_stride[0] + h * a.lse_stride[1] + nn * a.lse_stride[2]] =
        lsum > 0.f ? (m + __builtin_amdgcn_logf(lsum)) * kLn2 : -INFINITY;
}

// ---------------------------------------------------------------------------
// bf16 forward with the near band served from LDS (schedule DWARF_SCHED_BAND,
// online softmax).  Lane layout and per-pair arithmetic are those of
// dsqg_fwd_bf16_q4; the walk over the offsets is split in two:
//   1. the far walk: the wave's listed offsets j >= JB, gathered row by row
//      through buffer loads as in dsqg_fwd_bf16_q4;
//   2. the near walk: the leading offsets j < JB (ascending, each at most
//      kFwdWinBack; the reference's near loop, dsqg:752-810).  Their source
//      rows all lie in the tile's window of keys [n0 - kFwdWinBack, n0 + 64),
//      which is staged once per workgroup into LDS by DMA (K and V rows of
//      128 bytes, 16-byte chunks XOR-swizzled by row), and every near pair
//      reads its rows there.
// An LDS read of a row costs about 0.6 of a gather through the vector
// memory path, and a third of the valid pairs at T = 2048 are near pairs.
// One LDS region holds, in turn, the bf16 E rows (for the q.E MFMA), the far
// columns of the q.E table and the K/V window; the near columns have their
// own small table.  The walks keep one running maximum per query, so the
// softmax is the same online softmax over all offsets in another order.
// ---------------------------------------------------------------------------
constexpr int kFwdWinBack = 32;                    // largest near offset: the window's look-back
constexpr int kFwdWinRows = kQPB + kFwdWinBack;    // 96 keys in the window

struct FwdWinLayout {
  int JE, JL4, JBh, near_row, far_row, list_len;
  size_t off_ph, off_list, off_near, off_jn, off_big, bytes;
};

// Smallest row stride >= n words that is 4 mod 16: the 16 queries' entries of
// one column then fall in distinct LDS banks.
__host__ __device__ inline int pad_words_4mod16(int n) { return (n + 11) / 16 * 16 + 4; }

// JBh = min(J_small, kFwdWinBack) bounds the near band (the kernel counts JB <= JBh
// from the offsets); q.E columns j < JBh go to the near table [64][near_row], the
// others to the far table [64][far_row] at column j - JBh.
// LDS: s_pb[JE] f32, s_off[JE] i32, s_ph[JL4][4] float2, s_list[4][list_len] int2,
// s_near[64][near_row] f32, s_jn[kJnSize] (band slots of the deltas), then the shared region: sE[JE][72] bf16, later
// s_far[64][far_row] f32, later the window (K rows [96][128 B], V rows [96][128 B]).
__host__ __device__ inline FwdWinLayout fwd_win_layout(int J, int J_small, int J_large) {
  FwdWinLayout L;
  L.JE = (J + 1 + 15) / 16 * 16;
  L.JL4 = (J_large + 1) / 2 * 2;
  L.JBh = J_small < kFwdWinBack ? J_small : kFwdWinBack;
  L.near_row = pad_words_4mod16(L.JBh);
  L.far_row = pad_words_4mod16(L.JE - L.JBh);
  L.list_len = (L.JE + 4 + 1) / 2 * 2;   // list + padding for the prefetch overrun
  L.off_ph = static_cast<size_t>(2 * L.JE) * 4;
  L.off_list = L.off_ph + static_cast<size_t>(L.JL4) * 4 * 8;
  L.off_near = L.off_list + static_cast<size_t>(4 * L.list_len) * 8;
  L.off_jn = L.off_near + static_cast<size_t>(kQPB * L.near_row) * 4;
  L.off_big = L.off_jn + kJnSize * 4;
  const size_t e_bytes = static_cast<size_t>(L.JE) * kERowFwd * 2;
  const size_t far_bytes = static_cast<size_t>(kQPB * L.far_row) * 4;
  const size_t win_bytes = static_cast<size_t>(kFwdWinRows) * 256;
  size_t big = e_bytes > far_bytes ? e_bytes : far_bytes;
  big = big > win_bytes ? big : win_bytes;
  L.bytes = L.off_big + big;
  return L;
}

template <int SHIFT>
__global__ __launch_bounds__(kBlock, 2) void dsqg_fwd_bf16_win(const dwarf_dsqg_fwd_args a, int tiles, int total) {
  constexpr int CJ = 1;
  constexpr float kC = 0.125f * kLog2e;           // 1/sqrt(64) in base-2 score units
  constexpr float kSlack2 = 8.0f * kLog2e;        // kRescaleSlack in base 2
  static_assert(SHIFT + 1 < kHeadDim / kPlanes, "MOVT pair must stay inside one lane's slice");
  const int J = a.J, N = a.N, J_small = a.J_small;
  const FwdWinLayout lay = fwd_win_layout(J, J_small, a.J_large);
  extern __shared__ float smem[];
  char* sm = reinterpret_cast<char*>(smem);
  float* s_pb = smem;
  int* s_off = reinterpret_cast<int*>(smem + lay.JE);
  float2* s_ph = reinterpret_cast<float2*>(sm + lay.off_ph);
  int2* s_list_all = reinterpret_cast<int2*>(sm + lay.off_list);
  float* s_near = reinterpret_cast<float*>(sm + lay.off_near);
  int* s_jn = reinterpret_cast<int*>(sm + lay.off_jn);             // [0]: JB; [kJnBias + d]: band slot of d, or -1
  uint16_t* sE = reinterpret_cast<uint16_t*>(sm + lay.off_big);   // until the q.E tables are written
  float* s_far = reinterpret_cast<float*>(sm + lay.off_big);      // during the far walk
  char* s_kwin = sm + lay.off_big;                                 // during the near walk
  char* s_vwin = s_kwin + kFwdWinRows * 128;

  const int work = xcd_remap(blockIdx.x, total);
  const int bh = work / tiles;
  // late query tiles (more valid offsets) of each (b, h) are dispatched first
  const int tile = tiles - 1 - (work - bh * tiles);
  const int b = bh / a.H;
  const int h = bh - b * a.H;
  const int hk = h / (a.H / a.H_kv);

  const int lane = threadIdx.x;
  const int w = lane / kWave;
  const int l = lane % kWave;
  const int g = l & 3;
  const int qi = l >> 2;
  const int lr = l & 15, lc = l >> 4;
  const int n0 = tile * kQPB;
  const int n0w = n0 + w * kQPW;
  const int n = n0w + qi;
  const int n_hi = min(n0w + kQPW - 1, N - 1);
  const bool row_ok = n < N;
  const bool live = row_ok && n >= a.query_start;
  const int64_t nn = n;
  int2* s_list = s_list_all + w * lay.list_len;

  // the wave's q rows (MFMA operand layout and this lane's slice) and y first
  const bf16* qbase = reinterpret_cast<const bf16*>(a.q) + b * a.q_stride[0] + h * a.q_stride[1];
  uint4 xa[2] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
  if (n0w + lr < N) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      xa[ks] = *reinterpret_cast<const uint4*>(qbase + static_cast<int64_t>(n0w + lr) * a.q_stride[2] + 32 * ks + 8 * lc);
  }
  // with query_probes y is formed below from the q row (every row < N) and written to y_out
  const bool probed = a.query_probes != nullptr;
  uint4 qx0 = {0u, 0u, 0u, 0u}, qx1 = {0u, 0u, 0u, 0u};
  float yg = 0.f;
  if (probed ? row_ok : live) {
    const uint4* q4 = reinterpret_cast<const uint4*>(qbase + nn * a.q_stride[2] + 16 * g);
    qx0 = q4[0];
    qx1 = q4[1];
    if (!probed) yg = a.y_pre[b * a.y_stride[0] + h * a.y_stride[1] + nn * a.y_stride[2] + g];
  }

  stage_tables<true, true, true, true, true>(
      a, lay.JE, h, 1, TableStage{sE, kERowFwd, s_pb, 1.0f, s_off, s_ph, 0, s_jn, kFwdWinBack, lay.JBh, true});
  __syncthreads();

  // q.E tables, log2(e) * (<q, e_j> / 8 + pb_j) for the wave's 16 queries:
  // products into registers, a barrier (every wave is done reading sE), then
  // the near columns into s_near and the far columns over sE.
  {
    f32x4 c[kMaxQeBlocks];
#pragma unroll
    for (int bi = 0; bi < kMaxQeBlocks; ++bi) {
      c[bi] = zero4();
      if (bi * 16 < lay.JE) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const uint4 xb = *reinterpret_cast<const uint4*>(sE + (bi * 16 + lr) * kERowFwd + 32 * ks + 8 * lc);
          c[bi] = mfma16_bf16(bf16x8_from_bits(xa[ks]), bf16x8_from_bits(xb), c[bi]);
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int bi = 0; bi < kMaxQeBlocks; ++bi) {
      if (bi * 16 < lay.JE) {
        const int j = bi * 16 + lr;
        const float pb8 = 8.0f * s_pb[j];
        float* dst = j < lay.JBh ? s_near + (w * kQPW + 4 * lc) * lay.near_row + j
                                 : s_far + (w * kQPW + 4 * lc) * lay.far_row + (j - lay.JBh);
        const int stride = j < lay.JBh ? lay.near_row : lay.far_row;
#pragma unroll
        for (int r = 0; r < 4; ++r) dst[r * stride] = (c[bi][r] + pb8) * kC;
      }
    }
  }
  // JB: the leading offsets while they ascend and stay <= kFwdWinBack (at most JBh)
  const int JB = uniform(s_jn[0]);

  const uint32_t q32[8] = {qx0.x, qx0.y, qx0.z, qx0.w, qx1.x, qx1.y, qx1.z, qx1.w};
  if (probed) {   // y of plane g (dsqg:3231-3254); the four lanes of each query take part
    yg = probe_feature(q32, a.query_probes, g);
    if (row_ok) a.y_out[(static_cast<int64_t>(b * a.H + h) * N + n) * kPlanes + g] = yg;
  }
  // Per-lane byte offsets of row 0 shifted by the lane's query; a lane without
  // a live query uses n_eff = n0w - 2N, so n_eff - d < 0 for every listed d.
  const int n_eff = live ? n : n0w - 2 * N;
  const int ks_b = static_cast<int>(a.k_stride[2]) * 2, vs_b = static_cast<int>(a.v_stride[2]) * 2;
  const int zs_b = static_cast<int>(a.z_stride[2]) * 4;
  const __amdgpu_buffer_rsrc_t rk =
      rows_rsrc(reinterpret_cast<const bf16*>(a.k) + b * a.k_stride[0] + hk * a.k_stride[1], ks_b, N, 128);
  const __amdgpu_buffer_rsrc_t rv =
      rows_rsrc(reinterpret_cast<const bf16*>(a.v) + b * a.v_stride[0] + hk * a.v_stride[1], vs_b, N, 128);
  const __amdgpu_buffer_rsrc_t rz = rows_rsrc(a.z_pre + b * a.z_stride[0] + hk * a.z_stride[1], zs_b, N, 16);
  const int kb_lane = n_eff * ks_b + 32 * g;
  const int vb_lane = n_eff * vs_b + 32 * g;
  const int zb_lane = n_eff * zs_b + 4 * g;
  // this query's q.E row: near columns j < JBh, far columns j >= JBh (j uniform)
  const float* qe_near = s_near + (w * kQPW + qi) * lay.near_row;
  const float* qe_far = s_far + (w * kQPW + qi) * lay.far_row - lay.JBh;

  float acc[16];
#pragma unroll
  for (int d = 0; d < 16; ++d) acc[d] = 0.f;
  float m = -3.0e38f, lsum = 0.f;

  auto consume = [&](const FwdChunk<CJ>& c, const float* qe_row) {
    float sc[CJ];
    float cmax = -INFINITY;
#pragma unroll
    for (int jj = 0; jj < CJ; ++jj) {
      const uint32_t* kw = reinterpret_cast<const uint32_t*>(&c.k[jj][0]);
      float dot = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) dot = dot2bf(q32[i], kw[i], dot);
      dot = group_sum<4>(dot);
      const float s2 = fmaf(dot, kC, qe_row[c.j[jj]]);
      sc[jj] = c.ok[jj] ? s2 : -INFINITY;
      cmax = fmaxf(cmax, sc[jj]);
    }
    if (cmax > m + kSlack2) {
      const float f = __builtin_amdgcn_exp2f(m - cmax);   // 0 on the first valid chunk
#pragma unroll
      for (int d = 0; d < 16; ++d) acc[d] *= f;
      lsum *= f;
      m = cmax;
    }
#pragma unroll
    for (int jj = 0; jj < CJ; ++jj) {
      const float p = __builtin_amdgcn_exp2f(sc[jj] - m);  // m is finite: 0 without a source
      lsum += p;
      const uint32_t* vw = reinterpret_cast<const uint32_t*>(&c.v[jj][0]);
      float vf[16];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        vf[2 * i] = bf16_lo(vw[i]);
        vf[2 * i + 1] = bf16_hi(vw[i]);
      }
      const int j = c.j[jj];
      if (j >= J_small && j < J) {
        const float2 ph = s_ph[(j - J_small) * kPlanes + g];
        float sn, cs;
        dsincos<true>(fmaf(ph.y * yg, c.z[jj], ph.x), &sn, &cs);
        const float va = vf[SHIFT], vb = vf[SHIFT + 1];
        vf[SHIFT] = cs * va - sn * vb;
        vf[SHIFT + 1] = sn * va + cs * vb;
      }
#pragma unroll
      for (int d = 0; d < 16; ++d) acc[d] = fmaf(p, vf[d], acc[d]);
    }
  };

  // ---- 1. far walk: the listed offsets j >= JB, gathered ----
  if (n0w < N) {
    // The sentinel (index J) gets the offset n0w - N, out of range for every query.
    const int cnt = build_offset_list<CJ>(s_list, s_off, J, n0w, n_hi, N, 1, make_int2(J, n0w - N), JB);
    auto fetch = [&](int k0, FwdChunk<CJ>& c) {
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
        c.z[jj] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rz, zo, 0, 0));
      }
    };
    if (cnt > 0) {
      // every listed far offset has j >= JB; j in [JB, JBh) only when the small
      // offsets leave the window early, and reads the near table
      const bool all_far = JB == lay.JBh;
      FwdChunk<CJ> c0, c1;
      fetch(0, c0);
      for (int k0 = 0; k0 < cnt; k0 += 2 * CJ) {
        fetch(k0 + CJ, c1);        // past the list end this reads the sentinel: zeros
        consume(c0, all_far || c0.j[0] >= lay.JBh ? qe_far : qe_near);
        fetch(k0 + 2 * CJ, c0);
        consume(c1, all_far || c1.j[0] >= lay.JBh ? qe_far : qe_near);
      }
    }
  }

  // ---- 2. near band: offsets j < JB on the matrix cores, from the window in LDS ----
  __syncthreads();   // every wave is done with the far table: the window goes over it
  if (JB > 0) {
    // keys [n0 - kFwdWinBack, n0 + 64): 96 rows of K and of V, three 1 KB DMA
    // loads of each per wave; LDS chunk i & 7 of row i >> 3 holds the row's
    // 16-byte chunk (i & 7) ^ (row & 7).  Keys outside [0, N) read zeros.
    typedef __attribute__((address_space(3))) void lds_void;
#pragma unroll
    for (int u = 0; u < 3; ++u) {
      const int i = kBlock * u + lane;
      const int row = i >> 3, c = (i & 7) ^ (row & 7);
      const int key = n0 - kFwdWinBack + row;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void*)(void*)(s_kwin + 4096 * u + 1024 * w), 16,
                                               static_cast<uint32_t>(key * ks_b + 16 * c), 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_void*)(void*)(s_vwin + 4096 * u + 1024 * w), 16,
                                               static_cast<uint32_t>(key * vs_b + 16 * c), 0, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): this wave's window loads have landed
  }
  __syncthreads();   // the window is staged
  if (n0w < N && JB > 0) {
    // Band lane (lc, lr) serves query n0w + lr; in the MFMA C layout it holds
    // keys n0w - 32 + 16 tb + 4 lc + r of the wave's key blocks tb = 0..2.
    //   S^T = K_win Q^T                 (v_mfma_f32_16x16x32_bf16)
    //   P = exp2(S' - m) on the band's diagonals, m the query's running maximum
    //   O^T += V_win^T P^T               (v_mfma_f32_16x16x16_bf16, P as bf16 hi + lo)
    // then O^T joins the gather layout by ds_bpermute.
    const int nq = n0w + lr;
    const bool live_b = nq < N && nq >= a.query_start;
    auto win16 = [&](const char* base, int row, int c) { return base + row * 128 + 16 * (c ^ (row & 7)); };
    const float* qe_b = s_near + (w * kQPW + lr) * lay.near_row;
    // the far walk's running maximum of this query (gather lane 4 lr)
    const float m_q = __int_as_float(__builtin_amdgcn_ds_bpermute(4 * (4 * lr), __float_as_int(m)));
    float sb[3][4];
    float cmax = -INFINITY;
#pragma unroll
    for (int tb = 0; tb < 3; ++tb) {
      const int wr = 16 * (w + tb) + lr;               // window row of key n0w - 32 + 16 tb + lr
      const uint4 ka0 = *reinterpret_cast<const uint4*>(win16(s_kwin, wr, lc));
      const uint4 ka1 = *reinterpret_cast<const uint4*>(win16(s_kwin, wr, 4 + lc));
      f32x4 S = mfma16_bf16(bf16x8_from_bits(ka0), bf16x8_from_bits(xa[0]), zero4());
      S = mfma16_bf16(bf16x8_from_bits(ka1), bf16x8_from_bits(xa[1]), S);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        // band slot of the pair (query nq, key n0w - 32 + 16 tb + 4 lc + r): the delta lies in
        // [-15, 47], inside the table; computed for every lane and masked, with no branch
        const int slot = s_jn[kJnBias + lr + kFwdWinBack - 16 * tb - 4 * lc - r];
        const bool ok = slot >= 0 && live_b && n0w - kFwdWinBack + 16 * tb + 4 * lc + r >= 0;
        const float sc2 = fmaf(S[r], kC, qe_b[slot >= 0 ? slot : 0]);
        sb[tb][r] = ok ? sc2 : -INFINITY;
        cmax = fmaxf(cmax, sb[tb][r]);
      }
    }
    cmax = max_xor32(max_xor16(cmax));                 // over the four lanes of query lr
    // the band's reference: the running maximum, raised only past the slack (as the walk does)
    const float m_use = cmax > m_q + kSlack2 ? cmax : m_q;
    f32x4 acch[4];
#pragma unroll
    for (int db = 0; db < 4; ++db) acch[db] = zero4();
    float lb = 0.f;
#pragma unroll
    for (int tb = 0; tb < 3; ++tb) {
      float ph[4], pl[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = __builtin_amdgcn_exp2f(sb[tb][r] - m_use);   // 0 off the band
        lb += p;
        ph[r] = p;
        pl[r] = p - round_bf16(p);
      }
      const i16x4 bh = __builtin_bit_cast(i16x4, make_uint2(pack_bf16x2(ph[0], ph[1]), pack_bf16x2(ph[2], ph[3])));
      const i16x4 bl = __builtin_bit_cast(i16x4, make_uint2(pack_bf16x2(pl[0], pl[1]), pack_bf16x2(pl[2], pl[3])));
      // V^T read transposed from the window (rows 16 (w + tb) + 4 lc + e, dims
      // 16 (lr / 4) + 4 db + lr % 4 of MFMA row lr)
      const int R = 16 * (w + tb) + 4 * lc + (lr >> 2);
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const i16x4 av = lds_read_tr16(win16(s_vwin, R, 2 * (lr & 3) + (db >> 1)) + 8 * (db & 1));
        acch[db] = mfma16k16_bf16(av, bh, acch[db]);
        acch[db] = mfma16k16_bf16(av, bl, acch[db]);
      }
    }
    lb = add_xor32(add_xor16(lb));
    // into the gather layout: query qi, dims 16 g + 4 db + r <- band lane (lr = qi, lc = g)
    const int srcq = 4 * (qi + 16 * g);
    const float m_new = __int_as_float(__builtin_amdgcn_ds_bpermute(srcq, __float_as_int(m_use)));
    const float l_new = __int_as_float(__builtin_amdgcn_ds_bpermute(srcq, __float_as_int(lb)));
    const float f = __builtin_amdgcn_exp2f(m - m_new);   // 1 when the maximum stays; 0 with no far pair
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        acc[4 * db + r] = fmaf(acc[4 * db + r], f,
                               __int_as_float(__builtin_amdgcn_ds_bpermute(srcq, __float_as_int(acch[db][r]))));
    lsum = fmaf(lsum, f, l_new);
    m = m_new;
  }

  if (!row_ok) return;
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  uint4* o4 = reinterpret_cast<uint4*>(reinterpret_cast<bf16*>(a.out) + b * a.out_stride[0] + h * a.out_stride[1] +
                                       nn * a.out_stride[2] + 16 * g);
  uint4 x0, x1;
  x0.x = pack_bf16x2(acc[0] * inv, acc[1] * inv);
  x0.y = pack_bf16x2(acc[2] * inv, acc[3] * inv);
  x0.z = pack_bf16x2(acc[4] * inv, acc[5] * inv);
  x0.w = pack_bf16x2(acc[6] * inv, acc[7] * inv);
  x1.x = pack_bf16x2(acc[8] * inv, acc[9] * inv);
  x1.y = pack_bf16x2(acc[10] * inv, acc[11] * inv);
  x1.z = pack_bf16x2(acc[12] * inv, acc[13] * inv);
  x1.w = pack_bf16x2(acc[14] * inv, acc[15] * inv);
  o4[0] = x0;
  o4[1] = x1;
  if (g == 0)
    a.lse[b * a.lse_stride[0] + h * a.lse_stride[1] + nn * a.lse_stride[2]] =
        lsum > 0.f ? (m + __builtin_amdgcn_logf(lsum)) * kLn2 : -INFINITY;
}

hipError_t launch_fwd_bf16_win(const dwarf_dsqg_fwd_args& a, hipStream_t stream) {
  const int tiles = (a.N + kQPB - 1) / kQPB;
  const int total = tiles * a.B * a.H;
  if (total == 0) return hipSuccess;
  const size_t lds = fwd_win_layout(a.J, a.J_small, a.J_large).bytes;
#define DWARF_FWDWIN_CASE(S)                                                                                   \
  case S:                                                                                                       \
    hipLaunchKernelGGL((dsqg_fwd_bf16_win<S>), dim3(total), dim3(kBlock), lds, stream, a, tiles, total);       \
    break;
  switch (a.plane_shift) {
    DWARF_FWDWIN_CASE(0) DWARF_FWDWIN_CASE(1) DWARF_FWDWIN_CASE(2) DWARF_FWDWIN_CASE(3) DWARF_FWDWIN_CASE(4)
    DWARF_FWDWIN_CASE(5) DWARF_FWDWIN_CASE(6) DWARF_FWDWIN_CASE(7) DWARF_FWDWIN_CASE(8) DWARF_FWDWIN_CASE(9)
    DWARF_FWDWIN_CASE(10) DWARF_FWDWIN_CASE(11) DWARF_FWDWIN_CASE(12) DWARF_FWDWIN_CASE(13) DWARF_FWDWIN_CASE(14)
    default: return hipErrorInvalidValue;
  }
#undef DWARF_FWDWIN_CASE
  return hipGetLastError();
}

template <int CJ, bool TWO_PASS>
hipError_t launch_fwd_bf16_q4(const dwarf_dsqg_fwd_args& a, hipStream_t stream) {
  const int tiles = (a.N + kQPB - 1) / kQPB;
  const int total = tiles * a.B * a.H;
  if (total == 0) return hipSuccess;
  const size_t lds = fwd_layout(a.J, a.J_large, CJ).bytes;
#define DWARF_FWDQ4_CASE(S)                                                                                     \
  case S:                                                                                                       \
    hipLaunchKernelGGL((dsqg_fwd_bf16_q4<S, CJ, TWO_PASS>), dim3(total), dim3(kBlock), lds, stream, a, tiles,   \
                       total);                                                                                  \
    break;
  switch (a.plane_shift) {
    DWARF_FWDQ4_CASE(0) DWARF_FWDQ4_CASE(1) DWARF_FWDQ4_CASE(2) DWARF_FWDQ4_CASE(3) DWARF_FWDQ4_CASE(4)
    DWARF_FWDQ4_CASE(5) DWARF_FWDQ4_CASE(6) DWARF_FWDQ4_CASE(7) DWARF_FWDQ4_CASE(8) DWARF_FWDQ4_CASE(9)
    DWARF_FWDQ4_CASE(10) DWARF_FWDQ4_CASE(11) DWARF_FWDQ4_CASE(12) DWARF_FWDQ4_CASE(13) DWARF_FWDQ4_CASE(14)
    default: return hipErrorInvalidValue;
  }
#undef DWARF_FWDQ4_CASE
  return hipGetLastError();
}

template <typename T, int L, bool FAST, bool TWO_PASS>
hipError_t launch_shift(const dwarf_dsqg_fwd_args& a, hipStream_t stream) {
  constexpr int QPB = kBlock / L;
  const int tiles = (a.N + QPB - 1) / QPB;
  const int total = tiles * a.B * a.H;
  const size_t lds = static_cast<size_t>(a.J) * (kHeadDim + 2) * sizeof(float);
#define DWARF_FWD_CASE(S)                                                                        \
  case S:                                                                                        \
    hipLaunchKernelGGL((dsqg_fwd_kernel<T, S, L, FAST, TWO_PASS>), dim3(total), dim3(kBlock), lds, \
                       stream, a, tiles, total);                                                 \
    break;
  switch (a.plane_shift) {
    DWARF_FWD_CASE(0) DWARF_FWD_CASE(1) DWARF_FWD_CASE(2) DWARF_FWD_CASE(3) DWARF_FWD_CASE(4)
    DWARF_FWD_CASE(5) DWARF_FWD_CASE(6) DWARF_FWD_CASE(7) DWARF_FWD_CASE(8) DWARF_FWD_CASE(9)
    DWARF_FWD_CASE(10) DWARF_FWD_CASE(11) DWARF_FWD_CASE(12) DWARF_FWD_CASE(13) DWARF_FWD_CASE(14)
    default:
      return hipErrorInvalidValue;
  }
#undef DWARF_FWD_CASE
  return hipGetLastError();
}

}  // namespace

hipError_t launch_dsqg_fwd(const dwarf_dsqg_fwd_args& a, hipStream_t stream) {
  const bool two_pass = (a.schedule & DWARF_SCHED_TWO_PASS) != 0;
  if (a.dtype == DWARF_BF16) {
    if (two_pass) return launch_fwd_bf16_q4<kChunkFwd, true>(a, stream);
    if ((a.schedule & DWARF_SCHED_BAND) && a.J_small > 0) return launch_fwd_bf16_win(a, stream);
    return launch_fwd_bf16_q4<kChunkFwd, false>(a, stream);
  }
  return two_pass ? launch_shift<float, 2, false, true>(a, stream) : launch_shift<float, 2, false, false>(a, stream);
}

}  // namespace dwarf
