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

namespace dwarf {
namespace {

constexpr float kRescaleSlack = 8.0f;

template <typename T, int SHIFT, int L, bool FAST>
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

      if (score > m + kRescaleSlack) {
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

template <typename T, int L, bool FAST>
hipError_t launch_shift(const dwarf_dsqg_fwd_args& a, hipStream_t stream) {
  constexpr int QPB = kBlock / L;
  const int tiles = (a.N + QPB - 1) / QPB;
  const int total = tiles * a.B * a.H;
  const size_t lds = static_cast<size_t>(a.J) * (kHeadDim + 2) * sizeof(float);
#define DWARF_FWD_CASE(S)                                                                        \
  case S:                                                                                        \
    hipLaunchKernelGGL((dsqg_fwd_kernel<T, S, L, FAST>), dim3(total), dim3(kBlock), lds, \
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
  if (a.dtype == DWARF_BF16) return launch_shift<bf16, 2, true>(a, stream);
  return launch_shift<float, 2, false>(a, stream);
}

}  // namespace dwarf
