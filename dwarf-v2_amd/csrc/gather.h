// Shared pieces of the bf16 gather kernels (forward, dQ and dK/dV launches):
// packed-bf16 dot products, raw buffer loads with 32-bit offsets (an offset
// past the end of the tensor reads zeros) and the per-wave offset list.
#pragma once

#include "common.h"
#include "dsqg_internal.h"

namespace dwarf {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr uint32_t kOutOfRange = 0x80000000u;  // buffer offset past every tensor (spans are < 2^31)

// Near-band slot table in LDS, kJnSize ints: entry 0 holds the band's offset
// count JB, entry kJnBias + d the band slot of delta d, and -1 for every other
// delta in [1 - kJnBias, kJnSize - 1 - kJnBias].  The band kernels look up
// deltas in [-15, 47] without a range check (a range check around the LDS
// read becomes an exec-mask branch per lookup).  The band is the leading
// small offsets while they ascend and stay <= max_delta.  Thread 0 only.
constexpr int kJnBias = 16, kJnSize = 64;
__device__ __forceinline__ void build_band_slots(int* s_jn, const int* offsets, int J_small, int max_delta,
                                                 int max_slots, bool band) {
  for (int i = 1; i < kJnSize; ++i) s_jn[i] = -1;
  int jb = 0;
  while (band && jb < J_small && jb < max_slots) {
    const int d = offsets[jb];
    if (d < 1 || d > max_delta || (jb > 0 && d <= offsets[jb - 1])) break;
    s_jn[kJnBias + d] = jb++;
  }
  s_jn[0] = jb;
}

// The i-th of four values for a lane-varying i in [0, 4), as three selects on
// the bits of i.  A chained `i == 0 ? a : i == 1 ? b : ...` is lowered as a
// switch, i.e. nested exec-mask branches around empty blocks.
template <typename T>
__device__ __forceinline__ T pick4(int i, T a, T b, T c, T d) {
  const T lo = (i & 1) ? b : a;
  const T hi = (i & 1) ? d : c;
  return (i & 2) ? hi : lo;
}

__device__ __forceinline__ float dot2bf(uint32_t a, uint32_t b, float c) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
}

// Zero-instruction barrier on register values: the computations that produce
// them stay before this point (the compiler may not sink them into a later block).
template <int CNT>
__device__ __forceinline__ void pin_regs(float* v) {
#pragma unroll
  for (int i = 0; i < CNT; ++i) asm volatile("" : "+v"(v[i]));
}

__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  return uint4{v[0], v[1], v[2], v[3]};
}

__device__ __forceinline__ float buf_load_f32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

__device__ __forceinline__ uint16_t buf_load_u16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}

// Resource over `rows` rows of `row_bytes` stride whose last row is `tail` bytes.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const void* base, int64_t row_bytes, int rows, int tail) {
  const int64_t span = rows > 0 ? (rows - 1) * row_bytes + tail : 0;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(span), 0x00020000);
}

// E (scale_embed [J][64] fp32) into LDS as bf16 rows of `row` elements, rows
// J..JE-1 zero, rounded to nearest even (the reference GPU path's bf16 SE,
// dsqg:760-763).  Four values per thread step.  With unit-stride, 16-byte
// aligned rows (the usual layout) every load is an unconditional 16-byte
// buffer load, rows >= J reading zeros past the end of the buffer, and a
// thread issues all its loads before the first conversion: one memory round
// trip.  (A load under a branch with a zero default forces a wait for it at
// the join, which had turned the staging into one round trip per step.)
// Other layouts take a scalar path.
constexpr int kSeBatch = 8;
__device__ __forceinline__ void stage_se_bf16(const float* se, const int64_t* se_stride, int J, int JE,
                                              uint16_t* sE, int row) {
  // the vector path addresses rows with 32-bit offsets: row stride <= 2^20 elements keeps JE rows below 2 GiB
  const bool vec = se_stride[1] == 1 && (se_stride[0] & 3) == 0 && se_stride[0] <= (int64_t(1) << 20) &&
                   (reinterpret_cast<uintptr_t>(se) & 15) == 0;
  typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
  const int n = JE * 16;
  const int nt = static_cast<int>(blockDim.x);
  if (vec) {
    const int rb = static_cast<int>(se_stride[0]) * 4;   // row bytes
    const __amdgpu_buffer_rsrc_t r = rows_rsrc(se, rb, J, 256);
    for (int i0 = threadIdx.x; i0 < n; i0 += kSeBatch * nt) {
      uint4 x[kSeBatch];
#pragma unroll
      for (int u = 0; u < kSeBatch; ++u) {
        const int i = i0 + u * nt;
        x[u] = buf_load16(r, i < n ? static_cast<uint32_t>((i >> 4) * rb + 16 * (i & 15)) : kOutOfRange);
      }
#pragma unroll
      for (int u = 0; u < kSeBatch; ++u) {
        const int i = i0 + u * nt;
        if (i < n) {
          const bf16x4_t h = {static_cast<__bf16>(__uint_as_float(x[u].x)), static_cast<__bf16>(__uint_as_float(x[u].y)),
                              static_cast<__bf16>(__uint_as_float(x[u].z)), static_cast<__bf16>(__uint_as_float(x[u].w))};
          *reinterpret_cast<bf16x4_t*>(sE + (i >> 4) * row + 4 * (i & 15)) = h;
        }
      }
    }
    return;
  }
  for (int i = threadIdx.x; i < n; i += nt) {
    const int j = i >> 4, d = 4 * (i & 15);
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
    if (j < J) {
      const float* p = se + j * se_stride[0] + d * se_stride[1];
      x = make_float4(p[0], p[se_stride[1]], p[2 * se_stride[1]], p[3 * se_stride[1]]);
    }
    const bf16x4_t h = {static_cast<__bf16>(x.x), static_cast<__bf16>(x.y), static_cast<__bf16>(x.z),
                        static_cast<__bf16>(x.w)};
    *reinterpret_cast<bf16x4_t*>(sE + j * row + d) = h;
  }
}


// Destinations of the per-workgroup tables staged by stage_tables.
struct TableStage {
  uint16_t* sE;      // E rows in bf16, rows of e_row elements (rows J..JE-1 zero)
  int e_row;
  float* s_pb;       // pb_scale * pos_bias[j][h0 + hh] at hh * JE + j (0 for j >= J)
  float pb_scale;
  int* s_off;        // the offsets (0 for j >= J), JE entries
  float2* s_ph;      // (phase_base, phase_gain)[i][h0 + hh][r] at hh * ph_head + i * kPlanes + r
  int ph_head;
  int* s_jn;         // the near band's slot table (build_band_slots)
  int band_delta, band_slots;
  bool band;
};

// Stages the tables a gather workgroup reads (Args: the DSQG or q6 prefill arguments, which name them
// alike), for heads h0 .. h0 + nh - 1, with every global load of the
// first round in flight before the first LDS store.  A load under a condition is waited for at its join
// (one round trip each), so entries past a table read zeros through buffer loads instead; the band slot
// table (JN) is built by wave 0 from the offsets its lanes loaded, with what build_band_slots computes.
// Entries past the first round (J > 127, or the tables of several heads) take element loops; table
// layouts beyond 32-bit offsets take element loops throughout, with the slot table built by thread 0
// from memory.  The caller's barrier completes the staging.  band_delta <= kJnSize - 1 - kJnBias.
static_assert(kJnSize == kWave, "stage_tables builds the slot table one entry per lane of wave 0");

template <bool E, bool PB, bool OFF, bool PH, bool JN, typename Args>
__device__ __forceinline__ void stage_tables(const Args& f, int JE, int h0, int nh, const TableStage& d) {
  const int J = f.J, JL = f.J_large;
  const int64_t pbs0 = f.pb_stride[0], pbs1 = f.pb_stride[1];
  const int64_t bs0 = f.pbase_stride[0], bs1 = f.pbase_stride[1], gs0 = f.pgain_stride[0], gs1 = f.pgain_stride[1];
  const int64_t se0 = f.se_stride[0];
  constexpr int64_t kSpan = int64_t(1) << 31;
  const int64_t pb_span = ((J - 1) * pbs0 + (nh - 1) * pbs1 + 1) * 4;
  const int64_t b_span = JL > 0 ? ((JL - 1) * bs0 + (nh - 1) * bs1 + kPlanes) * 4 : 0;
  const int64_t g_span = JL > 0 ? ((JL - 1) * gs0 + (nh - 1) * gs1 + kPlanes) * 4 : 0;
  const bool fast =
      (!E || (f.se_stride[1] == 1 && (se0 & 3) == 0 && se0 <= (int64_t(1) << 20) &&
              (reinterpret_cast<uintptr_t>(f.scale_embed) & 15) == 0)) &&
      (!PB || (pbs0 >= 0 && pbs1 >= 0 && pb_span < kSpan)) &&
      (!PH || (bs0 >= 0 && bs1 >= 0 && b_span < kSpan && gs0 >= 0 && gs1 >= 0 && g_span < kSpan));
  const int tid = threadIdx.x, nt = static_cast<int>(blockDim.x);
  const int ne = JE * 16, npb = nh * JE, nph = nh * JL * kPlanes;
  typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
  auto put_e = [&](int i, uint4 x) {
    const bf16x4_t h = {static_cast<__bf16>(__uint_as_float(x.x)), static_cast<__bf16>(__uint_as_float(x.y)),
                        static_cast<__bf16>(__uint_as_float(x.z)), static_cast<__bf16>(__uint_as_float(x.w))};
    *reinterpret_cast<bf16x4_t*>(d.sE + (i >> 4) * d.e_row + 4 * (i & 15)) = h;
  };
  auto ph_slot = [&](int t) {   // entry t = (hh * JL + i) * kPlanes + r, t < nph
    const int hh = t / (JL * kPlanes);
    return hh * d.ph_head + (t - hh * JL * kPlanes);
  };
  if (!fast) {
    if (E) stage_se_bf16(f.scale_embed, f.se_stride, J, JE, d.sE, d.e_row);
    if (PB)
      for (int t = tid; t < npb; t += nt) {
        const int hh = t / JE, j = t - hh * JE;
        d.s_pb[t] = j < J ? d.pb_scale * f.pos_bias[j * pbs0 + (h0 + hh) * pbs1] : 0.f;
      }
    if (OFF)
      for (int j = tid; j < JE; j += nt) d.s_off[j] = j < J ? f.offsets[j] : 0;
    if (PH)
      for (int t = tid; t < nph; t += nt) {
        const int hh = t / (JL * kPlanes), rest = t - hh * JL * kPlanes;
        const int i = rest / kPlanes, r = rest - i * kPlanes;
        d.s_ph[ph_slot(t)] = make_float2(f.phase_base[i * bs0 + (h0 + hh) * bs1 + r],
                                         f.phase_gain[i * gs0 + (h0 + hh) * gs1 + r]);
      }
    if (JN && tid == 0) build_band_slots(d.s_jn, f.offsets, f.J_small, d.band_delta, d.band_slots, d.band);
    return;
  }
  const int rb = static_cast<int>(se0) * 4;   // E row bytes
  const __amdgpu_buffer_rsrc_t rse = rows_rsrc(f.scale_embed, rb, J, 256);
  const __amdgpu_buffer_rsrc_t rpb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(f.pos_bias + h0 * pbs1), 0, static_cast<int>(PB ? pb_span : 0), 0x00020000);
  const __amdgpu_buffer_rsrc_t rof = __builtin_amdgcn_make_buffer_rsrc(const_cast<int*>(f.offsets), 0, J * 4, 0x00020000);
  const __amdgpu_buffer_rsrc_t rbs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(f.phase_base + h0 * bs1), 0, static_cast<int>(PH ? b_span : 0), 0x00020000);
  const __amdgpu_buffer_rsrc_t rgn = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(f.phase_gain + h0 * gs1), 0, static_cast<int>(PH ? g_span : 0), 0x00020000);
  auto e_off = [&](int i) { return i < ne ? static_cast<uint32_t>((i >> 4) * rb + 16 * (i & 15)) : kOutOfRange; };
  auto pb_off = [&](int t) {   // entry t = hh * JE + j
    const int hh = t / JE, j = t - hh * JE;
    return t < npb && j < J ? static_cast<uint32_t>((j * pbs0 + hh * pbs1) * 4) : kOutOfRange;
  };
  auto ph_off = [&](int t, int64_t s0, int64_t s1) {
    if (t >= nph) return kOutOfRange;   // (every entry when JL = 0)
    const int hh = t / (JL * kPlanes), rest = t - hh * JL * kPlanes;
    const int i = rest / kPlanes, r = rest - i * kPlanes;
    return static_cast<uint32_t>((i * s0 + hh * s1 + r) * 4);
  };
  // first round: every load, then every store
  uint4 ex[E ? kSeBatch : 1];
  if (E) {
#pragma unroll
    for (int u = 0; u < kSeBatch; ++u) ex[u] = buf_load16(rse, e_off(tid + u * nt));
  }
  const float pbv = PB ? buf_load_f32(rpb, pb_off(tid)) : 0.f;
  const int ofv = OFF || JN ? static_cast<int>(__builtin_amdgcn_raw_buffer_load_b32(
                                  rof, tid < JE ? static_cast<uint32_t>(4 * tid) : kOutOfRange, 0, 0))
                            : 0;
  float phb[2] = {0.f, 0.f}, phg[2] = {0.f, 0.f};
  if (PH) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      phb[u] = buf_load_f32(rbs, ph_off(tid + u * nt, bs0, bs1));
      phg[u] = buf_load_f32(rgn, ph_off(tid + u * nt, gs0, gs1));
    }
  }
  if (E) {
#pragma unroll
    for (int u = 0; u < kSeBatch; ++u)
      if (tid + u * nt < ne) put_e(tid + u * nt, ex[u]);
  }
  if (PB && tid < npb) d.s_pb[tid] = d.pb_scale * pbv;
  if (OFF && tid < JE) d.s_off[tid] = ofv;
  if (PH) {
#pragma unroll
    for (int u = 0; u < 2; ++u)
      if (tid + u * nt < nph) d.s_ph[ph_slot(tid + u * nt)] = make_float2(phb[u], phg[u]);
  }
  if (JN && tid < kWave) {   // build_band_slots from the lanes' offsets j = lane
    const int prev = __shfl_up(ofv, 1);
    const bool ok = d.band && tid < f.J_small && tid < d.band_slots && ofv >= 1 && ofv <= d.band_delta &&
                    (tid == 0 || ofv > prev);
    const uint64_t m = __ballot(ok);
    const int jb = static_cast<int>(__builtin_ctzll(~m));
    d.s_jn[tid] = tid == 0 ? jb : -1;
    if (tid < jb) d.s_jn[kJnBias + ofv] = tid;   // after the lane's -1: a wave's LDS stores land in order
  }
  // what the first round did not cover
  if (E)
    for (int i = tid + kSeBatch * nt; i < ne; i += nt) put_e(i, buf_load16(rse, e_off(i)));
  if (PB)
    for (int t = tid + nt; t < npb; t += nt) d.s_pb[t] = d.pb_scale * buf_load_f32(rpb, pb_off(t));
  if (OFF)
    for (int j = tid + nt; j < JE; j += nt)
      d.s_off[j] = static_cast<int>(__builtin_amdgcn_raw_buffer_load_b32(rof, static_cast<uint32_t>(4 * j), 0, 0));
  if (PH)
    for (int t = tid + 2 * nt; t < nph; t += nt)
      d.s_ph[ph_slot(t)] = make_float2(buf_load_f32(rbs, ph_off(t, bs0, bs1)), buf_load_f32(rgn, ph_off(t, gs0, gs1)));
}

// Appends to `list` (wave-private LDS) the (index, offset) pairs of the
// offsets that give some position in [lo, hi] a partner position inside
// [0, N): partner = position - dir * offset, dir = +1 for queries looking
// back at keys, -1 for keys looking forward at queries.  Offsets j < j_skip
// are left out (served elsewhere).  Pads with `pad` up to a multiple of CJ
// plus two chunks.  Returns the (uniform) count.
template <int CJ>
__device__ __forceinline__ int build_offset_list(int2* list, const int* s_off, int J, int lo, int hi, int N, int dir,
                                                 int2 pad, int j_skip = 0) {
  const int l = threadIdx.x % kWave;
  int cnt = 0;
  for (int base = 0; base < J; base += kWave) {
    const int j = base + l;
    const int d = j < J ? s_off[j] : 0;
    const int sd = dir * d;
    const bool need = j < J && j >= j_skip && sd <= hi && sd >= lo - (N - 1);
    const uint64_t mask = __ballot(need);
    const int pos = cnt + __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0));
    if (need) list[pos] = make_int2(j, d);
    cnt += __popcll(mask);
  }
  cnt = uniform(cnt);
  const int cntp = (cnt + CJ - 1) / CJ * CJ;
  for (int t = cnt + l; t < cntp + 2 * CJ; t += kWave) list[t] = pad;
  __builtin_amdgcn_wave_barrier();
  return cnt;
}

// build_offset_list with the offsets already in registers: lane l holds offset j = 64 c + l in offv[c]
// (0 for j >= J), loaded with the kernel's other prologue loads, so the list waits on no memory.
template <int CJ, int NC>
__device__ __forceinline__ int build_offset_list_regs(int2* list, const int* offv, int J, int lo, int hi, int N,
                                                      int dir, int2 pad) {
  const int l = threadIdx.x % kWave;
  int cnt = 0;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int j = kWave * c + l;
    const int d = offv[c];
    const int sd = dir * d;
    const bool need = j < J && sd <= hi && sd >= lo - (N - 1);
    const uint64_t mask = __ballot(need);
    const int pos = cnt + __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0));
    if (need) list[pos] = make_int2(j, d);
    cnt += __popcll(mask);
  }
  cnt = uniform(cnt);
  const int cntp = (cnt + CJ - 1) / CJ * CJ;
  for (int t = cnt + l; t < cntp + 2 * CJ; t += kWave) list[t] = pad;
  __builtin_amdgcn_wave_barrier();
  return cnt;
}

// x + x of lane ^ 16 (v_permlane16_swap on copies of x: rows 0/2 receive
// rows 1/3 and the reverse) and x + x of lane ^ 32 (v_permlane32_swap, the
// two halves).  Both stay in the VALU, without an LDS round trip.
__device__ __forceinline__ float add_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Reduce-scatter halves of the two swaps: v_permlane32_swap exchanges the
// upper 32 lanes of its first operand with the lower 32 lanes of its second,
// so the sum of the two results is x + x of lane ^ 32 in lanes 0-31 and
// y + y of lane ^ 32 in lanes 32-63.  v_permlane16_swap does the same per
// pair of 16-lane rows: x sums in rows 0 and 2, y sums in rows 1 and 3.
__device__ __forceinline__ float add_swap32(float x, float y) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_swap16(float x, float y) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(y), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float max_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Sum over the 16 lanes of a wave that share (lane & 3): four queries of a
// 16-lane row by DPP rotation, then across the four rows.
__device__ __forceinline__ float sum_over_queries16(float x) {
  x += dpp_f<0x124>(x);  // row_ror:4
  x += dpp_f<0x128>(x);  // row_ror:8
  return add_xor32(add_xor16(x));
}

// ---------------------------------------------------------------------------
// Phase-probe features of a row held by a group of four lanes (lane g holds
// dims [16g, 16g + 16) as 8 bf16 pairs), the DSQG block's y/z
// (dsqg:3231-3254): f_r = s <x, p_r>, s = 1 / sqrt(|x|^2 + 1e-6 hd), with the
// probes p [4][64] fp32 (rows already normalised) read from global memory.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float probe_row_scale(const uint32_t* x32) {
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss = dot2bf(x32[i], x32[i], ss);
  return rsqrtf(group_sum<4>(ss) + 1e-6f * 64);   // head_dim 64
}

// Feature f_g of this lane's plane g.
__device__ __forceinline__ float probe_feature(const uint32_t* x32, const float* __restrict__ probes, int g) {
  const float4* p4 = reinterpret_cast<const float4*>(probes) + 4 * g;   // row r, dims 16g + 4i: p4[16 r + i]
  float f[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float x0 = bf16_lo(x32[2 * i]), x1 = bf16_hi(x32[2 * i]);
    const float x2 = bf16_lo(x32[2 * i + 1]), x3 = bf16_hi(x32[2 * i + 1]);
#pragma unroll
    for (int r = 0; r < kPlanes; ++r) {
      const float4 p = p4[16 * r + i];
      f[r] = fmaf(x0, p.x, f[r]);
      f[r] = fmaf(x1, p.y, f[r]);
      f[r] = fmaf(x2, p.z, f[r]);
      f[r] = fmaf(x3, p.w, f[r]);
    }
  }
#pragma unroll
  for (int r = 0; r < kPlanes; ++r) f[r] = group_sum<4>(f[r]);
  return pick4(g, f[0], f[1], f[2], f[3]) * probe_row_scale(x32);
}

// Adds the gradient reaching the row through its features to the lane's 16
// dims of dx: dx += s sum_r df_r p_r - s^2 (sum_r df_r f_r) x, where lane g of
// the group holds f_g and its gradient df_g.
__device__ __forceinline__ void fold_probe_grad(float* dx, const uint32_t* x32, const float* __restrict__ probes,
                                                int g, float fg, float dfg) {
  const float s = probe_row_scale(x32);
  const float c = group_sum<4>(dfg * fg) * s * s;
  // df_r of every plane: quad_perm broadcasts of lane r of the group
  const float d0 = s * dpp_f<0x00>(dfg), d1 = s * dpp_f<0x55>(dfg);
  const float d2 = s * dpp_f<0xAA>(dfg), d3 = s * dpp_f<0xFF>(dfg);
  const float4* p4 = reinterpret_cast<const float4*>(probes) + 4 * g;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 a = p4[i], b = p4[16 + i], e = p4[32 + i], h = p4[48 + i];
    const float x[4] = {bf16_lo(x32[2 * i]), bf16_hi(x32[2 * i]), bf16_lo(x32[2 * i + 1]), bf16_hi(x32[2 * i + 1])};
    const float pa[4] = {a.x, a.y, a.z, a.w}, pb[4] = {b.x, b.y, b.z, b.w};
    const float pe[4] = {e.x, e.y, e.z, e.w}, ph[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
    for (int k = 0; k < 4; ++k)
      dx[4 * i + k] += fmaf(d0, pa[k], fmaf(d1, pb[k], fmaf(d2, pe[k], fmaf(d3, ph[k], -c * x[k]))));
  }
}

}  // namespace dwarf
