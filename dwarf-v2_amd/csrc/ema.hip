// Causal EMA scan, y[t] = a x[t] + (1 - a) y[t-1], y[-1] = 0, fp32 state
// (reference: _CausalEMAFn ema:263-364 with kernels ema:73-260).
//
// Time is cut into chunks of kChunkT tokens.  Each lane owns VEC adjacent
// channels of one (b, chunk), so a wave reads 64*VEC consecutive channels of
// one token per load.
//   forward:  local  - chunk end state with zero carry-in (reads x)
//             carry  - one workgroup per (b, 16 channels) scans the chunk
//                      ends and writes each chunk's carry-in (tiny)
//             apply  - rescans the chunk from its carry-in, writes y
//   backward: the same three stages run in reverse time on dy for the
//             adjoint lambda[t] = dy[t] + (1 - a) lambda[t+1]; the apply
//             stage writes dx = a * lambda and a per-lane partial of
//             dalpha = sum lambda[t] (x[t] - y[t-1]); one workgroup per 16
//             channels sums the partials in a fixed order and applies the
//             projected-clamp rule of ema:357-364.
// The carry and dalpha stages read the [B][NC][D] per-chunk arrays in runs of
// 16 channels (lane = channel within the run) and combine in a fixed order.
// Alpha may be one value (the reference contract, ema:557-558) or one per
// channel; the clamp to [floor, ceiling] happens in-kernel (ema:274-277).
// Optional reset flags [B,N] zero the state before the tokens they mark
// (the reset-aware scan, ema:368-509): the local and apply stages apply them
// inside the chunk, the local stage records whether a chunk contains one, and
// the carry stage gives such a chunk a zero transfer factor.  In reverse
// time a reset at token t + 1 cuts the adjoint flowing into t, and y[t-1]
// does not enter dalpha at a reset token.
#include "ema_common.h"

namespace dwarf {

namespace {

// ---- forward --------------------------------------------------------------
template <typename T, int VEC, bool RESET>
__global__ __launch_bounds__(kEmaBlock) void ema_fwd_local(const T* __restrict__ x, int64_t sxb, int64_t sxn,
                                                          const float* __restrict__ alpha, float* __restrict__ ends,
                                                          EmaGeom g) {
  constexpr int R = kRows<T>;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * kEmaBlock + threadIdx.x;
  const int dv = tid % g.DV;
  const int c = (tid / g.DV) % g.NC;
  const int b = tid / (static_cast<int64_t>(g.DV) * g.NC);
  if (b >= g.B) return;
  const int d0 = dv * VEC;
  float a[VEC], st[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) { a[i] = clamp_alpha(alpha, g, d0 + i); st[i] = 0.f; }
  const int t0 = c * kChunkT;
  const int len = min(kChunkT, g.N - t0);
  const T* p = x + b * sxb + static_cast<int64_t>(t0) * sxn + d0;
  bool cut = false;
  for (int tb = 0; tb < len; tb += R) {
    float xv[R][VEC];
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (tb + r < len) ldv<T, VEC>(p + static_cast<int64_t>(tb + r) * sxn, xv[r]);
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (tb + r < len) {
        if constexpr (RESET) {
          if (reset_at(g, b, t0 + tb + r)) {
            cut = true;
#pragma unroll
            for (int i = 0; i < VEC; ++i) st[i] = 0.f;
          }
        }
#pragma unroll
        for (int i = 0; i < VEC; ++i) st[i] = fmaf(a[i], xv[r][i], (1.f - a[i]) * st[i]);
      }
  }
  float* e = ends + (static_cast<int64_t>(b) * g.NC + c) * g.D + d0;
#pragma unroll
  for (int i = 0; i < VEC; ++i) e[i] = st[i];
  if (RESET && dv == 0) g.cut[b * g.NC + c] = cut;   // a reset in [t0, t0 + len)
}

template <typename T, int VEC, bool RESET>
__global__ __launch_bounds__(kEmaBlock) void ema_fwd_apply(const T* __restrict__ x, int64_t sxb, int64_t sxn,
                                                          T* __restrict__ y, int64_t syb, int64_t syn,
                                                          const float* __restrict__ alpha,
                                                          const float* __restrict__ carries, EmaGeom g) {
  constexpr int R = kRows<T>;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * kEmaBlock + threadIdx.x;
  const int dv = tid % g.DV;
  const int c = (tid / g.DV) % g.NC;
  const int b = tid / (static_cast<int64_t>(g.DV) * g.NC);
  if (b >= g.B) return;
  const int d0 = dv * VEC;
  float a[VEC], st[VEC];
  const float* cr = carries + (static_cast<int64_t>(b) * g.NC + c) * g.D + d0;
#pragma unroll
  for (int i = 0; i < VEC; ++i) { a[i] = clamp_alpha(alpha, g, d0 + i); st[i] = cr[i]; }
  const int t0 = c * kChunkT;
  const int len = min(kChunkT, g.N - t0);
  const T* px = x + b * sxb + static_cast<int64_t>(t0) * sxn + d0;
  T* py = y + b * syb + static_cast<int64_t>(t0) * syn + d0;
  for (int tb = 0; tb < len; tb += R) {
    float xv[R][VEC];
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (tb + r < len) ldv<T, VEC>(px + static_cast<int64_t>(tb + r) * sxn, xv[r]);
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (tb + r < len) {
        if constexpr (RESET) {
          if (reset_at(g, b, t0 + tb + r)) {
#pragma unroll
            for (int i = 0; i < VEC; ++i) st[i] = 0.f;
          }
        }
#pragma unroll
        for (int i = 0; i < VEC; ++i) st[i] = fmaf(a[i], xv[r][i], (1.f - a[i]) * st[i]);
        stv<T, VEC>(py + static_cast<int64_t>(tb + r) * syn, st);
      }
  }
}

// ---- backward -------------------------------------------------------------
template <typename T, int VEC, bool RESET>
__global__ __launch_bounds__(kEmaBlock) void ema_bwd_local(const T* __restrict__ dy, int64_t sgb, int64_t sgn,
                                                          const float* __restrict__ alpha, float* __restrict__ starts,
                                                          EmaGeom g) {
  constexpr int R = kRows<T>;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * kEmaBlock + threadIdx.x;
  const int dv = tid % g.DV;
  const int c = (tid / g.DV) % g.NC;
  const int b = tid / (static_cast<int64_t>(g.DV) * g.NC);
  if (b >= g.B) return;
  const int d0 = dv * VEC;
  float dec[VEC], st[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) { dec[i] = 1.f - clamp_alpha(alpha, g, d0 + i); st[i] = 0.f; }
  const int t0 = c * kChunkT;
  const int len = min(kChunkT, g.N - t0);
  const T* p = dy + b * sgb + static_cast<int64_t>(t0) * sgn + d0;
  for (int tb = len - 1; tb >= 0; tb -= R) {   // rows tb, tb-1, ..., tb-R+1
    float gv[R][VEC];
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (tb - r >= 0) ldv<T, VEC>(p + static_cast<int64_t>(tb - r) * sgn, gv[r]);
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (tb - r >= 0) {
        if constexpr (RESET) {   // a reset at token t + 1 cuts the adjoint flowing back into t
          if (tb - r + 1 < len && reset_at(g, b, t0 + tb - r + 1)) {
#pragma unroll
            for (int i = 0; i < VEC; ++i) st[i] = 0.f;
          }
        }
#pragma unroll
        for (int i = 0; i < VEC; ++i) st[i] = fmaf(dec[i], st[i], gv[r][i]);
      }
  }
  float* e = starts + (static_cast<int64_t>(b) * g.NC + c) * g.D + d0;
#pragma unroll
  for (int i = 0; i < VEC; ++i) e[i] = st[i];
  if (RESET && dv == 0) {   // a reset in [t0 + 1, t0 + len] (tokens inside the sequence)
    bool cut = false;
    for (int t = t0 + 1; t <= t0 + len && t < g.N; ++t) cut = cut || reset_at(g, b, t);
    g.cut[b * g.NC + c] = cut;
  }
}

template <typename T, int VEC, bool RESET>
__global__ __launch_bounds__(kEmaBlock) void ema_bwd_apply(const T* __restrict__ x, int64_t sxb, int64_t sxn,
                                                          const T* __restrict__ y, int64_t syb, int64_t syn,
                                                          const T* __restrict__ dy, int64_t sgb, int64_t sgn,
                                                          T* __restrict__ dx, int64_t sdb, int64_t sdn,
                                                          const float* __restrict__ alpha,
                                                          const float* __restrict__ carries,
                                                          float* __restrict__ da_part, EmaGeom g) {
  constexpr int R = kRows<T> / 2;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * kEmaBlock + threadIdx.x;
  const int dv = tid % g.DV;
  const int c = (tid / g.DV) % g.NC;
  const int b = tid / (static_cast<int64_t>(g.DV) * g.NC);
  if (b >= g.B) return;
  const int d0 = dv * VEC;
  float a[VEC], st[VEC], da[VEC];
  const float* cr = carries + (static_cast<int64_t>(b) * g.NC + c) * g.D + d0;
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    a[i] = clamp_alpha(alpha, g, d0 + i);
    st[i] = cr[i];
    da[i] = 0.f;
  }
  const int t0 = c * kChunkT;
  const int len = min(kChunkT, g.N - t0);
  const T* pg = dy + b * sgb + static_cast<int64_t>(t0) * sgn + d0;
  const T* pxx = x + b * sxb + static_cast<int64_t>(t0) * sxn + d0;
  const T* pyy = y + b * syb + static_cast<int64_t>(t0) * syn + d0;
  T* pd = dx + b * sdb + static_cast<int64_t>(t0) * sdn + d0;
  for (int tb = len - 1; tb >= 0; tb -= R) {
    float gv[R][VEC], xv[R][VEC], yp[R][VEC];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int t = tb - r;
      if (t >= 0) {
        ldv<T, VEC>(pg + static_cast<int64_t>(t) * sgn, gv[r]);
        ldv<T, VEC>(pxx + static_cast<int64_t>(t) * sxn, xv[r]);
        if (t0 + t > 0) {
          ldv<T, VEC>(pyy + static_cast<int64_t>(t - 1) * syn, yp[r]);
        } else {
#pragma unroll
          for (int i = 0; i < VEC; ++i) yp[r][i] = 0.f;
        }
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int t = tb - r;
      if (t >= 0) {
        if constexpr (RESET) {
          if (t0 + t + 1 < g.N && reset_at(g, b, t0 + t + 1)) {   // cut from the future (or the carry)
#pragma unroll
            for (int i = 0; i < VEC; ++i) st[i] = 0.f;
          }
          if (reset_at(g, b, t0 + t)) {   // y[t-1] does not feed token t (ema:445-448)
#pragma unroll
            for (int i = 0; i < VEC; ++i) yp[r][i] = 0.f;
          }
        }
        float out[VEC];
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          st[i] = fmaf(1.f - a[i], st[i], gv[r][i]);
          out[i] = a[i] * st[i];
          da[i] = fmaf(st[i], xv[r][i] - yp[r][i], da[i]);
        }
        stv<T, VEC>(pd + static_cast<int64_t>(t) * sdn, out);
      }
    }
  }
  float* dp = da_part + (static_cast<int64_t>(b) * g.NC + c) * g.D + d0;
#pragma unroll
  for (int i = 0; i < VEC; ++i) dp[i] = da[i];
}

// ---------------------------------------------------------------------------
// Single-pass scan with decoupled look-back (used where every [N][D] slab of
// x, y, dy and dx spans less than 2 GiB, so rows take 32-bit buffer offsets).
//
// A tile is (b, block of 16 VEC channels, 4 SEG = 128 consecutive tokens),
// one wave: lane (cg = lane & 15, ts = lane >> 4) holds channels
// [16 VEC cb + VEC cg, +VEC) of tokens [s0, s0 + SEG), s0 = 4 SEG chunk +
// SEG ts, loaded once into registers.  A workgroup takes kLbWaves tiles that
// follow each other in scan order.  (64-token segments keep twice the rows
// per lane and half the waves: 5 us slower at [4, 8192, 512]; 16-token
// segments give more, shorter waits: 15 us slower.)  Each wave
//   1. scans each lane's segment from a zero state: its end L and its
//      transfer factor A = decay^len (0 when a reset falls inside);
//   2. composes the four segments of a channel in time order into the tile's
//      (P, Q), state after the tile = P s + Q, and each lane's prefix;
// then the workgroup (lb_join)
//   3. composes its tiles' maps in LDS into the workgroup's (P, Q) and
//      publishes Q as its aggregate, tagged with its factor: tag 1 for a full
//      workgroup's decay^(512), tag 3 for P = 0 (a reset inside, or a factor
//      below fp32's range);
//   4. forms the state entering it from the aggregates of the workgroups
//      before it in its run of kLbRun, composed in a fixed order and applied
//      to the inclusive state the previous run's last workgroup publishes
//      (tag 2); every input is published before its writer waits on anything,
//      so the result is the same bits every run; each wave composes its own
//      incoming state from that and the earlier tiles of its workgroup;
// and each wave
//   5. rescans its segments from their incoming states and writes y.
// A workgroup waits only on workgroups of lower index, which the hardware
// dispatches first; the only chain of waits is the runs' inclusive states,
// and it ends at the first run.  Four tiles to a workgroup cut the look-back
// walk fourfold (at [4, 8192, 512] one run of 16 workgroups per slice):
// 18.2 / 30.4 us forward / backward against 23.2 / 32.4 with one tile to a
// workgroup; two or eight tiles measured 20.3 / 32.2 and 18.2 / 31.3.  (A
// counter handing out tile indices in claim order measured 9 us slower: one
// contended atomic per tile.)  A value and its tag share one 64-bit word,
// written and read as one agent-scope atomic (coherent across the XCDs' L2s
// without a fence); `ema_lb_zero` clears the words before each scan.  A wait
// gives up after wait_limit polls and poisons its channel with NaN rather
// than hang.  The backward runs the same scan in reverse time over dy for
// the adjoint lambda, and in its rescan writes dx and each workgroup's dalpha
// partial.
// ---------------------------------------------------------------------------
template <typename T, int VEC, bool RESET>
__global__ __launch_bounds__(kWave * kLbWaves) void ema_fwd_lb(const T* __restrict__ x, int64_t sxb, int64_t sxn,
                                                     T* __restrict__ y, int64_t syb, int64_t syn,
                                                     const float* __restrict__ alpha, LbGeom g) {
  constexpr int SEG = kLbSeg;
  constexpr int CT = kLbGroups * VEC;   // channels (words) per tile
  __shared__ LbShared<1> sh;
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  const int cg = lane & 15, ts = lane >> 4;
  const int id = blockIdx.x;   // workgroups of lower index are dispatched first
  const int widx = id / g.S, slice = id - widx * g.S;
  const int chunk = widx * kLbWaves + w;   // a chunk past the last holds no tokens
  const int b = slice / g.CB, cb = slice - b * g.CB;
  const int d0 = (cb * kLbGroups + cg) * VEC;
  const bool dlive = d0 < g.D;
  const int s0 = (chunk * kLbSegs + ts) * SEG;
  const int len = max(0, min(SEG, g.N - s0));
  float a[VEC], dec[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    a[i] = dlive ? lb_alpha(alpha, g, d0 + i) : 0.f;
    dec[i] = 1.f - a[i];
  }
  const __amdgpu_buffer_rsrc_t rx = lb_rsrc(x, sxb, sxn, b, g.N);
  const uint32_t rsx = static_cast<uint32_t>(sxn * sizeof(T)), cox = static_cast<uint32_t>(d0 * sizeof(T));
  LbRaw<T, VEC> raw[SEG];
#pragma unroll
  for (int t = 0; t < SEG; ++t)
    raw[t].load(rx, t < len && dlive ? static_cast<uint32_t>(s0 + t) * rsx + cox : kOutOfRange);

  uint64_t rb = 0;   // reset flags of tokens s0 .. s0 + SEG
  if constexpr (RESET) rb = lb_reset_bits(g, b, s0);

  // 1. the segment from a zero state
  float L[VEC], A[VEC];
  bool cut = false;
#pragma unroll
  for (int i = 0; i < VEC; ++i) { L[i] = 0.f; A[i] = 1.f; }
#pragma unroll
  for (int t = 0; t < SEG; ++t) {
    if (t < len) {
      if constexpr (RESET) {
        if (lb_bit(rb, t)) {
          cut = true;
#pragma unroll
          for (int i = 0; i < VEC; ++i) L[i] = 0.f;
        }
      }
      float v[VEC];
      raw[t].widen(v);
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        L[i] = fmaf(a[i], v[i], dec[i] * L[i]);
        A[i] *= dec[i];
      }
    }
  }
  if (cut) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) A[i] = 0.f;
  }
  // 2. the four segments of each channel in time order: the tile's (P, Q) and this lane's prefix
  float P[VEC], Q[VEC], Pp[VEC], Qp[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) { P[i] = 1.f; Q[i] = 0.f; Pp[i] = 1.f; Qp[i] = 0.f; }
#pragma unroll
  for (int k = 0; k < kLbSegs; ++k) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      const float Ak = __shfl(A[i], cg + 16 * k), Lk = __shfl(L[i], cg + 16 * k);
      Pp[i] = k == ts ? P[i] : Pp[i];
      Qp[i] = k == ts ? Q[i] : Qp[i];
      Q[i] = fmaf(Ak, Q[i], Lk);
      P[i] *= Ak;
    }
  }
  // 3-4. the channel this lane publishes (VEC 4: channel ts of the group; VEC 1: lanes ts = 0)
  float full = 1.f;   // a full tile's factor, composed as a tile composes its segments
  const int io = VEC == 4 ? ts : 0;
  const bool owner = (VEC == 4 || ts == 0) && dlive && d0 + io < g.D;
  const float dec_o = VEC == 4 ? pick4(io, dec[0], dec[VEC > 1 ? 1 : 0], dec[VEC > 2 ? 2 : 0], dec[VEC > 3 ? 3 : 0])
                               : dec[0];
  const float Po = VEC == 4 ? pick4(io, P[0], P[VEC > 1 ? 1 : 0], P[VEC > 2 ? 2 : 0], P[VEC > 3 ? 3 : 0]) : P[0];
  const float Qo = VEC == 4 ? pick4(io, Q[0], Q[VEC > 1 ? 1 : 0], Q[VEC > 2 ? 2 : 0], Q[VEC > 3 ? 3 : 0]) : Q[0];
  {
    float seg = 1.f;
    for (int t = 0; t < SEG; ++t) seg *= dec_o;
#pragma unroll
    for (int k = 0; k < kLbSegs; ++k) full *= seg;
  }
  float full_wg = 1.f;   // a full workgroup's factor, composed as wave 0 composes the tiles
#pragma unroll
  for (int j = 0; j < kLbWaves; ++j) full_wg *= full;
  float C;
  lb_join<1>(g, sh, slice, cg * VEC + io, owner, CT, widx, w, &Po, &Qo, &full_wg, &C);
  // 5. incoming state of each channel of this lane's segment, then the rescan
  float st[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    const float Ci = __shfl(C, VEC == 4 ? cg + 16 * i : cg);
    st[i] = fmaf(Pp[i], Ci, Qp[i]);
  }
  const __amdgpu_buffer_rsrc_t ry = lb_rsrc(y, syb, syn, b, g.N);
  const uint32_t rsy = static_cast<uint32_t>(syn * sizeof(T)), coy = static_cast<uint32_t>(d0 * sizeof(T));
#pragma unroll
  for (int t = 0; t < SEG; ++t) {
    if (t < len) {
      if constexpr (RESET) {
        if (lb_bit(rb, t)) {
#pragma unroll
          for (int i = 0; i < VEC; ++i) st[i] = 0.f;
        }
      }
      float v[VEC];
      raw[t].widen(v);
#pragma unroll
      for (int i = 0; i < VEC; ++i) st[i] = fmaf(a[i], v[i], dec[i] * st[i]);
      lb_store<T, VEC>(ry, dlive ? static_cast<uint32_t>(s0 + t) * rsy + coy : kOutOfRange, st);
    }
  }
}

template <typename T, int VEC, bool RESET>
__global__ __launch_bounds__(kWave * kLbWaves) void ema_bwd_lb(const T* __restrict__ x, int64_t sxb, int64_t sxn,
                                                     const T* __restrict__ y, int64_t syb, int64_t syn,
                                                     const T* __restrict__ dy, int64_t sgb, int64_t sgn,
                                                     T* __restrict__ dx, int64_t sdb, int64_t sdn,
                                                     const float* __restrict__ alpha, LbGeom g) {
  constexpr int SEG = kLbSeg;
  constexpr int CT = kLbGroups * VEC;
  constexpr int R = 8;   // rows of x and y loaded per block of the rescan
  __shared__ LbShared<1> sh;
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  const int cg = lane & 15, ts = lane >> 4;
  const int id = blockIdx.x;   // workgroups of lower index are dispatched first
  const int widx = id / g.S, slice = id - widx * g.S;   // workgroup tiles in reverse time order
  const int chunk = g.NCH - 1 - (widx * kLbWaves + w);   // a chunk below 0 holds no tokens
  const int b = slice / g.CB, cb = slice - b * g.CB;
  const int d0 = (cb * kLbGroups + cg) * VEC;
  const bool dlive = d0 < g.D;
  const int s0 = (chunk * kLbSegs + ts) * SEG;
  const int len = chunk < 0 ? 0 : max(0, min(SEG, g.N - s0));
  float a[VEC], dec[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    a[i] = dlive ? lb_alpha(alpha, g, d0 + i) : 0.f;
    dec[i] = 1.f - a[i];
  }
  const __amdgpu_buffer_rsrc_t rg = lb_rsrc(dy, sgb, sgn, b, g.N);
  const uint32_t rsg = static_cast<uint32_t>(sgn * sizeof(T)), cog = static_cast<uint32_t>(d0 * sizeof(T));
  LbRaw<T, VEC> raw[SEG];
#pragma unroll
  for (int t = 0; t < SEG; ++t)
    raw[t].load(rg, t < len && dlive ? static_cast<uint32_t>(s0 + t) * rsg + cog : kOutOfRange);

  uint64_t rb = 0;   // reset flags of tokens s0 .. s0 + SEG
  if constexpr (RESET) rb = lb_reset_bits(g, b, s0);

  // 1. the segment in reverse time from a zero adjoint; a reset at token
  // t + 1 cuts what flows from t + 1 back into t (ema:478-509)
  float L[VEC], A[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) { L[i] = 0.f; A[i] = 1.f; }
#pragma unroll
  for (int t = SEG - 1; t >= 0; --t) {
    if (t < len) {
      if constexpr (RESET) {
        if (t + 1 < len && lb_bit(rb, t + 1)) {
#pragma unroll
          for (int i = 0; i < VEC; ++i) L[i] = 0.f;
        }
      }
      float v[VEC];
      raw[t].widen(v);
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        L[i] = fmaf(dec[i], L[i], v[i]);
        A[i] *= dec[i];
      }
    }
  }
  if constexpr (RESET) {   // a reset at any of s0 + 1 .. s0 + len cuts the segment's carry (bits past N are 0)
    const bool cut = len > 0 && ((rb >> 1) & ((uint64_t(1) << len) - 1)) != 0;
    if (cut) {
#pragma unroll
      for (int i = 0; i < VEC; ++i) A[i] = 0.f;
    }
  }
  // 2. segments composed in reverse time order (3, 2, 1, 0)
  float P[VEC], Q[VEC], Pp[VEC], Qp[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) { P[i] = 1.f; Q[i] = 0.f; Pp[i] = 1.f; Qp[i] = 0.f; }
#pragma unroll
  for (int k = kLbSegs - 1; k >= 0; --k) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      const float Ak = __shfl(A[i], cg + 16 * k), Lk = __shfl(L[i], cg + 16 * k);
      Pp[i] = k == ts ? P[i] : Pp[i];
      Qp[i] = k == ts ? Q[i] : Qp[i];
      Q[i] = fmaf(Ak, Q[i], Lk);
      P[i] *= Ak;
    }
  }
  // 3-4. publish and walk back over the later tiles
  const int io = VEC == 4 ? ts : 0;
  const bool owner = (VEC == 4 || ts == 0) && dlive && d0 + io < g.D;
  const float dec_o = VEC == 4 ? pick4(io, dec[0], dec[VEC > 1 ? 1 : 0], dec[VEC > 2 ? 2 : 0], dec[VEC > 3 ? 3 : 0])
                               : dec[0];
  const float Po = VEC == 4 ? pick4(io, P[0], P[VEC > 1 ? 1 : 0], P[VEC > 2 ? 2 : 0], P[VEC > 3 ? 3 : 0]) : P[0];
  const float Qo = VEC == 4 ? pick4(io, Q[0], Q[VEC > 1 ? 1 : 0], Q[VEC > 2 ? 2 : 0], Q[VEC > 3 ? 3 : 0]) : Q[0];
  float full = 1.f;
  {
    float seg = 1.f;
    for (int t = 0; t < SEG; ++t) seg *= dec_o;
#pragma unroll
    for (int k = 0; k < kLbSegs; ++k) full *= seg;
  }
  float full_wg = 1.f;   // a full workgroup's factor, composed as wave 0 composes the tiles
#pragma unroll
  for (int j = 0; j < kLbWaves; ++j) full_wg *= full;
  // predecessors: workgroup tiles widx - 1, ..., 0, i.e. the chunks after this workgroup's
  float C;
  lb_join<1>(g, sh, slice, cg * VEC + io, owner, CT, widx, w, &Po, &Qo, &full_wg, &C);
  // 5. rescan: lambda from the incoming adjoint, dx = a lambda, dalpha terms
  float st[VEC], da[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    const float Ci = __shfl(C, VEC == 4 ? cg + 16 * i : cg);
    st[i] = fmaf(Pp[i], Ci, Qp[i]);
    da[i] = 0.f;
  }
  const __amdgpu_buffer_rsrc_t rx = lb_rsrc(x, sxb, sxn, b, g.N);
  const __amdgpu_buffer_rsrc_t ry = lb_rsrc(y, syb, syn, b, g.N);
  const __amdgpu_buffer_rsrc_t rd = lb_rsrc(dx, sdb, sdn, b, g.N);
  const uint32_t rsx = static_cast<uint32_t>(sxn * sizeof(T)), cox = static_cast<uint32_t>(d0 * sizeof(T));
  const uint32_t rsy = static_cast<uint32_t>(syn * sizeof(T)), coy = static_cast<uint32_t>(d0 * sizeof(T));
  const uint32_t rsd = static_cast<uint32_t>(sdn * sizeof(T)), cod = static_cast<uint32_t>(d0 * sizeof(T));
#pragma unroll
  for (int tb = SEG - 1; tb >= 0; tb -= R) {
    LbRaw<T, VEC> xr[R], yr[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int t = tb - r;
      const bool ok = t < len && dlive;
      xr[r].load(rx, ok ? static_cast<uint32_t>(s0 + t) * rsx + cox : kOutOfRange);
      // y[t - 1]; before token 0 the state is zero (the offset wraps out of range)
      yr[r].load(ry, ok && s0 + t > 0 ? static_cast<uint32_t>(s0 + t - 1) * rsy + coy : kOutOfRange);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int t = tb - r;
      if (t < len) {
        float xv[VEC], yp[VEC], gv[VEC];
        xr[r].widen(xv);
        yr[r].widen(yp);
        raw[t].widen(gv);
        if constexpr (RESET) {
          if (lb_bit(rb, t + 1)) {   // cut from the future (or the carry; 0 past N)
#pragma unroll
            for (int i = 0; i < VEC; ++i) st[i] = 0.f;
          }
          if (lb_bit(rb, t)) {   // y[t-1] does not feed token t (ema:445-448)
#pragma unroll
            for (int i = 0; i < VEC; ++i) yp[i] = 0.f;
          }
        }
        float out[VEC];
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          st[i] = fmaf(dec[i], st[i], gv[i]);
          out[i] = a[i] * st[i];
          da[i] = fmaf(st[i], xv[i] - yp[i], da[i]);
        }
        lb_store<T, VEC>(rd, dlive ? static_cast<uint32_t>(s0 + t) * rsd + cod : kOutOfRange, out);
      }
    }
  }
  // the workgroup's dalpha partial of each channel: each tile's four segments in time order, then the
  // tiles in time order (waves kLbWaves - 1, ..., 0; a tile without tokens adds zero)
  __shared__ float sda[kLbWaves][kWave];
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < kLbSegs; ++k) s += __shfl(da[i], cg + 16 * k);
    if (ts == 0) sda[w][cg * VEC + i] = s;
  }
  __syncthreads();
  if (w == 0 && ts == 0) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      float s = 0.f;
#pragma unroll
      for (int j = kLbWaves - 1; j >= 0; --j) s += sda[j][cg * VEC + i];
      if (dlive && d0 + i < g.D) g.da_part[(static_cast<int64_t>(widx) * g.B + b) * g.D + d0 + i] = s;
    }
  }
}

inline size_t round256(size_t n) { return (n + 255) / 256 * 256; }

// Workspace of the look-back scans: a zero head, the words and, backward,
// the dalpha partials [NWG][B][D] and D channel sums.
inline size_t lb_workspace(int B, int N, int D, bool backward) {
  const LbPlan p = lb_plan(B, N, D, D % 4 == 0 ? 4 : 1, kLbSeg);
  size_t n = kLbHead + round256(p.words_bytes);
  if (backward) n += round256(static_cast<size_t>(p.NWG) * B * D * 4) + round256(static_cast<size_t>(D) * 4);
  return n;
}

template <typename T, int VEC>
LbGeom lb_geom(int B, int N, int D, int per_channel, float lo, float hi, const uint8_t* reset, const int64_t* rs,
               void* ws, int wait_limit, bool backward, LbPlan* plan) {
  const LbPlan p = lb_plan(B, N, D, VEC, kLbSeg);
  LbGeom g;
  g.B = B; g.N = N; g.D = D;
  g.CB = p.CB; g.NCH = p.NCH; g.NWG = p.NWG; g.S = p.S;
  g.per_channel = per_channel;
  g.lo = lo; g.hi = hi;
  g.reset = reset;
  g.srb = reset ? rs[0] : 0;
  g.srn = reset ? rs[1] : 0;
  char* w = static_cast<char*>(ws);
  g.words = reinterpret_cast<unsigned long long*>(w + kLbHead);
  g.runs = g.words + p.kw;
  g.kw = p.kw;
  g.kr = p.kr;
  g.da_part = backward ? reinterpret_cast<float*>(w + kLbHead + round256(p.words_bytes)) : nullptr;
  g.wait_limit = wait_limit > 0 ? wait_limit : kLbWaitLimit;
  *plan = p;
  return g;
}

template <typename T, int VEC, bool RESET>
hipError_t ema_fwd_typed(const dwarf_ema_fwd_args& a, hipStream_t stream) {
  const T* x = static_cast<const T*>(a.x);
  T* y = static_cast<T*>(a.y);
  if (lb_fits(a.N, a.x_stride[1], sizeof(T)) && lb_fits(a.N, a.y_stride[1], sizeof(T))) {
    LbPlan p;
    const LbGeom g = lb_geom<T, VEC>(a.B, a.N, a.D, a.alpha_per_channel, a.floor_, a.ceiling, a.reset,
                                     a.reset_stride, a.workspace, a.wait_limit, false, &p);
    lb_zero(g, p, stream);
    hipLaunchKernelGGL((ema_fwd_lb<T, VEC, RESET>), dim3(p.NWG * p.S), dim3(kWave * kLbWaves), 0, stream, x, a.x_stride[0],
                       a.x_stride[1], y, a.y_stride[0], a.y_stride[1], a.alpha, g);
    return hipGetLastError();
  }
  // three-stage chunked scan (local, carry, apply) for larger slabs
  const size_t nf = ws_floats(a.B, a.N, a.D);
  const EmaGeom g = make_geom(a.B, a.N, a.D, VEC, a.alpha_per_channel, a.floor_, a.ceiling, a.reset,
                              a.reset_stride, a.workspace, 2 * nf);
  float* ends = static_cast<float*>(a.workspace);
  float* carries = ends + nf;
  const int64_t lanes = static_cast<int64_t>(a.B) * g.NC * g.DV;
  const int blocks = static_cast<int>((lanes + kEmaBlock - 1) / kEmaBlock);
  hipLaunchKernelGGL((ema_fwd_local<T, VEC, RESET>), dim3(blocks), dim3(kEmaBlock), 0, stream, x, a.x_stride[0],
                     a.x_stride[1], a.alpha, ends, g);
  launch_carry<false, RESET>(ends, carries, a.alpha, g, a.B, a.D, stream);
  hipLaunchKernelGGL((ema_fwd_apply<T, VEC, RESET>), dim3(blocks), dim3(kEmaBlock), 0, stream, x, a.x_stride[0],
                     a.x_stride[1], y, a.y_stride[0], a.y_stride[1], a.alpha, carries, g);
  return hipGetLastError();
}

// dalpha from per-row partials [rows][D] (rows = B * nc): per channel, or summed over the channels.
inline void launch_dalpha(const float* da_part, const float* alpha, float* dalpha, float* chan, const EmaGeom& g,
                          int per_channel, int D, hipStream_t stream) {
  const int rb = (D + kDaChannels - 1) / kDaChannels;
  if (per_channel) {
    hipLaunchKernelGGL(ema_dalpha_channels, dim3(rb), dim3(kWave * kCarryWaves), 0, stream, da_part, alpha, dalpha,
                       g);
  } else {
    hipLaunchKernelGGL(ema_dalpha_channels, dim3(rb), dim3(kWave * kCarryWaves), 0, stream, da_part, alpha, chan, g);
    hipLaunchKernelGGL(ema_dalpha_scalar, dim3(1), dim3(kWave), 0, stream, chan, alpha, dalpha, g);
  }
}

template <typename T, int VEC, bool RESET>
hipError_t ema_bwd_typed(const dwarf_ema_bwd_args& a, hipStream_t stream) {
  const T* x = static_cast<const T*>(a.x);
  const T* y = static_cast<const T*>(a.y);
  const T* dy = static_cast<const T*>(a.dy);
  T* dx = static_cast<T*>(a.dx);
  if (lb_fits(a.N, a.x_stride[1], sizeof(T)) && lb_fits(a.N, a.y_stride[1], sizeof(T)) &&
      lb_fits(a.N, a.dy_stride[1], sizeof(T)) && lb_fits(a.N, a.dx_stride[1], sizeof(T))) {
    LbPlan p;
    const LbGeom g = lb_geom<T, VEC>(a.B, a.N, a.D, a.alpha_per_channel, a.floor_, a.ceiling, a.reset,
                                     a.reset_stride, a.workspace, a.wait_limit, true, &p);
    lb_zero(g, p, stream);
    hipLaunchKernelGGL((ema_bwd_lb<T, VEC, RESET>), dim3(p.NWG * p.S), dim3(kWave * kLbWaves), 0, stream, x, a.x_stride[0],
                       a.x_stride[1], y, a.y_stride[0], a.y_stride[1], dy, a.dy_stride[0], a.dy_stride[1], dx,
                       a.dx_stride[0], a.dx_stride[1], a.alpha, g);
    if (a.dalpha) {
      // the partials' rows are (workgroup tile, b): the reduction's geometry with NC = NWG
      EmaGeom eg = make_geom(a.B, p.NWG * kChunkT, a.D, VEC, a.alpha_per_channel, a.floor_, a.ceiling, nullptr,
                             nullptr, a.workspace, 0);
      float* chan = g.da_part + round256(static_cast<size_t>(p.NWG) * a.B * a.D * 4) / 4;
      launch_dalpha(g.da_part, a.alpha, a.dalpha, chan, eg, a.alpha_per_channel, a.D, stream);
    }
    return hipGetLastError();
  }
  const size_t nf = ws_floats(a.B, a.N, a.D);
  const EmaGeom g = make_geom(a.B, a.N, a.D, VEC, a.alpha_per_channel, a.floor_, a.ceiling, a.reset,
                              a.reset_stride, a.workspace, 3 * nf);
  float* starts = static_cast<float*>(a.workspace);
  float* carries = starts + nf;
  float* da_part = carries + nf;
  const int64_t lanes = static_cast<int64_t>(a.B) * g.NC * g.DV;
  const int blocks = static_cast<int>((lanes + kEmaBlock - 1) / kEmaBlock);
  hipLaunchKernelGGL((ema_bwd_local<T, VEC, RESET>), dim3(blocks), dim3(kEmaBlock), 0, stream, dy, a.dy_stride[0],
                     a.dy_stride[1], a.alpha, starts, g);
  launch_carry<true, RESET>(starts, carries, a.alpha, g, a.B, a.D, stream);
  hipLaunchKernelGGL((ema_bwd_apply<T, VEC, RESET>), dim3(blocks), dim3(kEmaBlock), 0, stream, x, a.x_stride[0],
                     a.x_stride[1], y, a.y_stride[0], a.y_stride[1], dy, a.dy_stride[0], a.dy_stride[1], dx,
                     a.dx_stride[0], a.dx_stride[1], a.alpha, carries, da_part, g);
  if (a.dalpha) launch_dalpha(da_part, a.alpha, a.dalpha, starts, g, a.alpha_per_channel, a.D, stream);
  return hipGetLastError();
}

}  // namespace

size_t ema_fwd_workspace(int B, int N, int D) {
  const size_t chunked = 2 * ws_floats(B, N, D) * sizeof(float) + ws_cut_bytes(B, N);
  const size_t lb = lb_workspace(B, N, D, false);
  return chunked > lb ? chunked : lb;
}
size_t ema_bwd_workspace(int B, int N, int D) {
  const size_t chunked = 3 * ws_floats(B, N, D) * sizeof(float) + ws_cut_bytes(B, N);
  const size_t lb = lb_workspace(B, N, D, true);
  return chunked > lb ? chunked : lb;
}

template <bool RESET>
hipError_t launch_ema_fwd_r(const dwarf_ema_fwd_args& a, hipStream_t stream) {
  const bool vec4 = (a.D % 4) == 0;
  if (a.dtype == DWARF_BF16)
    return vec4 ? ema_fwd_typed<bf16, 4, RESET>(a, stream) : ema_fwd_typed<bf16, 1, RESET>(a, stream);
  return vec4 ? ema_fwd_typed<float, 4, RESET>(a, stream) : ema_fwd_typed<float, 1, RESET>(a, stream);
}

template <bool RESET>
hipError_t launch_ema_bwd_r(const dwarf_ema_bwd_args& a, hipStream_t stream) {
  const bool vec4 = (a.D % 4) == 0;
  if (a.dtype == DWARF_BF16)
    return vec4 ? ema_bwd_typed<bf16, 4, RESET>(a, stream) : ema_bwd_typed<bf16, 1, RESET>(a, stream);
  return vec4 ? ema_bwd_typed<float, 4, RESET>(a, stream) : ema_bwd_typed<float, 1, RESET>(a, stream);
}

hipError_t launch_ema_fwd(const dwarf_ema_fwd_args& a, hipStream_t stream) {
  return a.reset ? launch_ema_fwd_r<true>(a, stream) : launch_ema_fwd_r<false>(a, stream);
}

hipError_t launch_ema_bwd(const dwarf_ema_bwd_args& a, hipStream_t stream) {
  return a.reset ? launch_ema_bwd_r<true>(a, stream) : launch_ema_bwd_r<false>(a, stream);
}

}  // namespace dwarf
