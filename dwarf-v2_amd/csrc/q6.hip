// q6 K/V cache: codec, prefill forward and decode step.
//
// Format (no counterpart in the reference repository):
// a head-dim row of 64 values is two groups of 32.  Per group
//   scale = fp16_rne(absmax / 31)   (fp32 division; +inf saturates to 65504)
//   code  = clamp(rint(x / float(scale)), -31, 31), 0 when scale == 0
// Codes are packed 4 per 24-bit little-endian word, w = sum (c_i & 63) << 6i,
// so element e of a group sits at bits [6e, 6e+6) of the group's 24 bytes.
// dequant(e) = float(sign_extend6(code)) * float(scale), exact in fp32.
//
// Cache slot, one per (b, kv head, t), 128 bytes:
//   [0,48) K codes   [48,52) K scales   [52,100) V codes   [100,104) V scales
//   [104,120) z[4] fp32 (key-probe features of the dequantised K row)
//   [120,128) zero
// A gathered offset therefore reads exactly one 128-byte line.
//
// Widened row (the prefill's workspace), one per cache slot, 160 bytes:
//   [0,64) K codes as bytes c + 32   [64,128) V codes as bytes c + 32
//   [128,160) per 16-dim chunk g: the fp16 K and V scales of its group and z[g]
// Byte c + 32 is the 6-bit field with its sign bit flipped (1..63).
#include <mutex>
#include <type_traits>

#include "common.h"
#include "dsqg_internal.h"
#include "gather.h"
#include "mfma.h"

namespace dwarf {
namespace {

constexpr int kSlot = DWARF_Q6_SLOT_BYTES;
constexpr int kGroup = DWARF_Q6_GROUP;
constexpr int kKCodes = 0, kKScales = 48, kVCodes = 52, kVScales = 100, kZ = 104;

__device__ __forceinline__ float half_bits_to_f32(uint16_t hbits) {
  return static_cast<float>(__builtin_bit_cast(_Float16, hbits));
}

// Quantise one group of 32 fp32 values; returns the fp16 scale bits.
__device__ __forceinline__ uint16_t q6_quantize_group(const float* x, uint8_t* codes24) {
  float amax = 0.f;
#pragma unroll
  for (int e = 0; e < kGroup; ++e) amax = fmaxf(amax, fabsf(x[e]));
  const _Float16 hs = static_cast<_Float16>(__fdiv_rn(amax, 31.f));  // round to nearest even
  uint16_t sbits = __builtin_bit_cast(uint16_t, hs);
  if ((sbits & 0x7fffu) == 0x7c00u) sbits = (sbits & 0x8000u) | 0x7bffu;  // saturate +inf
  const float sc = half_bits_to_f32(sbits);
  uint32_t w = 0;
#pragma unroll
  for (int e = 0; e < kGroup; ++e) {
    int c = 0;
    if (sc != 0.f) {
      const float r = rintf(__fdiv_rn(x[e], sc));
      c = static_cast<int>(fminf(fmaxf(r, -31.f), 31.f));
    }
    w |= (static_cast<uint32_t>(c) & 63u) << (6 * (e & 3));
    if ((e & 3) == 3) {
      const int k = e >> 2;
      codes24[3 * k + 0] = static_cast<uint8_t>(w);
      codes24[3 * k + 1] = static_cast<uint8_t>(w >> 8);
      codes24[3 * k + 2] = static_cast<uint8_t>(w >> 16);
      w = 0;
    }
  }
  return sbits;
}

// 32 signed codes of one group from its 24 bytes (6 dwords, 4-byte aligned).
__device__ __forceinline__ void q6_codes(const uint8_t* p, float* c) {
  uint32_t dw[7];
  const uint32_t* p32 = reinterpret_cast<const uint32_t*>(p);
#pragma unroll
  for (int i = 0; i < 6; ++i) dw[i] = p32[i];
  dw[6] = 0;
#pragma unroll
  for (int e = 0; e < kGroup; ++e) {
    const int bit = 6 * e;
    const int i = bit >> 5, sh = bit & 31;
    const uint64_t pair = (static_cast<uint64_t>(dw[i + 1]) << 32) | dw[i];
    const int v = static_cast<int>(static_cast<uint32_t>(pair >> sh) << 26) >> 26;
    c[e] = static_cast<float>(v);
  }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void q6_pack_kernel(int B, int Hkv, int N, const T* __restrict__ k,
                                                         const int64_t* ks, const T* __restrict__ v,
                                                         const int64_t* vs, uint8_t* __restrict__ cache,
                                                         const int64_t* cs, const float* __restrict__ kprobe,
                                                         int64_t ks0, int64_t ks1, int64_t ks2, int64_t vs0,
                                                         int64_t vs1, int64_t vs2, int64_t cs0, int64_t cs1,
                                                         int64_t cs2) {
  (void)ks; (void)vs; (void)cs;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (idx >= static_cast<int64_t>(B) * Hkv * N) return;
  const int t = idx % N;
  const int hk = (idx / N) % Hkv;
  const int b = idx / (static_cast<int64_t>(N) * Hkv);
  float kr[kHeadDim], vr[kHeadDim];
  load_f32<T, kHeadDim>(k + b * ks0 + hk * ks1 + static_cast<int64_t>(t) * ks2, kr);
  load_f32<T, kHeadDim>(v + b * vs0 + hk * vs1 + static_cast<int64_t>(t) * vs2, vr);
  alignas(16) uint8_t slot[kSlot];
#pragma unroll
  for (int i = 0; i < kSlot; ++i) slot[i] = 0;
  uint16_t sk0 = q6_quantize_group(kr, slot + kKCodes);
  uint16_t sk1 = q6_quantize_group(kr + kGroup, slot + kKCodes + 24);
  uint16_t sv0 = q6_quantize_group(vr, slot + kVCodes);
  uint16_t sv1 = q6_quantize_group(vr + kGroup, slot + kVCodes + 24);
  slot[kKScales + 0] = sk0 & 0xff; slot[kKScales + 1] = sk0 >> 8;
  slot[kKScales + 2] = sk1 & 0xff; slot[kKScales + 3] = sk1 >> 8;
  slot[kVScales + 0] = sv0 & 0xff; slot[kVScales + 1] = sv0 >> 8;
  slot[kVScales + 2] = sv1 & 0xff; slot[kVScales + 3] = sv1 >> 8;
  if (kprobe) {
    // z from the dequantised K row, as the prefill/decode kernels see it.
    float kq[kHeadDim];
    q6_codes(slot + kKCodes, kq);
    q6_codes(slot + kKCodes + 24, kq + kGroup);
    const float s0 = half_bits_to_f32(sk0), s1 = half_bits_to_f32(sk1);
    float ss = 0.f;
#pragma unroll
    for (int d = 0; d < kHeadDim; ++d) {
      kq[d] *= d < kGroup ? s0 : s1;
      ss = fmaf(kq[d], kq[d], ss);
    }
    const float inv = rsqrtf(ss + 1e-6f * kHeadDim);
    float z[4];
#pragma unroll
    for (int r = 0; r < kPlanes; ++r) {
      float acc = 0.f;
      for (int d = 0; d < kHeadDim; ++d) acc = fmaf(kq[d], kprobe[r * kHeadDim + d], acc);
      z[r] = acc * inv;
    }
    float* zp = reinterpret_cast<float*>(slot + kZ);
    zp[0] = z[0]; zp[1] = z[1]; zp[2] = z[2]; zp[3] = z[3];
  }
  uint4* dst = reinterpret_cast<uint4*>(cache + b * cs0 + hk * cs1 + static_cast<int64_t>(t) * cs2);
  const uint4* src = reinterpret_cast<const uint4*>(slot);
#pragma unroll
  for (int i = 0; i < kSlot / 16; ++i) dst[i] = src[i];
}

__global__ __launch_bounds__(kBlock) void q6_unpack_kernel(int B, int Hkv, int N, const uint8_t* __restrict__ cache,
                                                           int64_t cs0, int64_t cs1, int64_t cs2,
                                                           float* __restrict__ kout, float* __restrict__ vout) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  const int64_t rows = static_cast<int64_t>(B) * Hkv * N;
  if (idx >= rows * 4) return;
  const int part = idx % 4;  // K g0, K g1, V g0, V g1
  const int64_t row = idx / 4;
  const int t = row % N;
  const int hk = (row / N) % Hkv;
  const int b = row / (static_cast<int64_t>(N) * Hkv);
  const uint8_t* slot = cache + b * cs0 + hk * cs1 + static_cast<int64_t>(t) * cs2;
  const int grp = part & 1;
  const bool is_v = part >= 2;
  const uint8_t* codes = slot + (is_v ? kVCodes : kKCodes) + 24 * grp;
  const uint16_t sb = *reinterpret_cast<const uint16_t*>(slot + (is_v ? kVScales : kKScales) + 2 * grp);
  const float sc = half_bits_to_f32(sb);
  float c[kGroup];
  q6_codes(codes, c);
  float* dst = (is_v ? vout : kout) + row * kHeadDim + grp * kGroup;
#pragma unroll
  for (int e = 0; e < kGroup; ++e) dst[e] = c[e] * sc;
}

// Slot reads shared by prefill and decode.
__device__ __forceinline__ uint32_t cache_dword(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}

// Sixteen signed 6-bit codes of a 12-byte chunk (bits [6i, 6i+6) of w0:w1:w2).
// v_bfe_i32 sign-extends the field; the builtin is typed unsigned, so the
// result is reinterpreted as int before the conversion to float.
__device__ __forceinline__ float sfield6(uint32_t w, int bit) {
  return static_cast<float>(static_cast<int>(__builtin_amdgcn_sbfe(w, bit, 6)));
}

__device__ __forceinline__ void q6_codes16(uint32_t w0, uint32_t w1, uint32_t w2, float* c) {
#pragma unroll
  for (int i = 0; i < 5; ++i) c[i] = sfield6(w0, 6 * i);
  c[5] = sfield6(__builtin_amdgcn_alignbit(w1, w0, 30), 0);
#pragma unroll
  for (int i = 6; i < 10; ++i) c[i] = sfield6(w1, 6 * i - 32);
  c[10] = sfield6(__builtin_amdgcn_alignbit(w2, w1, 28), 0);
#pragma unroll
  for (int i = 11; i < 16; ++i) c[i] = sfield6(w2, 6 * i - 64);
}

// The bf16 pair (160 + c_a, 160 + c_b) of the two 6-bit codes in bits
// [0, 12) of t (c_a low): code c in two's complement with its sign bit
// flipped is c + 32, and bf16 0x4300 | m is 128 + m.
__device__ __forceinline__ uint32_t code_pair_bf16(uint32_t t) {
  const uint32_t f = t & 0xfffu;
  return ((f | (f << 10)) & 0x003f003fu) ^ 0x43204320u;
}

// sum_d q_d (160 + c_d) over the 16 codes of a 12-byte chunk, on bf16 pairs.
__device__ __forceinline__ float q6_dot16_biased(const uint32_t* q32, uint32_t w0, uint32_t w1, uint32_t w2) {
  float s = 0.f;
  s = dot2bf(q32[0], code_pair_bf16(w0), s);
  s = dot2bf(q32[1], code_pair_bf16(w0 >> 12), s);
  s = dot2bf(q32[2], code_pair_bf16(__builtin_amdgcn_alignbit(w1, w0, 24)), s);
  s = dot2bf(q32[3], code_pair_bf16(w1 >> 4), s);
  s = dot2bf(q32[4], code_pair_bf16(w1 >> 16), s);
  s = dot2bf(q32[5], code_pair_bf16(__builtin_amdgcn_alignbit(w2, w1, 28)), s);
  s = dot2bf(q32[6], code_pair_bf16(w2 >> 8), s);
  s = dot2bf(q32[7], code_pair_bf16(w2 >> 20), s);
  return s;
}

__device__ __forceinline__ float half_lo_or_hi(uint32_t pair, bool hi) {
  return half_bits_to_f32(static_cast<uint16_t>(hi ? pair >> 16 : pair));
}

// ---------------------------------------------------------------------------
// Prefill forward, four lanes per query (the bf16 forward's mapping).
//
// A workgroup of 4 waves handles 64 queries of one (b, h); lane c of a query
// holds head dims [16c, 16c+16).  A gathered slot is read as the lane's 12
// bytes of K codes and of V codes, the two fp16 scale pairs and (far offsets)
// its z plane, so the four lanes of a query read one 128-byte slot.  q.k is
// formed on the codes as biased bf16 pairs (q6_dot16_biased) and scaled once
// by the fp16 group scale; the V codes are widened to fp32 (v_bfe_i32),
// rotated (MOVT pair of plane c) and accumulated with weight P * scale.
// <q, e_j> + pb_j for the wave's 16 queries and all offsets is one MFMA pass
// at the start (E staged in bf16, as the GPU path rounds it).  y is computed
// in-kernel from q and the query probes (dsqg:3234-3249); z is read from the
// slot.  Each wave walks its list of offsets with a source for one of its
// queries, the next offset's slot reads in flight.
// ---------------------------------------------------------------------------
constexpr int kPfQPW = 16;          // queries per wave
constexpr int kPfQPB = 64;          // queries per workgroup
constexpr int kPfERow = 72;         // bf16 E row stride (elements)
constexpr int kPfMaxBlocks = 17;    // JE / 16 for J <= 256 plus the sentinel

struct PfLayout {
  int JE, JL4, qe_row, list_len;
  size_t off_ph, off_qp, off_list, off_big, bytes;
};

__host__ __device__ inline PfLayout pf_layout(int J, int J_large) {
  PfLayout L;
  L.JE = (J + 1 + 15) / 16 * 16;
  L.JL4 = (J_large + 1) / 2 * 2;
  L.qe_row = L.JE + 4;
  L.list_len = (L.JE + 4 + 1) / 2 * 2;
  L.off_ph = static_cast<size_t>(2 * L.JE) * 4;                       // s_pb[JE], s_off[JE]
  L.off_qp = L.off_ph + static_cast<size_t>(L.JL4) * 4 * 8;           // s_ph[JL4][4] float2
  L.off_list = L.off_qp + static_cast<size_t>(kPlanes * kHeadDim) * 4;   // s_qp[4][64]
  L.off_big = L.off_list + static_cast<size_t>(4 * L.list_len) * 8;    // s_list[4][list_len] int2
  const size_t e_bytes = static_cast<size_t>(L.JE) * kPfERow * 2;
  const size_t qe_bytes = static_cast<size_t>(4 * kPfQPW * L.qe_row) * 4;
  L.bytes = L.off_big + (e_bytes > qe_bytes ? e_bytes : qe_bytes);  // sE, then s_qe
  return L;
}

struct PfSlot {
  uint32_t k0, k1, k2, v0, v1, v2, ks, vs;
  float z;
  bool ok;
  int j;
};

constexpr int kXRow = 160;                       // widened row bytes
constexpr int kXK = 0, kXV = 64, kXMeta = 128;   // K bytes, V bytes, per-chunk (scales, z)

// A slot read from the widened rows: the lane's 16 K and 16 V code bytes and
// (K scale | V scale << 16, z of its plane).
struct PxSlot {
  uint4 k, v;
  uint2 meta;
  bool ok;
  int j;
};

// Sixteen 6-bit fields of a 12-byte chunk as bytes with the sign bit flipped
// (c + 32), four per dword in element order.
__device__ __forceinline__ uint4 q6_code_bytes16(uint32_t w0, uint32_t w1, uint32_t w2) {
  const uint64_t lo = (static_cast<uint64_t>(w1) << 32) | w0;
  const uint64_t hi = (static_cast<uint64_t>(w2) << 32) | w1;
  uint32_t o[4];
#pragma unroll
  for (int qd = 0; qd < 4; ++qd) {
    uint32_t x = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int bit = 6 * (4 * qd + e);
      const uint32_t f = static_cast<uint32_t>(bit < 32 ? lo >> bit : hi >> (bit - 32)) & 63u;
      x |= (f ^ 0x20u) << (8 * e);
    }
    o[qd] = x;
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// Widens every cache row of the prefill once: one thread per (row, 16-dim
// chunk); the four threads of a row write its 160 bytes.
__global__ __launch_bounds__(kBlock) void q6_widen_rows(int Hkv, int N, int64_t rows, const uint8_t* __restrict__ cache,
                                                        int64_t cs0, int64_t cs1, int64_t cs2, uint8_t* __restrict__ xr) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (i >= rows * 4) return;
  const int c = static_cast<int>(i & 3);
  const int64_t r = i >> 2;
  const int t = static_cast<int>(r % N);
  const int64_t bh = r / N;
  const int hk = static_cast<int>(bh % Hkv);
  const int64_t b = bh / Hkv;
  const uint8_t* s = cache + b * cs0 + hk * cs1 + t * cs2;
  const uint32_t* k32 = reinterpret_cast<const uint32_t*>(s + kKCodes + 12 * c);
  const uint32_t* v32 = reinterpret_cast<const uint32_t*>(s + kVCodes + 12 * c);
  const uint4 kb = q6_code_bytes16(k32[0], k32[1], k32[2]);
  const uint4 vb = q6_code_bytes16(v32[0], v32[1], v32[2]);
  const uint32_t ks = *reinterpret_cast<const uint32_t*>(s + kKScales);
  const uint32_t vs = *reinterpret_cast<const uint32_t*>(s + kVScales);
  const uint32_t z = *reinterpret_cast<const uint32_t*>(s + kZ + 4 * c);
  const int sh = c >= 2 ? 16 : 0;   // chunks 2, 3 are in group 1
  uint8_t* o = xr + r * kXRow;
  *reinterpret_cast<uint4*>(o + kXK + 16 * c) = kb;
  *reinterpret_cast<uint4*>(o + kXV + 16 * c) = vb;
  *reinterpret_cast<uint2*>(o + kXMeta + 8 * c) = make_uint2(((ks >> sh) & 0xffffu) | (((vs >> sh) & 0xffffu) << 16), z);
}

template <int SHIFT, bool WIDE>
__global__ __launch_bounds__(kBlock, 2) void q6_prefill_q4(const dwarf_dsqg_q6_prefill_args a,
                                                           const uint8_t* __restrict__ xr, int tiles, int total) {
  constexpr float kC = 0.125f * kLog2e;
  constexpr float kSlack2 = 8.0f * kLog2e;
  static_assert(SHIFT + 1 < kHeadDim / kPlanes, "MOVT pair must stay inside one lane's slice");
  const int J = a.J, N = a.N, J_small = a.J_small;
  const PfLayout lay = pf_layout(J, a.J_large);
  extern __shared__ float smem[];
  char* sm = reinterpret_cast<char*>(smem);
  float* s_pb = smem;
  int* s_off = reinterpret_cast<int*>(smem + lay.JE);
  float2* s_ph = reinterpret_cast<float2*>(sm + lay.off_ph);
  float* s_qp = reinterpret_cast<float*>(sm + lay.off_qp);
  int2* s_list_all = reinterpret_cast<int2*>(sm + lay.off_list);
  uint16_t* sE = reinterpret_cast<uint16_t*>(sm + lay.off_big);
  float* s_qe_all = reinterpret_cast<float*>(sm + lay.off_big);   // replaces sE after the second barrier

  const int work = xcd_remap(blockIdx.x, total);
  const int bh = work / tiles;
  const int tile = tiles - 1 - (work - bh * tiles);   // late query tiles first
  const int b = bh / a.H;
  const int h = bh - b * a.H;
  const int hk = h / (a.H / a.H_kv);

  const int lane = threadIdx.x;
  const int w = lane / kWave;
  const int l = lane % kWave;
  const int g = l & 3;
  const int qi = l >> 2;
  const int lr = l & 15, lc = l >> 4;
  const int n0w = tile * kPfQPB + w * kPfQPW;
  const int n = n0w + qi;
  const int n_hi = min(n0w + kPfQPW - 1, N - 1);
  const bool row_ok = n < N;
  const bool live = row_ok && n >= a.query_start;
  const int64_t nn = n;
  float* s_qe = s_qe_all + w * kPfQPW * lay.qe_row;
  int2* s_list = s_list_all + w * lay.list_len;

  // the wave's q rows (MFMA layout) and this lane's slice, requested first
  const bf16* qbase = reinterpret_cast<const bf16*>(a.q) + b * a.q_stride[0] + h * a.q_stride[1];
  uint4 xa[2] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
  if (n0w + lr < N) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      xa[ks] = *reinterpret_cast<const uint4*>(qbase + static_cast<int64_t>(n0w + lr) * a.q_stride[2] + 32 * ks + 8 * lc);
  }
  uint4 qx0 = {0u, 0u, 0u, 0u}, qx1 = {0u, 0u, 0u, 0u};
  if (live) {
    const uint4* q4 = reinterpret_cast<const uint4*>(qbase + nn * a.q_stride[2] + 16 * g);
    qx0 = q4[0];
    qx1 = q4[1];
  }

  static_assert(kPlanes * kHeadDim == kBlock, "one query-probe entry per thread");
  const float qpv = a.query_probes[threadIdx.x];   // in flight with the tables' loads
  stage_tables<true, true, true, true, false>(
      a, lay.JE, h, 1, TableStage{sE, kPfERow, s_pb, 1.0f, s_off, s_ph, 0, nullptr, 0, 0, false});
  s_qp[threadIdx.x] = qpv;
  __syncthreads();

  // s_qe[query][j] = log2(e) * (<q, e_j> / 8 + pb_j): products into registers,
  // a barrier (every wave is done reading sE), then the tables over sE.
  {
    f32x4 c[kPfMaxBlocks];
#pragma unroll
    for (int bi = 0; bi < kPfMaxBlocks; ++bi) {
      c[bi] = zero4();
      if (bi * 16 < lay.JE) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const uint4 xb = *reinterpret_cast<const uint4*>(sE + (bi * 16 + lr) * kPfERow + 32 * ks + 8 * lc);
          c[bi] = mfma16_bf16(bf16x8_from_bits(xa[ks]), bf16x8_from_bits(xb), c[bi]);
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int bi = 0; bi < kPfMaxBlocks; ++bi) {
      if (bi * 16 < lay.JE) {
        const float pb8 = 8.0f * s_pb[bi * 16 + lr];
#pragma unroll
        for (int r = 0; r < 4; ++r) s_qe[(4 * lc + r) * lay.qe_row + bi * 16 + lr] = (c[bi][r] + pb8) * kC;
      }
    }
  }
  if (n0w >= N) return;                       // whole wave past the end (no block barriers below)
  const int cnt = build_offset_list<1>(s_list, s_off, J, n0w, n_hi, N, 1, make_int2(J, n0w - N));

  // this lane's q slice (bf16 pairs and fp32), 160 * sum(q) for the biased
  // code pairs, and y of plane g = <q, probe_g> / sqrt(|q|^2 + 1e-6 hd)
  const uint32_t q32[8] = {qx0.x, qx0.y, qx0.z, qx0.w, qx1.x, qx1.y, qx1.z, qx1.w};
  float qf[16];
#pragma unroll
  for (int i = 0; i < 8; ++i) { qf[2 * i] = bf16_lo(q32[i]); qf[2 * i + 1] = bf16_hi(q32[i]); }
  float qbias = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) qbias = dot2bf(q32[i], 0x3f803f80u, qbias);   // (1, 1) in bf16
  qbias *= -160.f;
  float yg;
  {
    float ss = 0.f, yp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < 16; ++d) {
      ss = fmaf(qf[d], qf[d], ss);
#pragma unroll
      for (int r = 0; r < kPlanes; ++r) yp[r] = fmaf(qf[d], s_qp[r * kHeadDim + 16 * g + d], yp[r]);
    }
    ss = group_sum<4>(ss);
#pragma unroll
    for (int r = 0; r < kPlanes; ++r) yp[r] = group_sum<4>(yp[r]);
    yg = pick4(g, yp[0], yp[1], yp[2], yp[3]) * rsqrtf(ss + 1e-6f * kHeadDim);
  }

  const int n_eff = live ? n : n0w - 2 * N;   // no source for a query that is not live
  // rows of this (b, kv head): the cache slots, or their widened copies
  const int sstride = WIDE ? kXRow : static_cast<int>(a.cache_stride[2]);
  const __amdgpu_buffer_rsrc_t rc =
      WIDE ? rows_rsrc(xr + static_cast<int64_t>(b * a.H_kv + hk) * N * kXRow, kXRow, N, kXRow)
           : rows_rsrc(a.cache + b * a.cache_stride[0] + hk * a.cache_stride[1], sstride, N, kSlot);
  const int sb_lane = n_eff * sstride;
  const bool khi = g >= 2;   // this lane's 16 dims are in group g / 2: scale in the high half
  using Slot = typename std::conditional<WIDE, PxSlot, PfSlot>::type;

  float acc[16];
#pragma unroll
  for (int d = 0; d < 16; ++d) acc[d] = 0.f;
  float m = -3.0e38f, lsum = 0.f;
  float wsum = 0.f;   // widened rows: sum of the V weights, for the +32 carried by the V code bytes

  auto fetch = [&](int k0, Slot& s) {
    const int2 e = s_list[k0];
    const int j = uniform(e.x), d = uniform(e.y);
    s.j = j;
    s.ok = static_cast<uint32_t>(n_eff - d) < static_cast<uint32_t>(N);
    const uint32_t base = static_cast<uint32_t>(sb_lane - d * sstride);
    if constexpr (WIDE) {
      s.k = buf_load16(rc, base + kXK + 16 * g);
      s.v = buf_load16(rc, base + kXV + 16 * g);
      const auto mt = __builtin_amdgcn_raw_buffer_load_b64(rc, base + kXMeta + 8 * g, 0, 0);
      s.meta = make_uint2(mt[0], mt[1]);
    } else {
      const auto kx = __builtin_amdgcn_raw_buffer_load_b96(rc, base + kKCodes + 12 * g, 0, 0);
      const auto vx = __builtin_amdgcn_raw_buffer_load_b96(rc, base + kVCodes + 12 * g, 0, 0);
      s.k0 = kx[0]; s.k1 = kx[1]; s.k2 = kx[2];
      s.v0 = vx[0]; s.v1 = vx[1]; s.v2 = vx[2];
      s.ks = cache_dword(rc, base + kKScales);
      s.vs = cache_dword(rc, base + kVScales);
      const bool far = j >= J_small && j < J;
      s.z = __uint_as_float(cache_dword(rc, far ? base + kZ + 4 * g : kOutOfRange));
    }
  };

  auto consume = [&](const Slot& s) {
    float cf[16];
    float kd, ksc, vsc, zf;
    if constexpr (WIDE) {
      // K: v_perm puts two code bytes under the bf16 high byte 0x43, i.e. the
      // pair (128 + byte) = (160 + c); sum_d q_d (160 + c_d) as in the slot path
      const uint32_t kw[4] = {s.k.x, s.k.y, s.k.z, s.k.w};
      kd = qbias;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        kd = dot2bf(q32[2 * i], __builtin_amdgcn_perm(0x43434343u, kw[i], 0x04010400u), kd);
        kd = dot2bf(q32[2 * i + 1], __builtin_amdgcn_perm(0x43434343u, kw[i], 0x04030402u), kd);
      }
      ksc = half_bits_to_f32(static_cast<uint16_t>(s.meta.x));
      vsc = half_bits_to_f32(static_cast<uint16_t>(s.meta.x >> 16));
      zf = __uint_as_float(s.meta.y);
    } else {
      kd = q6_dot16_biased(q32, s.k0, s.k1, s.k2) + qbias;
      ksc = half_lo_or_hi(s.ks, khi);
      vsc = half_lo_or_hi(s.vs, khi);
      zf = s.z;
    }
    const float dot = group_sum<4>(kd * ksc);
    const float s2 = s.ok ? fmaf(dot, kC, s_qe[qi * lay.qe_row + s.j]) : -INFINITY;
    if (s2 > m + kSlack2) {
      const float f = __builtin_amdgcn_exp2f(m - s2);   // 0 on the first valid offset
#pragma unroll
      for (int d = 0; d < 16; ++d) acc[d] *= f;
      lsum *= f;
      if constexpr (WIDE) wsum *= f;
      m = s2;
    }
    const float p = __builtin_amdgcn_exp2f(s2 - m);   // m is finite: 0 without a source
    lsum += p;
    if constexpr (WIDE) {
      // V: each code byte to fp32 (v_cvt_f32_ubyte*): c + 32; the MOVT pair
      // drops the +32 here, the other dims when the row ends
      const uint32_t vw[4] = {s.v.x, s.v.y, s.v.z, s.v.w};
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) cf[4 * i + e] = static_cast<float>((vw[i] >> (8 * e)) & 0xffu);
      cf[SHIFT] -= 32.f;
      cf[SHIFT + 1] -= 32.f;
    } else {
      q6_codes16(s.v0, s.v1, s.v2, cf);
    }
    if (s.j >= J_small && s.j < J) {   // wave-uniform
      const float2 ph = s_ph[(s.j - J_small) * kPlanes + g];
      float sn, cs;
      dsincos<true>(fmaf(ph.y * yg, zf, ph.x), &sn, &cs);
      const float va = cf[SHIFT], vb = cf[SHIFT + 1];
      cf[SHIFT] = cs * va - sn * vb;
      cf[SHIFT + 1] = sn * va + cs * vb;
    }
    const float wgt = p * vsc;
    if constexpr (WIDE) wsum += wgt;
#pragma unroll
    for (int d = 0; d < 16; ++d) acc[d] = fmaf(wgt, cf[d], acc[d]);
    pin_regs<16>(acc);
  };

  if (cnt > 0) {
    Slot s0, s1;
    fetch(0, s0);
    for (int k0 = 0; k0 < cnt; k0 += 2) {
      fetch(k0 + 1, s1);   // past the list end this reads the sentinel: zeros
      consume(s0);
      fetch(k0 + 2, s0);
      consume(s1);
    }
  }

  if (!row_ok) return;
  if constexpr (WIDE) {
#pragma unroll
    for (int d = 0; d < 16; ++d)
      if (d != SHIFT && d != SHIFT + 1) acc[d] = fmaf(-32.f, wsum, acc[d]);
  }
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  uint4* o4 = reinterpret_cast<uint4*>(reinterpret_cast<bf16*>(a.out) + b * a.out_stride[0] + h * a.out_stride[1] +
                                       nn * a.out_stride[2] + 16 * g);
  uint4 x0, x1;
  x0.x = pack_bf16x2(acc[0] * inv, acc[1] * inv);   x0.y = pack_bf16x2(acc[2] * inv, acc[3] * inv);
  x0.z = pack_bf16x2(acc[4] * inv, acc[5] * inv);   x0.w = pack_bf16x2(acc[6] * inv, acc[7] * inv);
  x1.x = pack_bf16x2(acc[8] * inv, acc[9] * inv);   x1.y = pack_bf16x2(acc[10] * inv, acc[11] * inv);
  x1.z = pack_bf16x2(acc[12] * inv, acc[13] * inv); x1.w = pack_bf16x2(acc[14] * inv, acc[15] * inv);
  o4[0] = x0;
  o4[1] = x1;
  if (a.lse && g == 0)
    a.lse[b * a.lse_stride[0] + h * a.lse_stride[1] + nn * a.lse_stride[2]] =
        lsum > 0.f ? (m + __builtin_amdgcn_logf(lsum)) * kLn2 : -INFINITY;
}

// ---------------------------------------------------------------------------
// Prefill on widened rows with the near band on the matrix cores (used when a
// workspace is given and the lattice has small offsets).  As in the bf16
// forward (dsqg_fwd_bf16_win): the far offsets j >= JB are walked first,
// gathering widened rows as q6_prefill_q4 does, with the far q.E columns in
// the shared LDS region; then the tile's window of keys [n0 - 32, n0 + 64)
// goes over them, its K and V codes as exact bf16 integers c (16-byte chunks
// XOR-swizzled by row) and its group scales as fp32, and the leading small
// offsets j < JB are served on the matrix cores:
//   S_g^T = C_K,g Q_g^T per 32-dim group g   (v_mfma_f32_16x16x32_bf16)
//   score = sum_g sK_g(key) S_g
//   O^T  += C_V^T (P sV_g)^T                  (v_mfma_f32_16x16x16_bf16, P sV_g as bf16 hi + lo)
// A block of O^T rows spans both groups, so each block is formed with both
// groups' weights and each lane keeps the group of its own dims.
// ---------------------------------------------------------------------------
constexpr int kPfWinBack = 32;
constexpr int kPfWinRows = kPfQPB + kPfWinBack;   // 96 keys

struct PfWinLayout {
  int JE, JL4, JBh, near_row, far_row, list_len;
  size_t off_ph, off_qp, off_list, off_near, off_jn, off_big, off_vwin, off_scl, bytes;
};

__host__ __device__ inline int pf_pad_words(int n) { return (n + 11) / 16 * 16 + 4; }   // >= n, 4 mod 16

__host__ __device__ inline PfWinLayout pf_win_layout(int J, int J_small, int J_large) {
  PfWinLayout L;
  L.JE = (J + 1 + 15) / 16 * 16;
  L.JL4 = (J_large + 1) / 2 * 2;
  L.JBh = J_small < kPfWinBack ? J_small : kPfWinBack;
  L.near_row = pf_pad_words(L.JBh);
  L.far_row = pf_pad_words(L.JE - L.JBh);
  L.list_len = (L.JE + 4 + 1) / 2 * 2;
  L.off_ph = static_cast<size_t>(2 * L.JE) * 4;                          // s_pb[JE], s_off[JE]
  L.off_qp = L.off_ph + static_cast<size_t>(L.JL4) * 4 * 8;              // s_ph[JL4][4] float2
  L.off_list = L.off_qp + static_cast<size_t>(kPlanes * kHeadDim) * 4;   // s_qp[4][64]
  L.off_near = L.off_list + static_cast<size_t>(4 * L.list_len) * 8;     // s_list[4][list_len] int2
  L.off_jn = L.off_near + static_cast<size_t>(kPfQPB * L.near_row) * 4;  // s_near[64][near_row]
  L.off_big = L.off_jn + kJnSize * 4;                                    // s_jn[kJnSize]
  // shared region: sE[JE][72] bf16, then s_far[64][far_row] f32, then the window
  // (K codes [96][64] bf16, V codes [96][64] bf16, scales [96] float4)
  L.off_vwin = L.off_big + static_cast<size_t>(kPfWinRows) * 128;
  L.off_scl = L.off_vwin + static_cast<size_t>(kPfWinRows) * 128;
  const size_t e_bytes = static_cast<size_t>(L.JE) * kPfERow * 2;
  const size_t far_bytes = static_cast<size_t>(kPfQPB * L.far_row) * 4;
  const size_t win_bytes = static_cast<size_t>(kPfWinRows) * (128 + 128 + 16);
  size_t big = e_bytes > far_bytes ? e_bytes : far_bytes;
  big = big > win_bytes ? big : win_bytes;
  L.bytes = L.off_big + big;
  return L;
}

// Eight code bytes (c + 32) as eight bf16 values c (exact).
__device__ __forceinline__ uint4 code_bytes_to_bf16x8(uint32_t w0, uint32_t w1) {
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t w = i < 2 ? w0 : w1;
    const int sh = 16 * (i & 1);
    o[i] = pack_bf16x2(static_cast<float>((w >> sh) & 0xffu) - 32.f, static_cast<float>((w >> (sh + 8)) & 0xffu) - 32.f);
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

template <int SHIFT>
__global__ __launch_bounds__(kBlock, 2) void q6_prefill_win(const dwarf_dsqg_q6_prefill_args a,
                                                            const uint8_t* __restrict__ xr, int tiles, int total) {
  constexpr float kC = 0.125f * kLog2e;
  constexpr float kSlack2 = 8.0f * kLog2e;
  static_assert(SHIFT + 1 < kHeadDim / kPlanes, "MOVT pair must stay inside one lane's slice");
  const int J = a.J, N = a.N, J_small = a.J_small;
  const PfWinLayout lay = pf_win_layout(J, J_small, a.J_large);
  const int JE = lay.JE, JBh = lay.JBh, near_row = lay.near_row, far_row = lay.far_row, list_len = lay.list_len;
  extern __shared__ float smem[];
  char* sm = reinterpret_cast<char*>(smem);
  float* s_pb = smem;
  int* s_off = reinterpret_cast<int*>(smem + JE);
  float2* s_ph = reinterpret_cast<float2*>(sm + lay.off_ph);
  float* s_qp = reinterpret_cast<float*>(sm + lay.off_qp);
  int2* s_list_all = reinterpret_cast<int2*>(sm + lay.off_list);
  float* s_near = reinterpret_cast<float*>(sm + lay.off_near);
  int* s_jn = reinterpret_cast<int*>(sm + lay.off_jn);             // [0]: JB; [kJnBias + d]: band slot of d, or -1
  uint16_t* sE = reinterpret_cast<uint16_t*>(sm + lay.off_big);   // until the q.E tables are written
  float* s_far = reinterpret_cast<float*>(sm + lay.off_big);      // during the far walk
  char* s_kwin = sm + lay.off_big;                                 // during the band
  char* s_vwin = sm + lay.off_vwin;
  float4* s_scl = reinterpret_cast<float4*>(sm + lay.off_scl);    // (sK0, sK1, sV0, sV1) per window row

  const int work = xcd_remap(blockIdx.x, total);
  const int bh = work / tiles;
  const int tile = tiles - 1 - (work - bh * tiles);   // late query tiles first
  const int b = bh / a.H;
  const int h = bh - b * a.H;
  const int hk = h / (a.H / a.H_kv);

  const int lane = threadIdx.x;
  const int w = lane / kWave;
  const int l = lane % kWave;
  const int g = l & 3;
  const int qi = l >> 2;
  const int lr = l & 15, lc = l >> 4;
  const int n0 = tile * kPfQPB;
  const int n0w = n0 + w * kPfQPW;
  const int n = n0w + qi;
  const int n_hi = min(n0w + kPfQPW - 1, N - 1);
  const bool row_ok = n < N;
  const bool live = row_ok && n >= a.query_start;
  const int64_t nn = n;
  int2* s_list = s_list_all + w * list_len;
  // output addresses now, in vector registers, so the argument fields they come from do not
  // stay live in scalar registers through both walks
  uint4* o4 = reinterpret_cast<uint4*>(reinterpret_cast<bf16*>(a.out) + b * a.out_stride[0] + h * a.out_stride[1] +
                                       nn * a.out_stride[2] + 16 * g);
  float* lse_p = a.lse ? a.lse + b * a.lse_stride[0] + h * a.lse_stride[1] + nn * a.lse_stride[2] : nullptr;
  asm volatile("" : "+v"(o4), "+v"(lse_p));

  // the wave's q rows (MFMA layout) and this lane's slice, requested first
  const bf16* qbase = reinterpret_cast<const bf16*>(a.q) + b * a.q_stride[0] + h * a.q_stride[1];
  uint4 xa[2] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
  if (n0w + lr < N) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      xa[ks] = *reinterpret_cast<const uint4*>(qbase + static_cast<int64_t>(n0w + lr) * a.q_stride[2] + 32 * ks + 8 * lc);
  }
  uint4 qx0 = {0u, 0u, 0u, 0u}, qx1 = {0u, 0u, 0u, 0u};
  if (live) {
    const uint4* q4 = reinterpret_cast<const uint4*>(qbase + nn * a.q_stride[2] + 16 * g);
    qx0 = q4[0];
    qx1 = q4[1];
  }

  const float qpv = a.query_probes[threadIdx.x];   // in flight with the tables' loads
  stage_tables<true, true, true, true, true>(
      a, JE, h, 1, TableStage{sE, kPfERow, s_pb, 1.0f, s_off, s_ph, 0, s_jn, kPfWinBack, JBh, true});
  s_qp[threadIdx.x] = qpv;
  __syncthreads();

  // q.E tables: products into registers, a barrier (every wave is done
  // reading sE), then the near columns into s_near and the far ones over sE
  {
    f32x4 c[kPfMaxBlocks];
#pragma unroll
    for (int bi = 0; bi < kPfMaxBlocks; ++bi) {
      c[bi] = zero4();
      if (bi * 16 < JE) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const uint4 xb = *reinterpret_cast<const uint4*>(sE + (bi * 16 + lr) * kPfERow + 32 * ks + 8 * lc);
          c[bi] = mfma16_bf16(bf16x8_from_bits(xa[ks]), bf16x8_from_bits(xb), c[bi]);
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int bi = 0; bi < kPfMaxBlocks; ++bi) {
      if (bi * 16 < JE) {
        const int j = bi * 16 + lr;
        const float pb8 = 8.0f * s_pb[j];
        float* dst = j < JBh ? s_near + (w * kPfQPW + 4 * lc) * near_row + j
                                 : s_far + (w * kPfQPW + 4 * lc) * far_row + (j - JBh);
        const int stride = j < JBh ? near_row : far_row;
#pragma unroll
        for (int r = 0; r < 4; ++r) dst[r * stride] = (c[bi][r] + pb8) * kC;
      }
    }
  }
  const int JB = uniform(s_jn[0]);

  // this lane's q slice (bf16 pairs and fp32), 160 * sum(q) for the biased
  // code pairs, and y of plane g = <q, probe_g> / sqrt(|q|^2 + 1e-6 hd)
  const uint32_t q32[8] = {qx0.x, qx0.y, qx0.z, qx0.w, qx1.x, qx1.y, qx1.z, qx1.w};
  float qf[16];
#pragma unroll
  for (int i = 0; i < 8; ++i) { qf[2 * i] = bf16_lo(q32[i]); qf[2 * i + 1] = bf16_hi(q32[i]); }
  float qbias = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) qbias = dot2bf(q32[i], 0x3f803f80u, qbias);   // (1, 1) in bf16
  qbias *= -160.f;
  float yg;
  {
    float ss = 0.f, yp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < 16; ++d) {
      ss = fmaf(qf[d], qf[d], ss);
#pragma unroll
      for (int r = 0; r < kPlanes; ++r) yp[r] = fmaf(qf[d], s_qp[r * kHeadDim + 16 * g + d], yp[r]);
    }
    ss = group_sum<4>(ss);
#pragma unroll
    for (int r = 0; r < kPlanes; ++r) yp[r] = group_sum<4>(yp[r]);
    yg = pick4(g, yp[0], yp[1], yp[2], yp[3]) * rsqrtf(ss + 1e-6f * kHeadDim);
  }

  const int n_eff = live ? n : n0w - 2 * N;   // no source for a query that is not live
  const __amdgpu_buffer_rsrc_t rc = rows_rsrc(xr + static_cast<int64_t>(b * a.H_kv + hk) * N * kXRow, kXRow, N, kXRow);
  const int sb_lane = n_eff * kXRow;
  const float* qe_near = s_near + (w * kPfQPW + qi) * near_row;
  const float* qe_far = s_far + (w * kPfQPW + qi) * far_row - JBh;

  float acc[16];
#pragma unroll
  for (int d = 0; d < 16; ++d) acc[d] = 0.f;
  float m = -3.0e38f, lsum = 0.f;
  float wsum = 0.f;   // sum of the walk's V weights, for the +32 carried by the V code bytes

  // ---- 1. far walk: the listed offsets j >= JB, gathering widened rows ----
  if (n0w < N) {
    const int cnt = build_offset_list<1>(s_list, s_off, J, n0w, n_hi, N, 1, make_int2(J, n0w - N), JB);
    const bool all_far = JB == JBh;
    auto fetch = [&](int k0, PxSlot& s) {
      const int2 e = s_list[k0];
      const int j = uniform(e.x), d = uniform(e.y);
      s.j = j;
      s.ok = static_cast<uint32_t>(n_eff - d) < static_cast<uint32_t>(N);
      const uint32_t base = static_cast<uint32_t>(sb_lane - d * kXRow);
      s.k = buf_load16(rc, base + kXK + 16 * g);
      s.v = buf_load16(rc, base + kXV + 16 * g);
      const auto mt = __builtin_amdgcn_raw_buffer_load_b64(rc, base + kXMeta + 8 * g, 0, 0);
      s.meta = make_uint2(mt[0], mt[1]);
    };
    auto consume = [&](const PxSlot& s, const float* qe_row) {
      // K: v_perm puts two code bytes under the bf16 high byte 0x43, i.e. the
      // pair (128 + byte) = (160 + c); sum_d q_d (160 + c_d) - 160 sum_d q_d
      const uint32_t kw[4] = {s.k.x, s.k.y, s.k.z, s.k.w};
      float kd = qbias;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        kd = dot2bf(q32[2 * i], __builtin_amdgcn_perm(0x43434343u, kw[i], 0x04010400u), kd);
        kd = dot2bf(q32[2 * i + 1], __builtin_amdgcn_perm(0x43434343u, kw[i], 0x04030402u), kd);
      }
      const float ksc = half_bits_to_f32(static_cast<uint16_t>(s.meta.x));
      const float vsc = half_bits_to_f32(static_cast<uint16_t>(s.meta.x >> 16));
      const float zf = __uint_as_float(s.meta.y);
      const float dot = group_sum<4>(kd * ksc);
      const float s2 = s.ok ? fmaf(dot, kC, qe_row[s.j]) : -INFINITY;
      if (s2 > m + kSlack2) {
        const float f = __builtin_amdgcn_exp2f(m - s2);   // 0 on the first valid offset
#pragma unroll
        for (int d = 0; d < 16; ++d) acc[d] *= f;
        lsum *= f;
        wsum *= f;
        m = s2;
      }
      const float p = __builtin_amdgcn_exp2f(s2 - m);   // m is finite: 0 without a source
      lsum += p;
      // V: each code byte to fp32 (v_cvt_f32_ubyte*): c + 32; the MOVT pair
      // drops the +32 here, the other dims when the row ends
      float cf[16];
      const uint32_t vw[4] = {s.v.x, s.v.y, s.v.z, s.v.w};
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) cf[4 * i + e] = static_cast<float>((vw[i] >> (8 * e)) & 0xffu);
      cf[SHIFT] -= 32.f;
      cf[SHIFT + 1] -= 32.f;
      if (s.j >= J_small && s.j < J) {   // wave-uniform
        const float2 ph = s_ph[(s.j - J_small) * kPlanes + g];
        float sn, cs;
        dsincos<true>(fmaf(ph.y * yg, zf, ph.x), &sn, &cs);
        const float va = cf[SHIFT], vb = cf[SHIFT + 1];
        cf[SHIFT] = cs * va - sn * vb;
        cf[SHIFT + 1] = sn * va + cs * vb;
      }
      const float wgt = p * vsc;
      wsum += wgt;
#pragma unroll
      for (int d = 0; d < 16; ++d) acc[d] = fmaf(wgt, cf[d], acc[d]);
      pin_regs<16>(acc);
    };
    if (cnt > 0) {
      PxSlot s0, s1;
      fetch(0, s0);
      for (int k0 = 0; k0 < cnt; k0 += 2) {
        fetch(k0 + 1, s1);   // past the list end this reads the sentinel: zeros
        consume(s0, all_far || s0.j >= JBh ? qe_far : qe_near);
        fetch(k0 + 2, s0);
        consume(s1, all_far || s1.j >= JBh ? qe_far : qe_near);
      }
    }
  }
  // the walk's +32 on the V codes of the dims outside the MOVT pair
#pragma unroll
  for (int d = 0; d < 16; ++d)
    if (d != SHIFT && d != SHIFT + 1) acc[d] = fmaf(-32.f, wsum, acc[d]);

  // ---- 2. near band: offsets j < JB on the matrix cores, from the window in LDS ----
  __syncthreads();   // every wave is done with the far table: the window goes over it
  if (JB > 0) {
    // keys [n0 - 32, n0 + 64), one (row, 16-dim chunk) per unit: codes to bf16
    // c (keys outside [0, N) read zeros: their scores are masked), 16-byte
    // chunk cc of a row at position cc ^ (row & 7); the group scales of the
    // row from chunks 0 and 2
    for (int u = threadIdx.x; u < kPfWinRows * 4; u += kBlock) {
      const int row = u >> 2, ch = u & 3;
      const int key = n0 - kPfWinBack + row;
      const uint32_t base = static_cast<uint32_t>(key * kXRow);
      const uint4 kb = buf_load16(rc, base + kXK + 16 * ch);
      const uint4 vb = buf_load16(rc, base + kXV + 16 * ch);
      const uint32_t mt = __builtin_amdgcn_raw_buffer_load_b32(rc, base + kXMeta + 8 * ch, 0, 0);
      const int sw = row & 7;
      *reinterpret_cast<uint4*>(s_kwin + row * 128 + 16 * ((2 * ch) ^ sw)) = code_bytes_to_bf16x8(kb.x, kb.y);
      *reinterpret_cast<uint4*>(s_kwin + row * 128 + 16 * ((2 * ch + 1) ^ sw)) = code_bytes_to_bf16x8(kb.z, kb.w);
      *reinterpret_cast<uint4*>(s_vwin + row * 128 + 16 * ((2 * ch) ^ sw)) = code_bytes_to_bf16x8(vb.x, vb.y);
      *reinterpret_cast<uint4*>(s_vwin + row * 128 + 16 * ((2 * ch + 1) ^ sw)) = code_bytes_to_bf16x8(vb.z, vb.w);
      if ((ch & 1) == 0) {
        float* sc = reinterpret_cast<float*>(s_scl + row) + (ch >> 1);
        sc[0] = half_bits_to_f32(static_cast<uint16_t>(mt));          // K scale of group ch / 2
        sc[2] = half_bits_to_f32(static_cast<uint16_t>(mt >> 16));    // V scale of group ch / 2
      }
    }
  }
  __syncthreads();   // the window is staged
  if (n0w < N && JB > 0) {
    // Band lane (lc, lr) serves query n0w + lr; in the MFMA C layout it holds
    // keys n0w - 32 + 16 tb + 4 lc + r of the wave's key blocks tb = 0..2.
    const int nq = n0w + lr;
    const bool live_b = nq < N && nq >= a.query_start;
    auto win16 = [&](const char* base, int row, int c) { return base + row * 128 + 16 * (c ^ (row & 7)); };
    const float* qe_b = s_near + (w * kPfQPW + lr) * near_row;
    // the far walk's running maximum of this query (gather lane 4 lr)
    const float m_q = __int_as_float(__builtin_amdgcn_ds_bpermute(4 * (4 * lr), __float_as_int(m)));
    float sb[3][4];
    float cmax = -INFINITY;
#pragma unroll
    for (int tb = 0; tb < 3; ++tb) {
      const int wr = 16 * (w + tb) + lr;               // window row of key n0w - 32 + 16 tb + lr
      const uint4 ka0 = *reinterpret_cast<const uint4*>(win16(s_kwin, wr, lc));       // dims 8 lc + [0, 8): group 0
      const uint4 ka1 = *reinterpret_cast<const uint4*>(win16(s_kwin, wr, 4 + lc));   // group 1
      const f32x4 S0 = mfma16_bf16(bf16x8_from_bits(ka0), bf16x8_from_bits(xa[0]), zero4());
      const f32x4 S1 = mfma16_bf16(bf16x8_from_bits(ka1), bf16x8_from_bits(xa[1]), zero4());
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kr = 16 * (w + tb) + 4 * lc + r;     // window row of the entry's key
        const float4 scl = s_scl[kr];
        const int slot = s_jn[kJnBias + lr + kPfWinBack - 16 * tb - 4 * lc - r];
        const bool ok = slot >= 0 && live_b && n0w - kPfWinBack + 16 * tb + 4 * lc + r >= 0;
        const float sc2 = fmaf(fmaf(scl.x, S0[r], scl.y * S1[r]), kC, qe_b[slot >= 0 ? slot : 0]);
        sb[tb][r] = ok ? sc2 : -INFINITY;
        cmax = fmaxf(cmax, sb[tb][r]);
      }
    }
    cmax = max_xor32(max_xor16(cmax));                 // over the four lanes of query lr
    const float m_use = cmax > m_q + kSlack2 ? cmax : m_q;
    f32x4 acc0[4], acc1[4];
#pragma unroll
    for (int db = 0; db < 4; ++db) { acc0[db] = zero4(); acc1[db] = zero4(); }
    float lb = 0.f;
#pragma unroll
    for (int tb = 0; tb < 3; ++tb) {
      float p0h[4], p0l[4], p1h[4], p1l[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float4 scl = s_scl[16 * (w + tb) + 4 * lc + r];
        const float p = __builtin_amdgcn_exp2f(sb[tb][r] - m_use);   // 0 off the band
        lb += p;
        const float w0 = p * scl.z, w1 = p * scl.w;
        p0h[r] = w0; p0l[r] = w0 - round_bf16(w0);
        p1h[r] = w1; p1l[r] = w1 - round_bf16(w1);
      }
      const i16x4 b0h = __builtin_bit_cast(i16x4, make_uint2(pack_bf16x2(p0h[0], p0h[1]), pack_bf16x2(p0h[2], p0h[3])));
      const i16x4 b0l = __builtin_bit_cast(i16x4, make_uint2(pack_bf16x2(p0l[0], p0l[1]), pack_bf16x2(p0l[2], p0l[3])));
      const i16x4 b1h = __builtin_bit_cast(i16x4, make_uint2(pack_bf16x2(p1h[0], p1h[1]), pack_bf16x2(p1h[2], p1h[3])));
      const i16x4 b1l = __builtin_bit_cast(i16x4, make_uint2(pack_bf16x2(p1l[0], p1l[1]), pack_bf16x2(p1l[2], p1l[3])));
      // V code rows read transposed from the window (rows 16 (w + tb) + 4 lc + e,
      // dims 16 (lr / 4) + 4 db + lr % 4 of MFMA row lr)
      const int R = 16 * (w + tb) + 4 * lc + (lr >> 2);
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const i16x4 av = lds_read_tr16(win16(s_vwin, R, 2 * (lr & 3) + (db >> 1)) + 8 * (db & 1));
        acc0[db] = mfma16k16_bf16(av, b0h, acc0[db]);
        acc0[db] = mfma16k16_bf16(av, b0l, acc0[db]);
        acc1[db] = mfma16k16_bf16(av, b1h, acc1[db]);
        acc1[db] = mfma16k16_bf16(av, b1l, acc1[db]);
      }
    }
    lb = add_xor32(add_xor16(lb));
    // into the gather layout: query qi, dims 16 g + 4 db + r <- band lane (lr = qi, lc = g),
    // whose dims lie in group lc / 2
    const int srcq = 4 * (qi + 16 * g);
    const float m_new = __int_as_float(__builtin_amdgcn_ds_bpermute(srcq, __float_as_int(m_use)));
    const float l_new = __int_as_float(__builtin_amdgcn_ds_bpermute(srcq, __float_as_int(lb)));
    const float f = __builtin_amdgcn_exp2f(m - m_new);   // 1 when the maximum stays; 0 with no far pair
    const bool grp1 = lc >= 2;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float ob = grp1 ? acc1[db][r] : acc0[db][r];
        acc[4 * db + r] = fmaf(acc[4 * db + r], f, __int_as_float(__builtin_amdgcn_ds_bpermute(srcq, __float_as_int(ob))));
      }
    lsum = fmaf(lsum, f, l_new);
    m = m_new;
  }

  if (!row_ok) return;
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  uint4 x0, x1;
  x0.x = pack_bf16x2(acc[0] * inv, acc[1] * inv);   x0.y = pack_bf16x2(acc[2] * inv, acc[3] * inv);
  x0.z = pack_bf16x2(acc[4] * inv, acc[5] * inv);   x0.w = pack_bf16x2(acc[6] * inv, acc[7] * inv);
  x1.x = pack_bf16x2(acc[8] * inv, acc[9] * inv);   x1.y = pack_bf16x2(acc[10] * inv, acc[11] * inv);
  x1.z = pack_bf16x2(acc[12] * inv, acc[13] * inv); x1.w = pack_bf16x2(acc[14] * inv, acc[15] * inv);
  o4[0] = x0;
  o4[1] = x1;
  if (lse_p && g == 0) *lse_p = lsum > 0.f ? (m + __builtin_amdgcn_logf(lsum)) * kLn2 : -INFINITY;
}

// ---------------------------------------------------------------------------
// Decode.  One workgroup per (sequence, layer, group of kDecHeadsPerWg
// heads), one wave per head.
//
// A slot's codes come in 12-byte chunks of 16 head dims (K at 12c, V at
// 52 + 12c), so four lanes per gathered row -- lane c holding dims
// [16c, 16c+16) of K and of V -- cover a whole 128-byte slot, and one wave
// load instruction fetches 16 slots.  Each wave lists the offsets whose row
// t - delta is inside the cache and requests its first batch of 16 rows
// before the shared set-up:
//   - the table T[head][j] = log2(e) (<q_head, e_j> / 8 + pb_j) for all heads
//     of the workgroup and all offsets, one MFMA pass over 16-offset tiles
//     (E in bf16, as the GPU path rounds it; a bf16 low part is added when SE
//     is not rounded);
//   - y of the head's query, one wave reduction per probe plane.
// The wave then walks its list in batches of 16 rows with the next batch in
// flight.  Per row, q.k is formed on the codes: each pair of 6-bit codes is
// turned into the bf16 pair (160 + c_a, 160 + c_b) with three integer
// instructions and consumed by v_dot2_f32_bf16, and 160 * sum(q) is
// subtracted once; the fp16 group scale multiplies the lane's partial sum.
// V codes are widened to fp32 (v_bfe_i32), rotated by the MOVT pair of plane
// c and accumulated with weight P * scale under an online base-2 softmax in
// which each row group keeps its own running maximum.  At the end the groups
// are put on the wave's largest maximum and summed (lane swaps that
// reduce-scatter the 16 dims of a lane, then DPP row rotations).
// ---------------------------------------------------------------------------
constexpr int kDecRows = 16;      // rows per batch (one per 4-lane group)
constexpr int kMaxDecHeads = 16;  // heads the decode step takes
constexpr int kMaxDecOffsets = 256;   // offsets the decode step takes
// heads (waves) per decode workgroup: at cfg5 four per workgroup measured 43.0 / 47.9 / 53.1 us per step
// (warm / advancing / cold) against 44.0 / 49.4 / 54.4 with all eight heads in one workgroup (28 resident
// waves per CU instead of 24), two 43.2 / 48.2 / 53.6, one 43.4 / 48.1 / 53.0
constexpr int kDecHeadsPerWg = 4;

struct DecBatch {
  uint32_t k0, k1, k2, v0, v1, v2;
  uint32_t ks, vs;   // fp16 scale pairs of the two groups
  float z, base, gain;
  float t;           // the row's T entry: log2(e) (<q, e_j> / 8 + pb_j)
  int j;
  bool ok;
};

struct DecLayout {
  int JE, list_len;
  size_t bytes;
};

__host__ __device__ inline DecLayout dec_layout(int J, int H) {
  DecLayout L;
  L.JE = (J + 1 + 15) / 16 * 16;                                   // offsets, the sentinel column, padding
  L.list_len = (J + 3 * kDecRows + 1) / 2 * 2;
  L.bytes = static_cast<size_t>(H) * L.list_len * 8;               // s_list[H][list_len] int2
  return L;
}

// The decode step's T table, T[l][s][h][j] = log2(e) (<q, e_j> / 8 + pb_j)
// for every (layer, sequence, head) and offset, rows of JE floats with 0 at
// j >= J (the sentinel column).  A workgroup takes 64 (sequence, head) rows
// of one layer: it stages the layer's E rows in bf16 (as the GPU path rounds
// them; hi and lo halves for the fp32 table) and its pos_bias in LDS, then
// each wave multiplies its 16 q rows (A) by 16 E rows at a time (B).
constexpr int kTabRows = 64;    // (sequence, head) rows per workgroup
constexpr int kTabERow = 72;    // bf16 E row stride (elements)

__host__ __device__ inline size_t dec_table_lds(int JE, int H, bool split) {
  return static_cast<size_t>(JE) * kTabERow * 2 * (split ? 2 : 1) + static_cast<size_t>(JE) * H * 4;
}

__global__ __launch_bounds__(kBlock) void q6_decode_table(const dwarf_dsqg_q6_decode_args a, float* __restrict__ T,
                                                          int JE) {
  constexpr float kC = 0.125f * kLog2e;
  const int rows = a.S * a.H;
  const int per_layer = (rows + kTabRows - 1) / kTabRows;
  const int ly = blockIdx.x / per_layer;
  const int r0 = (blockIdx.x - ly * per_layer) * kTabRows + (threadIdx.x / kWave) * 16;
  const int l = threadIdx.x % kWave, lr = l & 15, lc = l >> 4;
  const int J = a.J, H = a.H;
  const bool split = !a.se_round_bf16;
  extern __shared__ float smem[];
  uint16_t* sEh = reinterpret_cast<uint16_t*>(smem);
  uint16_t* sEl = sEh + JE * kTabERow;                                  // used when split
  float* s_pb = reinterpret_cast<float*>(sEh + JE * kTabERow * (split ? 2 : 1));   // [JE][H]

  // this wave's q rows first, so their latency overlaps the staging; a row past the end loads
  // the last row instead (its products are never stored), so the load needs no condition
  uint4 xa[2];
  {
    const int rr = r0 + lr < rows ? r0 + lr : rows - 1;
    const int sq = rr / H, h = rr - sq * H;
    const bf16* qrow = reinterpret_cast<const bf16*>(a.q) + sq * a.q_stride[0] + ly * a.q_stride[1] + h * a.q_stride[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) xa[ks] = *reinterpret_cast<const uint4*>(qrow + 32 * ks + 8 * lc);
  }
  const float* se = a.scale_embed + ly * a.se_stride[0];
  const float* pbl = a.pos_bias + ly * a.pb_stride[0];
  // Staging, one memory round trip per round of kBatch steps: a round issues
  // every load before the first use, E rows (4 floats per load, 16 loads per
  // row) and the layer's pos_bias [J][H] alike.  Both come through buffer
  // loads, entries past a table (j >= J) reading zeros with no condition
  // around the load (a conditional load with a default value is waited for at
  // its join, one round trip each); the host bounds both spans below 2 GiB.
  constexpr int kBatch = 8;
  const int pb1 = static_cast<int>(a.pb_stride[1]), pb2 = static_cast<int>(a.pb_stride[2]);
  const __amdgpu_buffer_rsrc_t rpbl = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(pbl), 0, ((J - 1) * pb1 + (H - 1) * pb2 + 1) * 4, 0x00020000);
  const int se1 = static_cast<int>(a.se_stride[1]) * 4;   // E row bytes
  const __amdgpu_buffer_rsrc_t rse = rows_rsrc(se, se1, J, 256);
  const int ne = JE * 16, np = JE * H;
  // one round (the first is peeled off the loop: a loop header waits for every load in flight)
  auto stage_round = [&](int i0) {
    float4 v[kBatch];
    float pv[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int i = i0 + u * kBlock, j = i >> 4;
      const uint4 ev = buf_load16(rse, i < ne && j < J ? static_cast<uint32_t>(j * se1 + 16 * (i & 15)) : kOutOfRange);
      v[u] = make_float4(__uint_as_float(ev.x), __uint_as_float(ev.y), __uint_as_float(ev.z), __uint_as_float(ev.w));
      const int jp = i / H, hp = i - jp * H;
      pv[u] = buf_load_f32(rpbl, i < np && jp < J ? static_cast<uint32_t>((jp * pb1 + hp * pb2) * 4) : kOutOfRange);
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int i = i0 + u * kBlock;
      if (i < ne) {
        const float x[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
        uint16_t* dh = sEh + (i >> 4) * kTabERow + 4 * (i & 15);
        uint16_t* dl = sEl + (i >> 4) * kTabERow + 4 * (i & 15);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const __bf16 hi = static_cast<__bf16>(x[e]);
          dh[e] = __builtin_bit_cast(uint16_t, hi);
          if (split) dl[e] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(x[e] - static_cast<float>(hi)));
        }
      }
      if (i < np) s_pb[i] = pv[u];
    }
  };
  stage_round(threadIdx.x);
  for (int i0 = threadIdx.x + kBatch * kBlock; i0 < (ne > np ? ne : np); i0 += kBatch * kBlock) stage_round(i0);
  __syncthreads();
  if (r0 >= rows) return;   // whole wave, after the only barrier
  for (int tile = 0; tile < JE / 16; ++tile) {
    const int j = tile * 16 + lr;
    f32x4 acc = zero4();
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const uint4 eh = *reinterpret_cast<const uint4*>(sEh + j * kTabERow + 32 * ks + 8 * lc);
      acc = mfma16_bf16(bf16x8_from_bits(xa[ks]), bf16x8_from_bits(eh), acc);
      if (split) {
        const uint4 el = *reinterpret_cast<const uint4*>(sEl + j * kTabERow + 32 * ks + 8 * lc);
        acc = mfma16_bf16(bf16x8_from_bits(xa[ks]), bf16x8_from_bits(el), acc);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = r0 + 4 * lc + r;   // (sequence, head) row of the product
      if (i < rows) {
        const int sq = i / H, h = i - sq * H;
        T[(static_cast<int64_t>(ly * a.S + sq) * H + h) * JE + j] = j < J ? (acc[r] + 8.0f * s_pb[j * H + h]) * kC : 0.f;
      }
    }
  }
}

// Sum over all 64 lanes, in every lane.
__device__ __forceinline__ float wave_allsum(float x) { return sum_over_queries16(group_sum<4>(x)); }

template <int SHIFT>
__global__ __launch_bounds__(kWave * kMaxDecHeads) void q6_decode_q4(const dwarf_dsqg_q6_decode_args a,
                                                                    const float* __restrict__ T) {
  constexpr float kC = 0.125f * kLog2e;
  constexpr float kSlack2 = 8.0f * kLog2e;
  static_assert(SHIFT + 1 < kHeadDim / kPlanes, "MOVT pair must stay inside one lane's chunk");
  const int J = a.J, H = a.H, J_small = a.J_small;
  const DecLayout lay = dec_layout(J, H);
  extern __shared__ float smem[];
  int2* s_list_all = reinterpret_cast<int2*>(smem);

  constexpr int HPW = kDecHeadsPerWg;
  const int hgroups = (H + HPW - 1) / HPW;
  const int hg = blockIdx.x % hgroups;
  const int sl = blockIdx.x / hgroups;
  const int sq = sl / a.L;
  const int ly = sl - sq * a.L;
  const int wv = uniform(threadIdx.x / kWave);
  const int h = hg * HPW + wv;   // head = wave index within the group
  if (h >= H) return;
  const int l = threadIdx.x % kWave;
  const int c = l & 3;        // 16-dim chunk
  const int rr = l >> 2;      // row of the batch
  const int hk = h / (H / a.H_kv);
  // The prologue's independent loads go out together: the position, the offsets (lane l holds offset
  // 64 c + l; zeros past J), this head's query slice and the query probes; the offset list is then
  // built from registers.
  const int t = uniform(a.pos[sq]);
  constexpr int kOffChunks = (kMaxDecOffsets + kWave - 1) / kWave;
  int offv[kOffChunks];
  {
    const __amdgpu_buffer_rsrc_t rof =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<int*>(a.offsets), 0, J * 4, 0x00020000);
#pragma unroll
    for (int ci = 0; ci < kOffChunks; ++ci)
      offv[ci] = static_cast<int>(__builtin_amdgcn_raw_buffer_load_b32(rof, static_cast<uint32_t>(4 * (kWave * ci + l)), 0, 0));
  }
  const bf16* qrows = reinterpret_cast<const bf16*>(a.q) + sq * a.q_stride[0] + ly * a.q_stride[1];
  const bf16* qh = qrows + h * a.q_stride[2];
  uint32_t q32[8];
  {
    const uint4* q4 = reinterpret_cast<const uint4*>(qh + 16 * c);
    const uint4 x0 = q4[0], x1 = q4[1];
    q32[0] = x0.x; q32[1] = x0.y; q32[2] = x0.z; q32[3] = x0.w;
    q32[4] = x1.x; q32[5] = x1.y; q32[6] = x1.z; q32[7] = x1.w;
  }
  const float qd = __uint_as_float(static_cast<uint32_t>(reinterpret_cast<const uint16_t*>(qh)[l]) << 16);
  float qpl[kPlanes];
  {
    const float* qp = a.query_probes + ly * a.qprobe_layer_stride;
#pragma unroll
    for (int r = 0; r < kPlanes; ++r) qpl[r] = qp[r * kHeadDim + l];
  }
  const int Nc = a.Ncache;
  int2* list = s_list_all + wv * lay.list_len;
  // this (sequence, layer, head)'s row of the T table (q6_decode_table)
  const float* Th = T + (static_cast<int64_t>(ly * a.S + sq) * H + h) * lay.JE;
  // rows t - delta in [0, Nc); the sentinel (J, t + 1) gives row -1
  const int cnt = build_offset_list_regs<kDecRows, kOffChunks>(list, offv, J, t, t, Nc, 1, make_int2(J, t + 1));
  const int cntp = (cnt + kDecRows - 1) / kDecRows * kDecRows;

  const uint8_t* cb = a.cache + ly * a.cache_stride[0] + sq * a.cache_stride[1] + hk * a.cache_stride[2];
  const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(cb), 0, Nc * kSlot,
                                                                      0x00020000);
  // MOVT angle parameters of this head (uniform resources): far index i,
  // plane c at byte i * step + 4c
  const int ph_step = static_cast<int>(a.pbase_stride[1]) * 4, pg_step = static_cast<int>(a.pgain_stride[1]) * 4;
  const __amdgpu_buffer_rsrc_t rpb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(a.phase_base + ly * a.pbase_stride[0] + h * a.pbase_stride[2]), 0,
      a.J_large > 0 ? (a.J_large - 1) * ph_step + 4 * kPlanes : 0, 0x00020000);
  const __amdgpu_buffer_rsrc_t rpg = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(a.phase_gain + ly * a.pgain_stride[0] + h * a.pgain_stride[2]), 0,
      a.J_large > 0 ? (a.J_large - 1) * pg_step + 4 * kPlanes : 0, 0x00020000);
  const bool khi = c >= 2;    // K/V group of this chunk: scale in the high half of the pair

  auto fetch = [&](int k0, DecBatch& b) {
    const int2 e = list[k0 + rr];
    b.j = e.x;
    const int row = t - e.y;
    b.ok = static_cast<uint32_t>(row) < static_cast<uint32_t>(Nc);
    const uint32_t base = b.ok ? static_cast<uint32_t>(row) * kSlot : kOutOfRange;
    const auto kx = __builtin_amdgcn_raw_buffer_load_b96(rc, base + kKCodes + 12 * c, 0, 0);
    const auto vx = __builtin_amdgcn_raw_buffer_load_b96(rc, base + kVCodes + 12 * c, 0, 0);
    b.k0 = kx[0]; b.k1 = kx[1]; b.k2 = kx[2];
    b.v0 = vx[0]; b.v1 = vx[1]; b.v2 = vx[2];
    b.ks = cache_dword(rc, base + kKScales);
    b.vs = cache_dword(rc, base + kVScales);
    const bool far = e.x >= J_small && e.x < J;
    b.z = __builtin_bit_cast(float, cache_dword(rc, far ? base + kZ + 4 * c : kOutOfRange));
    const int i = e.x - J_small;
    b.base = buf_load_f32(rpb, far ? static_cast<uint32_t>(i * ph_step + 4 * c) : kOutOfRange);
    b.gain = buf_load_f32(rpg, far ? static_cast<uint32_t>(i * pg_step + 4 * c) : kOutOfRange);
    b.t = Th[e.x];
  };

  DecBatch b0, b1;
  if (cnt > 0) fetch(0, b0);

  // this head's query: lane c's 16 dims as bf16 pairs, their sum, and y of
  // plane c = <q, probe_c> / sqrt(|q|^2 + 1e-6 hd) (dsqg:3231-3249)
  float qbias = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) qbias = dot2bf(q32[i], 0x3f803f80u, qbias);   // (1, 1) in bf16
  qbias *= -160.f;
  float yg;
  {
    const float ss = wave_allsum(qd * qd);
    float yp[kPlanes];
#pragma unroll
    for (int r = 0; r < kPlanes; ++r) yp[r] = wave_allsum(qd * qpl[r]);
    yg = pick4(c, yp[0], yp[1], yp[2], yp[3]) * rsqrtf(ss + 1e-6f * kHeadDim);
  }

  float acc[16];
#pragma unroll
  for (int d = 0; d < 16; ++d) acc[d] = 0.f;
  float m = -3.0e38f, lsum = 0.f;

  auto consume = [&](int k0, const DecBatch& b) {
    const float kd = q6_dot16_biased(q32, b.k0, b.k1, b.k2) + qbias;
    const float dot = group_sum<4>(kd * half_lo_or_hi(b.ks, khi));
    const float s2 = b.ok ? fmaf(dot, kC, b.t) : -INFINITY;
    if (s2 > m + kSlack2) {   // per row group; the groups are put on one scale at the end
      const float f = __builtin_amdgcn_exp2f(m - s2);
#pragma unroll
      for (int d = 0; d < 16; ++d) acc[d] *= f;
      lsum *= f;
      m = s2;
    }
    const float p = __builtin_amdgcn_exp2f(s2 - m);
    lsum += p;
    float cf[16];
    q6_codes16(b.v0, b.v1, b.v2, cf);
    // MOVT pair of plane c (dims 16c + SHIFT, +1); near rows have angle 0.
    // The list is ordered by offset index, so a batch whose last row is near
    // has no far row.
    if (uniform(list[k0 + kDecRows - 1].x) >= J_small) {
      float sn, cs;
      dsincos<true>(fmaf(b.gain * yg, b.z, b.base), &sn, &cs);
      const float va = cf[SHIFT], vb = cf[SHIFT + 1];
      cf[SHIFT] = cs * va - sn * vb;
      cf[SHIFT + 1] = sn * va + cs * vb;
    }
    const float wgt = p * half_lo_or_hi(b.vs, khi);
#pragma unroll
    for (int d = 0; d < 16; ++d) acc[d] = fmaf(wgt, cf[d], acc[d]);
    pin_regs<16>(acc);
  };

  if (cnt > 0) {
    for (int k0 = 0; k0 < cntp; k0 += 2 * kDecRows) {
      fetch(k0 + kDecRows, b1);
      consume(k0, b0);
      fetch(k0 + 2 * kDecRows, b0);
      consume(k0 + kDecRows, b1);
    }
  }
  // Row groups onto the wave's largest reference, then the sum over the 16
  // groups of each (chunk, dim), reduce-scattered: after the two lane swaps
  // lane l holds dims 16c + 8 (l >> 5) + 4 ((l >> 4) & 1) + [0, 4) of four
  // groups, and two row rotations add the other twelve.
  float M = fmaxf(m, dpp_f<0x124>(m));
  M = fmaxf(M, dpp_f<0x128>(M));
  M = max_xor32(max_xor16(M));
  const float sc = __builtin_amdgcn_exp2f(m - M);   // 0 for a group that saw no row
  lsum = sum_over_queries16(lsum * sc);
  float o[4];
  {
    float r[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = add_swap32(acc[i] * sc, acc[i + 8] * sc);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float x = add_swap16(r[i], r[i + 4]);
      x += dpp_f<0x124>(x);   // row_ror:4
      x += dpp_f<0x128>(x);   // row_ror:8
      o[i] = x;
    }
  }
  if ((rr & 3) == 0) {
    const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
    const int d0 = 16 * c + 8 * (l >> 5) + 4 * ((l >> 4) & 1);
    uint2 x;
    x.x = pack_bf16x2(o[0] * inv, o[1] * inv);
    x.y = pack_bf16x2(o[2] * inv, o[3] * inv);
    *reinterpret_cast<uint2*>(reinterpret_cast<bf16*>(a.out) + sq * a.out_stride[0] + ly * a.out_stride[1] +
                              h * a.out_stride[2] + d0) = x;
  }
}

}  // namespace

hipError_t launch_q6_pack(int B, int Hkv, int N, int dtype, const void* k, const int64_t* ks, const void* v,
                          const int64_t* vs, uint8_t* cache, const int64_t* cs, const float* kprobe,
                          hipStream_t stream) {
  const int64_t rows = static_cast<int64_t>(B) * Hkv * N;
  const int blocks = static_cast<int>((rows + kBlock - 1) / kBlock);
  if (dtype == DWARF_BF16)
    hipLaunchKernelGGL(q6_pack_kernel<bf16>, dim3(blocks), dim3(kBlock), 0, stream, B, Hkv, N,
                       static_cast<const bf16*>(k), nullptr, static_cast<const bf16*>(v), nullptr, cache, nullptr,
                       kprobe, ks[0], ks[1], ks[2], vs[0], vs[1], vs[2], cs[0], cs[1], cs[2]);
  else
    hipLaunchKernelGGL(q6_pack_kernel<float>, dim3(blocks), dim3(kBlock), 0, stream, B, Hkv, N,
                       static_cast<const float*>(k), nullptr, static_cast<const float*>(v), nullptr, cache, nullptr,
                       kprobe, ks[0], ks[1], ks[2], vs[0], vs[1], vs[2], cs[0], cs[1], cs[2]);
  return hipGetLastError();
}

hipError_t launch_q6_unpack(int B, int Hkv, int N, const uint8_t* cache, const int64_t* cs, float* kout,
                            float* vout, hipStream_t stream) {
  const int64_t parts = static_cast<int64_t>(B) * Hkv * N * 4;
  const int blocks = static_cast<int>((parts + kBlock - 1) / kBlock);
  hipLaunchKernelGGL(q6_unpack_kernel, dim3(blocks), dim3(kBlock), 0, stream, B, Hkv, N, cache, cs[0], cs[1], cs[2],
                     kout, vout);
  return hipGetLastError();
}

size_t q6_prefill_workspace(const dwarf_dsqg_q6_prefill_args& a) {
  return static_cast<size_t>(a.B) * a.H_kv * a.N * kXRow;
}

template <bool WIDE>
hipError_t launch_prefill_rows(const dwarf_dsqg_q6_prefill_args& a, const uint8_t* xr, int tiles, int total,
                               hipStream_t stream) {
  const size_t lds = pf_layout(a.J, a.J_large).bytes;
#define DWARF_Q6P_CASE(S)                                                                                    \
  case S:                                                                                                    \
    hipLaunchKernelGGL((q6_prefill_q4<S, WIDE>), dim3(total), dim3(kBlock), lds, stream, a, xr, tiles, total); \
    break;
  switch (a.plane_shift) {
    DWARF_Q6P_CASE(0) DWARF_Q6P_CASE(1) DWARF_Q6P_CASE(2) DWARF_Q6P_CASE(3) DWARF_Q6P_CASE(4)
    DWARF_Q6P_CASE(5) DWARF_Q6P_CASE(6) DWARF_Q6P_CASE(7) DWARF_Q6P_CASE(8) DWARF_Q6P_CASE(9)
    DWARF_Q6P_CASE(10) DWARF_Q6P_CASE(11) DWARF_Q6P_CASE(12) DWARF_Q6P_CASE(13) DWARF_Q6P_CASE(14)
    default: return hipErrorInvalidValue;
  }
#undef DWARF_Q6P_CASE
  return hipGetLastError();
}

hipError_t launch_q6_prefill(const dwarf_dsqg_q6_prefill_args& a, hipStream_t stream) {
  const int tiles = (a.N + kPfQPB - 1) / kPfQPB;
  const int total = tiles * a.B * a.H;
  if (total == 0) return hipSuccess;
  if (!a.workspace) return launch_prefill_rows<false>(a, nullptr, tiles, total, stream);
  uint8_t* xr = static_cast<uint8_t*>(a.workspace);
  const int64_t rows = static_cast<int64_t>(a.B) * a.H_kv * a.N;
  hipLaunchKernelGGL(q6_widen_rows, dim3(static_cast<unsigned>((rows * 4 + kBlock - 1) / kBlock)), dim3(kBlock), 0,
                     stream, a.H_kv, a.N, rows, a.cache, a.cache_stride[0], a.cache_stride[1], a.cache_stride[2], xr);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (a.J_small > 0) {
    const size_t lds = pf_win_layout(a.J, a.J_small, a.J_large).bytes;
#define DWARF_Q6W_CASE(S)                                                                                  \
  case S:                                                                                                  \
    hipLaunchKernelGGL((q6_prefill_win<S>), dim3(total), dim3(kBlock), lds, stream, a, xr, tiles, total);   \
    break;
    switch (a.plane_shift) {
      DWARF_Q6W_CASE(0) DWARF_Q6W_CASE(1) DWARF_Q6W_CASE(2) DWARF_Q6W_CASE(3) DWARF_Q6W_CASE(4)
      DWARF_Q6W_CASE(5) DWARF_Q6W_CASE(6) DWARF_Q6W_CASE(7) DWARF_Q6W_CASE(8) DWARF_Q6W_CASE(9)
      DWARF_Q6W_CASE(10) DWARF_Q6W_CASE(11) DWARF_Q6W_CASE(12) DWARF_Q6W_CASE(13) DWARF_Q6W_CASE(14)
      default: return hipErrorInvalidValue;
    }
#undef DWARF_Q6W_CASE
    return hipGetLastError();
  }
  return launch_prefill_rows<true>(a, xr, tiles, total, stream);
}

size_t q6_decode_workspace(const dwarf_dsqg_q6_decode_args& a) {
  return static_cast<size_t>(a.S) * a.L * a.H * dec_layout(a.J, a.H).JE * sizeof(float);
}

hipError_t launch_q6_decode(const dwarf_dsqg_q6_decode_args& a, float* T, hipStream_t stream) {
  const DecLayout lay = dec_layout(a.J, a.H);
  const int table_blocks = a.L * ((a.S * a.H + kTabRows - 1) / kTabRows);
  hipLaunchKernelGGL(q6_decode_table, dim3(table_blocks), dim3(kBlock), dec_table_lds(lay.JE, a.H, !a.se_round_bf16),
                     stream, a, T, lay.JE);
  constexpr int HPW = kDecHeadsPerWg;
  const int wpb = a.H < HPW ? a.H : HPW;
  const int blocks = a.S * a.L * ((a.H + HPW - 1) / HPW);
  const size_t lds = static_cast<size_t>(wpb) * lay.list_len * 8;
#define DWARF_Q6D_CASE(S) \
  case S: hipLaunchKernelGGL(q6_decode_q4<S>, dim3(blocks), dim3(kWave * wpb), lds, stream, a, T); break;
  switch (a.plane_shift) {
    DWARF_Q6D_CASE(0) DWARF_Q6D_CASE(1) DWARF_Q6D_CASE(2) DWARF_Q6D_CASE(3) DWARF_Q6D_CASE(4)
    DWARF_Q6D_CASE(5) DWARF_Q6D_CASE(6) DWARF_Q6D_CASE(7) DWARF_Q6D_CASE(8) DWARF_Q6D_CASE(9)
    DWARF_Q6D_CASE(10) DWARF_Q6D_CASE(11) DWARF_Q6D_CASE(12) DWARF_Q6D_CASE(13) DWARF_Q6D_CASE(14)
    default: return hipErrorInvalidValue;
  }
#undef DWARF_Q6D_CASE
  return hipGetLastError();
}

int q6_max_decode_offsets() { return kMaxDecOffsets; }
int q6_max_decode_heads() { return kMaxDecHeads; }

}  // namespace dwarf

// ---------------------------------------------------------------------------
// Score table of the no-allocation decode step: a file-scope device array,
// one copy per GPU, held from module load until the process ends.  In host
// code `scratch` names a host-side stand-in, not device memory: its device
// address comes from hipGetSymbolAddress, looked up once per device (with
// that device current) and kept per device.  Every no-allocation decode on a
// GPU uses that GPU's one copy, so calls that overlap on one GPU race; each
// call rewrites every table entry it reads, so nothing needs clearing.
// ---------------------------------------------------------------------------
static __device__ __align__(256) float scratch[DWARF_Q6_DECODE_SCRATCH_BYTES / sizeof(float)];

namespace dwarf {

// The array of the GPU that `stream` belongs to (the current GPU for the null
// stream).  Its address is looked up with that GPU current, once per GPU.
hipError_t q6_decode_scratch(hipStream_t stream, float** ptr) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static float* addr[kMaxDevices] = {};
  int cur = -1;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return e;
  int dev = cur;
  if (stream != nullptr) {
    hipDevice_t sd = -1;
    if ((e = hipStreamGetDevice(stream, &sd)) != hipSuccess) return e;
    dev = static_cast<int>(sd);
  }
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess) return e;
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) {
      const hipError_t r = hipSetDevice(cur);
      if (e == hipSuccess) e = r;
    }
    if (e != hipSuccess) return e;
    addr[dev] = static_cast<float*>(p);
  }
  *ptr = addr[dev];
  return hipSuccess;
}

}  // namespace dwarf
