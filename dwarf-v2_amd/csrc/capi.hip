// extern "C" entry points of libdwarf_dsqg.so (declared in dwarf_dsqg.h).
// Every argument is validated on the host before a kernel is launched, so a
// malformed call returns a status instead of reaching the GPU.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>

#include "dsqg_internal.h"
#include "dwarf_dsqg.h"

namespace dwarf {
size_t ema_fwd_workspace(int B, int N, int D);
size_t ema_bwd_workspace(int B, int N, int D);
hipError_t launch_ema_fwd(const dwarf_ema_fwd_args& a, hipStream_t stream);
hipError_t launch_ema_bwd(const dwarf_ema_bwd_args& a, hipStream_t stream);
hipError_t launch_q6_pack(int B, int Hkv, int N, int dtype, const void* k, const int64_t* ks, const void* v,
                          const int64_t* vs, uint8_t* cache, const int64_t* cs, const float* kprobe,
                          hipStream_t stream);
hipError_t launch_q6_unpack(int B, int Hkv, int N, const uint8_t* cache, const int64_t* cs, float* kout,
                            float* vout, hipStream_t stream);
hipError_t launch_q6_prefill(const dwarf_dsqg_q6_prefill_args& a, hipStream_t stream);
size_t q6_prefill_workspace(const dwarf_dsqg_q6_prefill_args& a);
hipError_t launch_q6_decode(const dwarf_dsqg_q6_decode_args& a, float* table, hipStream_t stream);
hipError_t q6_decode_scratch(hipStream_t stream, float** ptr);
size_t q6_decode_workspace(const dwarf_dsqg_q6_decode_args& a);
int q6_max_decode_offsets();
int q6_max_decode_heads();
size_t phase_probe_bwd_workspace(const dwarf_phase_probe_bwd_args& a);
size_t npci_bwd_workspace(const dwarf_npci_bwd_args& a);
hipError_t launch_npci_fwd(const dwarf_npci_fwd_args& a, hipStream_t stream);
hipError_t launch_npci_bwd(const dwarf_npci_bwd_args& a, hipStream_t stream);
size_t packet_state_bytes(int B, int N, int D, int K);
size_t packet_fwd_workspace(int B, int N, int D, int K);
size_t packet_bwd_workspace(int B, int N, int D, int K);
int packet_max_scales();
hipError_t launch_packet_fwd(const dwarf_packet_pool_fwd_args& a, hipStream_t stream);
hipError_t launch_packet_bwd(const dwarf_packet_pool_bwd_args& a, hipStream_t stream);
size_t interference_packet_bwd_workspace(int B, int N, int D, int K, int dtype);
int packet_max_row_channels(int D);
hipError_t launch_interference_packet_fwd(const dwarf_packet_fwd_args& a, hipStream_t stream);
hipError_t launch_interference_packet_bwd(const dwarf_packet_bwd_args& a, hipStream_t stream);
hipError_t launch_phase_probe_fwd(const dwarf_phase_probe_fwd_args& a, hipStream_t stream);
hipError_t launch_phase_probe_bwd(const dwarf_phase_probe_bwd_args& a, hipStream_t stream);
}  // namespace dwarf

namespace {

thread_local char g_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_error[0] = '\0';
  return DWARF_OK;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return ok();
  return fail(DWARF_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

// Zeroes n floats: the parameter gradients of a call with no rows (a sum over
// nothing).  A kernel rather than a memset, so the call may be captured in a
// HIP graph.
__global__ void zero_floats_kernel(float* __restrict__ p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

int zero_floats(float* p, int64_t n, hipStream_t stream, const char* what) {
  if (!p || n <= 0) return ok();
  hipLaunchKernelGGL(zero_floats_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, stream, p,
                     static_cast<int>(n));
  return hip_status(hipGetLastError(), what);
}

constexpr int kMaxOffsets = 256;  // LDS tables of the DSQG kernels

size_t elem_size(int dtype) { return dtype == DWARF_BF16 ? 2 : 4; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// A [.., rows, hd] tensor read/written with 16-byte vectors along hd.
int check_rows(const char* name, const void* p, const int64_t* stride, int ndim_outer, int dtype) {
  if (!p) return fail(DWARF_ERR_INVALID_ARGUMENT, "%s is NULL", name);
  if (stride[ndim_outer] != 1) return fail(DWARF_ERR_INVALID_ARGUMENT, "%s needs unit stride on head_dim", name);
  if (!aligned16(p)) return fail(DWARF_ERR_INVALID_ARGUMENT, "%s must be 16-byte aligned", name);
  const int64_t per16 = 16 / static_cast<int64_t>(elem_size(dtype));
  for (int i = 0; i < ndim_outer; ++i)
    if (stride[i] % per16 != 0)
      return fail(DWARF_ERR_INVALID_ARGUMENT, "%s stride[%d]=%lld breaks 16-byte row alignment", name, i,
                  static_cast<long long>(stride[i]));
  return DWARF_OK;
}

// [B,H,N,4] fp32 plane features read as float4.
int check_planes(const char* name, const float* p, const int64_t* stride) {
  if (!p) return fail(DWARF_ERR_INVALID_ARGUMENT, "%s is NULL", name);
  if (!aligned16(p)) return fail(DWARF_ERR_INVALID_ARGUMENT, "%s must be 16-byte aligned", name);
  for (int i = 0; i < 3; ++i)
    if (stride[i] % 4 != 0) return fail(DWARF_ERR_INVALID_ARGUMENT, "%s stride[%d] must be a multiple of 4", name, i);
  return DWARF_OK;
}

int check_lattice(int H, int H_kv, int N, int hd, int J, int J_small, int J_large, int plane_shift, int query_start) {
  if (H <= 0 || H_kv <= 0 || N < 0) return fail(DWARF_ERR_INVALID_ARGUMENT, "bad sizes H=%d H_kv=%d N=%d", H, H_kv, N);
  if (H % H_kv != 0)
    return fail(DWARF_ERR_INVALID_ARGUMENT, "num query heads H=%d must be divisible by KV heads H_kv=%d", H, H_kv);
  if (hd != dwarf::kHeadDim) return fail(DWARF_ERR_UNSUPPORTED, "head_dim=%d is not built (head_dim 64 only)", hd);
  if (J < 1 || J_small < 0 || J_large < 0 || J_small + J_large != J)
    return fail(DWARF_ERR_INVALID_ARGUMENT, "J=%d must equal J_small=%d + J_large=%d and be >= 1", J, J_small, J_large);
  if (J > kMaxOffsets) return fail(DWARF_ERR_UNSUPPORTED, "J=%d exceeds the %d offsets the kernels stage", J, kMaxOffsets);
  const int segment = hd / DWARF_R_PLANES;
  if (plane_shift < 0 || plane_shift > segment - 2)
    return fail(DWARF_ERR_INVALID_ARGUMENT, "plane_shift=%d outside [0, %d]", plane_shift, segment - 2);
  if (query_start < 0 || query_start > N)
    return fail(DWARF_ERR_INVALID_ARGUMENT, "query_start=%d outside [0, N=%d]", query_start, N);
  return DWARF_OK;
}

// The bf16 kernels gather rows with 32-bit buffer offsets row * stride where
// the row index stays within 2N + 128 of zero in either direction.
int check_gather_span(const char* name, int64_t row_stride, int64_t elem, int N) {
  if (row_stride <= 0) return fail(DWARF_ERR_UNSUPPORTED, "%s needs a positive row stride", name);
  if ((2 * static_cast<int64_t>(N) + 128) * row_stride * elem >= (int64_t(1) << 31))
    return fail(DWARF_ERR_UNSUPPORTED, "%s: (2N+128) rows x stride must stay below 2 GiB for 32-bit gathers", name);
  return DWARF_OK;
}

// forward: the arguments of dwarf_dsqg_fwd (y_pre is not read when query_probes is set; y_out is written);
// otherwise those of a backward stage (y_pre holds the forward's y).
int check_fwd(const dwarf_dsqg_fwd_args& a, bool forward) {
  if (a.B < 0) return fail(DWARF_ERR_INVALID_ARGUMENT, "B=%d", a.B);
  int rc = check_lattice(a.H, a.H_kv, a.N, a.head_dim, a.J, a.J_small, a.J_large, a.plane_shift, a.query_start);
  if (rc) return rc;
  if (a.dtype != DWARF_BF16 && a.dtype != DWARF_F32) return fail(DWARF_ERR_INVALID_ARGUMENT, "dtype=%d", a.dtype);
  constexpr int32_t kKnownSchedule = DWARF_SCHED_BAND | DWARF_SCHED_TWO_PASS | DWARF_SCHED_DELTA_STAGE;
  if (a.schedule & ~kKnownSchedule)
    return fail(DWARF_ERR_INVALID_ARGUMENT, "schedule=%d holds bits outside DWARF_SCHED_BAND | TWO_PASS | DELTA_STAGE",
                a.schedule);
  const bool probed = a.query_probes || a.key_probes;
  if (probed && a.dtype != DWARF_BF16)
    return fail(DWARF_ERR_UNSUPPORTED, "query_probes/key_probes (probe features in the kernels) are built for bf16 only");
  if ((a.query_probes && !aligned16(a.query_probes)) || (a.key_probes && !aligned16(a.key_probes)))
    return fail(DWARF_ERR_INVALID_ARGUMENT, "query_probes/key_probes must be 16-byte aligned");
  if (a.B == 0 || a.N == 0) return DWARF_OK;   // no rows to read or write
  const bool reads_y = !(forward && a.query_probes);
  if (forward && a.query_probes && (!a.y_out || !aligned16(a.y_out)))
    return fail(DWARF_ERR_INVALID_ARGUMENT, "y_out must be a 16-byte aligned [B,H,N,4] fp32 buffer when query_probes is set");
  if ((rc = check_rows("q", a.q, a.q_stride, 3, a.dtype))) return rc;
  if ((rc = check_rows("k", a.k, a.k_stride, 3, a.dtype))) return rc;
  if ((rc = check_rows("v", a.v, a.v_stride, 3, a.dtype))) return rc;
  if ((rc = check_rows("out", a.out, a.out_stride, 3, a.dtype))) return rc;
  if (reads_y && (rc = check_planes("y_pre", a.y_pre, a.y_stride))) return rc;
  if ((rc = check_planes("z_pre", a.z_pre, a.z_stride))) return rc;
  if (!a.pos_bias || !a.scale_embed || !a.phase_base || !a.phase_gain || !a.offsets || !a.lse)
    return fail(DWARF_ERR_INVALID_ARGUMENT, "a parameter table, offsets or lse is NULL");
  if (a.dtype == DWARF_BF16) {
    if ((rc = check_gather_span("q", a.q_stride[2], 2, a.N))) return rc;
    if ((rc = check_gather_span("lse", a.lse_stride[2], 4, a.N))) return rc;
    if (reads_y && (rc = check_gather_span("y_pre", a.y_stride[2], 4, a.N))) return rc;
    if ((rc = check_gather_span("k", a.k_stride[2], 2, a.N))) return rc;
    if ((rc = check_gather_span("v", a.v_stride[2], 2, a.N))) return rc;
    if ((rc = check_gather_span("z_pre", a.z_stride[2], 4, a.N))) return rc;
  }
  return DWARF_OK;
}

int check_contig_rows(const char* name, const void* p, const int64_t* stride, int dtype) {
  return check_rows(name, p, stride, 3, dtype);
}

}  // namespace

extern "C" {

int dwarf_abi_version(void) { return DWARF_ABI_VERSION; }

const char* dwarf_last_error(void) { return g_error; }

int dwarf_dsqg_fwd(const dwarf_dsqg_fwd_args* args, dwarf_stream_t stream) {
  if (!args) return fail(DWARF_ERR_INVALID_ARGUMENT, "args is NULL");
  int rc = check_fwd(*args, true);
  if (rc) return rc;
  if (args->B == 0 || args->N == 0) return ok();
  return hip_status(dwarf::launch_dsqg_fwd(*args, reinterpret_cast<hipStream_t>(stream)), "dwarf_dsqg_fwd");
}

size_t dwarf_dsqg_bwd_workspace_bytes(const dwarf_dsqg_bwd_args* args) {
  if (!args) return 0;
  return dwarf::bwd_workspace_layout(*args).total;
}

static int bwd_stage(const dwarf_dsqg_bwd_args* args, dwarf_stream_t stream, bool do_dq, bool do_params,
                     bool do_dkdv, const char* name) {
  if (!args) return fail(DWARF_ERR_INVALID_ARGUMENT, "args is NULL");
  const dwarf_dsqg_bwd_args& a = *args;
  int rc = check_fwd(a.fwd, false);
  if (rc) return rc;
  if (a.fwd.B == 0 || a.fwd.N == 0) {   // the parameter gradients are sums over nothing
    if (!do_params) return ok();
    const dwarf_dsqg_fwd_args& f = a.fwd;
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int64_t jl = f.J_large > 0 ? f.J_large : 1;
    if ((rc = zero_floats(a.dpos_bias, static_cast<int64_t>(f.J) * f.H, s, name))) return rc;
    if ((rc = zero_floats(a.dscale_embed, static_cast<int64_t>(f.J) * f.head_dim, s, name))) return rc;
    if ((rc = zero_floats(a.dphase_base, jl * f.H * DWARF_R_PLANES, s, name))) return rc;
    return zero_floats(a.dphase_gain, jl * f.H * DWARF_R_PLANES, s, name);
  }
  const int dt = a.fwd.dtype;
  if (dt == DWARF_BF16) {
    // the dS matrix of one (b, h) is addressed with 32-bit offsets 4 (j N + n)
    if (4 * static_cast<int64_t>(a.fwd.J) * a.fwd.N >= (int64_t(1) << 31))
      return fail(DWARF_ERR_UNSUPPORTED, "bf16 backward: 4 x J x N bytes of dS per (b, h) must stay below 2 GiB");
    // the dK/dV launch stages every head of a GQA group's tables in LDS
    const size_t lds = dwarf::dkdv_lds_bytes(a.fwd.J, a.fwd.J_large, a.fwd.H / a.fwd.H_kv);
    if (do_dkdv && lds > dwarf::kMaxLdsBytes)
      return fail(DWARF_ERR_UNSUPPORTED, "bf16 dK/dV: %zu bytes of LDS tables for J=%d and %d query heads per KV head "
                  "exceed the %zu bytes of a workgroup", lds, a.fwd.J, a.fwd.H / a.fwd.H_kv, dwarf::kMaxLdsBytes);
  }
  if ((rc = check_contig_rows("dout", a.dout, a.dout_stride, dt))) return rc;
  if (dt == DWARF_BF16 && (rc = check_gather_span("dout", a.dout_stride[2], 2, a.fwd.N))) return rc;
  if (do_dq) {
    if ((rc = check_contig_rows("dq", a.dq, a.dq_stride, dt))) return rc;
    if (!a.fwd.query_probes) {   // with query_probes dy goes into dq instead
      if (!a.dy_pre) return fail(DWARF_ERR_INVALID_ARGUMENT, "dy_pre is NULL");
      if (!aligned16(a.dy_pre)) return fail(DWARF_ERR_INVALID_ARGUMENT, "dy_pre must be 16-byte aligned");
    }
  }
  if (do_params && (!a.dpos_bias || !a.dscale_embed || !a.dphase_base || !a.dphase_gain))
    return fail(DWARF_ERR_INVALID_ARGUMENT, "a parameter gradient output is NULL");
  if (do_dkdv) {
    if ((rc = check_contig_rows("dk", a.dk, a.dk_stride, dt))) return rc;
    if ((rc = check_contig_rows("dv", a.dv, a.dv_stride, dt))) return rc;
    if (!a.fwd.key_probes) {     // with key_probes dz goes into dk instead
      if (!a.dz_pre) return fail(DWARF_ERR_INVALID_ARGUMENT, "dz_pre is NULL");
      if (!aligned16(a.dz_pre)) return fail(DWARF_ERR_INVALID_ARGUMENT, "dz_pre must be 16-byte aligned");
    }
  }
  const dwarf::BwdWorkspace ws = dwarf::bwd_workspace_layout(a);
  if (!a.workspace || a.workspace_bytes < ws.total)
    return fail(DWARF_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu", ws.total, a.workspace_bytes);
  if ((reinterpret_cast<uintptr_t>(a.workspace) & 255u) != 0)
    return fail(DWARF_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  return hip_status(
      dwarf::launch_dsqg_bwd(a, ws, reinterpret_cast<hipStream_t>(stream), do_dq, do_params, do_dkdv), name);
}

int dwarf_dsqg_bwd(const dwarf_dsqg_bwd_args* args, dwarf_stream_t stream) {
  return bwd_stage(args, stream, true, true, true, "dwarf_dsqg_bwd");
}

int dwarf_dsqg_bwd_dq(const dwarf_dsqg_bwd_args* args, dwarf_stream_t stream) {
  return bwd_stage(args, stream, true, false, false, "dwarf_dsqg_bwd_dq");
}

int dwarf_dsqg_bwd_params(const dwarf_dsqg_bwd_args* args, dwarf_stream_t stream) {
  return bwd_stage(args, stream, false, true, false, "dwarf_dsqg_bwd_params");
}

int dwarf_dsqg_bwd_dkdv(const dwarf_dsqg_bwd_args* args, dwarf_stream_t stream) {
  return bwd_stage(args, stream, false, false, true, "dwarf_dsqg_bwd_dkdv");
}

int dwarf_dsqg_bwd_delta(const dwarf_dsqg_bwd_args* args, dwarf_stream_t stream) {
  if (!args) return fail(DWARF_ERR_INVALID_ARGUMENT, "args is NULL");
  const dwarf_dsqg_bwd_args& a = *args;
  int rc = check_fwd(a.fwd, false);
  if (rc) return rc;
  if (a.fwd.dtype != DWARF_BF16)
    return fail(DWARF_ERR_UNSUPPORTED, "dwarf_dsqg_bwd_delta: bf16 only (the fp32 dQ launch forms delta itself)");
  if (a.fwd.B == 0 || a.fwd.N == 0) return ok();
  if ((rc = check_contig_rows("dout", a.dout, a.dout_stride, a.fwd.dtype))) return rc;
  const dwarf::BwdWorkspace ws = dwarf::bwd_workspace_layout(a);
  if (!a.workspace || a.workspace_bytes < ws.total)
    return fail(DWARF_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu", ws.total, a.workspace_bytes);
  if ((reinterpret_cast<uintptr_t>(a.workspace) & 255u) != 0)
    return fail(DWARF_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  return hip_status(dwarf::launch_dsqg_bwd_delta(a, ws, reinterpret_cast<hipStream_t>(stream)),
                    "dwarf_dsqg_bwd_delta");
}

// ---- EMA --------------------------------------------------------------------
static int check_ema_common(int B, int N, int D, int dtype, int per_channel, float lo, float hi, const float* alpha) {
  if (B < 0 || N < 0 || D < 0) return fail(DWARF_ERR_INVALID_ARGUMENT, "bad sizes B=%d N=%d D=%d", B, N, D);
  if (dtype != DWARF_BF16 && dtype != DWARF_F32) return fail(DWARF_ERR_INVALID_ARGUMENT, "dtype=%d", dtype);
  if (!(lo > 0.f && lo < hi && hi < 1.f))
    return fail(DWARF_ERR_INVALID_ARGUMENT, "EMA bounds must satisfy 0 < floor < ceiling < 1");
  if (per_channel != 0 && per_channel != 1) return fail(DWARF_ERR_INVALID_ARGUMENT, "alpha_per_channel=%d", per_channel);
  if (!alpha) return fail(DWARF_ERR_INVALID_ARGUMENT, "alpha is NULL");
  return DWARF_OK;
}

static int check_btd(const char* name, const void* p, const int64_t* s, int dtype, int D) {
  if (!p) return fail(DWARF_ERR_INVALID_ARGUMENT, "%s is NULL", name);
  if (s[2] != 1) return fail(DWARF_ERR_INVALID_ARGUMENT, "%s needs unit stride on D", name);
  if (D % 4 == 0) {
    const uintptr_t align = dtype == DWARF_BF16 ? 8 : 16;
    if ((reinterpret_cast<uintptr_t>(p) % align) || s[0] % 4 || s[1] % 4)
      return fail(DWARF_ERR_INVALID_ARGUMENT, "%s: with D %% 4 == 0 rows must be %zu-byte aligned", name,
                  static_cast<size_t>(align));
  }
  return DWARF_OK;
}

size_t dwarf_ema_fwd_workspace_bytes(const dwarf_ema_fwd_args* a) {
  return a ? dwarf::ema_fwd_workspace(a->B, a->N, a->D) : 0;
}
size_t dwarf_ema_bwd_workspace_bytes(const dwarf_ema_bwd_args* a) {
  return a ? dwarf::ema_bwd_workspace(a->B, a->N, a->D) : 0;
}

static int check_reset(const uint8_t* reset, const int64_t* rs, int B, int N) {
  if (!reset) return DWARF_OK;
  if (rs[0] < 0 || rs[1] < 0 || (B > 1 && rs[0] == 0) || (N > 1 && rs[1] == 0))
    return fail(DWARF_ERR_INVALID_ARGUMENT, "reset strides (%lld, %lld) do not address a [B,N] mask",
                static_cast<long long>(rs[0]), static_cast<long long>(rs[1]));
  return DWARF_OK;
}

int dwarf_ema_fwd(const dwarf_ema_fwd_args* args, dwarf_stream_t stream) {
  if (!args) return fail(DWARF_ERR_INVALID_ARGUMENT, "args is NULL");
  const dwarf_ema_fwd_args& a = *args;
  int rc = check_ema_common(a.B, a.N, a.D, a.dtype, a.alpha_per_channel, a.floor_, a.ceiling, a.alpha);
  if (rc) return rc;
  if (a.B == 0 || a.N == 0 || a.D == 0) return ok();   // empty x: nothing to read or write
  if ((rc = check_btd("x", a.x, a.x_stride, a.dtype, a.D))) return rc;
  if ((rc = check_btd("y", a.y, a.y_stride, a.dtype, a.D))) return rc;
  if ((rc = check_reset(a.reset, a.reset_stride, a.B, a.N))) return rc;
  const size_t need = dwarf::ema_fwd_workspace(a.B, a.N, a.D);
  if (!a.workspace || a.workspace_bytes < need)
    return fail(DWARF_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu", need, a.workspace_bytes);
  if (!aligned16(a.workspace)) return fail(DWARF_ERR_WORKSPACE, "workspace must be 16-byte aligned");
  return hip_status(dwarf::launch_ema_fwd(a, reinterpret_cast<hipStream_t>(stream)), "dwarf_ema_fwd");
}

int dwarf_ema_bwd(const dwarf_ema_bwd_args* args, dwarf_stream_t stream) {
  if (!args) return fail(DWARF_ERR_INVALID_ARGUMENT, "args is NULL");
  const dwarf_ema_bwd_args& a = *args;
  int rc = check_ema_common(a.B, a.N, a.D, a.dtype, a.alpha_per_channel, a.floor_, a.ceiling, a.alpha);
  if (rc) return rc;
  if (a.B == 0 || a.N == 0 || a.D == 0)   // empty x: dalpha is a sum over nothing
    return zero_floats(a.dalpha, a.alpha_per_channel ? a.D : 1, reinterpret_cast<hipStream_t>(stream), "dwarf_ema_bwd");
  if ((rc = check_btd("x", a.x, a.x_stride, a.dtype, a.D))) return rc;
  if ((rc = check_btd("y", a.y, a.y_stride, a.dtype, a.D))) return rc;
  if ((rc = check_btd("dy", a.dy, a.dy_stride, a.dtype, a.D))) return rc;
  if ((rc = check_btd("dx", a.dx, a.dx_stride, a.dtype, a.D))) return rc;
  if ((rc = check_reset(a.reset, a.reset_stride, a.B, a.N))) return rc;
  const size_t need = dwarf::ema_bwd_workspace(a.B, a.N, a.D);
  if (!a.workspace || a.workspace_bytes < need)
    return fail(DWARF_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu", need, a.workspace_bytes);
  if (!aligned16(a.workspace)) return fail(DWARF_ERR_WORKSPACE, "workspace must be 16-byte aligned");
  return hip_status(dwarf::launch_ema_bwd(a, reinterpret_cast<hipStream_t>(stream)), "dwarf_ema_bwd");
}

// ---- InterferencePacket pool ---------------------------------------------------
static bool packet_empty(const dwarf_packet_pool_fwd_args& a) { return a.B == 0 || a.N == 0 || a.D == 0; }

static int check_packet(const dwarf_packet_pool_fwd_args& a, bool need_pooled) {
  if (a.K < 1 || a.K > dwarf::packet_max_scales() || a.K > DWARF_PACKET_MAX_SCALES)
    return fail(DWARF_ERR_UNSUPPORTED, "K=%d scales (1..%d are built)", a.K, DWARF_PACKET_MAX_SCALES);
  int rc = check_ema_common(a.B, a.N, a.D, a.dtype, 0, a.floor_, a.ceiling, a.alpha);
  if (rc) return rc;
  if (!a.weight) return fail(DWARF_ERR_INVALID_ARGUMENT, "weight is NULL");
  if (packet_empty(a)) return DWARF_OK;   // no rows to read or write
  if ((rc = check_btd("x", a.x, a.x_stride, a.dtype, a.D))) return rc;
  if (need_pooled && (rc = check_btd("pooled", a.pooled, a.pooled_stride, a.dtype, a.D))) return rc;
  if (a.B > 0 && a.N > 0 && a.D > 0 && !a.state) return fail(DWARF_ERR_INVALID_ARGUMENT, "state is NULL");
  if (reinterpret_cast<uintptr_t>(a.state) & 3u) return fail(DWARF_ERR_INVALID_ARGUMENT, "state must be 4-byte aligned");
  return DWARF_OK;
}

size_t dwarf_packet_pool_state_bytes(const dwarf_packet_pool_fwd_args* a) {
  return a && a->K >= 1 && a->K <= DWARF_PACKET_MAX_SCALES ? dwarf::packet_state_bytes(a->B, a->N, a->D, a->K) : 0;
}
size_t dwarf_packet_pool_fwd_workspace_bytes(const dwarf_packet_pool_fwd_args* a) {
  return a && a->K >= 1 && a->K <= DWARF_PACKET_MAX_SCALES ? dwarf::packet_fwd_workspace(a->B, a->N, a->D, a->K) : 0;
}
size_t dwarf_packet_pool_bwd_workspace_bytes(const dwarf_packet_pool_bwd_args* a) {
  const dwarf_packet_pool_fwd_args* f = a ? &a->fwd : nullptr;
  return f && f->K >= 1 && f->K <= DWARF_PACKET_MAX_SCALES ? dwarf::packet_bwd_workspace(f->B, f->N, f->D, f->K) : 0;
}

int dwarf_packet_pool_fwd(const dwarf_packet_pool_fwd_args* args, dwarf_stream_t stream) {
  if (!args) return fail(DWARF_ERR_INVALID_ARGUMENT, "args is NULL");
  const dwarf_packet_pool_fwd_args& a = *args;
  int rc = check_packet(a, true);
  if (rc) return rc;
  if (a.B == 0 || a.N == 0 || a.D == 0) return ok();
  const size_t need = dwarf::packet_fwd_workspace(a.B, a.N, a.D, a.K);
  if (!a.workspace || a.workspace_bytes < need)
    return fail(DWARF_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu", need, a.workspace_bytes);
  if (reinterpret_cast<uintptr_t>(a.workspace) & 15u) return fail(DWARF_ERR_WORKSPACE, "workspace must be 16-byte aligned");
  return hip_status(dwarf::launch_packet_fwd(a, reinterpret_cast<hipStream_t>(stream)), "dwarf_packet_pool_fwd");
}

static int check_packet_rows(const dwarf_packet_fwd_args& p, bool fwd) {
  const dwarf_packet_pool_fwd_args& a = p.pool;
  if (p.packet_dtype != DWARF_BF16 && p.packet_dtype != DWARF_F32)
    return fail(DWARF_ERR_INVALID_ARGUMENT, "packet_dtype=%d", p.packet_dtype);
  if (a.D > dwarf::packet_max_row_channels(a.D))
    return fail(DWARF_ERR_UNSUPPORTED, "D=%d: a row's channels are one workgroup's lanes (D <= %d)", a.D,
                dwarf::packet_max_row_channels(a.D));
  int rc = check_packet(a, fwd);
  if (rc) return rc;
  if (packet_empty(a)) return DWARF_OK;
  if ((rc = check_btd("gate", p.gate, p.gate_stride, p.packet_dtype, a.D))) return rc;
  if (fwd && (rc = check_btd("packet", p.packet, p.packet_stride, p.packet_dtype, a.D))) return rc;
  if (!fwd && (rc = check_btd("pooled", a.pooled, a.pooled_stride, a.dtype, a.D))) return rc;
  if (!p.ms) return fail(DWARF_ERR_INVALID_ARGUMENT, "ms is NULL");
  if (reinterpret_cast<uintptr_t>(p.ms) & 3u) return fail(DWARF_ERR_INVALID_ARGUMENT, "ms must be 4-byte aligned");
  return DWARF_OK;
}

int dwarf_packet_fwd(const dwarf_packet_fwd_args* args, dwarf_stream_t stream) {
  if (!args) return fail(DWARF_ERR_INVALID_ARGUMENT, "args is NULL");
  const dwarf_packet_fwd_args& p = *args;
  int rc = check_packet_rows(p, true);
  if (rc) return rc;
  const dwarf_packet_pool_fwd_args& a = p.pool;
  if (packet_empty(a)) return ok();
  const size_t need = dwarf::packet_fwd_workspace(a.B, a.N, a.D, a.K);
  if (!a.workspace || a.workspace_bytes < need)
    return fail(DWARF_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu", need, a.workspace_bytes);
  if (reinterpret_cast<uintptr_t>(a.workspace) & 15u) return fail(DWARF_ERR_WORKSPACE, "workspace must be 16-byte aligned");
  return hip_status(dwarf::launch_interference_packet_fwd(p, reinterpret_cast<hipStream_t>(stream)), "dwarf_packet_fwd");
}

size_t dwarf_packet_bwd_workspace_bytes(const dwarf_packet_bwd_args* a) {
  const dwarf_packet_pool_fwd_args* f = a ? &a->fwd.pool : nullptr;
  return f && f->K >= 1 && f->K <= DWARF_PACKET_MAX_SCALES && f->B >= 0 && f->N >= 0 && f->D >= 0
             ? dwarf::interference_packet_bwd_workspace(f->B, f->N, f->D, f->K, f->dtype)
             : 0;
}

int dwarf_packet_bwd(const dwarf_packet_bwd_args* args, dwarf_stream_t stream) {
  if (!args) return fail(DWARF_ERR_INVALID_ARGUMENT, "args is NULL");
  const dwarf_packet_bwd_args& p = *args;
  int rc = check_packet_rows(p.fwd, false);
  if (rc) return rc;
  const dwarf_packet_pool_fwd_args& f = p.fwd.pool;
  if (packet_empty(f)) {   // the factor and weight gradients are sums over nothing
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if ((rc = zero_floats(p.dalpha, f.K, s, "dwarf_packet_bwd"))) return rc;
    return zero_floats(p.dweight, f.K, s, "dwarf_packet_bwd");
  }
  if ((rc = check_btd("dpacket", p.dpacket, p.dpacket_stride, p.fwd.packet_dtype, f.D))) return rc;
  if ((rc = check_btd("dgate", p.dgate, p.dgate_stride, p.fwd.packet_dtype, f.D))) return rc;
  if ((rc = check_btd("dx", p.dx, p.dx_stride, f.dtype, f.D))) return rc;
  const size_t need = dwarf::interference_packet_bwd_workspace(f.B, f.N, f.D, f.K, f.dtype);
  if (!p.workspace || p.workspace_bytes < need)
    return fail(DWARF_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu", need, p.workspace_bytes);
  if (reinterpret_cast<uintptr_t>(p.workspace) & 255u) return fail(DWARF_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  return hip_status(dwarf::launch_interference_packet_bwd(p, reinterpret_cast<hipStream_t>(stream)), "dwarf_packet_bwd");
}

int dwarf_packet_pool_bwd(const dwarf_packet_pool_bwd_args* args, dwarf_stream_t stream) {
  if (!args) return fail(DWARF_ERR_INVALID_ARGUMENT, "args is NULL");
  const dwarf_packet_pool_bwd_args& a = *args;
  int rc = check_packet(a.fwd, false);
  if (rc) return rc;
  if (packet_empty(a.fwd)) {   // the factor and weight gradients are sums over nothing
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if ((rc = zero_floats(a.dalpha, a.fwd.K, s, "dwarf_packet_pool_bwd"))) return rc;
    return zero_floats(a.dweight, a.fwd.K, s, "dwarf_packet_pool_bwd");
  }
  if ((rc = check_btd("dpooled", a.dpooled, a.dpooled_stride, a.fwd.dtype, a.fwd.D))) return rc;
  if ((rc = check_btd("dx", a.dx, a.dx_stride, a.fwd.dtype, a.fwd.D))) return rc;
  if (a.fwd.B == 0 || a.fwd.N == 0 || a.fwd.D == 0) return ok();
  const size_t need = dwarf::packet_bwd_workspace(a.fwd.B, a.fwd.N, a.fwd.D, a.fwd.K);
  if (!a.workspace || a.workspace_bytes < need)
    return fail(DWARF_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu", need, a.workspace_bytes);
  if (reinterpret_cast<uintptr_t>(a.workspace) & 15u) return fail(DWARF_ERR_WORKSPACE, "workspace must be 16-byte aligned");
  return hip_status(dwarf::launch_packet_bwd(a, reinterpret_cast<hipStream_t>(stream)), "dwarf_packet_pool_bwd");
}

// ---- phase-probe features ---------------------------------------------------
static int check_probe_fwd(const dwarf_phase_probe_fwd_args& a, bool need_out) {
  if (a.B < 0 || a.H < 0 || a.N < 0) return fail(DWARF_ERR_INVALID_ARGUMENT, "bad sizes B=%d H=%d N=%d", a.B, a.H, a.N);
  if (a.head_dim != dwarf::kHeadDim || a.R != DWARF_R_PLANES)
    return fail(DWARF_ERR_UNSUPPORTED, "phase probes are built for head_dim %d and %d planes (got %d, %d)",
                dwarf::kHeadDim, DWARF_R_PLANES, a.head_dim, a.R);
  if (a.dtype != DWARF_BF16 && a.dtype != DWARF_F32) return fail(DWARF_ERR_INVALID_ARGUMENT, "dtype=%d", a.dtype);
  if (static_cast<int64_t>(a.B) * a.H * a.N >= (int64_t(1) << 31))
    return fail(DWARF_ERR_UNSUPPORTED, "B*H*N must stay below 2^31 rows");
  if (!a.probes || !aligned16(a.probes)) return fail(DWARF_ERR_INVALID_ARGUMENT, "probes NULL or not 16-byte aligned");
  if (static_cast<int64_t>(a.B) * a.H * a.N == 0) return DWARF_OK;   // no rows to read or write
  int rc = check_rows("x", a.x, a.x_stride, 3, a.dtype);
  if (rc) return rc;
  if (need_out && !a.out) return fail(DWARF_ERR_INVALID_ARGUMENT, "out is NULL");
  return DWARF_OK;
}

int dwarf_phase_probe_fwd(const dwarf_phase_probe_fwd_args* args, dwarf_stream_t stream) {
  if (!args) return fail(DWARF_ERR_INVALID_ARGUMENT, "args is NULL");
  int rc = check_probe_fwd(*args, true);
  if (rc) return rc;
  return hip_status(dwarf::launch_phase_probe_fwd(*args, reinterpret_cast<hipStream_t>(stream)),
                    "dwarf_phase_probe_fwd");
}

size_t dwarf_phase_probe_bwd_workspace_bytes(const dwarf_phase_probe_bwd_args* args) {
  return args ? dwarf::phase_probe_bwd_workspace(*args) : 0;
}

int dwarf_phase_probe_bwd(const dwarf_phase_probe_bwd_args* args, dwarf_stream_t stream) {
  if (!args) return fail(DWARF_ERR_INVALID_ARGUMENT, "args is NULL");
  const dwarf_phase_probe_bwd_args& a = *args;
  int rc = check_probe_fwd(a.fwd, false);
  if (rc) return rc;
  if (static_cast<int64_t>(a.fwd.B) * a.fwd.H * a.fwd.N == 0)   // dprobes is a sum over nothing
    return zero_floats(a.dprobes, static_cast<int64_t>(a.fwd.R) * a.fwd.head_dim, reinterpret_cast<hipStream_t>(stream),
                       "dwarf_phase_probe_bwd");
  if (!a.dout) return fail(DWARF_ERR_INVALID_ARGUMENT, "dout is NULL");
  if ((rc = check_rows("dx", a.dx, a.dx_stride, 3, a.fwd.dtype))) return rc;
  if (a.dprobes) {
    const size_t need = dwarf::phase_probe_bwd_workspace(a);
    if (need && (!a.workspace || a.workspace_bytes < need))
      return fail(DWARF_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu", need, a.workspace_bytes);
  }
  return hip_status(dwarf::launch_phase_probe_bwd(a, reinterpret_cast<hipStream_t>(stream)), "dwarf_phase_probe_bwd");
}

// ---- NPCI rotation ----------------------------------------------------------
static int check_npci(const dwarf_npci_fwd_args& a, bool need_out) {
  if (a.B < 0 || a.H < 0 || a.T < 0) return fail(DWARF_ERR_INVALID_ARGUMENT, "bad sizes B=%d H=%d T=%d", a.B, a.H, a.T);
  if (a.head_dim != dwarf::kHeadDim)
    return fail(DWARF_ERR_UNSUPPORTED, "NPCI is built for head_dim %d (got %d)", dwarf::kHeadDim, a.head_dim);
  if (!(a.strength_tau > 0.f) || !(a.strength_tau < 3.0e38f))
    return fail(DWARF_ERR_INVALID_ARGUMENT, "strength_tau must be finite and positive");
  for (int dt : {a.x_dtype, a.delta_dtype})
    if (dt != DWARF_BF16 && dt != DWARF_F32) return fail(DWARF_ERR_INVALID_ARGUMENT, "dtype=%d", dt);
  if (static_cast<int64_t>(a.B) * a.H * a.T >= (int64_t(1) << 31))
    return fail(DWARF_ERR_UNSUPPORTED, "B*H*T must stay below 2^31 rows");
  if (!a.theta && a.H > 0) return fail(DWARF_ERR_INVALID_ARGUMENT, "theta is NULL");
  if (static_cast<int64_t>(a.B) * a.H * a.T == 0) return DWARF_OK;   // no rows to read or write
  int rc = check_rows("x", a.x, a.x_stride, 3, a.x_dtype);
  if (rc) return rc;
  if ((rc = check_rows("delta", a.delta, a.delta_stride, 3, a.delta_dtype))) return rc;
  if (need_out && (rc = check_rows("out", a.out, a.out_stride, 3, a.x_dtype))) return rc;
  return DWARF_OK;
}

int dwarf_npci_fwd(const dwarf_npci_fwd_args* args, dwarf_stream_t stream) {
  if (!args) return fail(DWARF_ERR_INVALID_ARGUMENT, "args is NULL");
  int rc = check_npci(*args, true);
  if (rc) return rc;
  return hip_status(dwarf::launch_npci_fwd(*args, reinterpret_cast<hipStream_t>(stream)), "dwarf_npci_fwd");
}

size_t dwarf_npci_bwd_workspace_bytes(const dwarf_npci_bwd_args* args) {
  return args ? dwarf::npci_bwd_workspace(*args) : 0;
}

int dwarf_npci_bwd(const dwarf_npci_bwd_args* args, dwarf_stream_t stream) {
  if (!args) return fail(DWARF_ERR_INVALID_ARGUMENT, "args is NULL");
  const dwarf_npci_bwd_args& a = *args;
  int rc = check_npci(a.fwd, false);
  if (rc) return rc;
  if (!a.dtheta && a.fwd.H > 0) return fail(DWARF_ERR_INVALID_ARGUMENT, "dtheta is NULL");
  if (static_cast<int64_t>(a.fwd.B) * a.fwd.H * a.fwd.T == 0)   // dtheta is a sum over nothing
    return zero_floats(a.dtheta, a.fwd.H, reinterpret_cast<hipStream_t>(stream), "dwarf_npci_bwd");
  if ((rc = check_rows("grad", a.grad, a.grad_stride, 3, a.fwd.x_dtype))) return rc;
  if ((rc = check_rows("dx", a.dx, a.dx_stride, 3, a.fwd.x_dtype))) return rc;
  if ((rc = check_rows("ddelta", a.ddelta, a.ddelta_stride, 3, a.fwd.delta_dtype))) return rc;
  const size_t need = dwarf::npci_bwd_workspace(a);
  if (need && (!a.workspace || a.workspace_bytes < need))
    return fail(DWARF_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu", need, a.workspace_bytes);
  return hip_status(dwarf::launch_npci_bwd(a, reinterpret_cast<hipStream_t>(stream)), "dwarf_npci_bwd");
}

// ---- q6 ---------------------------------------------------------------------
static int check_cache(const uint8_t* cache, const int64_t* cs, int n_outer) {
  if (!cache) return fail(DWARF_ERR_INVALID_ARGUMENT, "cache is NULL");
  if (!aligned16(cache)) return fail(DWARF_ERR_INVALID_ARGUMENT, "cache must be 16-byte aligned");
  if (cs[n_outer] != DWARF_Q6_SLOT_BYTES)
    return fail(DWARF_ERR_INVALID_ARGUMENT, "cache slot stride must be %d bytes", DWARF_Q6_SLOT_BYTES);
  for (int i = 0; i < n_outer; ++i)
    if (cs[i] % 16) return fail(DWARF_ERR_INVALID_ARGUMENT, "cache stride[%d] must be a multiple of 16", i);
  return DWARF_OK;
}

int dwarf_q6_pack_kv(int32_t B, int32_t H_kv, int32_t N, int32_t head_dim, int32_t dtype, const void* k,
                     const int64_t k_stride[4], const void* v, const int64_t v_stride[4], uint8_t* cache,
                     const int64_t cache_stride[3], const float* key_probes, dwarf_stream_t stream) {
  if (B < 0 || H_kv < 0 || N < 0) return fail(DWARF_ERR_INVALID_ARGUMENT, "bad sizes");
  if (head_dim != dwarf::kHeadDim) return fail(DWARF_ERR_UNSUPPORTED, "head_dim=%d is not built (64 only)", head_dim);
  if (dtype != DWARF_BF16 && dtype != DWARF_F32) return fail(DWARF_ERR_INVALID_ARGUMENT, "dtype=%d", dtype);
  int rc;
  if ((rc = check_rows("k", k, k_stride, 3, dtype))) return rc;
  if ((rc = check_rows("v", v, v_stride, 3, dtype))) return rc;
  if ((rc = check_cache(cache, cache_stride, 2))) return rc;
  if (static_cast<int64_t>(B) * H_kv * N == 0) return ok();
  return hip_status(dwarf::launch_q6_pack(B, H_kv, N, dtype, k, k_stride, v, v_stride, cache, cache_stride,
                                          key_probes, reinterpret_cast<hipStream_t>(stream)),
                    "dwarf_q6_pack_kv");
}

int dwarf_q6_unpack_kv(int32_t B, int32_t H_kv, int32_t N, int32_t head_dim, const uint8_t* cache,
                       const int64_t cache_stride[3], float* k_out, float* v_out, dwarf_stream_t stream) {
  if (B < 0 || H_kv < 0 || N < 0) return fail(DWARF_ERR_INVALID_ARGUMENT, "bad sizes");
  if (head_dim != dwarf::kHeadDim) return fail(DWARF_ERR_UNSUPPORTED, "head_dim=%d is not built (64 only)", head_dim);
  int rc;
  if ((rc = check_cache(cache, cache_stride, 2))) return rc;
  if (!k_out || !v_out) return fail(DWARF_ERR_INVALID_ARGUMENT, "output is NULL");
  if (static_cast<int64_t>(B) * H_kv * N == 0) return ok();
  return hip_status(dwarf::launch_q6_unpack(B, H_kv, N, cache, cache_stride, k_out, v_out,
                                            reinterpret_cast<hipStream_t>(stream)),
                    "dwarf_q6_unpack_kv");
}

size_t dwarf_dsqg_q6_prefill_workspace_bytes(const dwarf_dsqg_q6_prefill_args* args) {
  if (!args || args->B < 0 || args->H_kv < 0 || args->N < 0) return 0;
  return dwarf::q6_prefill_workspace(*args);
}

int dwarf_dsqg_q6_prefill_fwd(const dwarf_dsqg_q6_prefill_args* args, dwarf_stream_t stream) {
  if (!args) return fail(DWARF_ERR_INVALID_ARGUMENT, "args is NULL");
  const dwarf_dsqg_q6_prefill_args& a = *args;
  if (a.B < 0) return fail(DWARF_ERR_INVALID_ARGUMENT, "B=%d", a.B);
  int rc = check_lattice(a.H, a.H_kv, a.N, a.head_dim, a.J, a.J_small, a.J_large, a.plane_shift, a.query_start);
  if (rc) return rc;
  if ((rc = check_rows("q", a.q, a.q_stride, 3, DWARF_BF16))) return rc;
  if ((rc = check_rows("out", a.out, a.out_stride, 3, DWARF_BF16))) return rc;
  if ((rc = check_cache(a.cache, a.cache_stride, 2))) return rc;
  if ((rc = check_gather_span("cache", DWARF_Q6_SLOT_BYTES, 1, a.N))) return rc;
  if (!a.pos_bias || !a.scale_embed || !a.phase_base || !a.phase_gain || !a.offsets || !a.query_probes)
    return fail(DWARF_ERR_INVALID_ARGUMENT, "a parameter table, probe table or offsets is NULL");
  if (a.workspace) {   // the widened-row schedule: 160-byte rows gathered with 32-bit offsets
    if ((rc = check_gather_span("widened cache rows", 160, 1, a.N))) return rc;
    const size_t need = dwarf::q6_prefill_workspace(a);
    if (a.workspace_bytes < need)
      return fail(DWARF_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu", need, a.workspace_bytes);
    if (reinterpret_cast<uintptr_t>(a.workspace) & 255u)
      return fail(DWARF_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  }
  if (a.B == 0 || a.N == 0) return ok();
  return hip_status(dwarf::launch_q6_prefill(a, reinterpret_cast<hipStream_t>(stream)), "dwarf_dsqg_q6_prefill_fwd");
}

size_t dwarf_dsqg_q6_decode_workspace_bytes(const dwarf_dsqg_q6_decode_args* args) {
  if (!args || args->S < 0 || args->L < 0 || args->H < 0 || args->J < 0) return 0;
  return dwarf::q6_decode_workspace(*args);
}

// Shapes and limits of the decode step (no pointer is dereferenced here).
static int check_decode_shape(const dwarf_dsqg_q6_decode_args& a) {
  if (a.S < 0 || a.L < 0 || a.Ncache < 0) return fail(DWARF_ERR_INVALID_ARGUMENT, "bad sizes");
  int rc = check_lattice(a.H, a.H_kv, a.Ncache, a.head_dim, a.J, a.J_small, a.J_large, a.plane_shift, 0);
  if (rc) return rc;
  if (a.J > dwarf::q6_max_decode_offsets())
    return fail(DWARF_ERR_UNSUPPORTED, "decode supports at most %d offsets", dwarf::q6_max_decode_offsets());
  if (a.H > dwarf::q6_max_decode_heads())
    return fail(DWARF_ERR_UNSUPPORTED, "decode runs one wave per head: at most %d heads", dwarf::q6_max_decode_heads());
  if (static_cast<int64_t>(a.Ncache) * DWARF_Q6_SLOT_BYTES >= (int64_t(1) << 31))
    return fail(DWARF_ERR_UNSUPPORTED, "decode gathers with 32-bit offsets: Ncache x 128 B must stay below 2 GiB");
  return DWARF_OK;
}

// Pointers, strides and table layouts of the decode step.
static int check_decode_args(const dwarf_dsqg_q6_decode_args& a) {
  int rc;
  if ((rc = check_rows("q", a.q, a.q_stride, 3, DWARF_BF16))) return rc;
  if ((rc = check_rows("out", a.out, a.out_stride, 3, DWARF_BF16))) return rc;
  if ((rc = check_cache(a.cache, a.cache_stride, 3))) return rc;
  if (!a.pos || !a.pos_bias || !a.scale_embed || !a.phase_base || !a.phase_gain || !a.offsets || !a.query_probes)
    return fail(DWARF_ERR_INVALID_ARGUMENT, "positions, a parameter table, probes or offsets is NULL");
  if (a.pb_stride[1] < 0 || a.pb_stride[2] < 0 ||
      ((static_cast<int64_t>(a.J) - 1) * a.pb_stride[1] + (a.H - 1) * a.pb_stride[2] + 1) * 4 >= (int64_t(1) << 31))
    return fail(DWARF_ERR_UNSUPPORTED, "decode reads a layer's pos_bias with 32-bit offsets (span below 2 GiB)");
  if (a.se_stride[2] != 1) return fail(DWARF_ERR_INVALID_ARGUMENT, "scale_embed needs unit stride on head_dim");
  if (!aligned16(a.scale_embed) || a.se_stride[0] % 4 || a.se_stride[1] % 4)
    return fail(DWARF_ERR_INVALID_ARGUMENT, "scale_embed rows must be 16-byte aligned (read as float4)");
  if (a.se_stride[1] > (int64_t(1) << 20))
    return fail(DWARF_ERR_UNSUPPORTED, "decode reads a layer's scale_embed with 32-bit offsets (row stride <= 2^20)");
  if (a.pbase_stride[1] < 0 || a.pgain_stride[1] < 0 ||
      (a.pbase_stride[1] + a.pgain_stride[1] + DWARF_R_PLANES) * 4 * static_cast<int64_t>(a.J_large) >= (int64_t(1) << 31))
    return fail(DWARF_ERR_UNSUPPORTED, "decode reads a head's phase tables with 32-bit offsets (span below 2 GiB)");
  return DWARF_OK;
}

int dwarf_dsqg_q6_decode(const dwarf_dsqg_q6_decode_args* args, dwarf_stream_t stream) {
  if (!args) return fail(DWARF_ERR_INVALID_ARGUMENT, "args is NULL");
  const dwarf_dsqg_q6_decode_args& a = *args;
  int rc;
  if ((rc = check_decode_shape(a)) || (rc = check_decode_args(a))) return rc;
  if (a.S == 0 || a.L == 0) return ok();
  const size_t need = dwarf::q6_decode_workspace(a);
  if (!a.workspace || a.workspace_bytes < need)
    return fail(DWARF_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu", need, a.workspace_bytes);
  if (!aligned16(a.workspace)) return fail(DWARF_ERR_WORKSPACE, "workspace must be 16-byte aligned");
  return hip_status(dwarf::launch_q6_decode(a, static_cast<float*>(a.workspace), reinterpret_cast<hipStream_t>(stream)),
                    "dwarf_dsqg_q6_decode");
}

int dwarf_dsqg_q6_decode_noalloc(const dwarf_dsqg_q6_decode_args* args, dwarf_stream_t stream) {
  if (!args) return fail(DWARF_ERR_INVALID_ARGUMENT, "args is NULL");
  const dwarf_dsqg_q6_decode_args& a = *args;
  int rc;
  if ((rc = check_decode_shape(a))) return rc;
  const size_t need = dwarf::q6_decode_workspace(a);
  if (need > DWARF_Q6_DECODE_SCRATCH_BYTES)
    return fail(DWARF_ERR_UNSUPPORTED,
                "no-allocation decode: the score table needs %zu bytes (S*L*H*JE fp32), above the %zu-byte "
                "device array; use dwarf_dsqg_q6_decode with a workspace", need,
                static_cast<size_t>(DWARF_Q6_DECODE_SCRATCH_BYTES));
  if ((rc = check_decode_args(a))) return rc;
  if (a.S == 0 || a.L == 0) return ok();
  float* table = nullptr;
  const hipError_t e = dwarf::q6_decode_scratch(reinterpret_cast<hipStream_t>(stream), &table);
  if (e != hipSuccess) return hip_status(e, "dwarf_dsqg_q6_decode_noalloc (device array address)");
  return hip_status(dwarf::launch_q6_decode(a, table, reinterpret_cast<hipStream_t>(stream)),
                    "dwarf_dsqg_q6_decode_noalloc");
}

}  // extern "C"
