/*
 * dwarf_dsqg.h -- C ABI of the MI355X (gfx950) DSQG offset-gather library.
 *
 * One shared library, libdwarf_dsqg.so, exports every entry point below.
 * The ABI carries plain device pointers, element strides and a hipStream_t;
 * no framework types cross it.  The caller owns every buffer: outputs,
 * gradients and the workspaces whose sizes the *_workspace_bytes queries
 * report.  Every entry point launches on the stream it is given, never
 * allocates device memory and never throws.  Every entry point but one is
 * stateless and re-entrant: dwarf_dsqg_q6_decode_noalloc keeps its score
 * table in one device array per GPU, so its calls that overlap on one GPU
 * race (see its declaration).  Each returns a dwarf_status;
 * dwarf_last_error() describes the most recent failure on the calling thread.
 *
 * Reference interfaces replaced (Lanerra/dwarf-v2):
 *   dsqg = kernels/dsqg_attention_v22.py, ema = kernels/causal_ema_scan.py
 */
#ifndef DWARF_DSQG_H
#define DWARF_DSQG_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DWARF_ABI_VERSION 9
#define DWARF_R_PLANES 4        /* MOVT planes per far offset: dsqg:69 */
#define DWARF_Q6_GROUP 32       /* head-dim elements per q6 scale group */
#define DWARF_Q6_SLOT_BYTES 128 /* one q6 K/V cache slot per (b, kv head, t) */
#define DWARF_Q6_DECODE_SCRATCH_BYTES (16u << 20) /* per-GPU score table of dwarf_dsqg_q6_decode_noalloc */

typedef struct ihipStream_t* dwarf_stream_t; /* == hipStream_t */

typedef enum {
  DWARF_OK = 0,
  DWARF_ERR_INVALID_ARGUMENT = 1, /* shapes, strides, offsets (ValueError)      */
  DWARF_ERR_UNSUPPORTED = 2,      /* legal but not built here (RuntimeError)     */
  DWARF_ERR_HIP = 3,              /* a HIP runtime call failed                   */
  DWARF_ERR_WORKSPACE = 4         /* workspace pointer missing or too small      */
} dwarf_status;

typedef enum { DWARF_BF16 = 0, DWARF_F32 = 1 } dwarf_dtype;

/* Library version (DWARF_ABI_VERSION) and last-error text for this thread. */
int dwarf_abi_version(void);
const char* dwarf_last_error(void);

/* ------------------------------------------------------------------------ */
/* DSQG offset-gather attention                                              */
/* ------------------------------------------------------------------------ */

/*
 * Forward inputs.  Shapes: q [B,H,N,hd]; k, v [B,H_kv,N,hd]; pos_bias [J,H];
 * scale_embed [J,hd]; phase_base, phase_gain [max(J_large,1),H,4];
 * y_pre [B,H,N,4]; z_pre [B,H_kv,N,4]; offsets [J] int32 on the device, in the
 * canonical order [small <= 28 ascending | large >= 48 ascending]; out like q;
 * lse [B,H,N] fp32.  Strides are in elements.  q/k/v/out need unit stride on
 * the last dimension and 16-byte aligned rows; the 4-plane tables need unit
 * stride on the plane dimension.  hd must be 64.
 *
 * se_round_bf16 = 1 rounds scale_embed to bf16 before use, as the reference's
 * GPU kernels do (dsqg:760-763); 0 uses it unrounded, as the eager oracle does
 * (dsqg:2660).  Rows n < query_start are written as out = 0, lse = -inf
 * (dsqg:2265-2268).
 */
typedef struct {
  int32_t B, H, H_kv, N, head_dim;
  int32_t J, J_small, J_large;
  int32_t plane_shift, query_start;
  int32_t dtype;          /* dwarf_dtype of q, k, v, out */
  int32_t se_round_bf16;
  const void* q;  int64_t q_stride[4];
  const void* k;  int64_t k_stride[4];
  const void* v;  int64_t v_stride[4];
  const float* pos_bias;    int64_t pb_stride[2];
  const float* scale_embed; int64_t se_stride[2];
  const float* phase_base;  int64_t pbase_stride[2];
  const float* phase_gain;  int64_t pgain_stride[2];
  const float* y_pre; int64_t y_stride[3];
  const float* z_pre; int64_t z_stride[3];
  const int32_t* offsets;
  void* out;  int64_t out_stride[4];
  float* lse; int64_t lse_stride[3];
  int32_t schedule;       /* DWARF_SCHED_* bit flags: which schedule of the same mathematics runs */
  /* Phase-probe features inside the kernels (bf16 only); NULL for the
   * reference op's contract, where y_pre and z_pre are inputs and dy_pre and
   * dz_pre outputs.  [4][hd] fp32, contiguous, 16-byte aligned, rows already
   * normalised (the block's F.normalize of its probes, dsqg:3231-3232). */
  const float* query_probes;
  const float* key_probes;
  float* y_out;           /* [B,H,N,4] fp32 contiguous: y written by the forward when query_probes is set */
} dwarf_dsqg_fwd_args;

/*
 * The probe features inside the kernels replace the DSQG block's y/z einsum
 * (DSQGAttentionV19.forward, dsqg:3231-3254: y = <q, p_r> / sqrt(|q|^2 + 1e-6
 * hd), z likewise from k) and its backward:
 *   - query_probes set: dwarf_dsqg_fwd forms y of every query row from q in
 *     its prologue instead of reading y_pre (which may then be NULL) and
 *     writes it to y_out (every row n < N).  The backward takes that y as
 *     y_pre and adds dy's contribution to dq in the dQ launch's epilogue,
 *     through the normalisation (dq += s sum_r dy_r p_r - s^2 (sum_r dy_r
 *     y_r) q, s = 1 / sqrt(|q|^2 + 1e-6 hd)), instead of writing dy_pre
 *     (which may then be NULL).
 *   - key_probes set: z_pre holds the key features (for instance from
 *     dwarf_phase_probe_fwd over k), and the dK/dV launch adds dz's
 *     contribution to dk in its epilogue the same way instead of writing
 *     dz_pre (which may then be NULL).  The forward does not read key_probes.
 * The probe gradients are not formed (the trainer's probes are frozen,
 * train:311); a caller that trains them uses y_pre/z_pre as the reference op
 * does.
 */

/*
 * Schedules (dwarf_dsqg_fwd_args.schedule).  They compute the same function;
 * results differ only by fp32 summation order.
 *   DWARF_SCHED_BAND: the bf16 forward, dQ and dK/dV launches serve the
 *     leading small offsets (ascending, <= 32) as a dense band on the matrix
 *     cores from K/V (forward, dQ) or q/dO (dK/dV) windows in LDS, the
 *     reference's overlap-slab formulation of the near offsets (grouped_mode
 *     overlap_slab / overlap_slab_bwd, dsqg:1047-1256, 1491-1727, 1957-2187);
 *     the two-pass forward and fp32 launches ignore it.
 *   DWARF_SCHED_TWO_PASS: the forward takes each row's score maximum first and
 *     then forms the softmax and the weighted sum without rescaling: the
 *     reference's offline-softmax kernel (online_softmax=False,
 *     _fwd_v18_grouped dsqg:863-1044).
 *   DWARF_SCHED_DELTA_STAGE: the backward's (delta, lse) pairs come from
 *     dwarf_dsqg_bwd_delta (bf16): the dQ launch forms delta for itself but
 *     does not write the pairs, and runs 400 persistent workgroups (about
 *     three per two CUs) so that a dK/dV launch on another stream can run
 *     beside it (the overlapped
 *     backward: delta then dK/dV on one stream, dQ then params on another).
 *     dwarf_dsqg_bwd, which runs every stage on one stream, then launches the
 *     delta stage first by itself.
 */
#define DWARF_SCHED_BAND 1
#define DWARF_SCHED_TWO_PASS 2
#define DWARF_SCHED_DELTA_STAGE 4

/*
 * Replaces the forward launch of _DSQGV18GroupedFn.forward (dsqg:2300-2314,
 * kernel _fwd_v22_online dsqg:698-860) together with the out/lse
 * initialisation it relies on (dsqg:2267-2268).
 */
int dwarf_dsqg_fwd(const dwarf_dsqg_fwd_args* args, dwarf_stream_t stream);

/*
 * Backward.  `fwd` holds the forward inputs plus the saved out and lse.
 * Gradient outputs: dq like q, dk/dv like k (all of `dtype`, written, not
 * accumulated); dpos_bias [J,H], dscale_embed [J,hd], dphase_base and
 * dphase_gain [max(J_large,1),H,4], dy_pre [B,H,N,4], dz_pre [B,H_kv,N,4],
 * all fp32 and contiguous.  Parameter gradients are reduced in a fixed order,
 * so results are bitwise reproducible run to run.
 */
typedef struct {
  dwarf_dsqg_fwd_args fwd;
  const void* dout; int64_t dout_stride[4];
  void* dq; int64_t dq_stride[4];
  void* dk; int64_t dk_stride[4];
  void* dv; int64_t dv_stride[4];
  float* dpos_bias;
  float* dscale_embed;
  float* dphase_base;
  float* dphase_gain;
  float* dy_pre;
  float* dz_pre;
  void* workspace; size_t workspace_bytes;
} dwarf_dsqg_bwd_args;

/* Bytes of device workspace dwarf_dsqg_bwd needs for these shapes. */
size_t dwarf_dsqg_bwd_workspace_bytes(const dwarf_dsqg_bwd_args* args);

/*
 * Replaces _DSQGV18GroupedFn.backward's launches (dsqg:2354-2552): the delta
 * pass _compute_D_v18_grouped (dsqg:1263-1289), the query-centric
 * _bwd_dq_v18_grouped (dsqg:1296-1488) and the key-centric
 * _bwd_dkdv_v18_grouped (dsqg:1734-1955), including native GQA.
 */
int dwarf_dsqg_bwd(const dwarf_dsqg_bwd_args* args, dwarf_stream_t stream);

/*
 * The same backward as three stages on one stream, sharing the workspace;
 * dq runs first, params and dkdv after it in either order.
 * dwarf_dsqg_bwd_dq replaces _compute_D_v18_grouped plus the query-centric
 * part of _bwd_dq_v18_grouped (dsqg:2378-2454): it writes delta and the
 * parameter-gradient inputs into the workspace, dq and dy_pre.
 * dwarf_dsqg_bwd_params completes the atomic parameter-gradient sums of
 * _bwd_dq_v18_grouped and _bwd_dkdv_v18_grouped (dsqg:1388-1392, 1464-1470, 1905-1907)
 * as fixed-order reductions: dpos_bias, dscale_embed, dphase_base and
 * dphase_gain.  dwarf_dsqg_bwd_dkdv replaces _bwd_dkdv_v18_grouped
 * (dsqg:2456-2544): it reads delta and writes dk, dv and dz_pre; in bf16
 * with grouped heads on a grid of fewer than 1536 (key tile, KV head) units
 * it splits the query heads of the units past the first 768 (of every
 * unit below 768) into subsets and keeps their fp32 partials in a
 * workspace region of its own (no other stage touches it), summed in fixed
 * order.  Fields a stage does not write may be NULL.
 */
int dwarf_dsqg_bwd_dq(const dwarf_dsqg_bwd_args* args, dwarf_stream_t stream);
int dwarf_dsqg_bwd_params(const dwarf_dsqg_bwd_args* args, dwarf_stream_t stream);
int dwarf_dsqg_bwd_dkdv(const dwarf_dsqg_bwd_args* args, dwarf_stream_t stream);

/*
 * The delta stage alone (bf16): replaces _compute_D_v18_grouped
 * (dsqg:1263-1289, launched at dsqg:2380-2386), delta = <dO, O> from the
 * stored bf16 O, and writes the (delta, lse) pairs that dwarf_dsqg_bwd_dkdv
 * reads, bit for bit as dwarf_dsqg_bwd_dq forms them.  With
 * DWARF_SCHED_DELTA_STAGE in args->fwd.schedule the stages may run as
 * delta -> dkdv on one stream beside dq -> params on another.
 */
int dwarf_dsqg_bwd_delta(const dwarf_dsqg_bwd_args* args, dwarf_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Causal EMA scan  y[t] = a*x[t] + (1-a)*y[t-1],  a = clamp(alpha, fl, ce)  */
/* ------------------------------------------------------------------------ */

/*
 * x, y [B,N,D] of `dtype` (unit stride on D); alpha fp32 on the device, one
 * value (alpha_per_channel = 0, the reference's contract, ema:557-558) or D
 * values (alpha_per_channel = 1).  State is fp32.  reset, when not NULL,
 * holds one byte per (b, t): nonzero zeroes the state before token t, the
 * reset-aware scan of _CausalEMAResetFn (ema:368-509).
 */
typedef struct {
  int32_t B, N, D;
  int32_t dtype;
  int32_t alpha_per_channel;
  float floor_, ceiling;
  const void* x; int64_t x_stride[3];
  const float* alpha;
  void* y; int64_t y_stride[3];
  void* workspace; size_t workspace_bytes;
  const uint8_t* reset; int64_t reset_stride[2];  /* [B,N] bool (1 byte), or NULL */
  int32_t wait_limit;     /* polls before a look-back wait gives up (0: the default, 1 << 22) */
} dwarf_ema_fwd_args;

size_t dwarf_ema_fwd_workspace_bytes(const dwarf_ema_fwd_args* args);

/* Replaces _CausalEMAFn.forward's three launches (ema:265-313) and, with
 * reset flags, _CausalEMAResetFn.forward's serial launch (ema:455-476).
 * Where each [N][D] slab of x and y spans less than 2 GiB the scan is one
 * pass with decoupled look-back (a zeroing launch, then the scan): each
 * workgroup of four 128-token tiles publishes its chunk state in the
 * workspace and waits for those of the workgroups before it, at most
 * wait_limit polls per wait; a wait that gives up writes NaN for its
 * channel's workgroup instead of hanging.  Larger slabs take a three-stage chunked scan.  Calls that share
 * a workspace must not overlap. */
int dwarf_ema_fwd(const dwarf_ema_fwd_args* args, dwarf_stream_t stream);

/*
 * dx [B,N,D] of `dtype`; dalpha fp32 with alpha's length, written (not
 * accumulated), already projected for the clamp as ema:357-364 does.
 * Pass dalpha = NULL when alpha needs no gradient.
 */
typedef struct {
  int32_t B, N, D;
  int32_t dtype;
  int32_t alpha_per_channel;
  float floor_, ceiling;
  const void* x;  int64_t x_stride[3];
  const void* y;  int64_t y_stride[3];
  const void* dy; int64_t dy_stride[3];
  const float* alpha;
  void* dx; int64_t dx_stride[3];
  float* dalpha;
  void* workspace; size_t workspace_bytes;
  const uint8_t* reset; int64_t reset_stride[2];  /* the forward's reset flags, or NULL */
  int32_t wait_limit;     /* as in dwarf_ema_fwd_args */
} dwarf_ema_bwd_args;

size_t dwarf_ema_bwd_workspace_bytes(const dwarf_ema_bwd_args* args);

/* Replaces _CausalEMAFn.backward's three launches (ema:315-364) and, with
 * reset flags, _CausalEMAResetFn.backward's serial launch (ema:478-509).
 * The same scan in reverse time (look-back or three-stage), then the
 * fixed-order dalpha reduction. */
int dwarf_ema_bwd(const dwarf_ema_bwd_args* args, dwarf_stream_t stream);

/* ------------------------------------------------------------------------ */
/* InterferencePacket pool: K causal EMA scans of one input and their mix    */
/* ------------------------------------------------------------------------ */

/*
 * x [B,N,D] of `dtype` (unit stride on D); alpha [K] and weight [K] fp32 on
 * the device, 1 <= K <= DWARF_PACKET_MAX_SCALES.  Computes
 *   scan_k = EMA(x, clamp(alpha[k], floor_, ceiling)), stored in dtype,
 *   pooled = (((w_0 scan_0) + w_1 scan_1) + ...), w_k = weight[k] in dtype,
 * every product and partial sum rounded to dtype as the reference's tensor
 * arithmetic rounds them (train:262-267 with K = 3 timescales).  `state`
 * (dwarf_packet_pool_state_bytes, fp32) receives each 16-token chunk's
 * incoming scan states; the backward reads it.  Workspaces are 16-byte
 * aligned.  Where every [N][D] slab of the operands spans less than 2 GiB,
 * forward and backward each run as one pass with the EMA's decoupled
 * look-back (a wait that gives up after 2^22 polls poisons its channels
 * with NaN instead of hanging); larger slabs take the three-stage scans.
 */
#define DWARF_PACKET_MAX_SCALES 4

typedef struct {
  int32_t B, N, D, K;
  int32_t dtype;
  float floor_, ceiling;
  const void* x; int64_t x_stride[3];
  const float* alpha;
  const float* weight;
  void* pooled; int64_t pooled_stride[3];
  float* state;
  void* workspace; size_t workspace_bytes;
} dwarf_packet_pool_fwd_args;

size_t dwarf_packet_pool_state_bytes(const dwarf_packet_pool_fwd_args* args);
size_t dwarf_packet_pool_fwd_workspace_bytes(const dwarf_packet_pool_fwd_args* args);

/* Replaces InterferencePacket.forward's K causal_ema_scan calls and the
 * weighted sum of their outputs (train:262-267). */
int dwarf_packet_pool_fwd(const dwarf_packet_pool_fwd_args* args, dwarf_stream_t stream);

/*
 * fwd as passed to the forward (pooled and fwd.workspace unused, state
 * read); dx [B,N,D] of `dtype`; dalpha [K] (projected for each factor's clamp
 * as ema:357-364 does) and dweight [K] (sum of dpooled * scan_k, rounded to
 * dtype) are written, each may be NULL.
 */
typedef struct {
  dwarf_packet_pool_fwd_args fwd;
  const void* dpooled; int64_t dpooled_stride[3];
  void* dx; int64_t dx_stride[3];
  float* dalpha;
  float* dweight;
  void* workspace; size_t workspace_bytes;
} dwarf_packet_pool_bwd_args;

size_t dwarf_packet_pool_bwd_workspace_bytes(const dwarf_packet_pool_bwd_args* args);

/* The gradients autograd forms for those K scans and the mix: x (summed over
 * the scans), each factor, each weight. */
int dwarf_packet_pool_bwd(const dwarf_packet_pool_bwd_args* args, dwarf_stream_t stream);

/*
 * InterferencePacket packet (train:262-273): the pool above, then per token,
 * with u the pooled values as stored,
 *   ms = mean_d u^2                      (written to ms[b*N + n], fp32)
 *   packet = P(((u rsqrt(ms + 1e-6)) tanh(sqrt(ms) / 0.25)) sigmoid(gate))
 * where gate [B,N,D] holds gate_proj's output (the logits) and P is
 * packet_dtype, the dtype of gate and packet (the reference casts the packet
 * to the block input's dtype).  pool.pooled is written (the backward reads
 * it); pool.workspace and pool.state as for the pool.  D <= 4096 (D <= 1024
 * when D % 4 != 0): a row's channels are the lanes of one workgroup.
 */
typedef struct {
  dwarf_packet_pool_fwd_args pool;
  int32_t packet_dtype;
  const void* gate; int64_t gate_stride[3];
  void* packet; int64_t packet_stride[3];
  float* ms;  /* [B*N] */
} dwarf_packet_fwd_args;

/* Replaces InterferencePacket.forward up to the packet (train:262-273): the
 * K scans, their mix, the RMS direction, the confidence and the gate. */
int dwarf_packet_fwd(const dwarf_packet_fwd_args* args, dwarf_stream_t stream);

/*
 * fwd as passed to the forward (pool.x, pool.pooled, pool.state, gate and ms
 * read); dpacket [B,N,D] and dgate [B,N,D] (the gradient of the logits) of
 * packet_dtype; dx, dalpha, dweight as for the pool's backward.
 */
typedef struct {
  dwarf_packet_fwd_args fwd;
  const void* dpacket; int64_t dpacket_stride[3];
  void* dgate; int64_t dgate_stride[3];
  void* dx; int64_t dx_stride[3];
  float* dalpha;
  float* dweight;
  void* workspace; size_t workspace_bytes;
} dwarf_packet_bwd_args;

/* The pool backward's workspace plus B*N*D values of pool.dtype (dpooled). */
size_t dwarf_packet_bwd_workspace_bytes(const dwarf_packet_bwd_args* args);

/* The gradients autograd forms for train:262-273: x, each factor, each
 * weight and the gate logits.  sqrt(ms) = 0 gives NaN as in the reference. */
int dwarf_packet_bwd(const dwarf_packet_bwd_args* args, dwarf_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Phase-probe features  y[b,h,n,r] = <x, p_r> / sqrt(|x|^2 + 1e-6 hd)       */
/* ------------------------------------------------------------------------ */

/*
 * x [B,H,N,hd] of `dtype` (unit stride on hd, 16-byte aligned rows); probes
 * [R,hd] fp32, contiguous and 16-byte aligned; R = DWARF_R_PLANES, hd = 64.
 * out [B,H,N,R] fp32, any strides.  Rows n in [start, end) get the features
 * and every other row is written 0; start and end are clamped to [0, N] as
 * dsqg:377-379 does.
 */
typedef struct {
  int32_t B, H, N, head_dim, R;
  int32_t start, end;
  int32_t dtype;
  const void* x; int64_t x_stride[4];
  const float* probes;
  float* out; int64_t out_stride[4];
} dwarf_phase_probe_fwd_args;

/* Replaces _PhaseProbeFn.forward's launch (dsqg:371-392; kernel dsqg:275-306). */
int dwarf_phase_probe_fwd(const dwarf_phase_probe_fwd_args* args, dwarf_stream_t stream);

/*
 * dout [B,H,N,R] fp32, any strides.  dx like x (unit stride on hd, 16-byte
 * aligned rows), written, 0 outside [start, end).  dprobes [R,hd] fp32
 * written in a fixed summation order, or NULL when the probes need no
 * gradient.  fwd.out is not used.
 */
typedef struct {
  dwarf_phase_probe_fwd_args fwd;
  const float* dout; int64_t dout_stride[4];
  void* dx; int64_t dx_stride[4];
  float* dprobes;
  void* workspace; size_t workspace_bytes;
} dwarf_phase_probe_bwd_args;

size_t dwarf_phase_probe_bwd_workspace_bytes(const dwarf_phase_probe_bwd_args* args);

/* Replaces _PhaseProbeFn.backward's launch (dsqg:394-419; kernel dsqg:309-369). */
int dwarf_phase_probe_bwd(const dwarf_phase_probe_bwd_args* args, dwarf_stream_t stream);

/* ------------------------------------------------------------------------ */
/* NPCI rotation of K/V rows toward an injected delta (kv_inject)            */
/* ------------------------------------------------------------------------ */

/*
 * x, delta [B,H,T,hd] (unit stride on hd, 16-byte aligned rows; x bf16 or
 * fp32 as x_dtype, delta as delta_dtype), theta [H] fp32, strength_tau > 0;
 * out [B,H,T,hd] of x_dtype.  Per row: n = max(|x|, 1e-12), u = x/n,
 * p = d - (d.u)u, m = |p|; where m > 1e-7 n, out = cos(a) x + sin(a) n p/m
 * with a = theta_h tanh(m / (tau n + 1e-12)), else out = x.  hd = 64.
 */
typedef struct {
  int32_t B, H, T, head_dim;
  int32_t x_dtype, delta_dtype;
  float strength_tau;
  const void* x; int64_t x_stride[4];
  const void* delta; int64_t delta_stride[4];
  const float* theta;
  void* out; int64_t out_stride[4];
} dwarf_npci_fwd_args;

/* Replaces npci_rotate's forward (dsqg:221-254), as applied at dsqg:3196-3229. */
int dwarf_npci_fwd(const dwarf_npci_fwd_args* args, dwarf_stream_t stream);

/*
 * grad [B,H,T,hd] of x_dtype (the output's gradient); dx of x_dtype and
 * ddelta of delta_dtype (both written, same layout rules as x); dtheta [H]
 * fp32 written in a fixed summation order.  fwd.out is not used.
 */
typedef struct {
  dwarf_npci_fwd_args fwd;
  const void* grad; int64_t grad_stride[4];
  void* dx; int64_t dx_stride[4];
  void* ddelta; int64_t ddelta_stride[4];
  float* dtheta;
  void* workspace; size_t workspace_bytes;
} dwarf_npci_bwd_args;

size_t dwarf_npci_bwd_workspace_bytes(const dwarf_npci_bwd_args* args);

/* The gradients autograd forms for npci_rotate (dsqg:221-254): x, delta, theta. */
int dwarf_npci_bwd(const dwarf_npci_bwd_args* args, dwarf_stream_t stream);

/* ------------------------------------------------------------------------ */
/* q6 K/V cache (no reference counterpart in the reference repository;      */
/* signed 6-bit codes, 4 codes per 3 bytes, group 32, fp16 absmax scale)     */
/* ------------------------------------------------------------------------ */

/*
 * Quantise K and V rows into q6 cache slots.  k, v [B,H_kv,N,hd] of `dtype`;
 * cache [B,H_kv,N] slots of DWARF_Q6_SLOT_BYTES with byte strides
 * cache_stride[3] (slot stride must be 128).  Slot layout for hd = 64:
 * bytes 0-47 K codes, 48-51 K fp16 scales, 52-99 V codes, 100-103 V scales,
 * 104-119 z[4] fp32, 120-127 zero.  z is the key-probe feature of the
 * dequantised K row, z_r = <k, p_r> / sqrt(|k|^2 + 1e-6 hd) with the
 * normalised key_probes [4,hd] fp32 (dsqg:3242-3254); key_probes = NULL
 * stores z = 0.  Codes and scales are bit-exact with the CPU codec.
 */
int dwarf_q6_pack_kv(int32_t B, int32_t H_kv, int32_t N, int32_t head_dim,
                     int32_t dtype,
                     const void* k, const int64_t k_stride[4],
                     const void* v, const int64_t v_stride[4],
                     uint8_t* cache, const int64_t cache_stride[3],
                     const float* key_probes,
                     dwarf_stream_t stream);

/* Dequantise cache slots back to fp32 K and V [B,H_kv,N,hd] (contiguous). */
int dwarf_q6_unpack_kv(int32_t B, int32_t H_kv, int32_t N, int32_t head_dim,
                       const uint8_t* cache, const int64_t cache_stride[3],
                       float* k_out, float* v_out, dwarf_stream_t stream);

/*
 * q6 prefill forward: the DSQG forward with K and V dequantised on read from
 * the cache slots.  y is computed in-kernel from q with the normalised
 * query_probes [4,hd] fp32 (dsqg:3234-3249); z is read from the slot (written
 * by dwarf_q6_pack_kv from the dequantised K).  q [B,H,N,hd] bf16; out like q;
 * lse may be NULL.
 *
 * workspace: NULL gathers the 128-byte slots directly and widens every code
 * at each of its uses (no allocation).  Otherwise it must hold
 * dwarf_dsqg_q6_prefill_workspace_bytes() bytes, 256-byte aligned: the
 * launch first widens each cache row once into it (the 6-bit codes as bytes,
 * with the row's scales and z beside them, 160 bytes per row) and the
 * attention gathers those rows.  Both give the same math: codes and scales
 * are exact either way and only the fp32 summation order differs.
 */
typedef struct {
  int32_t B, H, H_kv, N, head_dim;
  int32_t J, J_small, J_large;
  int32_t plane_shift, query_start;
  int32_t se_round_bf16;
  const void* q; int64_t q_stride[4];
  const uint8_t* cache; int64_t cache_stride[3];
  const float* pos_bias;    int64_t pb_stride[2];
  const float* scale_embed; int64_t se_stride[2];
  const float* phase_base;  int64_t pbase_stride[2];
  const float* phase_gain;  int64_t pgain_stride[2];
  const float* query_probes;
  const int32_t* offsets;
  void* out; int64_t out_stride[4];
  float* lse; int64_t lse_stride[3];
  void* workspace; size_t workspace_bytes;
} dwarf_dsqg_q6_prefill_args;

/* Bytes of the widened-row workspace: B * H_kv * N * 160 (0 for bad sizes). */
size_t dwarf_dsqg_q6_prefill_workspace_bytes(const dwarf_dsqg_q6_prefill_args* args);

int dwarf_dsqg_q6_prefill_fwd(const dwarf_dsqg_q6_prefill_args* args,
                              dwarf_stream_t stream);

/*
 * q6 decode step: S sequences x L layers, one new query per (sequence, layer)
 * at position pos[s] (int32, device).  q [S,L,H,hd] bf16; caches
 * [L,S,H_kv,Ncache] slots (byte strides cache_stride[4]); per-layer tables
 * with a leading layer stride (elements); out [S,L,H,hd] bf16.
 */
typedef struct {
  int32_t S, L, H, H_kv, Ncache, head_dim;
  int32_t J, J_small, J_large;
  int32_t plane_shift;
  int32_t se_round_bf16;
  const void* q; int64_t q_stride[4];
  const int32_t* pos;
  const uint8_t* cache; int64_t cache_stride[4];
  const float* pos_bias;    int64_t pb_stride[3];
  const float* scale_embed; int64_t se_stride[3];
  const float* phase_base;  int64_t pbase_stride[3];
  const float* phase_gain;  int64_t pgain_stride[3];
  const float* query_probes; int64_t qprobe_layer_stride; /* [L,4,hd] */
  const int32_t* offsets;    /* [J], shared by all layers */
  void* out; int64_t out_stride[4];
  void* workspace; size_t workspace_bytes;  /* dwarf_dsqg_q6_decode_workspace_bytes, 16-byte aligned */
} dwarf_dsqg_q6_decode_args;

/* The step's per-(sequence, layer, head) score table: S*L*H*JE fp32,
 * JE = (J + 16) rounded down to a multiple of 16. */
size_t dwarf_dsqg_q6_decode_workspace_bytes(const dwarf_dsqg_q6_decode_args* args);

int dwarf_dsqg_q6_decode(const dwarf_dsqg_q6_decode_args* args,
                         dwarf_stream_t stream);

/*
 * The decode step without allocation: no counterpart in the reference.  For
 * callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc).  Same arguments and results
 * as dwarf_dsqg_q6_decode, except that args->workspace is ignored: the score
 * table lives in a file-scope device array of DWARF_Q6_DECODE_SCRATCH_BYTES
 * (16 MiB) per GPU, held until the process ends.  Returns DWARF_ERR_UNSUPPORTED
 * when dwarf_dsqg_q6_decode_workspace_bytes(args) exceeds that size (S*L*H*JE
 * fp32 <= 4 Mi floats, e.g. 512 sequences x 9 layers x 8 heads at J = 96).
 * Calls no allocating routine.  The array used is that of the GPU `stream`
 * belongs to (the current GPU for the null stream).  All calls on one GPU
 * share its array: calls that overlap on one GPU (two streams, two threads)
 * race.
 */
int dwarf_dsqg_q6_decode_noalloc(const dwarf_dsqg_q6_decode_args* args,
                                 dwarf_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* DWARF_DSQG_H */
