"""DSQG offset-gather attention on MI355X: the drop-in for the reference op.

``dsqg_attention_v18_grouped`` keeps the reference signature
(kernels/dsqg_attention_v22.py:2691-2719) and ``_DSQGV18GroupedFn`` keeps the
25-argument autograd contract (dsqg:2194-2552).  Both run the HIP kernels of
libdwarf_dsqg.so through its C ABI; there is no CPU path.  A caller patches
the reference module's global::

    import importlib
    dsqg_amd = importlib.import_module("dwarf-v2_amd.dsqg")
    dsqg_attention_v22.dsqg_attention_v18_grouped = dsqg_amd.dsqg_attention_v18_grouped

Precision: bf16 inputs run the bf16 kernels with the reference GPU path's
numerics (scale embeddings rounded to bf16, dsqg:760-763; fp32 softmax and
accumulation; bf16 outputs and dQ/dK/dV).  fp32 inputs run fp32 kernels with
the eager oracle's numerics (unrounded scale embeddings, dsqg:2660); the
reference GPU path would round them to bf16 first (dsqg:2746-2749).  Any other
dtype is cast to bf16, as the reference does.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .lattice import GROUPED_MODE_IDS, R_PLANES

HEAD_DIM = 64
_SLAB_MODES = (GROUPED_MODE_IDS["overlap_slab"], GROUPED_MODE_IDS["overlap_slab_bwd"])
# Schedule of the baseline mode: the near band of the dQ and dK/dV launches on
# the matrix cores (DWARF_SCHED_BAND) measured faster than the gather loops
# alone at B15 H8 T2048 (dQ 271 vs 280-284 us, dK/dV 241 vs 262-265 us on one
# box), so it is the default; 0 selects the gather loops alone.  The
# overlap-slab modes always set it; online_softmax=False adds
# DWARF_SCHED_TWO_PASS (the offline-softmax forward).
DEFAULT_SCHEDULE = 1


def schedule_for(grouped_mode_id: int, online_softmax: bool) -> int:
    """DWARF_SCHED_* flags for the reference's mode arguments (dsqg:2271-2314, 2394, 2470)."""
    sched = DEFAULT_SCHEDULE
    if int(grouped_mode_id) in _SLAB_MODES:
        sched |= _lib.DWARF_SCHED_BAND
    if not online_softmax:
        sched |= _lib.DWARF_SCHED_TWO_PASS
    return sched


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _rows_ok(t: torch.Tensor) -> bool:
    """Unit head-dim stride and 16-byte aligned rows, as the kernels load them."""
    per16 = 16 // t.element_size()
    return (
        t.stride(-1) == 1
        and t.data_ptr() % 16 == 0
        and all(s % per16 == 0 for s in t.stride()[:-1])
    )


def _kernel_rows(t: torch.Tensor) -> torch.Tensor:
    return t if _rows_ok(t) else t.contiguous()


def _planes(t: torch.Tensor) -> torch.Tensor:
    t = t.contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


def _fill_fwd(a: _lib.DsqgFwdArgs, q, k, v, pos_bias, scale_embed, phase_base, phase_gain, y_pre, z_pre,
              offsets, j_small, j_large, plane_shift, query_start, out, lse, se_round, schedule=0) -> None:
    B, H, N, HD = q.shape
    a.B, a.H, a.H_kv, a.N, a.head_dim = B, H, k.shape[1], N, HD
    a.J, a.J_small, a.J_large = int(j_small) + int(j_large), int(j_small), int(j_large)
    a.plane_shift, a.query_start = int(plane_shift), int(query_start)
    a.dtype = _lib.DWARF_F32 if q.dtype == torch.float32 else _lib.DWARF_BF16
    a.se_round_bf16 = int(se_round)
    a.q, a.q_stride = q.data_ptr(), _lib.i64_array(q.stride())
    a.k, a.k_stride = k.data_ptr(), _lib.i64_array(k.stride())
    a.v, a.v_stride = v.data_ptr(), _lib.i64_array(v.stride())
    a.pos_bias, a.pb_stride = pos_bias.data_ptr(), _lib.i64_array(pos_bias.stride())
    a.scale_embed, a.se_stride = scale_embed.data_ptr(), _lib.i64_array(scale_embed.stride())
    a.phase_base, a.pbase_stride = phase_base.data_ptr(), _lib.i64_array(phase_base.stride()[:2])
    a.phase_gain, a.pgain_stride = phase_gain.data_ptr(), _lib.i64_array(phase_gain.stride()[:2])
    if y_pre is not None:
        a.y_pre, a.y_stride = y_pre.data_ptr(), _lib.i64_array(y_pre.stride()[:3])
    a.z_pre, a.z_stride = z_pre.data_ptr(), _lib.i64_array(z_pre.stride()[:3])
    a.offsets = offsets.data_ptr()
    a.out, a.out_stride = out.data_ptr(), _lib.i64_array(out.stride())
    a.lse, a.lse_stride = lse.data_ptr(), _lib.i64_array(lse.stride())
    a.schedule = int(schedule)


def _device_offsets(offsets_dev: torch.Tensor, device: torch.device, j_val: int) -> torch.Tensor:
    off = offsets_dev
    if off.device != device or off.dtype != torch.int32:
        off = off.to(device=device, dtype=torch.int32)
    off = off.contiguous()
    if off.numel() != j_val:
        raise ValueError(f"offsets_dev has {off.numel()} entries, expected j_val={j_val}")
    return off


def normalize_inputs(q, k, v, pos_bias, scale_embed, phase_base, phase_gain, y_pre, z_pre, offsets_dev, j_val):
    """Layouts the kernels read: q/k/v rows with unit head-dim stride and 16-byte alignment (k/v in q's
    dtype), contiguous fp32 tables and plane features (y_pre may be None), int32 offsets on q's device."""
    q = _kernel_rows(q)
    k, v = _kernel_rows(k.to(q.dtype)), _kernel_rows(v.to(q.dtype))
    tables = [t.float().contiguous() for t in (pos_bias, scale_embed, phase_base, phase_gain)]
    y_pre = None if y_pre is None else _planes(y_pre.float())
    z_pre = _planes(z_pre.float())
    offsets = _device_offsets(offsets_dev, q.device, int(j_val))
    return (q, k, v, *tables, y_pre, z_pre, offsets)


def dsqg_forward(q, k, v, pos_bias, scale_embed, phase_base, phase_gain, y_pre, z_pre, offsets_dev,
                 j_small, j_large, plane_shift=0, query_start=0, *, events=None, schedule=None,
                 query_probes=None):
    """Raw forward launch: returns (out, lse).  q/k/v share one dtype (bf16 or fp32).

    ``events``: optional (start, end) torch.cuda.Event pair recorded around the
    launch on the current stream.  ``schedule``: DWARF_SCHED_* flags (None: the
    default schedule, ``DEFAULT_SCHEDULE``).  ``query_probes`` (bf16 only):
    normalised [4,64] fp32 probes; the kernel forms y from q itself (y_pre is
    not read and may be None) and the call returns (out, lse, y) with y
    [B,H,N,4] fp32.
    """
    lib = _lib.load()
    B, H, N, _ = q.shape
    out = torch.empty((B, H, N, q.shape[3]), device=q.device, dtype=q.dtype)
    lse = torch.empty((B, H, N), device=q.device, dtype=torch.float32)
    args = _lib.DsqgFwdArgs()
    _fill_fwd(args, q, k, v, pos_bias, scale_embed, phase_base, phase_gain, y_pre, z_pre, offsets_dev,
              j_small, j_large, plane_shift, query_start, out, lse, se_round=q.dtype != torch.float32,
              schedule=DEFAULT_SCHEDULE if schedule is None else schedule)
    y = None
    if query_probes is not None:
        y = torch.empty((B, H, N, R_PLANES), device=q.device, dtype=torch.float32)
        args.query_probes, args.y_out = query_probes.data_ptr(), y.data_ptr()
    if events:
        events[0].record()
    _lib.check(lib.dwarf_dsqg_fwd(ctypes.byref(args), _stream(q.device)), "dwarf_dsqg_fwd")
    if events:
        events[1].record()
    return (out, lse) if y is None else (out, lse, y)


_SIDE_STREAMS: dict = {}


def _side_stream(device: torch.device) -> torch.cuda.Stream:
    """This device's second stream for the overlapped backward (default priority)."""
    key = torch.cuda._utils._get_device_index(device, optional=True)
    if key not in _SIDE_STREAMS:
        _SIDE_STREAMS[key] = torch.cuda.Stream(device=device)
    return _SIDE_STREAMS[key]


def dsqg_backward(dout, q, k, v, pos_bias, scale_embed, phase_base, phase_gain, y_pre, z_pre, offsets_dev,
                  out, lse, j_small, j_large, plane_shift=0, query_start=0, *, events=None, schedule=None,
                  overlap=None, one_call=False, overlap_events=None, query_probes=None, key_probes=None):
    """Raw backward.  Returns (dq, dk, dv, dpb, dse, dpbase, dpgain, dy, dz).

    bf16 (``overlap`` None or True, no ``events``): the delta stage and dK/dV
    run on a second stream beside dQ and the parameter gradients on the
    current stream, which waits for both (DWARF_SCHED_DELTA_STAGE); the two
    gather launches then share the CUs.  Otherwise, and for fp32, the dq,
    params and dkdv stages run in turn on the current stream.  ``events``:
    optional four torch.cuda.Events recorded before dq, after dq, after params
    and after dkdv (serial stages, so each interval is one stage).  Either way
    the results are the same bits.  ``one_call``: every stage through the
    single entry point ``dwarf_dsqg_bwd`` on the current stream (with the
    delta-stage flag when ``overlap`` is True; the library then launches the
    delta stage first), the same bits again.  ``overlap_events``: optional six
    torch.cuda.Events for the overlapped schedule, recorded on the stream each
    stage runs on: before dq, after dq, after params (current stream), before
    delta, after delta, after dkdv (second stream).  ``query_probes`` /
    ``key_probes`` (bf16, normalised [4,64] fp32): y_pre / z_pre came from
    these probes, and dy / dz are folded into dq / dk inside the kernels; the
    dy / dz slots of the result are then None.
    """
    lib = _lib.load()
    dev = q.device
    dout = _kernel_rows(dout.to(q.dtype))
    dq = torch.empty(q.shape, device=dev, dtype=q.dtype)
    dk = torch.empty(k.shape, device=dev, dtype=k.dtype)
    dv = torch.empty(v.shape, device=dev, dtype=v.dtype)
    dpb = torch.empty(pos_bias.shape, device=dev, dtype=torch.float32)
    dse = torch.empty(scale_embed.shape, device=dev, dtype=torch.float32)
    # the reduction writes every [J_large, H, 4] entry; the [1, H, 4] tables of a
    # lattice without far offsets stay zero
    alloc = torch.empty if j_large > 0 else torch.zeros
    dpbase = alloc(phase_base.shape, device=dev, dtype=torch.float32)
    dpgain = alloc(phase_gain.shape, device=dev, dtype=torch.float32)
    dy = torch.empty(y_pre.shape, device=dev, dtype=torch.float32) if query_probes is None else None
    dz = torch.empty(z_pre.shape, device=dev, dtype=torch.float32) if key_probes is None else None
    # the delta-stage flag is this function's to set: it only holds when the delta launch runs
    # below, and on its own it would leave dK/dV reading (delta, lse) pairs no stage wrote
    schedule = (DEFAULT_SCHEDULE if schedule is None else int(schedule)) & ~_lib.DWARF_SCHED_DELTA_STAGE
    args = _lib.DsqgBwdArgs()
    _fill_fwd(args.fwd, q, k, v, pos_bias, scale_embed, phase_base, phase_gain, y_pre, z_pre, offsets_dev,
              j_small, j_large, plane_shift, query_start, out, lse, se_round=q.dtype != torch.float32,
              schedule=schedule)
    args.dout, args.dout_stride = dout.data_ptr(), _lib.i64_array(dout.stride())
    args.dq, args.dq_stride = dq.data_ptr(), _lib.i64_array(dq.stride())
    args.dk, args.dk_stride = dk.data_ptr(), _lib.i64_array(dk.stride())
    args.dv, args.dv_stride = dv.data_ptr(), _lib.i64_array(dv.stride())
    args.dpos_bias, args.dscale_embed = dpb.data_ptr(), dse.data_ptr()
    args.dphase_base, args.dphase_gain = dpbase.data_ptr(), dpgain.data_ptr()
    args.dy_pre, args.dz_pre = _ptr(dy), _ptr(dz)
    args.fwd.query_probes, args.fwd.key_probes = _ptr(query_probes), _ptr(key_probes)
    if one_call:
        if events:
            raise ValueError("events time the stages of separate calls; one_call runs them in one")
        overlap = bool(overlap) and q.dtype == torch.bfloat16
    else:
        overlap = q.dtype == torch.bfloat16 and not events and (overlap is None or overlap)
    if overlap_events and (one_call or not overlap):
        raise ValueError("overlap_events time the stages of the overlapped two-stream schedule")
    if overlap:
        args.fwd.schedule |= _lib.DWARF_SCHED_DELTA_STAGE
    nbytes = lib.dwarf_dsqg_bwd_workspace_bytes(ctypes.byref(args))
    workspace = torch.empty(max(int(nbytes), 256), device=dev, dtype=torch.uint8)
    args.workspace, args.workspace_bytes = workspace.data_ptr(), workspace.numel()
    stream = _stream(dev)
    if one_call:
        _lib.check(lib.dwarf_dsqg_bwd(ctypes.byref(args), stream), "dwarf_dsqg_bwd")
        return dq, dk, dv, dpb, dse, dpbase, dpgain, dy, dz
    if overlap:
        main = torch.cuda.current_stream(dev)
        side = _side_stream(dev)
        fork = torch.cuda.Event()
        fork.record(main)
        # dQ goes first: its persistent workgroups take their two slots per CU before
        # dK/dV's thousands of workgroups fill the rest (the other way round dQ waits
        # for dK/dV to drain and the two barely overlap)
        ev = overlap_events
        if ev:
            ev[0].record(main)
        _lib.check(lib.dwarf_dsqg_bwd_dq(ctypes.byref(args), stream), "dwarf_dsqg_bwd_dq")
        if ev:
            ev[1].record(main)
        side.wait_event(fork)
        if ev:
            ev[3].record(side)
        _lib.check(lib.dwarf_dsqg_bwd_delta(ctypes.byref(args), side.cuda_stream), "dwarf_dsqg_bwd_delta")
        if ev:
            ev[4].record(side)
        _lib.check(lib.dwarf_dsqg_bwd_dkdv(ctypes.byref(args), side.cuda_stream), "dwarf_dsqg_bwd_dkdv")
        if ev:
            ev[5].record(side)
        _lib.check(lib.dwarf_dsqg_bwd_params(ctypes.byref(args), stream), "dwarf_dsqg_bwd_params")
        if ev:
            ev[2].record(main)
        main.wait_stream(side)
        # memory the second stream used must not be handed out again before it is done
        for t in (workspace, dk, dv, dz, dout, q, k, v, out, lse, y_pre, z_pre, pos_bias, scale_embed, phase_base,
                  phase_gain, offsets_dev, key_probes):
            if t is not None and t.is_cuda:
                t.record_stream(side)
        return dq, dk, dv, dpb, dse, dpbase, dpgain, dy, dz
    if events:
        events[0].record()
    _lib.check(lib.dwarf_dsqg_bwd_dq(ctypes.byref(args), stream), "dwarf_dsqg_bwd_dq")
    if events:
        events[1].record()
    _lib.check(lib.dwarf_dsqg_bwd_params(ctypes.byref(args), stream), "dwarf_dsqg_bwd_params")
    if events:
        events[2].record()
    _lib.check(lib.dwarf_dsqg_bwd_dkdv(ctypes.byref(args), stream), "dwarf_dsqg_bwd_dkdv")
    if events:
        events[3].record()
    return dq, dk, dv, dpb, dse, dpbase, dpgain, dy, dz


def _check_call(q, k, v, y_shape, z_shape, j_val, j_small, j_large, offsets_dev, grouped_mode_id) -> None:
    """The reference Function's checks (dsqg:2204-2228), in its order and with its exception types;
    y_shape / z_shape None for the probe-feature form (y and z formed here)."""
    B, H, N, HD = q.shape
    Bk, H_KV, Nk, HDk = k.shape
    if v.shape != k.shape:
        raise ValueError(f"k/v shape mismatch: k={tuple(k.shape)} v={tuple(v.shape)}")
    if Bk != B or Nk != N or HDk != HD:
        raise ValueError(f"native GQA requires q/k/v to share B,N,HD: q={tuple(q.shape)} k={tuple(k.shape)}")
    if H % H_KV != 0:
        raise ValueError(f"num query heads H={H} must be divisible by KV heads H_KV={H_KV}")
    if H != H_KV and int(grouped_mode_id) in _SLAB_MODES:
        raise NotImplementedError("native GQA is currently implemented for grouped_mode='baseline' only")
    if y_shape is not None and tuple(y_shape[:3]) != (B, H, N):
        raise ValueError(f"y_pre must have shape [B,Hq,N,R]; got {tuple(y_shape)} for q={tuple(q.shape)}")
    if z_shape is not None and tuple(z_shape[:3]) != (B, H_KV, N):
        raise ValueError(f"z_pre must have shape [B,Hkv,N,R]; got {tuple(z_shape)} for k={tuple(k.shape)}")
    assert q.dtype in (torch.bfloat16, torch.float32)
    if not q.is_cuda:
        raise RuntimeError("DSQG HIP kernels require device tensors")
    planes = R_PLANES if y_shape is None else y_shape[3]
    if HD != HEAD_DIM or planes != R_PLANES:
        raise RuntimeError(f"Unsupported DSQG launch shape: head_dim={HD}, planes={planes} "
                           f"(built for head_dim={HEAD_DIM}, {R_PLANES} planes)")
    if int(j_small) + int(j_large) != int(j_val):
        raise ValueError(f"j_val={j_val} != j_small={j_small} + j_large={j_large}")
    if offsets_dev.numel() != int(j_val):
        raise ValueError(f"offsets_dev has {offsets_dev.numel()} entries, expected j_val={j_val}")


class _DSQGV18GroupedFn(torch.autograd.Function):
    """Autograd wrapper with the reference's 25 positional arguments (dsqg:2197-2203).

    The launches are the custom ops ``torch.ops.dwarf.dsqg_fwd`` / ``dsqg_bwd``
    (registered in ``ops.py`` with fake implementations), so the Function traces
    under ``torch.compile``; validation here uses shapes only.
    """

    @staticmethod
    def forward(ctx, q, k, v, pos_bias, scale_embed, phase_base, phase_gain, y_pre, z_pre,
                j_val, j_small, j_large, offsets_dev, sparse_order_dev,
                group_start_dev, group_len_dev, group_dmin_dev, group_dmax_dev,
                k_group_size, grouped_mode_id, verify_mode, max_group_spread_observed,
                plane_shift, query_start, online_softmax):
        N = q.shape[2]
        query_start = max(0, min(int(query_start), N))
        _check_call(q, k, v, y_pre.shape, z_pre.shape, j_val, j_small, j_large, offsets_dev, grouped_mode_id)
        schedule = schedule_for(grouped_mode_id, bool(online_softmax))
        out, lse = torch.ops.dwarf.dsqg_fwd(q, k, v, pos_bias, scale_embed, phase_base, phase_gain, y_pre, z_pre,
                                            offsets_dev, int(j_small), int(j_large), int(plane_shift), query_start,
                                            schedule)
        ctx.save_for_backward(q, k, v, pos_bias, scale_embed, phase_base, phase_gain, y_pre, z_pre,
                              out, lse, offsets_dev)
        ctx.j_small, ctx.j_large = int(j_small), int(j_large)
        ctx.plane_shift, ctx.query_start = int(plane_shift), query_start
        ctx.schedule = schedule
        return out

    @staticmethod
    def backward(ctx, dout):
        (q, k, v, pos_bias, scale_embed, phase_base, phase_gain, y_pre, z_pre,
         out, lse, offsets) = ctx.saved_tensors
        grads = torch.ops.dwarf.dsqg_bwd(dout, q, k, v, pos_bias, scale_embed, phase_base, phase_gain, y_pre,
                                         z_pre, offsets, out, lse, ctx.j_small, ctx.j_large, ctx.plane_shift,
                                         ctx.query_start, ctx.schedule)
        dq, dk, dv, dpb, dse, dpbase, dpgain, dy, dz = grads
        return (dq, dk.to(k.dtype), dv.to(v.dtype), dpb.to(pos_bias.dtype), dse.to(scale_embed.dtype),
                dpbase.to(phase_base.dtype), dpgain.to(phase_gain.dtype), dy.to(y_pre.dtype),
                dz.to(z_pre.dtype)) + (None,) * 16


def dsqg_attention_v18_grouped(
    q, k, v, pos_bias, scale_embed, phase_base, phase_gain, y_pre, z_pre,
    j_val, j_small, j_large, offsets_dev, sparse_order_dev, group_start_dev, group_len_dev,
    group_dmin_dev, group_dmax_dev, k_group_size, grouped_mode_id, verify_mode,
    max_group_spread_observed, plane_shift=0, query_start=0, *, backend: str = "auto",
    online_softmax: bool = True,
):
    """DSQG attention on the HIP kernels (reference signature: dsqg:2691-2719).

    ``backend`` accepts the reference's values: "auto" and "triton" (both run
    the HIP kernels here; "hip" is an alias) and "eager", which the reference
    maps to its CPU oracle.  This library ships no CPU path, so "eager" and
    non-device tensors raise instead of falling back.  ``online_softmax`` and
    ``grouped_mode_id`` select schedules of the same mathematics, as in the
    reference (``schedule_for``): the overlap-slab modes (1, 3) serve the near
    offsets of the dQ launch as a dense band on the matrix cores, and
    online_softmax=False runs the two-pass (offline) softmax forward.  The
    slab plan buffers (sparse order, groups; built by ``planner.plan_sparse_groups``
    as the reference's module builds them, dsqg:2888-2923) describe a slab
    tiling of the far offsets, which these kernels gather per offset instead:
    they are accepted and not read.
    """
    del verify_mode, sparse_order_dev, group_start_dev, group_len_dev, group_dmin_dev, group_dmax_dev
    del k_group_size, max_group_spread_observed
    backend = str(backend).lower()
    if backend not in {"auto", "triton", "hip", "eager"}:
        raise ValueError("backend must be auto, triton, hip, or eager")
    if backend == "eager":
        raise NotImplementedError(
            "backend='eager' selects the reference's CPU oracle, which is not part of this library"
        )
    if not q.is_cuda:
        raise RuntimeError("DSQG HIP kernels were requested but the tensors are not on a GPU device")
    original_dtype = q.dtype
    compute = torch.float32 if q.dtype == torch.float32 else torch.bfloat16
    output = _DSQGV18GroupedFn.apply(
        q.to(compute), k.to(compute), v.to(compute),
        pos_bias.float(), scale_embed.float(), phase_base.float(), phase_gain.float(),
        y_pre.float(), z_pre.float(),
        int(j_val), int(j_small), int(j_large), offsets_dev, None, None, None, None, None,
        0, int(grouped_mode_id), False, 0, int(plane_shift), int(query_start), bool(online_softmax),
    )
    return output if output.dtype == original_dtype else output.to(original_dtype)


# ---- the op with the block's phase-probe features inside the kernels -------------------------------------------
class _DSQGProbedFn(torch.autograd.Function):
    """DSQG attention whose y and z come from probes inside the kernels (bf16).

    The DSQG block forms y = <q, p_r> / sqrt(|q|^2 + 1e-6 hd) and z likewise
    from k with an einsum over fp32 copies of q and k (dsqg:3231-3254) and
    passes them to the op.  Here the forward kernel forms y from each q row it
    loads anyway (and keeps it for the backward), z comes from the
    phase-probe kernel over k, and the backward kernels add dy's and dz's
    contributions to dq and dk in their epilogues, so neither y, dy nor dz
    round-trips through HBM outside the op.  Arguments: the probes already
    normalised, fp32 [4, 64], without gradient.
    """

    @staticmethod
    def forward(ctx, q, k, v, pos_bias, scale_embed, phase_base, phase_gain, query_probes, key_probes, offsets_dev,
                j_small, j_large, plane_shift, query_start, schedule):
        N = q.shape[2]
        z_pre = torch.ops.dwarf.phase_probe_fwd(k, key_probes, 0, N)
        out, lse, y_pre = torch.ops.dwarf.dsqg_fwd_probed(q, k, v, pos_bias, scale_embed, phase_base, phase_gain,
                                                          query_probes, z_pre, offsets_dev, int(j_small),
                                                          int(j_large), int(plane_shift), int(query_start),
                                                          int(schedule))
        ctx.save_for_backward(q, k, v, pos_bias, scale_embed, phase_base, phase_gain, query_probes, key_probes,
                              y_pre, z_pre, out, lse, offsets_dev)
        ctx.args = (int(j_small), int(j_large), int(plane_shift), int(query_start), int(schedule))
        return out

    @staticmethod
    def backward(ctx, dout):
        (q, k, v, pos_bias, scale_embed, phase_base, phase_gain, qp, kp, y_pre, z_pre, out, lse,
         offsets) = ctx.saved_tensors
        dq, dk, dv, dpb, dse, dpbase, dpgain = torch.ops.dwarf.dsqg_bwd_probed(
            dout, q, k, v, pos_bias, scale_embed, phase_base, phase_gain, qp, kp, y_pre, z_pre, offsets, out, lse,
            *ctx.args)
        return (dq, dk.to(k.dtype), dv.to(v.dtype), dpb.to(pos_bias.dtype), dse.to(scale_embed.dtype),
                dpbase.to(phase_base.dtype), dpgain.to(phase_gain.dtype)) + (None,) * 8


def dsqg_attention_with_probes(
    q, k, v, pos_bias, scale_embed, phase_base, phase_gain, query_probes, key_probes,
    j_val, j_small, j_large, offsets_dev, sparse_order_dev, group_start_dev, group_len_dev,
    group_dmin_dev, group_dmax_dev, k_group_size, grouped_mode_id, verify_mode,
    max_group_spread_observed, plane_shift=0, query_start=0, *, backend: str = "auto",
    online_softmax: bool = True,
):
    """``dsqg_attention_v18_grouped`` (dsqg:2691-2719) with the block's probes in place of y_pre / z_pre.

    query_probes / key_probes are the block's raw [4, 64] probe parameters;
    they are normalised here as the block does (F.normalize, dsqg:3231-3232)
    and y / z are the block's features of q and k (dsqg:3234-3254).  bf16
    (and fp16, cast as the reference casts) runs ``_DSQGProbedFn``: y, z and
    their gradients inside the kernels.  Probes that require a gradient
    (train_phase_probes=True) and fp32 inputs run the phase-probe kernels and
    ``dsqg_attention_v18_grouped`` one after the other (the probe gradients
    come from the phase-probe backward).  Everything else, errors included,
    is ``dsqg_attention_v18_grouped``'s.
    """
    backend = str(backend).lower()
    if backend not in {"auto", "triton", "hip", "eager"}:
        raise ValueError("backend must be auto, triton, hip, or eager")
    if backend == "eager":
        raise NotImplementedError(
            "backend='eager' selects the reference's CPU oracle, which is not part of this library"
        )
    if not q.is_cuda:
        raise RuntimeError("DSQG HIP kernels were requested but the tensors are not on a GPU device")
    qp = torch.nn.functional.normalize(query_probes.float(), dim=-1)
    kp = torch.nn.functional.normalize(key_probes.float(), dim=-1)
    probe_grad = torch.is_grad_enabled() and (qp.requires_grad or kp.requires_grad)
    if q.dtype == torch.float32 or probe_grad:
        from .probe import phase_probe_features

        y_pre = phase_probe_features(q, qp)
        z_pre = phase_probe_features(k, kp)
        return dsqg_attention_v18_grouped(
            q, k, v, pos_bias, scale_embed, phase_base, phase_gain, y_pre, z_pre, j_val, j_small, j_large,
            offsets_dev, sparse_order_dev, group_start_dev, group_len_dev, group_dmin_dev, group_dmax_dev,
            k_group_size, grouped_mode_id, verify_mode, max_group_spread_observed, plane_shift, query_start,
            backend=backend, online_softmax=online_softmax)
    original_dtype = q.dtype
    qb, kb, vb = q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)
    N = q.shape[2]
    _check_call(qb, kb, vb, None, None, j_val, j_small, j_large, offsets_dev, grouped_mode_id)
    output = _DSQGProbedFn.apply(
        qb, kb, vb, pos_bias.float(), scale_embed.float(), phase_base.float(), phase_gain.float(),
        qp.detach().to(q.device), kp.detach().to(q.device), offsets_dev, int(j_small), int(j_large), int(plane_shift),
        max(0, min(int(query_start), N)), schedule_for(grouped_mode_id, bool(online_softmax)))
    return output if output.dtype == original_dtype else output.to(original_dtype)
