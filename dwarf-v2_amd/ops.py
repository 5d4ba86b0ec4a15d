"""torch.library registration of the HIP launches.

``dwarf::dsqg_fwd``, ``dwarf::dsqg_bwd``, ``dwarf::dsqg_fwd_probed``,
``dwarf::dsqg_bwd_probed``, ``dwarf::ema_fwd``,
``dwarf::ema_bwd``, ``dwarf::phase_probe_fwd``, ``dwarf::phase_probe_bwd``,
``dwarf::npci_fwd``, ``dwarf::npci_bwd``, ``dwarf::packet_pool_fwd``,
``dwarf::packet_pool_bwd``, ``dwarf::packet_fwd`` and ``dwarf::packet_bwd`` are
custom ops with fake (shape-only) implementations, so ``torch.compile`` traces
the DSQG, EMA, phase-probe, NPCI and InterferencePacket autograd Functions
without graph breaks (the trainer
compiles the model, train:1083).  The real
implementations normalise layouts (unit head-dim stride, 16-byte rows,
contiguous fp32 tables and plane features, int32 offsets on the device) and
call the C ABI on the current stream.  The op names follow the drop-in
boundary of the reference ops (kernels/dsqg_attention_v22.py:2691-2777,
371-451 and 221-254, kernels/causal_ema_scan.py:263-509,
train/train_dwarf.py:260-267).
"""

from __future__ import annotations

from typing import Optional

import torch

from . import dsqg as _dsqg
from . import ema as _ema
from . import npci as _npci
from . import packet as _packet
from . import probe as _probe

Tensor = torch.Tensor


# ---- DSQG ------------------------------------------------------------------------------------
@torch.library.custom_op("dwarf::dsqg_fwd", mutates_args=())
def dsqg_fwd(q: Tensor, k: Tensor, v: Tensor, pos_bias: Tensor, scale_embed: Tensor, phase_base: Tensor,
             phase_gain: Tensor, y_pre: Tensor, z_pre: Tensor, offsets: Tensor, j_small: int, j_large: int,
             plane_shift: int, query_start: int,
             schedule: int = _dsqg.DEFAULT_SCHEDULE) -> tuple[Tensor, Tensor]:
    """Forward launch; returns (out like q, lse [B,H,N] fp32).  schedule: DWARF_SCHED_* flags."""
    t = _dsqg.normalize_inputs(q, k, v, pos_bias, scale_embed, phase_base, phase_gain, y_pre, z_pre, offsets,
                               j_small + j_large)
    return _dsqg.dsqg_forward(*t, j_small, j_large, plane_shift, query_start, schedule=schedule)


@dsqg_fwd.register_fake
def _dsqg_fwd_fake(q, k, v, pos_bias, scale_embed, phase_base, phase_gain, y_pre, z_pre, offsets, j_small, j_large,
                   plane_shift, query_start, schedule=_dsqg.DEFAULT_SCHEDULE):
    B, H, N, HD = q.shape
    return q.new_empty((B, H, N, HD)), q.new_empty((B, H, N), dtype=torch.float32)


@torch.library.custom_op("dwarf::dsqg_bwd", mutates_args=())
def dsqg_bwd(dout: Tensor, q: Tensor, k: Tensor, v: Tensor, pos_bias: Tensor, scale_embed: Tensor,
             phase_base: Tensor, phase_gain: Tensor, y_pre: Tensor, z_pre: Tensor, offsets: Tensor, out: Tensor,
             lse: Tensor, j_small: int, j_large: int, plane_shift: int, query_start: int,
             schedule: int = _dsqg.DEFAULT_SCHEDULE
             ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Backward launches; returns (dq, dk, dv, dpos_bias, dscale_embed, dphase_base, dphase_gain, dy, dz)."""
    t = _dsqg.normalize_inputs(q, k, v, pos_bias, scale_embed, phase_base, phase_gain, y_pre, z_pre, offsets,
                               j_small + j_large)
    return _dsqg.dsqg_backward(dout, *t, out, lse.contiguous(), j_small, j_large, plane_shift, query_start,
                               schedule=schedule)


@dsqg_bwd.register_fake
def _dsqg_bwd_fake(dout, q, k, v, pos_bias, scale_embed, phase_base, phase_gain, y_pre, z_pre, offsets, out, lse,
                   j_small, j_large, plane_shift, query_start, schedule=_dsqg.DEFAULT_SCHEDULE):
    f32 = torch.float32
    return (q.new_empty(q.shape), q.new_empty(k.shape), q.new_empty(v.shape),
            q.new_empty(pos_bias.shape, dtype=f32), q.new_empty(scale_embed.shape, dtype=f32),
            q.new_empty(phase_base.shape, dtype=f32), q.new_empty(phase_gain.shape, dtype=f32),
            q.new_empty(y_pre.shape, dtype=f32), q.new_empty(z_pre.shape, dtype=f32))


@torch.library.custom_op("dwarf::dsqg_fwd_probed", mutates_args=())
def dsqg_fwd_probed(q: Tensor, k: Tensor, v: Tensor, pos_bias: Tensor, scale_embed: Tensor, phase_base: Tensor,
                    phase_gain: Tensor, query_probes: Tensor, z_pre: Tensor, offsets: Tensor, j_small: int,
                    j_large: int, plane_shift: int, query_start: int,
                    schedule: int = _dsqg.DEFAULT_SCHEDULE) -> tuple[Tensor, Tensor, Tensor]:
    """Forward launch forming y from q and normalised query probes; returns (out, lse, y [B,H,N,4] fp32)."""
    t = _dsqg.normalize_inputs(q, k, v, pos_bias, scale_embed, phase_base, phase_gain, None, z_pre, offsets,
                               j_small + j_large)
    return _dsqg.dsqg_forward(*t, j_small, j_large, plane_shift, query_start, schedule=schedule,
                              query_probes=_dsqg._planes(query_probes.float()))


@dsqg_fwd_probed.register_fake
def _dsqg_fwd_probed_fake(q, k, v, pos_bias, scale_embed, phase_base, phase_gain, query_probes, z_pre, offsets,
                          j_small, j_large, plane_shift, query_start, schedule=_dsqg.DEFAULT_SCHEDULE):
    B, H, N, HD = q.shape
    f32 = torch.float32
    return q.new_empty((B, H, N, HD)), q.new_empty((B, H, N), dtype=f32), q.new_empty((B, H, N, 4), dtype=f32)


@torch.library.custom_op("dwarf::dsqg_bwd_probed", mutates_args=())
def dsqg_bwd_probed(dout: Tensor, q: Tensor, k: Tensor, v: Tensor, pos_bias: Tensor, scale_embed: Tensor,
                    phase_base: Tensor, phase_gain: Tensor, query_probes: Tensor, key_probes: Tensor, y_pre: Tensor,
                    z_pre: Tensor, offsets: Tensor, out: Tensor, lse: Tensor, j_small: int, j_large: int,
                    plane_shift: int, query_start: int, schedule: int = _dsqg.DEFAULT_SCHEDULE
                    ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Backward launches with dy and dz folded into dq and dk; returns (dq, dk, dv, dpos_bias, dscale_embed,
    dphase_base, dphase_gain)."""
    t = _dsqg.normalize_inputs(q, k, v, pos_bias, scale_embed, phase_base, phase_gain, y_pre, z_pre, offsets,
                               j_small + j_large)
    g = _dsqg.dsqg_backward(dout, *t, out, lse.contiguous(), j_small, j_large, plane_shift, query_start,
                            schedule=schedule, query_probes=_dsqg._planes(query_probes.float()),
                            key_probes=_dsqg._planes(key_probes.float()))
    return g[:7]


@dsqg_bwd_probed.register_fake
def _dsqg_bwd_probed_fake(dout, q, k, v, pos_bias, scale_embed, phase_base, phase_gain, query_probes, key_probes,
                          y_pre, z_pre, offsets, out, lse, j_small, j_large, plane_shift, query_start,
                          schedule=_dsqg.DEFAULT_SCHEDULE):
    f32 = torch.float32
    return (q.new_empty(q.shape), q.new_empty(k.shape), q.new_empty(v.shape),
            q.new_empty(pos_bias.shape, dtype=f32), q.new_empty(scale_embed.shape, dtype=f32),
            q.new_empty(phase_base.shape, dtype=f32), q.new_empty(phase_gain.shape, dtype=f32))


# ---- EMA -------------------------------------------------------------------------------------
@torch.library.custom_op("dwarf::ema_fwd", mutates_args=())
def ema_fwd(x: Tensor, alpha: Tensor, floor: float, ceiling: float, reset: Optional[Tensor] = None) -> Tensor:
    """y = causal EMA of x [B,N,D] (x's dtype); alpha fp32 with 1 or D values; reset [B,N] bool or None."""
    return _ema.ema_forward(_ema.normalize_x(x), _ema.normalize_alpha(alpha, x.device), floor, ceiling,
                            _ema.normalize_reset(reset, x))


@ema_fwd.register_fake
def _ema_fwd_fake(x, alpha, floor, ceiling, reset=None):
    return x.new_empty(x.shape)


@torch.library.custom_op("dwarf::ema_bwd", mutates_args=())
def ema_bwd(x: Tensor, y: Tensor, dy: Tensor, alpha: Tensor, floor: float, ceiling: float,
            reset: Optional[Tensor] = None) -> tuple[Tensor, Tensor]:
    """(dx like x, dalpha fp32 [alpha.numel()], clamp-projected)."""
    dx, dalpha = _ema.ema_backward(_ema.normalize_x(x), _ema.normalize_x(y), dy,
                                   _ema.normalize_alpha(alpha, x.device), floor, ceiling, True,
                                   _ema.normalize_reset(reset, x))
    return dx, dalpha


@ema_bwd.register_fake
def _ema_bwd_fake(x, y, dy, alpha, floor, ceiling, reset=None):
    return x.new_empty(x.shape), x.new_empty((alpha.numel(),), dtype=torch.float32)


# ---- phase-probe features ------------------------------------------------------------------
@torch.library.custom_op("dwarf::phase_probe_fwd", mutates_args=())
def phase_probe_fwd(values: Tensor, probes: Tensor, start: int, end: int) -> Tensor:
    """y [B,H,N,R] fp32; rows outside [start, end) are 0."""
    return _probe.probe_forward(values, probes, start, end)


@phase_probe_fwd.register_fake
def _phase_probe_fwd_fake(values, probes, start, end):
    return values.new_empty((*values.shape[:3], probes.shape[0]), dtype=torch.float32)


@torch.library.custom_op("dwarf::phase_probe_bwd", mutates_args=())
def phase_probe_bwd(values: Tensor, probes: Tensor, dout: Tensor, start: int, end: int,
                    need_dprobes: bool) -> tuple[Tensor, Tensor]:
    """(dx in the kernel dtype, dprobes fp32 [R,hd]; empty [0] when not needed)."""
    dx, dprobes = _probe.probe_backward(values, probes, dout, start, end, need_dprobes)
    return dx, dprobes if dprobes is not None else values.new_empty((0,), dtype=torch.float32)


@phase_probe_bwd.register_fake
def _phase_probe_bwd_fake(values, probes, dout, start, end, need_dprobes):
    dt = values.dtype if values.dtype in (torch.bfloat16, torch.float32) else torch.float32
    dp = probes.shape if need_dprobes else (0,)
    return values.new_empty(values.shape, dtype=dt), values.new_empty(dp, dtype=torch.float32)


# ---- NPCI rotation ---------------------------------------------------------------------------
@torch.library.custom_op("dwarf::npci_fwd", mutates_args=())
def npci_fwd(x: Tensor, x_delta: Tensor, theta_h: Tensor, tau: float) -> Tensor:
    """Rotated rows [B,H,T,hd] (kernel dtype of x)."""
    return _npci.npci_forward(x, x_delta, theta_h, tau)


def _npci_dtype(t):
    return t.dtype if t.dtype in (torch.bfloat16, torch.float32) else torch.float32


@npci_fwd.register_fake
def _npci_fwd_fake(x, x_delta, theta_h, tau):
    return x.new_empty(x.shape, dtype=_npci_dtype(x))


@torch.library.custom_op("dwarf::npci_bwd", mutates_args=())
def npci_bwd(x: Tensor, x_delta: Tensor, theta_h: Tensor, grad: Tensor, tau: float) -> tuple[Tensor, Tensor, Tensor]:
    """(dx, dx_delta, dtheta [H] fp32)."""
    return _npci.npci_backward(x, x_delta, theta_h, grad, tau)


@npci_bwd.register_fake
def _npci_bwd_fake(x, x_delta, theta_h, grad, tau):
    return (x.new_empty(x.shape, dtype=_npci_dtype(x)), x.new_empty(x.shape, dtype=_npci_dtype(x_delta)),
            x.new_empty((theta_h.numel(),), dtype=torch.float32))


# ---- InterferencePacket pool -----------------------------------------------------------------
@torch.library.custom_op("dwarf::packet_pool_fwd", mutates_args=())
def packet_pool_fwd(x: Tensor, alpha: Tensor, weight: Tensor, floor: float, ceiling: float) -> tuple[Tensor, Tensor]:
    """(pooled with x's dtype, per-chunk scan states fp32 [B, ceil(N/16), K*D])."""
    return _packet.pool_forward(x, alpha, weight, floor, ceiling)


@packet_pool_fwd.register_fake
def _packet_pool_fwd_fake(x, alpha, weight, floor, ceiling):
    return x.new_empty(x.shape), x.new_empty(_packet.state_shape(x, alpha.numel()), dtype=torch.float32)


@torch.library.custom_op("dwarf::packet_pool_bwd", mutates_args=())
def packet_pool_bwd(x: Tensor, alpha: Tensor, weight: Tensor, state: Tensor, dpooled: Tensor, floor: float,
                    ceiling: float) -> tuple[Tensor, Tensor, Tensor]:
    """(dx with x's dtype, dalpha [K] fp32 clamp-projected, dweight [K] fp32)."""
    return _packet.pool_backward(x, alpha, weight, state, dpooled, floor, ceiling)


@packet_pool_bwd.register_fake
def _packet_pool_bwd_fake(x, alpha, weight, state, dpooled, floor, ceiling):
    return (x.new_empty(x.shape), x.new_empty((alpha.numel(),), dtype=torch.float32),
            x.new_empty((alpha.numel(),), dtype=torch.float32))


# ---- InterferencePacket packet ---------------------------------------------------------------
@torch.library.custom_op("dwarf::packet_fwd", mutates_args=())
def packet_fwd(x: Tensor, alpha: Tensor, weight: Tensor, gate: Tensor, floor: float,
               ceiling: float) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """(packet with gate's dtype, pooled with x's dtype, per-chunk scan states fp32, ms [B,N] fp32)."""
    return _packet.packet_forward(x, alpha, weight, gate, floor, ceiling)


@packet_fwd.register_fake
def _packet_fwd_fake(x, alpha, weight, gate, floor, ceiling):
    return (x.new_empty(x.shape, dtype=gate.dtype), x.new_empty(x.shape),
            x.new_empty(_packet.state_shape(x, alpha.numel()), dtype=torch.float32),
            x.new_empty(x.shape[:2], dtype=torch.float32))


@torch.library.custom_op("dwarf::packet_bwd", mutates_args=())
def packet_bwd(x: Tensor, alpha: Tensor, weight: Tensor, gate: Tensor, pooled: Tensor, state: Tensor, ms: Tensor,
               dpacket: Tensor, floor: float, ceiling: float) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """(dx with x's dtype, dalpha [K] fp32 clamp-projected, dweight [K] fp32, dgate with gate's dtype)."""
    return _packet.packet_backward(x, alpha, weight, gate, pooled, state, ms, dpacket, floor, ceiling)


@packet_bwd.register_fake
def _packet_bwd_fake(x, alpha, weight, gate, pooled, state, ms, dpacket, floor, ceiling):
    return (x.new_empty(x.shape), x.new_empty((alpha.numel(),), dtype=torch.float32),
            x.new_empty((alpha.numel(),), dtype=torch.float32), x.new_empty(x.shape, dtype=gate.dtype))
