"""torch.library registration of the HIP launches.

``dwarf::dsqg_fwd``, ``dwarf::dsqg_bwd``, ``dwarf::ema_fwd`` and
``dwarf::ema_bwd`` are custom ops with fake (shape-only) implementations, so
``torch.compile`` traces the DSQG and EMA autograd Functions without graph
breaks (the trainer compiles the model, train:1083).  The real
implementations normalise layouts (unit head-dim stride, 16-byte rows,
contiguous fp32 tables and plane features, int32 offsets on the device) and
call the C ABI on the current stream.  The op names follow the drop-in
boundary of the reference op (kernels/dsqg_attention_v22.py:2691-2777,
kernels/causal_ema_scan.py:263-364).
"""

from __future__ import annotations

import torch

from . import dsqg as _dsqg
from . import ema as _ema

Tensor = torch.Tensor


# ---- DSQG ------------------------------------------------------------------------------------
@torch.library.custom_op("dwarf::dsqg_fwd", mutates_args=())
def dsqg_fwd(q: Tensor, k: Tensor, v: Tensor, pos_bias: Tensor, scale_embed: Tensor, phase_base: Tensor,
             phase_gain: Tensor, y_pre: Tensor, z_pre: Tensor, offsets: Tensor, j_small: int, j_large: int,
             plane_shift: int, query_start: int) -> tuple[Tensor, Tensor]:
    """Forward launch; returns (out like q, lse [B,H,N] fp32)."""
    t = _dsqg.normalize_inputs(q, k, v, pos_bias, scale_embed, phase_base, phase_gain, y_pre, z_pre, offsets,
                               j_small + j_large)
    return _dsqg.dsqg_forward(*t, j_small, j_large, plane_shift, query_start)


@dsqg_fwd.register_fake
def _dsqg_fwd_fake(q, k, v, pos_bias, scale_embed, phase_base, phase_gain, y_pre, z_pre, offsets, j_small, j_large,
                   plane_shift, query_start):
    B, H, N, HD = q.shape
    return q.new_empty((B, H, N, HD)), q.new_empty((B, H, N), dtype=torch.float32)


@torch.library.custom_op("dwarf::dsqg_bwd", mutates_args=())
def dsqg_bwd(dout: Tensor, q: Tensor, k: Tensor, v: Tensor, pos_bias: Tensor, scale_embed: Tensor,
             phase_base: Tensor, phase_gain: Tensor, y_pre: Tensor, z_pre: Tensor, offsets: Tensor, out: Tensor,
             lse: Tensor, j_small: int, j_large: int, plane_shift: int,
             query_start: int) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Backward launches; returns (dq, dk, dv, dpos_bias, dscale_embed, dphase_base, dphase_gain, dy, dz)."""
    t = _dsqg.normalize_inputs(q, k, v, pos_bias, scale_embed, phase_base, phase_gain, y_pre, z_pre, offsets,
                               j_small + j_large)
    return _dsqg.dsqg_backward(dout, *t, out, lse.contiguous(), j_small, j_large, plane_shift, query_start)


@dsqg_bwd.register_fake
def _dsqg_bwd_fake(dout, q, k, v, pos_bias, scale_embed, phase_base, phase_gain, y_pre, z_pre, offsets, out, lse,
                   j_small, j_large, plane_shift, query_start):
    f32 = torch.float32
    return (q.new_empty(q.shape), q.new_empty(k.shape), q.new_empty(v.shape),
            q.new_empty(pos_bias.shape, dtype=f32), q.new_empty(scale_embed.shape, dtype=f32),
            q.new_empty(phase_base.shape, dtype=f32), q.new_empty(phase_gain.shape, dtype=f32),
            q.new_empty(y_pre.shape, dtype=f32), q.new_empty(z_pre.shape, dtype=f32))


# ---- EMA -------------------------------------------------------------------------------------
@torch.library.custom_op("dwarf::ema_fwd", mutates_args=())
def ema_fwd(x: Tensor, alpha: Tensor, floor: float, ceiling: float) -> Tensor:
    """y = causal EMA of x [B,N,D] (x's dtype); alpha fp32 with 1 or D values."""
    return _ema.ema_forward(_ema.normalize_x(x), _ema.normalize_alpha(alpha, x.device), floor, ceiling)


@ema_fwd.register_fake
def _ema_fwd_fake(x, alpha, floor, ceiling):
    return x.new_empty(x.shape)


@torch.library.custom_op("dwarf::ema_bwd", mutates_args=())
def ema_bwd(x: Tensor, y: Tensor, dy: Tensor, alpha: Tensor, floor: float, ceiling: float) -> tuple[Tensor, Tensor]:
    """(dx like x, dalpha fp32 [alpha.numel()], clamp-projected)."""
    dx, dalpha = _ema.ema_backward(_ema.normalize_x(x), _ema.normalize_x(y), dy,
                                   _ema.normalize_alpha(alpha, x.device), floor, ceiling, True)
    return dx, dalpha


@ema_bwd.register_fake
def _ema_bwd_fake(x, y, dy, alpha, floor, ceiling):
    return x.new_empty(x.shape), x.new_empty((alpha.numel(),), dtype=torch.float32)
