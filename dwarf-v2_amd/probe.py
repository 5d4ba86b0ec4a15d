"""Phase-probe features on MI355X, drop-in for kernels/dsqg_attention_v22.py:371-451.

``phase_probe_features`` (dsqg:422-451) and ``_PhaseProbeFn`` (dsqg:371-419)
keep the reference's names, arguments and results:

    y[b,h,n,r] = <x[b,h,n], p_r> / sqrt(|x[b,h,n]|^2 + 1e-6 hd)

for rows n in [start, end) and 0 for every other row, fp32, with gradients
for x (in x's dtype) and for the probes.  The HIP kernels of
libdwarf_dsqg.so are built for head_dim 64 and R_PLANES = 4 probes, the DSQG
block's shapes (dsqg:3231-3254); x is bf16 or fp32 (other floating dtypes
are widened to fp32).  The dprobes sum has a fixed order.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .dsqg import HEAD_DIM, _kernel_rows, _planes, _stream
from .lattice import R_PLANES


def _span(n: int, start: int, end: int | None) -> tuple[int, int]:
    """Clamp [start, end) to [0, n] as dsqg:377-379 and 441-443 do."""
    s = max(0, min(int(start), n))
    e = n if end is None else max(s, min(int(end), n))
    return s, e


def _values(x: torch.Tensor) -> torch.Tensor:
    if x.dtype not in (torch.bfloat16, torch.float32):
        x = x.float()
    return _kernel_rows(x)


def _fill_fwd(a: _lib.PhaseProbeFwdArgs, x: torch.Tensor, probes: torch.Tensor, start: int, end: int) -> None:
    B, H, N, hd = x.shape
    a.B, a.H, a.N, a.head_dim, a.R = B, H, N, hd, probes.shape[0]
    a.start, a.end = start, end
    a.dtype = _lib.DWARF_BF16 if x.dtype == torch.bfloat16 else _lib.DWARF_F32
    a.x, a.x_stride = x.data_ptr(), _lib.i64_array(x.stride())
    a.probes = probes.data_ptr()


def probe_forward(values: torch.Tensor, probes: torch.Tensor, start: int, end: int) -> torch.Tensor:
    """Raw launch: y [B,H,N,R] fp32 (every row written)."""
    lib = _lib.load()
    x = _values(values)
    p = _planes(probes.detach().to(device=x.device, dtype=torch.float32))
    out = torch.empty((*x.shape[:3], p.shape[0]), device=x.device, dtype=torch.float32)
    a = _lib.PhaseProbeFwdArgs()
    _fill_fwd(a, x, p, start, end)
    a.out, a.out_stride = out.data_ptr(), _lib.i64_array(out.stride())
    _lib.check(lib.dwarf_phase_probe_fwd(ctypes.byref(a), _stream(x.device)), "dwarf_phase_probe_fwd")
    return out


def probe_backward(values: torch.Tensor, probes: torch.Tensor, dout: torch.Tensor, start: int, end: int,
                   need_dprobes: bool) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Raw launch: (dx in the kernel dtype, dprobes fp32 [R,hd] or None)."""
    lib = _lib.load()
    x = _values(values)
    p = _planes(probes.detach().to(device=x.device, dtype=torch.float32))
    g = dout.to(device=x.device, dtype=torch.float32)
    dx = torch.empty(x.shape, device=x.device, dtype=x.dtype)
    dprobes = torch.empty(p.shape, device=x.device, dtype=torch.float32) if need_dprobes else None
    a = _lib.PhaseProbeBwdArgs()
    _fill_fwd(a.fwd, x, p, start, end)
    a.dout, a.dout_stride = g.data_ptr(), _lib.i64_array(g.stride())
    a.dx, a.dx_stride = dx.data_ptr(), _lib.i64_array(dx.stride())
    a.dprobes = dprobes.data_ptr() if dprobes is not None else None
    ws = torch.empty(max(int(lib.dwarf_phase_probe_bwd_workspace_bytes(ctypes.byref(a))), 16), device=x.device,
                     dtype=torch.uint8)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    _lib.check(lib.dwarf_phase_probe_bwd(ctypes.byref(a), _stream(x.device)), "dwarf_phase_probe_bwd")
    return dx, dprobes


def _check(values: torch.Tensor, probes: torch.Tensor) -> None:
    if values.ndim != 4:
        raise ValueError(f"values must be [B,H,N,hd], got {tuple(values.shape)}")
    if probes.ndim != 2 or probes.shape[1] != values.shape[-1]:
        raise ValueError(f"probes must be [R,{values.shape[-1]}], got {tuple(probes.shape)}")
    if not values.is_cuda:
        raise RuntimeError("the phase-probe HIP kernels require device tensors")
    if values.shape[-1] != HEAD_DIM or probes.shape[0] != R_PLANES:
        raise RuntimeError(f"the phase-probe kernels are built for head_dim {HEAD_DIM} and {R_PLANES} probes, "
                           f"got head_dim {values.shape[-1]} and {probes.shape[0]} probes")


class _PhaseProbeFn(torch.autograd.Function):
    """Autograd wrapper (reference: dsqg:371-419) over ``torch.ops.dwarf.phase_probe_fwd`` /
    ``phase_probe_bwd`` (registered in ``ops.py``)."""

    @staticmethod
    def forward(ctx, values, probes, start: int, end: int):
        _check(values, probes)
        s, e = _span(values.shape[2], start, end)
        out = torch.ops.dwarf.phase_probe_fwd(values, probes, s, e)
        ctx.save_for_backward(values, probes)
        ctx.start, ctx.end = s, e
        return out

    @staticmethod
    def backward(ctx, grad_output):
        values, probes = ctx.saved_tensors
        need_probes = bool(ctx.needs_input_grad[1])
        dx, dprobes = torch.ops.dwarf.phase_probe_bwd(values, probes, grad_output, ctx.start, ctx.end, need_probes)
        return dx.to(values.dtype), (dprobes.to(probes.dtype) if need_probes else None), None, None


def phase_probe_features(values: torch.Tensor, probes: torch.Tensor, *, start: int = 0,
                         end: int | None = None) -> torch.Tensor:
    """Project RMS-normalised head vectors onto the probe bank (reference signature: dsqg:422-451).

    Rows outside [start, end) are zero.  values [B,H,N,64] on the GPU, probes [4,64].
    """
    _check(values, probes)
    s, e = _span(values.shape[2], start, end)
    return _PhaseProbeFn.apply(values, probes, s, e)
