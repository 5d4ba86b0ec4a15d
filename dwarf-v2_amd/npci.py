"""NPCI rotation on MI355X, drop-in for ``npci_rotate`` (kernels/dsqg_attention_v22.py:221-254).

``npci_rotate(x, x_delta, theta_h, *, strength_tau=0.25)`` keeps the
reference's arguments, errors and result: each row of x [B,H,T,hd] is turned
toward the part of its delta perpendicular to it by theta_h tanh(|p| /
(tau |x|)), preserving its norm (an exact no-op at a zero delta), and the
result has x's dtype.  The DSQG module applies it to K and V with the
kv_inject deltas (dsqg:3196-3229).  Forward and backward are fused HIP
kernels (the reference leaves the backward to autograd); dtheta is summed in
a fixed order.  Built for head_dim 64; x and the delta may be bf16 or fp32.
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _lib
from .dsqg import HEAD_DIM, _kernel_rows, _stream


def _dt(t: torch.Tensor) -> int:
    return _lib.DWARF_BF16 if t.dtype == torch.bfloat16 else _lib.DWARF_F32


def _operand(t: torch.Tensor) -> torch.Tensor:
    if t.dtype not in (torch.bfloat16, torch.float32):
        t = t.float()
    return _kernel_rows(t)


def _fill(a: _lib.NpciFwdArgs, x: torch.Tensor, d: torch.Tensor, theta: torch.Tensor, tau: float) -> None:
    B, H, T, hd = x.shape
    a.B, a.H, a.T, a.head_dim = B, H, T, hd
    a.x_dtype, a.delta_dtype = _dt(x), _dt(d)
    a.strength_tau = float(tau)
    a.x, a.x_stride = x.data_ptr(), _lib.i64_array(x.stride())
    a.delta, a.delta_stride = d.data_ptr(), _lib.i64_array(d.stride())
    a.theta = theta.data_ptr()


def _theta(theta_h: torch.Tensor, device) -> torch.Tensor:
    return theta_h.detach().to(device=device, dtype=torch.float32).reshape(-1).contiguous()


def npci_forward(x: torch.Tensor, x_delta: torch.Tensor, theta_h: torch.Tensor, tau: float) -> torch.Tensor:
    """Raw launch: the rotated rows, [B,H,T,hd] contiguous, in the kernel dtype of x."""
    lib = _lib.load()
    xx, dd = _operand(x), _operand(x_delta.to(x.device))
    th = _theta(theta_h, x.device)
    out = torch.empty(xx.shape, device=x.device, dtype=xx.dtype)
    a = _lib.NpciFwdArgs()
    _fill(a, xx, dd, th, tau)
    a.out, a.out_stride = out.data_ptr(), _lib.i64_array(out.stride())
    _lib.check(lib.dwarf_npci_fwd(ctypes.byref(a), _stream(x.device)), "dwarf_npci_fwd")
    return out


def npci_backward(x: torch.Tensor, x_delta: torch.Tensor, theta_h: torch.Tensor, grad: torch.Tensor,
                  tau: float) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Raw launch: (dx in x's kernel dtype, ddelta in the delta's kernel dtype, dtheta [H] fp32)."""
    lib = _lib.load()
    xx, dd = _operand(x), _operand(x_delta.to(x.device))
    th = _theta(theta_h, x.device)
    g = _kernel_rows(grad.to(device=x.device, dtype=xx.dtype))
    dx = torch.empty(xx.shape, device=x.device, dtype=xx.dtype)
    ddelta = torch.empty(dd.shape, device=x.device, dtype=dd.dtype)
    dtheta = torch.empty(th.shape, device=x.device, dtype=torch.float32)
    a = _lib.NpciBwdArgs()
    _fill(a.fwd, xx, dd, th, tau)
    a.grad, a.grad_stride = g.data_ptr(), _lib.i64_array(g.stride())
    a.dx, a.dx_stride = dx.data_ptr(), _lib.i64_array(dx.stride())
    a.ddelta, a.ddelta_stride = ddelta.data_ptr(), _lib.i64_array(ddelta.stride())
    a.dtheta = dtheta.data_ptr()
    ws = torch.empty(max(int(lib.dwarf_npci_bwd_workspace_bytes(ctypes.byref(a))), 16), device=x.device,
                     dtype=torch.uint8)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    _lib.check(lib.dwarf_npci_bwd(ctypes.byref(a), _stream(x.device)), "dwarf_npci_bwd")
    return dx, ddelta, dtheta


class _NPCIRotateFn(torch.autograd.Function):
    """Autograd wrapper over ``torch.ops.dwarf.npci_fwd`` / ``npci_bwd`` (registered in ``ops.py``)."""

    @staticmethod
    def forward(ctx, x, x_delta, theta_h, tau: float):
        out = torch.ops.dwarf.npci_fwd(x, x_delta, theta_h, tau)
        ctx.save_for_backward(x, x_delta, theta_h)
        ctx.tau = tau
        return out

    @staticmethod
    def backward(ctx, grad):
        x, x_delta, theta_h = ctx.saved_tensors
        dx, dd, dt = torch.ops.dwarf.npci_bwd(x, x_delta, theta_h, grad, ctx.tau)
        return (dx.to(x.dtype), dd.to(x_delta.dtype) if ctx.needs_input_grad[1] else None,
                dt.reshape(theta_h.shape).to(theta_h.dtype) if ctx.needs_input_grad[2] else None, None)


def npci_rotate(x: torch.Tensor, x_delta: torch.Tensor, theta_h: torch.Tensor, *,
                strength_tau: float = 0.25) -> torch.Tensor:
    """Magnitude-aware norm-preserving NPCI rotation (reference signature: dsqg:221-254)."""
    tau = float(strength_tau)
    if not math.isfinite(tau) or tau <= 0:
        raise ValueError("strength_tau must be finite and positive")
    if x.ndim != 4 or x_delta.shape != x.shape:
        raise ValueError(f"x and x_delta must be [B,H,T,hd] of one shape, got {tuple(x.shape)} and "
                         f"{tuple(x_delta.shape)}")
    if theta_h.numel() != x.shape[1]:
        raise ValueError(f"theta_h must hold one angle per head ({x.shape[1]}), got {theta_h.numel()}")
    if not x.is_cuda:
        raise RuntimeError("the NPCI HIP kernels require device tensors")
    if x.shape[-1] != HEAD_DIM:
        raise RuntimeError(f"the NPCI kernels are built for head_dim {HEAD_DIM}, got {x.shape[-1]}")
    out = _NPCIRotateFn.apply(x, x_delta, theta_h, tau)
    return out if out.dtype == x.dtype else out.to(x.dtype)
