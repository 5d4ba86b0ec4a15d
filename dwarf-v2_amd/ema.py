"""Causal EMA scan on MI355X, drop-in for kernels/causal_ema_scan.py.

``causal_ema_scan`` (ema:541-567), ``bounded_ema_factor`` (ema:37-47) and
``inverse_bounded_ema_factor`` (ema:50-61) keep the reference's names,
arguments and errors.  The scan runs the HIP kernels of libdwarf_dsqg.so:
y[t] = a x[t] + (1 - a) y[t-1] with fp32 state, a = clamp(ema_factor, floor,
ceiling).  ``ema_factor`` may hold one value (the reference contract) or one
value per channel of x (an extension used by the long-context benchmark).
With ``reset_mask`` [B,N] the state is zeroed before the marked tokens, the
reset-aware scan of ``_CausalEMAResetFn`` (ema:368-509), on the same kernels:
a single-pass scan with decoupled look-back (a three-stage chunked scan for
slabs over 2 GiB).
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _lib


def bounded_ema_factor(raw: torch.Tensor, *, floor: float = 1e-5, ceiling: float = 0.5) -> torch.Tensor:
    """Map an unconstrained value smoothly into (floor, ceiling)."""
    floor, ceiling = float(floor), float(ceiling)
    if not (math.isfinite(floor) and math.isfinite(ceiling) and 0 < floor < ceiling < 1):
        raise ValueError("EMA bounds must satisfy 0 < floor < ceiling < 1")
    return floor + (ceiling - floor) * torch.sigmoid(raw)


def inverse_bounded_ema_factor(alpha: float, *, floor: float = 1e-5, ceiling: float = 0.5) -> float:
    """Raw value whose bounded_ema_factor is ``alpha``."""
    alpha, floor, ceiling = float(alpha), float(floor), float(ceiling)
    if not floor < alpha < ceiling:
        raise ValueError(f"alpha must be strictly inside ({floor}, {ceiling})")
    p = (alpha - floor) / (ceiling - floor)
    return math.log(p / (1.0 - p))


def _btd_ok(t: torch.Tensor) -> bool:
    if t.stride(-1) != 1:
        return False
    if t.shape[-1] % 4:
        return True
    align = 8 if t.element_size() == 2 else 16
    return t.data_ptr() % align == 0 and t.stride(0) % 4 == 0 and t.stride(1) % 4 == 0


def _btd(t: torch.Tensor) -> torch.Tensor:
    return t if _btd_ok(t) else t.contiguous()


def normalize_x(x: torch.Tensor) -> torch.Tensor:
    """[B,N,D] rows the kernels read: unit channel stride, 8/16-byte vectors when D % 4 == 0."""
    return _btd(x)


def normalize_alpha(alpha: torch.Tensor, device: torch.device) -> torch.Tensor:
    return alpha.detach().to(device=device, dtype=torch.float32).reshape(-1).contiguous()


def normalize_reset(reset_mask: torch.Tensor | None, x: torch.Tensor) -> torch.Tensor | None:
    """[B,N] one byte per token on x's device (torch.bool), or None."""
    if reset_mask is None:
        return None
    if tuple(reset_mask.shape) != tuple(x.shape[:2]):
        raise ValueError(f"reset_mask must have shape {tuple(x.shape[:2])}")
    return reset_mask.to(device=x.device, dtype=torch.bool)


def _set_reset(a, reset: torch.Tensor | None) -> None:
    if reset is not None:
        a.reset, a.reset_stride = reset.data_ptr(), _lib.i64_array(reset.stride())


def ema_forward(x: torch.Tensor, alpha: torch.Tensor, floor: float, ceiling: float,
                reset: torch.Tensor | None = None, *, wait_limit: int = 0) -> torch.Tensor:
    """Raw launch: y with x's dtype.  alpha fp32 on x's device, numel 1 or D; reset [B,N] bool or None.
    wait_limit: polls before a look-back wait gives up (its channel's tile then holds NaN); 0: the default."""
    lib = _lib.load()
    B, N, D = x.shape
    y = torch.empty((B, N, D), device=x.device, dtype=x.dtype)
    a = _lib.EmaFwdArgs()
    a.B, a.N, a.D = B, N, D
    a.dtype = _lib.DWARF_F32 if x.dtype == torch.float32 else _lib.DWARF_BF16
    a.alpha_per_channel = int(alpha.numel() != 1)
    a.floor_, a.ceiling = float(floor), float(ceiling)
    a.x, a.x_stride = x.data_ptr(), _lib.i64_array(x.stride())
    a.alpha = alpha.data_ptr()
    a.y, a.y_stride = y.data_ptr(), _lib.i64_array(y.stride())
    a.wait_limit = int(wait_limit)
    _set_reset(a, reset)
    ws = torch.empty(max(int(lib.dwarf_ema_fwd_workspace_bytes(ctypes.byref(a))), 16), device=x.device,
                     dtype=torch.uint8)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    _lib.check(lib.dwarf_ema_fwd(ctypes.byref(a), torch.cuda.current_stream(x.device).cuda_stream), "dwarf_ema_fwd")
    return y


def ema_backward(x, y, dy, alpha, floor, ceiling, need_dalpha: bool, reset: torch.Tensor | None = None, *,
                 wait_limit: int = 0):
    """Raw launch: (dx, dalpha or None); dalpha already clamp-projected; reset and wait_limit as in
    ema_forward."""
    lib = _lib.load()
    B, N, D = x.shape
    dy = _btd(dy.to(x.dtype))
    dx = torch.empty((B, N, D), device=x.device, dtype=x.dtype)
    dalpha = torch.empty(alpha.numel(), device=x.device, dtype=torch.float32) if need_dalpha else None
    a = _lib.EmaBwdArgs()
    a.B, a.N, a.D = B, N, D
    a.dtype = _lib.DWARF_F32 if x.dtype == torch.float32 else _lib.DWARF_BF16
    a.alpha_per_channel = int(alpha.numel() != 1)
    a.floor_, a.ceiling = float(floor), float(ceiling)
    a.x, a.x_stride = x.data_ptr(), _lib.i64_array(x.stride())
    a.y, a.y_stride = y.data_ptr(), _lib.i64_array(y.stride())
    a.dy, a.dy_stride = dy.data_ptr(), _lib.i64_array(dy.stride())
    a.alpha = alpha.data_ptr()
    a.dx, a.dx_stride = dx.data_ptr(), _lib.i64_array(dx.stride())
    a.dalpha = dalpha.data_ptr() if dalpha is not None else None
    a.wait_limit = int(wait_limit)
    _set_reset(a, reset)
    ws = torch.empty(max(int(lib.dwarf_ema_bwd_workspace_bytes(ctypes.byref(a))), 16), device=x.device,
                     dtype=torch.uint8)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    _lib.check(lib.dwarf_ema_bwd(ctypes.byref(a), torch.cuda.current_stream(x.device).cuda_stream), "dwarf_ema_bwd")
    return dx, dalpha


class _CausalEMAFn(torch.autograd.Function):
    """Autograd wrapper (reference: ema:263-364) over the custom ops ``torch.ops.dwarf.ema_fwd`` /
    ``ema_bwd`` (registered in ``ops.py``)."""

    @staticmethod
    def forward(ctx, x, alpha_input, floor, ceiling):
        alpha = alpha_input.detach().to(device=x.device, dtype=torch.float32).reshape(-1)
        y = torch.ops.dwarf.ema_fwd(x, alpha, float(floor), float(ceiling))
        ctx.save_for_backward(x, y, alpha)
        ctx.floor, ctx.ceiling = float(floor), float(ceiling)
        ctx.alpha_shape, ctx.alpha_dtype = alpha_input.shape, alpha_input.dtype
        return y

    @staticmethod
    def backward(ctx, dy):
        x, y, alpha = ctx.saved_tensors
        dx, dalpha = torch.ops.dwarf.ema_bwd(x, y, dy, alpha, ctx.floor, ctx.ceiling)
        if not ctx.needs_input_grad[1]:
            return dx, None, None, None
        return dx, dalpha.reshape(ctx.alpha_shape).to(ctx.alpha_dtype), None, None


class _CausalEMAResetFn(torch.autograd.Function):
    """Reset-aware scan (reference: ema:455-509, same arguments and gradient slots) over the
    same custom ops with a reset mask."""

    @staticmethod
    def forward(ctx, x, alpha_input, reset_mask, floor, ceiling):
        reset = normalize_reset(reset_mask, x)
        alpha = alpha_input.detach().to(device=x.device, dtype=torch.float32).reshape(-1)
        y = torch.ops.dwarf.ema_fwd(x, alpha, float(floor), float(ceiling), reset)
        ctx.save_for_backward(x, y, alpha, reset)
        ctx.floor, ctx.ceiling = float(floor), float(ceiling)
        ctx.alpha_shape, ctx.alpha_dtype = alpha_input.shape, alpha_input.dtype
        return y

    @staticmethod
    def backward(ctx, dy):
        x, y, alpha, reset = ctx.saved_tensors
        dx, dalpha = torch.ops.dwarf.ema_bwd(x, y, dy, alpha, ctx.floor, ctx.ceiling, reset)
        if not ctx.needs_input_grad[1]:
            return dx, None, None, None, None
        return dx, dalpha.reshape(ctx.alpha_shape).to(ctx.alpha_dtype), None, None, None


def causal_ema_scan(x: torch.Tensor, ema_factor: torch.Tensor, floor: float = 1e-5, ceiling: float = 0.5, *,
                    reset_mask: torch.Tensor | None = None) -> torch.Tensor:
    """Causal EMA of x[B,N,D] on the HIP kernels (reference signature: ema:541-567)."""
    if x.ndim != 3:
        raise ValueError(f"x must be [B,N,D], got {tuple(x.shape)}")
    if ema_factor.numel() not in (1, x.shape[2]):
        raise ValueError("ema_factor must contain one scalar or one value per channel")
    if not (0 < float(floor) < float(ceiling) < 1):
        raise ValueError("EMA bounds must satisfy 0 < floor < ceiling < 1")
    if reset_mask is not None and tuple(reset_mask.shape) != tuple(x.shape[:2]):
        raise ValueError(f"reset_mask must have shape {tuple(x.shape[:2])}")
    if not x.is_cuda:
        raise RuntimeError("the EMA HIP kernels require device tensors")
    # bf16 runs the bf16 kernels; every other dtype computes in fp32 (the reference's state and
    # arithmetic, ema:272-278) and the result is cast back to x's dtype
    xin = x if x.dtype in (torch.float32, torch.bfloat16) else x.to(torch.float32)
    if reset_mask is not None:
        out = _CausalEMAResetFn.apply(xin, ema_factor, reset_mask, float(floor), float(ceiling))
    else:
        out = _CausalEMAFn.apply(xin, ema_factor, float(floor), float(ceiling))
    return out if out.dtype == x.dtype else out.to(x.dtype)
