"""InterferencePacket pool on MI355X (train/train_dwarf.py:260-284).

The reference's ``InterferencePacket.forward`` scans the L3 block's input
with ``causal_ema_scan`` once per timescale (three, train:131) and mixes the
scans with softmax weights (train:262-267): K reads of x, K scan outputs and
a chain of bf16 products and sums.  ``interference_pool`` returns the same
``pooled`` from one fused HIP pass (x read twice, pooled written once) and
its backward gives dx, the gradient of each factor (projected for its clamp
as ema:357-364 does) and of each mixture weight, all in a fixed summation
order.  ``interference_packet`` goes on to the packet itself (train:268-273:
the RMS direction, the tanh confidence and the sigmoid gate) in the same
pass, with its backward down to the gate logits.
``interference_packet_forward`` is ``InterferencePacket.forward`` on it; the
gate and key/value projections (GEMMs) stay in PyTorch.
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _lib
from .dsqg import _stream
from .ema import normalize_x

CHUNK_T = 16   # tokens per scan chunk of the HIP kernels (the state's second dimension)


def _fill(a: _lib.PacketPoolFwdArgs, x: torch.Tensor, alpha: torch.Tensor, weight: torch.Tensor, floor: float,
          ceiling: float) -> None:
    B, N, D = x.shape
    a.B, a.N, a.D, a.K = B, N, D, alpha.numel()
    a.dtype = _lib.DWARF_BF16 if x.dtype == torch.bfloat16 else _lib.DWARF_F32
    a.floor_, a.ceiling = float(floor), float(ceiling)
    a.x, a.x_stride = x.data_ptr(), _lib.i64_array(x.stride())
    a.alpha, a.weight = alpha.data_ptr(), weight.data_ptr()


def _vec(t: torch.Tensor, device) -> torch.Tensor:
    return t.detach().to(device=device, dtype=torch.float32).reshape(-1).contiguous()


def state_shape(x: torch.Tensor, K: int) -> tuple[int, int, int]:
    """[B, ceil(N/16), K*D]: each chunk's incoming scan states, written by the forward, read by the backward."""
    B, N, D = x.shape
    return B, (N + CHUNK_T - 1) // CHUNK_T, K * D


def pool_forward(x: torch.Tensor, alpha: torch.Tensor, weight: torch.Tensor, floor: float,
                 ceiling: float) -> tuple[torch.Tensor, torch.Tensor]:
    """Raw launch: (pooled with x's dtype, state fp32)."""
    lib = _lib.load()
    x = normalize_x(x)
    al, w = _vec(alpha, x.device), _vec(weight, x.device)
    pooled = torch.empty(x.shape, device=x.device, dtype=x.dtype)
    state = torch.empty(state_shape(x, al.numel()), device=x.device, dtype=torch.float32)
    a = _lib.PacketPoolFwdArgs()
    _fill(a, x, al, w, floor, ceiling)
    a.pooled, a.pooled_stride = pooled.data_ptr(), _lib.i64_array(pooled.stride())
    a.state = state.data_ptr()
    ws = torch.empty(max(int(lib.dwarf_packet_pool_fwd_workspace_bytes(ctypes.byref(a))), 16), device=x.device,
                     dtype=torch.uint8)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    _lib.check(lib.dwarf_packet_pool_fwd(ctypes.byref(a), _stream(x.device)), "dwarf_packet_pool_fwd")
    return pooled, state


def pool_backward(x: torch.Tensor, alpha: torch.Tensor, weight: torch.Tensor, state: torch.Tensor,
                  dpooled: torch.Tensor, floor: float, ceiling: float) -> tuple[torch.Tensor, torch.Tensor,
                                                                               torch.Tensor]:
    """Raw launch: (dx with x's dtype, dalpha [K] fp32 clamp-projected, dweight [K] fp32)."""
    lib = _lib.load()
    x = normalize_x(x)
    al, w = _vec(alpha, x.device), _vec(weight, x.device)
    g = normalize_x(dpooled.to(device=x.device, dtype=x.dtype))
    if tuple(state.shape) != state_shape(x, al.numel()) or state.dtype != torch.float32 or not state.is_contiguous():
        raise ValueError(f"state must be the forward's fp32 [{', '.join(map(str, state_shape(x, al.numel())))}]")
    dx = torch.empty(x.shape, device=x.device, dtype=x.dtype)
    dalpha = torch.empty(al.numel(), device=x.device, dtype=torch.float32)
    dweight = torch.empty(al.numel(), device=x.device, dtype=torch.float32)
    a = _lib.PacketPoolBwdArgs()
    _fill(a.fwd, x, al, w, floor, ceiling)
    a.fwd.state = state.data_ptr()
    a.dpooled, a.dpooled_stride = g.data_ptr(), _lib.i64_array(g.stride())
    a.dx, a.dx_stride = dx.data_ptr(), _lib.i64_array(dx.stride())
    a.dalpha, a.dweight = dalpha.data_ptr(), dweight.data_ptr()
    ws = torch.empty(max(int(lib.dwarf_packet_pool_bwd_workspace_bytes(ctypes.byref(a))), 16), device=x.device,
                     dtype=torch.uint8)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    _lib.check(lib.dwarf_packet_pool_bwd(ctypes.byref(a), _stream(x.device)), "dwarf_packet_pool_bwd")
    return dx, dalpha, dweight


def _dtype_code(dt: torch.dtype) -> int:
    return _lib.DWARF_BF16 if dt == torch.bfloat16 else _lib.DWARF_F32


def packet_forward(x: torch.Tensor, alpha: torch.Tensor, weight: torch.Tensor, gate: torch.Tensor, floor: float,
                   ceiling: float) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Raw launch: (packet with gate's dtype, pooled with x's dtype, state fp32, ms [B,N] fp32)."""
    lib = _lib.load()
    x = normalize_x(x)
    gate = normalize_x(gate)
    al, w = _vec(alpha, x.device), _vec(weight, x.device)
    B, N, D = x.shape
    pooled = torch.empty(x.shape, device=x.device, dtype=x.dtype)
    packet = torch.empty(x.shape, device=x.device, dtype=gate.dtype)
    state = torch.empty(state_shape(x, al.numel()), device=x.device, dtype=torch.float32)
    ms = torch.empty((B, N), device=x.device, dtype=torch.float32)
    a = _lib.PacketFwdArgs()
    _fill(a.pool, x, al, w, floor, ceiling)
    a.pool.pooled, a.pool.pooled_stride = pooled.data_ptr(), _lib.i64_array(pooled.stride())
    a.pool.state = state.data_ptr()
    ws = torch.empty(max(int(lib.dwarf_packet_pool_fwd_workspace_bytes(ctypes.byref(a.pool))), 16), device=x.device,
                     dtype=torch.uint8)
    a.pool.workspace, a.pool.workspace_bytes = ws.data_ptr(), ws.numel()
    a.packet_dtype = _dtype_code(gate.dtype)
    a.gate, a.gate_stride = gate.data_ptr(), _lib.i64_array(gate.stride())
    a.packet, a.packet_stride = packet.data_ptr(), _lib.i64_array(packet.stride())
    a.ms = ms.data_ptr()
    _lib.check(lib.dwarf_packet_fwd(ctypes.byref(a), _stream(x.device)), "dwarf_packet_fwd")
    return packet, pooled, state, ms


def packet_backward(x, alpha, weight, gate, pooled, state, ms, dpacket, floor: float, ceiling: float):
    """Raw launch: (dx with x's dtype, dalpha [K] fp32 clamp-projected, dweight [K] fp32, dgate with gate's
    dtype)."""
    lib = _lib.load()
    x = normalize_x(x)
    gate = normalize_x(gate)
    al, w = _vec(alpha, x.device), _vec(weight, x.device)
    g = normalize_x(dpacket.to(device=x.device, dtype=gate.dtype))
    if tuple(state.shape) != state_shape(x, al.numel()) or state.dtype != torch.float32 or not state.is_contiguous():
        raise ValueError(f"state must be the forward's fp32 [{', '.join(map(str, state_shape(x, al.numel())))}]")
    if tuple(ms.shape) != tuple(x.shape[:2]) or ms.dtype != torch.float32 or not ms.is_contiguous():
        raise ValueError("ms must be the forward's contiguous fp32 [B,N]")
    dx = torch.empty(x.shape, device=x.device, dtype=x.dtype)
    dgate = torch.empty(x.shape, device=x.device, dtype=gate.dtype)
    dalpha = torch.empty(al.numel(), device=x.device, dtype=torch.float32)
    dweight = torch.empty(al.numel(), device=x.device, dtype=torch.float32)
    a = _lib.PacketBwdArgs()
    _fill(a.fwd.pool, x, al, w, floor, ceiling)
    a.fwd.pool.pooled, a.fwd.pool.pooled_stride = pooled.data_ptr(), _lib.i64_array(pooled.stride())
    a.fwd.pool.state = state.data_ptr()
    a.fwd.packet_dtype = _dtype_code(gate.dtype)
    a.fwd.gate, a.fwd.gate_stride = gate.data_ptr(), _lib.i64_array(gate.stride())
    a.fwd.ms = ms.data_ptr()
    a.dpacket, a.dpacket_stride = g.data_ptr(), _lib.i64_array(g.stride())
    a.dgate, a.dgate_stride = dgate.data_ptr(), _lib.i64_array(dgate.stride())
    a.dx, a.dx_stride = dx.data_ptr(), _lib.i64_array(dx.stride())
    a.dalpha, a.dweight = dalpha.data_ptr(), dweight.data_ptr()
    ws = torch.empty(max(int(lib.dwarf_packet_bwd_workspace_bytes(ctypes.byref(a))), 16), device=x.device,
                     dtype=torch.uint8)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    _lib.check(lib.dwarf_packet_bwd(ctypes.byref(a), _stream(x.device)), "dwarf_packet_bwd")
    return dx, dalpha, dweight, dgate


class _InterferencePoolFn(torch.autograd.Function):
    """Autograd wrapper over ``torch.ops.dwarf.packet_pool_fwd`` / ``packet_pool_bwd`` (registered in
    ``ops.py``): gradients for the scan input, the K factors and the K mixture weights."""

    @staticmethod
    def forward(ctx, x, factors, weights, floor: float, ceiling: float):
        alpha = factors.detach().to(device=x.device, dtype=torch.float32).reshape(-1)
        w = weights.detach().to(device=x.device, dtype=torch.float32).reshape(-1)
        pooled, state = torch.ops.dwarf.packet_pool_fwd(x, alpha, w, float(floor), float(ceiling))
        ctx.save_for_backward(x, alpha, w, state)
        ctx.floor, ctx.ceiling = float(floor), float(ceiling)
        ctx.f_shape, ctx.f_dtype = factors.shape, factors.dtype
        ctx.w_shape, ctx.w_dtype = weights.shape, weights.dtype
        return pooled

    @staticmethod
    def backward(ctx, dpooled):
        x, alpha, w, state = ctx.saved_tensors
        dx, dalpha, dweight = torch.ops.dwarf.packet_pool_bwd(x, alpha, w, state, dpooled, ctx.floor, ctx.ceiling)
        df = dalpha.reshape(ctx.f_shape).to(ctx.f_dtype) if ctx.needs_input_grad[1] else None
        dw = dweight.reshape(ctx.w_shape).to(ctx.w_dtype) if ctx.needs_input_grad[2] else None
        return dx.to(x.dtype), df, dw, None, None


def interference_pool(scan_input: torch.Tensor, ema_factors: torch.Tensor, mixture: torch.Tensor, *,
                      floor: float = 1e-5, ceiling: float = 0.5) -> torch.Tensor:
    """``sum(w.to(dtype) * causal_ema_scan(scan_input, a.reshape(1)) for a, w in zip(ema_factors, mixture))``
    (train:262-267) in one fused pass.

    scan_input [B,N,D] bf16 or fp32 on the GPU; ema_factors and mixture hold K <= 4 values each (the
    reference: three timescales, ``bounded_ema_factor(ema_raw)`` and ``softmax(mix_logits)``).
    """
    if scan_input.ndim != 3:
        raise ValueError(f"x must be [B,N,D], got {tuple(scan_input.shape)}")
    K = ema_factors.numel()
    if K != mixture.numel():
        raise ValueError(f"ema_factors ({K}) and mixture ({mixture.numel()}) must have one value per scale")
    if not 1 <= K <= _lib.PACKET_MAX_SCALES:
        raise ValueError(f"1 to {_lib.PACKET_MAX_SCALES} timescales are supported, got {K}")
    if not (math.isfinite(float(floor)) and math.isfinite(float(ceiling)) and 0 < float(floor) < float(ceiling) < 1):
        raise ValueError("EMA bounds must satisfy 0 < floor < ceiling < 1")
    if not scan_input.is_cuda:
        raise RuntimeError("the InterferencePacket pool HIP kernels require device tensors")
    if scan_input.dtype not in (torch.bfloat16, torch.float32):
        raise RuntimeError(f"the InterferencePacket pool kernels take bf16 or fp32 input, got {scan_input.dtype}")
    return _InterferencePoolFn.apply(scan_input, ema_factors, mixture, float(floor), float(ceiling))


class _InterferencePacketFn(torch.autograd.Function):
    """Autograd wrapper over ``torch.ops.dwarf.packet_fwd`` / ``packet_bwd`` (registered in ``ops.py``):
    gradients for the scan input, the K factors, the K mixture weights and the gate logits."""

    @staticmethod
    def forward(ctx, x, factors, weights, gate, floor: float, ceiling: float):
        alpha = factors.detach().to(device=x.device, dtype=torch.float32).reshape(-1)
        w = weights.detach().to(device=x.device, dtype=torch.float32).reshape(-1)
        packet, pooled, state, ms = torch.ops.dwarf.packet_fwd(x, alpha, w, gate, float(floor), float(ceiling))
        ctx.save_for_backward(x, alpha, w, gate, pooled, state, ms)
        ctx.floor, ctx.ceiling = float(floor), float(ceiling)
        ctx.f_shape, ctx.f_dtype = factors.shape, factors.dtype
        ctx.w_shape, ctx.w_dtype = weights.shape, weights.dtype
        return packet

    @staticmethod
    def backward(ctx, dpacket):
        x, alpha, w, gate, pooled, state, ms = ctx.saved_tensors
        dx, dalpha, dweight, dgate = torch.ops.dwarf.packet_bwd(x, alpha, w, gate, pooled, state, ms, dpacket,
                                                                 ctx.floor, ctx.ceiling)
        df = dalpha.reshape(ctx.f_shape).to(ctx.f_dtype) if ctx.needs_input_grad[1] else None
        dw = dweight.reshape(ctx.w_shape).to(ctx.w_dtype) if ctx.needs_input_grad[2] else None
        dg = dgate if ctx.needs_input_grad[3] else None
        return dx.to(x.dtype), df, dw, dg, None, None


def interference_packet(scan_input: torch.Tensor, ema_factors: torch.Tensor, mixture: torch.Tensor,
                        gate_logits: torch.Tensor, *, floor: float = 1e-5, ceiling: float = 0.5) -> torch.Tensor:
    """The InterferencePacket's packet (train:262-273) in one fused pass: ``pooled`` as
    ``interference_pool`` gives it, then per token ``((u * rsqrt(mean(u^2) + 1e-6)) * tanh(rms(u) / 0.25))
    * sigmoid(gate_logits)`` in fp32 with u = pooled, cast to gate_logits' dtype.

    gate_logits [B,N,D] is ``gate_proj(normalized)`` (bf16 or fp32); the result has its dtype, as the
    reference casts the packet to ``normalized.dtype``.  D <= 4096 (<= 1024 when D % 4 != 0).
    """
    if scan_input.ndim != 3 or gate_logits.shape != scan_input.shape:
        raise ValueError(f"scan_input and gate_logits must both be [B,N,D], got {tuple(scan_input.shape)} and "
                         f"{tuple(gate_logits.shape)}")
    if gate_logits.dtype not in (torch.bfloat16, torch.float32):
        raise RuntimeError(f"the packet kernels take bf16 or fp32 gate logits, got {gate_logits.dtype}")
    K = ema_factors.numel()
    if K != mixture.numel():
        raise ValueError(f"ema_factors ({K}) and mixture ({mixture.numel()}) must have one value per scale")
    if not 1 <= K <= _lib.PACKET_MAX_SCALES:
        raise ValueError(f"1 to {_lib.PACKET_MAX_SCALES} timescales are supported, got {K}")
    if not (math.isfinite(float(floor)) and math.isfinite(float(ceiling)) and 0 < float(floor) < float(ceiling) < 1):
        raise ValueError("EMA bounds must satisfy 0 < floor < ceiling < 1")
    if not (scan_input.is_cuda and gate_logits.is_cuda):
        raise RuntimeError("the InterferencePacket HIP kernels require device tensors")
    if scan_input.dtype not in (torch.bfloat16, torch.float32):
        raise RuntimeError(f"the InterferencePacket pool kernels take bf16 or fp32 input, got {scan_input.dtype}")
    return _InterferencePacketFn.apply(scan_input, ema_factors, mixture, gate_logits, float(floor), float(ceiling))


def interference_packet_forward(self, normalized: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``InterferencePacket.forward`` (train:260-284) with the scans, the mix, the RMS direction, the
    confidence and the gate fused; bind it as the class's ``forward``.  Uses the module's ``ema_factors``,
    ``mix_logits``, ``gate_proj``, ``kv_proj``, ``heads`` and ``head_dim`` as the reference does."""
    scan_input = normalized.to(torch.bfloat16) if normalized.is_cuda else normalized
    mixture = torch.softmax(self.mix_logits.float(), dim=0)
    packet = interference_packet(scan_input, self.ema_factors, mixture, self.gate_proj(normalized))
    key_delta, value_delta = self.kv_proj(packet).chunk(2, dim=-1)
    batch, seq_len, _ = normalized.shape
    key_delta = key_delta.reshape(batch, seq_len, self.heads, self.head_dim).permute(0, 2, 1, 3)
    value_delta = value_delta.reshape(batch, seq_len, self.heads, self.head_dim).permute(0, 2, 1, 3)
    return key_delta, value_delta
