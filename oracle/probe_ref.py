"""CPU restatement of the phase-probe features -- test infrastructure, not the product.

Forward (kernels/dsqg_attention_v22.py:422-451, the eager branch, and the
kernel dsqg:275-306): for rows n in [start, end)

    y[b,h,n,r] = <x[b,h,n], p_r> / sqrt(sum_d x[b,h,n,d]^2 + 1e-6 hd)

and y = 0 outside [start, end).  Backward (the kernel dsqg:309-369), with
inv = 1/sqrt(|x|^2 + 1e-6 hd) and raw_r = <x, p_r>:

    dx[d]      = sum_r g_r (p_r[d] inv - raw_r x[d] inv^3)
    dprobes[r] = sum over rows of g_r inv x

dx is 0 outside [start, end).  float64 for float64 inputs, float32 otherwise.
"""

from __future__ import annotations

import torch


def _span(n: int, start: int, end: int | None) -> tuple[int, int]:
    s = max(0, min(int(start), n))
    e = n if end is None else max(s, min(int(end), n))
    return s, e


def phase_probe_features(x: torch.Tensor, probes: torch.Tensor, start: int = 0, end: int | None = None) -> torch.Tensor:
    acc = torch.float64 if x.dtype == torch.float64 else torch.float32
    s, e = _span(x.shape[2], start, end)
    out = torch.zeros(*x.shape[:3], probes.shape[0], dtype=acc)
    if e > s:
        xs = x[:, :, s:e].to(acc)
        inv = torch.rsqrt(xs.square().sum(-1, keepdim=True) + 1e-6 * x.shape[-1])
        out[:, :, s:e] = torch.einsum("bhnd,rd->bhnr", xs, probes.to(acc)) * inv
    return out


def phase_probe_backward(x: torch.Tensor, probes: torch.Tensor, dout: torch.Tensor, start: int = 0,
                         end: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    acc = torch.float64 if x.dtype == torch.float64 else torch.float32
    s, e = _span(x.shape[2], start, end)
    dx = torch.zeros(x.shape, dtype=acc)
    dprobes = torch.zeros(probes.shape, dtype=acc)
    if e > s:
        xs = x[:, :, s:e].to(acc)
        p = probes.to(acc)
        g = dout[:, :, s:e].to(acc)                                        # [b,h,n,r]
        inv = torch.rsqrt(xs.square().sum(-1, keepdim=True) + 1e-6 * x.shape[-1])
        raw = torch.einsum("bhnd,rd->bhnr", xs, p)
        dx[:, :, s:e] = torch.einsum("bhnr,rd->bhnd", g, p) * inv \
            - (g * raw).sum(-1, keepdim=True) * xs * inv ** 3
        dprobes = torch.einsum("bhnr,bhnd->rd", g * inv, xs)
    return dx, dprobes
