"""Seeded DSQG inputs shared by the GPU tests, the smoke check and the bench.

Inputs are drawn on the CPU from torch.Generator(seed) in a fixed order, so
the CPU oracle and the GPU see identical values.  y/z are the probe features
of q/k with the module's deterministic orthogonal probes (dsqg:257-268,
3231-3254).  Defaults follow the benchmark's synthetic recipe: q/k/v ~ N(0,1),
pos_bias ~ N(0, 0.02^2), centred scale_embed ~ N(0, 0.01^2),
phase_base ~ 0.5 N(0, 0.01^2), phase_gain ~ 0.5 N(0, 1.28^2).
"""

from __future__ import annotations

import torch

NAMES = ("q", "k", "v", "pos_bias", "scale_embed", "phase_base", "phase_gain", "y_pre", "z_pre")


def orthogonal_probes(hd: int, plane_shift: int):
    """Normalised q/k probes on the plane channel pairs (dsqg:257-268)."""
    import math

    q = torch.zeros(4, hd)
    k = torch.zeros(4, hd)
    seg = hd // 4
    for r in range(4):
        a, b = r * seg + plane_shift, r * seg + plane_shift + 1
        ang = 2.0 * math.pi * r / 4
        q[r, a], q[r, b] = math.cos(ang), math.sin(ang)
        k[r, a], k[r, b] = math.cos(ang + math.pi / 2), math.sin(ang + math.pi / 2)
    return q, k


def features(x: torch.Tensor, probes: torch.Tensor) -> torch.Tensor:
    xf = x.float()
    inv = torch.rsqrt(xf.square().sum(-1, keepdim=True) + 1e-6 * x.shape[-1])
    return (torch.einsum("bhnd,rd->bhnr", xf, torch.nn.functional.normalize(probes.float(), dim=-1)) * inv).contiguous()


def make_inputs(B, H, Hkv, N, offsets, j_small, *, seed=0, dtype=torch.float32, plane_shift=0,
                gain_std=1.28, hd=64):
    """Dict of CPU tensors.  q/k/v are rounded to ``dtype``; tables and y/z are fp32."""
    J = len(offsets)
    jl = max(J - j_small, 1)
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, N, hd, generator=g).to(dtype)
    k = torch.randn(B, Hkv, N, hd, generator=g).to(dtype)
    v = torch.randn(B, Hkv, N, hd, generator=g).to(dtype)
    pos_bias = 0.02 * torch.randn(J, H, generator=g)
    se = 0.01 * torch.randn(J, hd, generator=g)
    se = se - se.mean(0, keepdim=True)
    phase_base = 0.5 * 0.01 * torch.randn(jl, H, 4, generator=g)
    phase_gain = 0.5 * gain_std * torch.randn(jl, H, 4, generator=g)
    qp, kp = orthogonal_probes(hd, plane_shift)
    return dict(q=q, k=k, v=v, pos_bias=pos_bias, scale_embed=se, phase_base=phase_base,
                phase_gain=phase_gain, y_pre=features(q, qp), z_pre=features(k, kp))


def to_device(x: dict, device) -> dict:
    return {n: t.to(device) for n, t in x.items()}


def rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    """||a - b||_inf / ||b||_inf, the relative metric of the fp32 parity bar."""
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


def max_abs(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a.detach().double().cpu() - b.detach().double().cpu()).abs().max())
