"""CPU restatement of the NPCI rotation -- test infrastructure, not the product.

Follows ``npci_rotate`` (kernels/dsqg_attention_v22.py:221-254): per row x of
[B,H,T,hd] with delta d and the head's angle theta_h,

    n = max(|x|, 1e-12), u = x / n, p = d - (d.u) u, m = |p|
    active = m > 1e-7 n, e = p / max(m, 1e-20) (0 when not active)
    s = tanh(m / (tau n + 1e-12)), a = theta_h s
    r = cos(a) x + sin(a) n e          (r = x where not active)

in float64 for float64 inputs and float32 otherwise.  ``npci_rotate_backward``
restates the vector-Jacobian products of that expression for (x, d, theta).
"""

from __future__ import annotations

import torch


def _acc(x: torch.Tensor):
    return torch.float64 if x.dtype == torch.float64 else torch.float32


def npci_rotate(x: torch.Tensor, x_delta: torch.Tensor, theta_h: torch.Tensor, strength_tau: float = 0.25) -> torch.Tensor:
    acc = _acc(x)
    xf, df = x.to(acc), x_delta.to(acc)
    theta = theta_h.to(acc).reshape(1, -1, 1, 1)
    norm = xf.norm(dim=-1, keepdim=True).clamp_min(1e-12)
    unit = xf / norm
    perp = df - (df * unit).sum(dim=-1, keepdim=True) * unit
    pn = perp.norm(dim=-1, keepdim=True)
    active = pn > norm * 1e-7
    direction = torch.where(active, perp / pn.clamp_min(1e-20), torch.zeros_like(perp))
    strength = torch.tanh(pn / (strength_tau * norm + 1e-12))
    angle = theta * strength
    rotated = torch.cos(angle) * xf + torch.sin(angle) * norm * direction
    return torch.where(active, rotated, xf)


def npci_rotate_backward(x: torch.Tensor, x_delta: torch.Tensor, theta_h: torch.Tensor, grad: torch.Tensor,
                         strength_tau: float = 0.25):
    """(dx, dx_delta, dtheta [H]) of npci_rotate for the output gradient ``grad``."""
    acc = _acc(x)
    xf, df, g = x.to(acc), x_delta.to(acc), grad.to(acc)
    theta = theta_h.to(acc).reshape(1, -1, 1, 1)
    tau = float(strength_tau)
    raw = xf.norm(dim=-1, keepdim=True)
    clamped = raw < 1e-12
    norm = raw.clamp_min(1e-12)
    unit = xf / norm
    c1 = (df * unit).sum(-1, keepdim=True)
    p = df - c1 * unit
    m = p.norm(dim=-1, keepdim=True)
    active = m > norm * 1e-7
    e = torch.where(active, p / m.clamp_min(1e-20), torch.zeros_like(p))
    den = tau * norm + 1e-12
    s = torch.tanh(m / den)
    a = theta * s
    sa, ca = torch.sin(a), torch.cos(a)
    s_gx = (g * xf).sum(-1, keepdim=True)
    s_ge = (g * e).sum(-1, keepdim=True)
    ga = -sa * s_gx + ca * norm * s_ge
    dtheta = (ga * s).where(active, torch.zeros_like(s)).sum(dim=(0, 2, 3))
    gs = ga * theta
    gw = gs * (1 - s * s)
    gm = gw / den
    gn = -gw * m * tau / (den * den) + sa * s_ge
    ge = sa * norm * g
    gp = (ge - e * (e * ge).sum(-1, keepdim=True)) / m.clamp_min(1e-20) + gm * e
    ugp = (unit * gp).sum(-1, keepdim=True)
    gd = gp - unit * ugp
    gu = -c1 * gp - df * ugp
    ugu = (unit * gu).sum(-1, keepdim=True)
    gx_unit = torch.where(clamped, gu / norm, (gu - unit * ugu) / norm)
    gx_norm = torch.where(clamped, torch.zeros_like(gn), gn) * unit
    gx = ca * g + gx_unit + gx_norm
    dx = torch.where(active, gx, g)
    dd = torch.where(active, gd, torch.zeros_like(gd))
    return dx, dd, dtheta
