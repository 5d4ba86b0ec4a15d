"""Pin the CPU NPCI oracle (no GPU).

npci_rotate (kernels/dsqg_attention_v22.py:221-254) preserves the row norm,
turns x by exactly theta * tanh(|p| / (tau |x|)) toward the part of delta
perpendicular to x, and is the identity for a zero delta or a delta parallel
to x.  The restated backward equals autograd of the restated forward, which
passes gradcheck.
"""

import math

import pytest
import torch

from oracle import npci_ref


def _inputs(seed, B=2, H=3, T=7, hd=16):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, H, T, hd, generator=g, dtype=torch.float64)
    d = 0.3 * torch.randn(B, H, T, hd, generator=g, dtype=torch.float64)
    th = 0.25 * torch.tanh(torch.randn(H, generator=g, dtype=torch.float64))
    return x, d, th


def test_norm_preserved_and_angle_closed_form():
    x, d, th = _inputs(0)
    tau = 0.25
    r = npci_ref.npci_rotate(x, d, th, tau)
    assert float((r.norm(dim=-1) - x.norm(dim=-1)).abs().max()) < 1e-12
    n = x.norm(dim=-1)
    u = x / n[..., None]
    p = d - (d * u).sum(-1, keepdim=True) * u
    m = p.norm(dim=-1)
    want = th.reshape(1, -1, 1) * torch.tanh(m / (tau * n + 1e-12))
    cosang = (r * x).sum(-1) / (n * n)
    assert float((torch.acos(cosang.clamp(-1, 1)) - want.abs()).abs().max()) < 1e-6
    # the rotation stays in the plane of x and p
    resid = r - (r * u).sum(-1, keepdim=True) * u - (r * p).sum(-1, keepdim=True) * p / (m * m)[..., None]
    assert float(resid.abs().max()) < 1e-12


def test_identity_cases():
    x, d, th = _inputs(1)
    assert torch.equal(npci_ref.npci_rotate(x, torch.zeros_like(d), th), x)
    par = 2.5 * x
    assert float((npci_ref.npci_rotate(x, par, th) - x).abs().max()) < 1e-12
    assert float((npci_ref.npci_rotate(x, d, torch.zeros_like(th)) - x).abs().max()) < 1e-15


@pytest.mark.parametrize("seed", [2, 3])
def test_backward_restatement_equals_autograd(seed):
    x, d, th = _inputs(seed)
    x[0, 1, 2] = 0.0                    # a zero row: clamped norm
    d[1, 0, 3] = 0.0                    # an inactive row
    d[1, 2, 4] = 3.0 * x[1, 2, 4]       # a parallel (inactive) row
    x.requires_grad_(True), d.requires_grad_(True), th.requires_grad_(True)
    g = torch.randn(x.shape, generator=torch.Generator().manual_seed(seed + 10), dtype=torch.float64)
    r = npci_ref.npci_rotate(x, d, th, 0.3)
    gx, gd, gt = torch.autograd.grad(r, (x, d, th), g)
    dx, dd, dt = npci_ref.npci_rotate_backward(x.detach(), d.detach(), th.detach(), g, 0.3)
    assert float((dx - gx).abs().max()) < 1e-9
    assert float((dd - gd).abs().max()) < 1e-9
    assert float((dt - gt).abs().max()) < 1e-9


def test_gradcheck():
    x, d, th = _inputs(4, B=1, H=2, T=3, hd=8)
    args = (x.requires_grad_(True), d.requires_grad_(True), th.requires_grad_(True))
    assert torch.autograd.gradcheck(lambda a, b, c: npci_ref.npci_rotate(a, b, c, 0.25), args)
