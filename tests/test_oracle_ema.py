"""Pin the CPU EMA oracle (no GPU): closed form, reverse adjoint, gradcheck.

The recurrence y[t] = a x[t] + (1-a) y[t-1] (kernels/causal_ema_scan.py:3-11)
has the closed form y[t] = sum_{s<=t} a (1-a)^(t-s) x[s]; the adjoint of
ema:7-11 must equal autograd through the recurrence.
"""

import importlib

import pytest
import torch

from oracle import ema_ref


@pytest.mark.parametrize("per_channel", [False, True])
def test_scan_matches_closed_form(per_channel):
    g = torch.Generator().manual_seed(0)
    x = torch.randn(3, 37, 5, generator=g, dtype=torch.float64)
    alpha = (torch.rand(5 if per_channel else 1, generator=g, dtype=torch.float64) * 0.4 + 0.05)
    y = ema_ref.ema_scan(x, alpha)
    assert float((y - ema_ref.ema_closed_form(x, alpha)).abs().max()) < 1e-13


def test_scalar_is_special_case_of_per_channel():
    x = torch.randn(2, 20, 4, dtype=torch.float64)
    a = torch.tensor([0.125], dtype=torch.float64)
    assert torch.equal(ema_ref.ema_scan(x, a), ema_ref.ema_scan(x, a.expand(4).contiguous()))


def test_clamp():
    x = torch.randn(1, 6, 3, dtype=torch.float64)
    assert torch.equal(ema_ref.ema_scan(x, torch.tensor([0.9], dtype=torch.float64)),
                       ema_ref.ema_scan(x, torch.tensor([0.5], dtype=torch.float64)))


@pytest.mark.parametrize("per_channel", [False, True])
def test_adjoint_matches_autograd(per_channel):
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2, 23, 6, generator=g, dtype=torch.float64, requires_grad=True)
    alpha = (torch.rand(6 if per_channel else 1, generator=g, dtype=torch.float64) * 0.3 + 0.1).requires_grad_(True)
    y = ema_ref.ema_scan(x, alpha)
    dy = torch.randn(y.shape, generator=g, dtype=torch.float64)
    y.backward(dy)
    dx, da = ema_ref.ema_adjoint(x.detach(), y.detach(), dy, alpha.detach())
    assert float((dx - x.grad).abs().max()) < 1e-12
    assert float((da - alpha.grad).abs().max()) < 1e-11


def test_projected_clamp_rule():
    x = torch.ones(1, 4, 1, dtype=torch.float64)
    y = ema_ref.ema_scan(x, torch.tensor([0.5], dtype=torch.float64))
    dy = torch.ones_like(y)
    # alpha at the ceiling with a negative gradient is blocked, a positive one passes
    _, da = ema_ref.ema_adjoint(x, y, -dy, torch.tensor([0.7], dtype=torch.float64))
    assert float(da) == 0.0
    _, da = ema_ref.ema_adjoint(x, y, dy, torch.tensor([0.7], dtype=torch.float64))
    assert float(da) > 0.0


def test_gradcheck_through_bounded_factor():
    ema = importlib.import_module("dwarf-v2_amd.ema")
    torch.manual_seed(1)
    x = torch.randn(2, 9, 7, dtype=torch.float64, requires_grad=True)
    raw = torch.tensor(ema.inverse_bounded_ema_factor(0.05), dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda v, p: ema_ref.ema_scan(v, ema.bounded_ema_factor(p)), (x, raw))
    assert abs(float(ema.bounded_ema_factor(raw)) - 0.05) < 1e-12
    with pytest.raises(ValueError):
        ema.inverse_bounded_ema_factor(0.6)
    with pytest.raises(ValueError):
        ema.bounded_ema_factor(raw, floor=0.5, ceiling=0.4)
