"""Pin the CPU EMA oracle (no GPU): closed form, reverse adjoint, gradcheck.

The recurrence y[t] = a x[t] + (1-a) y[t-1] (kernels/causal_ema_scan.py:3-11)
has the closed form y[t] = sum_{s<=t} a (1-a)^(t-s) x[s]; the adjoint of
ema:7-11 must equal autograd through the recurrence.
"""

import importlib
import math

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


def test_reset_scan_is_independent_segments():
    """With resets the scan restarts: each segment between resets equals the
    closed form over that segment alone."""
    g = torch.Generator().manual_seed(11)
    x = torch.randn(2, 40, 3, generator=g, dtype=torch.float64)
    alpha = torch.tensor([0.2, 0.05, 0.4], dtype=torch.float64)
    reset = torch.zeros(2, 40, dtype=torch.bool)
    reset[0, [0, 7, 8, 31]] = True
    reset[1, [39]] = True
    y = ema_ref.ema_scan(x, alpha, reset_mask=reset)
    for b in range(2):
        cuts = [0] + [t for t in range(1, 40) if reset[b, t]] + [40]
        for s0, s1 in zip(cuts[:-1], cuts[1:]):
            want = ema_ref.ema_closed_form(x[b:b + 1, s0:s1], alpha)
            assert float((y[b:b + 1, s0:s1] - want).abs().max()) < 1e-13
    assert torch.equal(ema_ref.ema_scan(x, alpha, reset_mask=torch.zeros(2, 40, dtype=torch.bool)),
                       ema_ref.ema_scan(x, alpha))


@pytest.mark.parametrize("per_channel", [False, True])
def test_reset_adjoint_equals_autograd(per_channel):
    g = torch.Generator().manual_seed(12)
    x = torch.randn(2, 23, 4, generator=g, dtype=torch.float64, requires_grad=True)
    alpha = (torch.rand(4 if per_channel else 1, generator=g, dtype=torch.float64) * 0.3 + 0.05).requires_grad_(True)
    reset = torch.rand(2, 23, generator=g) < 0.2
    reset[:, 22] = True
    dy = torch.randn(2, 23, 4, generator=g, dtype=torch.float64)
    y = ema_ref.ema_scan(x, alpha, reset_mask=reset)
    gx, ga = torch.autograd.grad(y, (x, alpha), dy)
    dx, da = ema_ref.ema_adjoint(x.detach(), y.detach(), dy, alpha.detach(), reset_mask=reset)
    assert float((dx - gx).abs().max()) < 1e-12
    assert float((da - ga).abs().max()) < 1e-11


def test_packet_known_answers():
    """Rows with closed-form packets (train:268-273): a constant row c gives rms |c|, direction
    c / sqrt(c^2 + 1e-6) and confidence tanh(|c| / 0.25); tanh(1) and sigmoid(0) = 1/2, sigmoid(ln 3) = 3/4
    are textbook values."""
    D = 64
    tanh1 = 0.7615941559557649
    u = torch.full((1, 3, D), 0.25, dtype=torch.float64)
    u[0, 1] = -0.25
    u[0, 2, : D // 2], u[0, 2, D // 2:] = 0.5, -0.5           # rms 0.5: tanh(2)
    logits = torch.zeros(1, 3, D, dtype=torch.float64)
    logits[0, 1] = math.log(3.0)
    got = ema_ref.packet_from_pooled(u, logits, torch.float64)
    d = 0.25 / math.sqrt(0.0625 + 1e-6)
    assert torch.allclose(got[0, 0], torch.full((D,), d * tanh1 * 0.5, dtype=torch.float64), rtol=1e-15)
    assert torch.allclose(got[0, 1], torch.full((D,), -d * tanh1 * 0.75, dtype=torch.float64), rtol=1e-15)
    d2 = 0.5 / math.sqrt(0.25 + 1e-6)
    want = torch.tensor([d2] * (D // 2) + [-d2] * (D // 2), dtype=torch.float64) * math.tanh(2.0) * 0.5
    assert torch.allclose(got[0, 2], want, rtol=1e-15)


def test_packet_direction_has_unit_rms_and_gradcheck():
    g = torch.Generator().manual_seed(3)
    u = torch.randn(2, 5, 16, generator=g, dtype=torch.float64)
    logits = torch.randn(2, 5, 16, generator=g, dtype=torch.float64)
    big = torch.full_like(logits, 60.0)                         # sigmoid -> 1
    p = ema_ref.packet_from_pooled(u, big, torch.float64)
    ms = u.square().mean(-1, keepdim=True)
    conf = torch.tanh(ms.sqrt() / 0.25)
    assert torch.allclose((p / conf).square().mean(-1, keepdim=True), ms / (ms + 1e-6), rtol=1e-12)
    u.requires_grad_(True)
    logits.requires_grad_(True)
    assert torch.autograd.gradcheck(lambda a, b: ema_ref.packet_from_pooled(a, b, torch.float64), (u, logits))
