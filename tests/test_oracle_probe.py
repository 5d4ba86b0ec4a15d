"""Pin the CPU phase-probe oracle (no GPU).

The forward is a closed form on special inputs: a row equal to a * p_r for
orthonormal probes gives y_r = a / sqrt(a^2 + 1e-6 hd) and 0 on the other
planes; rows outside [start, end) are 0.  The backward restatement (the
reference kernel's formulas, dsqg:309-369) must equal autograd through the
forward expression, and the forward passes gradcheck.
"""

import math

import pytest
import torch

from oracle import probe_ref


def _orthonormal_probes(r, hd, seed):
    g = torch.Generator().manual_seed(seed)
    q, _ = torch.linalg.qr(torch.randn(hd, r, generator=g, dtype=torch.float64))
    return q.T.contiguous()   # [r, hd], orthonormal rows


def test_closed_form_on_probe_rows():
    hd, r = 64, 4
    p = _orthonormal_probes(r, hd, 0)
    a = torch.tensor([0.5, -3.0, 1e-4], dtype=torch.float64)
    x = torch.zeros(1, 1, 3 * r, hd, dtype=torch.float64)
    for i in range(3):
        for k in range(r):
            x[0, 0, i * r + k] = a[i] * p[k]
    y = probe_ref.phase_probe_features(x, p)
    for i in range(3):
        want = float(a[i]) / math.sqrt(float(a[i]) ** 2 + 1e-6 * hd)
        for k in range(r):
            row = y[0, 0, i * r + k]
            assert abs(float(row[k]) - want) < 1e-12
            assert float(row.abs().sum() - row[k].abs()) < 1e-12


def test_rows_outside_span_are_zero_and_span_is_clamped():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2, 3, 20, 64, generator=g, dtype=torch.float64)
    p = torch.randn(4, 64, generator=g, dtype=torch.float64)
    y = probe_ref.phase_probe_features(x, p, 5, 13)
    assert not y[:, :, :5].any() and not y[:, :, 13:].any()
    full = probe_ref.phase_probe_features(x, p)
    assert torch.equal(y[:, :, 5:13], full[:, :, 5:13])
    assert torch.equal(probe_ref.phase_probe_features(x, p, -4, 99), full)
    assert not probe_ref.phase_probe_features(x, p, 15, 3).any()


@pytest.mark.parametrize("span", [(0, None), (3, 17)])
def test_backward_restatement_equals_autograd(span):
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2, 2, 21, 64, generator=g, dtype=torch.float64, requires_grad=True)
    p = torch.randn(4, 64, generator=g, dtype=torch.float64, requires_grad=True)
    dout = torch.randn(2, 2, 21, 4, generator=g, dtype=torch.float64)
    y = probe_ref.phase_probe_features(x, p, *span)
    gx, gp = torch.autograd.grad(y, (x, p), dout)
    dx, dp = probe_ref.phase_probe_backward(x.detach(), p.detach(), dout, *span)
    assert float((dx - gx).abs().max()) < 1e-12
    assert float((dp - gp).abs().max()) < 1e-12


def test_gradcheck():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(1, 2, 5, 8, generator=g, dtype=torch.float64, requires_grad=True)
    p = torch.randn(4, 8, generator=g, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda a, b: probe_ref.phase_probe_features(a, b, 1, 4), (x, p))
