"""Pin the CPU restatement of the InterferencePacket pool (no GPU).

pooled = sum_k w_k EMA(x, a_k) (train/train_dwarf.py:262-267) is a causal
convolution of x with h[tau] = sum_k w_k a_k (1 - a_k)^tau: the float64
restatement equals that convolution evaluated directly.  Its restated
backward equals autograd of the forward (float64) and passes gradcheck; a
factor outside [floor, ceiling] gets the projected-clamp derivative of its
own scan (ema:357-364).  In bf16 every term is rounded, and the result stays
within the bf16 bar of the exact value.
"""

import pytest
import torch

from oracle import ema_ref


def _inputs(seed, B=2, N=37, D=6, K=3, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, N, D, generator=g, dtype=torch.float64).to(dtype)
    a = torch.tensor([1 / 16, 1 / 64, 1 / 256, 0.3][:K], dtype=torch.float64)
    w = torch.softmax(torch.randn(K, generator=g, dtype=torch.float64), 0)
    return x, a, w


@pytest.mark.parametrize("K", [1, 3, 4])
def test_pool_equals_direct_convolution(K):
    x, a, w = _inputs(0, K=K)
    N = x.shape[1]
    tau = torch.arange(N, dtype=torch.float64)
    h = (w[:, None] * a[:, None] * (1 - a[:, None]) ** tau[None, :]).sum(0)   # [tau]
    lag = torch.arange(N)[:, None] - torch.arange(N)[None, :]                 # t - s
    kern = torch.where(lag >= 0, h[lag.clamp(min=0)], torch.zeros((), dtype=torch.float64))
    direct = torch.einsum("ts,bsd->btd", kern, x)
    pooled = ema_ref.interference_pool(x, a, w)
    assert float((pooled - direct).abs().max()) < 1e-12


@pytest.mark.parametrize("seed", [1, 2])
def test_backward_restatement_equals_autograd(seed):
    x, a, w = _inputs(seed)
    g = torch.randn(x.shape, generator=torch.Generator().manual_seed(seed + 10), dtype=torch.float64)
    xr, ar, wr = x.clone().requires_grad_(True), a.clone().requires_grad_(True), w.clone().requires_grad_(True)
    ema_ref.interference_pool(xr, ar, wr).backward(g)
    dx, da, dw = ema_ref.interference_pool_backward(x, a, w, g)
    assert float((dx - xr.grad).abs().max()) < 1e-12
    assert float((da - ar.grad).abs().max()) < 1e-10
    assert float((dw - wr.grad).abs().max()) < 1e-10


def test_gradcheck():
    x, a, w = _inputs(3, B=1, N=9, D=2)
    ok = torch.autograd.gradcheck(lambda xx, aa, ww: ema_ref.interference_pool(xx, aa, ww),
                                  (x.requires_grad_(True), a.requires_grad_(True), w.requires_grad_(True)))
    assert ok


def test_clamped_factor_takes_the_projected_derivative():
    x, a, w = _inputs(4)
    a = a.clone()
    a[1] = 0.7   # above the ceiling: clamped to 0.5 in the scan
    g = torch.randn(x.shape, generator=torch.Generator().manual_seed(5), dtype=torch.float64)
    _, da, _ = ema_ref.interference_pool_backward(x, a, w, g)
    scan = ema_ref.ema_scan(x, a[1].reshape(1))
    _, da1 = ema_ref.ema_adjoint(x, scan, g * w[1], a[1].reshape(1))
    assert float(da[1]) == float(da1[0])
    # above the ceiling only a positive adjoint sum (pointing back inside) survives
    assert float(da[1]) >= 0.0


def test_bf16_terms_are_rounded_and_stay_close():
    x, a, w = _inputs(6, dtype=torch.bfloat16)
    pooled = ema_ref.interference_pool(x, a, w)
    assert pooled.dtype == torch.bfloat16
    exact = ema_ref.interference_pool(x.double(), a, w)
    assert float((pooled.double() - exact).abs().max()) < 2e-2
    # the first term alone is w_0 (in bf16) times the bf16 scan, rounded to bf16
    s0 = ema_ref.ema_scan(x, a[0].reshape(1))
    one = ema_ref.interference_pool(x, a[:1], w[:1])
    assert torch.equal(one, w[0].to(torch.bfloat16) * s0)
