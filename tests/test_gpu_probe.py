"""GPU parity of the phase-probe features against the CPU oracle (runs on an MI355X).

Forward y (fp32) and dprobes within 1e-5 relative of the float64 oracle on
the same (bf16-rounded) inputs; dx within 1e-5 relative in fp32 and within
the bf16 bar (2e-2 max-abs, rows of unit scale) in bf16.  Rows outside
[start, end) are exactly 0 in y and dx.  dprobes has a fixed summation
order: two runs agree bit for bit.
"""

import pytest
import torch

from oracle import probe_ref
from tests.dsqg_cases import max_abs, rel_err

pytestmark = pytest.mark.gpu


def inputs(B, H, N, dtype, seed, transposed=False):
    g = torch.Generator().manual_seed(seed)
    if transposed:   # [B,N,H,hd] storage viewed as [B,H,N,hd]
        x = torch.randn(B, N, H, 64, generator=g).to(dtype).transpose(1, 2)
    else:
        x = torch.randn(B, H, N, 64, generator=g).to(dtype)
    p = torch.nn.functional.normalize(torch.randn(4, 64, generator=g), dim=-1)
    dout = torch.randn(B, H, N, 4, generator=g)
    return x, p, dout


def run(pkg, x, p, dout, device, span, need_probes=True):
    xd = x.to(device).requires_grad_(True)
    pd = p.to(device).requires_grad_(need_probes)
    y = pkg.phase_probe_features(xd, pd, start=span[0], end=span[1])
    y.backward(dout.to(device))
    torch.cuda.synchronize()
    return y.detach().cpu(), xd.grad.cpu(), (pd.grad.cpu() if need_probes else None)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape,span,transposed", [((2, 3, 37), (0, None), False), ((2, 3, 9), (2, 7), False),
                                                    ((1, 8, 300), (5, 290), True),
                                                    ((3, 2, 64), (64, None), False), ((2, 8, 2048), (1, None), False)])
def test_matches_oracle(pkg, device, dtype, shape, span, transposed):
    B, H, N = shape
    x, p, dout = inputs(B, H, N, dtype, seed=N + H, transposed=transposed)
    y, dx, dp = run(pkg, x, p, dout, device, span)
    s, e = max(0, min(span[0], N)), N if span[1] is None else max(0, min(span[1], N))
    ry = probe_ref.phase_probe_features(x.double(), p.double(), *span)
    rdx, rdp = probe_ref.phase_probe_backward(x.double(), p.double(), dout.double(), *span)
    assert y.dtype == torch.float32 and dx.dtype == dtype
    if e > s:
        assert rel_err(y[:, :, s:e], ry[:, :, s:e]) < 1e-5
        assert rel_err(dp, rdp) < 1e-5
        if dtype == torch.float32:
            assert rel_err(dx[:, :, s:e], rdx[:, :, s:e]) < 1e-5
        else:
            assert max_abs(dx[:, :, s:e].float(), rdx[:, :, s:e]) < 2e-2
    assert not y[:, :, :s].any() and not y[:, :, e:].any()
    assert not dx[:, :, :s].any() and not dx[:, :, e:].any()


def test_probes_without_grad_and_deterministic_dprobes(pkg, device):
    x, p, dout = inputs(2, 8, 700, torch.bfloat16, seed=3)
    y0, dx0, none = run(pkg, x, p, dout, device, (0, None), need_probes=False)
    assert none is None
    y1, dx1, dp1 = run(pkg, x, p, dout, device, (0, None))
    y2, dx2, dp2 = run(pkg, x, p, dout, device, (0, None))
    assert torch.equal(y0, y1) and torch.equal(dx0, dx1)
    assert torch.equal(dp1, dp2)


def test_empty_span_gives_zeros(pkg, device):
    x, p, dout = inputs(1, 2, 50, torch.bfloat16, seed=4)
    y, dx, dp = run(pkg, x, p, dout, device, (40, 10))
    assert not y.any() and not dx.any() and not dp.any()


def test_torch_compile_traces_without_graph_breaks(pkg, device):
    x, p, _ = inputs(2, 4, 96, torch.bfloat16, seed=5)

    def step(xx, pp):
        return (pkg.phase_probe_features(xx, pp, start=1) ** 2).sum()

    results = []
    for fn in (step, torch.compile(step, backend="aot_eager", fullgraph=True)):
        xx = x.to(device).requires_grad_(True)
        pp = p.to(device).requires_grad_(True)
        loss = fn(xx, pp)
        loss.backward()
        torch.cuda.synchronize()
        results.append((loss.detach(), xx.grad, pp.grad))
    for a, b in zip(*results):
        assert torch.equal(a, b)


def test_empty_sequence(pkg, device):
    """N = 0: empty features and dx, and dprobes exactly 0."""
    x = torch.zeros(2, 3, 0, 64, device=device, dtype=torch.bfloat16, requires_grad=True)
    p = torch.nn.functional.normalize(torch.randn(4, 64), dim=-1).to(device).requires_grad_(True)
    y = pkg.phase_probe_features(x, p)
    assert y.shape == (2, 3, 0, 4)
    y.sum().backward()
    torch.cuda.synchronize()
    assert x.grad.shape == x.shape and torch.equal(p.grad.cpu(), torch.zeros(4, 64))
