"""GPU parity of the NPCI rotation against the CPU oracle (runs on an MI355X).

Forward and all three gradients (x, delta, theta) against the float64 oracle
(oracle/npci_ref.py, pinned to autograd): fp32 within 1e-5 relative (forward
and gradients); bf16 within 2e-2 max-abs.  Rows with a zero x,
a zero delta or a delta parallel to x take the reference's special paths (the
parallel row is exact in fp32: a delta that is parallel only up to rounding
sits on the 1e-7 activity threshold in any fp32 evaluation, the reference's
included).
dtheta has a fixed summation order: two runs agree bit for bit.  The shapes
cover B*T per head not a multiple of 4 (the reduction's single-entry path),
a multiple of 4 (16-byte vectors) and 32,800 entries (eight vectors in flight).
"""

import pytest
import torch

from oracle import npci_ref
from tests.dsqg_cases import max_abs, rel_err

pytestmark = pytest.mark.gpu


def inputs(B, H, T, xdt, ddt, seed, permuted=False):
    g = torch.Generator().manual_seed(seed)
    if permuted:   # a [B,T,H*hd] projection viewed as [B,H,T,hd] (dsqg:3191-3193)
        x = torch.randn(B, T, H * 64, generator=g).to(xdt).reshape(B, T, H, 64).permute(0, 2, 1, 3)
    else:
        x = torch.randn(B, H, T, 64, generator=g).to(xdt)
    d = (0.3 * torch.randn(B, H, T, 64, generator=g)).to(ddt)
    th = 0.25 * torch.tanh(torch.randn(H, generator=g))
    gr = torch.randn(B, H, T, 64, generator=g)
    if T > 5:
        x[0, 0, 1] = 0.0            # zero row: clamped norm
        d[0, 0, 2] = 0.0            # zero delta: identity
        x[0, 0, 3] = 0.0            # a delta parallel to x (exactly, so fp32 agrees): inactive
        x[0, 0, 3, 5] = 1.5
        d[0, 0, 3] = 0.0
        d[0, 0, 3, 5] = -4.0
    return x, d, th, gr


def run(pkg, x, d, th, gr, device, tau):
    xd = x.to(device).requires_grad_(True)
    dd = d.to(device).requires_grad_(True)
    td = th.to(device).requires_grad_(True)
    out = pkg.npci_rotate(xd, dd, td, strength_tau=tau)
    out.backward(gr.to(device=device, dtype=out.dtype))
    torch.cuda.synchronize()
    return out.detach().cpu(), xd.grad.cpu(), dd.grad.cpu(), td.grad.cpu()


@pytest.mark.parametrize("xdt,ddt", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                                     (torch.bfloat16, torch.float32), (torch.float32, torch.bfloat16)])
@pytest.mark.parametrize("shape,permuted", [((2, 3, 37), False), ((2, 3, 9), False), ((1, 8, 300), True),
                                            ((2, 2, 16400), False)])
def test_matches_oracle(pkg, device, xdt, ddt, shape, permuted):
    B, H, T = shape
    x, d, th, gr = inputs(B, H, T, xdt, ddt, seed=T + H, permuted=permuted)
    tau = 0.25
    out, dx, dd, dt = run(pkg, x, d, th, gr, device, tau)
    assert out.dtype == xdt and dx.dtype == xdt and dd.dtype == ddt
    g_used = gr.to(xdt).double()   # the gradient as it reaches the kernel (x's dtype)
    ro = npci_ref.npci_rotate(x.double(), d.double(), th.double(), tau)
    rdx, rdd, rdt = npci_ref.npci_rotate_backward(x.double(), d.double(), th.double(), g_used, tau)
    if xdt == torch.float32:
        assert rel_err(out, ro) < 1e-5
        assert rel_err(dx, rdx) < 1e-5
    else:
        assert max_abs(out, ro) < 2e-2
        assert max_abs(dx, rdx) < 2e-2
    if ddt == torch.float32 and xdt == torch.float32:
        assert rel_err(dd, rdd) < 1e-5
    else:
        assert max_abs(dd, rdd) < 2e-2
    assert rel_err(dt, rdt) < 1e-5
    if T > 5:   # the zero-delta row is returned exactly
        assert torch.equal(out[0, 0, 2], x[0, 0, 2])


def test_dtheta_deterministic_and_compile(pkg, device):
    x, d, th, gr = inputs(2, 8, 500, torch.bfloat16, torch.bfloat16, seed=3)
    a = run(pkg, x, d, th, gr, device, 0.25)
    b = run(pkg, x, d, th, gr, device, 0.25)
    assert all(torch.equal(u, v) for u, v in zip(a, b))

    def step(xx, dd, tt):
        return (pkg.npci_rotate(xx, dd, tt).float() ** 2).sum()

    results = []
    for fn in (step, torch.compile(step, backend="aot_eager", fullgraph=True)):
        xx = x.to(device).requires_grad_(True)
        dd = d.to(device).requires_grad_(True)
        tt = th.to(device).requires_grad_(True)
        loss = fn(xx, dd, tt)
        loss.backward()
        torch.cuda.synchronize()
        results.append((loss.detach(), xx.grad, dd.grad, tt.grad))
    for u, v in zip(*results):
        assert torch.equal(u, v)


def test_graph_replay_matches_eager(pkg, device):
    """Forward and backward launches captured in a HIP graph (as bench.py times them): every replay, with
    eager work and synchronisations between replays, equals the eager result bit for bit."""
    npci = pkg.npci
    x, d, th, gr = inputs(2, 8, 700, torch.bfloat16, torch.bfloat16, seed=12, permuted=True)
    x, d, th, gr = x.to(device), d.to(device), th.to(device), gr.to(device=device, dtype=torch.bfloat16)

    def step():
        return (npci.npci_forward(x, d, th, 0.25),) + npci.npci_backward(x, d, th, gr, 0.25)

    ref = [t.clone() for t in step()]
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step()
    for _ in range(3):
        npci.npci_forward(d, x, th, 0.25)   # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(u, v) for u, v in zip(outs, ref))


def test_empty_rows(pkg, device):
    """T = 0: an empty rotation, empty dx and ddelta, and dtheta exactly 0."""
    x = torch.zeros(2, 3, 0, 64, device=device, dtype=torch.bfloat16, requires_grad=True)
    d = torch.zeros(2, 3, 0, 64, device=device, dtype=torch.bfloat16, requires_grad=True)
    th = torch.full((3,), 0.1, device=device, requires_grad=True)
    out = pkg.npci_rotate(x, d, th)
    assert out.shape == (2, 3, 0, 64) and out.dtype == torch.bfloat16
    out.float().sum().backward()
    torch.cuda.synchronize()
    assert x.grad.shape == x.shape and d.grad.shape == d.shape
    assert torch.equal(th.grad.cpu(), torch.zeros(3))
