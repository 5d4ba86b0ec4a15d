"""GPU parity of the causal EMA scan against the CPU oracle (runs on an MI355X).

fp32: y, dx, dalpha within 1e-5 relative of the float64 oracle.  bf16: within
2e-2 max-abs of the oracle on the same bf16 inputs (dalpha, a sum over
B*N terms, is compared at 1e-3 relative to its magnitude).
"""

import pytest
import torch

from oracle import ema_ref
from tests.dsqg_cases import max_abs, rel_err

pytestmark = pytest.mark.gpu


def run(pkg, x, alpha, dy, device):
    xd = x.to(device).requires_grad_(True)
    ad = alpha.to(device).requires_grad_(True)
    y = pkg.causal_ema_scan(xd, ad)
    y.backward(dy.to(device=device, dtype=y.dtype))
    torch.cuda.synchronize()
    return y.detach().cpu(), xd.grad.cpu(), ad.grad.cpu()


def oracle(x, alpha, dy):
    x64, a64 = x.double(), alpha.double()
    y = ema_ref.ema_scan(x64, a64)
    y_in = ema_ref.ema_scan(x, alpha) if x.dtype != torch.float64 else y   # the stored (rounded) output
    dx, da = ema_ref.ema_adjoint(x64, y_in.double(), dy.double(), a64)
    return y, dx, da


@pytest.mark.parametrize("B,N,D,per_channel", [(2, 300, 64, False), (2, 257, 64, True), (2, 9, 7, False),
                                               (3, 130, 7, True), (1, 64, 512, True),
                                               (32, 100, 512, True), (16, 70, 512, False)])   # 64- and 32-wide carry runs
def test_fp32(pkg, device, B, N, D, per_channel):
    g = torch.Generator().manual_seed(N + D)
    x = torch.randn(B, N, D, generator=g)
    alpha = torch.rand(D if per_channel else 1, generator=g) * 0.2 + 0.01
    dy = torch.randn(B, N, D, generator=g)
    y, dx, da = run(pkg, x, alpha, dy, device)
    ry, rdx, rda = oracle(x, alpha, dy)
    assert rel_err(y, ry) < 1e-5
    assert rel_err(dx, rdx) < 1e-5
    assert rel_err(da, rda) < 1e-5


def test_bf16_long_context(pkg, device):
    """x [4,8192,512] bf16, per-channel decay ~ U(0.90, 0.999), fp32 state."""
    g = torch.Generator().manual_seed(0)
    x = torch.randn(4, 8192, 512, generator=g).to(torch.bfloat16)
    alpha = 1.0 - (0.90 + 0.099 * torch.rand(512, generator=g))
    dy = torch.randn(4, 8192, 512, generator=g).to(torch.bfloat16)
    y, dx, da = run(pkg, x, alpha, dy, device)
    assert y.dtype == torch.bfloat16
    ry = ema_ref.ema_scan(x.float(), alpha)
    assert max_abs(y, ry) < 2e-2
    rdx, rda = ema_ref.ema_adjoint(x.float(), y.float(), dy.float(), alpha)
    assert max_abs(dx, rdx) < 2e-2
    assert rel_err(da, rda) < 1e-3


@pytest.mark.parametrize("dtype", [torch.float16, torch.float64])
def test_other_dtypes_compute_in_fp32(pkg, device, dtype):
    """fp16 and fp64 inputs run the fp32 kernels and come back in their own dtype: y and dx match the
    oracle on the fp32-cast inputs to fp32 accuracy, plus the output dtype's rounding for fp16."""
    g = torch.Generator().manual_seed(11)
    x = torch.randn(2, 300, 64, generator=g).to(dtype)
    alpha = torch.rand(64, generator=g) * 0.2 + 0.01
    dy = torch.randn(2, 300, 64, generator=g).to(dtype)
    y, dx, da = run(pkg, x, alpha, dy, device)
    assert y.dtype == dtype and dx.dtype == dtype
    ry = ema_ref.ema_scan(x.double(), alpha.double())
    rdx, rda = ema_ref.ema_adjoint(x.double(), ry, dy.double(), alpha.double())
    tol = 1e-3 if dtype == torch.float16 else 1e-5
    assert rel_err(y, ry) < tol
    assert rel_err(dx, rdx) < tol
    assert rel_err(da, rda) < (1e-5 if dtype == torch.float64 else 1e-3)


def test_clamped_alpha_and_projection(pkg, device):
    x = torch.randn(1, 50, 8)
    dy = torch.ones(1, 50, 8)
    y, dx, da = run(pkg, x, torch.tensor([0.7]), dy, device)
    ry = ema_ref.ema_scan(x.double(), torch.tensor([0.5], dtype=torch.float64))
    assert rel_err(y, ry) < 1e-5
    _, rda = ema_ref.ema_adjoint(x.double(), ry, dy.double(), torch.tensor([0.7], dtype=torch.float64))
    assert (float(da) == 0.0) == (float(rda) == 0.0)


def test_torch_compile_traces_without_graph_breaks(pkg, device):
    x = torch.randn(2, 96, 64, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    raw = torch.randn(64, generator=torch.Generator().manual_seed(6))

    def step(xx, rr):
        y = pkg.causal_ema_scan(xx, pkg.bounded_ema_factor(rr))
        return (y.float() ** 2).sum()

    results = []
    for fn in (step, torch.compile(step, backend="aot_eager", fullgraph=True)):
        xx = x.to(device).requires_grad_(True)
        rr = raw.to(device).requires_grad_(True)
        loss = fn(xx, rr)
        loss.backward()
        torch.cuda.synchronize()
        results.append((loss.detach(), xx.grad, rr.grad))
    for a, b in zip(*results):
        assert torch.equal(a, b)


def test_graph_replay_matches_eager(pkg, device):
    """fwd + bwd launches captured in a HIP graph: every replay, with eager
    work and synchronisations between replays, equals the eager result bit
    for bit (the path records no memset nodes)."""
    ema = pkg.ema
    g = torch.Generator().manual_seed(3)
    B, N, D = 2, 1000, 256
    x = torch.randn(B, N, D, generator=g).to(torch.bfloat16).to(device)
    dy = torch.randn(B, N, D, generator=g).to(torch.bfloat16).to(device)
    alpha = (0.001 + 0.1 * torch.rand(D, generator=g)).to(device)

    def step():
        y = ema.ema_forward(x, alpha, 1e-5, 0.5)
        dx, da = ema.ema_backward(x, y, dy, alpha, 1e-5, 0.5, True)
        return y, dx, da

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
        other = ema.ema_forward(dy, alpha, 1e-5, 0.5)   # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for o, r in zip(outs, ref):
            assert torch.equal(o, r)
        del other


def run_reset(pkg, x, alpha, dy, reset, device):
    xd = x.to(device).requires_grad_(True)
    ad = alpha.to(device).requires_grad_(True)
    y = pkg.causal_ema_scan(xd, ad, reset_mask=reset.to(device))
    y.backward(dy.to(device=device, dtype=y.dtype))
    torch.cuda.synchronize()
    return y.detach().cpu(), xd.grad.cpu(), ad.grad.cpu()


def reset_pattern(B, N, g, kind):
    r = torch.zeros(B, N, dtype=torch.bool)
    if kind == "chunk_edges":      # at chunk starts, chunk ends, the first and last token, back to back
        # (the three-stage scan's 16-token chunks; the look-back scan's 32/64-token segments and 128/256-token tiles)
        for t in (0, 15, 16, 17, 31, 32, 33, 47, 48, 63, 64, 65, 127, 128, 129, 255, 256, 257, 511, 512, N - 1):
            if t < N:
                r[:, t] = True
    else:
        r = torch.rand(B, N, generator=g) < 0.05
    return r


@pytest.mark.parametrize("B,N,D,per_channel,kind", [(2, 300, 64, False, "random"), (2, 257, 64, True, "chunk_edges"),
                                                    (3, 130, 7, True, "random"), (2, 49, 8, False, "chunk_edges"),
                                                    (1, 1000, 512, True, "random"), (32, 100, 512, True, "random")])
def test_reset_fp32(pkg, device, B, N, D, per_channel, kind):
    """Reset-aware scan (ema:368-509) against the float64 oracle: y, dx, dalpha <= 1e-5 relative."""
    g = torch.Generator().manual_seed(N + D + 1)
    x = torch.randn(B, N, D, generator=g)
    alpha = torch.rand(D if per_channel else 1, generator=g) * 0.2 + 0.01
    dy = torch.randn(B, N, D, generator=g)
    reset = reset_pattern(B, N, g, kind)
    y, dx, da = run_reset(pkg, x, alpha, dy, reset, device)
    ry = ema_ref.ema_scan(x.double(), alpha.double(), reset_mask=reset)
    rdx, rda = ema_ref.ema_adjoint(x.double(), ry, dy.double(), alpha.double(), reset_mask=reset)
    assert rel_err(y, ry) < 1e-5
    assert rel_err(dx, rdx) < 1e-5
    assert rel_err(da, rda) < 1e-5


def test_reset_bf16_and_all_false_mask(pkg, device):
    g = torch.Generator().manual_seed(21)
    x = torch.randn(2, 3000, 512, generator=g).to(torch.bfloat16)
    alpha = 1.0 - (0.90 + 0.099 * torch.rand(512, generator=g))
    dy = torch.randn(2, 3000, 512, generator=g).to(torch.bfloat16)
    reset = torch.rand(2, 3000, generator=g) < 0.01
    y, dx, da = run_reset(pkg, x, alpha, dy, reset, device)
    ry = ema_ref.ema_scan(x.float(), alpha, reset_mask=reset)
    assert max_abs(y, ry) < 2e-2
    rdx, rda = ema_ref.ema_adjoint(x.float(), y.float(), dy.float(), alpha, reset_mask=reset)
    assert max_abs(dx, rdx) < 2e-2
    assert rel_err(da, rda) < 1e-3
    # an all-false mask runs the reset kernels and gives the plain scan's results bit for bit
    none = torch.zeros(2, 3000, dtype=torch.bool)
    assert all(torch.equal(a, b) for a, b in zip(run_reset(pkg, x, alpha, dy, none, device),
                                                 run(pkg, x, alpha, dy, device)))


@pytest.mark.parametrize("per_channel", [False, True])
def test_empty_sequence(pkg, device, per_channel):
    """x [B,0,D]: an empty scan, dx empty and dalpha exactly 0 (a sum over nothing)."""
    x = torch.zeros(2, 0, 8, device=device, dtype=torch.bfloat16, requires_grad=True)
    a = torch.full((8 if per_channel else 1,), 0.1, device=device, requires_grad=True)
    y = pkg.causal_ema_scan(x, a)
    assert y.shape == (2, 0, 8)
    y.float().sum().backward()
    torch.cuda.synchronize()
    assert x.grad.shape == (2, 0, 8) and torch.equal(a.grad.cpu(), torch.zeros(a.shape))


@pytest.mark.parametrize("B,N,D,per_channel,kind", [(2, 40000, 20, True, None), (1, 36000, 7, False, None),
                                                    (2, 36100, 12, True, "random"), (3, 17000, 64, False, "chunk_edges")])
def test_lookback_runs_fp32(pkg, device, B, N, D, per_channel, kind):
    """Sequences long enough for several runs of 32 look-back workgroups (a workgroup takes four 128-token
    tiles: N = 40000 is 313 tiles in 79 workgroups, 3 runs, the last workgroup with one tile and three
    without tokens; 17000: 2 runs), channel blocks cut by D (20, 12: one partial 64-channel block; 7: the
    one-channel lanes), with and without resets: y, dx, dalpha within 1e-5 relative of the float64 oracle."""
    g = torch.Generator().manual_seed(N + D + 7)
    x = torch.randn(B, N, D, generator=g)
    alpha = torch.rand(D if per_channel else 1, generator=g) * 0.2 + 0.01
    dy = torch.randn(B, N, D, generator=g)
    reset = None if kind is None else reset_pattern(B, N, g, kind)
    if reset is None:
        y, dx, da = run(pkg, x, alpha, dy, device)
    else:
        y, dx, da = run_reset(pkg, x, alpha, dy, reset, device)
    ry = ema_ref.ema_scan(x.double(), alpha.double(), reset_mask=reset)
    rdx, rda = ema_ref.ema_adjoint(x.double(), ry, dy.double(), alpha.double(), reset_mask=reset)
    assert rel_err(y, ry) < 1e-5
    assert rel_err(dx, rdx) < 1e-5
    assert rel_err(da, rda) < 1e-5


def test_lookback_is_deterministic(pkg, device):
    """The look-back scan forms each tile's incoming state from the published aggregates in a fixed order,
    so y, dx and dalpha are the same bits on every call, whatever order the workgroups ran in (bf16, 3 runs
    of 32 workgroups)."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 40000, 256, generator=g).to(torch.bfloat16).to(device)
    alpha = (0.01 + 0.2 * torch.rand(256, generator=g)).to(device)
    dy = torch.randn(2, 40000, 256, generator=g).to(torch.bfloat16).to(device)
    ema = pkg.ema if hasattr(pkg, "ema") else __import__("importlib").import_module("dwarf-v2_amd.ema")
    first = None
    for _ in range(4):
        y = ema.ema_forward(x, alpha, 1e-5, 0.5)
        dx, da = ema.ema_backward(x, y, dy, alpha, 1e-5, 0.5, True)
        torch.cuda.synchronize()
        if first is None:
            first = (y, dx, da)
        else:
            assert torch.equal(y, first[0]) and torch.equal(dx, first[1]) and torch.equal(da, first[2])


def test_wait_limit_gives_up_without_hanging(pkg, device):
    """A look-back wait is bounded by wait_limit polls.  Forced from the host to one poll, a workgroup whose
    predecessors have not published yet gives up and writes NaN for that channel's tiles instead of waiting;
    the call still returns, and every value that is not NaN is the value of the unbounded call."""
    import importlib

    ema = importlib.import_module("dwarf-v2_amd.ema")
    g = torch.Generator().manual_seed(6)
    x = torch.randn(4, 16384, 512, generator=g).to(torch.bfloat16).to(device)
    alpha = (0.01 + 0.2 * torch.rand(512, generator=g)).to(device)
    dy = torch.randn(4, 16384, 512, generator=g).to(torch.bfloat16).to(device)
    y_ref = ema.ema_forward(x, alpha, 1e-5, 0.5)
    dx_ref, _ = ema.ema_backward(x, y_ref, dy, alpha, 1e-5, 0.5, True)
    y = ema.ema_forward(x, alpha, 1e-5, 0.5, wait_limit=1)
    dx, _ = ema.ema_backward(x, y_ref, dy, alpha, 1e-5, 0.5, True, wait_limit=1)
    torch.cuda.synchronize()
    for got, ref in ((y, y_ref), (dx, dx_ref)):
        ok = torch.isnan(got) | (got == ref)
        assert bool(ok.all())


def test_three_stage_scan_for_slabs_over_2gib(pkg, device):
    """An x whose [N][row] slab spans more than 2 GiB (a [1, 300, 64] fp32 view of a wider buffer) is
    beyond the look-back scan's 32-bit buffer offsets, so both directions take the three-stage chunked
    scan: y, dx and dalpha within 1e-5 relative of the float64 oracle."""
    import importlib

    ema = importlib.import_module("dwarf-v2_amd.ema")
    g = torch.Generator().manual_seed(33)
    N, D = 300, 64
    x = torch.randn(1, N, D, generator=g)
    alpha = torch.rand(D, generator=g) * 0.2 + 0.01
    dy = torch.randn(1, N, D, generator=g)
    row = ((1 << 31) // (4 * N) + 8) // 4 * 4
    big = torch.zeros(1, N, row, device=device, dtype=torch.float32)
    xv = big[:, :, :D]
    xv.copy_(x.to(device))
    ad = alpha.to(device)
    y = ema.ema_forward(xv, ad, 1e-5, 0.5)
    dx, da = ema.ema_backward(xv, y, dy.to(device), ad, 1e-5, 0.5, True)
    torch.cuda.synchronize()
    ry, rdx, rda = oracle(x, alpha, dy)
    assert rel_err(y.cpu(), ry) < 1e-5
    assert rel_err(dx.cpu(), rdx) < 1e-5
    assert rel_err(da.cpu(), rda) < 1e-5
    del big


def test_reset_strided_mask(pkg, device):
    """A reset mask that is a strided view (every other column of a wider mask, and a transposed buffer):
    the kernels read it through its strides; y, dx, dalpha within 1e-5 relative of the float64 oracle."""
    g = torch.Generator().manual_seed(77)
    B, N, D = 2, 1100, 16
    x = torch.randn(B, N, D, generator=g)
    alpha = torch.rand(D, generator=g) * 0.2 + 0.01
    dy = torch.randn(B, N, D, generator=g)
    wide = reset_pattern(B, 2 * N, g, "random").to(device)
    edges = reset_pattern(B, N, g, "chunk_edges").to(device)
    for reset in (wide[:, ::2], edges.t().contiguous().t()):   # token strides 2 and B, on the device
        assert not reset.is_contiguous()
        y, dx, da = run_reset(pkg, x, alpha, dy, reset, device)
        rc = reset.cpu().contiguous()
        ry = ema_ref.ema_scan(x.double(), alpha.double(), reset_mask=rc)
        rdx, rda = ema_ref.ema_adjoint(x.double(), ry, dy.double(), alpha.double(), reset_mask=rc)
        assert rel_err(y, ry) < 1e-5
        assert rel_err(dx, rdx) < 1e-5
        assert rel_err(da, rda) < 1e-5
