"""GPU parity of the fused InterferencePacket pool against the CPU oracle (runs on an MI355X).

pooled, dx and the factor and mixture-weight gradients against
oracle/ema_ref.py's interference_pool(_backward) on the same inputs: fp32
within 1e-5 relative (pooled, dx) and 1e-4 relative (the factor and weight
gradients, sums over every element); bf16 within 2e-2 max-abs (pooled, dx)
against the oracle's bf16 rounding of each term, the factor gradients within
1e-3 and the weight gradients (returned in bf16 precision) within 1e-2
relative.  Cases: K = 1..4, D with and without 4-channel vectors, N below one
16-token chunk, not a multiple of 16, and long enough for the carry stage to
join many chunks, B*K*D wide enough for the 64- and 32-channel carry runs, a
strided x view, a factor outside [floor, ceiling];
determinism and torch.compile; and ``interference_packet_forward`` against
the same module composed of separate ``causal_ema_scan`` calls.
"""

import pytest
import torch

from oracle import ema_ref
from tests.dsqg_cases import max_abs, rel_err

pytestmark = pytest.mark.gpu

FACTORS = [1 / 16, 1 / 64, 1 / 256, 0.3]


def inputs(B, N, D, K, dtype, seed, strided=False):
    g = torch.Generator().manual_seed(seed)
    if strided:   # every other channel block of a wider projection
        x = torch.randn(B, N, 2 * D, generator=g)[:, :, :D].to(dtype)
    else:
        x = torch.randn(B, N, D, generator=g).to(dtype)
    a = torch.tensor(FACTORS[:K])
    w = torch.softmax(torch.randn(K, generator=g), 0)
    dp = torch.randn(B, N, D, generator=g).to(dtype)
    return x, a, w, dp


def run(pkg, x, a, w, dp, device):
    xd = x.to(device).requires_grad_(True)
    ad = a.to(device).requires_grad_(True)
    wd = w.to(device).requires_grad_(True)
    pooled = pkg.interference_pool(xd, ad, wd)
    pooled.backward(dp.to(device))
    torch.cuda.synchronize()
    return pooled.detach().cpu(), xd.grad.cpu(), ad.grad.cpu(), wd.grad.cpu()


def check(x, a, w, dp, got):
    pooled, dx, da, dw = got
    if x.dtype == torch.float32:
        ref = ema_ref.interference_pool(x.double(), a.double(), w.double())
        rdx, rda, rdw = ema_ref.interference_pool_backward(x.double(), a.double(), w.double(), dp.double())
        assert rel_err(pooled, ref) < 1e-5
        assert rel_err(dx, rdx) < 1e-5
        assert rel_err(da, rda) < 1e-4
        assert rel_err(dw, rdw) < 1e-4
    else:
        ref = ema_ref.interference_pool(x, a, w)
        rdx, rda, rdw = ema_ref.interference_pool_backward(x, a, w, dp)
        assert max_abs(pooled.float(), ref.float()) < 2e-2
        assert max_abs(dx.float(), rdx.float()) < 2e-2
        assert rel_err(da, rda) < 1e-3
        assert rel_err(dw, rdw) < 1e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,N,D,K,strided", [(2, 37, 64, 3, False), (1, 9, 12, 2, False), (2, 50, 6, 4, False),
                                             (1, 64, 512, 1, True), (2, 1000, 96, 3, False),
                                             (12, 150, 512, 3, False), (6, 100, 512, 3, False)])
def test_matches_oracle(pkg, device, dtype, B, N, D, K, strided):
    x, a, w, dp = inputs(B, N, D, K, dtype, seed=N + D + K, strided=strided)
    check(x, a, w, dp, run(pkg, x, a, w, dp, device))


def test_factor_outside_bounds_uses_projected_derivative(pkg, device):
    x, a, w, dp = inputs(2, 40, 16, 3, torch.float32, seed=7)
    a = a.clone()
    a[0], a[2] = 0.7, 1e-7   # above the ceiling, below the floor
    check(x, a, w, dp, run(pkg, x, a, w, dp, device))


def test_deterministic_and_compile(pkg, device):
    x, a, w, dp = inputs(2, 300, 64, 3, torch.bfloat16, seed=9)
    r1 = run(pkg, x, a, w, dp, device)
    r2 = run(pkg, x, a, w, dp, device)
    assert all(torch.equal(u, v) for u, v in zip(r1, r2))

    def step(xx, aa, ww):
        return (pkg.interference_pool(xx, aa, ww).float() ** 2).sum()

    results = []
    for fn in (step, torch.compile(step, backend="aot_eager", fullgraph=True)):
        xx = x.to(device).requires_grad_(True)
        aa = a.to(device).requires_grad_(True)
        ww = w.to(device).requires_grad_(True)
        loss = fn(xx, aa, ww)
        loss.backward()
        torch.cuda.synchronize()
        results.append((loss.detach(), xx.grad, aa.grad, ww.grad))
    for u, v in zip(*results):
        assert torch.equal(u, v)


class _Packet(torch.nn.Module):
    """The InterferencePacket's parameters and attributes (train:243-258) at a small width."""

    def __init__(self, pkg, dim=64, heads=2, timescales=(16.0, 64.0, 256.0)):
        super().__init__()
        self.heads, self.head_dim = heads, dim // heads
        raw = [pkg.inverse_bounded_ema_factor(1.0 / t) for t in timescales]
        self.ema_raw = torch.nn.Parameter(torch.tensor(raw, dtype=torch.float32))
        self.mix_logits = torch.nn.Parameter(torch.tensor([0.3, -0.2, 0.1]))
        self.gate_proj = torch.nn.Linear(dim, dim)
        self.kv_proj = torch.nn.Linear(dim, 2 * dim, bias=False)
        self._bound = pkg.bounded_ema_factor

    @property
    def ema_factors(self):
        return self._bound(self.ema_raw)


def _composed_forward(pkg, self, normalized):
    """InterferencePacket.forward as the reference writes it (train:260-284), one causal_ema_scan per
    timescale."""
    scan_input = normalized.to(torch.bfloat16)
    scans = [pkg.causal_ema_scan(scan_input, factor.reshape(1)) for factor in self.ema_factors]
    mixture = torch.softmax(self.mix_logits.float(), dim=0)
    pooled = sum(weight.to(scans[0].dtype) * scan for weight, scan in zip(mixture, scans))
    pf = pooled.float()
    rms = pf.square().mean(-1, keepdim=True).sqrt()
    direction = pf * torch.rsqrt(pf.square().mean(-1, keepdim=True) + 1e-6)
    confidence = torch.tanh(rms / 0.25)
    gate = torch.sigmoid(self.gate_proj(normalized).float())
    packet = (direction * confidence * gate).to(normalized.dtype)
    kd, vd = self.kv_proj(packet).chunk(2, dim=-1)
    B, N, _ = normalized.shape
    return (kd.reshape(B, N, self.heads, self.head_dim).permute(0, 2, 1, 3),
            vd.reshape(B, N, self.heads, self.head_dim).permute(0, 2, 1, 3))


def test_packet_forward_matches_composed_scans(pkg, device):
    torch.manual_seed(0)
    mod = _Packet(pkg).to(device)
    normalized = torch.randn(2, 200, 64, device=device)
    outs, grads = [], []
    for fwd in (lambda m, n: pkg.interference_packet_forward(m, n), lambda m, n: _composed_forward(pkg, m, n)):
        mod.zero_grad()
        nd = normalized.clone().requires_grad_(True)
        kd, vd = fwd(mod, nd)
        ((kd.float() ** 2).sum() + (vd.float() * 0.5).sum()).backward()
        torch.cuda.synchronize()
        outs.append((kd.detach().cpu(), vd.detach().cpu()))
        grads.append([nd.grad.cpu()] + [p.grad.detach().cpu().clone() for p in mod.parameters()])
    for u, v in zip(*outs):
        assert max_abs(u, v) < 2e-2
    for u, v in zip(*grads):
        assert rel_err(u, v) < 2e-2


def test_graph_replay_matches_eager(pkg, device):
    """The pool's forward and backward launches captured in a HIP graph (as bench.py times them): every
    replay, with eager work and synchronisations between replays, equals the eager result bit for bit."""
    packet = pkg.packet
    x, a, w, dp = inputs(3, 700, 512, 3, torch.bfloat16, seed=11)
    x, a, w, dp = x.to(device), a.to(device), w.to(device), dp.to(device)

    def step():
        pooled, state = packet.pool_forward(x, a, w, 1e-5, 0.5)
        return (pooled,) + packet.pool_backward(x, a, w, state, dp, 1e-5, 0.5)

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
        packet.pool_forward(dp, a, w, 1e-5, 0.5)   # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(u, v) for u, v in zip(outs, ref))


def test_empty_sequence(pkg, device):
    """x [B,0,D]: an empty pool, dx empty, and the factor and weight gradients exactly 0."""
    x = torch.zeros(2, 0, 16, device=device, dtype=torch.bfloat16, requires_grad=True)
    a = torch.tensor(FACTORS[:3], device=device, requires_grad=True)
    w = torch.full((3,), 1 / 3, device=device, requires_grad=True)
    pooled = pkg.interference_pool(x, a, w)
    assert pooled.shape == (2, 0, 16)
    pooled.float().sum().backward()
    torch.cuda.synchronize()
    assert x.grad.shape == x.shape
    assert torch.equal(a.grad.cpu(), torch.zeros(3)) and torch.equal(w.grad.cpu(), torch.zeros(3))
