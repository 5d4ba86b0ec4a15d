"""GPU parity of the fused InterferencePacket pool against the CPU oracle (runs on an MI355X).

pooled, dx and the factor and mixture-weight gradients against
oracle/ema_ref.py's interference_pool(_backward) on the same inputs: fp32
within 1e-5 relative (pooled, dx, and the factor and weight gradients, sums
over every element); bf16 within 2e-2 max-abs (pooled, dx)
against the oracle's bf16 rounding of each term, the factor gradients within
1e-3 and the weight gradients (returned in bf16 precision) within 1e-2
relative.  Cases: K = 1..4, D with and without 4-channel vectors, N below one
16-token chunk, not a multiple of 16, and long enough for the carry stage to
join many chunks and for the look-back scans to span two runs of workgroup
tiles (17,000 tokens), B*K*D wide enough for the 64- and 32-channel carry runs, a
strided x view, a factor outside [floor, ceiling];
determinism and torch.compile; and ``interference_packet_forward`` against
the same module composed of separate ``causal_ema_scan`` calls.

The packet (``interference_packet``, train:262-273): the packet against
oracle/ema_ref.py's packet_from_pooled of the kernel's own pooled values
(fp32 within 1e-5 relative; bf16 within one bf16 ulp (2^-7 |value|) plus 1e-6,
the cast's own rounding on both sides), pooled against the pool oracle as
above; the gradients against autograd through packet_from_pooled (dgate:
fp32 1e-5 relative, bf16 the same one-ulp bar; dpooled as autograd rounds it to
the pool dtype) followed by interference_pool_backward, at the pool's bars.
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
        assert rel_err(da, rda) < 1e-5
        assert rel_err(dw, rdw) < 1e-5
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
                                             (12, 150, 512, 3, False), (6, 100, 512, 3, False),
                                             (1, 2100, 64, 3, True), (1, 17000, 64, 3, False),
                                             (2, 700, 128, 4, False)])
def test_matches_oracle(pkg, device, dtype, B, N, D, K, strided):
    x, a, w, dp = inputs(B, N, D, K, dtype, seed=N + D + K, strided=strided)
    check(x, a, w, dp, run(pkg, x, a, w, dp, device))


def test_factor_outside_bounds_uses_projected_derivative(pkg, device):
    x, a, w, dp = inputs(2, 40, 16, 3, torch.float32, seed=7)
    a = a.clone()
    a[0], a[2] = 0.7, 1e-7   # above the ceiling, below the floor
    check(x, a, w, dp, run(pkg, x, a, w, dp, device))


def test_deterministic_and_compile(pkg, device):
    # 17,000 tokens: 34 workgroup tiles of the look-back scans per channel block, in two runs
    xl, al, wl, dpl = inputs(2, 17000, 128, 3, torch.bfloat16, seed=10)
    r1 = run(pkg, xl, al, wl, dpl, device)
    r2 = run(pkg, xl, al, wl, dpl, device)
    assert all(torch.equal(u, v) for u, v in zip(r1, r2))
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


def packet_inputs(B, N, D, K, dtype, gdtype, seed):
    x, a, w, dp = inputs(B, N, D, K, dtype, seed)
    g = torch.Generator().manual_seed(seed + 1)
    gate = (1.5 * torch.randn(B, N, D, generator=g)).to(gdtype)
    dpk = torch.randn(B, N, D, generator=g).to(gdtype)
    return x, a, w, gate, dpk


def packet_oracle(x, a, w, gate, pooled, dpk):
    """(packet from the kernel's pooled, dx, dalpha, dweight, dgate): autograd through packet_from_pooled
    (fp64 for fp32 tensors), then interference_pool_backward on the pooled gradient autograd forms."""
    wide = x.dtype == torch.float32
    u = (pooled.double() if wide else pooled).clone().requires_grad_(True)
    gl = (gate.double() if gate.dtype == torch.float32 else gate).clone().requires_grad_(True)
    out = ema_ref.packet_from_pooled(u, gl, gl.dtype)
    out.backward(dpk.to(out.dtype))
    xs, av, wv = (x.double(), a.double(), w.double()) if wide else (x, a, w)
    rdx, rda, rdw = ema_ref.interference_pool_backward(xs, av, wv, u.grad)
    return out.detach(), rdx, rda, rdw, gl.grad


def bf16_close(got, ref, floor=1e-6, rel=2.0 ** -7):
    g, r = got.double(), ref.double()
    return float(((g - r).abs() - (floor + rel * r.abs())).max()) <= 0


@pytest.mark.parametrize("dtype,gdtype", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                                          (torch.bfloat16, torch.float32)])
@pytest.mark.parametrize("B,N,D,K", [(2, 37, 64, 3), (1, 9, 12, 2), (2, 300, 512, 3), (1, 50, 1000, 4),
                                     (1, 20, 4096, 1)])
def test_packet_matches_oracle(pkg, device, dtype, gdtype, B, N, D, K):
    x, a, w, gate, dpk = packet_inputs(B, N, D, K, dtype, gdtype, seed=N + D + K)
    packet_mod = pkg.packet
    xd, ad, wd, gd = x.to(device), a.to(device), w.to(device), gate.to(device)
    pk, pooled, state, ms = packet_mod.packet_forward(xd, ad, wd, gd, 1e-5, 0.5)
    dx, da, dw, dg = packet_mod.packet_backward(xd, ad, wd, gd, pooled, state, ms, dpk.to(device), 1e-5, 0.5)
    torch.cuda.synchronize()
    pk, pooled, ms, dx, da, dw, dg = (t.cpu() for t in (pk, pooled, ms, dx, da, dw, dg))
    assert pk.dtype == gdtype and dg.dtype == gdtype and pooled.dtype == dtype
    wide = dtype == torch.float32
    ref_pool = ema_ref.interference_pool(*((x.double(), a.double(), w.double()) if wide else (x, a, w)))
    rpk, rdx, rda, rdw, rdg = packet_oracle(x, a, w, gate, pooled, dpk)
    assert torch.allclose(ms.double(), pooled.double().square().mean(-1), rtol=1e-5, atol=1e-12)
    if dtype == torch.float32:
        assert rel_err(pooled, ref_pool) < 1e-5
        assert rel_err(pk, rpk) < 1e-5
        assert rel_err(dg, rdg) < 1e-5
        assert rel_err(dx, rdx) < 1e-5
        assert rel_err(da, rda) < 1e-5
        assert rel_err(dw, rdw) < 1e-5
    else:
        assert max_abs(pooled.float(), ref_pool.float()) < 2e-2
        if gdtype == torch.float32:
            assert rel_err(pk, rpk) < 1e-5
            assert rel_err(dg, rdg) < 1e-5
        else:
            assert bf16_close(pk, rpk)
            assert bf16_close(dg, rdg)
        assert max_abs(dx.float(), rdx.float()) < 2e-2
        assert rel_err(da, rda) < 1e-3
        assert rel_err(dw, rdw) < 1e-2


def test_packet_deterministic_compile_and_graph(pkg, device):
    """interference_packet twice bit-equal, under torch.compile (fullgraph) bit-equal to eager, and its raw
    forward + backward launches replayed from a HIP graph equal to eager on every replay."""
    x, a, w, gate, dpk = packet_inputs(2, 300, 512, 3, torch.bfloat16, torch.bfloat16, seed=21)
    x, a, w, gate, dpk = (t.to(device) for t in (x, a, w, gate, dpk))

    def step(xx, aa, ww, gg):
        return (pkg.interference_packet(xx, aa, ww, gg).float() * dpk.float()).sum()

    results = []
    for fn in (step, step, torch.compile(step, backend="aot_eager", fullgraph=True)):
        leaves = [t.clone().requires_grad_(True) for t in (x, a, w, gate)]
        loss = fn(*leaves)
        loss.backward()
        torch.cuda.synchronize()
        results.append([loss.detach()] + [t.grad for t in leaves])
    for other in results[1:]:
        assert all(torch.equal(u, v) for u, v in zip(results[0], other))

    packet = pkg.packet

    def launches():
        pk, pooled, state, ms = packet.packet_forward(x, a, w, gate, 1e-5, 0.5)
        return (pk, pooled, ms) + packet.packet_backward(x, a, w, gate, pooled, state, ms, dpk, 1e-5, 0.5)

    ref = [t.clone() for t in launches()]
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        launches()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = launches()
    for _ in range(3):
        packet.packet_forward(dpk, a, w, gate, 1e-5, 0.5)   # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(u, v) for u, v in zip(outs, ref))



def _wide_view(B, N, D, like):
    """A [B, N, D] fp32 view of a wider device buffer whose [N][row] slab spans more than 2 GiB, holding
    like's values: the kernels' 32-bit buffer offsets cannot reach it, so the forward takes its three-stage
    path (local, carry, apply) instead of the look-back pass."""
    row = ((1 << 31) // (4 * N) + 8) // 4 * 4
    big = torch.zeros(B, N, row, device=like.device, dtype=torch.float32)
    v = big[:, :, :D]
    v.copy_(like)
    return big, v


def test_three_stage_forward_for_slabs_over_2gib(pkg, device):
    """Slabs past 2 GiB take the three-stage forward: pooled, dx and the factor and weight gradients
    within 1e-5 relative of the float64 oracle, and pooled and the chunk states (what the backward
    reads) within 1e-6 relative of the look-back pass on the same values in a contiguous tensor."""
    import importlib

    packet = importlib.import_module("dwarf-v2_amd.packet")
    B, N, D, K = 1, 300, 64, 3
    x, a, w, dp = inputs(B, N, D, K, torch.float32, seed=31)
    xd = x.to(device)
    big, xv = _wide_view(B, N, D, xd)
    pooled, state = packet.pool_forward(xv, a, w, 1e-5, 0.5)
    dx, da, dw = packet.pool_backward(xv, a, w, state, dp.to(device), 1e-5, 0.5)
    torch.cuda.synchronize()
    check(x, a, w, dp, (pooled.cpu(), dx.cpu(), da.cpu(), dw.cpu()))
    pooled_lb, state_lb = packet.pool_forward(xd, a, w, 1e-5, 0.5)
    torch.cuda.synchronize()
    assert rel_err(pooled.cpu(), pooled_lb.cpu()) < 1e-6
    assert rel_err(state.cpu(), state_lb.cpu()) < 1e-6
    del big


def test_packet_three_stage_for_slabs_over_2gib(pkg, device):
    """x past 2 GiB per slab: the packet's forward takes the three-stage chunk states and the row kernel
    that rescans each chunk, its backward the three-stage pool backward. The packet and every gradient
    against the oracle at the fp32 bars, and the packet, pooled and ms within 1e-6 relative of the
    look-back forward on the same values in a contiguous tensor."""
    packet_mod = pkg.packet
    B, N, D, K = 1, 300, 64, 3
    x, a, w, gate, dpk = packet_inputs(B, N, D, K, torch.float32, torch.float32, seed=41)
    xd, ad, wd, gd = x.to(device), a.to(device), w.to(device), gate.to(device)
    big, xv = _wide_view(B, N, D, xd)
    pk, pooled, state, ms = packet_mod.packet_forward(xv, ad, wd, gd, 1e-5, 0.5)
    dx, da, dw, dg = packet_mod.packet_backward(xv, ad, wd, gd, pooled, state, ms, dpk.to(device), 1e-5, 0.5)
    pk_lb, pooled_lb, _, ms_lb = packet_mod.packet_forward(xd, ad, wd, gd, 1e-5, 0.5)
    torch.cuda.synchronize()
    pk, pooled, ms, dx, da, dw, dg = (t.cpu() for t in (pk, pooled, ms, dx, da, dw, dg))
    rpk, rdx, rda, rdw, rdg = packet_oracle(x, a, w, gate, pooled, dpk)
    assert rel_err(pooled, ema_ref.interference_pool(x.double(), a.double(), w.double())) < 1e-5
    for got, ref in ((pk, rpk), (dg, rdg), (dx, rdx), (da, rda), (dw, rdw)):
        assert rel_err(got, ref) < 1e-5
    for got, ref in ((pk, pk_lb), (pooled, pooled_lb), (ms, ms_lb)):
        assert rel_err(got, ref.cpu()) < 1e-6
    del big
