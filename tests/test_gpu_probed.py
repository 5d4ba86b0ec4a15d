"""GPU parity of the op with the block's phase-probe features inside the kernels (runs on an MI355X).

``dsqg_attention_with_probes`` replaces the DSQG block's y/z einsum
(dsqg:3231-3254) and the op call after it (dsqg:3257-3284): y is formed in
the forward kernel from q, z by the phase-probe kernel from k, and dy / dz go
into dq / dk inside the backward kernels.  The oracle composes the same two
steps on the CPU: ``dsqg_ref.probe_features`` (the block's einsum, probes
normalised as the block does) then ``dsqg_ref.dsqg_forward`` (dsqg:2602-2688),
with autograd through both, in float64 on the bf16-rounded inputs and with
the GPU path's bf16 conventions (bf16 scale embeddings, delta from the bf16
output).

Bars: bf16 within 2e-2 max-abs of that oracle (out and the gradients of q,
k, v and the four tables), plus half a bf16 ulp of the oracle value for the
bf16 results (out, dq, dk, dv: a bf16 result carries its own rounding,
2^-9 |x|, which passes 2e-2 once |x| > 8); fp32 within 1e-5 relative; where
the result must not depend on the route (the probe form and the
reference-contract op on y/z from the phase-probe kernels), two bf16 ulps of
the value plus 1e-3 (the composed route rounds dq and dk to bf16 twice, the
probe form once).
"""

from __future__ import annotations

import pytest
import torch

import bench
from oracle import dsqg_ref
from tests.dsqg_cases import make_inputs, orthogonal_probes

pytestmark = pytest.mark.gpu

BF16_ABS = 2e-2
TABLES = ("pos_bias", "scale_embed", "phase_base", "phase_gain")
LEAVES = ("q", "k", "v") + TABLES


def oracle(x, qp, kp, offsets, js, shift, qs, dout, bf16, probe_grads=False, ct=torch.float64):
    """(out, grads) of the composed oracle; grads keyed by LEAVES (+ qp, kp with probe_grads)."""
    leaves = {n: x[n].to(ct).detach().clone().requires_grad_(True) for n in LEAVES}
    pq = qp.to(ct).detach().clone().requires_grad_(probe_grads)
    pk = kp.to(ct).detach().clone().requires_grad_(probe_grads)
    y = dsqg_ref.probe_features(leaves["q"], pq)
    z = dsqg_ref.probe_features(leaves["k"], pk)
    out, lse = dsqg_ref.dsqg_forward(*(leaves[n] for n in LEAVES), y, z, offsets, js, plane_shift=shift,
                                     query_start=qs, round_se=bf16, return_lse=True)
    g = dout.to(ct)
    loss = (out * g).sum()
    if bf16:   # the GPU backward's delta = <dO, bf16(O)> (see dsqg_ref.dsqg_forward_backward)
        eps = (g * (out.detach().to(torch.bfloat16).to(ct) - out.detach())).sum(-1)
        loss = loss - (eps * torch.where(torch.isfinite(lse), lse, torch.zeros_like(lse))).sum()
    loss.backward()
    grads = {n: leaves[n].grad for n in LEAVES}
    if probe_grads:
        grads["qp"], grads["kp"] = pq.grad, pk.grad
    return out.detach(), grads


def run_probed(pkg, x, qp, kp, offsets, js, shift, qs, dout, device, mode=0, online=True, probe_grads=False,
               fn=None):
    xd = {n: x[n].to(device).detach().clone().requires_grad_(True) for n in LEAVES}
    pq = qp.to(device).detach().clone().requires_grad_(probe_grads)
    pk = kp.to(device).detach().clone().requires_grad_(probe_grads)
    off = torch.tensor(offsets, dtype=torch.int32, device=device)
    op = fn or pkg.dsqg_attention_with_probes
    out = op(*(xd[n] for n in LEAVES), pq, pk, len(offsets), js, len(offsets) - js, off, None, None, None, None,
             None, 3, mode, False, 0, shift, qs, online_softmax=online)
    out.backward(dout.to(device=device, dtype=out.dtype))
    torch.cuda.synchronize()
    grads = {n: xd[n].grad for n in LEAVES}
    if probe_grads:
        grads["qp"], grads["kp"] = pq.grad, pk.grad
    return out.detach(), grads


def max_abs(a, b):
    return float((a.detach().double().cpu() - b.detach().double().cpu()).abs().max())


def excess(got, ref, name):
    """Largest |got - ref| beyond the bar (<= 0 passes): 2e-2, plus half a bf16 ulp for bf16 results."""
    g, r = got.detach().double().cpu(), ref.detach().double().cpu()
    bar = BF16_ABS + (r.abs() * 2.0 ** -9 if name in ("out", "q", "k", "v") else 0.0)
    return float(((g - r).abs() - bar).max())


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


def case(pkg, B, H, Hkv, N, offsets, js, seed, shift, dtype=torch.bfloat16, gain_std=6.0):
    x = make_inputs(B, H, Hkv, N, offsets, js, seed=seed, dtype=dtype, plane_shift=shift, gain_std=gain_std)
    qp, kp = orthogonal_probes(64, shift)
    g = torch.Generator().manual_seed(seed + 1000)
    # non-unit raw probes off the channel pairs: the op normalises them, and every dim takes part
    qp = 1.7 * qp + 0.3 * torch.randn(qp.shape, generator=g)
    kp = 0.6 * kp + 0.3 * torch.randn(kp.shape, generator=g)
    dout = torch.randn(B, H, N, 64, generator=g).to(dtype)
    return x, qp, kp, dout


@pytest.mark.parametrize("mode,online", [(0, True), (3, True), (0, False)])
def test_probed_bf16_full_lattice(pkg, device, mode, online):
    """Full 96-offset lattice, hot MOVT angles, plane shift 4, in the band schedule, the overlap-slab mode and
    the two-pass forward (the forward kernel without the band)."""
    offsets = list(pkg.ALL_OFFSETS)
    x, qp, kp, dout = case(pkg, 2, 4, 4, 320, offsets, 17, 71, 4)
    out, grads = run_probed(pkg, x, qp, kp, offsets, 17, 4, 1, dout, device, mode=mode, online=online)
    assert out.dtype == torch.bfloat16
    ro, rg = oracle(x, qp, kp, offsets, 17, 4, 1, dout, True)
    assert excess(out, ro, "out") <= 0
    for n in LEAVES:
        assert excess(grads[n], rg[n], n) <= 0, (n, max_abs(grads[n], rg[n]))


def test_probed_bf16_gqa_query_start_no_small_offsets(pkg, device):
    """Grouped K/V heads (H8 over 2), query_start 9 (rows before it: out 0 and no gradient), a ragged N, and a
    lattice without small offsets (the forward kernel without the band)."""
    for offsets, js in (([1, 2, 3, 5, 8, 13, 21, 48, 64, 96, 121], 7), ([48, 64, 96, 121, 300], 0)):
        x, qp, kp, dout = case(pkg, 2, 8, 2, 333, offsets, js, 73 + js, 2)
        out, grads = run_probed(pkg, x, qp, kp, offsets, js, 2, 9, dout, device)
        ro, rg = oracle(x, qp, kp, offsets, js, 2, 9, dout, True)
        assert torch.equal(out[:, :, :9].cpu(), torch.zeros_like(out[:, :, :9].cpu()))
        assert excess(out, ro, "out") <= 0
        for n in LEAVES:
            assert excess(grads[n], rg[n], n) <= 0, (offsets, n, max_abs(grads[n], rg[n]))
        assert torch.equal(grads["q"][:, :, :9].cpu(), torch.zeros_like(grads["q"][:, :, :9].cpu()))


def test_probed_matches_the_composed_route(pkg, device):
    """The probe form and the reference-contract op fed y/z from the phase-probe kernels compute the same
    function by different routes (y in the forward kernel vs the probe kernel; dy/dz folded in the backward
    kernels vs the probe backward): out and the gradients agree to a bf16 ulp of their values plus 1e-3."""
    offsets = list(pkg.ALL_OFFSETS)
    x, qp, kp, dout = case(pkg, 2, 4, 2, 400, offsets, 17, 75, 6)

    def composed(q, k, v, pb, se, pbase, pgain, pq, pk, *rest, **kw):
        qpn = torch.nn.functional.normalize(pq.float(), dim=-1)
        kpn = torch.nn.functional.normalize(pk.float(), dim=-1)
        y = pkg.phase_probe_features(q, qpn)
        z = pkg.phase_probe_features(k, kpn)
        return pkg.dsqg_attention_v18_grouped(q, k, v, pb, se, pbase, pgain, y, z, *rest, **kw)

    out_a, ga = run_probed(pkg, x, qp, kp, offsets, 17, 6, 1, dout, device)
    out_b, gb = run_probed(pkg, x, qp, kp, offsets, 17, 6, 1, dout, device, fn=composed)
    pairs = [("out", out_a, out_b)] + [(n, ga[n], gb[n]) for n in LEAVES]
    for n, a, b in pairs:
        a, b = a.double().cpu(), b.double().cpu()
        bar = 1e-3 + b.abs() * 2.0 ** -7
        assert bool(((a - b).abs() <= bar).all()), (n, float((a - b).abs().max()))


def test_probe_gradients_and_fp32_take_the_composed_route(pkg, device):
    """Probes that require a gradient (train_phase_probes=True) and fp32 inputs run the phase-probe kernels and
    the reference-contract op: probe gradients against the oracle (bf16: 2e-2 max-abs; fp32: 1e-5 relative,
    with every other gradient)."""
    offsets = [1, 2, 3, 5, 8, 13, 21, 48, 64, 96, 121]
    x, qp, kp, dout = case(pkg, 1, 4, 4, 200, offsets, 7, 77, 3)
    out, grads = run_probed(pkg, x, qp, kp, offsets, 7, 3, 1, dout, device, probe_grads=True)
    ro, rg = oracle(x, qp, kp, offsets, 7, 3, 1, dout, True, probe_grads=True)
    assert excess(out, ro, "out") <= 0
    for n in LEAVES + ("qp", "kp"):
        assert excess(grads[n], rg[n], n) <= 0, (n, max_abs(grads[n], rg[n]))
    x, qp, kp, dout = case(pkg, 1, 4, 2, 200, offsets, 7, 79, 3, dtype=torch.float32)
    out, grads = run_probed(pkg, x, qp, kp, offsets, 7, 3, 1, dout, device, probe_grads=True)
    assert out.dtype == torch.float32
    ro, rg = oracle(x, qp, kp, offsets, 7, 3, 1, dout, False, probe_grads=True)
    assert rel(out, ro) < 1e-5
    for n in LEAVES + ("qp", "kp"):
        assert rel(grads[n], rg[n]) < 1e-5, (n, rel(grads[n], rg[n]))


def test_probed_fullgraph_compile_equals_eager(pkg, device):
    """torch.compile(fullgraph=True) traces the probe form through its custom ops and runs the same kernels."""
    offsets = list(pkg.ALL_OFFSETS)
    x, qp, kp, dout = case(pkg, 1, 4, 2, 192, offsets, 17, 81, 3)
    off = torch.tensor(offsets, dtype=torch.int32, device=device)
    dd = dout.to(device)
    pq, pk = qp.to(device), kp.to(device)

    def step(*ts):
        out = pkg.dsqg_attention_with_probes(*ts, pq, pk, 96, 17, 79, off, None, None, None, None, None, 3, 0,
                                             False, 0, 3, 1)
        return (out.float() * dd.float()).sum()

    results = []
    for fn in (step, torch.compile(step, backend="aot_eager", fullgraph=True)):
        xd = {n: x[n].to(device).requires_grad_(True) for n in LEAVES}
        loss = fn(*(xd[n] for n in LEAVES))
        loss.backward()
        torch.cuda.synchronize()
        results.append([loss.detach()] + [xd[n].grad for n in LEAVES])
    for a, b in zip(*results):
        assert torch.equal(a, b)


def test_probed_cfg2_as_benched(pkg, device):
    """B15 H8 T2048 on bench.py's seed-0 inputs with the module's orthogonal probes (the benched probe form):
    out and the q/k/v/table gradients against the oracle per batch row (tables summed over rows)."""
    t, js, jl = bench.synth(pkg, 15, 8, 2048, 0, torch.device("cpu"))
    offsets = list(pkg.ALL_OFFSETS)
    x = {n: t[n] for n in LEAVES}
    out, grads = run_probed(pkg, x, t["qp"], t["kp"], offsets, js, 0, 1, t["dout"], device)
    sums = {n: torch.zeros_like(t[n], dtype=torch.float64) for n in TABLES}
    worst = {}
    for b in range(15):
        xb = {n: (x[n][b:b + 1] if n in ("q", "k", "v") else x[n]) for n in LEAVES}
        ro, rg = oracle(xb, t["qp"], t["kp"], offsets, js, 0, 1, t["dout"][b:b + 1], True, ct=torch.float32)
        for n, got, ref in [("out", out[b:b + 1], ro)] + [(n, grads[n][b:b + 1], rg[n]) for n in ("q", "k", "v")]:
            worst[n] = max(worst.get(n, 0.0), max_abs(got, ref))
            assert excess(got, ref, n) <= 0, (n, b, max_abs(got, ref))
        for n in TABLES:
            sums[n] += rg[n]
        print(f"[probed] row {b} of 15 checked", flush=True)
    for n in TABLES:
        worst[n] = max_abs(grads[n], sums[n])
        assert worst[n] < BF16_ABS, (n, worst[n])
    print("[probed] largest |gpu - oracle| (bar 2e-2): " + ", ".join(f"{n} {v:.2e}" for n, v in worst.items()),
          flush=True)
