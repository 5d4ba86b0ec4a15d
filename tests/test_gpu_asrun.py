"""GPU parity at the sizes bench.py times, on the data it times (runs on an MI355X).

The kernels' persistent launches walk several tiles per workgroup only at
these sizes (cfg2 has 3,840 query tiles against 768 dQ and 1,024 dSE
workgroups), so the tile walk, the per-head table reuse across tiles and the
register-carried dSE partials are checked here against the oracle rather than
at test sizes.  The oracle (oracle/dsqg_ref.py, the restatement of
dsqg:2602-2688 with the GPU path's conventions) runs in fp32 on the host one
batch row at a time; per-row outputs and dq/dk/dv/dy/dz are compared row by
row, and dpos_bias / dscale_embed / dphase against the oracle's sum over all
rows.

Bar: bf16 results within 2e-2 max-abs of the oracle, added to half a bf16 ulp
of the oracle value for the bf16 outputs (out, dq, dk, dv): a bf16 result
carries its own rounding, half an ulp of its value, whatever the kernel does
(2^-9 |x|, which passes 2e-2 once |x| > 8).  fp32 outputs (dy, dz and the
parameter gradients) take the plain 2e-2.
"""

from __future__ import annotations

import importlib
import sys

import numpy as np
import pytest
import torch

import bench
from oracle import dsqg_ref, q6_ref
from tests.dsqg_cases import NAMES, features, make_inputs

pytestmark = pytest.mark.gpu

BF16_ABS = 2e-2
PARAMS = ("pos_bias", "scale_embed", "phase_base", "phase_gain")
BF16_OUT = ("q", "k", "v")


def note(msg: str) -> None:
    print(f"[asrun] {msg}", file=sys.stderr, flush=True)


MAX_ERR: dict = {}   # largest plain |got - ref| per result name over a test (the ulp term left out)


def excess(got: torch.Tensor, ref: torch.Tensor, bf16: bool, name: str | None = None) -> float:
    """Largest |got - ref| beyond the bar (<= 0 passes); with ``name``, also records the largest plain
    |got - ref| in MAX_ERR."""
    g = got.detach().double().cpu()
    r = ref.detach().double().cpu()
    err = (g - r).abs()
    if name is not None:
        MAX_ERR[name] = max(MAX_ERR.get(name, 0.0), float(err.max()))
    bar = BF16_ABS + (r.abs() * 2.0 ** -9 if bf16 else 0.0)
    return float((err - bar).max())


def run_gpu(pkg, t, offsets, js, shift, qs, device, mode=0):
    xd = {n: t[n].to(device).detach().clone().requires_grad_(True) for n in NAMES}
    off = torch.tensor(offsets, dtype=torch.int32, device=device)
    out = pkg.dsqg_attention_v18_grouped(*(xd[n] for n in NAMES), len(offsets), js, len(offsets) - js, off,
                                         None, None, None, None, None, 3, mode, False, 0, shift, qs)
    out.backward(t["dout"].to(device=device, dtype=out.dtype))
    torch.cuda.synchronize()
    return out.detach().cpu(), {n: xd[n].grad.cpu() for n in NAMES}


def check_rows(pkg, t, offsets, js, shift, qs, device, head_chunk=None, mode=0):
    """GPU fwd+bwd on the whole batch, oracle per batch row (and head chunk): returns nothing, asserts."""
    out, grads = run_gpu(pkg, t, offsets, js, shift, qs, device, mode)
    MAX_ERR.clear()
    cpu = {n: t[n].detach().cpu() for n in list(NAMES) + ["dout"]}
    B, H, N, _ = cpu["q"].shape
    Hkv = cpu["k"].shape[1]
    grp = H // Hkv
    chunk = head_chunk or H
    assert chunk % grp == 0
    sums = {n: torch.zeros_like(cpu[n], dtype=torch.float64) for n in PARAMS}
    worst = {}
    for b in range(B):
        for h0 in range(0, H, chunk):
            hs, ks = slice(h0, h0 + chunk), slice(h0 // grp, (h0 + chunk) // grp)
            sl = {n: cpu[n][b:b + 1, hs] for n in ("q", "y_pre", "dout")}
            sl.update({n: cpu[n][b:b + 1, ks] for n in ("k", "v", "z_pre")})
            sl["pos_bias"] = cpu["pos_bias"][:, hs]
            sl["scale_embed"] = cpu["scale_embed"]
            sl["phase_base"] = cpu["phase_base"][:, hs]
            sl["phase_gain"] = cpu["phase_gain"][:, hs]
            inp = {n: sl[n].float() for n in NAMES}
            ro, _, rg = dsqg_ref.dsqg_forward_backward(inp, offsets, js, sl["dout"].float(), plane_shift=shift,
                                                       query_start=qs, round_se=True, delta_from_bf16_out=True)
            e = excess(out[b:b + 1, hs], ro, True, "out")
            worst["out"] = max(worst.get("out", -1.0), e)
            assert e <= 0, ("out", b, h0, e)
            for n, got in (("q", grads["q"][b:b + 1, hs]), ("y_pre", grads["y_pre"][b:b + 1, hs]),
                           ("k", grads["k"][b:b + 1, ks]), ("v", grads["v"][b:b + 1, ks]),
                           ("z_pre", grads["z_pre"][b:b + 1, ks])):
                e = excess(got, rg[n], n in BF16_OUT, n)
                worst[n] = max(worst.get(n, -1.0), e)
                assert e <= 0, (n, b, h0, e)
            sums["pos_bias"][:, hs] += rg["pos_bias"].double()
            sums["scale_embed"] += rg["scale_embed"].double()
            sums["phase_base"][:, hs] += rg["phase_base"].double()
            sums["phase_gain"][:, hs] += rg["phase_gain"].double()
        note(f"row {b} of {B} checked")
    for n in PARAMS:
        e = excess(grads[n], sums[n], False, n)
        worst[n] = e
        assert e <= 0, (n, e)
    note("worst excess over the bar: " + ", ".join(f"{n} {v:+.2e}" for n, v in worst.items()))
    note("largest |gpu - oracle| (bar 2e-2): " + ", ".join(f"{n} {v:.2e}" for n, v in MAX_ERR.items()))


@pytest.mark.parametrize("mode", [0, 3])
def test_cfg2_training_microbatch_as_benched(pkg, device, mode):
    """B15 H8 T2048 bf16 fwd+bwd on bench.py's seed-0 inputs (3,840 query tiles), in the baseline and the
    overlap-slab schedule."""
    note(f"cfg2 B15 H8 T2048 bf16 fwd+bwd, grouped mode {mode}")
    t, js, jl = bench.synth(pkg, 15, 8, 2048, 0, torch.device("cpu"))
    check_rows(pkg, t, list(pkg.ALL_OFFSETS), js, 0, 1, device, mode=mode)


def test_cfg4_long_context_as_benched(pkg, device):
    """B4 H8 T8192 bf16 fwd+bwd on bench.py's seed-4 inputs (4,096 query tiles); oracle per 4 heads."""
    note("cfg4 B4 H8 T8192 bf16 fwd+bwd")
    t, js, jl = bench.synth(pkg, 4, 8, 8192, 4, torch.device("cpu"))
    check_rows(pkg, t, list(pkg.ALL_OFFSETS), js, 0, 1, device, head_chunk=4)


@pytest.mark.parametrize("gain_scale", [1.0, 40.0])
def test_cfg1_fp32_full_lattice_as_benched(pkg, device, gain_scale):
    """cfg1's shape in fp32: B1 H8 T2048 on bench.py's seed-0 inputs, all 96 offsets (92 with a source, 75
    of them far), forward and backward through the fp32 kernels, against the float64 oracle one head at a
    time.  gain_scale 40 multiplies phase_gain (std 0.64 -> 25.6) so the MOVT angles are O(1) rather than
    O(0.01).  Bar: 1e-5 relative (||a-b||_inf / ||b||_inf) for out and all nine gradients, per head for
    out/dq/dk/dv/dy/dz and over the head-summed parameter gradients."""
    note(f"cfg1 B1 H8 T2048 fp32 fwd+bwd, phase_gain x{gain_scale}")
    t, js, jl = bench.synth(pkg, 1, 8, 2048, 0, torch.device("cpu"), dtype=torch.float32)
    t["phase_gain"] = t["phase_gain"] * gain_scale
    offsets = list(pkg.ALL_OFFSETS)
    out, grads = run_gpu(pkg, t, offsets, js, 0, 1, device)
    assert out.dtype == torch.float32
    H = t["q"].shape[1]
    sums = {n: torch.zeros_like(t[n], dtype=torch.float64) for n in PARAMS}
    worst = {}

    def rel(a, b):
        a, b = a.detach().double().cpu(), b.detach().double().cpu()
        return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))

    for h in range(H):
        hs = slice(h, h + 1)
        inp = {n: t[n][:, hs].double() for n in ("q", "k", "v", "y_pre", "z_pre")}
        inp["pos_bias"] = t["pos_bias"][:, hs].double()
        inp["scale_embed"] = t["scale_embed"].double()
        inp["phase_base"] = t["phase_base"][:, hs].double()
        inp["phase_gain"] = t["phase_gain"][:, hs].double()
        ro, _, rg = dsqg_ref.dsqg_forward_backward(inp, offsets, js, t["dout"][:, hs].double(), query_start=1,
                                                   round_se=False)
        checks = [("out", out[:, hs], ro)] + [(n, grads[n][:, hs], rg[n])
                                              for n in ("q", "k", "v", "y_pre", "z_pre")]
        for n, got, ref in checks:
            e = rel(got, ref)
            worst[n] = max(worst.get(n, 0.0), e)
            assert e < 1e-5, (n, h, e)
        sums["pos_bias"][:, hs] += rg["pos_bias"]
        sums["scale_embed"] += rg["scale_embed"]
        sums["phase_base"][:, hs] += rg["phase_base"]
        sums["phase_gain"][:, hs] += rg["phase_gain"]
        note(f"head {h} of {H} checked")
    for n in PARAMS:
        worst[n] = rel(grads[n], sums[n])
        assert worst[n] < 1e-5, (n, worst[n])
    note("worst relative error (bar 1e-5): " + ", ".join(f"{n} {v:.2e}" for n, v in worst.items()))


def test_bf16_gqa_ragged_many_tiles(pkg, device):
    """bf16 with GQA (H8 over 2 KV heads), a ragged N = 2047 (tail masks), query_start 3, plane shift 5, hot
    MOVT angles and 1,280 query tiles (more than either persistent grid)."""
    note("B5 H8 Hkv2 N2047 bf16 fwd+bwd")
    offsets = list(pkg.ALL_OFFSETS)
    t = make_inputs(5, 8, 2, 2047, offsets, 17, seed=77, dtype=torch.bfloat16, plane_shift=5, gain_std=6.0)
    t["dout"] = torch.randn(5, 8, 2047, 64, generator=torch.Generator().manual_seed(78)).to(torch.bfloat16)
    check_rows(pkg, t, offsets, 17, 5, 3, device)


def _q6_oracle(q, kd, vd, tables, offsets, js, qpn, kpn, qs):
    """Oracle forward on dequantised K/V (fp32), y from q and z from the dequantised K."""
    inp = {"q": q.float(), "k": kd, "v": vd, **{n: tables[n].float() for n in PARAMS}}
    inp["y_pre"] = features(q.float(), qpn)
    inp["z_pre"] = features(kd, kpn)
    return dsqg_ref.dsqg_forward(*(inp[n] for n in NAMES), offsets, js, query_start=qs, round_se=True)


def test_cfg3_q6_prefill_as_benched(pkg, device):
    """B20 H8 T2048 q6 prefill on bench.py's inputs: 16 (b, h) slices against the oracle."""
    note("cfg3 q6 prefill B20 H8 T2048")
    t, js, jl = bench.synth(pkg, 20, 8, 2048, 3, device)
    kpn = torch.nn.functional.normalize(t["kp"], dim=-1)
    qpn = torch.nn.functional.normalize(t["qp"], dim=-1)
    cache = pkg.q6.pack_kv(t["k"], t["v"], kpn.to(device))
    out = pkg.q6.q6_prefill(t["q"], cache, t["pos_bias"], t["scale_embed"], t["phase_base"], t["phase_gain"],
                            qpn.to(device), t["offsets"], js, jl, 0, 1)
    torch.cuda.synchronize()
    out = out.cpu()
    offsets = t["offsets"].tolist()
    rng = np.random.default_rng(3)
    picks = [(0, 0), (19, 7)] + [(int(rng.integers(20)), int(rng.integers(8))) for _ in range(14)]
    MAX_ERR.clear()
    worst = -1.0
    for b, h in picks:
        kd, vd, _ = q6_ref.unpack_slots(cache[b:b + 1, h:h + 1].cpu().numpy())
        tables = {"pos_bias": t["pos_bias"][:, h:h + 1].cpu(), "scale_embed": t["scale_embed"].cpu(),
                  "phase_base": t["phase_base"][:, h:h + 1].cpu(), "phase_gain": t["phase_gain"][:, h:h + 1].cpu()}
        ref = _q6_oracle(t["q"][b:b + 1, h:h + 1].cpu(), torch.from_numpy(kd), torch.from_numpy(vd), tables,
                         offsets, js, qpn, kpn, 1)
        e = excess(out[b:b + 1, h:h + 1], ref, True, "out")
        worst = max(worst, e)
        assert e <= 0, (b, h, e)
    note(f"worst excess over the bar: out {worst:+.2e}; largest |gpu - oracle| {MAX_ERR['out']:.2e} (bar 2e-2)")


def test_cfg5_q6_decode_as_benched(pkg, device):
    """256 sequences x 9 layers x H8 decode step on bench.py's inputs: 16 (sequence, layer) pairs, all heads,
    against the oracle on the dequantised cache rows 0..t."""
    note("cfg5 q6 decode 256 x 9 x H8")
    w = bench.decode_workload(pkg, device)
    out = pkg.q6.q6_decode(w["qdec"], w["pos"].to(device), w["caches"], w["pos_bias"], w["scale_embed"],
                           w["phase_base"], w["phase_gain"], w["qps"], w["off"], w["js"],
                           len(w["offsets"]) - w["js"], 0)
    torch.cuda.synchronize()
    out = out.cpu()
    rng = np.random.default_rng(5)
    picks = [(0, 0), (255, 8)] + [(int(rng.integers(256)), int(rng.integers(9))) for _ in range(14)]
    MAX_ERR.clear()
    worst = -1.0
    for s, l in picks:
        tpos = int(w["pos"][s])
        kd, vd, _ = q6_ref.unpack_slots(w["caches"][l, s:s + 1, :, :tpos + 1].cpu().numpy())
        q = torch.zeros(1, w["H"], tpos + 1, 64)
        q[0, :, tpos] = w["qdec"][s, l].cpu().float()
        tables = {n: w[n][l].cpu() for n in PARAMS}
        ref = _q6_oracle(q, torch.from_numpy(kd), torch.from_numpy(vd), tables, w["offsets"], w["js"],
                         w["qpn"], w["kpn"], 0)
        e = excess(out[s, l], ref[0, :, tpos], True, "out")
        worst = max(worst, e)
        assert e <= 0, (s, l, tpos, e)
    note(f"worst excess over the bar: out {worst:+.2e}; largest |gpu - oracle| {MAX_ERR['out']:.2e} (bar 2e-2)")
    del w
    torch.cuda.empty_cache()
