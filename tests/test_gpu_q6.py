"""GPU q6 path against the CPU codec and oracle (runs on an MI355X).

Codec: GPU-packed slots byte-identical to the CPU codec, GPU dequant equal to
the CPU dequant (both exact).  Prefill/decode: within 2e-2 max-abs of the DSQG
oracle evaluated on the dequantised K/V, with y from q and z from the
dequantised K, and bf16-rounded scale embeddings.
"""

import numpy as np
import pytest
import torch

from oracle import dsqg_ref, q6_ref
from tests.dsqg_cases import NAMES, features, make_inputs, max_abs, orthogonal_probes

pytestmark = pytest.mark.gpu


def edge_rows(shape, g):
    x = torch.randn(*shape, generator=g)
    x[..., 0, :] = 0.0                          # all-zero row -> zero scales
    x[..., 1, :32] = 1e-7                       # fp16-subnormal scale
    x[..., 2, 5] = 4.0e6                        # saturating scale
    x[..., 3, :] = torch.arange(64) - 31.5      # half-way codes
    return x


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_pack_matches_cpu_codec_bit_exact(pkg, device, dtype):
    g = torch.Generator().manual_seed(1)
    k = edge_rows((2, 3, 37, 64), g).to(dtype)
    v = (3.0 * torch.randn(2, 3, 37, 64, generator=g)).to(dtype)
    _, kp = orthogonal_probes(64, 4)
    kpn = torch.nn.functional.normalize(kp, dim=-1)
    cache = pkg.q6.pack_kv(k.to(device), v.to(device), kpn.to(device)).cpu().numpy()
    ref = q6_ref.pack_slots(k.float().numpy(), v.float().numpy(), None)
    assert np.array_equal(cache[..., :104], ref[..., :104])
    assert not cache[..., 120:].any()
    kd, vd = pkg.q6.unpack_kv(torch.from_numpy(cache).to(device))
    rk, rv, _ = q6_ref.unpack_slots(cache)
    assert np.array_equal(kd.cpu().numpy(), rk) and np.array_equal(vd.cpu().numpy(), rv)
    z = np.ascontiguousarray(cache[..., 104:120]).view(np.float32).reshape(2, 3, 37, 4)
    rz = features(torch.from_numpy(rk), kpn).numpy()
    assert np.allclose(z, rz, rtol=1e-5, atol=1e-6)


def _oracle_on_cache(x, cache_np, offsets, js, shift, qp, kp, qs, return_lse=False, round_se=True):
    kd, vd, _ = q6_ref.unpack_slots(cache_np)
    inp = dict(x)
    inp["k"] = torch.from_numpy(kd).double()
    inp["v"] = torch.from_numpy(vd).double()
    inp["y_pre"] = features(x["q"].double(), qp).double()
    inp["z_pre"] = features(torch.from_numpy(kd).double(), kp).double()
    return dsqg_ref.dsqg_forward(*(inp[n].double() for n in NAMES), offsets, js, plane_shift=shift,
                                 query_start=qs, round_se=round_se, return_lse=return_lse)


@pytest.mark.parametrize("widen,shift", [(True, 2), (False, 2), (True, 7), (True, 14)])
def test_prefill_matches_oracle(pkg, device, widen, shift):
    """Both prefill schedules (cache rows widened once into a workspace, or slots gathered directly), GQA, a
    ragged N, query_start 1 and hot MOVT angles; odd and last plane shifts on the widened rows, whose MOVT
    pair is the one accumulated without the code bytes' +32."""
    offsets = list(pkg.ALL_OFFSETS)
    x = make_inputs(2, 4, 2, 300, offsets, 17, seed=3, dtype=torch.bfloat16, plane_shift=shift, gain_std=6.0)
    qp, kp = orthogonal_probes(64, shift)
    qp, kp = torch.nn.functional.normalize(qp, dim=-1), torch.nn.functional.normalize(kp, dim=-1)
    xd = {n: t.to(device) for n, t in x.items()}
    cache = pkg.q6.pack_kv(xd["k"], xd["v"], kp.to(device))
    off = torch.tensor(offsets, dtype=torch.int32, device=device)
    out, lse = pkg.q6.q6_prefill(xd["q"], cache, xd["pos_bias"], xd["scale_embed"], xd["phase_base"],
                                 xd["phase_gain"], qp.to(device), off, 17, 79, shift, 1, return_lse=True,
                                 widen=widen)
    ref, rlse = _oracle_on_cache(x, cache.cpu().numpy(), offsets, 17, shift, qp, kp, 1, return_lse=True)
    assert max_abs(out, ref) < 2e-2
    # lse (natural log, -inf before query_start) within the bf16 bar
    assert torch.equal(torch.isinf(lse.cpu()), torch.isinf(rlse))
    fin = torch.isfinite(rlse)
    assert (lse.cpu().double()[fin] - rlse[fin]).abs().max().item() < 2e-2


@pytest.mark.parametrize("offsets,js", [
    ([1, 2, 3, 5, 8, 13, 21, 40, 48, 64, 96], 8),   # a small offset above 32: the band takes 7 of 8
    ([2, 1, 4, 3, 48, 96], 4),                      # unsorted small offsets: the band stops at the descent
    ([40, 33, 64, 96], 2),                          # small offsets all above 32: no band, near table read by the walk
    ([48, 64, 96], 0),                              # no small offsets: the widened-row gather alone
])
def test_prefill_band_lattice_edges(pkg, device, offsets, js):
    """Widened rows with lattices whose small offsets the near band takes only in part or not at
    all; against the oracle on the dequantised cache, ragged N, query_start 1."""
    x = make_inputs(1, 2, 2, 200, offsets, js, seed=97, dtype=torch.bfloat16, gain_std=4.0)
    qp, kp = orthogonal_probes(64, 0)
    qp, kp = torch.nn.functional.normalize(qp, dim=-1), torch.nn.functional.normalize(kp, dim=-1)
    xd = {n: t.to(device) for n, t in x.items()}
    cache = pkg.q6.pack_kv(xd["k"], xd["v"], kp.to(device))
    off = torch.tensor(offsets, dtype=torch.int32, device=device)
    out = pkg.q6.q6_prefill(xd["q"], cache, xd["pos_bias"], xd["scale_embed"], xd["phase_base"], xd["phase_gain"],
                            qp.to(device), off, js, len(offsets) - js, 0, 1, widen=True)
    ref = _oracle_on_cache(x, cache.cpu().numpy(), offsets, js, 0, qp, kp, 1)
    assert max_abs(out, ref) < 2e-2, (offsets, max_abs(out, ref))


@pytest.mark.parametrize("widen", [True, False])
def test_prefill_fp32_scale_embed(pkg, device, widen):
    """round_se=False: the prefill's <q, e_j> table takes SE in fp32, against the oracle without SE
    rounding; SE scaled up so its rounding would show."""
    offsets = list(pkg.ALL_OFFSETS)
    x = make_inputs(1, 4, 2, 260, offsets, 17, seed=5, dtype=torch.bfloat16, gain_std=6.0)
    x["scale_embed"] = 40.0 * x["scale_embed"]
    qp, kp = orthogonal_probes(64, 0)
    qp, kp = torch.nn.functional.normalize(qp, dim=-1), torch.nn.functional.normalize(kp, dim=-1)
    xd = {n: t.to(device) for n, t in x.items()}
    cache = pkg.q6.pack_kv(xd["k"], xd["v"], kp.to(device))
    off = torch.tensor(offsets, dtype=torch.int32, device=device)
    out = pkg.q6.q6_prefill(xd["q"], cache, xd["pos_bias"], xd["scale_embed"], xd["phase_base"], xd["phase_gain"],
                            qp.to(device), off, 17, 79, 0, 1, round_se=False, widen=widen)
    ref = _oracle_on_cache(x, cache.cpu().numpy(), offsets, 17, 0, qp, kp, 1, round_se=False)
    assert max_abs(out, ref) < 2e-2


def test_decode_matches_oracle(pkg, device):
    offsets = list(pkg.ALL_OFFSETS)
    shift = 0
    S, L, H, Hkv, N = 3, 2, 4, 2, 300
    g = torch.Generator().manual_seed(7)
    layers = [make_inputs(S, H, Hkv, N, offsets, 17, seed=50 + l, dtype=torch.bfloat16, plane_shift=shift,
                          gain_std=6.0) for l in range(L)]
    pos = torch.tensor([299, 96, 150], dtype=torch.int32)
    qp, kp = orthogonal_probes(64, shift)
    qp, kp = torch.nn.functional.normalize(qp, dim=-1), torch.nn.functional.normalize(kp, dim=-1)
    caches = torch.stack([pkg.q6.pack_kv(x["k"].to(device), x["v"].to(device), kp.to(device)) for x in layers])
    qdec = torch.stack([torch.stack([layers[l]["q"][s, :, int(pos[s])] for l in range(L)]) for s in range(S)])
    tables = {n: torch.stack([x[n] for x in layers]).to(device) for n in ("pos_bias", "scale_embed", "phase_base",
                                                                          "phase_gain")}
    off = torch.tensor(offsets, dtype=torch.int32, device=device)
    out = pkg.q6.q6_decode(qdec.to(device), pos.to(device), caches, tables["pos_bias"], tables["scale_embed"],
                           tables["phase_base"], tables["phase_gain"], torch.stack([qp] * L).to(device), off,
                           17, 79, shift).cpu()
    for l in range(L):
        ref = _oracle_on_cache(layers[l], caches[l].cpu().numpy(), offsets, 17, shift, qp, kp, 0)
        for s in range(S):
            t = int(pos[s])
            assert max_abs(out[s, l], ref[s, :, t]) < 2e-2, (s, l)


def test_decode_fp32_scale_embed(pkg, device):
    """round_se=False: the score table takes SE in fp32 (bf16 hi + lo halves on the MFMA), against the
    oracle without SE rounding; SE scaled up so its rounding would show."""
    offsets = list(pkg.ALL_OFFSETS)
    S, L, H, Hkv, N = 2, 2, 4, 2, 400
    layers = [make_inputs(S, H, Hkv, N, offsets, 17, seed=70 + l, dtype=torch.bfloat16, gain_std=6.0)
              for l in range(L)]
    for x in layers:
        x["scale_embed"] = 40.0 * x["scale_embed"]
    pos = torch.tensor([399, 130], dtype=torch.int32)
    qp, kp = orthogonal_probes(64, 0)
    qp, kp = torch.nn.functional.normalize(qp, dim=-1), torch.nn.functional.normalize(kp, dim=-1)
    caches = torch.stack([pkg.q6.pack_kv(x["k"].to(device), x["v"].to(device), kp.to(device)) for x in layers])
    qdec = torch.stack([torch.stack([layers[l]["q"][s, :, int(pos[s])] for l in range(L)]) for s in range(S)])
    tables = {n: torch.stack([x[n] for x in layers]).to(device) for n in ("pos_bias", "scale_embed", "phase_base",
                                                                          "phase_gain")}
    off = torch.tensor(offsets, dtype=torch.int32, device=device)
    out = pkg.q6.q6_decode(qdec.to(device), pos.to(device), caches, tables["pos_bias"], tables["scale_embed"],
                           tables["phase_base"], tables["phase_gain"], torch.stack([qp] * L).to(device), off,
                           17, 79, 0, round_se=False).cpu()
    for l in range(L):
        ref = _oracle_on_cache(layers[l], caches[l].cpu().numpy(), offsets, 17, 0, qp, kp, 0, round_se=False)
        for s in range(S):
            assert max_abs(out[s, l], ref[s, :, int(pos[s])]) < 2e-2, (s, l)


def test_decode_full_lattice_eight_heads(pkg, device):
    """H = H_kv = 8 (one table tile per wave but one), plane shift 5, a row
    with no valid offset (t = 0 gives out = 0), a row with only near offsets
    and one past the largest offset (all 96 valid)."""
    offsets = list(pkg.ALL_OFFSETS)
    shift = 5
    S, H, N = 4, 8, 2300
    x = make_inputs(S, H, H, N, offsets, 17, seed=91, dtype=torch.bfloat16, plane_shift=shift, gain_std=6.0)
    pos = torch.tensor([0, 40, 1000, 2250], dtype=torch.int32)
    qp, kp = orthogonal_probes(64, shift)
    qp, kp = torch.nn.functional.normalize(qp, dim=-1), torch.nn.functional.normalize(kp, dim=-1)
    cache = pkg.q6.pack_kv(x["k"].to(device), x["v"].to(device), kp.to(device))
    qdec = torch.stack([x["q"][s, :, int(pos[s])] for s in range(S)]).unsqueeze(1)
    tables = {n: x[n].unsqueeze(0).to(device) for n in ("pos_bias", "scale_embed", "phase_base", "phase_gain")}
    off = torch.tensor(offsets, dtype=torch.int32, device=device)
    out = pkg.q6.q6_decode(qdec.to(device), pos.to(device), cache.unsqueeze(0), tables["pos_bias"],
                           tables["scale_embed"], tables["phase_base"], tables["phase_gain"],
                           qp.unsqueeze(0).to(device), off, 17, 79, shift).cpu()
    assert not out[0].any()
    ref = _oracle_on_cache(x, cache.cpu().numpy(), offsets, 17, shift, qp, kp, 0)
    for s in range(S):
        assert max_abs(out[s, 0], ref[s, :, int(pos[s])]) < 2e-2, s


def test_decode_graph_replay_matches_eager(pkg, device):
    """The decode launch captured in a HIP graph: each replay (eager work and
    synchronisations between them) equals the eager output bit for bit."""
    offsets = list(pkg.ALL_OFFSETS)
    S, H, N = 5, 8, 600
    x = make_inputs(S, H, 2, N, offsets, 17, seed=13, dtype=torch.bfloat16, plane_shift=2, gain_std=3.0)
    qp, kp = orthogonal_probes(64, 2)
    qp, kp = torch.nn.functional.normalize(qp, dim=-1), torch.nn.functional.normalize(kp, dim=-1)
    cache = pkg.q6.pack_kv(x["k"].to(device), x["v"].to(device), kp.to(device)).unsqueeze(0)
    pos = torch.tensor([99, 300, 599, 150, 420], dtype=torch.int32, device=device)
    qdec = torch.stack([x["q"][s, :, int(pos[s])] for s in range(S)]).unsqueeze(1).to(device)
    tab = {n: x[n].unsqueeze(0).to(device) for n in ("pos_bias", "scale_embed", "phase_base", "phase_gain")}
    off = torch.tensor(offsets, dtype=torch.int32, device=device)
    qps = qp.unsqueeze(0).to(device)

    def step():
        return pkg.q6.q6_decode(qdec, pos, cache, tab["pos_bias"], tab["scale_embed"], tab["phase_base"],
                                tab["phase_gain"], qps, off, 17, 79, 2)

    ref = step().clone()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step()
    for _ in range(3):
        other = pkg.q6.pack_kv(x["v"].to(device), x["k"].to(device), kp.to(device))   # eager work
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        del other


def test_decode_maximum_sizes(pkg, device):
    """J = 256 offsets (17 near, 239 far) and H = 16 heads (four workgroups of four heads per
    (sequence, layer), H_kv = 4): the decode step against the oracle on the dequantised cache."""
    offsets = list(range(1, 18)) + list(range(48, 48 + 239))
    S, H, Hkv, N = 2, 16, 4, 320
    x = make_inputs(S, H, Hkv, N, offsets, 17, seed=81, dtype=torch.bfloat16, gain_std=6.0)
    pos = torch.tensor([319, 200], dtype=torch.int32)
    qp, kp = orthogonal_probes(64, 0)
    qp, kp = torch.nn.functional.normalize(qp, dim=-1), torch.nn.functional.normalize(kp, dim=-1)
    cache = pkg.q6.pack_kv(x["k"].to(device), x["v"].to(device), kp.to(device))
    qdec = torch.stack([x["q"][s, :, int(pos[s])] for s in range(S)]).unsqueeze(1)   # [S,1,H,64]
    tab = {n: x[n].unsqueeze(0).to(device) for n in ("pos_bias", "scale_embed", "phase_base", "phase_gain")}
    off = torch.tensor(offsets, dtype=torch.int32, device=device)
    out = pkg.q6.q6_decode(qdec.to(device), pos.to(device), cache.unsqueeze(0), tab["pos_bias"], tab["scale_embed"],
                           tab["phase_base"], tab["phase_gain"], qp.unsqueeze(0).to(device), off, 17, 239, 0).cpu()
    ref = _oracle_on_cache(x, cache.cpu().numpy(), offsets, 17, 0, qp, kp, 0)
    for s in range(S):
        assert max_abs(out[s, 0], ref[s, :, int(pos[s])]) < 2e-2, s


@pytest.mark.parametrize("H,Hkv", [(3, 3), (6, 3)])
def test_decode_head_groups(pkg, device, H, Hkv):
    """A decode workgroup takes four heads: H = 3 is one workgroup of three waves; H = 6 (GQA, two query
    heads per KV head) is two workgroups per (sequence, layer), the second with two heads and two waves
    without one.  Every head against the oracle on the dequantised cache, at the full lattice."""
    offsets = list(pkg.ALL_OFFSETS)
    S, L, N = 3, 2, 700
    layers = [make_inputs(S, H, Hkv, N, offsets, 17, seed=120 + 10 * H + l, dtype=torch.bfloat16, plane_shift=3,
                          gain_std=6.0) for l in range(L)]
    pos = torch.tensor([699, 97, 400], dtype=torch.int32)
    qp, kp = orthogonal_probes(64, 3)
    qp, kp = torch.nn.functional.normalize(qp, dim=-1), torch.nn.functional.normalize(kp, dim=-1)
    caches = torch.stack([pkg.q6.pack_kv(x["k"].to(device), x["v"].to(device), kp.to(device)) for x in layers])
    qdec = torch.stack([torch.stack([layers[l]["q"][s, :, int(pos[s])] for l in range(L)]) for s in range(S)])
    tables = {n: torch.stack([x[n] for x in layers]).to(device) for n in ("pos_bias", "scale_embed", "phase_base",
                                                                          "phase_gain")}
    off = torch.tensor(offsets, dtype=torch.int32, device=device)
    out = pkg.q6.q6_decode(qdec.to(device), pos.to(device), caches, tables["pos_bias"], tables["scale_embed"],
                           tables["phase_base"], tables["phase_gain"], torch.stack([qp] * L).to(device), off,
                           17, 79, 3).cpu()
    for l in range(L):
        ref = _oracle_on_cache(layers[l], caches[l].cpu().numpy(), offsets, 17, 3, qp, kp, 0)
        for s in range(S):
            assert max_abs(out[s, l], ref[s, :, int(pos[s])]) < 2e-2, (H, s, l)


@pytest.mark.parametrize("widen", [True, False])
def test_prefill_maximum_offsets(pkg, device, widen):
    """J = 256 offsets (17 near, 239 far) in the prefill, against the oracle on the dequantised cache."""
    offsets = list(range(1, 18)) + list(range(48, 48 + 239))
    x = make_inputs(1, 4, 2, 320, offsets, 17, seed=83, dtype=torch.bfloat16, gain_std=6.0)
    qp, kp = orthogonal_probes(64, 0)
    qp, kp = torch.nn.functional.normalize(qp, dim=-1), torch.nn.functional.normalize(kp, dim=-1)
    xd = {n: t.to(device) for n, t in x.items()}
    cache = pkg.q6.pack_kv(xd["k"], xd["v"], kp.to(device))
    off = torch.tensor(offsets, dtype=torch.int32, device=device)
    out = pkg.q6.q6_prefill(xd["q"], cache, xd["pos_bias"], xd["scale_embed"], xd["phase_base"], xd["phase_gain"],
                            qp.to(device), off, 17, 239, 0, 1, widen=widen)
    ref = _oracle_on_cache(x, cache.cpu().numpy(), offsets, 17, 0, qp, kp, 1)
    assert max_abs(out, ref) < 2e-2
