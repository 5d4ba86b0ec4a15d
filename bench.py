"""Benchmark of the DSQG offset-gather path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Headline workload (the training microbatch): one DSQG layer forward+backward,
bf16, B=15, H=8, T=2048, head_dim=64, the 96-offset lattice, synthetic seeded
inputs resident in HBM.  A step is dwarf_dsqg_fwd + dwarf_dsqg_bwd_dq +
dwarf_dsqg_bwd_params + dwarf_dsqg_bwd_dkdv on the current stream.  value = tokens (B*T) per second.

Also reported under "extra": the q6 decode step (256 sequences x 9 layers,
cache length 2048), the q6 prefill forward (B=20) and the long-context
DSQG fwd+bwd + EMA fwd+bwd (B=4, T=8192).  cpu_baseline times the CPU
restatement of the reference's eager path (oracle/) on a bounded sample.

Prints one JSON line.  Runs on one GPU only.
"""

from __future__ import annotations

import argparse
import importlib
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK = 8.0e12            # MI355X HBM3E, bytes/s
TABLE_BYTES = 47_872         # pos_bias + scale_embed + phase tables per layer (J=96, H=8, hd=64)
FWD_BYTES_PER_TH = 548       # q,k,v (3x128) + y,z (2x16) + out (128) + lse (4)
BWD_BYTES_PER_TH = 1092      # read q,k,v,o,dO + lse + y,z; write dq,dk,dv + dy,dz
DQ_BYTES_PER_TH = 820        # dq launch: read q,k,v,o,dO,lse,y,z; write dq,dy
DKDV_BYTES_PER_TH = 820      # dkdv launch: read k,v,q,dO,lse,y,z; write dk,dv,dz
PARAMS_BYTES_PER_TH = 128    # params launch: read q (dS^T q); the parameter gradients are the tables
DELTA_BYTES_PER_TH = 260     # delta launch (overlapped schedule): read o, dO (2x128) and lse (4)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def synth(pkg, B, H, N, seed, device, dtype=torch.bfloat16, plane_shift=0):
    """Seeded synthetic DSQG inputs (draw order fixed; CPU generator, then copied)."""
    offsets = list(pkg.ALL_OFFSETS)
    J, js = len(offsets), 17
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, N, 64, generator=g).to(dtype)
    k = torch.randn(B, H, N, 64, generator=g).to(dtype)
    v = torch.randn(B, H, N, 64, generator=g).to(dtype)
    dout = torch.randn(B, H, N, 64, generator=g).to(dtype)
    pb = 0.02 * torch.randn(J, H, generator=g)
    se = 0.01 * torch.randn(J, 64, generator=g)
    se = se - se.mean(0, keepdim=True)
    pbase = 0.5 * 0.01 * torch.randn(J - js, H, 4, generator=g)
    pgain = 0.5 * 1.28 * torch.randn(J - js, H, 4, generator=g)
    qp, kp = pkg._orthogonal_phase_probes(4, 64, plane_shift)

    def feat(x, p):
        xf = x.float()
        inv = torch.rsqrt(xf.square().sum(-1, keepdim=True) + 64e-6)
        return (torch.einsum("bhnd,rd->bhnr", xf, torch.nn.functional.normalize(p, dim=-1)) * inv).contiguous()

    t = dict(q=q, k=k, v=v, dout=dout, pos_bias=pb, scale_embed=se, phase_base=pbase, phase_gain=pgain,
             y_pre=feat(q, qp), z_pre=feat(k, kp))
    t = {n: x.to(device) for n, x in t.items()}
    t["offsets"] = torch.tensor(offsets, dtype=torch.int32, device=device)
    t["qp"], t["kp"] = qp, kp
    return t, js, J - js


class CacheFlush:
    """Evicts every cache level (L2, the 256 MB MALL) by READING 1 GiB: a write would leave dirty lines
    behind, and the timed kernel would then pay for their write-back."""

    def __init__(self, device):
        self.buf = torch.ones(1 << 28, dtype=torch.float32, device=device)

    def __call__(self):
        self.buf.sum()


def time_dsqg_step(pkg, t, js, jl, steps, warmup, flush=None, stages=True):
    """Returns (ms_per_step, serial per-launch ms dict, overlapped per-launch ms dict).

    The step time comes from K steps bracketed by two events only; the step
    is the forward plus the backward on its default bf16 schedule, delta and
    dK/dV on a second stream beside dQ and params.  The per-launch durations
    come from two more runs of K steps with events between launches (each
    event record costs the stream a gap of several µs, so those events stay
    out of the step's clock): the serial schedule (every stage alone on the
    chip) and the overlapped schedule the step runs (events on the stream
    each stage is launched on; dQ and dK/dV then share the CUs, so each takes
    longer than alone).  With ``flush`` (cold clock) every step is preceded by
    a cache-evicting read and timed by its own two events.
    """
    ops = pkg.dsqg if hasattr(pkg, "dsqg") else importlib.import_module("dwarf-v2_amd.dsqg")
    args = (t["q"], t["k"], t["v"], t["pos_bias"], t["scale_embed"], t["phase_base"], t["phase_gain"],
            t["y_pre"], t["z_pre"], t["offsets"])

    def step(ev_f=None, ev_b=None, ev_o=None):
        out, lse = ops.dsqg_forward(*args, js, jl, 0, 1, events=ev_f)
        ops.dsqg_backward(t["dout"], *args, out, lse, js, jl, 0, 1, events=ev_b, overlap_events=ev_o)

    def ev(n):
        return [torch.cuda.Event(enable_timing=True) for _ in range(n)]

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    if flush is None:
        start, end = ev(2)
        torch.cuda.synchronize()
        start.record()
        for _ in range(steps):
            step()
        end.record()
        torch.cuda.synchronize()
        total_ms = start.elapsed_time(end)
    else:
        marks = [ev(2) for _ in range(steps)]
        for s, e in marks:
            flush()
            s.record()
            step()
            e.record()
        torch.cuda.synchronize()
        total_ms = sum(s.elapsed_time(e) for s, e in marks)
    if not stages:
        return total_ms / steps, None, None
    evs = [(ev(2), ev(4)) for _ in range(steps)]
    for ef, eb in evs:
        if flush is not None:
            flush()
        step(ef, eb)
    torch.cuda.synchronize()
    per = {
        "fwd": sum(ef[0].elapsed_time(ef[1]) for ef, _ in evs) / steps,
        "bwd_dq": sum(eb[0].elapsed_time(eb[1]) for _, eb in evs) / steps,
        "bwd_params": sum(eb[1].elapsed_time(eb[2]) for _, eb in evs) / steps,
        "bwd_dkdv": sum(eb[2].elapsed_time(eb[3]) for _, eb in evs) / steps,
    }
    evo = [(ev(2), ev(6)) for _ in range(steps)]
    for ef, eo in evo:
        if flush is not None:
            flush()
        step(ef, None, eo)
    torch.cuda.synchronize()
    per_o = {
        "fwd": sum(ef[0].elapsed_time(ef[1]) for ef, _ in evo) / steps,
        "bwd_dq": sum(eo[0].elapsed_time(eo[1]) for _, eo in evo) / steps,
        "bwd_params": sum(eo[1].elapsed_time(eo[2]) for _, eo in evo) / steps,
        "bwd_delta": sum(eo[3].elapsed_time(eo[4]) for _, eo in evo) / steps,
        "bwd_dkdv": sum(eo[4].elapsed_time(eo[5]) for _, eo in evo) / steps,
    }
    return total_ms / steps, per, per_o


def cpu_cores() -> tuple[int, int, int | None]:
    """(threads used, affinity cores, cgroup quota cores or None): every core the process may run on,
    i.e. the affinity set, capped by the cgroup's CPU quota where one is set (more threads than the
    quota only queue behind it)."""
    aff = len(os.sched_getaffinity(0))
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, per = f.read().split()[:2]
        if q != "max":
            quota = max(1, int(q) // int(per))
    except (OSError, ValueError):
        pass
    return (min(aff, quota) if quota else aff), aff, quota


def cpu_model() -> str:
    """The host CPU as /proc/cpuinfo names it, with family/model/stepping (the name alone can be generic)."""
    want = ("model name", "cpu family", "model", "stepping")
    got: dict[str, str] = {}
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                k, _, v = ln.partition(":")
                k = k.strip()
                if k in want and k not in got:
                    got[k] = v.strip()
                if len(got) == len(want):
                    break
    except OSError:
        return "unknown CPU"
    return (f"{got.get('model name', 'unknown CPU')} (family {got.get('cpu family', '?')}, "
            f"model {got.get('model', '?')}, stepping {got.get('stepping', '?')})")


def median_seconds(fn, budget_s: float, min_reps: int = 3, max_reps: int = 50) -> tuple[float, int]:
    times: list[float] = []
    end = time.perf_counter() + budget_s
    while len(times) < min_reps or (time.perf_counter() < end and len(times) < max_reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


def cpu_baseline(pkg):
    """The CPU restatements of the reference's eager paths (oracle/), timed on this host's cores.

    value: cfg2's fwd+bwd in its own dtype (bf16 inputs) on batch row 0 (B=1 of 15, the rows are
    independent, so tokens/s scales to the whole microbatch).  Also timed: the same in fp32, cfg1's
    forward (fp32 B1 H8 T2048, the whole config) and the EMA restatement of ``_reference``
    (ema:511-538) at cfg4's x [4,8192,512] bf16.  The DSQG restatement computes in fp32 for bf16
    inputs, as the reference eager computes its scores (dsqg:2658-2662).  Medians of >= 3 runs."""
    from oracle import dsqg_ref, ema_ref

    threads, aff, quota = cpu_cores()
    torch.set_num_threads(threads)
    cpu = torch.device("cpu")
    names = ("q", "k", "v", "pos_bias", "scale_embed", "phase_base", "phase_gain", "y_pre", "z_pre")
    res = {}
    for tag, dt in (("bf16", torch.bfloat16), ("fp32", torch.float32)):
        t, js, _ = synth(pkg, 1, 8, 2048, 0, cpu, dtype=dt)
        inputs = {n: t[n] for n in names}
        offsets = t["offsets"].tolist()
        sec, reps = median_seconds(
            lambda: dsqg_ref.dsqg_forward_backward(inputs, offsets, js, t["dout"], query_start=1), 5.0)
        res[f"cfg2_fwd_bwd_{tag}"] = {"tokens_per_s": 2048 / sec, "s_per_row": sec, "runs": reps}
        if tag == "fp32":
            sec, reps = median_seconds(lambda: dsqg_ref.dsqg_forward(*(inputs[n] for n in names), offsets, js,
                                                                     query_start=1), 3.0)
            res["cfg1_fwd_fp32"] = {"tokens_per_s": 2048 / sec, "s_per_call": sec, "runs": reps}
    g = torch.Generator().manual_seed(0)
    x = torch.randn(4, 8192, 512, generator=g).to(torch.bfloat16)
    alpha = 1.0 - (0.90 + 0.099 * torch.rand(512, generator=g))
    sec, reps = median_seconds(lambda: ema_ref.ema_scan(x, alpha), 3.0)
    res["cfg4_ema_fwd_bf16"] = {"tokens_per_s": 4 * 8192 / sec, "s_per_call": sec, "runs": reps}
    head = res["cfg2_fwd_bwd_bf16"]
    return {"value": head["tokens_per_s"], "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": (f"oracle/dsqg_ref fwd+bwd of batch row 0 of cfg2 (B=1 of 15, H=8, T=2048, J=96), bf16 "
                       f"inputs, median of {head['runs']} runs of {head['s_per_row']:.2f} s; {threads} threads "
                       f"(affinity {aff} cores, cgroup quota {quota if quota else 'none'}); {cpu_model()}"),
            "breakdown": res}


def decode_workload(pkg, device):
    """The cfg5 decode step's inputs: 256 sequences x 9 layers x H8, q6 caches of length 2048 (seeded)."""
    S, L, H, N = 256, 9, 8, 2048
    offsets = list(pkg.ALL_OFFSETS)
    J, js = len(offsets), 17
    g = torch.Generator().manual_seed(0)
    pos = torch.randint(96, N, (S,), generator=g, dtype=torch.int32)
    qdec = torch.randn(S, L, H, 64, generator=g).to(torch.bfloat16).to(device)
    pb = (0.02 * torch.randn(L, J, H, generator=g)).to(device)
    se = (0.01 * torch.randn(L, J, 64, generator=g)).to(device)
    pbase = (0.005 * torch.randn(L, J - js, H, 4, generator=g)).to(device)
    pgain = (0.64 * torch.randn(L, J - js, H, 4, generator=g)).to(device)
    qp, kp = pkg._orthogonal_phase_probes(4, 64, 0)
    qpn = torch.nn.functional.normalize(qp, dim=-1)
    kpn = torch.nn.functional.normalize(kp, dim=-1)
    caches = torch.empty((L, S, H, N, 128), dtype=torch.uint8, device=device)
    gd = torch.Generator(device=device).manual_seed(1)
    for l in range(L):
        k = torch.randn(S, H, N, 64, generator=gd, device=device, dtype=torch.bfloat16)
        v = torch.randn(S, H, N, 64, generator=gd, device=device, dtype=torch.bfloat16)
        caches[l] = pkg.q6.pack_kv(k, v, kpn.to(device))
        del k, v
    return dict(S=S, L=L, H=H, N=N, offsets=offsets, js=js, pos=pos, qdec=qdec, pos_bias=pb, scale_embed=se,
                phase_base=pbase, phase_gain=pgain, qpn=qpn, kpn=kpn, caches=caches,
                off=torch.tensor(offsets, dtype=torch.int32, device=device),
                qps=torch.stack([qpn] * L).to(device))


def decode_bytes(pos, offsets, js, L, H) -> int:
    """Algorithmic bytes of one decode step: per (sequence, layer, head) the bf16 query and output
    (256 B), 104 B of q6 K+V per valid cache row and 16 B of stored z per valid far row, plus the
    per-layer tables."""
    nv = [sum(1 for d in offsets if int(t) - d >= 0) for t in pos]
    nf = [sum(1 for d in offsets[js:] if int(t) - d >= 0) for t in pos]
    return sum(L * H * (256 + 104 * a + 16 * b) for a, b in zip(nv, nf)) + L * TABLE_BYTES


def q6_decode_extra(pkg, device, steps, warmup):
    """The cfg5 decode step timed three ways: HIP-graph replays at fixed positions (warm: the 109 MB
    working set stays in the 256 MB MALL), graph replays of ten steps whose positions advance by one
    per step, and single steps after a 1 GiB read that evicts the caches (cold), positions advancing."""
    w = decode_workload(pkg, device)
    S, L, H, N, offsets, js, pos = w["S"], w["L"], w["H"], w["N"], w["offsets"], w["js"], w["pos"]
    J = len(offsets)
    qdec, pb, se, pbase, pgain, caches = (w[n] for n in ("qdec", "pos_bias", "scale_embed", "phase_base",
                                                         "phase_gain", "caches"))
    off, qps = w["off"], w["qps"]
    posd = pos.to(device)
    adv = [(pos + i).clamp(max=N - 1).to(torch.int32) for i in range(10)]
    advd = [p.to(device) for p in adv]

    def run(p=posd):
        return pkg.q6.q6_decode(qdec, p, caches, pb, se, pbase, pgain, qps, off, js, J - js, 0)

    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        run()
    b.record()
    torch.cuda.synchronize()
    ms_eager = a.elapsed_time(b) / steps
    ms = graph_ms(run, max(steps, 20), warmup)
    turn = [0]

    def run_adv():
        p = advd[turn[0] % len(advd)]
        turn[0] += 1
        return run(p)

    ms_adv = graph_ms(run_adv, max(steps, 20), warmup)
    flush = CacheFlush(device)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(20)]
    for i, (ea, eb) in enumerate(evs):
        flush()
        ea.record()
        run(advd[i % len(advd)])
        eb.record()
    torch.cuda.synchronize()
    ms_cold = sum(ea.elapsed_time(eb) for ea, eb in evs) / len(evs)
    del flush
    bytes_ = decode_bytes(pos.tolist(), offsets, js, L, H)
    bytes_adv = sum(decode_bytes(p.tolist(), offsets, js, L, H) for p in adv) / len(adv)
    del caches, w
    torch.cuda.empty_cache()
    return {"tokens_per_s": S / (ms * 1e-3), "ms_per_step": ms, "ms_per_step_eager": ms_eager,
            "ms_per_step_advancing": ms_adv, "ms_per_step_cold_advancing": ms_cold,
            "algorithmic_bytes": bytes_, "algorithmic_bytes_advancing": bytes_adv,
            "achieved_GBps": bytes_ / (ms * 1e-3) / 1e9, "hbm_frac": bytes_ / (ms * 1e-3) / HBM_PEAK,
            "hbm_frac_advancing": bytes_adv / (ms_adv * 1e-3) / HBM_PEAK,
            "hbm_frac_cold_advancing": bytes_adv / (ms_cold * 1e-3) / HBM_PEAK,
            "config": "S=256 seqs x L=9 layers x H=8, cache 2048, positions U{96..2047} seed 0; "
                      "bytes count 104 B q6 K+V per valid row + 16 B stored z per valid far row; "
                      "ms_per_step from HIP-graph replays (10 steps per graph) at fixed positions, "
                      "ms_per_step_advancing from replays of 10 steps at positions t..t+9, "
                      "ms_per_step_cold_advancing per step after a 1 GiB read (caches evicted, clean), "
                      "eager launch loop in ms_per_step_eager"}


def q6_prefill_extra(pkg, device, steps, warmup):
    B, H, N = 20, 8, 2048
    t, js, jl = synth(pkg, B, H, N, 3, device)
    kpn = torch.nn.functional.normalize(t["kp"], dim=-1).to(device)
    qpn = torch.nn.functional.normalize(t["qp"], dim=-1).to(device)
    cache = pkg.q6.pack_kv(t["k"], t["v"], kpn)

    def run():
        return pkg.q6.q6_prefill(t["q"], cache, t["pos_bias"], t["scale_embed"], t["phase_base"],
                                 t["phase_gain"], qpn, t["offsets"], js, jl, 0, 1)

    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        run()
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / steps
    bytes_ = B * H * N * (128 + 104 + 16 + 128) + TABLE_BYTES
    return {"tokens_per_s": B * N / (ms * 1e-3), "ms_per_step": ms, "algorithmic_bytes": bytes_,
            "hbm_frac": bytes_ / (ms * 1e-3) / HBM_PEAK,
            "config": "B=20 H=8 T=2048 q6 K/V (+16 B stored z per row), y in-kernel"}


def graph_ms(fn, steps, warmup, reps=10):
    """GPU time per call of fn, from `reps` calls captured in one HIP graph and
    replayed: small launches are timed without the host's launch gaps (how a
    serving loop or a compiled training step runs them)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(reps):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    n = max(1, steps // reps)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(n):
        graph.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / (n * reps)


def phase_probe_extra(pkg, device, steps, warmup):
    """phase_probe_features fwd and bwd (with dprobes) on q of the training microbatch."""
    B, H, N = 15, 8, 2048
    g = torch.Generator().manual_seed(0)
    x = torch.randn(B, H, N, 64, generator=g).to(torch.bfloat16).to(device)
    p = torch.nn.functional.normalize(torch.randn(4, 64, generator=g), dim=-1).to(device)
    dout = torch.randn(B, H, N, 4, generator=g).to(device)
    probe = importlib.import_module("dwarf-v2_amd.probe")
    ms_f = graph_ms(lambda: probe.probe_forward(x, p, 0, N), max(steps, 20), warmup)
    ms_b = graph_ms(lambda: probe.probe_backward(x, p, dout, 0, N, True), max(steps, 20), warmup)
    rows = B * H * N
    fb, bb = rows * (128 + 16), rows * (128 + 16 + 128)
    return {"ms_fwd": ms_f, "ms_bwd": ms_b, "fwd_hbm_frac": fb / (ms_f * 1e-3) / HBM_PEAK,
            "bwd_hbm_frac": bb / (ms_b * 1e-3) / HBM_PEAK, "fwd_bytes": fb, "bwd_bytes": bb,
            "config": "q [15,8,2048,64] bf16, 4 probes; fwd 144 B/row (x + y), bwd 272 B/row (x + dy + dx) "
                      "plus dprobes; timed from HIP-graph replays"}


def probe_fusion_extra(pkg, device, steps, warmup):
    """The DSQG block's y/z (row f1) at the training microbatch: fwd+bwd with autograd through q and k of
    (a) the block's own route, y and z by an fp32 einsum over q and k (dsqg:3231-3254) and the op on them,
    and (b) the op in its probe form (y in the forward kernel, z by the phase-probe kernel, dy and dz folded
    into dq and dk).  Each step is timed by two events on the launch stream (which waits for the backward's
    second stream); medians of `steps` steps."""
    B, H, N = 15, 8, 2048
    t, js, jl = synth(pkg, B, H, N, 0, device)
    qp_raw, kp_raw = t["qp"].to(device), t["kp"].to(device)
    off = t["offsets"]
    tables = [t[n] for n in ("pos_bias", "scale_embed", "phase_base", "phase_gain")]
    leaves = [t[n].detach().clone().requires_grad_(True) for n in ("q", "k", "v")]
    dout = t["dout"]

    def einsum_route():
        q, k, v = leaves
        qp = torch.nn.functional.normalize(qp_raw.float(), dim=-1)
        kp = torch.nn.functional.normalize(kp_raw.float(), dim=-1)
        qf, kf = q.float(), k.float()
        y = (torch.einsum("bhnd,rd->bhnr", qf, qp) * torch.rsqrt(qf.square().sum(-1, keepdim=True) + 64e-6)).contiguous()
        z = (torch.einsum("bhnd,rd->bhnr", kf, kp) * torch.rsqrt(kf.square().sum(-1, keepdim=True) + 64e-6)).contiguous()
        out = pkg.dsqg_attention_v18_grouped(q, k, v, *tables, y, z, js + jl, js, jl, off, None, None, None, None,
                                             None, 3, 0, False, 0, 0, 1)
        out.backward(dout)

    def probe_route():
        q, k, v = leaves
        out = pkg.dsqg_attention_with_probes(q, k, v, *tables, qp_raw, kp_raw, js + jl, js, jl, off, None, None,
                                             None, None, None, 3, 0, False, 0, 0, 1)
        out.backward(dout)

    res = {}
    for name, fn in (("einsum", einsum_route), ("probes_in_kernels", probe_route)):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(max(steps, 10)):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            torch.cuda.synchronize()
            ts.append(a.elapsed_time(b))
        ts.sort()
        res[f"ms_{name}"] = ts[len(ts) // 2]
        for x in leaves:
            x.grad = None
    res["config"] = ("B15 H8 T2048 bf16 fwd+bwd with autograd through q and k; einsum = the block's fp32 einsum "
                     "features then the reference-contract op; probes_in_kernels = dsqg_attention_with_probes")
    return res


def npci_extra(pkg, device, steps, warmup):
    """npci_rotate fwd and bwd (dx, ddelta, dtheta) on the training microbatch's keys: x a [B,N,H,hd] storage
    viewed as [B,H,N,hd], as the DSQG block hands it over, bf16 deltas."""
    B, H, N = 15, 8, 2048
    g = torch.Generator().manual_seed(0)
    x = torch.randn(B, N, H, 64, generator=g).to(torch.bfloat16).to(device).transpose(1, 2)
    d = (0.3 * torch.randn(B, H, N, 64, generator=g)).to(torch.bfloat16).to(device)
    theta = (0.5 * torch.tanh(torch.randn(H, generator=g))).to(device)
    dy = torch.randn(B, H, N, 64, generator=g).to(torch.bfloat16).to(device)
    npci = importlib.import_module("dwarf-v2_amd.npci")
    ms_f = graph_ms(lambda: npci.npci_forward(x, d, theta, 0.25), max(steps, 20), warmup)
    ms_b = graph_ms(lambda: npci.npci_backward(x, d, theta, dy, 0.25), max(steps, 20), warmup)
    rows = B * H * N
    fb, bb = rows * 3 * 128, rows * (5 * 128 + 8)
    return {"ms_fwd": ms_f, "ms_bwd": ms_b, "fwd_hbm_frac": fb / (ms_f * 1e-3) / HBM_PEAK,
            "bwd_hbm_frac": bb / (ms_b * 1e-3) / HBM_PEAK, "fwd_bytes": fb, "bwd_bytes": bb,
            "config": "k [15,8,2048,64] bf16 (head-interleaved storage), bf16 delta, tau 0.25; fwd 384 B/row "
                      "(x + delta + out), bwd 648 B/row (x + delta + dy + dx + ddelta + the per-row dtheta "
                      "term written and read); timed from HIP-graph replays"}


def packet_extra(pkg, device, steps, warmup):
    """The InterferencePacket at the training microbatch, x [15, 2048, 512] bf16 and gate logits of the same
    shape: the fused pool (three EMA timescales and their mix) fwd and bwd; the fused packet (pool + RMS
    direction, confidence and gate, train:262-273) fwd and bwd; beside them the reference's composition on
    this build's kernels (three separate EMA scans and the bf16 mix; the pool followed by PyTorch's
    elementwise packet)."""
    B, N, D = 15, 2048, 512
    g = torch.Generator().manual_seed(0)
    x = torch.randn(B, N, D, generator=g).to(torch.bfloat16).to(device)
    dp = torch.randn(B, N, D, generator=g).to(torch.bfloat16).to(device)
    gate = (1.5 * torch.randn(B, N, D, generator=g)).to(torch.bfloat16).to(device)
    a = torch.tensor([1 / 16, 1 / 64, 1 / 256], device=device)
    w = torch.softmax(torch.tensor([0.3, -0.2, 0.1]), 0).to(device)
    packet = importlib.import_module("dwarf-v2_amd.packet")
    ema = importlib.import_module("dwarf-v2_amd.ema")
    _, state = packet.pool_forward(x, a, w, 1e-5, 0.5)
    ms_f = graph_ms(lambda: packet.pool_forward(x, a, w, 1e-5, 0.5), max(steps, 20), warmup)
    ms_b = graph_ms(lambda: packet.pool_backward(x, a, w, state, dp, 1e-5, 0.5), max(steps, 20), warmup)
    _, pooled, pstate, ms_rows = packet.packet_forward(x, a, w, gate, 1e-5, 0.5)
    ms_pf = graph_ms(lambda: packet.packet_forward(x, a, w, gate, 1e-5, 0.5), max(steps, 20), warmup)
    ms_pb = graph_ms(lambda: packet.packet_backward(x, a, w, gate, pooled, pstate, ms_rows, dp, 1e-5, 0.5),
                     max(steps, 20), warmup)
    wb = w.to(torch.bfloat16)

    def composed():
        scans = [ema.ema_forward(x, a[k:k + 1], 1e-5, 0.5) for k in range(3)]
        return (wb[0] * scans[0] + wb[1] * scans[1]) + wb[2] * scans[2]

    def composed_packet():
        pf = packet.pool_forward(x, a, w, 1e-5, 0.5)[0].float()
        rms = pf.square().mean(-1, keepdim=True).sqrt()
        direction = pf * torch.rsqrt(pf.square().mean(-1, keepdim=True) + 1e-6)
        return (direction * torch.tanh(rms / 0.25) * torch.sigmoid(gate.float())).to(torch.bfloat16)

    ms_c = graph_ms(composed, max(steps, 20), warmup)
    ms_cp = graph_ms(composed_packet, max(steps, 20), warmup)
    n = B * N * D
    fb, bb = 4 * n, 6 * n
    pfb, pbb = 8 * n + 4 * B * N, 12 * n + 4 * B * N
    return {"ms_fwd": ms_f, "ms_bwd": ms_b, "ms_fwd_composed": ms_c,
            "fwd_hbm_frac": fb / (ms_f * 1e-3) / HBM_PEAK, "bwd_hbm_frac": bb / (ms_b * 1e-3) / HBM_PEAK,
            "fwd_bytes": fb, "bwd_bytes": bb,
            "packet_ms_fwd": ms_pf, "packet_ms_bwd": ms_pb, "packet_ms_fwd_composed": ms_cp,
            "packet_fwd_bytes": pfb, "packet_bwd_bytes": pbb,
            "packet_fwd_hbm_frac": pfb / (ms_pf * 1e-3) / HBM_PEAK,
            "packet_bwd_hbm_frac": pbb / (ms_pb * 1e-3) / HBM_PEAK,
            "config": "x and gate logits [15,2048,512] bf16, timescales 16/64/256; algorithmic bytes: pool fwd "
                      "4 B/element (x read, pooled written), pool bwd 6 B/element (dpooled and x read, dx "
                      "written); packet fwd 8 B/element (x and gate read, pooled and packet written) + 4 B/token "
                      "(ms), packet bwd 12 B/element (dpacket, gate, pooled, x read; dgate, dx written) + 4 B/token; "
                      "composed = three EMA scans + bf16 mix, composed packet = fused pool + PyTorch elementwise "
                      "packet; timed from HIP-graph replays"}


def gqa_extra(pkg, device, steps, warmup):
    """The training microbatch with grouped K/V heads: H8 over 2 and over 1 KV heads (the query side, tables and
    dO as benched; K, V and z the first H_kv heads of the benched ones)."""
    B, H, N = 15, 8, 2048
    t, js, jl = synth(pkg, B, H, N, 0, device)
    res = {}
    for hkv in (2, 1):
        u = dict(t)
        for n in ("k", "v", "z_pre"):
            u[n] = t[n][:, :hkv].contiguous()
        ms, per, _ = time_dsqg_step(pkg, u, js, jl, steps, warmup)
        res[f"hkv{hkv}"] = {"tokens_per_s": B * N / (ms * 1e-3), "ms_per_step": ms, "per_launch_ms_serial": per}
        del u
    res["config"] = ("B=15 H=8 T=2048 bf16 DSQG fwd+bwd with H_kv 2 and 1 (GQA groups of 4 and 8); "
                     "step on the overlapped schedule, per-launch times on the serial one")
    return res


def long_context_extra(pkg, device, steps, warmup):
    B, H, N = 4, 8, 8192
    t, js, jl = synth(pkg, B, H, N, 4, device)
    ms_dsqg, _, _ = time_dsqg_step(pkg, t, js, jl, steps, warmup, stages=False)
    del t
    g = torch.Generator().manual_seed(5)
    x = torch.randn(B, N, 512, generator=g).to(torch.bfloat16).to(device)
    dy = torch.randn(B, N, 512, generator=g).to(torch.bfloat16).to(device)
    alpha = (1.0 - (0.90 + 0.099 * torch.rand(512, generator=g))).to(device)
    ema = importlib.import_module("dwarf-v2_amd.ema")

    def run():
        y = ema.ema_forward(x, alpha, 1e-5, 0.5)
        ema.ema_backward(x, y, dy, alpha, 1e-5, 0.5, True)

    ms_ema = graph_ms(run, max(steps, 20), warmup)
    dsqg_bytes = B * H * N * (FWD_BYTES_PER_TH + BWD_BYTES_PER_TH) + 2 * TABLE_BYTES
    ema_bytes = 12 * B * N * 512
    total = ms_dsqg + ms_ema
    return {"tokens_per_s": B * N / (total * 1e-3), "ms_per_step": total, "ms_dsqg": ms_dsqg, "ms_ema": ms_ema,
            "ema_hbm_frac": ema_bytes / (ms_ema * 1e-3) / HBM_PEAK,
            "hbm_frac": (dsqg_bytes + ema_bytes) / (total * 1e-3) / HBM_PEAK,
            "config": "B=4 H=8 T=8192 bf16 DSQG fwd+bwd + EMA fwd+bwd x[4,8192,512], per-channel alpha; "
                      "EMA timed from HIP-graph replays (10 fwd+bwd per graph)"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # untimed steps before the clock starts; the first ~40 training steps of a process run up to 8% slower
    # than the steady state (measured in 20-step windows: 0.60 ms, then 0.575-0.579 ms from step 40 on)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--extra-only", choices=["q6_decode", "q6_prefill", "long_context", "phase_probe", "npci", "packet",
                                             "probe_fusion", "gqa"],
                    help="run only this extra workload and print its JSON (for per-workload profiles)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a 256 MiB device-to-device copy 10 times (scales HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the DSQG op shards over batch/heads with no exchange; no multi-GPU figure is produced)",
              file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    device = torch.device("cuda", 0)
    if args.calibrate_copy:
        src = torch.ones(1 << 28, dtype=torch.uint8, device=device)
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": src.numel(), "launches": 10}))
        return 0
    pkg = importlib.import_module("dwarf-v2_amd")
    pkg._lib.load()
    if args.extra_only:
        fn = {"q6_decode": q6_decode_extra, "q6_prefill": q6_prefill_extra,
              "long_context": long_context_extra, "phase_probe": phase_probe_extra,
              "npci": npci_extra, "packet": packet_extra, "probe_fusion": probe_fusion_extra,
              "gqa": gqa_extra}[args.extra_only]
        print(json.dumps({args.extra_only: fn(pkg, device, args.steps, args.warmup)}), flush=True)
        return 0
    B, H, N = 15, 8, 2048
    log("training microbatch: DSQG fwd+bwd B15 H8 T2048 bf16")
    t, js, jl = synth(pkg, B, H, N, 0, device)
    ms, per, per_o = time_dsqg_step(pkg, t, js, jl, args.steps, args.warmup)
    flush = CacheFlush(device)
    ms_cold, per_cold, per_o_cold = time_dsqg_step(pkg, t, js, jl, max(5, args.steps // 2), 1, flush=flush)
    del flush
    th = B * H * N
    bytes_launch = {"fwd": th * FWD_BYTES_PER_TH + TABLE_BYTES,
                    "bwd_dq": th * DQ_BYTES_PER_TH + TABLE_BYTES,
                    "bwd_params": th * PARAMS_BYTES_PER_TH + TABLE_BYTES,
                    "bwd_delta": th * DELTA_BYTES_PER_TH,
                    "bwd_dkdv": th * DKDV_BYTES_PER_TH + TABLE_BYTES}
    # the roofline's dispatch: the longest one of the schedule the step clock times (overlapped)
    dominant = max(per_o, key=per_o.get)
    achieved = bytes_launch[dominant] / (per_o[dominant] * 1e-3)
    dominant_s = max(per, key=per.get)
    achieved_s = bytes_launch[dominant_s] / (per[dominant_s] * 1e-3)
    path_bytes = th * (FWD_BYTES_PER_TH + BWD_BYTES_PER_TH) + 2 * TABLE_BYTES
    del t
    torch.cuda.empty_cache()

    extra = {"per_launch_ms_overlapped": per_o, "per_launch_ms_overlapped_cold": per_o_cold,
             "per_launch_ms_serial": per, "per_launch_ms_serial_cold": per_cold, "ms_per_step_cold": ms_cold,
             "launch_bytes": bytes_launch,
             "roofline_serial": {"kernel": dominant_s, "achieved": achieved_s / 1e9, "unit": "GB/s",
                                 "frac": achieved_s / HBM_PEAK,
                                 "schedule": "serial: each stage alone on the chip, events between launches"},
             "path_roofline": {"bytes": path_bytes, "achieved_GBps": path_bytes / (ms * 1e-3) / 1e9,
                               "frac": path_bytes / (ms * 1e-3) / HBM_PEAK}}
    if not args.no_extra:
        log("q6 decode step: 256 seqs x 9 layers")
        extra["q6_decode"] = q6_decode_extra(pkg, device, args.steps, args.warmup)
        log("q6 prefill: B20 H8 T2048")
        extra["q6_prefill"] = q6_prefill_extra(pkg, device, args.steps, args.warmup)
        log("long context: B4 T8192 DSQG fwd+bwd + EMA fwd+bwd")
        extra["long_context"] = long_context_extra(pkg, device, args.steps, args.warmup)
        log("phase-probe features: q of the training microbatch")
        extra["phase_probe"] = phase_probe_extra(pkg, device, args.steps, args.warmup)
        log("block y/z: einsum route vs probe features inside the kernels")
        extra["probe_fusion"] = probe_fusion_extra(pkg, device, args.steps, args.warmup)
        log("NPCI rotation: k of the training microbatch")
        extra["npci"] = npci_extra(pkg, device, args.steps, args.warmup)
        log("InterferencePacket pool: x [15,2048,512], three timescales")
        extra["packet"] = packet_extra(pkg, device, args.steps, args.warmup)
        log("training microbatch with grouped K/V heads: H8 over 2 and 1")
        extra["gqa"] = gqa_extra(pkg, device, args.steps, args.warmup)
    # HBM bytes per launch from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE runs (profiles/traffic.json,
    # stamped with the commit they were measured at); counters cannot run inside this timed process
    traffic, traffic_commit = None, None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            tj = json.load(f)
        traffic, traffic_commit = tj.get("overlapped", {}).get(dominant), tj.get("commit")
        extra["roofline_serial"]["traffic"] = tj.get("serial", {}).get(dominant_s)
    line = {
        "metric": "DSQG fwd+bwd tokens/s (B15 T2048 bf16) + % HBM roofline; q6 decode tok/s",
        "value": B * N / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/k/v/dO, reference-calibrated parameter tables)",
        "config": {"workload": "dsqg_fwd_bwd_training_microbatch", "batch": B, "heads": H, "seq_len": N,
                   "head_dim": 64, "offsets": 96, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": dominant, "achieved": achieved / 1e9, "peak": HBM_PEAK / 1e9,
                     "unit": "GB/s", "frac": achieved / HBM_PEAK, "traffic": traffic, "traffic_commit": traffic_commit,
                     "schedule": "overlapped (the timed step): dQ and params on the launch stream, delta and "
                                 "dK/dV on a second stream; duration from events on the kernel's own stream"},
        "extra": extra,
    }
    if not args.no_cpu_baseline:
        log("cpu baseline: oracle cfg2 bf16/fp32 fwd+bwd rows, cfg1 forward, cfg4 EMA")
        line["cpu_baseline"] = cpu_baseline(pkg)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
