"""GPU parity of ``dsqg_block_forward``, the DSQG block's forward with y/z inside the kernels (MI355X).

The module is a stand-in that carries the attributes DSQGAttentionV19 sets
(dsqg:2790-2978) with seeded values; the block runs in bf16 as under the
trainer's autocast (train:1128).  The oracle restates DSQGAttentionV19.forward
(dsqg:3144-3284) on the CPU in float64: the projections (cropped to the
support rows when the minimum offset reaches support_crop_min_offset,
dsqg:3158-3187), rounded to bf16 as the GPU's bf16 projections are; the NPCI
rotation of the live key/value prefix (``oracle/npci_ref.py``); the block's
y/z einsum (``dsqg_ref.probe_features``); the op (``dsqg_ref.dsqg_forward``,
bf16 scale embeddings); the head gain, the content gate and the output
projection.  Gradients come from autograd through that restatement.

The fp32 block (no autocast) takes the op's fp32 route and is held to 1e-5
relative on everything; the bf16 block to 2e-2 max-abs on the output and dx
and 2e-2 of the largest magnitude on the parameter gradients (sums over every
token).
"""

from __future__ import annotations

import pytest
import torch
import torch.nn as nn

from oracle import dsqg_ref, npci_ref
from tests.dsqg_cases import orthogonal_probes

pytestmark = pytest.mark.gpu


class StandInBlock(nn.Module):
    """The attributes DSQGAttentionV19.forward reads, with seeded values."""

    def __init__(self, D, H, offsets, js, shift, crop_min, seed):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        hd = D // H
        J, jl = len(offsets), max(len(offsets) - js, 1)
        self.num_heads, self.head_dim = H, hd
        self.minimum_offset = min(offsets)
        self.support_crop_projections, self.support_crop_min_offset = True, crop_min
        self.qkvg_proj = nn.Linear(D, 4 * D, bias=True)
        self.out_proj = nn.Linear(D, D, bias=False)
        with torch.no_grad():
            self.qkvg_proj.weight.copy_(torch.randn(4 * D, D, generator=g) / D ** 0.5)
            self.qkvg_proj.bias.copy_(0.1 * torch.randn(4 * D, generator=g))
            self.out_proj.weight.copy_(torch.randn(D, D, generator=g) / D ** 0.5)
        self.npci_theta_k = nn.Parameter(0.8 * torch.randn(H, generator=g))
        self.npci_theta_v = nn.Parameter(0.8 * torch.randn(H, generator=g))
        self.npci_strength_tau = 0.25
        qp, kp = orthogonal_probes(hd, shift)
        self.query_probes = nn.Parameter(qp + 0.2 * torch.randn(qp.shape, generator=g), requires_grad=False)
        self.key_probes = nn.Parameter(kp + 0.2 * torch.randn(kp.shape, generator=g), requires_grad=False)
        self.phase_gate = nn.Parameter(torch.randn(jl, generator=g))
        self.pos_bias = nn.Parameter(0.02 * torch.randn(J, H, generator=g))
        self.centered_scale_embed = nn.Parameter(0.01 * torch.randn(J, hd, generator=g))
        self.phase_base = nn.Parameter(0.05 * torch.randn(jl, H, 4, generator=g))
        self.phase_gain = nn.Parameter(4.0 * torch.randn(jl, H, 4, generator=g))
        self.if_gain = nn.Parameter(1.0 + 0.2 * torch.randn(H, generator=g))
        self.j_val, self.j_small, self.j_large = J, js, J - js
        self.register_buffer("offsets_dev", torch.tensor(offsets, dtype=torch.int32))
        self.sparse_order_dev = self.group_start_dev = self.group_len_dev = None
        self.group_dmin_dev = self.group_dmax_dev = None
        self.k_group_size, self.grouped_mode_id, self.verify_mode, self.max_group_spread_observed = 3, 0, False, 0
        self.plane_shift, self.backend, self.online_softmax = shift, "auto", True
        self.dropout = nn.Dropout(0.0)


PARAMS = ("qkvg_proj.weight", "qkvg_proj.bias", "out_proj.weight", "npci_theta_k", "npci_theta_v", "phase_gate",
          "pos_bias", "centered_scale_embed", "phase_base", "phase_gain", "if_gain")


def _round(t, bf16):
    """bf16 rounding with a straight-through gradient where the GPU's bf16 autocast rounds; else t."""
    return t + (t.to(torch.bfloat16).to(t.dtype) - t).detach() if bf16 else t


def block_oracle(p, x, kv, blk, bf16):
    """DSQGAttentionV19.forward (dsqg:3144-3284) in float64 from the parameter dict p; with bf16, the
    roundings of bf16 autocast: linear layers take bf16 weights and inputs and give bf16 outputs, the
    sigmoid of the bf16 gate is bf16, and the op and the NPCI rotation return bf16."""
    def _bf16(t):
        return _round(t, bf16)

    B, N, D = x.shape
    H, hd = blk.num_heads, blk.head_dim
    qs = min(blk.minimum_offset, N)
    ke = N - qs
    W, b = _bf16(p["qkvg_proj.weight"]), _bf16(p["qkvg_proj.bias"])
    full = _bf16(x) @ W.t() + b
    q, k, v, gate = (_bf16(t) for t in full.split(D, dim=-1))
    if blk.support_crop_projections and qs >= blk.support_crop_min_offset:
        rows = torch.arange(N).view(1, N, 1)
        q, gate = q * (rows >= qs), gate * (rows >= qs)
        k, v = k * (rows < ke), v * (rows < ke)
    q, k, v = (t.reshape(B, N, H, hd).permute(0, 2, 1, 3) for t in (q, k, v))
    if kv is not None:
        kd, vd = kv[0].double()[:, :, :ke], kv[1].double()[:, :, :ke]
        rk = _bf16(npci_ref.npci_rotate(k[:, :, :ke], kd, 0.25 * torch.tanh(p["npci_theta_k"]), 0.25))
        rv = _bf16(npci_ref.npci_rotate(v[:, :, :ke], vd, 0.25 * torch.tanh(p["npci_theta_v"]), 0.25))
        k, v = torch.cat((rk, k[:, :, ke:]), 2), torch.cat((rv, v[:, :, ke:]), 2)
    y = dsqg_ref.probe_features(q, blk.query_probes.detach().double())
    z = dsqg_ref.probe_features(k, blk.key_probes.detach().double())
    pg = torch.sigmoid(p["phase_gate"])[:, None, None]
    out = dsqg_ref.dsqg_forward(q, k, v, p["pos_bias"], p["centered_scale_embed"], p["phase_base"] * pg,
                                p["phase_gain"] * pg, y, z, blk.offsets_dev.tolist(), blk.j_small,
                                plane_shift=blk.plane_shift, query_start=qs, round_se=bf16)
    out = _bf16(out) * p["if_gain"].reshape(1, H, 1, 1)
    merged = out.permute(0, 2, 1, 3).reshape(B, N, D)
    return _bf16(_bf16(merged * _bf16(torch.sigmoid(gate))) @ _bf16(p["out_proj.weight"]).t())


def _lattice(pkg, name):
    if name == "canonical":
        return list(pkg.ALL_OFFSETS), 17, 3
    return [64, 96, 128, 200, 333], 0, 5


def _compare(pkg, device, lattice, inject, dtype, bar_out, bar_param):
    offsets, js, shift = _lattice(pkg, lattice)
    B, N, D, H = 2, 300, 256, 4
    blk = StandInBlock(D, H, offsets, js, shift, 64, seed=90 + js)   # for the oracle's settings
    g = torch.Generator().manual_seed(91)
    x = torch.randn(B, N, D, generator=g).to(dtype)
    dy = torch.randn(B, N, D, generator=g).to(dtype)
    kv = None
    if inject:
        kv = (torch.randn(B, H, N, 64, generator=g).to(dtype), torch.randn(B, H, N, 64, generator=g).to(dtype))
    bf16 = dtype == torch.bfloat16
    # the GPU block: fp32 parameters; bf16 runs under bf16 autocast (the trainer's setting, train:1128)
    gblk = StandInBlock(D, H, offsets, js, shift, 64, seed=90 + js).to(device)
    xg = x.to(device).requires_grad_(True)
    kvg = None if kv is None else tuple(t.to(device) for t in kv)
    with torch.autocast("cuda", dtype=torch.bfloat16, enabled=bf16):
        out = pkg.dsqg_block_forward(gblk, xg, kvg)
    out.backward(dy.to(device))
    torch.cuda.synchronize()
    assert out.dtype == dtype
    # the oracle on the same parameters, in float64
    named = dict(gblk.named_parameters())
    p = {n: named[n].detach().double().cpu().requires_grad_(True) for n in PARAMS}
    xo = x.double().requires_grad_(True)
    ro = block_oracle(p, xo, kv, blk, bf16)
    (ro * dy.double()).sum().backward()

    def rel(a, b):
        return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))

    errs = {"out": (out.detach().double().cpu(), ro.detach()), "dx": (xg.grad.double().cpu(), xo.grad)}
    for n, (a, b) in errs.items():
        e = float((a - b).abs().max()) if bf16 else rel(a, b)
        assert e < bar_out, (n, e)
    for n in PARAMS:
        ref = p[n].grad
        if named[n].grad is None:   # a parameter that takes no part (NPCI angles without kv_inject)
            assert ref is None or not bool(ref.any()), n
            continue
        e = rel(named[n].grad.double().cpu(), ref)
        assert e < bar_param, (n, e)


@pytest.mark.parametrize("lattice", ["canonical", "far"])
def test_block_forward_bf16_probes_in_kernels(pkg, device, lattice):
    """bf16 under autocast: the op in its probe form (y/z and their gradients inside the kernels).
    canonical: the 96-offset lattice (minimum offset 1, no cropping).  far: offsets >= 64 only (support
    cropping on: q/gate rows before 64 and k/v rows past N - 64 are never projected).  Bars: out and dx 2e-2
    max-abs; parameter gradients 2e-2 of their largest magnitude."""
    _compare(pkg, device, lattice, False, torch.bfloat16, 2e-2, 2e-2)


def test_block_forward_fp32_crop_and_kv_inject(pkg, device):
    """fp32 (the phase-probe kernels and the fp32 op), the far lattice with support cropping and a full-shape
    kv_inject through the NPCI rotation of the live key/value prefix: out, dx and every parameter gradient
    within 1e-5 relative of the float64 restatement."""
    _compare(pkg, device, "far", True, torch.float32, 1e-5, 1e-5)
