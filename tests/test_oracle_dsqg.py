"""Pin the CPU DSQG oracle before trusting it (no GPU).

  * golden vectors written from the reference's own eager oracle
    (tests/golden/make_golden.py -> kernels/dsqg_attention_v22.py:2602-2688),
    forward and all nine gradients, with data-dependent MOVT angles and GQA;
  * MOVT off: equal to PyTorch's scaled_dot_product_attention with a dense
    additive mask that holds pos_bias + <q, e_j>/sqrt(hd) on the lattice
    diagonals (a textbook routine fixes gather, mask and softmax);
  * constant MOVT angle: equal to the same SDPA with V's channel pairs
    rotated beforehand (fixes channel choice and rotation sign);
  * one-hot selection, rows before query_start, log-sum-exp, causality;
  * float64 gradcheck of the backward.
"""

import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import dsqg_ref
from tests.conftest import GOLDEN

NAMES = ("q", "k", "v", "pos_bias", "scale_embed", "phase_base", "phase_gain", "y_pre", "z_pre")


def rel(a, b):
    a, b = torch.as_tensor(a, dtype=torch.float64), torch.as_tensor(b, dtype=torch.float64)
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


@pytest.mark.parametrize("case", ["movt_small", "gqa", "lattice96"])
def test_oracle_matches_reference_golden(case):
    data = np.load(os.path.join(GOLDEN, f"dsqg_eager_{case}.npz"))
    B, H, Hkv, N, hd, js, jl, shift = [int(x) for x in data["meta"]]
    inputs = {n: torch.from_numpy(data[f"in_{n}"]) for n in NAMES}
    out, lse, grads = dsqg_ref.dsqg_forward_backward(
        inputs, data["offsets"].tolist(), js, torch.from_numpy(data["dout"]), plane_shift=shift
    )
    # The reference eager evaluates scores and rotations in float32 (dsqg:2659, 2669).
    assert rel(out, data["out"]) < 1e-6
    for n in NAMES:
        assert rel(grads[n], data[f"grad_{n}"]) < 2e-6, n


def _random_inputs(B, H, Hkv, N, hd, J, j_small, seed, dtype=torch.float64, gain=1.0):
    g = torch.Generator().manual_seed(seed)
    jl = max(J - j_small, 1)
    return dict(
        q=torch.randn(B, H, N, hd, generator=g, dtype=dtype),
        k=torch.randn(B, Hkv, N, hd, generator=g, dtype=dtype),
        v=torch.randn(B, Hkv, N, hd, generator=g, dtype=dtype),
        pos_bias=0.3 * torch.randn(J, H, generator=g, dtype=dtype),
        scale_embed=0.2 * torch.randn(J, hd, generator=g, dtype=dtype),
        phase_base=0.5 * torch.randn(jl, H, 4, generator=g, dtype=dtype),
        phase_gain=gain * torch.randn(jl, H, 4, generator=g, dtype=dtype),
        y_pre=torch.rand(B, H, N, 4, generator=g, dtype=dtype) * 2 - 1,
        z_pre=torch.rand(B, Hkv, N, 4, generator=g, dtype=dtype) * 2 - 1,
    )


def _sdpa_reference(x, offsets, value=None):
    """Dense-mask SDPA: mask[n, n-d_j] = pos_bias[j,h] + <q[n], e_j>/sqrt(hd)."""
    q, k = x["q"], x["k"]
    v = x["v"] if value is None else value
    B, H, N, hd = q.shape
    c = 1.0 / math.sqrt(hd)
    mask = torch.full((B, H, N, N), float("-inf"), dtype=q.dtype)
    n = torch.arange(N)
    for j, d in enumerate(offsets):
        rows = n[n >= d]
        qe = (q[:, :, rows] * x["scale_embed"][j]).sum(-1) * c
        mask[:, :, rows, rows - d] = x["pos_bias"][j].reshape(1, H, 1) + qe
    has = torch.isfinite(mask).any(-1, keepdim=True)
    safe = torch.where(has, mask, torch.zeros_like(mask))
    out = F.scaled_dot_product_attention(q, k, v, attn_mask=safe, scale=c)
    return torch.where(has, out, torch.zeros_like(out))


def test_movt_off_equals_masked_sdpa():
    offsets = [1, 2, 3, 5, 8, 13, 48, 50, 64]
    x = _random_inputs(2, 3, 3, 70, 16, len(offsets), 6, seed=1)
    x["phase_base"].zero_()
    x["phase_gain"].zero_()
    out = dsqg_ref.dsqg_forward(*(x[n] for n in NAMES), offsets, 6)
    ref = _sdpa_reference(x, offsets)
    assert rel(out, ref) < 1e-12


def test_constant_angle_equals_prerotated_sdpa():
    offsets = [48, 50, 57, 64, 70]           # all far: every offset is rotated
    shift = 2
    x = _random_inputs(1, 2, 2, 90, 16, len(offsets), 0, seed=2)
    theta = torch.randn(2, 4, dtype=torch.float64)       # per (h, plane), same for every offset
    x["phase_base"] = theta.unsqueeze(0).expand(len(offsets), 2, 4).contiguous()
    x["phase_gain"].zero_()
    out = dsqg_ref.dsqg_forward(*(x[n] for n in NAMES), offsets, 0, plane_shift=shift)
    v = x["v"].clone()
    seg = 16 // 4
    for r in range(4):
        a, b = r * seg + shift, r * seg + shift + 1
        c, s = torch.cos(theta[:, r]).reshape(1, 2, 1), torch.sin(theta[:, r]).reshape(1, 2, 1)
        va, vb = x["v"][..., a], x["v"][..., b]
        v[..., a] = c * va - s * vb
        v[..., b] = s * va + c * vb
    ref = _sdpa_reference(x, offsets, value=v)
    assert rel(out, ref) < 1e-12


def test_single_offset_selects_source_row():
    for d in (1, 5):
        x = _random_inputs(1, 2, 2, 20, 8, 1, 1, seed=3)
        out = dsqg_ref.dsqg_forward(*(x[n] for n in NAMES), [d], 1)
        assert torch.equal(out[:, :, :d], torch.zeros_like(out[:, :, :d]))
        assert torch.equal(out[:, :, d:], x["v"][:, :, : 20 - d])


def test_dominant_bias_selects_offset():
    offsets = [1, 2, 4, 7]
    x = _random_inputs(1, 1, 1, 30, 8, 4, 4, seed=4)
    x["pos_bias"][:] = 0.0
    x["pos_bias"][2, 0] = 1e4               # offset 4 wins wherever it is valid
    out = dsqg_ref.dsqg_forward(*(x[n] for n in NAMES), offsets, 4)
    assert torch.allclose(out[0, 0, 4:], x["v"][0, 0, :26], atol=0, rtol=0)


def test_query_start_rows_and_lse():
    offsets = [1, 3, 48]
    x = _random_inputs(1, 2, 2, 60, 8, 3, 2, seed=5)
    out, lse = dsqg_ref.dsqg_forward(*(x[n] for n in NAMES), offsets, 2, query_start=6, return_lse=True)
    assert torch.equal(out[:, :, :6], torch.zeros_like(out[:, :, :6]))
    assert torch.isinf(lse[:, :, :6]).all() and (lse[:, :, :6] < 0).all()
    # brute-force log-sum-exp of the valid scores for one row
    n, h = 50, 1
    c = 1 / math.sqrt(8)
    s = [float((x["q"][0, h, n] * (x["k"][0, h, n - d] + x["scale_embed"][j])).sum() * c + x["pos_bias"][j, h])
         for j, d in enumerate(offsets) if n - d >= 0]
    assert abs(float(lse[0, h, n]) - math.log(sum(math.exp(v) for v in s))) < 1e-12


def test_causality():
    offsets = [1, 2, 5, 48]
    x = _random_inputs(1, 2, 1, 64, 8, 4, 3, seed=6, gain=2.0)
    base = dsqg_ref.dsqg_forward(*(x[n] for n in NAMES), offsets, 3)
    y = {n: t.clone() for n, t in x.items()}
    for n in ("q", "k", "v", "y_pre", "z_pre"):
        y[n][:, :, 40:] += 10 * torch.randn_like(y[n][:, :, 40:])
    moved = dsqg_ref.dsqg_forward(*(y[n] for n in NAMES), offsets, 3)
    assert torch.equal(base[:, :, :40], moved[:, :, :40])


def test_gradcheck_float64():
    offsets = [1, 2, 3, 4]
    x = _random_inputs(1, 2, 1, 9, 8, 4, 2, seed=7, gain=1.5)
    leaves = [x[n].clone().requires_grad_(True) for n in NAMES]

    def fn(*args):
        return dsqg_ref.dsqg_forward(*args, offsets, 2, query_start=1)

    assert torch.autograd.gradcheck(fn, leaves, eps=1e-6, atol=1e-7)


def test_round_se_is_straight_through():
    offsets = [1, 2, 48]
    x = _random_inputs(1, 1, 1, 55, 8, 3, 2, seed=8)
    x["scale_embed"] = x["scale_embed"] * 3.7
    rounded = dict(x)
    rounded["scale_embed"] = x["scale_embed"].to(torch.bfloat16).to(torch.float64)
    a = dsqg_ref.dsqg_forward(*(x[n] for n in NAMES), offsets, 2, round_se=True)
    b = dsqg_ref.dsqg_forward(*(rounded[n] for n in NAMES), offsets, 2)
    assert torch.equal(a, b)
    dout = torch.randn_like(a)
    _, _, g1 = dsqg_ref.dsqg_forward_backward(x, offsets, 2, dout, round_se=True)
    _, _, g2 = dsqg_ref.dsqg_forward_backward(rounded, offsets, 2, dout)
    assert rel(g1["scale_embed"], g2["scale_embed"]) < 1e-14


def test_delta_from_bf16_out_matches_explicit_formula():
    """The surrogate-loss form of the GPU convention equals the explicit
    dS = P (g - <dO, bf16(O)>) backward, checked on dpos_bias = sum_n dS."""
    offsets = [1, 2, 5, 48]
    x = _random_inputs(1, 2, 2, 40, 8, 4, 3, seed=9, gain=1.0)
    dout = torch.randn(1, 2, 40, 8, dtype=torch.float64)
    out, lse, g = dsqg_ref.dsqg_forward_backward(x, offsets, 3, dout, delta_from_bf16_out=True)
    o16 = out.to(torch.bfloat16).to(torch.float64)
    delta = (dout * o16).sum(-1)
    c = 1 / math.sqrt(8)
    expect = torch.zeros(4, 2, dtype=torch.float64)
    pairs = dsqg_ref.channel_pairs(8, 0)
    for j, d in enumerate(offsets):
        for n in range(d, 40):
            for h in range(2):
                s = float((x["q"][0, h, n] * (x["k"][0, h, n - d] + x["scale_embed"][j])).sum() * c + x["pos_bias"][j, h])
                P = math.exp(s - float(lse[0, h, n]))
                v = x["v"][0, h, n - d].clone()
                if j >= 3:
                    for r, (a, b) in enumerate(pairs):
                        th = float(x["phase_base"][j - 3, h, r] + x["phase_gain"][j - 3, h, r]
                                   * x["y_pre"][0, h, n, r] * x["z_pre"][0, h, n - d, r])
                        va, vb = float(v[a]), float(v[b])
                        v[a], v[b] = math.cos(th) * va - math.sin(th) * vb, math.sin(th) * va + math.cos(th) * vb
                gd = float((dout[0, h, n] * v).sum())
                expect[j, h] += P * (gd - float(delta[0, h, n]))
    assert rel(g["pos_bias"], expect) < 1e-12
