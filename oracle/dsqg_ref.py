"""CPU restatement of DSQG attention -- test infrastructure, not the product.

Follows the reference's eager oracle ``_eager_dsqg_attention``
(kernels/dsqg_attention_v22.py:2602-2688) and ``_rotate_sparse_value_eager``
(dsqg:2560-2599):

  score[n,j] = <q[n], k[n-d_j] + e_j> / sqrt(hd) + pos_bias[j,h]   (dsqg:2658-2662)
  for far offsets j >= j_small and planes r with channels (a_r, b_r):
      theta = phase_base[i,h,r] + phase_gain[i,h,r] * y[n,r] * z[n-d_j,r]
      v_a' = cos(theta) v_a - sin(theta) v_b;  v_b' = sin(theta) v_a + cos(theta) v_b
  P = softmax over the offsets with a source (n - d_j >= 0); rows without one
  give out = 0 (dsqg:2683-2688).

plus the GPU path's conventions the kernels also follow: ``round_se`` rounds
the scale embedding to bf16 (dsqg:760-763) with a straight-through gradient
(dsqg:1391, 1466); rows n < query_start give out = 0 and lse = -inf
(dsqg:2265-2268); lse = log sum exp of the scores (dsqg:845-851).

Compute precision: float64 inputs compute in float64, anything else in
float32.  (The reference eager casts scores to float32 even for float64
inputs, dsqg:2659; this restatement keeps float64 so it can be gradchecked.)
Gradients come from autograd through this forward.
"""

from __future__ import annotations

import math
from typing import Sequence

import torch

R_PLANES = 4


def channel_pairs(head_dim: int, plane_shift: int) -> list[tuple[int, int]]:
    """Rotated channel pairs (r*hd/4 + shift, +1), the kernels' form (dsqg:814-815)."""
    seg = head_dim // R_PLANES
    return [(r * seg + plane_shift, r * seg + plane_shift + 1) for r in range(R_PLANES)]


def probe_features(x: torch.Tensor, probes: torch.Tensor) -> torch.Tensor:
    """y/z features (dsqg:3231-3254): <x, p_r/|p_r|> / sqrt(|x|^2 + 1e-6 hd)."""
    xf = x.to(torch.float64 if x.dtype == torch.float64 else torch.float32)
    p = torch.nn.functional.normalize(probes.to(xf.dtype), dim=-1)
    inv = torch.rsqrt(xf.square().sum(-1, keepdim=True) + 1e-6 * x.shape[-1])
    return torch.einsum("bhnd,rd->bhnr", xf, p) * inv


def _straight_through_bf16(x: torch.Tensor) -> torch.Tensor:
    return x + (x.to(torch.bfloat16).to(x.dtype) - x).detach()


def dsqg_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    pos_bias: torch.Tensor,
    scale_embed: torch.Tensor,
    phase_base: torch.Tensor,
    phase_gain: torch.Tensor,
    y_pre: torch.Tensor,
    z_pre: torch.Tensor,
    offsets: Sequence[int],
    j_small: int,
    *,
    plane_shift: int = 0,
    query_start: int = 0,
    round_se: bool = False,
    return_lse: bool = False,
):
    ct = torch.float64 if q.dtype == torch.float64 else torch.float32
    offsets = [int(d) for d in offsets]
    B, H, N, hd = q.shape
    Hkv = k.shape[1]
    head_map = torch.arange(H) // (H // Hkv)
    qf = q.to(ct)
    kx = k.to(ct)[:, head_map]
    vx = v.to(ct)[:, head_map]
    zx = z_pre.to(ct)[:, head_map]
    yf = y_pre.to(ct)
    se = scale_embed.to(ct)
    if round_se:
        se = _straight_through_bf16(se)
    pb = pos_bias.to(ct)
    pbase = phase_base.to(ct)
    pgain = phase_gain.to(ct)
    pairs = channel_pairs(hd, plane_shift)
    scale = 1.0 / math.sqrt(hd)
    pos = torch.arange(N)

    scores, values, valids = [], [], []
    for j, delta in enumerate(offsets):
        src = pos - delta
        valid = (src >= 0) & (src < N) & (pos >= query_start)
        safe = src.clamp(0, N - 1)
        kj = kx[:, :, safe]
        vj = vx[:, :, safe]
        s = (qf * (kj + se[j])).sum(-1) * scale + pb[j].reshape(1, H, 1)
        s = s.masked_fill(~valid.reshape(1, 1, N), float("-inf"))
        if j >= j_small:
            i = j - j_small
            theta = pbase[i].reshape(1, H, 1, R_PLANES) + pgain[i].reshape(1, H, 1, R_PLANES) * yf * zx[:, :, safe]
            cos, sin = torch.cos(theta), torch.sin(theta)
            vj = vj.clone()
            for r, (a, b) in enumerate(pairs):
                va, vb = vj[..., a].clone(), vj[..., b].clone()
                vj[..., a] = cos[..., r] * va - sin[..., r] * vb
                vj[..., b] = sin[..., r] * va + cos[..., r] * vb
        scores.append(s)
        values.append(vj)
        valids.append(valid)

    S = torch.stack(scores, -1)                      # [B,H,N,J]
    V = torch.stack(values, -2)                      # [B,H,N,J,hd]
    valid = torch.stack(valids, -1).reshape(1, 1, N, -1)
    any_valid = valid.any(-1)                        # [1,1,N]
    # Softmax is shift-invariant, so the reference point m carries no gradient.
    m = torch.where(any_valid, S.detach().masked_fill(~valid, float("-inf")).amax(-1), torch.zeros((), dtype=ct))
    P = torch.where(valid, torch.exp(S - m.unsqueeze(-1)), torch.zeros((), dtype=ct))
    l = P.sum(-1)
    denom = torch.where(any_valid, l, torch.ones((), dtype=ct))
    out = (P.unsqueeze(-1) * V).sum(-2) / denom.unsqueeze(-1)
    out = torch.where(any_valid.unsqueeze(-1), out, torch.zeros((), dtype=ct))
    if not return_lse:
        return out
    lse = torch.where(any_valid, m + torch.log(denom), torch.full((), float("-inf"), dtype=ct))
    return out, lse


def dsqg_forward_backward(inputs: dict, offsets, j_small, dout: torch.Tensor, *, delta_from_bf16_out=False, **kw):
    """(out, lse, grads) with grads keyed like the reference's 9 gradient slots (dsqg:2546-2547).

    delta_from_bf16_out: the reference GPU backward forms delta = <dO, O> from
    the bf16 output it stored (dsqg:1263-1289, 2380-2386) rather than the exact
    O.  With eps[n] = <dO[n], bf16(O[n]) - O[n]> held constant, that backward
    is exactly the gradient of <dO, out> - sum_n eps[n] * lse[n], because
    d lse / d score = P; this option evaluates that.
    """
    names = ("q", "k", "v", "pos_bias", "scale_embed", "phase_base", "phase_gain", "y_pre", "z_pre")
    leaves = {n: inputs[n].detach().clone().requires_grad_(True) for n in names}
    out, lse = dsqg_forward(*(leaves[n] for n in names), offsets, j_small, return_lse=True, **kw)
    g = dout.to(out.dtype)
    loss = (out * g).sum()
    if delta_from_bf16_out:
        eps = (g * (out.detach().to(torch.bfloat16).to(out.dtype) - out.detach())).sum(-1)
        loss = loss - (eps * torch.where(torch.isfinite(lse), lse, torch.zeros_like(lse))).sum()
    loss.backward()
    grads = {n: leaves[n].grad for n in names}
    return out.detach(), lse.detach(), grads


def valid_pairs_per_head(offsets: Sequence[int], seq_len: int) -> int:
    """Brute-force count of (n, j) with n - d_j >= 0 (for pinning the index math)."""
    return sum(1 for n in range(seq_len) for d in offsets if n - d >= 0)
