"""The DSQG block's forward with the phase-probe features inside the kernels.

``DSQGAttentionV19.forward`` (kernels/dsqg_attention_v22.py:3144-3284) forms
the MOVT phase features y (from q) and z (from k) with an einsum over fp32
copies of q and k (dsqg:3231-3254) and hands them to the op as y_pre and
z_pre; their backward is a second pass over q and k.  ``dsqg_block_forward``
is a forward for that module: the same attributes, the same arguments and
the same result, with the op called in its probe form
(``dsqg_attention_with_probes``): y formed in the forward kernel from the q
rows it loads, z from the phase-probe kernel over k, and dy / dz added to dq
/ dk inside the backward kernels.  A maintainer binds it as the method::

    DSQGAttentionV19.forward = amd.dsqg_block_forward

Module attributes read (all set by DSQGAttentionV19.__init__, dsqg:2790-2978):
num_heads, head_dim, minimum_offset, support_crop_projections,
support_crop_min_offset, qkvg_proj, npci_theta_k, npci_theta_v,
npci_strength_tau, query_probes, key_probes, phase_gate, pos_bias,
centered_scale_embed, phase_base, phase_gain, j_val, j_small, j_large,
offsets_dev, the five sparse-plan buffers, k_group_size, grouped_mode_id,
verify_mode, max_group_spread_observed, plane_shift, backend,
online_softmax, if_gain, out_proj, dropout.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from .dsqg import dsqg_attention_with_probes
from .npci import npci_rotate

NPCI_THETA_MAX = 0.25   # bound of the NPCI rotation angle, theta = 0.25 tanh(raw) (dsqg:71, 3216, 3222)


def _projections(block, x: torch.Tensor, query_start: int, key_end: int):
    """q, k, v and the content gate, each [B, N, D].

    With support cropping (dsqg:3158-3187) only the rows that can take part
    are projected: q and the gate for rows >= query_start (no offset reaches
    an earlier query), k and v for rows < key_end (no query reaches a later
    source); the other rows are zero.  Otherwise one fused projection.
    """
    D = x.shape[-1]
    crop = block.support_crop_projections and query_start >= block.support_crop_min_offset
    if not crop:
        return block.qkvg_proj(x).split(D, dim=-1)
    w, b = block.qkvg_proj.weight, block.qkvg_proj.bias
    q, k, v, gate = (x.new_zeros(x.shape) for _ in range(4))
    tail, head = x[:, query_start:], x[:, :key_end]
    q[:, query_start:] = F.linear(tail, w[:D], b[:D])
    gate[:, query_start:] = F.linear(tail, w[3 * D:], b[3 * D:])
    kv = F.linear(head, w[D:3 * D], b[D:3 * D])
    k[:, :key_end], v[:, :key_end] = kv[..., :D], kv[..., D:]
    return q, k, v, gate


def _inject(block, k: torch.Tensor, v: torch.Tensor, kv_inject, key_end: int):
    """NPCI rotation of the live key/value prefix by the injected deltas (dsqg:3196-3229).

    The deltas are full [B,H,N,hd] tensors (their first key_end rows are
    used) or exactly the live prefix [B,H,key_end,hd]; anything else raises
    ValueError.  Rows >= key_end are kept as they are.
    """
    dk, dv = kv_inject
    B, H, N, hd = k.shape
    if dk.shape == k.shape and dv.shape == k.shape:
        dk, dv = dk[:, :, :key_end], dv[:, :, :key_end]
    elif not (dk.shape == (B, H, key_end, hd) and dv.shape == (B, H, key_end, hd)):
        raise ValueError("kv_inject must contain full [B,H,N,HD] tensors or the "
                         "exact live source prefix [B,H,N-min_offset,HD]")
    tau = block.npci_strength_tau
    rk = npci_rotate(k[:, :, :key_end], dk, NPCI_THETA_MAX * torch.tanh(block.npci_theta_k), strength_tau=tau)
    rv = npci_rotate(v[:, :, :key_end], dv, NPCI_THETA_MAX * torch.tanh(block.npci_theta_v), strength_tau=tau)
    if key_end == N:
        return rk, rv
    return torch.cat((rk, k[:, :, key_end:]), dim=2), torch.cat((rv, v[:, :, key_end:]), dim=2)


def dsqg_block_forward(block, x: torch.Tensor, kv_inject=None) -> torch.Tensor:
    """DSQGAttentionV19.forward (dsqg:3144-3284) with y/z and their gradients inside the kernels.

    x [B, N, D] -> [B, N, D].  When no offset has a source at this length the
    result is zeros (dsqg:3153-3156).
    """
    B, N, D = x.shape
    H, hd = block.num_heads, block.head_dim
    query_start = min(block.minimum_offset, N)
    if query_start >= N:
        return torch.zeros_like(x)
    key_end = max(0, N - query_start)
    q, k, v, gate = _projections(block, x, query_start, key_end)
    # [B, N, H*hd] -> [B, H, N, hd] views over the projection rows
    q, k, v = (t.reshape(B, N, H, hd).permute(0, 2, 1, 3) for t in (q, k, v))
    if kv_inject is not None:
        k, v = _inject(block, k, v, kv_inject, key_end)
    phase_gate = torch.sigmoid(block.phase_gate)[:, None, None]
    out = dsqg_attention_with_probes(
        q, k, v, block.pos_bias, block.centered_scale_embed, block.phase_base * phase_gate,
        block.phase_gain * phase_gate, block.query_probes, block.key_probes, block.j_val, block.j_small,
        block.j_large, block.offsets_dev, block.sparse_order_dev, block.group_start_dev, block.group_len_dev,
        block.group_dmin_dev, block.group_dmax_dev, block.k_group_size, block.grouped_mode_id, block.verify_mode,
        block.max_group_spread_observed, block.plane_shift, query_start, backend=block.backend,
        online_softmax=block.online_softmax)
    out = out * block.if_gain.reshape(1, H, 1, 1)
    merged = out.permute(0, 2, 1, 3).reshape(B, N, D)
    return block.dropout(block.out_proj(merged * torch.sigmoid(gate)))
