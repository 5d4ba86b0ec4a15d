"""CPU restatement of the causal EMA scan -- test infrastructure, not the product.

Follows the reference recurrence (kernels/causal_ema_scan.py:3-11) and its
eager ``_reference`` (ema:511-538): a = clamp(alpha, floor, ceiling),
y[t] = a x[t] + (1 - a) y[t-1], y[-1] = 0, with float64 state for float64
inputs and float32 state otherwise.  alpha may be one value or one per
channel ([D]); ``_reference`` broadcasts a [D] alpha the same way.  An
optional reset_mask [B,N] zeroes the state before the tokens it marks
(ema:368-509, 533-535).  ``interference_pool`` and its backward restate the
InterferencePacket's K scans of one input and their weighted sum
(train/train_dwarf.py:260-267) on top of these, and ``packet_from_pooled``
the packet that InterferencePacket.forward forms from the pool
(train:268-273), differentiable so its gradients come from autograd.
"""

from __future__ import annotations

import torch


def ema_scan(x: torch.Tensor, alpha: torch.Tensor, floor: float = 1e-5, ceiling: float = 0.5,
             reset_mask: torch.Tensor | None = None) -> torch.Tensor:
    """reset_mask [B,N] bool: the state is zeroed before token t where set (ema:533-535)."""
    acc = torch.float64 if x.dtype == torch.float64 else torch.float32
    a = alpha.to(acc).clamp(floor, ceiling).reshape(-1)
    decay = 1.0 - a
    xf = x.to(acc)
    state = torch.zeros(x.shape[0], x.shape[2], dtype=acc)
    rows = []
    for t in range(x.shape[1]):
        if reset_mask is not None:
            state = torch.where(reset_mask[:, t, None], torch.zeros_like(state), state)
        state = a * xf[:, t] + decay * state
        rows.append(state)
    if not rows:
        return torch.empty_like(x)
    return torch.stack(rows, dim=1).to(x.dtype)


def ema_closed_form(x: torch.Tensor, alpha: torch.Tensor) -> torch.Tensor:
    """y[t] = sum_{s<=t} a (1-a)^(t-s) x[s], evaluated directly in float64 (alpha unclamped)."""
    x64 = x.to(torch.float64)
    a = alpha.to(torch.float64).reshape(-1)
    N = x.shape[1]
    t = torch.arange(N, dtype=torch.float64)
    lag = (t[:, None] - t[None, :])                      # [t, s]
    mask = lag >= 0
    w = torch.where(mask[..., None], a * (1 - a) ** lag.clamp(min=0)[..., None], torch.zeros((), dtype=torch.float64))
    return torch.einsum("tsd,bsd->btd", w, x64)


def ema_adjoint(x: torch.Tensor, y: torch.Tensor, dy: torch.Tensor, alpha: torch.Tensor,
                floor: float = 1e-5, ceiling: float = 0.5, reset_mask: torch.Tensor | None = None):
    """Reverse adjoint (ema:3-11): lambda[t] = dy[t] + (1-a) lambda[t+1], dx = a lambda,
    dalpha = sum lambda[t] (x[t] - y[t-1]); dalpha per channel summed over batch and time,
    then zeroed where the clamp blocks it (ema:357-364).  With reset_mask
    (ema:427-451): lambda[t+1] is cut where token t+1 resets, and y[t-1] is 0
    where token t resets."""
    acc = torch.float64 if x.dtype == torch.float64 else torch.float32
    a_in = alpha.to(acc).reshape(-1)
    a = a_in.clamp(floor, ceiling)
    xf, yf, g = x.to(acc), y.to(acc), dy.to(acc)
    B, N, D = x.shape
    lam = torch.zeros(B, D, dtype=acc)
    dx = torch.zeros(B, N, D, dtype=acc)
    da = torch.zeros(B, D, dtype=acc)
    zero = torch.zeros(B, D, dtype=acc)
    for t in range(N - 1, -1, -1):
        if reset_mask is not None and t + 1 < N:
            lam = torch.where(reset_mask[:, t + 1, None], zero, lam)
        lam = g[:, t] + (1 - a) * lam
        dx[:, t] = a * lam
        prev = yf[:, t - 1] if t > 0 else zero
        if reset_mask is not None:
            prev = torch.where(reset_mask[:, t, None], zero, prev)
        da += lam * (xf[:, t] - prev)
    da = da.sum(0)
    if a_in.numel() == 1:
        da = da.sum().reshape(1)
    blocked = ((a_in <= floor) & (da > 0)) | ((a_in >= ceiling) & (da < 0))
    da = torch.where(blocked, torch.zeros_like(da), da)
    return dx, da


def interference_pool(x: torch.Tensor, factors: torch.Tensor, weights: torch.Tensor, floor: float = 1e-5,
                      ceiling: float = 0.5) -> torch.Tensor:
    """The InterferencePacket's pooled scans (train:262-267): scan_k = ema_scan(x, factor_k) in x's dtype,
    pooled = ((w_0 scan_0 + w_1 scan_1) + ...) with w_k cast to x's dtype and each product and partial
    sum evaluated in x's dtype, as the reference's tensor arithmetic does."""
    dt = x.dtype
    pooled = None
    for f, w in zip(factors.reshape(-1), weights.reshape(-1)):
        term = w.to(dt) * ema_scan(x, f.reshape(1), floor, ceiling)
        pooled = term if pooled is None else pooled + term
    return pooled


def interference_pool_backward(x: torch.Tensor, factors: torch.Tensor, weights: torch.Tensor,
                               dpooled: torch.Tensor, floor: float = 1e-5, ceiling: float = 0.5):
    """(dx, dfactors [K], dweights [K]) of ``interference_pool`` for the output gradient ``dpooled``.

    The gradient of scan_k is dpooled * w_k in x's dtype; each scan's adjoint is ``ema_adjoint`` with
    its own clamp projection; dx is the sum over the scans in the accumulation dtype, rounded once to
    x's dtype (the reference's autograd adds the K bf16 gradients one by one: the two differ by bf16
    rounding only); dweight_k = sum of (dpooled * scan_k) in x's dtype, accumulated in the accumulation
    dtype and rounded to x's dtype, as a bf16 sum-reduction returns it."""
    dt = x.dtype
    acc = torch.float64 if dt == torch.float64 else torch.float32
    g = dpooled.to(dt)
    dx = torch.zeros(x.shape, dtype=acc)
    dfs, dws = [], []
    for f, w in zip(factors.reshape(-1), weights.reshape(-1)):
        scan = ema_scan(x, f.reshape(1), floor, ceiling)
        dxk, dak = ema_adjoint(x, scan, g * w.to(dt), f.reshape(1), floor, ceiling)
        dx += dxk
        dfs.append(dak.reshape(()))
        dws.append((g * scan).to(acc).sum().to(dt).to(acc))
    return dx.to(dt), torch.stack(dfs), torch.stack(dws)


def packet_from_pooled(pooled: torch.Tensor, gate_logits: torch.Tensor, out_dtype: torch.dtype) -> torch.Tensor:
    """train:268-273: with u = pooled in fp32 (fp64 for fp64 input), rms = sqrt(mean u^2),
    direction = u rsqrt(mean u^2 + 1e-6), confidence = tanh(rms / 0.25), gate = sigmoid(logits),
    packet = (direction * confidence * gate) cast to out_dtype."""
    acc = torch.float64 if pooled.dtype == torch.float64 else torch.float32
    u = pooled.to(acc)
    rms = u.square().mean(-1, keepdim=True).sqrt()
    direction = u * torch.rsqrt(u.square().mean(-1, keepdim=True) + 1e-6)
    confidence = torch.tanh(rms / 0.25)
    gate = torch.sigmoid(gate_logits.to(acc))
    return (direction * confidence * gate).to(out_dtype)

