"""Sparse-offset grouping planner of the overlap-slab modes (host logic).

Drop-in for the reference's ``_normalize_grouping_args`` (dsqg:498-533),
``_plan_sparse_groups`` (dsqg:536-671) and ``_verify_sparse_plan``
(dsqg:674-691): same names, arguments, dict keys, exception types and
messages, so module code that builds the plan buffers for
``dsqg_attention_v18_grouped`` (dsqg:2888-2923) keeps working unchanged.

The plan partitions the far ("sparse") offsets, sorted by delta, into
contiguous groups of at most ``max_group_size`` offsets whose delta spread
stays within ``max_group_spread``.  Among all such partitions it takes one
of least total cost sum_g (slab_block_n + spread_g), the K columns a slab
tiling loads per query block; ties go to the partition whose last group
starts earliest, then recursively the same for the prefix (the reference's
reconstruction order, so the buffers come out identical).

This build's kernels do not tile far offsets into slabs: grouped modes 1 and
3 select the near-band schedule of the dQ launch, and the far offsets are
gathered per offset either way.  The plan is still produced and checked
here because it is part of the op's interface: callers compute it once per
module and pass its buffers to every call.
"""

from __future__ import annotations

from typing import Sequence

from .lattice import GROUPED_MODE_IDS

_SLAB_MODES = (GROUPED_MODE_IDS["overlap_slab"], GROUPED_MODE_IDS["overlap_slab_bwd"])
_SLAB_DEFAULT_SPREAD = 64   # the reference's default spread cap for the slab modes (dsqg:522-528)


def _normalize_int_arg(name: str, value, *, minimum: int) -> int:
    """An int >= minimum from anything with __index__ other than bool (dsqg:482-495)."""
    if isinstance(value, bool):
        raise TypeError(f"{name} must be an integer >= {minimum}, got bool")
    index = getattr(type(value), "__index__", None)
    if index is None:
        raise TypeError(f"{name} must be an integer >= {minimum}, got {type(value).__name__}")
    try:
        ivalue = index(value)
    except TypeError as exc:
        raise TypeError(f"{name} must be an integer >= {minimum}, got {type(value).__name__}") from exc
    if ivalue < minimum:
        raise ValueError(f"{name}={ivalue} must be >= {minimum}")
    return int(ivalue)


def normalize_grouping_args(k_group_size, max_group_size, max_group_spread,
                            grouped_mode_id: int | None = None) -> tuple[int, int, int | None]:
    """(k_group_size, max_group_size, max_group_spread) in canonical form.

    k_group_size is the group capacity; max_group_size caps the planner and
    defaults to it, never above it; the slab modes cap the spread at 64 unless
    the caller sets one.
    """
    k_group_size = _normalize_int_arg("k_group_size", k_group_size, minimum=1)
    if max_group_size is None:
        max_group_size = k_group_size
    else:
        max_group_size = _normalize_int_arg("max_group_size", max_group_size, minimum=1)
        if max_group_size > k_group_size:
            raise ValueError(
                f"max_group_size={max_group_size} cannot exceed k_group_size={k_group_size}; "
                "overlap-slab kernels iterate only K_GROUP_SIZE slots per group"
            )
    if max_group_spread is None and grouped_mode_id in _SLAB_MODES:
        max_group_spread = _SLAB_DEFAULT_SPREAD
    if max_group_spread is not None:
        max_group_spread = _normalize_int_arg("max_group_spread", max_group_spread, minimum=0)
    return k_group_size, max_group_size, max_group_spread


def _best_partition(deltas: Sequence[int], gmax: int, spread_cap: int | None, block_n: int):
    """Group boundaries [(i0, i1), ...] of a least-cost partition of the sorted deltas, or None.

    best[i] is the least cost of covering deltas[:i]; choice[i] the start of
    the last group of that covering, the smallest start among the optimal
    ones (starts are tried in increasing order and only a strict improvement
    replaces a choice).  A group's spread is deltas[i1-1] - deltas[i0] since
    the deltas are sorted.
    """
    n = len(deltas)
    best: list[float | None] = [None] * (n + 1)
    choice = [-1] * (n + 1)
    best[0] = 0
    for i0 in range(n):
        if best[i0] is None:
            continue
        for i1 in range(i0 + 1, min(n, i0 + gmax) + 1):
            spread = deltas[i1 - 1] - deltas[i0]
            if spread_cap is not None and spread > spread_cap:
                break
            cost = best[i0] + float(block_n) + spread
            if best[i1] is None or cost < best[i1]:
                best[i1] = cost
                choice[i1] = i0
    if best[n] is None:
        return None
    bounds = []
    end = n
    while end > 0:
        start = choice[end]
        bounds.append((start, end))
        end = start
    bounds.reverse()
    return bounds


def plan_sparse_groups(offsets: list[int], j_small: int, k_group_size: int, max_group_size: int | None = None,
                       max_group_spread: int | None = None, slab_block_n: int = 64) -> dict:
    """Group the far offsets (logical indices j_small..J-1) for a slab tiling.

    Returns the reference's plan dict: sparse_order (logical indices, group
    by group), group_start / group_len into it, group_dmin / group_dmax, per
    group its indices (group_i) and their distances below the group's largest
    delta (group_rel), and the largest group length and spread observed.
    """
    k_group_size, max_group_size, max_group_spread = normalize_grouping_args(
        k_group_size, max_group_size, max_group_spread)
    sparse = sorted(range(j_small, len(offsets)), key=lambda i: offsets[i])
    plan = {"sparse_order": [], "group_start": [], "group_len": [], "group_dmin": [], "group_dmax": [],
            "group_i": [], "group_rel": [], "max_group_len": 0, "max_group_spread": 0}
    if not sparse:
        return plan
    deltas = [offsets[i] for i in sparse]
    bounds = _best_partition(deltas, max_group_size, max_group_spread, slab_block_n)
    if bounds is None:   # no partition meets the caps: fixed-size chunks of the sorted indices
        bounds = [(i0, min(i0 + max_group_size, len(sparse))) for i0 in range(0, len(sparse), max_group_size)]
    for i0, i1 in bounds:
        idxs = sparse[i0:i1]
        ds = [offsets[i] for i in idxs]
        lo, hi = min(ds), max(ds)
        plan["group_start"].append(len(plan["sparse_order"]))
        plan["group_len"].append(len(idxs))
        plan["group_dmin"].append(lo)
        plan["group_dmax"].append(hi)
        plan["group_i"].append(idxs)
        plan["group_rel"].append([hi - d for d in ds])
        plan["sparse_order"].extend(idxs)
        plan["max_group_len"] = max(plan["max_group_len"], len(idxs))
        plan["max_group_spread"] = max(plan["max_group_spread"], hi - lo)
    return plan


def verify_sparse_plan(offsets: list[int], j_small: int, plan: dict) -> None:
    """AssertionError unless the plan covers every far index once and its rel entries match the deltas."""
    order = list(plan["sparse_order"])
    if sorted(order) != list(range(j_small, len(offsets))):
        raise AssertionError("Sparse plan does not include each sparse logical index exactly once")
    for gi, start in enumerate(plan["group_start"]):
        dmax = plan["group_dmax"][gi]
        for t in range(plan["group_len"][gi]):
            idx = order[start + t]
            rel = plan["group_rel"][gi][t]
            delta = offsets[idx]
            if rel != dmax - delta:
                raise AssertionError(
                    f"Invalid rel mapping at group={gi}, t={t}: rel={rel}, dmax={dmax}, delta={delta}"
                )


# The reference's private names, for module code written against them.
_normalize_grouping_args = normalize_grouping_args
_plan_sparse_groups = plan_sparse_groups
_verify_sparse_plan = verify_sparse_plan
