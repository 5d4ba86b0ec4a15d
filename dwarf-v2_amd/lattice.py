"""Offset lattice, canonical ordering and MOVT channel map.

Host-side integer logic with the reference's names and error behaviour:
``ALL_OFFSETS`` and ``R_PLANES`` (kernels/dsqg_attention_v22.py:69, 84-94),
``_canonicalize_offsets`` (dsqg:155-186), ``_normalize_plane_shift``
(dsqg:109-127), ``_phase_plane_channels`` (dsqg:130-152),
``_orthogonal_phase_probes`` (dsqg:257-268), the grouped-mode table
(dsqg:462-480), and the trainer's ``build_offset_groups`` /
``_small_large_counts`` (train/train_dwarf.py:157-178).
"""

from __future__ import annotations

import math
from typing import Iterable, Sequence

import torch

R_PLANES = 4
SMALL_MAX = 28   # offsets <= 28 form the dense "small" band
LARGE_MIN = 48   # offsets >= 48 form the sparse "large" band

# The 96-offset causal lattice (data; identical to dsqg:84-94).
ALL_OFFSETS = [
    1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 13, 15, 16, 19, 21, 23, 28,
    48, 64, 96, 121, 161, 192, 212, 245, 273, 295, 342, 375, 384,
    413, 441, 473, 512, 549, 579, 593, 631, 653, 694, 716, 768,
    826, 846, 900, 936, 970, 1000, 1024, 1074, 1108, 1144, 1166,
    1190, 1218, 1244, 1288, 1322, 1385, 1423, 1451, 1497, 1522,
    1550, 1581, 1603, 1617, 1634, 1651, 1661, 1710, 1743, 1780,
    1810, 1820, 1852, 1860, 1876, 1886, 1897, 1903, 1916, 1926,
    1929, 1941, 1965, 1983, 2006, 2011, 2029, 2037, 2044, 2068,
    2097, 2113, 2199,
]

GROUPED_MODE_IDS = {"baseline": 0, "overlap_slab": 1, "overlap_slab_bwd": 3}
_UNIMPLEMENTED_GROUPED_MODES = {"packed_kv"}


def _as_index(value, what: str) -> int:
    """Accept ints and __index__-able values; reject bool and floats."""
    if isinstance(value, bool):
        raise TypeError(f"{what} must be an integer, got bool")
    try:
        return int(value.__index__())
    except (AttributeError, TypeError) as exc:
        raise TypeError(f"{what} must be an integer, got {type(value).__name__}") from exc


def _normalize_plane_shift(r_planes: int, hd: int, plane_shift: int = 0) -> int:
    """Validate the within-segment MOVT pair shift (dsqg:109-127)."""
    shift = _as_index(plane_shift, "plane_shift")
    if hd < 2 * r_planes:
        raise ValueError(f"head_dim={hd} must be >= 2*r_planes={2 * r_planes}")
    segment = max(2, hd // r_planes)
    if not 0 <= shift <= segment - 2:
        raise ValueError(
            f"plane_shift={shift} must keep each MOVT pair inside its hd/r segment; "
            f"allowed range is [0, {segment - 2}] for head_dim={hd}, r_planes={r_planes}"
        )
    return shift


def _phase_plane_channels(r_planes: int, hd: int, plane_shift: int = 0) -> list[tuple[int, int]]:
    """Channel pairs (a, a+1) rotated by the MOVT planes (dsqg:130-152).

    Plane r uses a = min(r*stride + shift, hd - 2) with stride = max(2, hd//r);
    if that pair collides with an earlier plane, the lowest free adjacent pair
    is used instead.
    """
    shift = _normalize_plane_shift(r_planes, hd, plane_shift)
    stride = max(2, hd // r_planes)
    taken: set[int] = set()
    pairs: list[tuple[int, int]] = []
    for plane in range(r_planes):
        first = min(plane * stride + shift, hd - 2)
        if first in taken or first + 1 in taken:
            free = [c for c in range(hd - 1) if c not in taken and c + 1 not in taken]
            if not free:
                raise ValueError(f"Could not assign {r_planes} disjoint MOVT planes in head_dim={hd}")
            first = free[0]
        taken.update((first, first + 1))
        pairs.append((first, first + 1))
    return pairs


def _canonicalize_offsets(offsets: Sequence[int], j_small: int, j_large: int) -> tuple[list[int], int, int]:
    """Sort offsets into the kernels' [small ascending | large ascending] order (dsqg:155-186)."""
    values = []
    for d in offsets:
        if isinstance(d, bool):
            raise TypeError(f"DSQG offsets must be integer positive causal deltas, got bool: {d!r}")
        try:
            ivalue = d.__index__()
        except (AttributeError, TypeError) as exc:
            raise TypeError(
                f"DSQG offsets must be integer positive causal deltas, got {type(d).__name__}: {d!r}"
            ) from exc
        if ivalue <= 0:
            raise ValueError(f"DSQG offsets must be positive causal deltas; got {ivalue}")
        values.append(int(ivalue))
    if len(set(values)) != len(values):
        raise ValueError(f"Duplicate DSQG offsets are not supported: {values}")
    middle = [d for d in values if SMALL_MAX < d < LARGE_MIN]
    if middle:
        raise ValueError(f"Offsets must be <={SMALL_MAX} or >={LARGE_MIN} for the DSQG split; got middle offsets {middle}")
    small = sorted(d for d in values if d <= SMALL_MAX)
    large = sorted(d for d in values if d >= LARGE_MIN)
    if (len(small), len(large)) != (int(j_small), int(j_large)):
        raise ValueError(
            "j_small/j_large mismatch after canonicalization: "
            f"declared ({j_small}, {j_large}) vs actual ({len(small)}, {len(large)})"
        )
    return small + large, len(small), len(large)


def _orthogonal_phase_probes(r_planes: int, hd: int, plane_shift: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
    """Unit q/k probes on each plane's channel pair, k a quarter turn ahead of q (dsqg:257-268)."""
    assert hd >= 2 * r_planes
    q = torch.zeros(r_planes, hd, dtype=torch.float32)
    k = torch.zeros(r_planes, hd, dtype=torch.float32)
    for plane, (a, b) in enumerate(_phase_plane_channels(r_planes, hd, plane_shift)):
        angle = 2.0 * math.pi * plane / max(r_planes, 1)
        q[plane, a], q[plane, b] = math.cos(angle), math.sin(angle)
        k[plane, a], k[plane, b] = math.cos(angle + math.pi / 2.0), math.sin(angle + math.pi / 2.0)
    return q, k


def _resolve_grouped_mode(mode: str) -> int:
    """Map a grouped_mode name to its id (dsqg:470-480)."""
    if not isinstance(mode, str):
        raise TypeError(f"grouped_mode must be a string, got {type(mode).__name__}")
    if mode in _UNIMPLEMENTED_GROUPED_MODES:
        raise NotImplementedError(
            f"grouped_mode='{mode}' is advertised by older configs but is not implemented in this kernel"
        )
    if mode not in GROUPED_MODE_IDS:
        raise ValueError(f"Unknown grouped_mode='{mode}'. Allowed: {', '.join(sorted(GROUPED_MODE_IDS))}")
    return GROUPED_MODE_IDS[mode]


def _small_large_counts(offsets: Iterable[int]) -> tuple[int, int]:
    """(#small, #large) of an offset group (train/train_dwarf.py:171-178)."""
    values = tuple(int(v) for v in offsets)
    small = sum(v <= SMALL_MAX for v in values)
    large = sum(v >= LARGE_MIN for v in values)
    if small + large != len(values):
        raise ValueError("DSQG offsets must remain in the supported kernel bands")
    return small, large


def build_offset_groups(model_length: int, min_offset_support: int = 64) -> tuple[tuple[int, ...], ...]:
    """The trainer's three per-block offset groups (train/train_dwarf.py:157-168).

    Offsets are kept when model_length - offset >= min_offset_support, then
    dealt round-robin into three groups (offsets[i::3]).
    """
    offsets = tuple(sorted(int(v) for v in ALL_OFFSETS))
    if len(offsets) != len(set(offsets)):
        raise ValueError("canonical DSQG offsets must be unique")
    kept = tuple(d for d in offsets if model_length - d >= min_offset_support)
    groups = tuple(tuple(kept[i::3]) for i in range(3))
    if any(not g for g in groups):
        raise ValueError("offset pruning left an empty DSQG group")
    return groups


def plane_shift_schedule(head_dim: int, n_dsqg_blocks: int) -> list[int]:
    """Per-DSQG-block plane shifts used by the trainer (train/train_dwarf.py:375-391)."""
    segment = max(2, head_dim // R_PLANES)
    return [2 * (i % max(1, segment // 2)) for i in range(n_dsqg_blocks)]


def valid_pair_count(offsets: Sequence[int], seq_len: int, query_start: int = 0) -> int:
    """Number of (query, offset) pairs with a source row, for one (b, h)."""
    total = 0
    for d in offsets:
        lo = max(int(d), int(query_start))
        total += max(0, seq_len - lo)
    return total
