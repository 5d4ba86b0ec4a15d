"""The sparse-group planner (host logic) against the reference's own outputs and against brute force.

golden: tests/golden/plan_golden.json holds ``_plan_sparse_groups`` (dsqg:536-671) evaluated by the
reference on the canonical lattice and 24 seeded random lattices under ten grouping settings, and the
errors of ``_normalize_grouping_args`` (dsqg:498-533); the plans must match exactly.  brute force:
enumerating every contiguous partition of the sorted far deltas fixes the least cost and, with the
reconstruction rule (the last group starts earliest, then the same for the prefix), the partition.
"""

from __future__ import annotations

import copy
import importlib
import itertools
import json
import os
import random

import pytest

planner = importlib.import_module("dwarf-v2_amd.planner")
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "plan_golden.json")


@pytest.fixture(scope="module")
def golden():
    with open(GOLDEN) as f:
        return json.load(f)


def test_plans_match_reference(golden):
    assert len(golden["cases"]) == 250
    for c in golden["cases"]:
        got = planner.plan_sparse_groups(c["offsets"], c["j_small"], c["k_group_size"],
                                         max_group_size=c["max_group_size"],
                                         max_group_spread=c["max_group_spread"], slab_block_n=c["slab_block_n"])
        assert got == c["plan"], (c["offsets"][:5], c["j_small"], c["k_group_size"], c["max_group_size"],
                                  c["max_group_spread"], c["slab_block_n"])
        planner.verify_sparse_plan(c["offsets"], c["j_small"], got)


def test_argument_errors_match_reference(golden):
    for e in golden["errors"]:
        if e["type"] is None:
            planner.normalize_grouping_args(*e["args"])
            continue
        with pytest.raises(Exception) as info:
            planner.normalize_grouping_args(*e["args"])
        assert type(info.value).__name__ == e["type"] and str(info.value) == e["message"], e["args"]
    for d in golden["defaults"]:
        assert list(planner.normalize_grouping_args(3, None, None, d["mode"])) == d["result"]


def _brute(deltas, gmax, cap, block_n):
    """Every contiguous partition meeting the caps, as (cost, reversed group starts, bounds)."""
    n = len(deltas)
    out = []
    for cuts in itertools.product((0, 1), repeat=max(n - 1, 0)):
        starts = [0] + [i + 1 for i, c in enumerate(cuts) if c]
        bounds = list(zip(starts, starts[1:] + [n]))
        if any(i1 - i0 > gmax or (cap is not None and deltas[i1 - 1] - deltas[i0] > cap) for i0, i1 in bounds):
            continue
        cost = sum(block_n + deltas[i1 - 1] - deltas[i0] for i0, i1 in bounds)
        out.append((cost, [b[0] for b in reversed(bounds)], bounds))
    return out


@pytest.mark.parametrize("seed", range(40))
def test_least_cost_partition_by_brute_force(seed):
    rng = random.Random(seed)
    n = rng.randint(1, 11)
    J = n + rng.randint(0, 4)
    offsets = sorted(rng.sample(range(1, 200), J))
    j_small = J - n
    gmax = rng.randint(1, 5)
    cap = rng.choice([None, 0, 3, 10, 40])
    block_n = rng.choice([1, 8, 64])
    plan = planner.plan_sparse_groups(offsets, j_small, gmax, max_group_spread=cap, slab_block_n=block_n)
    planner.verify_sparse_plan(offsets, j_small, plan)
    deltas = offsets[j_small:]   # sorted, so the far deltas in sorted order
    cands = _brute(deltas, gmax, cap, block_n)
    if not cands:   # no partition meets the caps: fixed-size chunks
        assert plan["group_len"] == [min(gmax, n - i) for i in range(0, n, gmax)]
        return
    best = min(c[0] for c in cands)
    want = min((c for c in cands if c[0] == best), key=lambda c: c[1])[2]
    got = [(s, s + g) for s, g in zip(plan["group_start"], plan["group_len"])]
    assert got == want
    assert sum(block_n + hi - lo for lo, hi in zip(plan["group_dmin"], plan["group_dmax"])) == best
    assert plan["max_group_len"] <= gmax
    if cap is not None:
        assert plan["max_group_spread"] <= cap


def test_canonical_lattice_slab_defaults():
    from importlib import import_module
    lattice = import_module("dwarf-v2_amd.lattice")
    k, m, s = planner.normalize_grouping_args(3, None, None, lattice.GROUPED_MODE_IDS["overlap_slab"])
    assert (k, m, s) == (3, 3, 64)
    plan = planner.plan_sparse_groups(list(lattice.ALL_OFFSETS), 17, k, max_group_size=m, max_group_spread=s)
    assert sorted(plan["sparse_order"]) == list(range(17, 96))
    assert plan["max_group_spread"] <= 64 and plan["max_group_len"] <= 3
    assert planner._plan_sparse_groups is planner.plan_sparse_groups


def test_verify_rejects_broken_plans():
    offsets = [1, 2, 3, 50, 60, 90, 200]
    plan = planner.plan_sparse_groups(offsets, 3, 3)
    planner.verify_sparse_plan(offsets, 3, plan)
    bad = copy.deepcopy(plan)
    bad["sparse_order"][0] = bad["sparse_order"][1]
    with pytest.raises(AssertionError, match="exactly once"):
        planner.verify_sparse_plan(offsets, 3, bad)
    bad = copy.deepcopy(plan)
    bad["group_rel"][0][0] += 1
    with pytest.raises(AssertionError, match="Invalid rel mapping at group=0, t=0"):
        planner.verify_sparse_plan(offsets, 3, bad)
    assert planner.plan_sparse_groups(offsets, 7, 3)["sparse_order"] == []
