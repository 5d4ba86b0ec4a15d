"""Write golden vectors for the sparse-group planner from the reference itself.

Run once in the build container (the reference checkout exists only there):

    python tests/golden/make_plan_golden.py /root/reference

It imports kernels/dsqg_attention_v22.py from the reference checkout and
records ``_plan_sparse_groups`` (dsqg:536-671) on the canonical lattice under
several grouping settings and on seeded random lattices, and the exception
type and message ``_normalize_grouping_args`` (dsqg:498-533) gives for bad
arguments, as JSON next to this script.  Only the data travels; the tests
never read the reference.

This function is imported because the checks that need no import (brute-force
least cost over all partitions, the plan invariants of ``_verify_sparse_plan``)
fix the plan's cost but not which of several equal-cost partitions the
reference returns.
"""

from __future__ import annotations

import importlib.util
import json
import os
import random
import sys

HERE = os.path.dirname(os.path.abspath(__file__))

SETTINGS = [   # (k_group_size, max_group_size, max_group_spread, slab_block_n)
    (3, None, None, 64), (3, None, 64, 64), (3, 2, 64, 64), (4, None, 32, 64), (8, None, None, 64),
    (8, None, 16, 64), (1, None, None, 64), (6, 5, 200, 16), (5, None, 0, 64), (3, None, None, 1000),
]


def load_reference(root: str):
    path = os.path.join(root, "kernels", "dsqg_attention_v22.py")
    spec = importlib.util.spec_from_file_location("_reference_dsqg_v22", path)
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


def random_lattice(rng: random.Random):
    J = rng.randint(1, 40)
    offsets = sorted(rng.sample(range(1, 3000), J))
    j_small = rng.randint(0, J)
    return offsets, j_small


def main(root: str) -> None:
    ref = load_reference(root)
    cases = []
    lattices = [(list(ref.ALL_OFFSETS), 17)]
    rng = random.Random(2024)
    lattices += [random_lattice(rng) for _ in range(24)]
    for offsets, j_small in lattices:
        for kg, mg, ms, bn in SETTINGS:
            plan = ref._plan_sparse_groups(offsets, j_small, kg, max_group_size=mg, max_group_spread=ms,
                                           slab_block_n=bn)
            cases.append({"offsets": offsets, "j_small": j_small, "k_group_size": kg, "max_group_size": mg,
                          "max_group_spread": ms, "slab_block_n": bn, "plan": plan})
    errors = []
    for args in ([True, None, None], [0, None, None], [3.0, None, None], [3, 4, None], [3, 0, None],
                 [3, None, -1], [3, None, 2.5], ["3", None, None], [3, False, None]):
        try:
            ref._normalize_grouping_args(*args)
            errors.append({"args": args, "type": None, "message": None})
        except Exception as exc:   # recorded, not raised
            errors.append({"args": args, "type": type(exc).__name__, "message": str(exc)})
    defaults = []
    for mode in (0, 1, 3):
        defaults.append({"mode": mode, "result": list(ref._normalize_grouping_args(3, None, None, mode))})
    path = os.path.join(HERE, "plan_golden.json")
    with open(path, "w") as f:
        json.dump({"cases": cases, "errors": errors, "defaults": defaults}, f, separators=(",", ":"))
    print(f"wrote {path}: {len(cases)} plans, {len(errors)} error cases")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
