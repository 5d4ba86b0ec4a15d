"""Host-side behaviour of the Python mirror of the reference interface (no GPU).

Errors are raised with the reference's exception types before any device
work: ValueError for shapes/arguments (dsqg:2209-2225), NotImplementedError
for unsupported modes (dsqg:2217-2221), RuntimeError when no GPU tensors are
given -- this library has no CPU fallback.
"""

import importlib

import pytest
import torch


def _args(B=1, H=2, Hkv=2, N=8, hd=64, J=3, js=2):
    return dict(
        q=torch.zeros(B, H, N, hd), k=torch.zeros(B, Hkv, N, hd), v=torch.zeros(B, Hkv, N, hd),
        pos_bias=torch.zeros(J, H), scale_embed=torch.zeros(J, hd),
        phase_base=torch.zeros(max(J - js, 1), H, 4), phase_gain=torch.zeros(max(J - js, 1), H, 4),
        y_pre=torch.zeros(B, H, N, 4), z_pre=torch.zeros(B, Hkv, N, 4),
    )


def _call(pkg, a, J=3, js=2, backend="auto", mode=0):
    return pkg.dsqg_attention_v18_grouped(
        a["q"], a["k"], a["v"], a["pos_bias"], a["scale_embed"], a["phase_base"], a["phase_gain"],
        a["y_pre"], a["z_pre"], J, js, J - js, torch.tensor([1, 2, 48], dtype=torch.int32),
        None, None, None, None, None, 3, mode, False, 0, 0, 1, backend=backend,
    )


def _fn(pkg, a, mode=0):
    return pkg._DSQGV18GroupedFn.apply(
        a["q"], a["k"], a["v"], a["pos_bias"], a["scale_embed"], a["phase_base"], a["phase_gain"],
        a["y_pre"], a["z_pre"], 3, 2, 1, torch.tensor([1, 2, 48], dtype=torch.int32),
        None, None, None, None, None, 3, mode, False, 0, 0, 1, True,
    )


def test_backend_selection(pkg):
    a = _args()
    with pytest.raises(ValueError):
        _call(pkg, a, backend="cuda")
    with pytest.raises(NotImplementedError):
        _call(pkg, a, backend="eager")
    with pytest.raises(RuntimeError):
        _call(pkg, a)                 # CPU tensors: no fallback
    with pytest.raises(RuntimeError):
        _call(pkg, a, backend="triton")


def test_function_shape_errors(pkg):
    a = _args()
    a["v"] = torch.zeros(1, 2, 9, 64)
    with pytest.raises(ValueError, match="k/v shape mismatch"):
        _fn(pkg, a)
    a = _args(H=3, Hkv=2)
    with pytest.raises(ValueError, match="divisible"):
        _fn(pkg, a)
    a = _args(H=4, Hkv=2)
    with pytest.raises(NotImplementedError):
        _fn(pkg, a, mode=1)
    a = _args()
    a["y_pre"] = torch.zeros(1, 2, 7, 4)
    with pytest.raises(ValueError, match="y_pre"):
        _fn(pkg, a)
    a = _args()
    a["z_pre"] = torch.zeros(1, 1, 8, 4)
    with pytest.raises(ValueError, match="z_pre"):
        _fn(pkg, a)
    a = _args()
    with pytest.raises(RuntimeError, match="device"):
        _fn(pkg, a)


def test_ema_errors(pkg):
    x = torch.zeros(2, 5, 3)
    a = torch.tensor([0.1])
    with pytest.raises(ValueError):
        pkg.causal_ema_scan(torch.zeros(5, 3), a)
    with pytest.raises(ValueError):
        pkg.causal_ema_scan(x, torch.tensor([0.1, 0.2]))
    with pytest.raises(ValueError):
        pkg.causal_ema_scan(x, a, 0.6, 0.5)
    with pytest.raises(ValueError):   # reset_mask must be [B,N] (ema:463-464)
        pkg.causal_ema_scan(x, a, reset_mask=torch.zeros(2, 4, dtype=torch.bool))
    with pytest.raises(RuntimeError):
        pkg.causal_ema_scan(x, a, reset_mask=torch.zeros(2, 5, dtype=torch.bool))
    with pytest.raises(RuntimeError):
        pkg.causal_ema_scan(x, a)
    with pytest.raises(RuntimeError):
        pkg.causal_ema_scan(x, torch.full((3,), 0.1))   # per-channel accepted, but no CPU path


def test_interference_pool_errors(pkg):
    x = torch.zeros(2, 5, 3)
    a, w = torch.tensor([0.1, 0.01, 0.001]), torch.full((3,), 1 / 3)
    with pytest.raises(ValueError):
        pkg.interference_pool(torch.zeros(5, 3), a, w)
    with pytest.raises(ValueError):   # one weight per factor
        pkg.interference_pool(x, a, w[:2])
    with pytest.raises(ValueError):   # at most four timescales
        pkg.interference_pool(x, torch.full((5,), 0.1), torch.full((5,), 0.2))
    with pytest.raises(ValueError):
        pkg.interference_pool(x, a, w, floor=0.6, ceiling=0.5)
    with pytest.raises(RuntimeError):   # no CPU path
        pkg.interference_pool(x, a, w)


def test_q6_errors(pkg):
    with pytest.raises(ValueError):
        pkg.q6.pack_kv(torch.zeros(1, 1, 4, 64), torch.zeros(1, 1, 5, 64))
    with pytest.raises(RuntimeError):
        pkg.q6.pack_kv(torch.zeros(1, 1, 4, 64), torch.zeros(1, 1, 4, 64))
    with pytest.raises(ValueError):
        pkg.q6.unpack_kv(torch.zeros(1, 1, 4, 100, dtype=torch.uint8))


def test_library_is_the_only_path(pkg):
    """The package loads its HIP library eagerly on use and never imports the oracle."""
    import sys

    for name in list(sys.modules):
        if name.startswith("dwarf-v2_amd"):
            mod = sys.modules[name]
            src = open(mod.__file__).read() if getattr(mod, "__file__", None) else ""
            assert "import oracle" not in src and "from oracle" not in src
    assert pkg.native_library_path().endswith("libdwarf_dsqg.so")


def test_backward_sets_the_delta_stage_flag_itself(pkg, monkeypatch):
    """A caller's schedule that carries DWARF_SCHED_DELTA_STAGE does not reach the serial stages (the dQ
    launch would then skip the (delta, lse) pairs dK/dV reads and no delta launch would write them): the
    flag is cleared and set only where the delta launch runs.  The C ABI is replaced by a recorder."""
    dsqg = importlib.import_module("dwarf-v2_amd.dsqg")
    L = pkg._lib
    seen = []

    class Recorder:
        def dwarf_dsqg_bwd_workspace_bytes(self, args):
            return 256

        def __getattr__(self, name):
            def launch(args, stream):
                seen.append((name, args._obj.fwd.schedule))
                return 0
            return launch

    monkeypatch.setattr(dsqg._lib, "load", lambda: Recorder())
    monkeypatch.setattr(dsqg, "_stream", lambda device: 0)
    a = _args(N=8, J=3, js=2)
    a = {n: t.to(torch.bfloat16) if n in ("q", "k", "v") else t for n, t in a.items()}
    off = torch.tensor([1, 2, 48], dtype=torch.int32)
    out, lse = torch.zeros_like(a["q"]), torch.zeros(1, 2, 8)
    for sched in (L.DWARF_SCHED_DELTA_STAGE, L.DWARF_SCHED_BAND | L.DWARF_SCHED_DELTA_STAGE):
        seen.clear()
        dsqg.dsqg_backward(torch.zeros_like(a["q"]), a["q"], a["k"], a["v"], a["pos_bias"], a["scale_embed"],
                           a["phase_base"], a["phase_gain"], a["y_pre"], a["z_pre"], off, out, lse, 2, 1,
                           schedule=sched, overlap=False)
        assert [n for n, _ in seen] == ["dwarf_dsqg_bwd_dq", "dwarf_dsqg_bwd_params", "dwarf_dsqg_bwd_dkdv"]
        assert all(s & L.DWARF_SCHED_DELTA_STAGE == 0 for _, s in seen), seen
        assert all(s == sched & ~L.DWARF_SCHED_DELTA_STAGE for _, s in seen), seen
        seen.clear()
        dsqg.dsqg_backward(torch.zeros_like(a["q"]), a["q"], a["k"], a["v"], a["pos_bias"], a["scale_embed"],
                           a["phase_base"], a["phase_gain"], a["y_pre"], a["z_pre"], off, out, lse, 2, 1,
                           schedule=sched, overlap=True, one_call=True)
        assert seen == [("dwarf_dsqg_bwd", sched)]


def test_custom_ops_default_to_the_python_schedule(pkg):
    """dwarf::dsqg_fwd / dsqg_bwd called without a schedule run the schedule dsqg_forward/backward and the
    autograd Function run (DEFAULT_SCHEDULE), not the gather loops alone."""
    import inspect

    ops = importlib.import_module("dwarf-v2_amd.ops")
    dsqg = importlib.import_module("dwarf-v2_amd.dsqg")
    for fn in (ops.dsqg_fwd, ops.dsqg_bwd):
        schema = fn._opoverload._schema
        arg = [x for x in schema.arguments if x.name == "schedule"][0]
        assert arg.default_value == dsqg.DEFAULT_SCHEDULE
    assert inspect.signature(ops._dsqg_fwd_fake).parameters["schedule"].default == dsqg.DEFAULT_SCHEDULE


def test_integration_guide_names_exist(pkg):
    """Every ``amd.<name>`` the drop-in guide tells a maintainer to bind exists in the package, so the
    rebinding it shows runs as written."""
    import os
    import re

    guide = open(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "INTEGRATION.md")).read()
    names = sorted(set(re.findall(r"\bamd\.([A-Za-z_][A-Za-z0-9_]*)", guide)))
    assert len(names) >= 15
    missing = [n for n in names if not hasattr(pkg, n)]
    assert not missing, missing
