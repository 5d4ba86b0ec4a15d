"""The custom-op boundary (torch.library): registration and fake (shape) implementations, no GPU needed."""

import torch


def _meta_inputs(B=2, H=4, Hk=2, N=64, J=96, JL=79):
    m = torch.device("meta")
    q = torch.empty(B, H, N, 64, device=m, dtype=torch.bfloat16)
    k = torch.empty(B, Hk, N, 64, device=m, dtype=torch.bfloat16)
    return dict(q=q, k=k, v=k.clone(), pb=torch.empty(J, H, device=m), se=torch.empty(J, 64, device=m),
                pbase=torch.empty(JL, H, 4, device=m), pgain=torch.empty(JL, H, 4, device=m),
                y=torch.empty(B, H, N, 4, device=m), z=torch.empty(B, Hk, N, 4, device=m),
                off=torch.empty(J, dtype=torch.int32, device=m))


def test_ops_are_registered(pkg):
    for name in ("dsqg_fwd", "dsqg_bwd", "ema_fwd", "ema_bwd"):
        assert hasattr(torch.ops.dwarf, name), name


def test_dsqg_fake_shapes(pkg):
    t = _meta_inputs()
    out, lse = torch.ops.dwarf.dsqg_fwd(t["q"], t["k"], t["v"], t["pb"], t["se"], t["pbase"], t["pgain"], t["y"],
                                        t["z"], t["off"], 17, 79, 0, 1)
    assert out.shape == t["q"].shape and out.dtype == torch.bfloat16
    assert lse.shape == t["q"].shape[:3] and lse.dtype == torch.float32
    grads = torch.ops.dwarf.dsqg_bwd(out, t["q"], t["k"], t["v"], t["pb"], t["se"], t["pbase"], t["pgain"], t["y"],
                                     t["z"], t["off"], out, lse, 17, 79, 0, 1)
    want = [t["q"], t["k"], t["v"], t["pb"], t["se"], t["pbase"], t["pgain"], t["y"], t["z"]]
    assert [g.shape for g in grads] == [w.shape for w in want]
    assert [g.dtype for g in grads] == [torch.bfloat16] * 3 + [torch.float32] * 6


def test_ema_fake_shapes(pkg):
    m = torch.device("meta")
    x = torch.empty(2, 8, 16, device=m, dtype=torch.bfloat16)
    for alpha in (torch.empty(1, device=m), torch.empty(16, device=m)):
        y = torch.ops.dwarf.ema_fwd(x, alpha, 1e-5, 0.5)
        dx, da = torch.ops.dwarf.ema_bwd(x, y, y, alpha, 1e-5, 0.5)
        assert y.shape == x.shape and dx.shape == x.shape and da.shape == (alpha.numel(),)
