"""Write golden vectors for the DSQG eager oracle from the reference itself.

Run once in the build container (the reference checkout exists only there):

    python tests/golden/make_golden.py /root/reference

It imports kernels/dsqg_attention_v22.py from the reference checkout and
evaluates ``_eager_dsqg_attention`` (dsqg:2602-2688) and its autograd
gradients on small seeded float64 inputs, then saves inputs and outputs as
plain .npz arrays (no pickles) next to this script.  Only the data travels;
the tests never read the reference.

This function is imported because the closed-form checks (a dense-mask SDPA
equivalence with MOVT off, a constant-angle rotation equivalence, one-hot
selection and gradcheck) do not pin the eager composition with
data-dependent MOVT angles and GQA head mapping.
"""

from __future__ import annotations

import importlib.util
import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))

CASES = {
    # name: (B, H, Hkv, N, offsets, j_small, plane_shift, phase_gain_std, seed)
    "movt_small": (1, 2, 2, 96, [1, 2, 3, 5, 8, 13, 21, 48, 64, 80], 7, 2, 3.0, 11),
    "gqa": (2, 4, 2, 80, [1, 2, 4, 8, 16, 48], 5, 0, 1.5, 12),
    "lattice96": (1, 1, 1, 256, None, 17, 6, 2.0, 13),
}


def load_reference(root: str):
    path = os.path.join(root, "kernels", "dsqg_attention_v22.py")
    spec = importlib.util.spec_from_file_location("_reference_dsqg_v22", path)
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


def make_case(ref, B, H, Hkv, N, offsets, j_small, shift, gain_std, seed):
    hd = 64
    if offsets is None:
        offsets = list(ref.ALL_OFFSETS)
    J = len(offsets)
    j_large = J - j_small
    g = torch.Generator().manual_seed(seed)
    f64 = torch.float64
    q = torch.randn(B, H, N, hd, generator=g, dtype=f64)
    k = torch.randn(B, Hkv, N, hd, generator=g, dtype=f64)
    v = torch.randn(B, Hkv, N, hd, generator=g, dtype=f64)
    pos_bias = 0.02 * torch.randn(J, H, generator=g, dtype=f64)
    scale_embed = 0.05 * torch.randn(J, hd, generator=g, dtype=f64)
    phase_base = 0.3 * torch.randn(max(j_large, 1), H, 4, generator=g, dtype=f64)
    phase_gain = gain_std * torch.randn(max(j_large, 1), H, 4, generator=g, dtype=f64)
    qp, kp = ref._orthogonal_phase_probes(4, hd, shift)
    qpn = torch.nn.functional.normalize(qp.to(f64), dim=-1)
    kpn = torch.nn.functional.normalize(kp.to(f64), dim=-1)
    y = torch.einsum("bhnd,rd->bhnr", q, qpn) * torch.rsqrt(q.square().sum(-1, keepdim=True) + 1e-6 * hd)
    z = torch.einsum("bhnd,rd->bhnr", k, kpn) * torch.rsqrt(k.square().sum(-1, keepdim=True) + 1e-6 * hd)
    dout = torch.randn(B, H, N, hd, generator=g, dtype=f64)

    inputs = dict(q=q, k=k, v=v, pos_bias=pos_bias, scale_embed=scale_embed, phase_base=phase_base,
                  phase_gain=phase_gain, y_pre=y.contiguous(), z_pre=z.contiguous())
    leaves = {n: t.clone().requires_grad_(True) for n, t in inputs.items()}
    out = ref._eager_dsqg_attention(
        leaves["q"], leaves["k"], leaves["v"], leaves["pos_bias"], leaves["scale_embed"],
        leaves["phase_base"], leaves["phase_gain"], leaves["y_pre"], leaves["z_pre"],
        offsets, j_small, plane_shift=shift,
    )
    out.backward(dout)
    arrays = {f"in_{n}": t.numpy() for n, t in inputs.items()}
    arrays.update({f"grad_{n}": leaves[n].grad.numpy() for n in inputs})
    arrays["out"] = out.detach().numpy()
    arrays["dout"] = dout.numpy()
    arrays["offsets"] = np.asarray(offsets, dtype=np.int32)
    arrays["meta"] = np.asarray([B, H, Hkv, N, hd, j_small, j_large, shift], dtype=np.int64)
    return arrays


def main(root: str) -> None:
    torch.set_num_threads(4)
    ref = load_reference(root)
    for name, spec in CASES.items():
        arrays = make_case(ref, *spec)
        path = os.path.join(HERE, f"dsqg_eager_{name}.npz")
        np.savez_compressed(path, **arrays)
        print(f"wrote {path}: out {arrays['out'].shape}, |out|max {np.abs(arrays['out']).max():.4f}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
