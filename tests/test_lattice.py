"""Offset lattice, canonical order, channel map and trainer grouping: closed forms.

Expected values are fixed by arithmetic on the literal lattice
(kernels/dsqg_attention_v22.py:84-94) and the trainer's rules
(train/train_dwarf.py:157-178, 375-391), so these checks are bit-exact.
"""

import pytest
import torch

from oracle import dsqg_ref


def test_lattice_shape(pkg):
    offs = pkg.ALL_OFFSETS
    assert len(offs) == 96 and len(set(offs)) == 96
    assert offs == sorted(offs)
    small = [d for d in offs if d <= 28]
    large = [d for d in offs if d >= 48]
    assert (len(small), len(large)) == (17, 79)
    assert not [d for d in offs if 28 < d < 48]
    assert min(offs) == 1 and max(offs) == 2199
    assert pkg.R_PLANES == 4


def test_canonicalize_sorts_and_splits(pkg):
    mixed = [64, 3, 1, 2199, 28, 48]
    canon, js, jl = pkg._canonicalize_offsets(mixed, 3, 3)
    assert canon == [1, 3, 28, 48, 64, 2199] and (js, jl) == (3, 3)
    canon, js, jl = pkg._canonicalize_offsets(list(reversed(pkg.ALL_OFFSETS)), 17, 79)
    assert canon == pkg.ALL_OFFSETS


@pytest.mark.parametrize(
    "offsets,js,jl,exc",
    [
        ([1, 1, 48], 2, 1, ValueError),       # duplicate
        ([1, 30, 48], 2, 1, ValueError),      # middle band 29..47
        ([0, 48], 1, 1, ValueError),          # not positive
        ([-3, 48], 1, 1, ValueError),
        ([True, 48], 1, 1, TypeError),        # bool rejected
        ([1.0, 48], 1, 1, TypeError),         # float rejected
        ([1, 2, 48], 1, 2, ValueError),       # declared split mismatch
    ],
)
def test_canonicalize_rejects(pkg, offsets, js, jl, exc):
    with pytest.raises(exc):
        pkg._canonicalize_offsets(offsets, js, jl)


def test_plane_channels_and_shift(pkg):
    for shift in range(0, 15):
        pairs = pkg._phase_plane_channels(4, 64, shift)
        assert pairs == [(shift, shift + 1), (16 + shift, 17 + shift), (32 + shift, 33 + shift), (48 + shift, 49 + shift)]
        assert pairs == dsqg_ref.channel_pairs(64, shift)
    for bad in (-1, 15, 16):
        with pytest.raises(ValueError):
            pkg._normalize_plane_shift(4, 64, bad)
    with pytest.raises(TypeError):
        pkg._normalize_plane_shift(4, 64, True)
    with pytest.raises(ValueError):
        pkg._normalize_plane_shift(4, 6, 0)  # head_dim < 2*planes


def test_orthogonal_probes(pkg):
    q, k = pkg._orthogonal_phase_probes(4, 64, 2)
    assert torch.allclose(q.norm(dim=-1), torch.ones(4))
    assert torch.allclose(k.norm(dim=-1), torch.ones(4))
    # k is a quarter turn ahead of q on each plane: <q_r, k_r> = 0
    assert torch.allclose((q * k).sum(-1), torch.zeros(4), atol=1e-7)
    assert q[0, 2] == 1.0 and q[0, 3] == 0.0  # plane 0 at angle 0 on channels (2, 3)


def test_trainer_offset_groups(pkg):
    groups = pkg.build_offset_groups(2047, 64)
    kept = sorted(d for g in groups for d in g)
    assert len(kept) == 87
    pruned = sorted(set(pkg.ALL_OFFSETS) - set(kept))
    assert pruned == [2006, 2011, 2029, 2037, 2044, 2068, 2097, 2113, 2199]
    counts = [pkg.lattice._small_large_counts(g) for g in groups]
    assert counts == [(6, 23), (6, 23), (5, 24)]
    assert [min(g) for g in groups] == [1, 2, 3]
    assert pkg.lattice.plane_shift_schedule(64, 9) == [0, 2, 4, 6, 8, 10, 12, 14, 0]


def test_valid_pair_counts(pkg):
    """Valid (query, offset) pairs per (b, h): closed form vs brute force, plus the dead offsets."""
    offs = pkg.ALL_OFFSETS
    n2048 = pkg.lattice.valid_pair_count(offs, 2048)
    assert n2048 == dsqg_ref.valid_pairs_per_head(offs, 2048) == 100_641
    assert [d for d in offs if d >= 2048] == [2068, 2097, 2113, 2199]
    assert pkg.lattice.valid_pair_count(offs, 8192) == 690_180
    # query_start = 1 (the minimum offset) removes nothing
    assert pkg.lattice.valid_pair_count(offs, 2048, query_start=1) == n2048
    assert pkg.lattice.valid_pair_count([5], 10, query_start=7) == 3


def test_grouped_modes(pkg):
    assert pkg.lattice._resolve_grouped_mode("baseline") == 0
    with pytest.raises(NotImplementedError):
        pkg.lattice._resolve_grouped_mode("packed_kv")
    with pytest.raises(ValueError):
        pkg.lattice._resolve_grouped_mode("nope")
