"""Known-answer tests of the q6 codec specification (no GPU, no reference counterpart).

Byte patterns are worked out by hand from the format: 4 signed 6-bit codes per
24-bit little-endian word, w = sum (code_i & 63) << 6i.
"""

import numpy as np

from oracle import q6_ref


def test_hand_packed_word():
    # codes 1, -1, 31, -31 -> fields 000001, 111111, 011111, 100001
    # w = 100001 011111 111111 000001 (binary, c3..c0) = 0x85FFC1
    codes = np.zeros(32, dtype=np.int8)
    codes[:4] = [1, -1, 31, -31]
    b = q6_ref.pack_codes(codes)
    assert b.shape == (24,)
    assert list(b[:3]) == [0xC1, 0xFF, 0x85]
    assert not b[3:].any()
    assert np.array_equal(q6_ref.unpack_codes(b), codes)


def test_all_codes_round_trip():
    codes = np.arange(-31, 32, dtype=np.int8)            # 63 values, pad to 2 groups
    codes = np.concatenate([codes, np.zeros(1, dtype=np.int8)]).reshape(2, 32)
    assert np.array_equal(q6_ref.unpack_codes(q6_ref.pack_codes(codes)), codes)


def test_exact_multiples_quantize_to_their_code():
    scale = np.float16(0.5)
    k = np.arange(-31, 32)
    x = np.zeros((2, 32), dtype=np.float32)
    x.reshape(-1)[:63] = k * np.float32(scale)
    codes, sc = q6_ref.quantize_groups(x)
    assert sc[0] == scale                                # absmax 15.5 / 31 = 0.5 exactly
    assert np.array_equal(codes.reshape(-1)[:63], k.astype(np.int8))
    assert np.array_equal(q6_ref.dequantize(codes, sc), x)


def test_zero_group_and_half_even_rounding():
    codes, sc = q6_ref.quantize_groups(np.zeros(32, dtype=np.float32))
    assert sc == 0 and not codes.any()
    x = np.zeros(32, dtype=np.float32)
    x[0] = 31.0                                          # scale 1.0
    x[1:6] = [2.5, 3.5, -2.5, 0.5, -0.5]
    codes, sc = q6_ref.quantize_groups(x)
    assert sc == 1.0
    assert list(codes[:6]) == [31, 2, 4, -2, 0, 0]


def test_scale_rounds_to_fp16_and_saturates():
    x = np.zeros(32, dtype=np.float32)
    x[3] = 1.0                                           # 1/31 -> fp16 0.03226 (RNE)
    _, sc = q6_ref.quantize_groups(x)
    assert sc == np.float16(np.float32(1.0) / np.float32(31.0))
    x[3] = 3.0e6                                         # 3e6/31 > 65504 -> saturate
    codes, sc = q6_ref.quantize_groups(x)
    assert sc == np.float16(65504.0) and codes[3] == 31


def test_slot_layout():
    rng = np.random.default_rng(0)
    k = rng.standard_normal((5, 64)).astype(np.float32)
    v = rng.standard_normal((5, 64)).astype(np.float32)
    probes = np.eye(4, 64)
    slot = q6_ref.pack_slots(k, v, probes)
    assert slot.shape == (5, 128) and not slot[:, 120:].any()
    kd, vd, z = q6_ref.unpack_slots(slot)
    # dequantisation error is at most half a step of each group's scale
    for x, xd in ((k, kd), (v, vd)):
        step = np.abs(x.reshape(5, 2, 32)).max(-1, keepdims=True) / 31
        assert (np.abs(x - xd).reshape(5, 2, 32) <= 0.5 * step * 1.01 + 1e-7).all()
    expect = kd[:, :4] / np.sqrt((kd.astype(np.float64) ** 2).sum(-1, keepdims=True) + 64e-6)
    assert np.allclose(z, expect, rtol=1e-6, atol=1e-7)
