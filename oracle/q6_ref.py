"""CPU q6 codec -- test infrastructure, not the product.

The q6 cache format has no counterpart in the reference repository; this is
the specification the GPU codec must match bit for bit:

  group   32 consecutive head-dim values of one row (2 groups at hd = 64)
  scale   fp16_rne(absmax / 31) with an fp32 division; +inf saturates to 65504
  code    clamp(rint(x / float(scale)), -31, 31) with an fp32 division, 0 when
          scale == 0 (rint rounds half to even)
  packing 4 codes per 24-bit little-endian word w = sum (code_i & 63) << 6i,
          stored as bytes w, w>>8, w>>16
  dequant float(sign_extend6(code)) * float(scale)   (exact in fp32)
  slot    128 bytes per (b, kv head, t): K codes [0,48), K scales [48,52),
          V codes [52,100), V scales [100,104), z fp32[4] [104,120), zero [120,128)
"""

from __future__ import annotations

import numpy as np

GROUP = 32
SLOT = 128
HEAD_DIM = 64
FP16_MAX = np.float16(65504.0)


def quantize_groups(x: np.ndarray):
    """x [..., 32] float32 -> (codes int8 [..., 32], scale float16 [...])."""
    x = np.asarray(x, dtype=np.float32)
    amax = np.max(np.abs(x), axis=-1)
    with np.errstate(over="ignore"):
        scale = (amax / np.float32(31.0)).astype(np.float32).astype(np.float16)
    scale = np.where(np.isinf(scale), FP16_MAX, scale).astype(np.float16)
    sc32 = scale.astype(np.float32)[..., None]
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.rint(x / np.where(sc32 == 0, np.float32(1.0), sc32))
    codes = np.clip(r, -31, 31)
    codes = np.where(sc32 == 0, 0, codes).astype(np.int8)
    return codes, scale


def pack_codes(codes: np.ndarray) -> np.ndarray:
    """codes int8 [..., 32] -> bytes uint8 [..., 24]."""
    c = (codes.astype(np.int32) & 63).astype(np.uint32)
    c = c.reshape(*c.shape[:-1], GROUP // 4, 4)
    w = c[..., 0] | (c[..., 1] << 6) | (c[..., 2] << 12) | (c[..., 3] << 18)
    out = np.stack([w & 0xFF, (w >> 8) & 0xFF, (w >> 16) & 0xFF], axis=-1).astype(np.uint8)
    return out.reshape(*codes.shape[:-1], GROUP // 4 * 3)


def unpack_codes(b: np.ndarray) -> np.ndarray:
    """bytes uint8 [..., 24] -> codes int8 [..., 32] (sign-extended)."""
    b = b.astype(np.uint32).reshape(*b.shape[:-1], GROUP // 4, 3)
    w = b[..., 0] | (b[..., 1] << 8) | (b[..., 2] << 16)
    c = np.stack([(w >> (6 * i)) & 63 for i in range(4)], axis=-1).astype(np.int32)
    c = np.where(c >= 32, c - 64, c)
    return c.reshape(*b.shape[:-2], GROUP).astype(np.int8)


def dequantize(codes: np.ndarray, scale: np.ndarray) -> np.ndarray:
    return codes.astype(np.float32) * scale.astype(np.float32)[..., None]


def quantize_row(x: np.ndarray):
    """x [..., 64] -> (code bytes [..., 48], scale bytes [..., 4], dequantised [..., 64])."""
    g = np.asarray(x, dtype=np.float32).reshape(*x.shape[:-1], HEAD_DIM // GROUP, GROUP)
    codes, scale = quantize_groups(g)
    packed = pack_codes(codes).reshape(*x.shape[:-1], HEAD_DIM // GROUP * 24)
    sbytes = scale.view(np.uint8).reshape(*x.shape[:-1], HEAD_DIM // GROUP * 2)
    deq = dequantize(codes, scale).reshape(*x.shape[:-1], HEAD_DIM)
    return packed, sbytes, deq


def pack_slots(k: np.ndarray, v: np.ndarray, key_probes: np.ndarray | None = None) -> np.ndarray:
    """K, V [..., 64] float32 -> slots uint8 [..., 128]; z from the dequantised K."""
    kc, ks, kd = quantize_row(k)
    vc, vs, _ = quantize_row(v)
    slot = np.zeros((*k.shape[:-1], SLOT), dtype=np.uint8)
    slot[..., 0:48] = kc
    slot[..., 48:52] = ks
    slot[..., 52:100] = vc
    slot[..., 100:104] = vs
    if key_probes is not None:
        p = np.asarray(key_probes, dtype=np.float64)
        kd64 = kd.astype(np.float64)
        inv = 1.0 / np.sqrt((kd64 * kd64).sum(-1, keepdims=True) + 1e-6 * HEAD_DIM)
        z = (kd64 @ p.T) * inv
        slot[..., 104:120] = z.astype(np.float32).view(np.uint8).reshape(*k.shape[:-1], 16)
    return slot


def unpack_slots(slot: np.ndarray):
    """slots uint8 [..., 128] -> (K, V float32 [..., 64], z float32 [..., 4])."""
    def half(codes_lo, scale_lo):
        c = unpack_codes(slot[..., codes_lo:codes_lo + 48].reshape(*slot.shape[:-1], 2, 24))
        s = np.ascontiguousarray(slot[..., scale_lo:scale_lo + 4]).view(np.float16).reshape(*slot.shape[:-1], 2)
        return dequantize(c, s).reshape(*slot.shape[:-1], HEAD_DIM)
    k = half(0, 48)
    v = half(52, 100)
    z = np.ascontiguousarray(slot[..., 104:120]).view(np.float32).reshape(*slot.shape[:-1], 4)
    return k, v, z
