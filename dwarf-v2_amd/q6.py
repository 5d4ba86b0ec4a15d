"""q6 quantised K/V cache: GPU codec, prefill forward and decode step.

The reference repository has no q6 code (its .gitignore:37 keeps a private
q6 directory), so this format is this library's own: a 64-wide head row is
two groups of 32 values; each group stores an fp16 scale
fp16_rne(absmax/31) and signed 6-bit codes clamp(rint(x/scale), -31, 31),
packed 4 codes per 24-bit little-endian word.  A cache slot of 128 bytes per
(b, kv head, t) holds the K row (52 B), the V row (52 B) and z[4] fp32, the
key-probe feature of the dequantised K row (dsqg:3242-3254).

The attention math of prefill and decode is the DSQG forward
(dsqg:698-860) with K/V dequantised on read and y computed in-kernel from q.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

SLOT_BYTES = 128
GROUP = 32
HEAD_DIM = 64


def _p64(values):
    return _lib.i64_array(values)


def _u8p(t: torch.Tensor):
    return ctypes.cast(ctypes.c_void_p(t.data_ptr()), ctypes.POINTER(ctypes.c_uint8))


def _rows(t: torch.Tensor) -> torch.Tensor:
    per16 = 16 // t.element_size()
    ok = t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all(s % per16 == 0 for s in t.stride()[:-1])
    return t if ok else t.contiguous()


def normalized_probes(probes: torch.Tensor) -> torch.Tensor:
    """Row-normalised probes, as the module uses them (dsqg:3231-3232)."""
    return torch.nn.functional.normalize(probes.float(), dim=-1).contiguous()


def pack_kv(k: torch.Tensor, v: torch.Tensor, key_probes: torch.Tensor | None = None) -> torch.Tensor:
    """Quantise K/V [B,Hkv,N,64] (bf16 or fp32) into a uint8 cache [B,Hkv,N,128].

    ``key_probes`` [4,64] (normalised) fills the z bytes; None stores zeros.
    """
    if k.shape != v.shape or k.dim() != 4 or k.shape[-1] != HEAD_DIM:
        raise ValueError(f"k and v must share a [B,Hkv,N,{HEAD_DIM}] shape; got {tuple(k.shape)}, {tuple(v.shape)}")
    if not k.is_cuda:
        raise RuntimeError("the q6 HIP kernels require device tensors")
    dtype = torch.float32 if k.dtype == torch.float32 else torch.bfloat16
    k, v = _rows(k.to(dtype)), _rows(v.to(dtype))
    B, Hkv, N, _ = k.shape
    cache = torch.empty((B, Hkv, N, SLOT_BYTES), device=k.device, dtype=torch.uint8)
    kp = None if key_probes is None else key_probes.to(device=k.device, dtype=torch.float32).contiguous()
    lib = _lib.load()
    rc = lib.dwarf_q6_pack_kv(
        B, Hkv, N, HEAD_DIM, _lib.DWARF_F32 if dtype == torch.float32 else _lib.DWARF_BF16,
        k.data_ptr(), _p64(k.stride()), v.data_ptr(), _p64(v.stride()),
        _u8p(cache), _p64(cache.stride()[:3]), None if kp is None else kp.data_ptr(),
        torch.cuda.current_stream(k.device).cuda_stream,
    )
    _lib.check(rc, "dwarf_q6_pack_kv")
    return cache


def unpack_kv(cache: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Dequantise a cache [B,Hkv,N,128] into fp32 K and V [B,Hkv,N,64]."""
    if cache.dtype != torch.uint8 or cache.dim() != 4 or cache.shape[-1] != SLOT_BYTES:
        raise ValueError(f"cache must be uint8 [B,Hkv,N,{SLOT_BYTES}]")
    cache = cache.contiguous()
    B, Hkv, N, _ = cache.shape
    k = torch.empty((B, Hkv, N, HEAD_DIM), device=cache.device, dtype=torch.float32)
    v = torch.empty_like(k)
    lib = _lib.load()
    rc = lib.dwarf_q6_unpack_kv(B, Hkv, N, HEAD_DIM, _u8p(cache), _p64(cache.stride()[:3]), k.data_ptr(),
                                v.data_ptr(), torch.cuda.current_stream(cache.device).cuda_stream)
    _lib.check(rc, "dwarf_q6_unpack_kv")
    return k, v


def q6_prefill(q, cache, pos_bias, scale_embed, phase_base, phase_gain, query_probes, offsets_dev,
               j_small, j_large, plane_shift=0, query_start=0, *, return_lse=False, round_se=True, widen=True):
    """DSQG forward over a q6 cache.  q [B,H,N,64] bf16; returns bf16 out (and lse).  round_se rounds
    scale_embed to bf16 as the GPU path does (dsqg:760-763); False keeps it in fp32.

    widen=True widens every cache row once into a workspace (160 bytes per row: the codes as bytes, the
    scales and z) and gathers those; widen=False gathers the 128-byte slots and widens each code at every
    use, with no workspace.  Both compute the same math."""
    if not q.is_cuda:
        raise RuntimeError("the q6 HIP kernels require device tensors")
    q = _rows(q.to(torch.bfloat16))
    B, H, N, HD = q.shape
    if cache.shape[:3] != (B, cache.shape[1], N) or H % cache.shape[1]:
        raise ValueError(f"cache {tuple(cache.shape)} does not match q {tuple(q.shape)}")
    cache = cache.contiguous()
    pos_bias = pos_bias.float().contiguous()
    scale_embed = scale_embed.float().contiguous()
    phase_base = phase_base.float().contiguous()
    phase_gain = phase_gain.float().contiguous()
    qp = query_probes.float().contiguous()
    offsets = offsets_dev.to(device=q.device, dtype=torch.int32).contiguous()
    out = torch.empty((B, H, N, HD), device=q.device, dtype=torch.bfloat16)
    lse = torch.empty((B, H, N), device=q.device, dtype=torch.float32) if return_lse else None
    a = _lib.Q6PrefillArgs()
    a.B, a.H, a.H_kv, a.N, a.head_dim = B, H, cache.shape[1], N, HD
    a.J, a.J_small, a.J_large = int(j_small) + int(j_large), int(j_small), int(j_large)
    a.plane_shift, a.query_start = int(plane_shift), max(0, min(int(query_start), N))
    a.se_round_bf16 = int(bool(round_se))
    a.q, a.q_stride = q.data_ptr(), _p64(q.stride())
    a.cache, a.cache_stride = cache.data_ptr(), _p64(cache.stride()[:3])
    a.pos_bias, a.pb_stride = pos_bias.data_ptr(), _p64(pos_bias.stride())
    a.scale_embed, a.se_stride = scale_embed.data_ptr(), _p64(scale_embed.stride())
    a.phase_base, a.pbase_stride = phase_base.data_ptr(), _p64(phase_base.stride()[:2])
    a.phase_gain, a.pgain_stride = phase_gain.data_ptr(), _p64(phase_gain.stride()[:2])
    a.query_probes = qp.data_ptr()
    a.offsets = offsets.data_ptr()
    a.out, a.out_stride = out.data_ptr(), _p64(out.stride())
    if lse is not None:
        a.lse, a.lse_stride = lse.data_ptr(), _p64(lse.stride())
    lib = _lib.load()
    workspace = None
    if widen:
        nbytes = int(lib.dwarf_dsqg_q6_prefill_workspace_bytes(ctypes.byref(a)))
        workspace = torch.empty(max(nbytes, 256), device=q.device, dtype=torch.uint8)
        a.workspace, a.workspace_bytes = workspace.data_ptr(), workspace.numel()
    _lib.check(lib.dwarf_dsqg_q6_prefill_fwd(ctypes.byref(a), torch.cuda.current_stream(q.device).cuda_stream),
               "dwarf_dsqg_q6_prefill_fwd")
    return (out, lse) if return_lse else out


def _decode_args(q, pos, caches, pos_bias, scale_embed, phase_base, phase_gain, query_probes, offsets_dev,
                 j_small, j_large, plane_shift, round_se, out):
    """Validated tensors and the filled Q6DecodeArgs of one decode step (the tensors are returned so that
    they outlive the call)."""
    if not q.is_cuda:
        raise RuntimeError("the q6 HIP kernels require device tensors")
    q = _rows(q.to(torch.bfloat16))
    S, L, H, HD = q.shape
    caches = caches.contiguous()
    if caches.shape[0] != L or caches.shape[1] != S or caches.shape[-1] != SLOT_BYTES:
        raise ValueError(f"caches {tuple(caches.shape)} do not match q {tuple(q.shape)}")
    pos = pos.to(device=q.device, dtype=torch.int32).contiguous()
    pos_bias = pos_bias.float().contiguous()
    scale_embed = scale_embed.float().contiguous()
    phase_base = phase_base.float().contiguous()
    phase_gain = phase_gain.float().contiguous()
    qp = query_probes.float().contiguous()
    offsets = offsets_dev.to(device=q.device, dtype=torch.int32).contiguous()
    if out is None:
        out = torch.empty((S, L, H, HD), device=q.device, dtype=torch.bfloat16)
    elif out.shape != (S, L, H, HD) or out.dtype != torch.bfloat16 or out.device != q.device:
        raise ValueError(f"out must be a bf16 [{S},{L},{H},{HD}] tensor on {q.device}")
    a = _lib.Q6DecodeArgs()
    a.S, a.L, a.H, a.H_kv, a.Ncache, a.head_dim = S, L, H, caches.shape[2], caches.shape[3], HD
    a.J, a.J_small, a.J_large = int(j_small) + int(j_large), int(j_small), int(j_large)
    a.plane_shift = int(plane_shift)
    a.se_round_bf16 = int(bool(round_se))
    a.q, a.q_stride = q.data_ptr(), _p64(q.stride())
    a.pos = pos.data_ptr()
    a.cache, a.cache_stride = caches.data_ptr(), _p64(caches.stride()[:4])
    a.pos_bias, a.pb_stride = pos_bias.data_ptr(), _p64(pos_bias.stride())
    a.scale_embed, a.se_stride = scale_embed.data_ptr(), _p64(scale_embed.stride())
    a.phase_base, a.pbase_stride = phase_base.data_ptr(), _p64(phase_base.stride()[:3])
    a.phase_gain, a.pgain_stride = phase_gain.data_ptr(), _p64(phase_gain.stride()[:3])
    a.query_probes, a.qprobe_layer_stride = qp.data_ptr(), qp.stride(0)
    a.offsets = offsets.data_ptr()
    a.out, a.out_stride = out.data_ptr(), _p64(out.stride())
    keep = (q, caches, pos, pos_bias, scale_embed, phase_base, phase_gain, qp, offsets)
    return a, out, keep


def q6_decode(q, pos, caches, pos_bias, scale_embed, phase_base, phase_gain, query_probes, offsets_dev,
              j_small, j_large, plane_shift=0, round_se=True):
    """One decode step over L layers.

    q [S,L,H,64] bf16 (one new query per sequence and layer), pos [S] int32
    positions, caches [L,S,Hkv,Ncache,128] uint8, per-layer tables with a
    leading L dimension: pos_bias [L,J,H], scale_embed [L,J,64], phase_base /
    phase_gain [L,J_L,H,4], query_probes [L,4,64] (normalised).  Returns
    out [S,L,H,64] bf16.  round_se rounds scale_embed to bf16 as the GPU path
    does (dsqg:760-763); False keeps it in fp32 (bf16 hi + lo on the MFMA).
    """
    a, out, keep = _decode_args(q, pos, caches, pos_bias, scale_embed, phase_base, phase_gain, query_probes,
                                offsets_dev, j_small, j_large, plane_shift, round_se, None)
    lib = _lib.load()
    ws = torch.empty(max(int(lib.dwarf_dsqg_q6_decode_workspace_bytes(ctypes.byref(a))), 16), device=out.device,
                     dtype=torch.uint8)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    _lib.check(lib.dwarf_dsqg_q6_decode(ctypes.byref(a), torch.cuda.current_stream(out.device).cuda_stream),
               "dwarf_dsqg_q6_decode")
    del keep
    return out


def q6_decode_noalloc(q, pos, caches, pos_bias, scale_embed, phase_base, phase_gain, query_probes, offsets_dev,
                      j_small, j_large, plane_shift=0, round_se=True, *, out=None):
    """q6_decode through dwarf_dsqg_q6_decode_noalloc: the library allocates nothing (its score table is a
    per-GPU device array of 16 MiB, so S*L*H*JE fp32 must fit; concurrent calls on one GPU race).  Pass
    ``out`` (bf16 [S,L,H,64]) and already-normalised tensors to keep the whole call free of allocation."""
    a, out, keep = _decode_args(q, pos, caches, pos_bias, scale_embed, phase_base, phase_gain, query_probes,
                                offsets_dev, j_small, j_large, plane_shift, round_se, out)
    lib = _lib.load()
    _lib.check(lib.dwarf_dsqg_q6_decode_noalloc(ctypes.byref(a), torch.cuda.current_stream(out.device).cuda_stream),
               "dwarf_dsqg_q6_decode_noalloc")
    del keep
    return out
