"""The C-ABI library: exports, struct layout and host-side validation (no GPU).

No kernel is launched here: every call below fails validation on the host,
which the library does before touching the HIP runtime.
"""

import ctypes
import os
import re
import shutil
import subprocess

import pytest

from tests.conftest import ROOT

HEADER = os.path.join(ROOT, "include", "dwarf_dsqg.h")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(dwarf_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def lib(pkg):
    return pkg._lib.load()


def test_exports_every_declared_symbol(pkg, lib):
    names = declared_functions()
    assert len(names) == 34
    assert sorted(pkg._lib.EXPORTED_SYMBOLS) == names
    for name in names:
        assert hasattr(lib, name), name
    assert lib.dwarf_abi_version() == pkg._lib.ABI_VERSION


STRUCTS = {
    "dwarf_dsqg_fwd_args": "DsqgFwdArgs",
    "dwarf_dsqg_bwd_args": "DsqgBwdArgs",
    "dwarf_ema_fwd_args": "EmaFwdArgs",
    "dwarf_ema_bwd_args": "EmaBwdArgs",
    "dwarf_dsqg_q6_prefill_args": "Q6PrefillArgs",
    "dwarf_dsqg_q6_decode_args": "Q6DecodeArgs",
    "dwarf_phase_probe_fwd_args": "PhaseProbeFwdArgs",
    "dwarf_phase_probe_bwd_args": "PhaseProbeBwdArgs",
    "dwarf_npci_fwd_args": "NpciFwdArgs",
    "dwarf_npci_bwd_args": "NpciBwdArgs",
    "dwarf_packet_pool_fwd_args": "PacketPoolFwdArgs",
    "dwarf_packet_pool_bwd_args": "PacketPoolBwdArgs",
    "dwarf_packet_fwd_args": "PacketFwdArgs",
    "dwarf_packet_bwd_args": "PacketBwdArgs",
}


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_ctypes_layout_matches_header(pkg, tmp_path):
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "dwarf_dsqg.h"', "int main(void) {"]
    for cname, pyname in STRUCTS.items():
        struct = getattr(pkg._lib, pyname)
        lines.append(f'printf("{cname} sizeof %zu\\n", sizeof({cname}));')
        for field, _ in struct._fields_:
            lines.append(f'printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.dirname(HEADER), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    for line in filter(None, out):
        cname, field, value = line.split()
        struct = getattr(pkg._lib, STRUCTS[cname])
        got = ctypes.sizeof(struct) if field == "sizeof" else getattr(struct, field).offset
        assert got == int(value), (cname, field, got, value)


def test_validation_errors_without_gpu(pkg, lib):
    L = pkg._lib
    assert lib.dwarf_dsqg_fwd(None, None) == L.DWARF_ERR_INVALID_ARGUMENT
    assert b"NULL" in lib.dwarf_last_error()
    a = L.DsqgFwdArgs()
    a.B, a.H, a.H_kv, a.N, a.head_dim, a.J, a.J_small, a.J_large = 1, 3, 2, 16, 64, 2, 1, 1
    assert lib.dwarf_dsqg_fwd(ctypes.byref(a), None) == L.DWARF_ERR_INVALID_ARGUMENT
    assert b"divisible" in lib.dwarf_last_error()
    a.H_kv, a.head_dim = 1, 128
    assert lib.dwarf_dsqg_fwd(ctypes.byref(a), None) == L.DWARF_ERR_UNSUPPORTED
    a.head_dim, a.plane_shift = 64, 15
    assert lib.dwarf_dsqg_fwd(ctypes.byref(a), None) == L.DWARF_ERR_INVALID_ARGUMENT
    assert b"plane_shift" in lib.dwarf_last_error()
    a.plane_shift, a.J = 0, 5
    assert lib.dwarf_dsqg_fwd(ctypes.byref(a), None) == L.DWARF_ERR_INVALID_ARGUMENT
    a.J, a.query_start = 2, 17
    assert lib.dwarf_dsqg_fwd(ctypes.byref(a), None) == L.DWARF_ERR_INVALID_ARGUMENT
    a.query_start = 0
    assert lib.dwarf_dsqg_fwd(ctypes.byref(a), None) == L.DWARF_ERR_INVALID_ARGUMENT  # q is NULL
    assert b"q is NULL" in lib.dwarf_last_error()
    e = L.EmaFwdArgs()
    e.B, e.N, e.D, e.floor_, e.ceiling = 1, 4, 4, 0.6, 0.5
    assert lib.dwarf_ema_fwd(ctypes.byref(e), None) == L.DWARF_ERR_INVALID_ARGUMENT
    with pytest.raises(ValueError):
        L.check(lib.dwarf_ema_fwd(ctypes.byref(e), None), "dwarf_ema_fwd")
    d = L.Q6DecodeArgs()
    d.S, d.L, d.H, d.H_kv, d.Ncache, d.head_dim, d.J, d.J_small, d.J_large = 1, 1, 1, 1, 64, 64, 300, 150, 150
    assert lib.dwarf_dsqg_q6_decode(ctypes.byref(d), None) == L.DWARF_ERR_UNSUPPORTED   # more than 256 offsets
    d.J, d.J_small, d.J_large, d.H, d.H_kv = 96, 17, 79, 32, 32
    assert lib.dwarf_dsqg_q6_decode(ctypes.byref(d), None) == L.DWARF_ERR_UNSUPPORTED   # one wave per head, <= 16
    assert b"heads" in lib.dwarf_last_error()
    d.S, d.L, d.H, d.H_kv = 3, 2, 8, 8   # the T table: S*L*H rows of JE = 112 fp32 at J = 96
    assert lib.dwarf_dsqg_q6_decode_workspace_bytes(ctypes.byref(d)) == 3 * 2 * 8 * 112 * 4
    # the no-allocation decode keeps the table in a 16 MiB device array: 4,681 x 1 x 8 x 112 fp32 fit
    # (16,776,704 bytes), one sequence more does not; rejected before any pointer or HIP call
    d.S, d.L = 4682, 1
    assert lib.dwarf_dsqg_q6_decode_noalloc(ctypes.byref(d), None) == L.DWARF_ERR_UNSUPPORTED
    assert b"16777216-byte device array" in lib.dwarf_last_error()
    d.S = 4681
    assert lib.dwarf_dsqg_q6_decode_noalloc(ctypes.byref(d), None) == L.DWARF_ERR_INVALID_ARGUMENT   # q is NULL
    assert lib.dwarf_dsqg_q6_decode_noalloc(None, None) == L.DWARF_ERR_INVALID_ARGUMENT
    p = L.PhaseProbeFwdArgs()
    p.B, p.H, p.N, p.head_dim, p.R, p.end = 1, 1, 8, 32, 4, 8
    assert lib.dwarf_phase_probe_fwd(ctypes.byref(p), None) == L.DWARF_ERR_UNSUPPORTED   # head_dim 64 only
    p.head_dim, p.R = 64, 3
    assert lib.dwarf_phase_probe_fwd(ctypes.byref(p), None) == L.DWARF_ERR_UNSUPPORTED   # four probes only
    p.R, p.dtype = 4, L.DWARF_BF16
    assert lib.dwarf_phase_probe_fwd(ctypes.byref(p), None) == L.DWARF_ERR_INVALID_ARGUMENT   # x is NULL
    pb = L.PhaseProbeBwdArgs()
    pb.fwd = p
    assert lib.dwarf_phase_probe_bwd(ctypes.byref(pb), None) == L.DWARF_ERR_INVALID_ARGUMENT
    n = L.NpciFwdArgs()
    n.B, n.H, n.T, n.head_dim, n.strength_tau = 1, 1, 4, 32, 0.25
    assert lib.dwarf_npci_fwd(ctypes.byref(n), None) == L.DWARF_ERR_UNSUPPORTED   # head_dim 64 only
    n.head_dim, n.strength_tau = 64, -1.0
    assert lib.dwarf_npci_fwd(ctypes.byref(n), None) == L.DWARF_ERR_INVALID_ARGUMENT   # tau must be positive
    n.strength_tau = 0.25
    assert lib.dwarf_npci_fwd(ctypes.byref(n), None) == L.DWARF_ERR_INVALID_ARGUMENT   # x is NULL
    k = L.PacketPoolFwdArgs()
    k.B, k.N, k.D, k.K, k.dtype, k.floor_, k.ceiling = 1, 32, 8, 5, L.DWARF_BF16, 1e-5, 0.5
    assert lib.dwarf_packet_pool_fwd(ctypes.byref(k), None) == L.DWARF_ERR_UNSUPPORTED   # at most 4 scales
    assert lib.dwarf_packet_pool_state_bytes(ctypes.byref(k)) == 0
    k.K = 3
    assert lib.dwarf_packet_pool_state_bytes(ctypes.byref(k)) == 1 * 2 * 3 * 8 * 4      # [B][N/16][K*D] fp32
    assert lib.dwarf_packet_pool_fwd(ctypes.byref(k), None) == L.DWARF_ERR_INVALID_ARGUMENT   # alpha is NULL
    k.floor_, k.ceiling = 0.6, 0.5
    assert lib.dwarf_packet_pool_fwd(ctypes.byref(k), None) == L.DWARF_ERR_INVALID_ARGUMENT   # bad bounds
    kb = L.PacketPoolBwdArgs()
    kb.fwd = k
    assert lib.dwarf_packet_pool_bwd(ctypes.byref(kb), None) == L.DWARF_ERR_INVALID_ARGUMENT
    # the larger of the three-stage backward's (starts and carries [B][N/16][K*D] fp32, then 2K slots per
    # apply workgroup, one here: 408 bytes) and the look-back's: a 256-byte head, the words of K scales
    # (one workgroup tile's aggregates, 16 VEC channels; VEC 4 is the larger; a single run keeps no run
    # states), then 2K slots per workgroup
    three_stage = (2 * 1 * 2 * 3 * 8 + 2 * 3) * 4
    lookback = 256 + 3 * 64 * 8 + 2 * 3 * 4
    assert lib.dwarf_packet_pool_bwd_workspace_bytes(ctypes.byref(kb)) == max(three_stage, lookback)
    pf = L.PacketFwdArgs()
    pf.pool = k
    pf.pool.floor_, pf.pool.ceiling = 1e-5, 0.5
    pf.pool.alpha = pf.pool.weight = 0x10000
    pf.packet_dtype = 7
    assert lib.dwarf_packet_fwd(ctypes.byref(pf), None) == L.DWARF_ERR_INVALID_ARGUMENT   # packet dtype
    assert b"packet_dtype" in lib.dwarf_last_error()
    pf.packet_dtype, pf.pool.D = L.DWARF_BF16, 4100
    assert lib.dwarf_packet_fwd(ctypes.byref(pf), None) == L.DWARF_ERR_UNSUPPORTED       # D above 4096
    pbk = L.PacketBwdArgs()
    pbk.fwd = pf
    pbk.fwd.pool.D = 8
    # the pool's backward workspace (256-byte aligned), then dpooled [B,N,D] bf16
    assert lib.dwarf_packet_bwd_workspace_bytes(ctypes.byref(pbk)) == 2048 + 1 * 32 * 8 * 2   # 1816 -> 2048
    assert lib.dwarf_packet_bwd(ctypes.byref(pbk), None) == L.DWARF_ERR_INVALID_ARGUMENT  # x is NULL


def _fake_fwd(L, B, H, H_kv, N, J, J_small):
    """Forward args with aligned placeholder pointers (validation never dereferences them)."""
    a = L.DsqgFwdArgs()
    a.B, a.H, a.H_kv, a.N, a.head_dim = B, H, H_kv, N, 64
    a.J, a.J_small, a.J_large = J, J_small, J - J_small
    a.dtype = L.DWARF_BF16
    p = 0x10000
    for name in ("q", "k", "v", "out"):
        setattr(a, name, p)
    for name, rows in (("q", H), ("out", H), ("k", H_kv), ("v", H_kv)):
        setattr(a, name + "_stride", L.i64_array((rows * N * 64, N * 64, 64, 1)))
    a.pos_bias = a.scale_embed = a.phase_base = a.phase_gain = a.lse = p
    a.y_pre, a.z_pre, a.offsets = p, p, p
    a.y_stride = L.i64_array((H * N * 4, N * 4, 4))
    a.z_stride = L.i64_array((H_kv * N * 4, N * 4, 4))
    a.lse_stride = L.i64_array((H * N, N, 1))
    return a


def test_backward_limits_without_gpu(pkg, lib):
    """bf16 backward shapes the kernels cannot address or stage are refused before any launch: the dS
    matrix's 32-bit offsets (4 J N bytes per (b, h)) and the dK/dV launch's LDS tables of a GQA group."""
    L = pkg._lib
    b = L.DsqgBwdArgs()
    b.fwd = _fake_fwd(L, 1, 1, 1, 2_100_000, 256, 17)         # 4 x 256 x 2.1M bytes of dS
    b.dout, b.dout_stride = 0x10000, L.i64_array((2_100_000 * 64, 2_100_000 * 64, 64, 1))
    assert lib.dwarf_dsqg_bwd_dq(ctypes.byref(b), None) == L.DWARF_ERR_UNSUPPORTED
    assert b"dS" in lib.dwarf_last_error()
    b.fwd = _fake_fwd(L, 1, 16, 1, 512, 256, 17)              # 16 heads' tables per KV head at J = 256
    b.dout_stride = L.i64_array((16 * 512 * 64, 512 * 64, 64, 1))
    assert lib.dwarf_dsqg_bwd_dkdv(ctypes.byref(b), None) == L.DWARF_ERR_UNSUPPORTED
    assert b"LDS" in lib.dwarf_last_error()


def test_gqa_head_split_workspace_without_gpu(pkg, lib):
    """bf16 dK/dV with grouped heads splits the query heads of the (key tile, KV head) units past the 768 that
    one round of resident workgroups takes whole, and keeps their fp32 partials (dK and dV 64 floats each, dZ
    4, per key of the unit's 64 and subset) in the workspace: B1 H8 over one KV head at N 2048 (32 units, no
    whole round) takes all 8 subsets of every unit; B15 over 2 KV heads (960 units) splits the last 192 in 4;
    B15 over one KV head at N 8192 (1,920 units, two rounds) and fp32 split none, so those sizes equal the MHA
    layout's."""
    L = pkg._lib

    def need(B, H, H_kv, N, dtype):
        b = L.DsqgBwdArgs()
        b.fwd = _fake_fwd(L, B, H, H_kv, N, 96, 17)
        b.fwd.dtype = dtype
        b.dout, b.dout_stride = 0x10000, L.i64_array((H * N * 64, N * 64, 64, 1))
        return lib.dwarf_dsqg_bwd_workspace_bytes(ctypes.byref(b))

    assert need(1, 8, 1, 2048, L.DWARF_BF16) - need(1, 8, 8, 2048, L.DWARF_BF16) == 8 * 2048 * (2 * 64 + 4) * 4
    assert need(2, 8, 1, 2048, L.DWARF_BF16) - need(2, 8, 8, 2048, L.DWARF_BF16) == 8 * 2 * 2048 * (2 * 64 + 4) * 4
    assert need(15, 8, 2, 2048, L.DWARF_BF16) - need(15, 8, 8, 2048, L.DWARF_BF16) == 4 * 192 * 64 * (2 * 64 + 4) * 4
    assert need(15, 8, 1, 8192, L.DWARF_BF16) == need(15, 8, 8, 8192, L.DWARF_BF16)
    assert need(1, 8, 1, 2048, L.DWARF_F32) == need(1, 8, 8, 2048, L.DWARF_F32)


def test_prefill_gather_span_without_gpu(pkg, lib):
    """The q6 prefill gathers cache rows with 32-bit offsets: (2N + 128) x 128 B must stay below 2 GiB."""
    L = pkg._lib
    a = L.Q6PrefillArgs()
    N = 8_400_000
    a.B, a.H, a.H_kv, a.N, a.head_dim, a.J, a.J_small, a.J_large = 1, 1, 1, N, 64, 96, 17, 79
    a.q = a.out = a.cache = 0x10000
    a.q_stride = a.out_stride = L.i64_array((N * 64, N * 64, 64, 1))
    a.cache_stride = L.i64_array((N * 128, N * 128, 128))
    assert lib.dwarf_dsqg_q6_prefill_fwd(ctypes.byref(a), None) == L.DWARF_ERR_UNSUPPORTED
    assert b"cache" in lib.dwarf_last_error()


def test_prefill_workspace_without_gpu(pkg, lib):
    """The widened-row prefill: its workspace size, and a short, misaligned or unaddressable workspace refused
    before any launch (a NULL workspace keeps the direct slot schedule)."""
    L = pkg._lib
    a = L.Q6PrefillArgs()
    a.B, a.H, a.H_kv, a.N, a.head_dim, a.J, a.J_small, a.J_large = 2, 6, 3, 100, 64, 96, 17, 79
    assert lib.dwarf_dsqg_q6_prefill_workspace_bytes(ctypes.byref(a)) == 2 * 3 * 100 * 160
    assert lib.dwarf_dsqg_q6_prefill_workspace_bytes(None) == 0
    N = a.N
    a.q = a.out = a.cache = 0x10000
    a.q_stride = a.out_stride = L.i64_array((6 * N * 64, N * 64, 64, 1))
    a.cache_stride = L.i64_array((3 * N * 128, N * 128, 128))
    a.pos_bias = a.scale_embed = a.phase_base = a.phase_gain = a.offsets = a.query_probes = 0x10000
    a.workspace, a.workspace_bytes = 0x10000, 2 * 3 * 100 * 160 - 1
    assert lib.dwarf_dsqg_q6_prefill_fwd(ctypes.byref(a), None) == L.DWARF_ERR_WORKSPACE
    assert b"needs 96000 bytes" in lib.dwarf_last_error()
    a.workspace, a.workspace_bytes = 0x10010, 2 * 3 * 100 * 160
    assert lib.dwarf_dsqg_q6_prefill_fwd(ctypes.byref(a), None) == L.DWARF_ERR_WORKSPACE
    assert b"256-byte aligned" in lib.dwarf_last_error()
    # 160-byte rows reach 2 GiB of 32-bit gather offsets sooner than the 128-byte slots do
    N = 6_800_000
    a.B, a.H, a.H_kv, a.N = 1, 1, 1, N
    a.q_stride = a.out_stride = L.i64_array((N * 64, N * 64, 64, 1))
    a.cache_stride = L.i64_array((N * 128, N * 128, 128))
    a.workspace, a.workspace_bytes = 0x10000, N * 160
    assert lib.dwarf_dsqg_q6_prefill_fwd(ctypes.byref(a), None) == L.DWARF_ERR_UNSUPPORTED
    assert b"widened" in lib.dwarf_last_error()


def test_delta_stage_validation_without_gpu(pkg, lib):
    """dwarf_dsqg_bwd_delta refuses a NULL argument block, fp32 (the fp32 dQ launch forms delta itself)
    and a missing or short workspace before any launch; an empty batch is a no-op."""
    L = pkg._lib
    assert lib.dwarf_dsqg_bwd_delta(None, None) == L.DWARF_ERR_INVALID_ARGUMENT
    b = L.DsqgBwdArgs()
    b.fwd = _fake_fwd(L, 1, 2, 2, 256, 96, 17)
    b.fwd.schedule = L.DWARF_SCHED_DELTA_STAGE
    b.dout, b.dout_stride = 0x10000, L.i64_array((2 * 256 * 64, 256 * 64, 64, 1))
    assert lib.dwarf_dsqg_bwd_delta(ctypes.byref(b), None) == L.DWARF_ERR_WORKSPACE
    need = lib.dwarf_dsqg_bwd_workspace_bytes(ctypes.byref(b))
    assert need > 0
    b.workspace, b.workspace_bytes = 0x10000, need - 256
    assert lib.dwarf_dsqg_bwd_delta(ctypes.byref(b), None) == L.DWARF_ERR_WORKSPACE
    b.fwd.dtype = L.DWARF_F32
    assert lib.dwarf_dsqg_bwd_delta(ctypes.byref(b), None) == L.DWARF_ERR_UNSUPPORTED
    b.fwd.dtype = L.DWARF_BF16
    b.fwd.B = 0
    assert lib.dwarf_dsqg_bwd_delta(ctypes.byref(b), None) == L.DWARF_OK


def test_unknown_schedule_bits_refused_without_gpu(pkg, lib):
    """Schedule bits outside DWARF_SCHED_BAND | TWO_PASS | DELTA_STAGE are refused by the forward and by
    every backward stage before any launch; each known flag alone passes validation up to the workspace."""
    L = pkg._lib
    a = _fake_fwd(L, 1, 2, 2, 256, 96, 17)
    for bad in (8, 16, 1 << 30, -1):
        a.schedule = bad
        assert lib.dwarf_dsqg_fwd(ctypes.byref(a), None) == L.DWARF_ERR_INVALID_ARGUMENT
        assert b"schedule" in lib.dwarf_last_error()
    b = L.DsqgBwdArgs()
    b.fwd = _fake_fwd(L, 1, 2, 2, 256, 96, 17)
    b.dout, b.dout_stride = 0x10000, L.i64_array((2 * 256 * 64, 256 * 64, 64, 1))
    for fn in (lib.dwarf_dsqg_bwd, lib.dwarf_dsqg_bwd_dq, lib.dwarf_dsqg_bwd_params, lib.dwarf_dsqg_bwd_dkdv,
               lib.dwarf_dsqg_bwd_delta):
        b.fwd.schedule = L.DWARF_SCHED_BAND | 32
        assert fn(ctypes.byref(b), None) == L.DWARF_ERR_INVALID_ARGUMENT
        assert b"schedule" in lib.dwarf_last_error()
    for good in (0, L.DWARF_SCHED_BAND, L.DWARF_SCHED_TWO_PASS, L.DWARF_SCHED_DELTA_STAGE, 7):
        b.fwd.schedule = good
        assert lib.dwarf_dsqg_bwd_delta(ctypes.byref(b), None) == L.DWARF_ERR_WORKSPACE   # got past the flags
