"""ctypes binding of libdwarf_dsqg.so (declarations: include/dwarf_dsqg.h).

The structures below mirror the C structs field for field.  Loading never
builds anything: a missing library raises, so no code path silently falls
back to a CPU implementation.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_int64, c_size_t, c_uint8, c_void_p

LIB_NAME = "libdwarf_dsqg.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
ABI_VERSION = 9

DWARF_OK = 0
DWARF_ERR_INVALID_ARGUMENT = 1
DWARF_ERR_UNSUPPORTED = 2
DWARF_ERR_HIP = 3
DWARF_ERR_WORKSPACE = 4

DWARF_BF16 = 0
DWARF_F32 = 1

EXPORTED_SYMBOLS = (
    "dwarf_abi_version",
    "dwarf_last_error",
    "dwarf_dsqg_fwd",
    "dwarf_dsqg_bwd_workspace_bytes",
    "dwarf_dsqg_bwd",
    "dwarf_dsqg_bwd_dq",
    "dwarf_dsqg_bwd_params",
    "dwarf_dsqg_bwd_dkdv",
    "dwarf_dsqg_bwd_delta",
    "dwarf_ema_fwd_workspace_bytes",
    "dwarf_ema_fwd",
    "dwarf_ema_bwd_workspace_bytes",
    "dwarf_ema_bwd",
    "dwarf_q6_pack_kv",
    "dwarf_q6_unpack_kv",
    "dwarf_dsqg_q6_prefill_workspace_bytes",
    "dwarf_dsqg_q6_prefill_fwd",
    "dwarf_dsqg_q6_decode",
    "dwarf_dsqg_q6_decode_workspace_bytes",
    "dwarf_dsqg_q6_decode_noalloc",
    "dwarf_phase_probe_fwd",
    "dwarf_phase_probe_bwd_workspace_bytes",
    "dwarf_phase_probe_bwd",
    "dwarf_npci_fwd",
    "dwarf_npci_bwd_workspace_bytes",
    "dwarf_npci_bwd",
    "dwarf_packet_pool_state_bytes",
    "dwarf_packet_pool_fwd_workspace_bytes",
    "dwarf_packet_pool_fwd",
    "dwarf_packet_pool_bwd_workspace_bytes",
    "dwarf_packet_pool_bwd",
    "dwarf_packet_fwd",
    "dwarf_packet_bwd_workspace_bytes",
    "dwarf_packet_bwd",
)


def _i64(n):
    return c_int64 * n


class DsqgFwdArgs(ctypes.Structure):
    _fields_ = [
        ("B", c_int32), ("H", c_int32), ("H_kv", c_int32), ("N", c_int32), ("head_dim", c_int32),
        ("J", c_int32), ("J_small", c_int32), ("J_large", c_int32),
        ("plane_shift", c_int32), ("query_start", c_int32),
        ("dtype", c_int32), ("se_round_bf16", c_int32),
        ("q", c_void_p), ("q_stride", _i64(4)),
        ("k", c_void_p), ("k_stride", _i64(4)),
        ("v", c_void_p), ("v_stride", _i64(4)),
        ("pos_bias", c_void_p), ("pb_stride", _i64(2)),
        ("scale_embed", c_void_p), ("se_stride", _i64(2)),
        ("phase_base", c_void_p), ("pbase_stride", _i64(2)),
        ("phase_gain", c_void_p), ("pgain_stride", _i64(2)),
        ("y_pre", c_void_p), ("y_stride", _i64(3)),
        ("z_pre", c_void_p), ("z_stride", _i64(3)),
        ("offsets", c_void_p),
        ("out", c_void_p), ("out_stride", _i64(4)),
        ("lse", c_void_p), ("lse_stride", _i64(3)),
        ("schedule", c_int32),
        ("query_probes", c_void_p), ("key_probes", c_void_p), ("y_out", c_void_p),
    ]


DWARF_SCHED_BAND = 1
DWARF_SCHED_TWO_PASS = 2
DWARF_SCHED_DELTA_STAGE = 4


class DsqgBwdArgs(ctypes.Structure):
    _fields_ = [
        ("fwd", DsqgFwdArgs),
        ("dout", c_void_p), ("dout_stride", _i64(4)),
        ("dq", c_void_p), ("dq_stride", _i64(4)),
        ("dk", c_void_p), ("dk_stride", _i64(4)),
        ("dv", c_void_p), ("dv_stride", _i64(4)),
        ("dpos_bias", c_void_p),
        ("dscale_embed", c_void_p),
        ("dphase_base", c_void_p),
        ("dphase_gain", c_void_p),
        ("dy_pre", c_void_p),
        ("dz_pre", c_void_p),
        ("workspace", c_void_p), ("workspace_bytes", c_size_t),
    ]


class EmaFwdArgs(ctypes.Structure):
    _fields_ = [
        ("B", c_int32), ("N", c_int32), ("D", c_int32),
        ("dtype", c_int32), ("alpha_per_channel", c_int32),
        ("floor_", c_float), ("ceiling", c_float),
        ("x", c_void_p), ("x_stride", _i64(3)),
        ("alpha", c_void_p),
        ("y", c_void_p), ("y_stride", _i64(3)),
        ("workspace", c_void_p), ("workspace_bytes", c_size_t),
        ("reset", c_void_p), ("reset_stride", _i64(2)),
        ("wait_limit", c_int32),
    ]


class EmaBwdArgs(ctypes.Structure):
    _fields_ = [
        ("B", c_int32), ("N", c_int32), ("D", c_int32),
        ("dtype", c_int32), ("alpha_per_channel", c_int32),
        ("floor_", c_float), ("ceiling", c_float),
        ("x", c_void_p), ("x_stride", _i64(3)),
        ("y", c_void_p), ("y_stride", _i64(3)),
        ("dy", c_void_p), ("dy_stride", _i64(3)),
        ("alpha", c_void_p),
        ("dx", c_void_p), ("dx_stride", _i64(3)),
        ("dalpha", c_void_p),
        ("workspace", c_void_p), ("workspace_bytes", c_size_t),
        ("reset", c_void_p), ("reset_stride", _i64(2)),
        ("wait_limit", c_int32),
    ]


class Q6PrefillArgs(ctypes.Structure):
    _fields_ = [
        ("B", c_int32), ("H", c_int32), ("H_kv", c_int32), ("N", c_int32), ("head_dim", c_int32),
        ("J", c_int32), ("J_small", c_int32), ("J_large", c_int32),
        ("plane_shift", c_int32), ("query_start", c_int32),
        ("se_round_bf16", c_int32),
        ("q", c_void_p), ("q_stride", _i64(4)),
        ("cache", c_void_p), ("cache_stride", _i64(3)),
        ("pos_bias", c_void_p), ("pb_stride", _i64(2)),
        ("scale_embed", c_void_p), ("se_stride", _i64(2)),
        ("phase_base", c_void_p), ("pbase_stride", _i64(2)),
        ("phase_gain", c_void_p), ("pgain_stride", _i64(2)),
        ("query_probes", c_void_p),
        ("offsets", c_void_p),
        ("out", c_void_p), ("out_stride", _i64(4)),
        ("lse", c_void_p), ("lse_stride", _i64(3)),
        ("workspace", c_void_p), ("workspace_bytes", c_size_t),
    ]


class Q6DecodeArgs(ctypes.Structure):
    _fields_ = [
        ("S", c_int32), ("L", c_int32), ("H", c_int32), ("H_kv", c_int32), ("Ncache", c_int32),
        ("head_dim", c_int32),
        ("J", c_int32), ("J_small", c_int32), ("J_large", c_int32),
        ("plane_shift", c_int32),
        ("se_round_bf16", c_int32),
        ("q", c_void_p), ("q_stride", _i64(4)),
        ("pos", c_void_p),
        ("cache", c_void_p), ("cache_stride", _i64(4)),
        ("pos_bias", c_void_p), ("pb_stride", _i64(3)),
        ("scale_embed", c_void_p), ("se_stride", _i64(3)),
        ("phase_base", c_void_p), ("pbase_stride", _i64(3)),
        ("phase_gain", c_void_p), ("pgain_stride", _i64(3)),
        ("query_probes", c_void_p), ("qprobe_layer_stride", c_int64),
        ("offsets", c_void_p),
        ("out", c_void_p), ("out_stride", _i64(4)),
        ("workspace", c_void_p), ("workspace_bytes", c_size_t),
    ]


_LIB = None


class PhaseProbeFwdArgs(ctypes.Structure):
    _fields_ = [
        ("B", c_int32), ("H", c_int32), ("N", c_int32), ("head_dim", c_int32), ("R", c_int32),
        ("start", c_int32), ("end", c_int32),
        ("dtype", c_int32),
        ("x", c_void_p), ("x_stride", _i64(4)),
        ("probes", c_void_p),
        ("out", c_void_p), ("out_stride", _i64(4)),
    ]


class PhaseProbeBwdArgs(ctypes.Structure):
    _fields_ = [
        ("fwd", PhaseProbeFwdArgs),
        ("dout", c_void_p), ("dout_stride", _i64(4)),
        ("dx", c_void_p), ("dx_stride", _i64(4)),
        ("dprobes", c_void_p),
        ("workspace", c_void_p), ("workspace_bytes", c_size_t),
    ]


class NpciFwdArgs(ctypes.Structure):
    _fields_ = [
        ("B", c_int32), ("H", c_int32), ("T", c_int32), ("head_dim", c_int32),
        ("x_dtype", c_int32), ("delta_dtype", c_int32),
        ("strength_tau", c_float),
        ("x", c_void_p), ("x_stride", _i64(4)),
        ("delta", c_void_p), ("delta_stride", _i64(4)),
        ("theta", c_void_p),
        ("out", c_void_p), ("out_stride", _i64(4)),
    ]


class NpciBwdArgs(ctypes.Structure):
    _fields_ = [
        ("fwd", NpciFwdArgs),
        ("grad", c_void_p), ("grad_stride", _i64(4)),
        ("dx", c_void_p), ("dx_stride", _i64(4)),
        ("ddelta", c_void_p), ("ddelta_stride", _i64(4)),
        ("dtheta", c_void_p),
        ("workspace", c_void_p), ("workspace_bytes", c_size_t),
    ]


PACKET_MAX_SCALES = 4


class PacketPoolFwdArgs(ctypes.Structure):
    _fields_ = [
        ("B", c_int32), ("N", c_int32), ("D", c_int32), ("K", c_int32),
        ("dtype", c_int32),
        ("floor_", c_float), ("ceiling", c_float),
        ("x", c_void_p), ("x_stride", _i64(3)),
        ("alpha", c_void_p),
        ("weight", c_void_p),
        ("pooled", c_void_p), ("pooled_stride", _i64(3)),
        ("state", c_void_p),
        ("workspace", c_void_p), ("workspace_bytes", c_size_t),
    ]


class PacketPoolBwdArgs(ctypes.Structure):
    _fields_ = [
        ("fwd", PacketPoolFwdArgs),
        ("dpooled", c_void_p), ("dpooled_stride", _i64(3)),
        ("dx", c_void_p), ("dx_stride", _i64(3)),
        ("dalpha", c_void_p),
        ("dweight", c_void_p),
        ("workspace", c_void_p), ("workspace_bytes", c_size_t),
    ]


class PacketFwdArgs(ctypes.Structure):
    _fields_ = [
        ("pool", PacketPoolFwdArgs),
        ("packet_dtype", c_int32),
        ("gate", c_void_p), ("gate_stride", _i64(3)),
        ("packet", c_void_p), ("packet_stride", _i64(3)),
        ("ms", c_void_p),
    ]


class PacketBwdArgs(ctypes.Structure):
    _fields_ = [
        ("fwd", PacketFwdArgs),
        ("dpacket", c_void_p), ("dpacket_stride", _i64(3)),
        ("dgate", c_void_p), ("dgate_stride", _i64(3)),
        ("dx", c_void_p), ("dx_stride", _i64(3)),
        ("dalpha", c_void_p),
        ("dweight", c_void_p),
        ("workspace", c_void_p), ("workspace_bytes", c_size_t),
    ]


class NativeLibraryError(RuntimeError):
    """The HIP library is missing, stale or failed a call."""


def library_path() -> str:
    return LIB_PATH


def load() -> ctypes.CDLL:
    """Load libdwarf_dsqg.so once, declaring every entry point's signature."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise NativeLibraryError(
            f"{LIB_NAME} is not built at {LIB_PATH}; build it with "
            "`make -C dwarf-v2_amd/csrc` or __graft_entry__.build()"
        )
    lib = ctypes.CDLL(LIB_PATH)
    lib.dwarf_abi_version.restype = c_int
    lib.dwarf_abi_version.argtypes = []
    lib.dwarf_last_error.restype = c_char_p
    lib.dwarf_last_error.argtypes = []
    lib.dwarf_dsqg_fwd.restype = c_int
    lib.dwarf_dsqg_fwd.argtypes = [POINTER(DsqgFwdArgs), c_void_p]
    lib.dwarf_dsqg_bwd_workspace_bytes.restype = c_size_t
    lib.dwarf_dsqg_bwd_workspace_bytes.argtypes = [POINTER(DsqgBwdArgs)]
    lib.dwarf_dsqg_bwd.restype = c_int
    lib.dwarf_dsqg_bwd.argtypes = [POINTER(DsqgBwdArgs), c_void_p]
    for name in ("dwarf_dsqg_bwd_dq", "dwarf_dsqg_bwd_params", "dwarf_dsqg_bwd_dkdv", "dwarf_dsqg_bwd_delta"):
        getattr(lib, name).restype = c_int
        getattr(lib, name).argtypes = [POINTER(DsqgBwdArgs), c_void_p]
    lib.dwarf_ema_fwd_workspace_bytes.restype = c_size_t
    lib.dwarf_ema_fwd_workspace_bytes.argtypes = [POINTER(EmaFwdArgs)]
    lib.dwarf_ema_fwd.restype = c_int
    lib.dwarf_ema_fwd.argtypes = [POINTER(EmaFwdArgs), c_void_p]
    lib.dwarf_ema_bwd_workspace_bytes.restype = c_size_t
    lib.dwarf_ema_bwd_workspace_bytes.argtypes = [POINTER(EmaBwdArgs)]
    lib.dwarf_ema_bwd.restype = c_int
    lib.dwarf_ema_bwd.argtypes = [POINTER(EmaBwdArgs), c_void_p]
    lib.dwarf_q6_pack_kv.restype = c_int
    lib.dwarf_q6_pack_kv.argtypes = [
        c_int32, c_int32, c_int32, c_int32, c_int32,
        c_void_p, POINTER(c_int64), c_void_p, POINTER(c_int64),
        POINTER(c_uint8), POINTER(c_int64), c_void_p, c_void_p,
    ]
    lib.dwarf_q6_unpack_kv.restype = c_int
    lib.dwarf_q6_unpack_kv.argtypes = [
        c_int32, c_int32, c_int32, c_int32,
        POINTER(c_uint8), POINTER(c_int64), c_void_p, c_void_p, c_void_p,
    ]
    lib.dwarf_dsqg_q6_prefill_workspace_bytes.restype = c_size_t
    lib.dwarf_dsqg_q6_prefill_workspace_bytes.argtypes = [POINTER(Q6PrefillArgs)]
    lib.dwarf_dsqg_q6_prefill_fwd.restype = c_int
    lib.dwarf_dsqg_q6_prefill_fwd.argtypes = [POINTER(Q6PrefillArgs), c_void_p]
    lib.dwarf_dsqg_q6_decode.restype = c_int
    lib.dwarf_dsqg_q6_decode.argtypes = [POINTER(Q6DecodeArgs), c_void_p]
    lib.dwarf_dsqg_q6_decode_noalloc.restype = c_int
    lib.dwarf_dsqg_q6_decode_noalloc.argtypes = [POINTER(Q6DecodeArgs), c_void_p]
    lib.dwarf_phase_probe_fwd.restype = c_int
    lib.dwarf_phase_probe_fwd.argtypes = [POINTER(PhaseProbeFwdArgs), c_void_p]
    lib.dwarf_phase_probe_bwd_workspace_bytes.restype = c_size_t
    lib.dwarf_phase_probe_bwd_workspace_bytes.argtypes = [POINTER(PhaseProbeBwdArgs)]
    lib.dwarf_phase_probe_bwd.restype = c_int
    lib.dwarf_phase_probe_bwd.argtypes = [POINTER(PhaseProbeBwdArgs), c_void_p]
    lib.dwarf_npci_fwd.restype = c_int
    lib.dwarf_npci_fwd.argtypes = [POINTER(NpciFwdArgs), c_void_p]
    lib.dwarf_npci_bwd_workspace_bytes.restype = c_size_t
    lib.dwarf_npci_bwd_workspace_bytes.argtypes = [POINTER(NpciBwdArgs)]
    lib.dwarf_npci_bwd.restype = c_int
    lib.dwarf_npci_bwd.argtypes = [POINTER(NpciBwdArgs), c_void_p]
    for name in ("dwarf_packet_pool_state_bytes", "dwarf_packet_pool_fwd_workspace_bytes"):
        getattr(lib, name).restype = c_size_t
        getattr(lib, name).argtypes = [POINTER(PacketPoolFwdArgs)]
    lib.dwarf_dsqg_q6_decode_workspace_bytes.restype = c_size_t
    lib.dwarf_dsqg_q6_decode_workspace_bytes.argtypes = [POINTER(Q6DecodeArgs)]
    lib.dwarf_packet_pool_fwd.restype = c_int
    lib.dwarf_packet_pool_fwd.argtypes = [POINTER(PacketPoolFwdArgs), c_void_p]
    lib.dwarf_packet_pool_bwd_workspace_bytes.restype = c_size_t
    lib.dwarf_packet_pool_bwd_workspace_bytes.argtypes = [POINTER(PacketPoolBwdArgs)]
    lib.dwarf_packet_pool_bwd.restype = c_int
    lib.dwarf_packet_pool_bwd.argtypes = [POINTER(PacketPoolBwdArgs), c_void_p]
    lib.dwarf_packet_fwd.restype = c_int
    lib.dwarf_packet_fwd.argtypes = [POINTER(PacketFwdArgs), c_void_p]
    lib.dwarf_packet_bwd_workspace_bytes.restype = c_size_t
    lib.dwarf_packet_bwd_workspace_bytes.argtypes = [POINTER(PacketBwdArgs)]
    lib.dwarf_packet_bwd.restype = c_int
    lib.dwarf_packet_bwd.argtypes = [POINTER(PacketBwdArgs), c_void_p]
    version = lib.dwarf_abi_version()
    if version != ABI_VERSION:
        raise NativeLibraryError(f"{LIB_NAME} ABI {version} does not match the binding's ABI {ABI_VERSION}")
    _LIB = lib
    return lib


def check(status: int, what: str) -> None:
    """Map a dwarf_status to the exception type the reference raises."""
    if status == DWARF_OK:
        return
    message = (load().dwarf_last_error() or b"").decode(errors="replace")
    text = f"{what}: {message}"
    if status == DWARF_ERR_INVALID_ARGUMENT:
        raise ValueError(text)
    raise NativeLibraryError(text)


def i64_array(values):
    values = [int(v) for v in values]
    return (c_int64 * len(values))(*values)
