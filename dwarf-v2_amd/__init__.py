"""dwarf-v2_amd: MI355X (gfx950) kernels for DWARF-v2's DSQG offset-gather path.

The directory name is not a Python identifier; import it with
``importlib.import_module("dwarf-v2_amd")``.

Public surface (reference names, Lanerra/dwarf-v2):
  dsqg_attention_v18_grouped, _DSQGV18GroupedFn      kernels/dsqg_attention_v22.py
  dsqg_attention_with_probes, _DSQGProbedFn,
  dsqg_block_forward (block module)                  the op and DSQGAttentionV19.forward with the
                                                     block's y/z features inside the kernels
  ALL_OFFSETS, R_PLANES and the lattice helpers      kernels/dsqg_attention_v22.py
  causal_ema_scan, bounded_ema_factor,
  inverse_bounded_ema_factor                         kernels/causal_ema_scan.py
  phase_probe_features, _PhaseProbeFn                kernels/dsqg_attention_v22.py
  npci_rotate                                        kernels/dsqg_attention_v22.py
  _plan_sparse_groups, _verify_sparse_plan,
  _normalize_grouping_args (planner module)          kernels/dsqg_attention_v22.py
  interference_pool, interference_packet,
  interference_packet_forward                        train/train_dwarf.py (InterferencePacket)
  q6: pack_kv, unpack_kv, q6_prefill, q6_decode      (no reference counterpart)
"""

from . import _lib, block, lattice, npci, ops, packet, planner, probe, q6
from .block import dsqg_block_forward
from .dsqg import (_DSQGProbedFn, _DSQGV18GroupedFn, dsqg_attention_v18_grouped, dsqg_attention_with_probes,
                   dsqg_backward, dsqg_forward)
from .ema import bounded_ema_factor, causal_ema_scan, inverse_bounded_ema_factor
from .npci import npci_rotate
from .packet import _InterferencePacketFn, _InterferencePoolFn, interference_packet, interference_packet_forward, interference_pool
from .planner import _normalize_grouping_args, _plan_sparse_groups, _verify_sparse_plan
from .probe import _PhaseProbeFn, phase_probe_features
from .lattice import (
    ALL_OFFSETS,
    GROUPED_MODE_IDS,
    R_PLANES,
    _canonicalize_offsets,
    _normalize_plane_shift,
    _orthogonal_phase_probes,
    _phase_plane_channels,
    build_offset_groups,
)

__all__ = [
    "ALL_OFFSETS",
    "GROUPED_MODE_IDS",
    "R_PLANES",
    "_DSQGProbedFn",
    "_DSQGV18GroupedFn",
    "_InterferencePacketFn",
    "_InterferencePoolFn",
    "_PhaseProbeFn",
    "_canonicalize_offsets",
    "_normalize_grouping_args",
    "_normalize_plane_shift",
    "_orthogonal_phase_probes",
    "_phase_plane_channels",
    "_plan_sparse_groups",
    "_verify_sparse_plan",
    "bounded_ema_factor",
    "build_offset_groups",
    "causal_ema_scan",
    "dsqg_attention_v18_grouped",
    "dsqg_attention_with_probes",
    "dsqg_block_forward",
    "dsqg_backward",
    "dsqg_forward",
    "interference_packet",
    "interference_packet_forward",
    "interference_pool",
    "inverse_bounded_ema_factor",
    "npci_rotate",
    "phase_probe_features",
    "q6",
]


def native_library_path() -> str:
    """Path of the HIP library every op in this package calls."""
    return _lib.library_path()
