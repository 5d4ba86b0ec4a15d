// Internal launch interface between the C-ABI layer (capi.hip) and the
// kernel translation units.  Nothing here is exported.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "dwarf_dsqg.h"

namespace dwarf {

constexpr int kHeadDim = 64;
constexpr int kBlock = 256;  // threads per workgroup for the DSQG kernels

// Workgroup index -> work item, so that consecutive work items (the query
// tiles of one (b, h), which share K/V rows) land on the same XCD and share
// its L2.  Workgroups are dealt round-robin over the 8 XCDs of an MI355X.
constexpr int kXcds = 8;   // XCDs of an MI355X; workgroups are dealt round-robin over them

__device__ __forceinline__ int xcd_remap(int block_linear, int total) {
  constexpr int kXcd = kXcds;
  const int per = total / kXcd, rem = total % kXcd;
  const int xcd = block_linear % kXcd, idx = block_linear / kXcd;
  return xcd * per + (xcd < rem ? xcd : rem) + idx;
}

// Geometry shared by the DSQG kernels.
struct DsqgGeom {
  int queries_per_block;
  int tiles;   // query tiles per (b, h)
  int blocks;  // tiles * B * H
};

hipError_t launch_dsqg_fwd(const dwarf_dsqg_fwd_args& a, hipStream_t stream);

// Backward workspace layout (bytes, 256-byte aligned sections).  The dq
// launch writes one partial slot per workgroup (slot = (h*B + b)*n_tg + tg);
// the reduce launch sums them in a fixed order.
struct BwdWorkspace {
  size_t delta_off, delta_bytes;        // bf16: [B,H,N] (delta, log2 lse) fp32 pairs; fp32: [B,H,N] delta
  size_t part_se_off, part_se_bytes;    // [W][J][64] fp32
  size_t part_pb_off, part_pb_bytes;    // [H][pb_rows][J] fp32
  size_t part_ph_off, part_ph_bytes;    // [H][ph_rows][J_L][8] fp32
  size_t ds_off, ds_bytes;              // bf16 launch: dS [B*H][J][N] fp32
  size_t red_off, red_bytes;            // stage-1 sums of the reduction
  size_t kv_part_off, kv_part_bytes;    // bf16, kv_split > 1: [kv_split][split units x 64 keys] partial dK and
                                        // dV (64 fp32 each), then dZ (4 fp32), of each subset of the query heads
  size_t total;
  int dq_tiles;   // query tiles per (b, h)
  int dq_tpw;     // tiles per workgroup (fp32 launch)
  int dq_ntg;     // workgroups per (b, h) (fp32 launch)
  int dq_wgs;     // W: workgroups of the dq launch = dSE partial slots (bf16: of the dSE launch)
  int dq_gather_wgs;   // bf16: persistent workgroups of the dQ gather launch
  int pb_rows, ph_rows;   // dPB / dPhase partial rows per head
  int red_groups_se, red_groups_pb, red_groups_ph;  // stage-1 row groups per segment
  int kv_split;   // bf16: workgroups sharing one split (key tile, KV head), each over a subset of its query heads
  int kv_whole;   // bf16: (key tile, KV head) units taken whole, before the split ones
};
BwdWorkspace bwd_workspace_layout(const dwarf_dsqg_bwd_args& a);
struct KvSplit {
  int whole;    // (key tile, KV head) units a workgroup takes with the whole query-head group
  int nsplit;   // subsets of the query heads for each of the other units (1: none)
};
// do_dq: delta + dQ/dY + the parameter-gradient inputs in the workspace (bf16:
// the dS matrix and dPhase partials; fp32: all partials); do_params: the
// parameter gradients from those (bf16: the dSE/dPB launch, then the fixed-
// order reduction); do_dkdv: dK/dV/dZ (reads the delta of the dq stage).
hipError_t launch_dsqg_bwd(const dwarf_dsqg_bwd_args& a, const BwdWorkspace& ws, hipStream_t stream, bool do_dq,
                           bool do_params, bool do_dkdv);
hipError_t launch_dsqg_bwd_dq(const dwarf_dsqg_bwd_args& a, const BwdWorkspace& ws, hipStream_t stream);
hipError_t launch_dsqg_bwd_delta(const dwarf_dsqg_bwd_args& a, const BwdWorkspace& ws, hipStream_t stream);
hipError_t launch_dsqg_bwd_dse(const dwarf_dsqg_bwd_args& a, const BwdWorkspace& ws, hipStream_t stream);
size_t dq_lds_bytes(int J, int J_large, int dtype);
size_t dkdv_lds_bytes(int J, int J_large, int group);   // bf16 dK/dV launch, per workgroup
constexpr size_t kMaxLdsBytes = 160 * 1024;             // LDS per workgroup on gfx950
int dq_tile_queries(int dtype);   // queries per tile of the dQ launch
int dq_gather_wgs_per_cu();       // resident workgroups per CU of the bf16 dQ gather launch
int dq_dse_wgs_per_cu(int J);     // resident workgroups per CU of the bf16 dSE launch

}  // namespace dwarf
