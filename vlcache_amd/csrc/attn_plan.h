// Constants shared by the attention planner (host) and the attention kernels.
#pragma once

#include <stdint.h>

namespace vlc {
namespace attn {

constexpr int kHeadDim = 128;   // head row length of q, k, v and out (elements)
// The other head_dim the kernel computes: 80 active dims in 128-element head rows
// (the vision tower's heads, zero-padded), contiguous K/V only.
constexpr int kHeadDimNarrow = 80;
constexpr int kTileK = 64;      // keys per LDS tile; split boundaries are multiples of it
constexpr int kCols = 128;      // (query position, q head) columns per workgroup
constexpr int kBlocksPerCU = 2; // attention workgroups resident per CU
constexpr int kItemInts = 16;   // int32 per work item / combine item (64 bytes, one scalar load)
constexpr int kHeaderInts = 16; // int32 plan header
constexpr int32_t kPlanMagic = 0x564c4331;  // "VLC1"
constexpr int kMinChunkTiles = 4;           // smallest split: 4 key tiles = 256 keys
constexpr int kMaxSplits = 256;
constexpr int kMaxItemTiles = 1024;        // key tiles per work item (the kernel's page-id table)

// Plan header fields (int32 offsets).
enum PlanField {
  kPMagic = 0,
  kPNumItems = 1,
  kPNumCombine = 2,
  kPNumSlots = 3,
  kPCols = 4,
  kPPositionsPerTile = 5,
  kPGroup = 6,
  kPNumSeqs = 7,
  kPNumHeadsKv = 8,
  kPCausal = 9,
  kPHeadDim = 10,
  kPPrio = 11,     // wave issue priority: kPrioEqual, kPrioAlternate or kPrioRemaining
};

// Issue-priority policies of the attention steps (plan field kPPrio).  Two workgroups
// share each CU; with equal priorities the older one's waves win the issue arbitration.
enum PrioMode {
  kPrioEqual = 0,      // equal priorities
  kPrioAlternate = 1,  // 0 and 2 on the two steps of each pair (their steps are not in phase)
  kPrioRemaining = 2,  // by the item's remaining key tiles: a workgroup that falls behind catches up
};

// Work item (int32 x 16): one workgroup.
//   [0] seq  [1] kv_head  [2] q_start  [3] q_count  [4] k_begin  [5] k_end
//   [6] partial slot (-1 = write the normalised output)
//   [7] q0 = cu_seqlens_q[seq]  [8] sq  [9] k0 = cu_seqlens_k[seq]  [10] sk  [11..15] unused
// Combine item (int32 x 16): merges the partial slots of one query tile.
//   [0] seq  [1] kv_head  [2] q_start  [3] q_count  [4] first slot  [5] num splits
//   [7] q0  [8] sq  [9] k0  [10] sk  [6, 11..15] unused
// Carrying the sequence bounds in the item saves the kernels a dependent load.

// Bytes of workspace per partial slot: bf16 O/l [kCols][kHeadDim] + fp32 (m, l) [kCols].
constexpr int64_t kSlotBytes = (int64_t)kCols * kHeadDim * 2 + (int64_t)kCols * 2 * 4;

}  // namespace attn
}  // namespace vlc
