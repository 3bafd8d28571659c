// Constants shared by the attention planner (host) and the attention kernels.
#pragma once

#include <stdint.h>

namespace vlc {
namespace attn {

constexpr int kHeadDim = 128;   // only head_dim supported by the MFMA kernel
constexpr int kTileK = 64;      // keys per LDS tile; split boundaries are multiples of it
constexpr int kCols = 128;      // (query position, q head) columns per workgroup
constexpr int kItemInts = 8;    // int32 per work item / combine item
constexpr int kHeaderInts = 16; // int32 plan header
constexpr int32_t kPlanMagic = 0x564c4331;  // "VLC1"
constexpr int kMinChunkTiles = 4;           // smallest split: 4 key tiles = 256 keys
constexpr int kMaxSplits = 256;

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
};

// Work item (int32 x 8): one workgroup.
//   [0] seq  [1] kv_head  [2] q_start  [3] q_count  [4] k_begin  [5] k_end
//   [6] partial slot (-1 = write the normalised output)  [7] unused
// Combine item (int32 x 8): merges the partial slots of one query tile.
//   [0] seq  [1] kv_head  [2] q_start  [3] q_count  [4] first slot  [5] num splits
//   [6..7] unused

// Bytes of workspace per partial slot: fp32 O [kCols][kHeadDim] + fp32 (m, l) [kCols].
constexpr int64_t kSlotBytes = (int64_t)kCols * kHeadDim * 4 + (int64_t)kCols * 2 * 4;

}  // namespace attn
}  // namespace vlc
