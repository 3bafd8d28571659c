// Host-side work planner for the varlen attention kernel.
//
// flash-attn decides its grid from max_seqlen inside the library that the
// reference calls (layers/attention.py:67-70); here the host, which already
// knows every sequence length when it prepares the step
// (engine/model_runner.py:194-320), builds an explicit work list once per step
// and every layer reuses it:
//   * one item per (sequence, kv head, tile of query positions); a tile holds
//     kCols / group positions so that the group's q heads fill the MFMA columns
//     and share every K/V tile that is staged in LDS;
//   * the key range of an item stops at the causal limit of its last row
//     (bottom-right alignment), so masked tiles are never visited;
//   * items whose key range is much longer than the average are split into
//     chunks of whole 64-key tiles (split-KV); their partial (O, m, l) go to a
//     workspace slot and a combine pass merges them with a log-sum-exp rule;
//   * items are ordered longest first so the dispatcher hands the long ones out
//     before the short ones (longest-processing-time order).
#include <algorithm>
#include <cstring>
#include <vector>

#include "attn_plan.h"
#include "common_host.h"

namespace {

using namespace vlc::attn;

struct Item {
  int32_t v[kItemInts];
  int64_t cost;
};

// The dispatcher places the first num_cus workgroups of a launch one per CU and
// workgroup num_cus + i next to workgroup i (measured on MI355X for a grid of two
// resident workgroups per CU).  When every item fits in one such wave, pair them
// so that CU loads even out: the largest items run alone, the rest pair a large
// item with a small one.  `items` is sorted longest first; multi-wave plans keep
// that order (each freed slot takes the next longest item).
void pair_for_cus(std::vector<Item>& items, int num_cus) {
  const int64_t n = (int64_t)items.size(), c = num_cus;
  if (n <= c || n > 2 * c) return;
  const int64_t m = n - c;  // items in second slots
  std::vector<Item> out(items.size());
  // first slots: [0, m) the paired ones (the smallest m of the c largest, largest
  // first), [m, c) the c - m largest, alone on their CU
  for (int64_t k = 0; k < m; ++k) out[k] = items[c - m + k];
  for (int64_t j = 0; j < c - m; ++j) out[m + j] = items[j];
  // second slot of first slot k: the k-th smallest of the remaining items
  for (int64_t k = 0; k < m; ++k) out[c + k] = items[n - 1 - k];
  items.swap(out);
}

}  // namespace

VLC_HOST_API int vlc_attn_plan(const int32_t* cu_q, const int32_t* cu_k, int num_seqs,
                               int num_heads_q, int num_heads_kv, int head_dim, int causal,
                               int num_cus, int32_t* plan, int64_t plan_capacity,
                               int64_t* plan_len, int64_t* workspace_bytes) {
  if (!cu_q || !cu_k || !plan_len || !workspace_bytes || num_seqs < 0) return VLC_ERR_INVALID;
  if (num_heads_q <= 0 || num_heads_kv <= 0 || num_heads_q % num_heads_kv != 0) return VLC_ERR_INVALID;
  if (head_dim != kHeadDim && head_dim != kHeadDimNarrow) return VLC_ERR_UNSUPPORTED;
  const int group = num_heads_q / num_heads_kv;
  if (group > kCols) return VLC_ERR_UNSUPPORTED;
  const int ppt = kCols / group;
  const bool allow_split = num_cus >= 0;  // num_cus < 0: one item per query tile, no split-KV
  if (num_cus <= 0) num_cus = 256;

  struct Tile {
    int b, g, qs, qc, kmax, nkt;
  };
  auto bounds = [&](int32_t* v, int b) {
    v[7] = cu_q[b];
    v[8] = cu_q[b + 1] - cu_q[b];
    v[9] = cu_k[b];
    v[10] = cu_k[b + 1] - cu_k[b];
  };
  std::vector<Tile> tiles;
  int64_t total = 0;
  bool reused_context = false;
  for (int b = 0; b < num_seqs; ++b) {
    const int64_t sq = (int64_t)cu_q[b + 1] - cu_q[b];
    const int64_t sk = (int64_t)cu_k[b + 1] - cu_k[b];
    if (sq < 0 || sk < 0 || cu_q[b] < 0 || cu_k[b] < 0) return VLC_ERR_INVALID;
    reused_context = reused_context || sk > sq;
    for (int64_t qs = 0; qs < sq; qs += ppt) {
      const int qc = (int)std::min<int64_t>(ppt, sq - qs);
      int64_t kmax = sk;
      if (causal) kmax = std::max<int64_t>(0, std::min<int64_t>(sk, qs + qc + sk - sq));
      const int nkt = (int)((kmax + kTileK - 1) / kTileK);
      for (int g = 0; g < num_heads_kv; ++g) {
        tiles.push_back({b, g, (int)qs, qc, (int)kmax, nkt});
        total += std::max(nkt, 1);
      }
    }
  }

  // Split long key ranges so that every resident workgroup slot has work.
  const int64_t target_blocks = (int64_t)kBlocksPerCU * num_cus;
  int64_t chunk = (total + target_blocks - 1) / std::max<int64_t>(1, target_blocks);
  chunk = std::max<int64_t>(chunk, kMinChunkTiles);

  std::vector<Item> items;
  std::vector<Item> combines;
  int32_t next_slot = 0;
  items.reserve(tiles.size());
  for (const Tile& t : tiles) {
    // Round to the nearest number of chunks: a range up to 1.5 chunks stays whole.
    int nsplit = (int)std::min<int64_t>(kMaxSplits, std::max<int64_t>(1, (2 * t.nkt + chunk) / (2 * chunk)));
    if (!allow_split) nsplit = 1;
    // No item longer than kMaxItemTiles key tiles.
    nsplit = std::max(nsplit, (t.nkt + kMaxItemTiles - 1) / kMaxItemTiles);
    if (nsplit > kMaxSplits) return VLC_ERR_UNSUPPORTED;
    if (nsplit <= 1) {
      Item it{};
      it.v[0] = t.b; it.v[1] = t.g; it.v[2] = t.qs; it.v[3] = t.qc;
      it.v[4] = 0; it.v[5] = t.kmax; it.v[6] = -1;
      bounds(it.v, t.b);
      it.cost = std::max(t.nkt, 1);
      items.push_back(it);
      continue;
    }
    const int per = (t.nkt + nsplit - 1) / nsplit;  // key tiles per split
    nsplit = (t.nkt + per - 1) / per;
    Item c{};
    c.v[0] = t.b; c.v[1] = t.g; c.v[2] = t.qs; c.v[3] = t.qc; c.v[4] = next_slot; c.v[5] = nsplit;
    bounds(c.v, t.b);
    c.cost = nsplit;
    combines.push_back(c);
    for (int s = 0; s < nsplit; ++s) {
      Item it{};
      const int kb = s * per * kTileK;
      const int ke = std::min(t.kmax, (s + 1) * per * kTileK);
      it.v[0] = t.b; it.v[1] = t.g; it.v[2] = t.qs; it.v[3] = t.qc;
      it.v[4] = kb; it.v[5] = ke; it.v[6] = next_slot + s;
      bounds(it.v, t.b);
      it.cost = (ke - kb + kTileK - 1) / kTileK;
      items.push_back(it);
    }
    next_slot += nsplit;
  }
  std::stable_sort(items.begin(), items.end(),
                   [](const Item& a, const Item& b) { return a.cost > b.cost; });
  pair_for_cus(items, num_cus);

  const int64_t need = kHeaderInts + (int64_t)(items.size() + combines.size()) * kItemInts;
  *plan_len = need;
  *workspace_bytes = (int64_t)next_slot * kSlotBytes;
  if (!plan || plan_capacity < need) return VLC_ERR_CAPACITY;
  std::memset(plan, 0, sizeof(int32_t) * kHeaderInts);
  plan[kPMagic] = kPlanMagic;
  plan[kPNumItems] = (int32_t)items.size();
  plan[kPNumCombine] = (int32_t)combines.size();
  plan[kPNumSlots] = next_slot;
  plan[kPCols] = kCols;
  plan[kPPositionsPerTile] = ppt;
  plan[kPGroup] = group;
  plan[kPNumSeqs] = num_seqs;
  plan[kPNumHeadsKv] = num_heads_kv;
  plan[kPCausal] = causal ? 1 : 0;
  plan[kPHeadDim] = head_dim;
  // One wave of workgroups (each CU runs its two items to the end together): priority by
  // remaining tiles, which evens out the two workgroups of a CU (warm 4K request 28.6
  // against 29.3 us with alternating priorities, its 64 x 10741 suffix alone 23.8
  // against 24.3).  Several waves over reused context: alternating priorities (8 requests
  // sharing an image 170.8 against 177.7 us with the remaining-tile rule).  Square causal
  // calls of several waves: equal priorities (dense 4096^2 83.8 against 84.8 us).
  const bool one_wave = (int64_t)items.size() <= (int64_t)kBlocksPerCU * num_cus;
  plan[kPPrio] = one_wave ? kPrioRemaining : reused_context ? kPrioAlternate : kPrioEqual;
  int32_t* w = plan + kHeaderInts;
  for (const Item& it : items) { std::memcpy(w, it.v, sizeof(it.v)); w += kItemInts; }
  for (const Item& c : combines) { std::memcpy(w, c.v, sizeof(c.v)); w += kItemInts; }
  return VLC_OK;
}
