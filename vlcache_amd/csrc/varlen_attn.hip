// Varlen paged GQA attention (prefill) for gfx950: the replacement of
// flash_attn_varlen_func(q, k, v, ..., causal=True, block_table) as called at
// layers/attention.py:67-70.
//
// Work decomposition (built on the host by vlc_attn_plan): a workgroup of four
// wave64s owns one work item = (sequence, kv head, tile of query positions,
// key range); two workgroups share a CU.  Its 128 "columns" are (query
// position, q head) pairs: the `group` q heads that share the kv head are
// packed side by side, so one K/V tile staged in LDS feeds every head of the
// group.
//
// Per 64-key tile each wave computes S^T = K * Q^T (keys x its 32 columns) with
// v_mfma_f32_32x32x16_bf16.  In that orientation a lane owns ONE column and 16
// keys of each 32-key block, so the softmax row reductions are lane-local plus
// a single exchange between the two half-waves.  The probabilities P^T are
// already in the B-operand layout of the second product O^T += V^T P^T, so they
// never leave registers; V stays row-major in LDS and is read transposed
// (ds_read_b64_tr_b16).
//
// The tile loop is software-pipelined inside each wave: step t issues the PV
// product of tile t-1 and the QK product of tile t+1 on the matrix pipe while
// the VALU runs the softmax of tile t, with the instruction order fixed by hand.
// K/V tiles go global -> LDS by DMA (global_load_lds_dwordx4), two tiles ahead.
//
// Online softmax in fp32 with exp2 (the softmax scale and log2(e) are folded
// into one multiply-add) and a lazy running max, P rounded to bf16 for the PV
// product, O accumulated in fp32 and normalised once at the end.  Items whose
// key range was split write their normalised O (bf16) with (m, l) to a
// workspace slot; attn_combine merges the slots of a query tile.
#include <type_traits>
#include <utility>

#include "attn_plan.h"
#include "common.h"

namespace vlc {
namespace attn {
namespace {

constexpr int kThreads = 256;  // four wave64s, one per SIMD

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));

struct Params {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const int32_t* block_table;
  const int32_t* cu_q;
  const int32_t* cu_k;
  const int32_t* items;
  const int32_t* combine;
  uint16_t* out;
  uint16_t* part_o;  // [slots][kCols][kHeadDim] bf16: the split's own normalised output O_s / l_s
  float* part_ml;    // [slots][kCols][2] fp32: (m_s in scaled log2 units, l_s)
  int64_t q_row_stride;
  int64_t k_row_stride;
  int64_t v_row_stride;
  int64_t bt_row_stride;
  int64_t out_row_stride;
  int64_t num_blocks;
  int page_size;
  int group;
  int causal;
  int prio_mode;  // the plan's kPPrio
  float scale_log2;
};

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }


typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Round two fp32 to bf16 (nearest even) with the hardware pack conversion.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2 v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// How keys map to rows of k/v.
enum KvMode {
  kContiguous = 0,  // key j of sequence b is row cu_k[b] + j
  kPagedTiles = 1,  // paged, page_size % 64 == 0: a 64-key tile lies inside one page
  kPagedRows = 2,   // paged, page_size % 16 == 0: the 16 rows a wave loads lie inside one page
};

// Online-softmax threshold (log2 units): the running max only moves when a tile's
// max exceeds it by more than this, so P stays <= 2^8 and O is rarely rescaled.
constexpr float kRescaleThreshold = 8.0f;

// XOR swizzle of the 16-byte chunks of a 256-byte LDS row: chunk c of row r lives in
// slot c ^ swz(r).  swz is a bijection on r mod 16 (so the 16 rows of a b128 operand
// read hit 16 distinct slots) whose high two bits follow r mod 4 (so the 4 rows x 4
// chunks of a half-wave's transpose reads also hit 16 distinct slots).
__device__ __forceinline__ int swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

// All-zero rows: the source of keys past the end of a sequence and of pages whose
// block id is outside the cache (they read as zeros).
__device__ __attribute__((aligned(256))) const uint32_t kZeroRow[64] = {};

typedef __attribute__((address_space(3))) void lds_void;

// ---- LDS-DMA and barriers ----------------------------------------------------
// Tile loads go global -> LDS with global_load_lds_dwordx4 (lane i's 16 bytes land
// at M0 + 16 i).  They are issued through inline assembly: the compiler's model
// of an LDS DMA in flight is a flat access of unknown order, which would force
// every later LDS read wait to drain the whole queue (lgkmcnt(0)) and break the
// operand pipeline of the products.  The hardware counts these loads in vmcnt
// only, and every read of a loaded buffer is preceded by sync_tiles(), which waits
// for vmcnt(0) and is a compiler memory barrier, so no LDS value is cached across
// it.
__device__ __forceinline__ uint32_t lds_u32(const void* ptr) {
  return (uint32_t)(uintptr_t)(const lds_void*)ptr;
}
// Uniform base + per-lane 32-bit offset.
__device__ __forceinline__ void dma16(const void* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :
               : "s"(lds), "v"(voff), "s"(base)
               : "m0");
}
// Per-lane 64-bit address.
__device__ __forceinline__ void dma16_addr(const void* addr, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(lds), "v"(addr)
               : "m0");
}
// Every tile load of this wave has landed, every LDS access of this wave is done,
// then the workgroup barrier.
__device__ __forceinline__ void sync_tiles() {
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// One work item = (sequence, kv head, kCols = 128 columns, key range): four waves,
// one per SIMD, each owning 32 columns; two workgroups share a CU.
//
// Software pipeline over key tiles: step t runs, in one instruction stream,
//   O^T += V^T P^T of tile t-1   (16 MFMAs, V tile t-1 from LDS)
//   S^T  = K Q^T  of tile t+1    (16 MFMAs, K tile t+1 from LDS)
//   softmax of tile t            (VALU: max, exp2, sum, bf16 pack)
// which are independent, so the VALU work issues while the matrix pipe is busy.
// The rescale of O by the softmax of tile t waits until the products of tile
// t-1 are in.  During step t the loads of K tile t+2 and V tile t fill the
// buffers that step t-1 read.
// max(x) over lanes l and l ^ 32.  v_permlane32_swap exchanges the upper half of
// its first operand with the lower half of its second; with both operands x the
// two results hold, in every lane, the lane's own x and its partner's.  A VALU
// operation, so the softmax that depends on it does not wait behind the LDS reads
// of the products (as ds_bpermute would).  Issued through inline assembly with
// both registers as in/out operands: the compiler (ROCm 7.2) folds the two results
// of the swap builtin into one, which drops the partner's value.  The s_nop covers
// the VALU-write -> permlane-read hazard, which it does not track through inline
// assembly.
__device__ __forceinline__ float half_wave_max(float x) {
  float a = x, b = x;
  asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return fmaxf(a, b);
}

// KS: 16-dim steps of q.k (head_dim / 16); MB: 32-dim blocks of the output (head_dim / 32,
// rounded up).  Heads are 128-element rows either way; with head_dim 80 (KS 5, MB 3) the
// products skip dims 80..127 of q and k and 96..127 of v (output dims 96..127 are zero,
// 80..95 take v's values there).
// AHEAD (kPagedTiles only): read the block ids of a step's tiles one step early; see
// the launch for where it is used.
template <int MODE, int KS = 8, int MB = 4, bool AHEAD = false>
__global__ __launch_bounds__(kThreads, kBlocksPerCU) void attn_fwd_kernel(const Params p) {
  constexpr bool kAheadSrc = MODE == kPagedTiles && AHEAD;
  static_assert(KS >= 1 && KS <= 8 && MB >= 1 && MB <= 4 && 2 * MB >= KS, "head_dim <= 128");
  constexpr int NPV = 4 * MB;       // O^T += V^T P^T MFMAs per tile
  constexpr int NQK = 2 * KS;       // S^T = K Q^T MFMAs per tile
  constexpr int NU = NPV + NQK;     // units of a pipelined step
  __shared__ __attribute__((aligned(1024))) uint8_t k_buf0[kTileK * 256];
  __shared__ __attribute__((aligned(1024))) uint8_t k_buf1[kTileK * 256];
  __shared__ __attribute__((aligned(1024))) uint8_t v_buf0[kTileK * 256];
  __shared__ __attribute__((aligned(1024))) uint8_t v_buf1[kTileK * 256];
  __shared__ int32_t tile_blk[kMaxItemTiles];  // kPagedTiles: block id of each key tile

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int lc = lane & 31;
  const int hf = lane >> 5;

  const int32_t* it = p.items + (int64_t)blockIdx.x * kItemInts;
  const int b = it[0], g = it[1], q_start = it[2], q_count = it[3];
  const int k_begin = it[4], k_end = it[5], slot = it[6];
  const int q0 = it[7], sq = it[8], k0 = it[9], sk = it[10];
  const int n_tiles = (k_end - k_begin + kTileK - 1) / kTileK;

  // ---- the lane's column: wave*32 + lc ----------------------------------------------
  const int col = wave * 32 + lc;
  const int pos = col / p.group;
  const int hh = col - pos * p.group;
  const bool valid = pos < q_count;
  const int qpos = q_start + pos;
  const int head = g * p.group + hh;
  const int limit = p.causal ? qpos + sk - sq : sk - 1;             // last visible key
  const int blk_min_limit = p.causal ? q_start + sk - sq : sk - 1;  // smallest limit in the item
  const int last_key = min(blk_min_limit, k_end - 1);              // keys <= last_key need no mask
  // Leading tiles that need no mask.
  const int n_plain = max(0, min(n_tiles, (last_key - k_begin + 1) / kTileK));

  // Q^T fragment (B operand of S^T = K Q^T): lane holds Q[col][16*kk + 8*hf .. +8].
  // Invalid columns load row 0 (always readable) and are zeroed.
  bf16x8 qf[KS];
  {
    const uint16_t* qrow = p.q + (valid ? (int64_t)(q0 + qpos) * p.q_row_stride + (int64_t)head * kHeadDim : 0) +
                           8 * hf;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      u32x4v w = *reinterpret_cast<const u32x4v*>(qrow + 16 * kk);
      if (!valid) w = u32x4v{0u, 0u, 0u, 0u};
      qf[kk] = __builtin_bit_cast(bf16x8, w);
    }
  }

  // ---- LDS read offsets (bytes, within a tile buffer) ---------------------------
  // K operand of S^T: row kb*32 + lc, chunk 2kk + hf, i.e. byte offset
  // koff0 ^ (kk << 5) (the chunk field is bits 4..7 and 2kk, hf are disjoint bits).
  const uint32_t koff0 = lc * 256 + ((hf ^ swz(lc)) << 4);
  // Lane offsets are recomputed from an opaque copy of their base where they are
  // used (an XOR or a multiply-add each) rather than hoisted out of the tile loop
  // as live registers: registers are the limit of this kernel.
  auto opaque = [](uint32_t x) __attribute__((always_inline)) {
    asm volatile("" : "+v"(x));
    return x;
  };
  // V^T operand through ds_read_b64_tr_b16: in each 16-lane group, lane 4f + r reads
  // dims 4r..4r+3 (of the group's 16-dim half) of key row f, and the transpose
  // hands lane j the 4 keys of dim j.  Group bit 0 = dim half, bit 1 = key half
  // (+4 keys); the second read of an operand is 8 keys further.  Dim block mb
  // XORs chunk bits (mb << 2) and +8 keys XORs row bit 3 and chunk bit 1 (swz of
  // row + 8 is swz(row) ^ 2), so every offset is voff0 ^ a constant.
  uint32_t voff0;
  {
    const int s = lane & 15, lg = lane >> 4;
    const int y = 2 * (lg & 1) + ((s & 3) >> 1);
    const int row = 4 * (lg >> 1) + (s >> 2);  // + 8rd + kb*32 + 16c
    voff0 = row * 256 + ((y ^ swz(row)) << 4) + ((s & 1) << 3);
  }


  // The eight K and eight V operand offsets of a step, kept in registers across
  // the tile loop (each is the lane's base offset XOR a constant).
  uint32_t kofs[KS], vofs[2 * MB];
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) kofs[kk] = koff0 ^ (uint32_t)(kk << 5);
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    vofs[2 * mb] = voff0 ^ ((uint32_t)mb << 6);
    vofs[2 * mb + 1] = voff0 ^ (((uint32_t)mb << 6) | 32u | 2048u);
  }

  // ---- tile loads: wave w fills rows 16w .. 16w+15, 4 rows per instruction -----
  // Lane i writes LDS slot i%16 of row 16w + 4j + i/16, so it loads that row's
  // chunk (i%16) ^ swz(row) = (i%16) ^ ((i/16) << 2) ^ j.
  const char* kcol = reinterpret_cast<const char*>(p.k + (int64_t)g * kHeadDim);
  const char* vcol = reinterpret_cast<const char*>(p.v + (int64_t)g * kHeadDim);
  const int64_t kst = p.k_row_stride * 2, vst = p.v_row_stride * 2;  // bytes
  const uint32_t lrow0 = 16 * wave + (lane >> 4);
  const uint32_t lchunk0 = (uint32_t)((lane & 15) ^ ((lane >> 4) << 2));
  const char* zero = reinterpret_cast<const char*>(kZeroRow);

  // ---- state ---------------------------------------------------------------------
  f32x16 o[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[mb][e] = 0.f;
  f32x16 s_even[2], s_odd[2];        // S^T of even / odd tiles: [key block]
  bf16x8 pk[2][2];                   // P^T between its softmax and its product: [key block][chunk]
  float m_run = -INFINITY;           // running max, scaled to log2 units
  float l_run = 0.f;

  // S^T = K Q^T of one tile (K from LDS): NQK operand reads, NQK MFMAs.
  auto qk = [&](const uint8_t* kb_lds, f32x16 (&S)[2]) __attribute__((always_inline)) {
    const uint32_t kof = opaque(koff0);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; ++e) S[kb][e] = 0.f;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(kb_lds + kb * 32 * 256 + (kof ^ (kk << 5)));
        S[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[kk], S[kb], 0, 0, 0);
      }
  };
  // Instruction order hint for the products of the prologue (sched groups: 0x008
  // MFMA, 0x100 LDS read): operand reads run a few MFMAs ahead of their use.
  auto order_qk = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int i = 0; i < NQK - 4; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
  };
  auto rescale = [&](float alpha) __attribute__((always_inline)) {
    if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[mb][e] *= alpha;
    }
  };

  // Source of one tile load: a uniform base and the last row to read.  Lane row r
  // (lrow0 + 4j) reads base + min(r, last) rows: rows past the sequence read its last
  // row (their keys are masked, so the products never use them); tiles past the item
  // and pages outside the cache read the zero row (last = 0).
  struct DmaSrc {
    const char* base;
    uint32_t last;
  };
  // Paged tiles: the tile's block id, from the LDS copy of the item's page table, or
  // with `direct` from the block table (scalar load), for the prologue, which does not
  // wait for that copy.  Paged rows: the block id of the wave's 16 rows (one page,
  // page_size % 16 == 0), a scalar load of the block table; base is then that page
  // row minus the wave's first tile row, so lane row r still reads base + r rows.
  typedef const __attribute__((address_space(4))) int32_t* const_i32p;
  auto dma_src = [&](int u, const char* colbase, int64_t st, bool direct = false) __attribute__((always_inline)) {
    const int kt = k_begin + u * kTileK;
    bool ok = u < n_tiles;
    if (MODE == kContiguous) {
      const int64_t row0 = (int64_t)k0 + kt;
      return DmaSrc{ok ? colbase + row0 * st : zero, ok ? (uint32_t)min(kTileK - 1, sk - 1 - kt) : 0u};
    }
    const const_i32p bt_row = (const_i32p)(uintptr_t)(p.block_table + (int64_t)b * p.bt_row_stride);
    if (MODE == kPagedTiles) {
      const int32_t blk = direct ? (ok ? bt_row[kt / p.page_size] : 0)
                                 : __builtin_amdgcn_readfirstlane(tile_blk[min(u, max(n_tiles - 1, 0))]);
      ok = ok && blk >= 0 && blk < p.num_blocks;
      const int64_t row0 = (int64_t)blk * p.page_size + (kt % p.page_size);
      return DmaSrc{ok ? colbase + row0 * st : zero, ok ? (uint32_t)min(kTileK - 1, sk - 1 - kt) : 0u};
    }
    const int g0 = kt + 16 * wave;  // first key of the wave's rows
    ok = ok && g0 < sk;
    const int pg = g0 / p.page_size;
    const int32_t blk = ok ? bt_row[pg] : 0;
    ok = ok && blk >= 0 && blk < p.num_blocks;
    const int64_t row0 = (int64_t)blk * p.page_size + (g0 - pg * p.page_size) - 16 * wave;
    return DmaSrc{ok ? colbase + row0 * st : zero, ok ? (uint32_t)(16 * wave + min(15, sk - 1 - g0)) : 0u};
  };
  // kAheadSrc: the source of a paged tile load split in two, so that a step can read
  // the block ids of the next step's tiles early and use them a step later: the LDS
  // read of tile u's block id (a VGPR, uniform), then the source from it.
  auto tile_blk_raw = [&](int u) __attribute__((always_inline)) {
    return tile_blk[min(u, max(n_tiles - 1, 0))];
  };
  // Branch-free (the address is formed from a clamped block id and then selected): a
  // branch here would split the step's straight-line code in the middle.  off: the
  // tile's first row within its page (split boundaries and page sizes are multiples of
  // 64 keys, so the next tile's offset is this one's + 64, wrapped at the page size).
  const int64_t kpage = (int64_t)p.page_size * kst, vpage = (int64_t)p.page_size * vst;
  auto paged_src = [&](int u, int32_t raw, const char* colbase, int64_t st, int64_t page_bytes, uint32_t off)
      __attribute__((always_inline)) {
    const int kt = k_begin + u * kTileK;
    const int32_t blk = __builtin_amdgcn_readfirstlane(raw);
    const bool ok = u < n_tiles && blk >= 0 && blk < p.num_blocks;
    const char* base = colbase + (int64_t)(ok ? blk : 0) * page_bytes + (int64_t)off * st;
    asm volatile("" : "+s"(base));
    return DmaSrc{ok ? base : zero, ok ? (uint32_t)min(kTileK - 1, sk - 1 - kt) : 0u};
  };
  auto next_off = [&](uint32_t off) __attribute__((always_inline)) {
    off += kTileK;
    return off >= (uint32_t)p.page_size ? off - (uint32_t)p.page_size : off;
  };
  // kAheadSrc: the sources of the current step's tile loads (K tile t + 2, V tile t),
  // computed during the previous step (the prologue for step 0).
  DmaSrc dk_cur{zero, 0u}, dv_cur{zero, 0u};
  uint32_t koff_nx = 0, voff_nx = 0;  // in-page rows of the next step's K tile t + 3 and V tile t + 1

  // O^T += V^T P^T of the last tile, reads a few MFMAs ahead (sched groups: 0x008
  // MFMA, 0x100 LDS read).  MFMA j: dim block j % MB, 16-key chunk (j / MB) & 1, key
  // block j / (2 MB).
  auto pv_last = [&](const uint8_t* v_rd) __attribute__((always_inline)) {
    const uint32_t vof = opaque(voff0);
#pragma unroll
    for (int j = 0; j < NPV; ++j) {
      const int mbi = j % MB, ch = (j / MB) & 1, kb = j / (2 * MB);
      const uint8_t* vr = v_rd + (kb * 32 + 16 * ch) * 256;
      const uint32_t mb = (uint32_t)mbi << 6;
      const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4*)(vr + (vof ^ mb)));
      const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4*)(vr + (vof ^ (mb | 32u | 2048u))));
      const s16x8 w = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      o[mbi] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, w), pk[kb][ch], o[mbi], 0, 0, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
#pragma unroll
    for (int i = 0; i < NPV - 3; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 3, 0);
  };

  // One step t with explicit buffers and S registers: K tile t+1 and V tile t-1
  // are read from buffer (t+1)&1, K tile t+2 and V tile t are loaded into buffer
  // t&1.  The step is straight-line code: at t = 0 the products read a zeroed V
  // buffer with P = 0, at t = n-1 they compute an S^T that is never used and load
  // zero rows.
  //
  // Its instruction order is fixed by hand, in NU units (32 for 128-dim heads)
  // separated by sched_barrier: unit i issues MFMA i (PV for i < NPV, QK after), the operand
  // read of MFMA i + kAhead, one tile load (units 0..7) and a slice of the
  // softmax of tile t (mask and max in units 0..2, the new running max in unit
  // 3, one or two exp2 per unit after), so the VALU work fills the matrix pipe's
  // shadow.  P^T of tile t-1 is read by the PV MFMAs before the softmax packs the
  // new one after the last unit.
  auto step_body = [&](auto masked, int t, f32x16 (&s_cur)[2], f32x16 (&s_nxt)[2], uint8_t* k_rd, uint8_t* v_rd,
                       uint8_t* k_ld, uint8_t* v_ld) __attribute__((always_inline)) {
    constexpr bool MASKED = decltype(masked)::value;
    constexpr int kAhead = 3;
    const int kt = k_begin + t * kTileK;
    // kAheadSrc: the sources were computed a step ahead (reading the block ids here
    // waits for two LDS round trips before the step's first operand read); the next
    // step's sources are computed in units kRawUnit (block id reads) and kSrcUnit.
    constexpr int kRawUnit = 8, kSrcUnit = 20;
    static_assert(!kAheadSrc || kSrcUnit < NU, "the next step's sources are computed inside the step");
    const DmaSrc dk = kAheadSrc ? dk_cur : dma_src(t + 2, kcol, kst);
    const DmaSrc dv = kAheadSrc ? dv_cur : dma_src(t, vcol, vst);
    int32_t raw_k = 0, raw_v = 0;
    const uint32_t lr = opaque(lrow0), lcn = opaque(lchunk0);
    const int rel = min(limit, k_end - 1) - kt - 4 * hf;  // MASKED: keys past rel are masked

    bf16x8 op[NU];
    auto read_op = [&](int j) __attribute__((always_inline)) {
      if (j < NPV) {  // V^T operand: dim block j % MB, 16-key chunk (j / MB) & 1, key block j / (2 MB)
        const int mbi = j % MB, ch = (j / MB) & 1, kb = j / (2 * MB);
        const uint8_t* vr = v_rd + (kb * 32 + 16 * ch) * 256;
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s16x4*)(vr + vofs[2 * mbi]));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s16x4*)(vr + vofs[2 * mbi + 1]));
        const s16x8 w = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        op[j] = __builtin_bit_cast(bf16x8, w);
      } else {  // K operand: head-dim step (j - NPV) >> 1, key block (j - NPV) & 1
        const int kk = (j - NPV) >> 1, kb = (j - NPV) & 1;
        op[j] = *reinterpret_cast<const bf16x8*>(k_rd + kb * 32 * 256 + kofs[kk]);
      }
    };
    auto mfma_op = [&](int j) __attribute__((always_inline)) {
      if (j < NPV) {
        const int mbi = j % MB, ch = (j / MB) & 1, kb = j / (2 * MB);
        o[mbi] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op[j], pk[kb][ch], o[mbi], 0, 0, 0);
      } else {
        const int kk = (j - NPV) >> 1, kb = (j - NPV) & 1;
        const f32x16 zacc = {};
        s_nxt[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op[j], qf[kk], kk == 0 ? zacc : s_nxt[kb], 0, 0, 0);
      }
    };
    // element n = 0..31 of the tile for this lane: key block n >> 4, element n & 15
    auto get = [&](int n) __attribute__((always_inline)) { return s_cur[n >> 4][n & 15]; };
    auto set = [&](int n, float v) __attribute__((always_inline)) { s_cur[n >> 4][n & 15] = v; };
    float mxp[3] = {-INFINITY, -INFINITY, -INFINITY};
    float alpha = 1.f, m_base = 0.f, rs = 0.f;
    // An empty asm that takes a value in a register: the computation of the value
    // stays before it (the compiler would otherwise sink the softmax past the
    // barrier at the end of the step, next to its consumers).
    auto pin = [](float& x) __attribute__((always_inline)) { asm volatile("" : "+v"(x)); };
    // The row sum adds each exp2 result one exp later (pend holds the last one): an
    // add right behind its transcendental needs a wait state, which the compiler
    // fills with an s_nop.
    float pend = 0.f;
    auto exp_elem = [&](int n) __attribute__((always_inline)) {
      float pe = fast_exp2(__builtin_fmaf(get(n), p.scale_log2, -m_base));
      pin(pe);
      set(n, pe);
      if (n > 0) rs += pend;
      pend = pe;
    };

    // exp2 slices: units 4 .. 4 + kTwo - 1 take two elements each, the rest one, so the
    // 32 elements of the tile are spread over units 4 .. NU - 1.
    constexpr int kTwo = 32 - (NU - 4);
    static_assert(kTwo >= 0 && kTwo <= NU - 4, "the softmax slices must fit the step's units");
#pragma unroll
    for (int j = 0; j < kAhead; ++j) read_op(j);
#pragma unroll
    for (int i = 0; i < NU; ++i) {
      if (i + kAhead < NU) read_op(i + kAhead);
      mfma_op(i);
      // row (< 64) x row stride (< 2^24 bytes, checked on the host): a 24-bit multiply-add
      if (i < 4) {
        dma16(dk.base, __umul24(min(lr + 4 * i, dk.last), (uint32_t)kst) + ((lcn ^ (uint32_t)i) << 4),
              lds_u32(k_ld + (16 * wave + 4 * i) * 256));
      } else if (i < 8) {
        const int r = i - 4;
        dma16(dv.base, __umul24(min(lr + 4 * r, dv.last), (uint32_t)vst) + ((lcn ^ (uint32_t)r) << 4),
              lds_u32(v_ld + (16 * wave + 4 * r) * 256));
      }
      if constexpr (kAheadSrc) {  // the next step loads K tile t + 3 and V tile t + 1
        if (i == kRawUnit) {
          raw_k = tile_blk_raw(t + 3);
          raw_v = tile_blk_raw(t + 1);
        } else if (i == kSrcUnit) {
          dk_cur = paged_src(t + 3, raw_k, kcol, kst, kpage, koff_nx);
          dv_cur = paged_src(t + 1, raw_v, vcol, vst, vpage, voff_nx);
          koff_nx = next_off(koff_nx);
          voff_nx = next_off(voff_nx);
        }
      }
      if (i < 3) {  // mask and partial max of elements 11i .. 11i+10
#pragma unroll
        for (int n = 11 * i; n < min(32, 11 * i + 11); ++n) {
          if (MASKED) {
            // element n is key kt + 32(n >> 4) + 8((n & 15) >> 2) + 4hf + (n & 3)
            if (32 * (n >> 4) + 8 * ((n & 15) >> 2) + (n & 3) > rel) set(n, -INFINITY);
          }
          mxp[i] = fmaxf(mxp[i], get(n));
        }
        pin(mxp[i]);
      } else if (i == 3) {
        // Lazy rescale: the running max moves only when the tile's max exceeds it
        // by more than kRescaleThreshold; O and l are zero until the first move.
        const float mx = half_wave_max(fmaxf(fmaxf(mxp[0], mxp[1]), mxp[2])) * p.scale_log2;
        const bool grow = mx > m_run + kRescaleThreshold;
        const float m_new = grow ? mx : m_run;
        alpha = (grow && m_run != -INFINITY) ? fast_exp2(m_run - m_new) : 1.f;
        m_run = m_new;
        m_base = (m_new == -INFINITY) ? 0.f : m_new;
        pin(m_base);
        pin(alpha);
      } else if (i < 4 + kTwo) {  // two elements per unit, then one
        exp_elem(2 * (i - 4));
        exp_elem(2 * (i - 4) + 1);
      } else {
        exp_elem(2 * kTwo + (i - 4 - kTwo));
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    rs += pend;
    l_run = l_run * alpha + rs;
    // P^T as bf16 B operands: chunk ch of key block kb = elements 8ch .. 8ch+7
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int ch = 0; ch < 2; ++ch) {
        u32x4v w;
#pragma unroll
        for (int u = 0; u < 4; ++u) w[u] = pack_bf16x2(s_cur[kb][8 * ch + 2 * u], s_cur[kb][8 * ch + 2 * u + 1]);
        pk[kb][ch] = __builtin_bit_cast(bf16x8, w);
        asm volatile("" : "+v"(pk[kb][ch]));
      }
    asm volatile("" : "+v"(l_run), "+v"(m_run));
    rescale(alpha);
    sync_tiles();
  };
  auto step = [&](auto par, auto masked, int t) __attribute__((always_inline)) {
    if constexpr (decltype(par)::value != 0)
      step_body(masked, t, s_odd, s_even, k_buf0, v_buf0, k_buf1, v_buf1);
    else
      step_body(masked, t, s_even, s_odd, k_buf1, v_buf1, k_buf0, v_buf0);
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using Masked = std::integral_constant<bool, true>;
  using Plain = std::integral_constant<bool, false>;

  // ---- prologue: V buffer 1 zeroed, K tiles 0 and 1, S^T of tile 0 ----------------
  if (n_tiles > 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<u32x4v*>(v_buf1 + (i * kThreads + tid) * 16) = u32x4v{0u, 0u, 0u, 0u};
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int ch = 0; ch < 2; ++ch) pk[kb][ch] = __builtin_bit_cast(bf16x8, u32x4v{0u, 0u, 0u, 0u});
    {
      const DmaSrc d0 = dma_src(0, kcol, kst, true), d1 = dma_src(1, kcol, kst, true);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t off = ((lchunk0 ^ (uint32_t)j) << 4);
        dma16(d0.base, min(lrow0 + 4 * j, d0.last) * (uint32_t)kst + off, lds_u32(k_buf0 + (16 * wave + 4 * j) * 256));
        dma16(d1.base, min(lrow0 + 4 * j, d1.last) * (uint32_t)kst + off, lds_u32(k_buf1 + (16 * wave + 4 * j) * 256));
      }
    }
    // Paged: block ids of the item's tiles, read once into LDS (the steps take them
    // from there); the barrier below publishes them.
    if (MODE == kPagedTiles) {
      for (int i = tid; i < n_tiles; i += kThreads)
        tile_blk[i] = p.block_table[(int64_t)b * p.bt_row_stride + (k_begin + i * kTileK) / p.page_size];
    }
    sync_tiles();
    qk(k_buf0, s_even);
    order_qk();
    if constexpr (kAheadSrc) {  // step 0 loads K tile 2 and V tile 0
      const uint32_t ps = (uint32_t)p.page_size, kb = (uint32_t)k_begin % ps;
      dk_cur = paged_src(2, tile_blk_raw(2), kcol, kst, kpage, (kb + 2 * kTileK) % ps);
      dv_cur = paged_src(0, tile_blk_raw(0), vcol, vst, vpage, kb);
      koff_nx = (kb + 3 * kTileK) % ps;
      voff_nx = (kb + kTileK) % ps;
    }
    sync_tiles();  // K buffer 0 is reloaded during step 0

    // ---- steps: unmasked pairs, masked pairs, a masked single step if n is odd ---
    // Issue priority per the plan (kPPrio).  Alternating (0 and 2 on the two steps of a
    // pair) applies to paged calls only: 8 requests sharing an image 169.5 against 177.3
    // us with equal priorities, the two-image 7B batch 113.3 against 114.8 us; square
    // causal calls, paged or contiguous, measured slower with it (paged 10741^2 481.3
    // against 467.6 us) and the planner leaves them at equal priorities.  By remaining
    // tiles: 3 for six or more, 2 for four or five, 1 for two or three, 0 for the last.
    const int prio_mode = p.prio_mode;
    auto prio = [&](int t, auto high) __attribute__((always_inline)) {
      if (prio_mode == kPrioRemaining) {
        const int r = n_tiles - t;
        if (r >= 6) __builtin_amdgcn_s_setprio(3);
        else if (r >= 4) __builtin_amdgcn_s_setprio(2);
        else if (r >= 2) __builtin_amdgcn_s_setprio(1);
        else __builtin_amdgcn_s_setprio(0);
      } else if constexpr (MODE != kContiguous) {
        if (prio_mode == kPrioAlternate) __builtin_amdgcn_s_setprio(decltype(high)::value ? 2 : 0);
      }
    };
    int t = 0;
    for (; t + 1 < n_plain; t += 2) {
      prio(t, std::false_type{});
      step(I0{}, Plain{}, t);
      prio(t + 1, std::true_type{});
      step(I1{}, Plain{}, t + 1);
    }
    for (; t + 1 < n_tiles; t += 2) {
      prio(t, std::false_type{});
      step(I0{}, Masked{}, t);
      prio(t + 1, std::true_type{});
      step(I1{}, Masked{}, t + 1);
    }
    prio(t, std::false_type{});
    if (t < n_tiles) step(I0{}, Masked{}, t);  // t is even here
    // ---- drain: O^T += V^T P^T of the last tile ---------------------------------------
    if ((n_tiles - 1) & 1) pv_last(v_buf1);
    else pv_last(v_buf0);
  }

  // ---- epilogue: lane holds O^T[d = 32mb + 8i + 4hf + j][col] in o[mb][4i + j] ----
  // The wave's 32 columns are staged in LDS as bf16 rows of 256 bytes (16-byte
  // chunk c of column x at slot c ^ (x & 15)) and then stored as whole rows, 16
  // bytes per lane: the rows of the `group` heads of one position are adjacent in
  // the output (and all rows of a workspace slot are), so each store instruction
  // writes 1 KB of contiguous memory.  The stores write through L2 (st16_wt): the
  // next kernel reads them, and dirty L2 lines would be written back between the two
  // kernels.  The K buffers are free here.
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  uint8_t* stage = (wave < 2 ? k_buf0 : k_buf1) + (wave & 1) * (kTileK * 256 / 2);
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      u32x2v w;
      w[0] = pack_bf16x2(o[mb][4 * i] * inv, o[mb][4 * i + 1] * inv);
      w[1] = pack_bf16x2(o[mb][4 * i + 2] * inv, o[mb][4 * i + 3] * inv);
      *reinterpret_cast<u32x2v*>(stage + lc * 256 + (((4 * mb + i) ^ (lc & 15)) << 4) + 8 * hf) = w;
    }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the wave's staging writes are done
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int x = 4 * r + (lane >> 4);  // column of the wave
    const int ch = lane & 15;            // 16-byte chunk (dims 8ch .. 8ch+7)
    const u32x4v v = *reinterpret_cast<const u32x4v*>(stage + x * 256 + ((ch ^ (x & 15)) << 4));
    const int colx = wave * 32 + x;
    const int posx = colx / p.group;
    if (posx < q_count) {
      // A split of a longer key range writes its normalised partial in bf16 plus
      // (m, l) in fp32 to its workspace slot.
      uint16_t* dst = slot < 0 ? p.out + (int64_t)(q0 + q_start + posx) * p.out_row_stride +
                                     (int64_t)(g * p.group + colx - posx * p.group) * kHeadDim
                               : p.part_o + ((int64_t)slot * kCols + colx) * kHeadDim;
      st16_wt(dst + 8 * ch, v);
    }
  }
  if (slot >= 0 && valid && hf == 0)
    st8_wt(p.part_ml + ((int64_t)slot * kCols + col) * 2,
           (uint64_t)__float_as_uint(m_run) | ((uint64_t)__float_as_uint(l_tot) << 32));
}

// Merge the split-KV partials of one query tile:
//   O = sum_s 2^(m_s - M) l_s Ohat_s / sum_s 2^(m_s - M) l_s,  M = max_s m_s,
// with Ohat_s = O_s / l_s stored in bf16.  grid = (combine items, kCols /
// kCombineCols): a workgroup owns kCombineCols columns and each lane one 8-dim
// (16-byte) slice of a column.  The merge is latency-bound (a few KB per split),
// so it keeps many loads in flight: the 16 lanes of a column share the (m, l)
// loads of the max and reduce it with shuffles, and the weighted sum is unrolled
// B splits deep.  The first B partials do not depend on the max, so they are
// loaded together with the maxima: one round trip instead of two.
constexpr int kCombineCols = kThreads / (kHeadDim / 8);  // 16 columns per workgroup

// Weighted sum of one column slice over the splits: a.acc += sum_s w_s Ohat_s and
// a.lsum += sum_s w_s, w_s = 2^(m_s - M) l_s.  The 16 lanes of a column form one
// DPP row: lane j loads (m, l) of splits j, j + 16, j + 32, j + 48 of each chunk of 64,
// computes their weights, and a row broadcast (row_newbcast) hands w_s to the row when
// split s is accumulated, so (m, l) is loaded once per split and column instead of
// once per lane.  The partials are loaded in batches of B (indices clamped to the last
// split, extra terms weighted 0) so that a batch is in flight at once; the first batch
// does not depend on the max and is issued with the (m, l) loads.
constexpr int kCombineLanes = kHeadDim / 8;  // lanes per column = one DPP row
static_assert(kCombineLanes == 16, "a column is one DPP row");
constexpr int64_t kPartMlStride = (int64_t)kCols * 2;
constexpr int64_t kPartOStride = (int64_t)kCols * kHeadDim;

template <int J>
__device__ __forceinline__ float row_bcast(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x150 + J, 0xf,
                                                               0xf, false));
}

struct CombineAcc {
  float acc[8];
  float lsum;
};

// Splits s16 + J0 + k, k < B, whose weights lanes J0 + k of the row hold in wsrc.
template <int J0, int B, int... K>
__device__ __forceinline__ void accumulate_batch(std::integer_sequence<int, K...>, float wsrc,
                                                 const u32x4v (&v)[B], CombineAcc& a) {
  auto one = [&](auto j, const u32x4v& x) __attribute__((always_inline)) {
    const float wl = row_bcast<decltype(j)::value>(wsrc);
    a.lsum += wl;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      a.acc[2 * t] += wl * bf16_bits_to_f32(x[t] & 0xffffu);
      a.acc[2 * t + 1] += wl * bf16_bits_to_f32(x[t] >> 16);
    }
  };
  (one(std::integral_constant<int, J0 + K>{}, v[K]), ...);
}

template <int B>
__device__ __forceinline__ void load_partials(const uint16_t* po, int s0, int nsplit, u32x4v (&v)[B]) {
#pragma unroll
  for (int k = 0; k < B; ++k) v[k] = *reinterpret_cast<const u32x4v*>(po + min(s0 + k, nsplit - 1) * kPartOStride);
}

// The batches of one broadcast slot (splits s16 .. s16 + 15) from J0 on, stopping at nsplit.
template <int J0, int B>
__device__ __forceinline__ void slot_batches(const uint16_t* po, int s16, int nsplit, float wsrc, CombineAcc& a) {
  if constexpr (J0 < kCombineLanes) {
    if (s16 + J0 >= nsplit) return;
    u32x4v v[B];
    load_partials<B>(po, s16 + J0, nsplit, v);
    accumulate_batch<J0, B>(std::make_integer_sequence<int, B>{}, wsrc, v, a);
    slot_batches<J0 + B, B>(po, s16, nsplit, wsrc, a);
  }
}

template <int B>
__device__ __forceinline__ void combine_slice(const float* ml, const uint16_t* po, int nsplit, int sub,
                                              CombineAcc& a) {
  static_assert(kCombineLanes % B == 0, "a batch lies inside one broadcast slot");
  constexpr int kChunk = 4 * kCombineLanes;  // splits whose (m, l) one load round covers
  auto load_ml = [&](int c0, float2(&m4)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < 4; ++k)
      m4[k] = *reinterpret_cast<const float2*>(ml + min(c0 + sub + k * kCombineLanes, nsplit - 1) * kPartMlStride);
  };
  float2 m4[4];
  load_ml(0, m4);
  u32x4v v0[B];
  load_partials<B>(po, 0, nsplit, v0);
  float mmax = -INFINITY;
#pragma unroll
  for (int k = 0; k < 4; ++k) mmax = fmaxf(mmax, m4[k].x);
  for (int c0 = kChunk; c0 < nsplit; c0 += kChunk) {
    float2 mc[4];
    load_ml(c0, mc);
#pragma unroll
    for (int k = 0; k < 4; ++k) mmax = fmaxf(mmax, mc[k].x);
  }
#pragma unroll
  for (int x = 1; x < kCombineLanes; x <<= 1) mmax = fmaxf(mmax, __shfl_xor(mmax, x));
  // Every split empty (mmax = -inf): every weight is 0.  The first batch is used
  // unconditionally, so the compiler cannot sink its loads below the max.
  const bool any = mmax != -INFINITY;
  float w4[4];
  auto weights = [&](int c0) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < 4; ++k)
      w4[k] = any && c0 + sub + k * kCombineLanes < nsplit ? fast_exp2(m4[k].x - mmax) * m4[k].y : 0.f;
  };
  weights(0);
  accumulate_batch<0, B>(std::make_integer_sequence<int, B>{}, w4[0], v0, a);
  slot_batches<B, B>(po, 0, nsplit, w4[0], a);
  for (int s16 = kCombineLanes; s16 < nsplit; s16 += kCombineLanes) {
    const int c0 = s16 & ~(kChunk - 1);
    if (c0 == s16) {
      load_ml(c0, m4);
      weights(c0);
    }
    const int slot = (s16 - c0) / kCombineLanes;
    const float wsrc = slot == 0 ? w4[0] : slot == 1 ? w4[1] : slot == 2 ? w4[2] : w4[3];
    slot_batches<0, B>(po, s16, nsplit, wsrc, a);
  }
}

__global__ __launch_bounds__(kThreads) void attn_combine_kernel(const Params p) {
  const int32_t* it = p.combine + (int64_t)blockIdx.x * kItemInts;
  const int g = it[1], q_start = it[2], q_count = it[3];
  const int first = it[4], nsplit = it[5];
  const int q0 = it[7];
  const int sub = threadIdx.x % (kHeadDim / 8);  // the lane's slice; lanes of a column are adjacent
  const int col = blockIdx.y * kCombineCols + threadIdx.x / (kHeadDim / 8);
  const int d = 8 * sub;
  const int pos = col / p.group;
  // Whole 16-lane groups agree (same column), so the shuffles inside stay within
  // active lanes.
  if (pos >= q_count) return;
  const float* ml = p.part_ml + ((int64_t)first * kCols + col) * 2;
  const uint16_t* po = p.part_o + ((int64_t)first * kCols + col) * kHeadDim + d;
  CombineAcc a = {};
  // Batch depth by split count: deep batches for long merges, no wasted loads for
  // short ones.
  if (nsplit > 8)
    combine_slice<16>(ml, po, nsplit, sub, a);
  else
    combine_slice<4>(ml, po, nsplit, sub, a);
  const float lsum = a.lsum;
  const float(&acc)[8] = a.acc;
  const int hh = col - pos * p.group;
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  uint16_t* orow = p.out + (int64_t)(q0 + q_start + pos) * p.out_row_stride +
                   (int64_t)(g * p.group + hh) * kHeadDim + d;
  u32x4v w;
#pragma unroll
  for (int t = 0; t < 4; ++t) w[t] = pack_bf16x2(acc[2 * t] * inv, acc[2 * t + 1] * inv);
  st16_wt(orow, w);
}

}  // namespace
}  // namespace attn
}  // namespace vlc

VLC_API int vlc_varlen_attn_fwd(const void* q, int64_t q_row_stride, const void* k,
                                int64_t k_row_stride, const void* v, int64_t v_row_stride,
                                const int32_t* block_table, int64_t bt_row_stride, int page_size,
                                int64_t num_blocks, const int32_t* cu_seqlens_q,
                                const int32_t* cu_seqlens_k, int num_seqs, int num_heads_q,
                                int num_heads_kv, int head_dim, float softmax_scale, int causal,
                                const int32_t* plan_host, const int32_t* plan_dev, int64_t plan_len,
                                void* out, int64_t out_row_stride, void* workspace,
                                int64_t workspace_bytes, void* stream) {
  using namespace vlc;
  using namespace vlc::attn;
  if (head_dim != kHeadDim && head_dim != kHeadDimNarrow) return VLC_ERR_UNSUPPORTED;
  if (head_dim == kHeadDimNarrow && block_table) return VLC_ERR_UNSUPPORTED;  // contiguous K/V only
  if (num_heads_q <= 0 || num_heads_kv <= 0 || num_heads_q % num_heads_kv != 0) return VLC_ERR_INVALID;
  if (!plan_host || !plan_dev || plan_len < kHeaderInts) return VLC_ERR_PLAN;
  const int32_t* h = plan_host;
  const int group = num_heads_q / num_heads_kv;
  if (h[kPMagic] != kPlanMagic || h[kPGroup] != group || h[kPNumSeqs] != num_seqs ||
      h[kPNumHeadsKv] != num_heads_kv || h[kPCausal] != (causal ? 1 : 0) ||
      h[kPHeadDim] != head_dim || h[kPCols] != kCols)
    return VLC_ERR_PLAN;
  const int64_t n_items = h[kPNumItems], n_comb = h[kPNumCombine], n_slots = h[kPNumSlots];
  if (plan_len < kHeaderInts + (n_items + n_comb) * kItemInts) return VLC_ERR_PLAN;
  if (n_items == 0) return VLC_OK;
  // The kernels index with the plan's fields: check them against the call.
  for (int64_t i = 0; i < n_items + n_comb; ++i) {
    const int32_t* v = h + kHeaderInts + i * kItemInts;
    const bool is_item = i < n_items;
    if (v[0] < 0 || v[0] >= num_seqs || v[1] < 0 || v[1] >= num_heads_kv || v[2] < 0 || v[3] < 0 ||
        v[3] > kCols / group)
      return VLC_ERR_PLAN;
    if (is_item && (v[4] < 0 || v[5] < v[4] || (int64_t)v[5] - v[4] > (int64_t)kMaxItemTiles * kTileK ||
                    v[6] >= n_slots || v[5] > v[10]))
      return VLC_ERR_PLAN;
    if (!is_item && (v[4] < 0 || v[5] < 1 || (int64_t)v[4] + v[5] > n_slots)) return VLC_ERR_PLAN;
  }
  if (!q || !k || !v || !out) return VLC_ERR_INVALID;
  if (!(softmax_scale > 0.f)) return VLC_ERR_INVALID;
  // 16-byte vector access of every row.
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out) || q_row_stride % 8 ||
      k_row_stride % 8 || v_row_stride % 8 || out_row_stride % 8)
    return VLC_ERR_INVALID;
  // tile-load offsets are 24-bit products: row (< 64) x row stride in bytes
  if (k_row_stride * 2 >= (int64_t(1) << 24) || v_row_stride * 2 >= (int64_t(1) << 24)) return VLC_ERR_UNSUPPORTED;
  if (q_row_stride < (int64_t)num_heads_q * kHeadDim || out_row_stride < (int64_t)num_heads_q * kHeadDim ||
      k_row_stride < (int64_t)num_heads_kv * kHeadDim || v_row_stride < (int64_t)num_heads_kv * kHeadDim)
    return VLC_ERR_INVALID;
  if (block_table && (page_size <= 0 || bt_row_stride <= 0 || num_blocks <= 0)) return VLC_ERR_INVALID;
  // Paged K/V: a wave loads 16 consecutive keys of a tile, which must share a page.
  if (block_table && page_size % 16 != 0) return VLC_ERR_UNSUPPORTED;
  if (n_slots > 0 && (!workspace || workspace_bytes < n_slots * kSlotBytes || !aligned16(workspace)))
    return VLC_ERR_WORKSPACE;

  Params prm{};
  prm.q = static_cast<const uint16_t*>(q);
  prm.k = static_cast<const uint16_t*>(k);
  prm.v = static_cast<const uint16_t*>(v);
  prm.block_table = block_table;
  prm.cu_q = cu_seqlens_q;
  prm.cu_k = cu_seqlens_k;
  prm.items = plan_dev + kHeaderInts;
  prm.combine = plan_dev + kHeaderInts + n_items * kItemInts;
  prm.out = static_cast<uint16_t*>(out);
  prm.part_o = static_cast<uint16_t*>(workspace);
  prm.part_ml = n_slots > 0 ? reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                                        n_slots * (int64_t)kCols * kHeadDim * 2)
                            : nullptr;
  prm.q_row_stride = q_row_stride;
  prm.k_row_stride = k_row_stride;
  prm.v_row_stride = v_row_stride;
  prm.bt_row_stride = bt_row_stride;
  prm.out_row_stride = out_row_stride;
  prm.num_blocks = num_blocks;
  prm.page_size = block_table ? page_size : 1;
  prm.group = group;
  prm.causal = causal ? 1 : 0;
  prm.prio_mode = h[kPPrio];
  prm.scale_log2 = softmax_scale * 1.4426950408889634f;

  hipStream_t s = as_stream(stream);
  const int mode = !block_table ? kContiguous : (page_size % kTileK == 0 ? kPagedTiles : kPagedRows);
  if (head_dim == kHeadDimNarrow)
    hipLaunchKernelGGL((attn_fwd_kernel<kContiguous, kHeadDimNarrow / 16, (kHeadDimNarrow + 31) / 32>),
                       dim3((unsigned)n_items), dim3(kThreads), 0, s, prm);
  else if (mode == kContiguous)
    hipLaunchKernelGGL(attn_fwd_kernel<kContiguous>, dim3((unsigned)n_items), dim3(kThreads), 0, s, prm);
  else if (mode == kPagedTiles) {
    // Reading block ids a step ahead: paged 10741^2 473.3 against 480.1 us, 8 requests
    // sharing an image 169.6 against 175.4, the two-image 7B batch 114.6 against 116.5.
    // One-wave plans (kPrioRemaining: the warm 4K request) read 0.6-0.9 % slower with it,
    // in runs where a byte-identical copy of a build read 0.3-0.4 % slower than the
    // original; they keep the in-step reads.
    if (prm.prio_mode == kPrioRemaining)
      hipLaunchKernelGGL(attn_fwd_kernel<kPagedTiles>, dim3((unsigned)n_items), dim3(kThreads), 0, s, prm);
    else
      hipLaunchKernelGGL((attn_fwd_kernel<kPagedTiles, 8, 4, true>), dim3((unsigned)n_items), dim3(kThreads), 0, s,
                         prm);
  } else
    hipLaunchKernelGGL(attn_fwd_kernel<kPagedRows>, dim3((unsigned)n_items), dim3(kThreads), 0, s, prm);
  int st = launch_status();
  if (st != VLC_OK) return st;
  if (n_comb > 0) {
    hipLaunchKernelGGL(attn_combine_kernel, dim3((unsigned)n_comb, kCols / kCombineCols), dim3(kThreads), 0,
                       s, prm);
    st = launch_status();
  }
  return st;
}
