// Paged GQA decode attention for gfx950: the replacement of
// flash_attn_with_kvcache(q.unsqueeze(1), k_cache, v_cache, cache_seqlens=context_lens,
// block_table=block_tables, softmax_scale=scale, causal=True) at layers/attention.py:71-74.
//
// One query per sequence; query b attends keys [0, cache_seqlens[b]) of its paged
// cache.  The work is bandwidth: every K/V row of every sequence is read once.
//
// Decomposition: one workgroup per (key chunk, kv head, sequence), grid
// (splits, Hkv, B).  Its four waves each stream a contiguous quarter of the
// chunk in 32-key tiles, double-buffered global -> LDS by DMA into the wave's own
// LDS region, so the waves never wait for each other inside the loop.  The 16
// MFMA columns are the q heads of the kv head (group <= 16):
//   S^T (16 keys x 16 heads) = K (16 x 32 dims) . Q^T        v_mfma_f32_16x16x32_bf16
//   O^T (16 dims x 16 heads) += V^T (16 dims x 32 keys) . P^T
// A lane owns one head and 4 keys of each 16-key block, so P^T leaves the S^T
// accumulators already in the B-operand layout of the second product; V is
// read transposed from LDS (ds_read_b64_tr_b16).  The column max and sum cross
// the four 16-lane groups with v_permlane16_swap / v_permlane32_swap (VALU).
//
// Merge: the four waves merge (O, m, l) through LDS.  A sequence-head pair whose
// keys span several chunks writes each chunk's (O, m, l) to the workspace; the
// workgroup that finishes last (a device-scope ticket counter, taken once the
// partials have landed) merges all chunks with the log-sum-exp rule, writes the
// output and resets its counter to zero, so one launch does the whole call.
#include <algorithm>
#include <mutex>

#include "common.h"

namespace vlc {
namespace decode {
namespace {

constexpr int kHeadDim = 128;
constexpr int kMinTileKeys = 16;                  // page_size must be a multiple of this
constexpr int kCols = 16;                         // MFMA columns = q heads of one kv head
constexpr int kWgKeys = 128;                      // key chunks are multiples of this
constexpr int kMaxPagesPerWave = 64;              // block ids a wave keeps in a register

// Kernel shapes: W waves per workgroup, S pipeline stages per wave, T keys per
// tile (16 or 32).  A wave keeps S - 1 tiles in flight while it computes one, in
// W * S * T * 512 bytes of LDS (K and V of a tile: T rows of 256 bytes each).  A
// tile takes T / 2 LDS-DMA instructions, so S - 1 tiles ahead need a wait count of
// (S - 1) T / 2 <= 63.
constexpr int pipeline_code(int w, int s, int t) { return (t == 16 ? 0x100 : 0) | (16 * w + s); }

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;

struct Params {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const int32_t* block_table;
  const int32_t* seqlens;
  uint16_t* out;
  uint32_t* counters;  // [B * Hkv], zero between calls
  float* part_ml;      // [B * Hkv][grid_splits][kCols][2]: (m in scaled log2 units, l)
  float* part_o;       // [B * Hkv][grid_splits][kCols][kHeadDim]: unnormalised O
  int64_t q_row_stride;    // elements between sequences of q
  int64_t out_row_stride;  // elements between sequences of out
  int64_t cache_row_stride;  // elements per cache row (token)
  int64_t bt_row_stride;
  int64_t num_blocks;
  int page_size;
  int bt_cols;
  int group;
  int num_heads_kv;
  int key_chunk;    // keys per workgroup (multiple of kWgKeys)
  int max_keys;     // keys the grid and the block table cover
  float scale_log2;
};

// All-zero row: the source of keys past the end of a sequence and of pages whose
// block id is outside the cache.
__device__ __attribute__((aligned(256))) const uint32_t kZeroRow[64] = {};

// 16-byte chunk c of LDS row r lives in slot c ^ swizzle(r).
//   K (read 16 rows x one chunk per 16-lane group, ds_read_b128): r mod 16.
//   V (transpose reads: rows 4q + f, chunks 2mb, 2mb + 1 for groups q = 0, 1 of a
//   half-wave): bits 2-3 follow r mod 4, bit 1 follows (r / 4) mod 2, so the 16
//   (row, chunk) pairs of a half-wave hit 16 distinct slots.
__device__ __forceinline__ int swz_k(int r) { return r & 15; }
__device__ __forceinline__ int swz_v(int r) { return ((r & 3) << 2) | (((r >> 2) & 1) << 1); }

__device__ __forceinline__ uint32_t lds_u32(const void* ptr) {
  return (uint32_t)(uintptr_t)(const lds_void*)ptr;
}
// global_load_lds_dwordx4 from a per-lane 64-bit address: lane i's 16 bytes land at
// LDS M0 + 16 i.  Issued through inline assembly so that the compiler does not model
// it as a flat access of unknown order; the hardware counts it in vmcnt.  The memory
// clobber keeps every LDS read of the buffer it overwrites (issued earlier in program
// order) ahead of it.  kNt sets the nontemporal cache policy: for the batch 4 x 13.4k
// call (110 MB) it measured 29.2 against 30.5 us; the host uses it when a call reads
// at most 1 GiB (beyond that the re-rotation kernel measured nontemporal loads slower).
template <bool kNt>
__device__ __forceinline__ void dma16_addr(const void* addr, uint32_t lds) {
  // lds is uniform (wave and stage); readfirstlane keeps it in a scalar register
  // where the compiler's divergence analysis cannot tell.
  if (kNt)
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off nt"
                 :
                 : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(addr)
                 : "m0", "memory");
  else
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                 :
                 : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(addr)
                 : "m0", "memory");
}
constexpr int64_t kNtMaxBytes = (int64_t)1 << 30;

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2 v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// Reductions over the four 16-lane groups (lanes l, l ^ 16, l ^ 32, l ^ 48).
// v_permlane16_swap with both operands holding x leaves, in every lane, x of the
// lane in one register and x of its partner 16 lanes away in the other (rows
// 0 <-> 1, 2 <-> 3); v_permlane32_swap does the same for the two half-waves.
// Issued through inline assembly with both registers as in/out operands: the
// compiler (ROCm 7.2) folds the two results of the swap builtins into one, which
// drops the partner's value.  The s_nop covers the VALU-write -> permlane-read
// hazard, which the compiler does not track through inline assembly.
__device__ __forceinline__ void swap16(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap32(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ float group4_max(float x) {
  float a = x, b = x;
  swap16(a, b);
  a = b = fmaxf(a, b);
  swap32(a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float group4_sum(float x) {
  float a = x, b = x;
  swap16(a, b);
  a = b = a + b;
  swap32(a, b);
  return a + b;
}

// Waits until at most `ahead` (<= MAX) tiles of DMA instructions (D per tile) are in flight.
template <int D, int MAX>
__device__ __forceinline__ void wait_tiles(int ahead) {
  static_assert(MAX * D <= 63 && MAX <= 7, "vmcnt range");
  if (ahead <= 0) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    return;
  }
#define VLC_WAIT_CASE(K)                                                 \
  if constexpr (MAX >= K)                                                \
    if (ahead == K) {                                                    \
      asm volatile("s_waitcnt vmcnt(%0)" : : "n"(K * D) : "memory");    \
      return;                                                            \
    }
  VLC_WAIT_CASE(1)
  VLC_WAIT_CASE(2)
  VLC_WAIT_CASE(3)
  VLC_WAIT_CASE(4)
  VLC_WAIT_CASE(5)
  VLC_WAIT_CASE(6)
  VLC_WAIT_CASE(7)
#undef VLC_WAIT_CASE
}

// 16- and 8-byte accesses at agent scope (sc1: written through to, and read from,
// the level that is coherent across XCDs).  The 16-byte ones are inline assembly
// (the compiler's atomics stop at 8 bytes); the compiler does not count those
// loads in its waits, so their results are used only after an explicit vmcnt(0)
// that takes them as operands.
__device__ __forceinline__ void st16_agent(void* addr, f32x4 v) {
  st16_wt(addr, __builtin_bit_cast(u32x4_vec, v));
}
__device__ __forceinline__ f32x4 ld16_agent(const void* addr) {
  f32x4 v;
  asm volatile("global_load_dwordx4 %0, %1, off sc1" : "=v"(v) : "v"(addr) : "memory");
  return v;
}
__device__ __forceinline__ void st_ml_agent(float* addr, float m, float l) {
  st8_wt(addr, (uint64_t)__float_as_uint(m) | ((uint64_t)__float_as_uint(l) << 32));
}
__device__ __forceinline__ float2 ld_ml_agent(const float* addr) {
  const uint64_t bits =
      __hip_atomic_load(reinterpret_cast<const uint64_t*>(addr), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_float2(__uint_as_float((uint32_t)bits), __uint_as_float((uint32_t)(bits >> 32)));
}

__device__ __forceinline__ float merge_weight(float m, float mx) {
  return m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - mx);
}

template <int W, int S, int T, bool NT>
__global__ __launch_bounds__(W * 64) void decode_attn_kernel(const Params p) {
  constexpr int kThreads = W * 64;
  constexpr int kTileKeys = T;
  constexpr int kTileBytes = T * kHeadDim * 2;  // K (or V) of one tile
  constexpr int kStageBytes = 2 * kTileBytes;
  constexpr int kWaveLds = S * kStageBytes;
  constexpr int kDma = T / 2;                   // LDS-DMA instructions per tile (K and V)
  constexpr int kBlocks = T / 16;               // 16-key blocks per tile
  static_assert((S - 1) * kDma <= 63, "vmcnt range");
  static_assert(kCols * kHeadDim * 4 + kCols * 8 <= kWaveLds, "merge scratch fits the wave's LDS");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[W * kWaveLds];
  __shared__ int last_flag;

  const int split = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int c = lane & 15;   // column (q head within the group)
  const int q4 = lane >> 4;  // 16-lane group

  // The wave's page ids and q fragments do not depend on the context length, so
  // they are loaded before it (in bounds whatever it is): the three loads overlap
  // instead of the page ids waiting for the length.
  const int wchunk = p.key_chunk / W;
  const int64_t wkb64 = (int64_t)split * p.key_chunk + (int64_t)wave * wchunk;
  // Block ids of the wave's pages: lane i holds the id of page first_page + i.
  const int64_t first_page64 = wkb64 / p.page_size;
  int blk_reg = -1;
  {
    const int64_t pg = first_page64 + lane;
    if (pg < p.bt_cols && lane < kMaxPagesPerWave) blk_reg = p.block_table[(int64_t)b * p.bt_row_stride + pg];
  }

  // Q^T fragments (B operand of S^T = K Q^T): lane holds Q[head c][32 kk + 8 q4 .. + 8].
  const bool col_ok = c < p.group;
  bf16x8 qf[4];
  {
    const uint16_t* qrow = p.q + (int64_t)b * p.q_row_stride +
                           (int64_t)(g * p.group + (col_ok ? c : 0)) * kHeadDim + 8 * q4;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      u32x4v w = *reinterpret_cast<const u32x4v*>(qrow + 32 * kk);
      if (!col_ok) w = u32x4v{0u, 0u, 0u, 0u};
      qf[kk] = __builtin_bit_cast(bf16x8, w);
    }
  }

  int ctx = p.seqlens[b];
  ctx = max(0, min(ctx, p.max_keys));
  const int n_splits = max(1, (ctx + p.key_chunk - 1) / p.key_chunk);
  if (split >= n_splits) return;  // uniform over the workgroup, before any barrier
  const int kb = split * p.key_chunk;
  const int ke = min(ctx, kb + p.key_chunk);
  const int wkb = kb + wave * wchunk;
  const int wke = min(ke, wkb + wchunk);
  const int n_tiles = wke > wkb ? (wke - wkb + kTileKeys - 1) / kTileKeys : 0;
  const int first_page = wkb / p.page_size;

  uint8_t* wbuf = lds + wave * kWaveLds;
  const char* kbase = reinterpret_cast<const char*>(p.k + (int64_t)g * kHeadDim);
  const char* vbase = reinterpret_cast<const char*>(p.v + (int64_t)g * kHeadDim);
  const int64_t row_bytes = p.cache_row_stride * 2;
  const char* zero = reinterpret_cast<const char*>(kZeroRow);

  // Tile t of the wave -> stage st.  Instruction j moves rows 4j .. 4j+3 (1 KB): lane i
  // fills slot i % 16 of row 4j + i / 16, so it loads that row's chunk
  // (i % 16) ^ swizzle(row).  A tile lies inside one page (page_size % T == 0).
  auto dma_tile = [&](int t, int st) __attribute__((always_inline)) {
    const int kt = wkb + t * kTileKeys;
    const int pg = kt / p.page_size;
    const int blk = __builtin_amdgcn_readlane(blk_reg, pg - first_page);
    const bool blk_ok = blk >= 0 && blk < p.num_blocks;
    const int64_t row0 = (int64_t)blk * p.page_size + (kt - pg * p.page_size);
    uint8_t* kdst = wbuf + st * kStageBytes;
    uint8_t* vdst = kdst + kTileBytes;
#pragma unroll
    for (int j = 0; j < T / 4; ++j) {
      const int r = 4 * j + (lane >> 4);
      const bool ok = blk_ok && kt + r < wke;
      const int kc = (lane & 15) ^ swz_k(r);
      const int vc = (lane & 15) ^ swz_v(r);
      const char* ks = ok ? kbase + (row0 + r) * row_bytes + kc * 16 : zero + kc * 16;
      const char* vs = ok ? vbase + (row0 + r) * row_bytes + vc * 16 : zero + vc * 16;
      dma16_addr<NT>(ks, lds_u32(kdst + j * 1024));
      dma16_addr<NT>(vs, lds_u32(vdst + j * 1024));
    }
  };

  // V^T operand offsets (ds_read_b64_tr_b16): in 16-lane group q4, lane 4f + r reads
  // dims 16 mb + 4r .. +4 of row 4 q4 + f (+16 for the second read); the transpose
  // hands lane j of the group dim 16 mb + j of those 4 rows.
  const int vf = (lane & 15) >> 2, vr = lane & 3;
  auto voff = [&](int mb, int second) __attribute__((always_inline)) {
    const int row = 4 * q4 + vf + 16 * second;
    const int chunk = 2 * mb + (vr >> 1);
    return row * 256 + ((chunk ^ swz_v(row)) << 4) + 8 * (vr & 1);
  };

  f32x4 o[8];
#pragma unroll
  for (int mb = 0; mb < 8; ++mb) o[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f;

#pragma unroll
  for (int u = 0; u < S - 1; ++u)
    if (u < n_tiles) dma_tile(u, u);
  int st = 0;  // stage of tile t
  for (int t = 0; t < n_tiles; ++t) {
    // Tile t + S - 1 goes into the stage tile t - 1 used (read in the previous step).
    if (t + S - 1 < n_tiles) dma_tile(t + S - 1, st == 0 ? S - 1 : st - 1);
    // Tiles issued after tile t may stay in flight; tile t has landed.
    const int ahead = min(S - 1, n_tiles - 1 - t);
    wait_tiles<kDma, S - 1>(ahead);
    const uint8_t* kb_ = wbuf + st * kStageBytes;
    st = st + 1 == S ? 0 : st + 1;
    const uint8_t* vb_ = kb_ + kTileBytes;
    const int kt = wkb + t * kTileKeys;

    // S^T for keys 16 blk + 4 q4 + i
    f32x4 sacc[kBlocks];
#pragma unroll
    for (int blk = 0; blk < kBlocks; ++blk) {
      sacc[blk] = f32x4{0.f, 0.f, 0.f, 0.f};
      const int r = 16 * blk + c;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const bf16x8 ka = *reinterpret_cast<const bf16x8*>(kb_ + r * 256 + (((4 * kk + q4) ^ swz_k(r)) << 4));
        sacc[blk] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qf[kk], sacc[blk], 0, 0, 0);
      }
    }
    float x[4 * kBlocks];
#pragma unroll
    for (int blk = 0; blk < kBlocks; ++blk)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = kt + 16 * blk + 4 * q4 + i;
        x[4 * blk + i] = key < wke ? sacc[blk][i] * p.scale_log2 : -INFINITY;
      }
    float mx = x[0];
#pragma unroll
    for (int i = 1; i < 4 * kBlocks; ++i) mx = fmaxf(mx, x[i]);
    mx = group4_max(mx);
    const float m_new = fmaxf(m_run, mx);  // finite: the tile holds at least one key of the wave
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    m_run = m_new;
    float pr[4 * kBlocks], psum = 0.0f;
#pragma unroll
    for (int i = 0; i < 4 * kBlocks; ++i) {
      pr[i] = __builtin_amdgcn_exp2f(x[i] - m_new);
      psum += pr[i];
    }
    l_run = l_run * alpha + psum;
    // P^T operand: k-element 4 blk + e is key 16 blk + 4 q4 + e, the keys the lane's
    // S^T accumulators hold; the V^T operand reads the same keys (rows 16 blk + 4 q4 + f).
    uint32_t pw[2 * kBlocks];
#pragma unroll
    for (int i = 0; i < 2 * kBlocks; ++i) pw[i] = pack_bf16x2(pr[2 * i], pr[2 * i + 1]);
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) {
      const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4*)(lds_u32(vb_) + voff(mb, 0)));
      o[mb] *= alpha;
      if constexpr (kBlocks == 2) {
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s16x4*)(lds_u32(vb_) + voff(mb, 1)));
        const u32x2v lw = __builtin_bit_cast(u32x2v, lo), hw = __builtin_bit_cast(u32x2v, hi);
        const u32x4v vw = {lw[0], lw[1], hw[0], hw[1]};
        const u32x4v pv = {pw[0], pw[1], pw[2], pw[3]};
        o[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, vw), __builtin_bit_cast(bf16x8, pv),
                                                        o[mb], 0, 0, 0);
      } else {
        const u32x2v pv = {pw[0], pw[1]};
        o[mb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(lo, __builtin_bit_cast(s16x4, pv), o[mb], 0, 0, 0);
      }
    }
  }

  // ---- merge the W waves through LDS (each wave reuses its own region) -------------
  const float l_tot = group4_sum(l_run);
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");  // this wave's DMAs and reads are done
  float* lo_ = reinterpret_cast<float*>(wbuf);                  // [kCols][kHeadDim] fp32
  float* lml = reinterpret_cast<float*>(wbuf + kCols * kHeadDim * 4);  // [kCols][2]
#pragma unroll
  for (int mb = 0; mb < 8; ++mb)
    *reinterpret_cast<f32x4*>(lo_ + c * kHeadDim + 16 * mb + 4 * q4) = o[mb];
  if (q4 == 0) {
    lml[2 * c] = m_run;
    lml[2 * c + 1] = l_tot;
  }
  __syncthreads();

  // Thread (c2, piece): column c2, dims 8 piece .. 8 piece + 7, pieces strided by W * 4.
  const int c2 = tid & 15;
  float mw[W], lw[W];
  float mmax = -INFINITY;
#pragma unroll
  for (int w = 0; w < W; ++w) {
    const float* ml = reinterpret_cast<const float*>(lds + w * kWaveLds + kCols * kHeadDim * 4);
    mw[w] = ml[2 * c2];
    lw[w] = ml[2 * c2 + 1];
    mmax = fmaxf(mmax, mw[w]);
  }
  float lsum = 0.0f;
#pragma unroll
  for (int w = 0; w < W; ++w) lsum += merge_weight(mw[w], mmax) * lw[w];
  constexpr int kPieces = W <= 4 ? 4 / W : 1;  // 8-dim pieces per thread (16 per column, 4W threads each)
  float acc[kPieces][8];
#pragma unroll
  for (int pc = 0; pc < kPieces; ++pc) {
    const int d0 = min((tid >> 4) + pc * (W * 4), 15) * 8;  // W = 8: threads past piece 15 repeat it
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[pc][i] = 0.0f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float wt = merge_weight(mw[w], mmax);
      const float* src = reinterpret_cast<const float*>(lds + w * kWaveLds) + c2 * kHeadDim + d0;
      const f32x4 a0 = *reinterpret_cast<const f32x4*>(src);
      const f32x4 a1 = *reinterpret_cast<const f32x4*>(src + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[pc][i] += wt * a0[i];
        acc[pc][4 + i] += wt * a1[i];
      }
    }
  }

  if (n_splits == 1) {
    if (c2 < p.group && (tid >> 4) < 16) {
      const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
#pragma unroll
      for (int pc = 0; pc < kPieces; ++pc) {
        const int d0 = ((tid >> 4) + pc * (W * 4)) * 8;
        const float* a = acc[pc];
        const u32x4v w = {pack_bf16x2(a[0] * inv, a[1] * inv), pack_bf16x2(a[2] * inv, a[3] * inv),
                          pack_bf16x2(a[4] * inv, a[5] * inv), pack_bf16x2(a[6] * inv, a[7] * inv)};
        *reinterpret_cast<u32x4v*>(p.out + (int64_t)b * p.out_row_stride +
                                   (int64_t)(g * p.group + c2) * kHeadDim + d0) = w;
      }
    }
    return;
  }

  // ---- several chunks: publish this chunk's (O, m, l), the last one merges ----------
  // The partials cross workgroups (and XCDs, whose L2 caches are not coherent with
  // each other) as agent-scope atomic stores and loads, which the compiler emits as
  // single sc1 accesses, coherent at agent scope.  Each thread waits until its
  // stores have completed before the barrier that precedes the ticket, so the
  // ticket order orders them.  (An agent-scope release/acquire fence would do
  // the same by writing back and invalidating the whole L2 in every workgroup.)
  // Only the group's columns are stored: [pair][split][group][kHeadDim] and
  // [pair][split][group][2].
  const int64_t pair = (int64_t)b * p.num_heads_kv + g;
  const int64_t grid_splits = gridDim.x;
  const int grp = p.group;
  if (c2 < grp && (tid >> 4) < 16) {
#pragma unroll
    for (int pc = 0; pc < kPieces; ++pc) {
      const int d0 = ((tid >> 4) + pc * (W * 4)) * 8;
      float* po = p.part_o + ((pair * grid_splits + split) * grp + c2) * kHeadDim + d0;
      st16_agent(po, f32x4{acc[pc][0], acc[pc][1], acc[pc][2], acc[pc][3]});
      st16_agent(po + 4, f32x4{acc[pc][4], acc[pc][5], acc[pc][6], acc[pc][7]});
    }
    if ((tid >> 4) == 0) st_ml_agent(p.part_ml + ((pair * grid_splits + split) * grp + c2) * 2, mmax, lsum);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partials have landed
  __syncthreads();
  if (tid == 0)
    last_flag = __hip_atomic_fetch_add(p.counters + pair, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                (unsigned)(n_splits - 1);
  __syncthreads();
  if (!last_flag) return;

  // Online merge over the chunks, kMergeBatch chunks of loads in flight at a time;
  // thread (col, 4 dims) over the group's columns.
  constexpr int kMergeBatch = 16;
  for (int idx = tid; idx < grp * (kHeadDim / 4); idx += kThreads) {
    const int col = idx / (kHeadDim / 4);
    const int dd = (idx - col * (kHeadDim / 4)) * 4;
    float run_m = -INFINITY, run_l = 0.0f, tot[4] = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < n_splits; s0 += kMergeBatch) {
      float ms[kMergeBatch], ls[kMergeBatch];
      f32x4 a[kMergeBatch];
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u) {
        const int sx = min(s0 + u, n_splits - 1);  // clamped: extra slots get weight 0 below
        a[u] = ld16_agent(p.part_o + ((pair * grid_splits + sx) * grp + col) * kHeadDim + dd);
        const float2 ml = ld_ml_agent(p.part_ml + ((pair * grid_splits + sx) * grp + col) * 2);
        ms[u] = ml.x;
        ls[u] = ml.y;
      }
      static_assert(kMergeBatch == 16, "one wait covers the batch");
      asm volatile("s_waitcnt vmcnt(0)"
                   : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]), "+v"(a[5]), "+v"(a[6]),
                     "+v"(a[7]), "+v"(a[8]), "+v"(a[9]), "+v"(a[10]), "+v"(a[11]), "+v"(a[12]), "+v"(a[13]),
                     "+v"(a[14]), "+v"(a[15])
                   :
                   : "memory");
      float bm = run_m;
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u)
        if (s0 + u < n_splits) bm = fmaxf(bm, ms[u]);
      const float rescale = merge_weight(run_m, bm);
      run_l *= rescale;
#pragma unroll
      for (int i = 0; i < 4; ++i) tot[i] *= rescale;
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u) {
        const float wt = s0 + u < n_splits ? merge_weight(ms[u], bm) : 0.0f;
        run_l += wt * ls[u];
#pragma unroll
        for (int i = 0; i < 4; ++i) tot[i] += wt * a[u][i];
      }
      run_m = bm;
    }
    const float inv = run_l > 0.0f ? 1.0f / run_l : 0.0f;
    const u32x2v w = {pack_bf16x2(tot[0] * inv, tot[1] * inv), pack_bf16x2(tot[2] * inv, tot[3] * inv)};
    *reinterpret_cast<u32x2v*>(p.out + (int64_t)b * p.out_row_stride + (int64_t)(g * grp + col) * kHeadDim + dd) = w;
  }
  if (tid == 0) __hip_atomic_store(p.counters + pair, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // next call
}

}  // namespace
}  // namespace decode
}  // namespace vlc

using vlc::decode::kCols;
using vlc::decode::kHeadDim;
using vlc::decode::kMaxPagesPerWave;
using vlc::decode::kMinTileKeys;
using vlc::decode::kWgKeys;
using vlc::decode::pipeline_code;

namespace {
int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }
// Workspace layout: counters [B*Hkv] u32 | part_ml [B*Hkv][splits][kCols][2] f32 |
// part_o [B*Hkv][splits][kCols][kHeadDim] f32.
void ws_layout(int batch, int num_heads_kv, int grid_splits, int64_t* off_ml, int64_t* off_o, int64_t* total) {
  const int64_t pairs = (int64_t)batch * num_heads_kv;
  *off_ml = align256(pairs * 4);
  *off_o = *off_ml + align256(pairs * grid_splits * kCols * 2 * 4);
  *total = *off_o + pairs * grid_splits * kCols * kHeadDim * 4;
}
// Kernel shapes the library has: pipeline code -> (waves, stages, tile keys).
struct Shape {
  int code, waves, stages, tile;
};
constexpr Shape kShapes[] = {
    {pipeline_code(4, 2, 32), 4, 2, 32}, {pipeline_code(2, 2, 32), 2, 2, 32}, {pipeline_code(2, 3, 32), 2, 3, 32},
    {pipeline_code(2, 4, 32), 2, 4, 32}, {pipeline_code(1, 4, 32), 1, 4, 32}, {pipeline_code(4, 2, 16), 4, 2, 16},
    {pipeline_code(4, 4, 16), 4, 4, 16}, {pipeline_code(8, 2, 16), 8, 2, 16}, {pipeline_code(2, 4, 16), 2, 4, 16},
};
const Shape* find_shape(int code) {
  for (const Shape& sh : kShapes)
    if (sh.code == code) return &sh;
  return nullptr;
}
// Workgroups that fit one CU (160 KB of LDS).
int wgs_per_cu(const Shape& sh) { return std::max(1, 160 * 1024 / (sh.waves * sh.stages * sh.tile * 512)); }
}  // namespace

VLC_API int vlc_decode_attn_plan(int batch, int num_heads_q, int num_heads_kv, int head_dim, int page_size,
                                 int max_seqlen_k, int num_cus, int num_splits, int pipeline,
                                 int32_t* key_chunk, int32_t* grid_splits, int32_t* pipeline_out,
                                 int64_t* workspace_bytes) {
  if (!key_chunk || !grid_splits || !pipeline_out || !workspace_bytes) return VLC_ERR_INVALID;
  if (batch < 0 || num_heads_kv <= 0 || num_heads_q <= 0 || num_heads_q % num_heads_kv != 0 ||
      max_seqlen_k < 0 || page_size <= 0)
    return VLC_ERR_INVALID;
  if (head_dim != kHeadDim || num_heads_q / num_heads_kv > kCols || page_size % kMinTileKeys != 0)
    return VLC_ERR_UNSUPPORTED;
  if (pipeline == 0) pipeline = page_size % 32 == 0 ? pipeline_code(4, 2, 32) : pipeline_code(4, 2, 16);
  const Shape* sh = find_shape(pipeline);
  if (!sh) return VLC_ERR_UNSUPPORTED;
  if (page_size % sh->tile != 0) return VLC_ERR_UNSUPPORTED;
  const int waves = sh->waves;
  if (num_cus <= 0) num_cus = 256;
  const int64_t pairs = std::max<int64_t>(1, (int64_t)batch * num_heads_kv);
  int splits = num_splits;
  if (splits <= 0) {
    // One wave of workgroups over the CUs, at most 32 chunks to merge per pair.
    const int64_t slots = (int64_t)num_cus * wgs_per_cu(*sh);
    splits = (int)std::max<int64_t>(1, std::min<int64_t>(32, slots / pairs));
  }
  int64_t chunk = ((int64_t)std::max(1, max_seqlen_k) + splits - 1) / splits;
  chunk = (chunk + kWgKeys - 1) / kWgKeys * kWgKeys;
  // A wave's share of the chunk must fit the block ids it keeps in a register.
  const int64_t max_chunk = (int64_t)waves * (kMaxPagesPerWave - 1) * page_size;
  if (chunk > max_chunk) chunk = max_chunk / kWgKeys * kWgKeys;
  if (chunk <= 0 || chunk > (1 << 30)) return VLC_ERR_UNSUPPORTED;
  const int64_t gs = std::max<int64_t>(1, ((int64_t)max_seqlen_k + chunk - 1) / chunk);
  if (gs > 65535) return VLC_ERR_UNSUPPORTED;
  int64_t off_ml, off_o, total;
  ws_layout(batch, num_heads_kv, (int)gs, &off_ml, &off_o, &total);
  *key_chunk = (int32_t)chunk;
  *grid_splits = (int32_t)gs;
  *pipeline_out = pipeline;
  *workspace_bytes = total;
  return VLC_OK;
}

namespace {
// ---- fixed scratch of vlc_decode_attn_noalloc ------------------------------------
// The ticket counters and split partials of an allocation-free call live in this
// file-scope device array; every device the library runs on holds its own copy
// until the process ends.  In host code `scratch` names a host-side stand-in, not
// a device address: host code uses only the address hipGetSymbolAddress returns
// for the current device (g_scratch_addr), never the array's name.
constexpr int64_t kScratchBytes = VLC_DECODE_NOALLOC_MAX_BYTES;
// The counters sit at the front of the layout ([B * Hkv] words); this much is
// cleared once per device.  A call whose partials fit the scratch has fewer than
// kScratchBytes / 16644 < 1024 pairs, so its counters fit in the first 4 KiB.
constexpr int64_t kScratchClearBytes = int64_t(64) << 10;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
std::mutex g_scratch_mutex;
void* g_scratch_addr[kMaxDevices] = {};

__global__ void clear_words_kernel(uint32_t* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// Address of the current device's scratch.  The first call on a device looks it
// up (with that device current) and enqueues, on `st`, a kernel that zeroes the
// counter area (a kernel rather than hipMemsetAsync, so a caller may capture it in
// a HIP graph; the loader also zero-fills the array, which is uninitialised device
// data).  Later calls return the cached address.
int scratch_address(hipStream_t st, void** addr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (dev < 0 || dev >= kMaxDevices) return VLC_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_addr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return static_cast<int>(e);
    if (!p) return VLC_ERR_INVALID;
    const int64_t words = kScratchClearBytes / 4;
    hipLaunchKernelGGL(clear_words_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, st,
                       static_cast<uint32_t*>(p), words);
    const int ls = vlc::launch_status();
    if (ls != VLC_OK) return ls;
    g_scratch_addr[dev] = p;
  }
  *addr = g_scratch_addr[dev];
  return VLC_OK;
}

// Shared body of vlc_decode_attn and vlc_decode_attn_noalloc.  use_scratch: the
// workspace is the device's fixed scratch (workspace/workspace_bytes ignored).
int decode_attn_run(const void* q, int64_t q_row_stride, const void* k_cache, const void* v_cache,
                    int64_t cache_row_stride, int page_size, int64_t num_blocks,
                    const int32_t* block_table, int64_t bt_row_stride, int bt_cols,
                    const int32_t* cache_seqlens, int batch, int num_heads_q, int num_heads_kv,
                    int head_dim, float softmax_scale, int key_chunk, int grid_splits, int pipeline,
                    void* out, int64_t out_row_stride, void* workspace, int64_t workspace_bytes,
                    bool use_scratch, void* stream) {
  using namespace vlc;
  if (batch < 0 || num_heads_kv <= 0 || num_heads_q <= 0 || num_heads_q % num_heads_kv != 0)
    return VLC_ERR_INVALID;
  if (head_dim != kHeadDim || num_heads_q / num_heads_kv > kCols || page_size <= 0)
    return VLC_ERR_UNSUPPORTED;
  const Shape* sh = find_shape(pipeline);
  if (!sh) return VLC_ERR_INVALID;
  if (page_size % sh->tile != 0) return VLC_ERR_UNSUPPORTED;
  const int waves = sh->waves;
  if (batch == 0) return VLC_OK;
  if (batch > 65535 || num_heads_kv > 65535) return VLC_ERR_UNSUPPORTED;  // grid z / y
  if (!q || !k_cache || !v_cache || !block_table || !cache_seqlens || !out || (!workspace && !use_scratch))
    return VLC_ERR_INVALID;
  if (key_chunk <= 0 || key_chunk % kWgKeys != 0 || grid_splits <= 0 || grid_splits > 65535 || bt_cols <= 0)
    return VLC_ERR_INVALID;
  if ((int64_t)key_chunk > (int64_t)waves * (kMaxPagesPerWave - 1) * page_size) return VLC_ERR_INVALID;
  const int64_t group = num_heads_q / num_heads_kv;
  if (q_row_stride < num_heads_q * (int64_t)kHeadDim || out_row_stride < num_heads_q * (int64_t)kHeadDim ||
      cache_row_stride < num_heads_kv * (int64_t)kHeadDim || bt_row_stride < bt_cols || num_blocks <= 0)
    return VLC_ERR_INVALID;
  if (!aligned16(q) || !aligned16(out) || !aligned16(k_cache) || !aligned16(v_cache) || q_row_stride % 8 ||
      out_row_stride % 8 || cache_row_stride % 8 || (!use_scratch && !aligned16(workspace)))
    return VLC_ERR_INVALID;
  int64_t off_ml, off_o, total;
  ws_layout(batch, num_heads_kv, grid_splits, &off_ml, &off_o, &total);
  hipStream_t st = as_stream(stream);
  if (use_scratch) {
    // With one chunk per pair the kernel touches no workspace at all.
    if (grid_splits > 1 && total > kScratchBytes) return VLC_ERR_SCRATCH;
    const int s = scratch_address(st, &workspace);
    if (s != VLC_OK) return s;
  } else if (workspace_bytes < total) {
    return VLC_ERR_WORKSPACE;
  }
  decode::Params p;
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k_cache);
  p.v = static_cast<const uint16_t*>(v_cache);
  p.block_table = block_table;
  p.seqlens = cache_seqlens;
  p.out = static_cast<uint16_t*>(out);
  p.counters = static_cast<uint32_t*>(workspace);
  p.part_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) + off_ml);
  p.part_o = reinterpret_cast<float*>(static_cast<char*>(workspace) + off_o);
  p.q_row_stride = q_row_stride;
  p.out_row_stride = out_row_stride;
  p.cache_row_stride = cache_row_stride;
  p.bt_row_stride = bt_row_stride;
  p.num_blocks = num_blocks;
  p.page_size = page_size;
  p.bt_cols = bt_cols;
  p.group = (int)group;
  p.num_heads_kv = num_heads_kv;
  p.key_chunk = key_chunk;
  const int64_t cover = std::min<int64_t>((int64_t)bt_cols * page_size, (int64_t)grid_splits * key_chunk);
  p.max_keys = (int)std::min<int64_t>(cover, INT32_MAX);
  p.scale_log2 = softmax_scale * 1.4426950408889634f;
  const dim3 grid(grid_splits, num_heads_kv, batch);
  // bytes the call may read: K and V rows of every covered key of every sequence
  const bool nt = (int64_t)batch * p.max_keys * num_heads_kv * kHeadDim * 2 * 2 <= decode::kNtMaxBytes;
  switch (pipeline) {
#define VLC_DECODE_CASE(W, S, T)                                                                       \
  case pipeline_code(W, S, T):                                                                         \
    if (nt)                                                                                            \
      hipLaunchKernelGGL((decode::decode_attn_kernel<W, S, T, true>), grid, dim3(W * 64), 0, st, p);   \
    else                                                                                               \
      hipLaunchKernelGGL((decode::decode_attn_kernel<W, S, T, false>), grid, dim3(W * 64), 0, st, p);  \
    break;
    VLC_DECODE_CASE(4, 2, 32)
    VLC_DECODE_CASE(2, 2, 32)
    VLC_DECODE_CASE(2, 3, 32)
    VLC_DECODE_CASE(2, 4, 32)
    VLC_DECODE_CASE(1, 4, 32)
    VLC_DECODE_CASE(4, 2, 16)
    VLC_DECODE_CASE(4, 4, 16)
    VLC_DECODE_CASE(8, 2, 16)
    VLC_DECODE_CASE(2, 4, 16)
#undef VLC_DECODE_CASE
    default: return VLC_ERR_INVALID;
  }
  return launch_status();
}
}  // namespace

VLC_API int vlc_decode_attn(const void* q, int64_t q_row_stride, const void* k_cache, const void* v_cache,
                            int64_t cache_row_stride, int page_size, int64_t num_blocks,
                            const int32_t* block_table, int64_t bt_row_stride, int bt_cols,
                            const int32_t* cache_seqlens, int batch, int num_heads_q, int num_heads_kv,
                            int head_dim, float softmax_scale, int key_chunk, int grid_splits, int pipeline,
                            void* out, int64_t out_row_stride, void* workspace, int64_t workspace_bytes,
                            void* stream) {
  return decode_attn_run(q, q_row_stride, k_cache, v_cache, cache_row_stride, page_size, num_blocks, block_table,
                         bt_row_stride, bt_cols, cache_seqlens, batch, num_heads_q, num_heads_kv, head_dim,
                         softmax_scale, key_chunk, grid_splits, pipeline, out, out_row_stride, workspace,
                         workspace_bytes, false, stream);
}

VLC_API int vlc_decode_attn_noalloc(const void* q, int64_t q_row_stride, const void* k_cache,
                                    const void* v_cache, int64_t cache_row_stride, int page_size,
                                    int64_t num_blocks, const int32_t* block_table, int64_t bt_row_stride,
                                    int bt_cols, const int32_t* cache_seqlens, int batch, int num_heads_q,
                                    int num_heads_kv, int head_dim, float softmax_scale, int key_chunk,
                                    int grid_splits, int pipeline, void* out, int64_t out_row_stride,
                                    void* stream) {
  return decode_attn_run(q, q_row_stride, k_cache, v_cache, cache_row_stride, page_size, num_blocks, block_table,
                         bt_row_stride, bt_cols, cache_seqlens, batch, num_heads_q, num_heads_kv, head_dim,
                         softmax_scale, key_chunk, grid_splits, pipeline, out, out_row_stride, nullptr, 0, true,
                         stream);
}
