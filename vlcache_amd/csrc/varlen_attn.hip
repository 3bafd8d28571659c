// Varlen paged GQA attention (prefill) for gfx950: the replacement of
// flash_attn_varlen_func(q, k, v, ..., causal=True, block_table) as called at
// layers/attention.py:67-70.
//
// Work decomposition (built on the host by vlc_attn_plan): a workgroup of four
// wave64s owns one work item = (sequence, kv head, tile of query positions,
// key range).  Its 128 "columns" are (query position, q head) pairs: the
// `group` q heads that share the kv head are packed side by side, so one K/V
// tile staged in LDS feeds every head of the group.
//
// Per 64-key tile each wave computes S^T = K * Q^T (keys x its 32 columns) with
// v_mfma_f32_32x32x16_bf16.  In that orientation a lane owns ONE column and 16
// keys of each 32-key block, so the softmax row reductions are lane-local plus
// a single exchange between the two half-waves.  The probabilities P^T are
// already in the B-operand layout of the second product O^T += V^T P^T, so they
// never leave registers; V is transposed into LDS when it is staged.
//
// Online softmax in fp32 with exp2 (the softmax scale and log2(e) are folded
// into one multiply-add), P rounded to bf16 for the PV product, O accumulated
// in fp32 and normalised once at the end.  Items whose key range was split
// write unnormalised O with (m, l) to a workspace slot; attn_combine merges
// the slots of a query tile.
#include "attn_plan.h"
#include "common.h"

namespace vlc {
namespace attn {
namespace {

constexpr int kThreads = 256;

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
  float scale_log2;
};

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }


typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Round two fp32 to bf16 (nearest even) with the hardware pack conversion.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2 v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// Physical row of key `key` of sequence b through the block table, or -1 when the
// key is past the sequence or its block id is outside the cache.
__device__ __forceinline__ int64_t paged_row_of(const Params& p, int b, int sk, int key) {
  const int kc = min(key, sk - 1);
  const int pg = kc / p.page_size;
  const int32_t blk = p.block_table[(int64_t)b * p.bt_row_stride + pg];
  const bool ok = key < sk && blk >= 0 && blk < p.num_blocks;
  return ok ? (int64_t)blk * p.page_size + (kc - pg * p.page_size) : -1;
}

// How keys map to rows of k/v.
enum KvMode {
  kContiguous = 0,  // key j of sequence b is row cu_k[b] + j
  kPagedTiles = 1,  // paged, page_size % 64 == 0: a 64-key tile lies inside one page
  kPagedRows = 2,   // paged, any page size: one block-table lookup per row
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

template <int MODE>
__global__ __launch_bounds__(kThreads, 2) void attn_fwd_kernel(const Params p) {
  // Two K and two V tile buffers (double buffering): 64 rows x 256 bytes each, swizzled.
  __shared__ __attribute__((aligned(1024))) uint8_t k_buf0[kTileK * 256];
  __shared__ __attribute__((aligned(1024))) uint8_t k_buf1[kTileK * 256];
  __shared__ __attribute__((aligned(1024))) uint8_t v_buf0[kTileK * 256];
  __shared__ __attribute__((aligned(1024))) uint8_t v_buf1[kTileK * 256];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int lc = lane & 31;
  const int hf = lane >> 5;

  const int32_t* it = p.items + (int64_t)blockIdx.x * kItemInts;
  const int b = it[0], g = it[1], q_start = it[2], q_count = it[3];
  const int k_begin = it[4], k_end = it[5], slot = it[6];
  const int q0 = it[7], sq = it[8], k0 = it[9], sk = it[10];

  const int col = wave * 32 + lc;
  const int pos = col / p.group;
  const int hh = col - pos * p.group;
  const bool valid = pos < q_count;
  const int qpos = q_start + pos;
  const int head = g * p.group + hh;
  const int limit = p.causal ? qpos + sk - sq : sk - 1;             // last visible key
  const int blk_min_limit = p.causal ? q_start + sk - sq : sk - 1;  // smallest limit in the block

  // Q^T fragment (B operand of S^T = K Q^T): lane holds Q[col][16*kk + 8*hf .. +8].
  // Invalid columns load row 0 (always readable) and are zeroed.
  bf16x8 qf[8];
  {
    const uint16_t* qrow = p.q + (valid ? (int64_t)(q0 + qpos) * p.q_row_stride + (int64_t)head * kHeadDim : 0) +
                           8 * hf;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      u32x4v w = *reinterpret_cast<const u32x4v*>(qrow + 16 * kk);
      if (!valid) w = u32x4v{0u, 0u, 0u, 0u};
      qf[kk] = __builtin_bit_cast(bf16x8, w);
    }
  }

  // ---- LDS read offsets (bytes, within a tile buffer) ---------------------------
  // K operand of S^T: row kb*32 + lc, chunk 2kk + hf.
  uint32_t koff[8];
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) koff[kk] = lc * 256 + (((2 * kk + hf) ^ swz(lc)) << 4);
  // V^T operand through ds_read_b64_tr_b16: in each 16-lane group, lane 4f + r reads
  // dims 4r..4r+3 (of the group's 16-dim half) of key row f, and the transpose
  // hands lane j the 4 keys of dim j.  Group bit 0 = dim half, bit 1 = key half
  // (+4 keys); the second read of an operand is 8 keys further.
  uint32_t voff[4][2];
  {
    const int s = lane & 15, grp = lane >> 4;
    const int y = 2 * (grp & 1) + ((s & 3) >> 1);
#pragma unroll
    for (int rd = 0; rd < 2; ++rd) {
      const int row = 4 * (grp >> 1) + (s >> 2) + 8 * rd;  // + kb*32 + 16c (multiple of 16)
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
        voff[mb][rd] = row * 256 + (((4 * mb + y) ^ swz(row)) << 4) + ((s & 1) << 3);
    }
  }

  // ---- K/V tile loads straight into LDS (global_load_lds_dwordx4) --------------
  // Wave w fills rows 16w .. 16w+15 of both tiles, 4 rows per instruction: lane i
  // writes LDS slot i%16 of row 16w + 4j + i/16, so it loads that row's chunk
  // (i%16) ^ swz(row).
  const char* kcol = reinterpret_cast<const char*>(p.k + (int64_t)g * kHeadDim);
  const char* vcol = reinterpret_cast<const char*>(p.v + (int64_t)g * kHeadDim);
  const int64_t kst = p.k_row_stride * 2, vst = p.v_row_stride * 2;  // bytes
  // Row 16w + 4j + (lane >> 4) of the tile, chunk (lane & 15) ^ swz(4j + (lane >> 4))
  // = ((lane & 15) ^ ((lane >> 4) << 2)) ^ j: both recomputed per load from one value.
  const int lrow0 = 16 * wave + (lane >> 4);
  const uint32_t lchunk0 = (uint32_t)((lane & 15) ^ ((lane >> 4) << 2));
  const char* zero = reinterpret_cast<const char*>(kZeroRow);

  auto issue_loads = [&](int kt, uint8_t* kdst, uint8_t* vdst) {
    // Physical row of the tile's first key (kContiguous / kPagedTiles) and validity.
    int64_t row0 = 0;
    bool ok = true;
    if (MODE == kContiguous) {
      row0 = (int64_t)k0 + kt;
    } else if (MODE == kPagedTiles) {
      const int pg = kt / p.page_size;
      const int32_t blk = p.block_table[(int64_t)b * p.bt_row_stride + pg];  // uniform: scalar load
      ok = blk >= 0 && blk < p.num_blocks;
      row0 = (int64_t)blk * p.page_size + (kt - pg * p.page_size);
    }
    const bool full = ok && kt + kTileK <= sk;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int lrow_j = lrow0 + 4 * j;
      const uint32_t lchunk_j = (lchunk0 ^ (uint32_t)j) << 4;
      const char* ks;
      const char* vs;
      if (MODE == kPagedRows) {
        const int64_t pr = paged_row_of(p, b, sk, kt + lrow_j);
        ks = pr >= 0 ? kcol + pr * kst + lchunk_j : zero + lchunk_j;
        vs = pr >= 0 ? vcol + pr * vst + lchunk_j : zero + lchunk_j;
      } else if (full) {
        ks = kcol + (row0 + lrow_j) * kst + lchunk_j;
        vs = vcol + (row0 + lrow_j) * vst + lchunk_j;
      } else {
        const bool rv = ok && kt + lrow_j < sk;
        ks = rv ? kcol + (row0 + lrow_j) * kst + lchunk_j : zero + lchunk_j;
        vs = rv ? vcol + (row0 + lrow_j) * vst + lchunk_j : zero + lchunk_j;
      }
      const int lds_row = 16 * wave + 4 * j;
      __builtin_amdgcn_global_load_lds(ks, (lds_void*)(kdst + lds_row * 256), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(vs, (lds_void*)(vdst + lds_row * 256), 16, 0, 0);
    }
  };

  f32x16 o[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[mb][e] = 0.f;
  float mb_run = -INFINITY;  // running max, already scaled to log2 units
  float l = 0.f;

  // ---- one 64-key tile from LDS: S^T, mask, online softmax, O^T += V^T P^T ----
  auto compute = [&](int kt, const uint8_t* kb_lds, const uint8_t* vb_lds) {
    f32x16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; ++e) s[kb][e] = 0.f;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(kb_lds + kb * 32 * 256 + koff[kk]);
        s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[kk], s[kb], 0, 0, 0);
      }
    }
    // mask: element e = 4i + j of block kb is key kt + 32kb + 8i + 4hf + j
    if ((kt + kTileK - 1 > blk_min_limit) || (kt + kTileK > k_end)) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int key = kt + kb * 32 + 8 * (e >> 2) + 4 * hf + (e & 3);
          if (key > limit || key >= k_end) s[kb][e] = -INFINITY;
        }
    }
    // online softmax (lane = column; the two half-waves share the max)
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[kb][e]);
    mx = fmaxf(mx, __shfl_xor(mx, 32)) * p.scale_log2;
    const bool grow = mx > mb_run + kRescaleThreshold;
    if (__builtin_amdgcn_ballot_w64(grow)) {  // rare after the first tile
      const float mb_new = grow ? mx : mb_run;
      const float alpha = grow ? fast_exp2(mb_run - mb_new) : 1.f;  // first growth: 2^-inf = 0
      mb_run = mb_new;
      l *= alpha;
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[mb][e] *= alpha;
    }
    const float m_base = (mb_run == -INFINITY) ? 0.f : mb_run;
    float rs = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float pe = fast_exp2(__builtin_fmaf(s[kb][e], p.scale_log2, -m_base));
        s[kb][e] = pe;
        rs += pe;
      }
    l += rs;
    // P^T as bf16 B operands: chunk c of block kb = elements 8c..8c+7
    bf16x8 pk[2][2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        u32x4v w;
#pragma unroll
        for (int t = 0; t < 4; ++t) w[t] = pack_bf16x2(s[kb][8 * c + 2 * t], s[kb][8 * c + 2 * t + 1]);
        pk[kb][c] = __builtin_bit_cast(bf16x8, w);
      }
    // O^T += V^T P^T
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
          const uint8_t* vr = vb_lds + (kb * 32 + 16 * c) * 256;
          const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) s16x4*)(vr + voff[mb][0]));
          const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) s16x4*)(vr + voff[mb][1]));
          const s16x8 w = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          o[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, w), pk[kb][c],
                                                          o[mb], 0, 0, 0);
        }
  };

  // ---- main loop: two tiles per iteration so each buffer is a static array ----
  // Order per tile: wait for this wave's loads of the tile, barrier (all loads of the
  // tile landed; every wave is done with the other buffer), start the next tile's
  // loads into the other buffer, compute.
  if (k_begin < k_end) issue_loads(k_begin, k_buf0, v_buf0);
  for (int kt = k_begin; kt < k_end; kt += 2 * kTileK) {
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
    __syncthreads();
    if (kt + kTileK < k_end) issue_loads(kt + kTileK, k_buf1, v_buf1);
    compute(kt, k_buf0, v_buf0);
    if (kt + kTileK >= k_end) break;
    __builtin_amdgcn_s_waitcnt(0x0f70);
    __syncthreads();
    if (kt + 2 * kTileK < k_end) issue_loads(kt + 2 * kTileK, k_buf0, v_buf0);
    compute(kt + kTileK, k_buf1, v_buf1);
  }

  // ---- epilogue: lane holds O^T[d = 32mb + 8i + 4hf + j][col] in o[mb][4i + j] ----
  const float l_tot = l + __shfl_xor(l, 32);
  if (!valid) return;
  if (slot < 0) {
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    uint16_t* orow = p.out + (int64_t)(q0 + qpos) * p.out_row_stride + (int64_t)head * kHeadDim;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = 32 * mb + 8 * i + 4 * hf;
        u32x2v w;
        w[0] = pack_bf16x2(o[mb][4 * i] * inv, o[mb][4 * i + 1] * inv);
        w[1] = pack_bf16x2(o[mb][4 * i + 2] * inv, o[mb][4 * i + 3] * inv);
        *reinterpret_cast<u32x2v*>(orow + d) = w;
      }
  } else {
    // Split of a longer key range: the normalised partial in bf16 plus (m, l) in fp32.
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    uint16_t* po = p.part_o + ((int64_t)slot * kCols + col) * kHeadDim;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = 32 * mb + 8 * i + 4 * hf;
        u32x2v w;
        w[0] = pack_bf16x2(o[mb][4 * i] * inv, o[mb][4 * i + 1] * inv);
        w[1] = pack_bf16x2(o[mb][4 * i + 2] * inv, o[mb][4 * i + 3] * inv);
        *reinterpret_cast<u32x2v*>(po + d) = w;
      }
    if (hf == 0) {
      float* ml = p.part_ml + ((int64_t)slot * kCols + col) * 2;
      ml[0] = mb_run;
      ml[1] = l_tot;
    }
  }
}

// Merge the split-KV partials of one query tile:
//   O = sum_s 2^(m_s - M) l_s Ohat_s / sum_s 2^(m_s - M) l_s,  M = max_s m_s,
// with Ohat_s = O_s / l_s stored in bf16.  grid = (combine items, kCols /
// kCombineCols): a workgroup owns kCombineCols columns and each lane one 8-dim
// (16-byte) slice of a column, so the loads of the split loop are independent.
constexpr int kCombineCols = kThreads / (kHeadDim / 8);  // 16 columns per workgroup

__global__ __launch_bounds__(kThreads) void attn_combine_kernel(const Params p) {
  const int32_t* it = p.combine + (int64_t)blockIdx.x * kItemInts;
  const int g = it[1], q_start = it[2], q_count = it[3];
  const int first = it[4], nsplit = it[5];
  const int q0 = it[7];
  const int col = blockIdx.y * kCombineCols + threadIdx.x / (kHeadDim / 8);
  const int d = 8 * (threadIdx.x % (kHeadDim / 8));
  const int pos = col / p.group;
  if (pos >= q_count) return;
  const int hh = col - pos * p.group;
  const float* ml = p.part_ml + ((int64_t)first * kCols + col) * 2;
  const uint16_t* po = p.part_o + ((int64_t)first * kCols + col) * kHeadDim + d;
  const int64_t ml_stride = (int64_t)kCols * 2;
  const int64_t po_stride = (int64_t)kCols * kHeadDim;
  float mmax = -INFINITY;
#pragma unroll 8
  for (int s = 0; s < nsplit; ++s) mmax = fmaxf(mmax, ml[s * ml_stride]);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float lsum = 0.f;
  if (mmax != -INFINITY) {
#pragma unroll 4
    for (int s = 0; s < nsplit; ++s) {
      const float2 mls = *reinterpret_cast<const float2*>(ml + s * ml_stride);
      const u32x4v v = *reinterpret_cast<const u32x4v*>(po + s * po_stride);
      const float wl = fast_exp2(mls.x - mmax) * mls.y;
      lsum += wl;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        acc[2 * t] += wl * bf16_bits_to_f32(v[t] & 0xffffu);
        acc[2 * t + 1] += wl * bf16_bits_to_f32(v[t] >> 16);
      }
    }
  }
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  uint16_t* orow = p.out + (int64_t)(q0 + q_start + pos) * p.out_row_stride +
                   (int64_t)(g * p.group + hh) * kHeadDim + d;
  u32x4v w;
#pragma unroll
  for (int t = 0; t < 4; ++t) w[t] = pack_bf16x2(acc[2 * t] * inv, acc[2 * t + 1] * inv);
  *reinterpret_cast<u32x4v*>(orow) = w;
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
  if (head_dim != kHeadDim) return VLC_ERR_UNSUPPORTED;
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
  if (!q || !k || !v || !out) return VLC_ERR_INVALID;
  if (!(softmax_scale > 0.f)) return VLC_ERR_INVALID;
  // 16-byte vector access of every row.
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out) || q_row_stride % 8 ||
      k_row_stride % 8 || v_row_stride % 8 || out_row_stride % 8)
    return VLC_ERR_INVALID;
  if (q_row_stride < (int64_t)num_heads_q * kHeadDim || out_row_stride < (int64_t)num_heads_q * kHeadDim ||
      k_row_stride < (int64_t)num_heads_kv * kHeadDim || v_row_stride < (int64_t)num_heads_kv * kHeadDim)
    return VLC_ERR_INVALID;
  if (block_table && (page_size <= 0 || bt_row_stride <= 0 || num_blocks <= 0)) return VLC_ERR_INVALID;
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
  prm.scale_log2 = softmax_scale * 1.4426950408889634f;

  hipStream_t s = as_stream(stream);
  const int mode = !block_table ? kContiguous : (page_size % kTileK == 0 ? kPagedTiles : kPagedRows);
  if (mode == kContiguous)
    hipLaunchKernelGGL(attn_fwd_kernel<kContiguous>, dim3((unsigned)n_items), dim3(kThreads), 0, s, prm);
  else if (mode == kPagedTiles)
    hipLaunchKernelGGL(attn_fwd_kernel<kPagedTiles>, dim3((unsigned)n_items), dim3(kThreads), 0, s, prm);
  else
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
