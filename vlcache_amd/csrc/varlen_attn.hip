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
constexpr int kKS = kHeadDim + 8;  // LDS row stride (bf16) of the K tile: 272 B, conflict-free b128 reads
constexpr int kVS = kTileK + 4;    // LDS row stride (bf16) of the transposed V tile: 136 B

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

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
  float* part_o;   // [slots][kCols][kHeadDim]
  float* part_ml;  // [slots][kCols][2]  (m * scale * log2e, l)
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

// Physical row (in elements of k/v row stride) of key `key` of sequence b; -1 if
// the block id is outside the cache.
__device__ __forceinline__ int64_t key_row(const Params& p, int b, int k0, int key) {
  if (!p.block_table) return (int64_t)k0 + key;
  const int pg = key / p.page_size;
  const int32_t blk = p.block_table[(int64_t)b * p.bt_row_stride + pg];
  if (blk < 0 || blk >= p.num_blocks) return -1;
  return (int64_t)blk * p.page_size + (key - pg * p.page_size);
}

__global__ __launch_bounds__(kThreads, 2) void attn_fwd_kernel(const Params p) {
  __shared__ __attribute__((aligned(16))) uint16_t k_lds[kTileK * kKS];
  __shared__ __attribute__((aligned(16))) uint16_t vt_lds[kHeadDim * kVS];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int lc = lane & 31;
  const int hf = lane >> 5;

  const int32_t* it = p.items + (int64_t)blockIdx.x * kItemInts;
  const int b = it[0], g = it[1], q_start = it[2], q_count = it[3];
  const int k_begin = it[4], k_end = it[5], slot = it[6];
  const int q0 = p.cu_q[b];
  const int sq = p.cu_q[b + 1] - q0;
  const int k0 = p.cu_k[b];
  const int sk = p.cu_k[b + 1] - k0;

  const int col = wave * 32 + lc;
  const int pos = col / p.group;
  const int hh = col - pos * p.group;
  const bool valid = pos < q_count;
  const int qpos = q_start + pos;
  const int head = g * p.group + hh;
  const int limit = p.causal ? qpos + sk - sq : sk - 1;               // last visible key
  const int blk_min_limit = p.causal ? q_start + sk - sq : sk - 1;    // smallest limit in the block

  // Q^T fragment (B operand of S^T = K Q^T): lane holds Q[col][16*kk + 8*hf .. +8].
  bf16x8 qf[8];
  {
    const uint16_t* qrow = p.q + (int64_t)(q0 + (valid ? qpos : 0)) * p.q_row_stride +
                           (int64_t)head * kHeadDim + 8 * hf;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      u32x4v w = {0u, 0u, 0u, 0u};
      if (valid) w = *reinterpret_cast<const u32x4v*>(qrow + 16 * kk);
      qf[kk] = __builtin_bit_cast(bf16x8, w);
    }
  }

  f32x16 o[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[mb][e] = 0.f;
  float m = -INFINITY;
  float l = 0.f;

  const bool one_page_tiles = p.block_table && (p.page_size % kTileK == 0);

  for (int kt = k_begin; kt < k_end; kt += kTileK) {
    __syncthreads();  // the previous tile is fully consumed
    // ---- stage K (row-major) and V (transposed) into LDS; keys >= sk read as zeros ----
    int64_t tile_row0 = 0;
    bool tile_ok = true;
    if (one_page_tiles) {
      const int pg = kt / p.page_size;
      const int32_t blk = p.block_table[(int64_t)b * p.bt_row_stride + pg];
      tile_ok = blk >= 0 && blk < p.num_blocks;
      tile_row0 = (int64_t)blk * p.page_size + (kt - pg * p.page_size);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int id = r * kThreads + tid;
      const int row = id >> 4;
      const int dc = id & 15;
      const int key = kt + row;
      u32x4v w = {0u, 0u, 0u, 0u};
      if (key < sk) {
        int64_t prow;
        if (one_page_tiles) prow = tile_ok ? tile_row0 + row : -1;
        else prow = key_row(p, b, k0, key);
        if (prow >= 0)
          w = *reinterpret_cast<const u32x4v*>(p.k + prow * p.k_row_stride + (int64_t)g * kHeadDim + dc * 8);
      }
      *reinterpret_cast<u32x4v*>(k_lds + row * kKS + dc * 8) = w;
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int id = r * kThreads + tid;
      const int kp = id >> 4;  // key pair 0..31
      const int dc = id & 15;
      u32x4v va = {0u, 0u, 0u, 0u}, vb = {0u, 0u, 0u, 0u};
      const int key = kt + 2 * kp;
      if (key < sk) {
        int64_t prow;
        if (one_page_tiles) prow = tile_ok ? tile_row0 + 2 * kp : -1;
        else prow = key_row(p, b, k0, key);
        if (prow >= 0)
          va = *reinterpret_cast<const u32x4v*>(p.v + prow * p.v_row_stride + (int64_t)g * kHeadDim + dc * 8);
      }
      if (key + 1 < sk) {
        int64_t prow;
        if (one_page_tiles) prow = tile_ok ? tile_row0 + 2 * kp + 1 : -1;
        else prow = key_row(p, b, k0, key + 1);
        if (prow >= 0)
          vb = *reinterpret_cast<const u32x4v*>(p.v + prow * p.v_row_stride + (int64_t)g * kHeadDim + dc * 8);
      }
      uint32_t* vt32 = reinterpret_cast<uint32_t*>(vt_lds);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t a = va[e], c = vb[e];
        // d = dc*8 + 2e holds the low halves, d + 1 the high halves.
        vt32[((dc * 8 + 2 * e) * kVS + 2 * kp) >> 1] = (a & 0xffffu) | (c << 16);
        vt32[((dc * 8 + 2 * e + 1) * kVS + 2 * kp) >> 1] = (a >> 16) | (c & 0xffff0000u);
      }
    }
    __syncthreads();

    // ---- S^T = K Q^T for two 32-key blocks ----
    f32x16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int e = 0; e < 16; ++e) s[kb][e] = 0.f;
      const uint16_t* kr = k_lds + (kb * 32 + lc) * kKS + 8 * hf;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(kr + 16 * kk);
        s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[kk], s[kb], 0, 0, 0);
      }
    }

    // ---- mask: element e = 4i + j of block kb is key kt + 32kb + 8i + 4hf + j ----
    const bool need_mask = (kt + kTileK - 1 > blk_min_limit) || (kt + kTileK > k_end);
    if (need_mask) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int key = kt + kb * 32 + 8 * (e >> 2) + 4 * hf + (e & 3);
          if (key > limit || key >= k_end) s[kb][e] = -INFINITY;
        }
    }

    // ---- online softmax (per lane = per column; the two half-waves share the max) ----
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[kb][e]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m, mx);
    const float m_base = (m_new == -INFINITY) ? 0.f : m_new * p.scale_log2;
    const float alpha = fast_exp2(m * p.scale_log2 - m_base);
    float rs = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float pe = fast_exp2(__builtin_fmaf(s[kb][e], p.scale_log2, -m_base));
        s[kb][e] = pe;
        rs += pe;
      }
    l = l * alpha + rs;
    m = m_new;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[mb][e] *= alpha;

    // ---- P^T as bf16 B operands: chunk c of block kb = elements 8c..8c+7 ----
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

    // ---- O^T += V^T P^T: lane supplies V^T[d][keys 16c+4hf+0..3, 16c+8+4hf+0..3] ----
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      const uint16_t* vr = vt_lds + (mb * 32 + lc) * kVS + 4 * hf;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const int base = kb * 32 + 16 * c;
          const u32x2v lo = *reinterpret_cast<const u32x2v*>(vr + base);
          const u32x2v hi = *reinterpret_cast<const u32x2v*>(vr + base + 8);
          const u32x4v w = {lo[0], lo[1], hi[0], hi[1]};
          o[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, w), pk[kb][c],
                                                          o[mb], 0, 0, 0);
        }
    }
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
    float* po = p.part_o + ((int64_t)slot * kCols + col) * kHeadDim;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = 32 * mb + 8 * i + 4 * hf;
        float4 w = make_float4(o[mb][4 * i], o[mb][4 * i + 1], o[mb][4 * i + 2], o[mb][4 * i + 3]);
        *reinterpret_cast<float4*>(po + d) = w;
      }
    if (hf == 0) {
      float* ml = p.part_ml + ((int64_t)slot * kCols + col) * 2;
      ml[0] = (m == -INFINITY) ? -INFINITY : m * p.scale_log2;
      ml[1] = l_tot;
    }
  }
}

// Merge the split-KV partials of one query tile:
//   O = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s,  M = max_s m_s.
__global__ __launch_bounds__(kThreads) void attn_combine_kernel(const Params p) {
  const int32_t* it = p.combine + (int64_t)blockIdx.x * kItemInts;
  const int b = it[0], g = it[1], q_start = it[2], q_count = it[3];
  const int first = it[4], nsplit = it[5];
  const int q0 = p.cu_q[b];
  for (int u = threadIdx.x; u < kCols * (kHeadDim / 4); u += kThreads) {
    const int col = u / (kHeadDim / 4);
    const int d = 4 * (u - col * (kHeadDim / 4));
    const int pos = col / p.group;
    if (pos >= q_count) continue;
    const int hh = col - pos * p.group;
    float mmax = -INFINITY;
    for (int s = 0; s < nsplit; ++s)
      mmax = fmaxf(mmax, p.part_ml[((int64_t)(first + s) * kCols + col) * 2]);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    float lsum = 0.f;
    if (mmax != -INFINITY) {
      for (int s = 0; s < nsplit; ++s) {
        const float* ml = p.part_ml + ((int64_t)(first + s) * kCols + col) * 2;
        const float w = fast_exp2(ml[0] - mmax);
        lsum += w * ml[1];
        const float4 v = *reinterpret_cast<const float4*>(
            p.part_o + ((int64_t)(first + s) * kCols + col) * kHeadDim + d);
        acc.x += w * v.x; acc.y += w * v.y; acc.z += w * v.z; acc.w += w * v.w;
      }
    }
    const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
    uint16_t* orow = p.out + (int64_t)(q0 + q_start + pos) * p.out_row_stride +
                     (int64_t)(g * p.group + hh) * kHeadDim + d;
    u32x2v w;
    w[0] = pack_bf16x2(acc.x * inv, acc.y * inv);
    w[1] = pack_bf16x2(acc.z * inv, acc.w * inv);
    *reinterpret_cast<u32x2v*>(orow) = w;
  }
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
  if (!q || !k || !v || !out || !cu_seqlens_q || !cu_seqlens_k) return VLC_ERR_INVALID;
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
  prm.part_o = static_cast<float*>(workspace);
  prm.part_ml = n_slots > 0 ? reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                                        n_slots * (int64_t)kCols * kHeadDim * 4)
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
  hipLaunchKernelGGL(attn_fwd_kernel, dim3((unsigned)n_items), dim3(kThreads), 0, s, prm);
  int st = launch_status();
  if (st != VLC_OK) return st;
  if (n_comb > 0) {
    hipLaunchKernelGGL(attn_combine_kernel, dim3((unsigned)n_comb), dim3(kThreads), 0, s, prm);
    st = launch_status();
  }
  return st;
}
