// Fused rotary embedding of the recomputed tokens with the paged KV store.
//
// Per layer the reference rotates q and k in RotaryEmbedding.forward
// (layers/rotary_embedding.py:37-48: gather (cos, sin) rows of an fp32 cache at
// the token positions, rotate-half in fp32, cast back) and then copies k and v
// into the paged cache (store_kvcache, layers/attention.py:33-40), in that order
// (models/qwen3.py:84-85).  This kernel does both in one pass over the q/k/v
// rows of the QKV projection: q heads are rotated into q_out, k heads are
// rotated and written straight to their cache slot (and, when the caller needs
// contiguous keys, to k_out), v heads are copied to their cache slot.
//
// Rotation of pair i (dims i and i + hd/2 of a head) of token n:
//   p  = positions[section(i) * position_row_stride + n]   (1-D positions: row 0)
//   c  = cos_sin_cache[p * cache_row_stride + i]
//   s  = cos_sin_cache[p * cache_row_stride + hd/2 + i]
//   y1 = x1*c - x2*s,  y2 = x2*c + x1*s
// in fp32 with every product and sum rounded (no fused multiply-add), then
// rounded to bf16 (nearest even): the same operations, in the same order, as
// the reference's eager fp32 formula, so the output is bit-identical to it.
// section(i) is Qwen2.5-VL's M-RoPE layout: 0 (t) for i < s0, 1 (h) for
// i < s0 + s1, 2 (w) otherwise, for mrope_section (s0, s1, s2).
//
// Work layout: a "unit" is 8 pairs of one head, i.e. 16 bytes of dims
// [8j, 8j+8) and the partner 16 bytes [hd/2+8j, hd/2+8j+8).  A token owns
// (Hq + Hkv [+ Hkv for v]) * hd/16 units, enumerated head by head, so the
// hd/16 lanes of a head read and write its whole 2*hd-byte row with 16-byte
// accesses.  Each lane handles kUPT units spaced by the grid, all their loads
// in flight before the first store; one unit per lane (the most workgroups)
// measured fastest for the 1247-token warm step (4.5 us against 5.1 us with two).
// The stores take the policy store_mode_for picks from the bytes the call writes: at
// agent scope (written through L2, so the attention that reads q_out and the cache
// next starts without waiting for a write-back of dirty lines) up to 64 MB,
// nontemporal up to 256 MB, plain above.  Nontemporal against plain: 1247 / 10741 /
// 32768 tokens in 3.7-3.9 / 19.5 / 54.0 us against 4.1 / 20.4 / 60 us (36 calls in one
// graph, distinct caches); nontemporal cache stores with a plain q_out store gained
// less (4.1 / 19.9 / 59 us).  Agent scope against nontemporal in the same loop: 3.76
// against 3.67 us at 1247 tokens, 6.45 against 6.71 at 4096, 59.9 against 54.9 at 32768;
// in the warm request's step, where the attention follows, 1.231 against 1.249 ms.
#include <type_traits>

#include "common.h"

namespace vlc {
namespace {

constexpr int kThreads = 256;
constexpr int kUPT = 1;  // units per thread

struct RopeArgs {
  const uint16_t* q;
  int64_t q_rs;
  uint16_t* q_out;
  int64_t qo_rs;
  const uint16_t* k;
  int64_t k_rs;
  uint16_t* k_out;  // nullable
  int64_t ko_rs;
  const uint16_t* v;  // nullable when no cache
  int64_t v_rs;
  uint16_t* k_cache;  // nullable (no store)
  uint16_t* v_cache;
  int64_t num_slots;
  const int32_t* slot_mapping;
  const int64_t* positions;
  int64_t pos_rs;  // elements between position rows (0 for 1-D)
  int sec_b1, sec_b2;  // pair bounds of sections 1 and 2
  const float* cos_sin;
  int64_t cs_rs;
  int64_t max_pos;
  int num_heads_q, num_heads_kv, head_dim;
  int uph;   // units per head = hd / 16
  int upt;   // units per token
  uint32_t total;
};

__device__ __forceinline__ void rope_word(uint32_t& a, uint32_t& b, float c0, float s0, float c1,
                                          float s1) {
#pragma clang fp contract(off)
  // a holds x1 of pairs (p, p+1) in its low/high halves, b holds x2 of the same pairs.
  const float a0 = bf16_bits_to_f32(a & 0xffffu), a1 = bf16_bits_to_f32(a >> 16);
  const float b0 = bf16_bits_to_f32(b & 0xffffu), b1 = bf16_bits_to_f32(b >> 16);
  const float y10 = a0 * c0 - b0 * s0;
  const float y20 = b0 * c0 + a0 * s0;
  const float y11 = a1 * c1 - b1 * s1;
  const float y21 = b1 * c1 + a1 * s1;
  a = f32_to_bf16_bits(y10) | (f32_to_bf16_bits(y11) << 16);
  b = f32_to_bf16_bits(y20) | (f32_to_bf16_bits(y21) << 16);
}

__device__ __forceinline__ int section_of(int pair, int b1, int b2) {
  return pair < b1 ? 0 : (pair < b2 ? 1 : 2);
}

__device__ __forceinline__ int64_t clamp_pos(int64_t p, int64_t max_pos) {
  return p < 0 ? 0 : (p >= max_pos ? max_pos - 1 : p);
}

// kPerPair = false: the 8 pairs of a unit share one position row (section
// bounds are multiples of 8) and cos/sin rows are 16-byte aligned, so a unit
// reads one position and 2 x 32 contiguous bytes of cos/sin.  kPerPair = true:
// position and cos/sin are read pair by pair (any section bounds, any alignment).
template <bool kPerPair, int kSt>
__global__ __launch_bounds__(kThreads) void rope_store_kv_kernel(const RopeArgs a) {
  const int hd = a.head_dim;
  const int half = hd >> 1;
  const int64_t row_elems = (int64_t)a.num_heads_kv * hd;  // cache row
  const uint32_t stride = gridDim.x * kThreads;
  const bool store = a.k_cache != nullptr;

  // Straight-line per unit: every independent load (position, slot, data) is
  // issued for all kUPT units before the first wait, then the cos/sin loads that
  // depend on the positions, then the rotation, then the stores.
  struct Unit {
    bool live;
    int kind;  // 0 = q, 1 = k, 2 = v
    int j;
    uint32_t n;
    int64_t off;  // element offset of dims [8j, 8j+8) inside the token row
    const uint16_t* src;
    u32x4 lo, hi;
    int64_t pos[kPerPair ? 8 : 1];
    int32_t slot;
    float c[8], s[8];
  };
  for (uint32_t u0 = blockIdx.x * kThreads + threadIdx.x; u0 < a.total; u0 += stride * kUPT) {
    Unit un[kUPT];
#pragma unroll
    for (int k = 0; k < kUPT; ++k) {
      const uint32_t u_raw = u0 + k * stride;
      Unit& x = un[k];
      x.live = u_raw < a.total;
      const uint32_t u = x.live ? u_raw : a.total - 1;  // dead lanes load in bounds, store nothing
      x.n = u / (uint32_t)a.upt;
      const int r = (int)(u - x.n * (uint32_t)a.upt);
      const int hh = r / a.uph;
      x.j = r - hh * a.uph;
      x.kind = hh < a.num_heads_q ? 0 : (hh < a.num_heads_q + a.num_heads_kv ? 1 : 2);
      const int lh = hh - (x.kind == 0 ? 0 : a.num_heads_q) - (x.kind == 2 ? a.num_heads_kv : 0);
      x.off = (int64_t)lh * hd + 8 * x.j;
      const uint16_t* src = x.kind == 0 ? a.q + (int64_t)x.n * a.q_rs
                          : (x.kind == 1 ? a.k + (int64_t)x.n * a.k_rs : a.v + (int64_t)x.n * a.v_rs);
      x.src = src + x.off;
      if (kPerPair) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
          x.pos[i] = a.positions[section_of(8 * x.j + i, a.sec_b1, a.sec_b2) * a.pos_rs + x.n];
      } else {
        x.pos[0] = a.positions[section_of(8 * x.j, a.sec_b1, a.sec_b2) * a.pos_rs + x.n];
      }
      x.slot = store ? a.slot_mapping[x.n] : -1;
    }
    // Data loads after the position loads: loads retire in order, so the wait for
    // the positions (needed by the cos/sin loads) leaves these in flight.
#pragma unroll
    for (int k = 0; k < kUPT; ++k) {
      Unit& x = un[k];
      x.lo = *reinterpret_cast<const u32x4*>(x.src);
      x.hi = *reinterpret_cast<const u32x4*>(x.src + half);
    }
    // Phase fences: keep the compiler from moving a use of a loaded value (and
    // the wait it implies) above loads that do not depend on it.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < kUPT; ++k) {
      Unit& x = un[k];
      const int p0 = 8 * x.j;
      if (kPerPair) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float* row = a.cos_sin + clamp_pos(x.pos[i], a.max_pos) * a.cs_rs;
          x.c[i] = row[p0 + i];
          x.s[i] = row[half + p0 + i];
        }
      } else {
        const float* row = a.cos_sin + clamp_pos(x.pos[0], a.max_pos) * a.cs_rs;
        const float4 c0 = *reinterpret_cast<const float4*>(row + p0);
        const float4 c1 = *reinterpret_cast<const float4*>(row + p0 + 4);
        const float4 s0 = *reinterpret_cast<const float4*>(row + half + p0);
        const float4 s1 = *reinterpret_cast<const float4*>(row + half + p0 + 4);
        x.c[0] = c0.x; x.c[1] = c0.y; x.c[2] = c0.z; x.c[3] = c0.w;
        x.c[4] = c1.x; x.c[5] = c1.y; x.c[6] = c1.z; x.c[7] = c1.w;
        x.s[0] = s0.x; x.s[1] = s0.y; x.s[2] = s0.z; x.s[3] = s0.w;
        x.s[4] = s1.x; x.s[5] = s1.y; x.s[6] = s1.z; x.s[7] = s1.w;
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    // All results before the first store: vmcnt counts stores too, so a store
    // issued ahead of the last unit's math would be waited for with its loads.
#pragma unroll
    for (int k = 0; k < kUPT; ++k) {
      Unit& x = un[k];
      u32x4 lo = x.lo, hi = x.hi;
      rope_word(lo.x, hi.x, x.c[0], x.s[0], x.c[1], x.s[1]);
      rope_word(lo.y, hi.y, x.c[2], x.s[2], x.c[3], x.s[3]);
      rope_word(lo.z, hi.z, x.c[4], x.s[4], x.c[5], x.s[5]);
      rope_word(lo.w, hi.w, x.c[6], x.s[6], x.c[7], x.s[7]);
      if (x.kind != 2) {  // v stays a bit copy
        x.lo = lo;
        x.hi = hi;
      }
    }
#pragma unroll
    for (int k = 0; k < kUPT; ++k) {
      Unit& x = un[k];
      const u32x4 lo = x.lo, hi = x.hi;
      const bool slot_ok = x.slot >= 0 && x.slot < a.num_slots;
      uint16_t* dst0 = x.kind == 0 ? a.q_out + (int64_t)x.n * a.qo_rs
                     : (x.kind == 1 ? a.k_cache : a.v_cache) + (int64_t)x.slot * row_elems;
      const bool st0 = x.live && (x.kind == 0 || (store && slot_ok));
      if (st0) {
        st16<kSt>(dst0 + x.off, lo);
        st16<kSt>(dst0 + x.off + half, hi);
      }
      if (x.live && x.kind == 1 && a.k_out) {
        uint16_t* dst1 = a.k_out + (int64_t)x.n * a.ko_rs + x.off;
        st16<kSt>(dst1, lo);
        st16<kSt>(dst1 + half, hi);
      }
    }
  }
}

inline bool rows16(const void* p, int64_t row_stride_elems) {
  return aligned16(p) && (row_stride_elems * 2) % 16 == 0;
}

}  // namespace
}  // namespace vlc

VLC_API int vlc_rope_store_kvcache(const void* q, int64_t q_row_stride, void* q_out,
                                   int64_t q_out_row_stride, const void* k, int64_t k_row_stride,
                                   void* k_out, int64_t k_out_row_stride, const void* v,
                                   int64_t v_row_stride, int num_heads_q, int num_heads_kv,
                                   int head_dim, const int64_t* positions, int num_position_rows,
                                   int64_t position_row_stride, const int32_t* mrope_section,
                                   const float* cos_sin_cache, int64_t cache_row_stride,
                                   int64_t max_positions, void* k_cache, void* v_cache,
                                   int64_t num_slots, const int32_t* slot_mapping,
                                   int64_t num_tokens, void* stream) {
  using namespace vlc;
  if (num_tokens < 0 || num_heads_q <= 0 || num_heads_kv <= 0 || num_slots < 0) return VLC_ERR_INVALID;
  if (head_dim <= 0 || head_dim % 16 != 0) return VLC_ERR_UNSUPPORTED;
  const int half = head_dim / 2;
  int b1 = half, b2 = half;  // 1-D: every pair in section 0
  int64_t pos_rs = 0;
  if (num_position_rows == 3) {
    if (!mrope_section || mrope_section[0] < 0 || mrope_section[1] < 0 || mrope_section[2] < 0 ||
        mrope_section[0] + mrope_section[1] + mrope_section[2] != half)
      return VLC_ERR_INVALID;
    if (position_row_stride < num_tokens) return VLC_ERR_INVALID;
    b1 = mrope_section[0];
    b2 = mrope_section[0] + mrope_section[1];
    pos_rs = position_row_stride;
  } else if (num_position_rows != 1) {
    return VLC_ERR_INVALID;
  }
  if (max_positions <= 0 || cache_row_stride < head_dim) return VLC_ERR_INVALID;
  const bool store = k_cache != nullptr || v_cache != nullptr;
  if (store && (!k_cache || !v_cache || !slot_mapping || !v)) return VLC_ERR_INVALID;
  if (num_tokens == 0) return VLC_OK;
  if (!q || !q_out || !k || !positions || !cos_sin_cache) return VLC_ERR_INVALID;
  const int64_t q_row = (int64_t)num_heads_q * head_dim, kv_row = (int64_t)num_heads_kv * head_dim;
  if (q_row_stride < q_row || q_out_row_stride < q_row || k_row_stride < kv_row) return VLC_ERR_INVALID;
  if (!rows16(q, q_row_stride) || !rows16(q_out, q_out_row_stride) || !rows16(k, k_row_stride))
    return VLC_ERR_INVALID;
  if (k_out && (k_out_row_stride < kv_row || !rows16(k_out, k_out_row_stride))) return VLC_ERR_INVALID;
  if (store && (v_row_stride < kv_row || !rows16(v, v_row_stride) || !aligned16(k_cache) ||
                !aligned16(v_cache)))
    return VLC_ERR_INVALID;
  const int uph = head_dim / 16;
  const int64_t upt = (int64_t)(num_heads_q + num_heads_kv + (store ? num_heads_kv : 0)) * uph;
  const int64_t total = num_tokens * upt;
  if (total >= (int64_t)1 << 30) return VLC_ERR_UNSUPPORTED;

  RopeArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q_rs = q_row_stride;
  a.q_out = static_cast<uint16_t*>(q_out);
  a.qo_rs = q_out_row_stride;
  a.k = static_cast<const uint16_t*>(k);
  a.k_rs = k_row_stride;
  a.k_out = static_cast<uint16_t*>(k_out);
  a.ko_rs = k_out_row_stride;
  a.v = static_cast<const uint16_t*>(v);
  a.v_rs = v_row_stride;
  a.k_cache = static_cast<uint16_t*>(k_cache);
  a.v_cache = static_cast<uint16_t*>(v_cache);
  a.num_slots = num_slots;
  a.slot_mapping = slot_mapping;
  a.positions = positions;
  a.pos_rs = pos_rs;
  a.sec_b1 = b1;
  a.sec_b2 = b2;
  a.cos_sin = cos_sin_cache;
  a.cs_rs = cache_row_stride;
  a.max_pos = max_positions;
  a.num_heads_q = num_heads_q;
  a.num_heads_kv = num_heads_kv;
  a.head_dim = head_dim;
  a.uph = uph;
  a.upt = (int)upt;
  a.total = (uint32_t)total;
  const bool per_pair = !aligned16(cos_sin_cache) || cache_row_stride % 4 != 0 || b1 % 8 != 0 || b2 % 8 != 0;
  int64_t blocks = (total + (int64_t)kThreads * kUPT - 1) / ((int64_t)kThreads * kUPT);
  if (blocks > 65535) blocks = 65535;
  // bytes written: q_out, the cache's k and v rows, k_out
  const int64_t written = num_tokens * head_dim * 2 *
                          ((int64_t)num_heads_q + (store ? 2 : 0) * num_heads_kv + (k_out ? num_heads_kv : 0));
  const int mode = store_mode_for(written);
  auto pick = [&](auto per_pair_c) {
    constexpr bool kP = decltype(per_pair_c)::value;
    return mode == kStWt   ? rope_store_kv_kernel<kP, kStWt>
           : mode == kStNt ? rope_store_kv_kernel<kP, kStNt>
                           : rope_store_kv_kernel<kP, kStPlain>;
  };
  auto kernel = per_pair ? pick(std::true_type{}) : pick(std::false_type{});
  hipLaunchKernelGGL(kernel, dim3((unsigned)blocks), dim3(kThreads), 0, as_stream(stream), a);
  return launch_status();
}
