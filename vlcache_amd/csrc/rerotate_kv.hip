// All-layer reuse copy of cached image KV with M-RoPE re-rotation of K.
//
// The reference moves reused image KV with one torch gather/scatter over every
// layer (ModelRunner.copy_image_kv, engine/model_runner.py:170-180): it reads
// the old slots into a temporary and writes the temporary to the new slots,
// without touching the rotary phase of K.  Here a single streaming launch reads
// each source row once and writes each destination row once (no temporary),
// and rotates K from the position it was cached at to its new position.
//
// Rotation: K was stored as R(pos_old) k.  Rotary embedding composes additively,
// so R(pos_new) k = R(pos_new - pos_old) R(pos_old) k.  For pair i (dims i and
// i + hd/2, the rotate-half convention of layers/rotary_embedding.py:6-14) the
// angle is delta_section(i) * inv_freq[i]; the host passes (cos, sin) per
// (segment, pair), so the kernel only multiplies.  The products are evaluated
// exactly as the fp32 reference formula writes them (x1*cos - x2*sin,
// x2*cos + x1*sin, each product and sum rounded; no fused multiply-add), then
// rounded to bf16.  A pair whose entry is (1, 0) is copied bit for bit.
//
// Work layout: a "unit" is 8 rotation pairs of one head: 16 bytes of dims
// [8j, 8j+8) and the partner 16 bytes [hd/2+8j, hd/2+8j+8).  hd/16 units cover
// a head, so for 2 kv heads x 128 dims one token row (512 B) is 16 consecutive
// lanes.  A lane moves the same unit of K and of V (four 16-byte loads in flight,
// one slot lookup for both, then four 16-byte stores).  grid.y walks layers;
// grid.x walks tokens, one unit per lane (see kStreamThreads).  Against one
// plane per lane in 256-lane workgroups this measured 114 us against 129 us for
// the 700 MB of the 4K-image request (clean MALL) and 831 against 956 us for
// 5.9 GB; more layers per lane (fewer workgroups) measured slower.
#include "common.h"

namespace vlc {
namespace {

// Workgroup size: 256 lanes for calls that stream past the MALL (124.9 against
// 125.9 us at 512 with a dirty MALL, 124.4 against 125.2 clean, on the 0.70 GB call),
// 512 for the larger calls (831 against 856 us at 256 on 5.9 GB).
constexpr int kStreamThreads = 256;
constexpr int kPlainThreads = 512;
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void rotate_word(uint32_t& a, uint32_t& b, float2 cs0, float2 cs1) {
#pragma clang fp contract(off)
  // a holds x1 for pairs (p, p+1) in its low/high halves, b holds x2 for the same pairs.
  const float a0 = bf16_bits_to_f32(a & 0xffffu), a1 = bf16_bits_to_f32(a >> 16);
  const float b0 = bf16_bits_to_f32(b & 0xffffu), b1 = bf16_bits_to_f32(b >> 16);
  uint32_t ya0 = a & 0xffffu, ya1 = a >> 16, yb0 = b & 0xffffu, yb1 = b >> 16;
  if (!(cs0.x == 1.0f && cs0.y == 0.0f)) {
    const float y1 = a0 * cs0.x - b0 * cs0.y;
    const float y2 = b0 * cs0.x + a0 * cs0.y;
    ya0 = f32_to_bf16_bits(y1);
    yb0 = f32_to_bf16_bits(y2);
  }
  if (!(cs1.x == 1.0f && cs1.y == 0.0f)) {
    const float y1 = a1 * cs1.x - b1 * cs1.y;
    const float y2 = b1 * cs1.x + a1 * cs1.y;
    ya1 = f32_to_bf16_bits(y1);
    yb1 = f32_to_bf16_bits(y2);
  }
  a = ya0 | (ya1 << 16);
  b = yb0 | (yb1 << 16);
}

// Calls that move at most kStreamMaxBytes (read + write) stream past the MALL: loads
// nontemporal and stores at agent scope with the nontemporal hint (st16_wt_nt, written
// through L2 and not allocated in the MALL).  The warm request's call meets a MALL full
// of the previous request's dirty KV lines; any access that allocates there first
// writes those back.  Measured on the 4K request's 0.70 GB (cold, median, clean / dirty
// MALL, us): nontemporal loads with these stores 124.8 / 124.8; with agent-scope
// stores that allocate 108.3 / 132.5; nontemporal stores 125.5 / 125.4; plain loads and
// stores 116.3 / 159.6.  Larger calls (1.48 GB and up) use plain loads and stores, which
// stream faster once the MALL's contents are a small part of the call: 5.9 GB in
// 855 / 883 us against 1091 / 1128 us with nontemporal loads.
constexpr int64_t kStreamMaxBytes = (int64_t)1 << 30;

// 16-byte store at agent scope with the nontemporal hint; same inline-assembly caveats
// as st16_wt.
__device__ __forceinline__ void st16_wt_nt(void* p, const u32x4_vec& w) {
  asm volatile("global_store_dwordx4 %0, %1, off sc1 nt\n\ts_nop 1" : : "v"(p), "v"(w) : "memory");
}

template <bool kStream, int kThreads = kStream ? kStreamThreads : kPlainThreads>
__global__ __launch_bounds__(kThreads) void rerotate_copy_kv_kernel(
    uint16_t* __restrict__ kv, int64_t plane_stride, int64_t layer_stride, int num_layers,
    const int64_t* __restrict__ old_slots, const int64_t* __restrict__ new_slots,
    int64_t num_tokens, int64_t num_slots, int row_elems, int head_dim, int units_per_token,
    const int32_t* __restrict__ seg_of_token, const float2* __restrict__ cos_sin,
    int num_segments, int rotate_k) {
  const int layer = blockIdx.y;
  uint16_t* const base0 = kv + (int64_t)layer * layer_stride;
  const int half = head_dim >> 1;
  const int units_per_head = head_dim >> 4;
  const int64_t total = num_tokens * units_per_token;
  const int64_t stride = (int64_t)gridDim.x * kThreads;

  struct Unit {
    u32x4 lo, hi;
    uint16_t* dst;  // nullptr = nothing to store
  };
  // Loads (and for K rotates) unit u of one plane (0 = K, 1 = V); u < total < 2^32.
  auto fetch = [&](int64_t u, int plane) -> Unit {
    uint16_t* base = base0 + plane * plane_stride;
    const bool rot = rotate_k && plane == 0;
    Unit un{{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}, nullptr};
    if (u >= total) return un;
    const uint32_t u32 = (uint32_t)u;
    const uint32_t n = u32 / (uint32_t)units_per_token;
    const int rem = (int)(u32 - n * (uint32_t)units_per_token);
    const int hh = rem / units_per_head;
    const int j = rem - hh * units_per_head;
    const int64_t os = old_slots[n], ns = new_slots[n];
    if (os < 0 || os >= num_slots || ns < 0 || ns >= num_slots) return un;
    const int64_t off = (int64_t)hh * head_dim + 8 * j;
    const uint16_t* src = base + os * row_elems + off;
    const u32x4v* s0 = reinterpret_cast<const u32x4v*>(src);
    const u32x4v* s1 = reinterpret_cast<const u32x4v*>(src + half);
    u32x4 lo = __builtin_bit_cast(u32x4, kStream ? __builtin_nontemporal_load(s0) : *s0);
    u32x4 hi = __builtin_bit_cast(u32x4, kStream ? __builtin_nontemporal_load(s1) : *s1);
    if (rot) {
      int sgi = seg_of_token ? seg_of_token[n] : 0;
      sgi = sgi < 0 ? 0 : (sgi >= num_segments ? num_segments - 1 : sgi);
      const float2* cs = cos_sin + (int64_t)sgi * half + 8 * j;
      rotate_word(lo.x, hi.x, cs[0], cs[1]);
      rotate_word(lo.y, hi.y, cs[2], cs[3]);
      rotate_word(lo.z, hi.z, cs[4], cs[5]);
      rotate_word(lo.w, hi.w, cs[6], cs[7]);
    }
    un.lo = lo;
    un.hi = hi;
    un.dst = base + ns * row_elems + off;
    return un;
  };
  for (int64_t u0 = (int64_t)blockIdx.x * kThreads + threadIdx.x; u0 < total; u0 += stride) {
    Unit un[2];
    un[0] = fetch(u0, 0);
    un[1] = fetch(u0, 1);
#pragma unroll
    for (int k = 0; k < 2; ++k)
      if (un[k].dst) {
        if constexpr (kStream) {
          st16_wt_nt(un[k].dst, __builtin_bit_cast(u32x4_vec, un[k].lo));
          st16_wt_nt(un[k].dst + half, __builtin_bit_cast(u32x4_vec, un[k].hi));
        } else {
          *reinterpret_cast<u32x4v*>(un[k].dst) = __builtin_bit_cast(u32x4v, un[k].lo);
          *reinterpret_cast<u32x4v*>(un[k].dst + half) = __builtin_bit_cast(u32x4v, un[k].hi);
        }
      }
  }
}

}  // namespace
}  // namespace vlc

VLC_API int vlc_rerotate_copy_kv(void* kv_cache, int64_t plane_stride, int64_t layer_stride,
                                 int num_layers, const int64_t* old_slots,
                                 const int64_t* new_slots, int64_t num_tokens, int64_t num_slots,
                                 int num_kv_heads, int head_dim, const int32_t* seg_of_token,
                                 const float* cos_sin, int num_segments, int rotate_k,
                                 void* stream) {
  using namespace vlc;
  if (num_tokens < 0 || num_layers <= 0 || num_kv_heads <= 0 || num_slots <= 0) return VLC_ERR_INVALID;
  if (head_dim <= 0 || head_dim % 16 != 0) return VLC_ERR_UNSUPPORTED;
  if (num_tokens == 0) return VLC_OK;
  if (!kv_cache || !old_slots || !new_slots) return VLC_ERR_INVALID;
  if (rotate_k && (!cos_sin || num_segments <= 0)) return VLC_ERR_INVALID;
  if (!aligned16(kv_cache) || (plane_stride * 2) % 16 != 0 || (layer_stride * 2) % 16 != 0)
    return VLC_ERR_INVALID;
  const int row_elems = num_kv_heads * head_dim;
  if (layer_stride < num_slots * row_elems || plane_stride < (int64_t)num_layers * layer_stride)
    return VLC_ERR_INVALID;
  if (num_layers > 65535) return VLC_ERR_UNSUPPORTED;
  const int units_per_token = num_kv_heads * (head_dim / 16);
  const int64_t total = num_tokens * units_per_token;
  if (total >= ((int64_t)1 << 32)) return VLC_ERR_UNSUPPORTED;  // 32-bit unit index
  const int64_t moved = num_tokens * num_layers * 2 * (int64_t)row_elems * 2 * 2;  // K+V, read+write
  const bool past_mall = moved <= kStreamMaxBytes;
  const int threads = past_mall ? kStreamThreads : kPlainThreads;
  int64_t bx = (total + threads - 1) / threads;
  if (bx > 65535) bx = 65535;
  auto kernel = past_mall ? rerotate_copy_kv_kernel<true> : rerotate_copy_kv_kernel<false>;
  hipLaunchKernelGGL(kernel, dim3((unsigned)bx, num_layers), dim3(threads), 0,
                     as_stream(stream), static_cast<uint16_t*>(kv_cache), plane_stride, layer_stride,
                     num_layers, old_slots, new_slots, num_tokens, num_slots, row_elems, head_dim,
                     units_per_token, seg_of_token, reinterpret_cast<const float2*>(cos_sin),
                     rotate_k ? num_segments : 1, rotate_k);
  return launch_status();
}
