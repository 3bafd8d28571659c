// Paged KV-cache scatter: the gfx950 replacement of the reference's Triton
// store_kvcache_kernel (layers/attention.py:10-30).
//
// Semantics (bit copy): for token n with slot = slot_mapping[n] >= 0, K row n and
// V row n (row_bytes each) go to row `slot` of k_cache / v_cache; slot < 0 skips.
//
// Layout of the work: a lane moves 16-byte chunk c of both the K row and the V
// row of its token (one slot lookup, two loads in flight, then two stores).  A
// token owns C = row_bytes/16 chunks, so for Qwen2.5-VL-3B (2 kv heads x 128 dims,
// 512 B per row) 32 consecutive lanes read and write a whole K row and a whole V
// row, fully coalesced.  Against one chunk of K or of V per lane this measured
// 4.89 us against 5.72 us for the 22 MB of a 10741-token layer (2.2 us either
// way for 1247 tokens, where the launch dominates).  The cache rows are stored with
// the policy store_mode_for picks from the bytes the call writes: at agent scope
// (written through L2) up to 64 MB, nontemporally up to 256 MB (22 MB in 3.16
// against 4.29 us with plain stores, 67 MB in 9.9 against 11.7 us; 36 calls in one
// graph, distinct caches), plain above; nontemporal loads measured slower (3.4 and
// 10.4 us).
#include "common.h"

namespace vlc {
namespace {

constexpr int kThreads = 256;

template <int kSt>
__global__ __launch_bounds__(kThreads) void store_kvcache_vec16(
    const char* __restrict__ key, int64_t key_stride_b, const char* __restrict__ value,
    int64_t value_stride_b, char* __restrict__ k_cache, char* __restrict__ v_cache,
    int64_t num_slots, const int32_t* __restrict__ slot_mapping, int64_t num_tokens,
    int chunks_per_row, int64_t row_bytes) {
  const int64_t total = num_tokens * (int64_t)chunks_per_row;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  for (int64_t u = (int64_t)blockIdx.x * kThreads + threadIdx.x; u < total; u += stride) {
    const uint32_t n = (uint32_t)u / (uint32_t)chunks_per_row;
    const int cc = (int)((uint32_t)u - n * (uint32_t)chunks_per_row);
    // The slot and the two rows are independent loads: all three are in flight
    // before the slot is tested (the rows of token n are always readable), so the
    // stores wait for one memory round trip, not two.
    const int32_t slot = slot_mapping[n];
    const u32x4 kd = *reinterpret_cast<const u32x4*>(key + (int64_t)n * key_stride_b + (int64_t)cc * 16);
    const u32x4 vd = *reinterpret_cast<const u32x4*>(value + (int64_t)n * value_stride_b + (int64_t)cc * 16);
    // keeps the three loads above the test (and the test below the last load)
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::"v"(slot), "v"(kd.x), "v"(kd.y), "v"(kd.z), "v"(kd.w), "v"(vd.x), "v"(vd.y), "v"(vd.z),
                 "v"(vd.w));
    if (slot < 0 || slot >= num_slots) continue;
    const int64_t o = (int64_t)slot * row_bytes + (int64_t)cc * 16;
    st16<kSt>(k_cache + o, kd);
    st16<kSt>(v_cache + o, vd);
  }
}

// Fallback for rows or strides that are not 16-byte aligned: element-wise copy.
template <typename T>
__global__ __launch_bounds__(kThreads) void store_kvcache_scalar(
    const T* __restrict__ key, int64_t key_stride, const T* __restrict__ value,
    int64_t value_stride, T* __restrict__ k_cache, T* __restrict__ v_cache,
    int64_t num_slots, const int32_t* __restrict__ slot_mapping, int64_t num_tokens,
    int64_t row_elems) {
  const int64_t per_token = 2 * row_elems;
  const int64_t total = num_tokens * per_token;
  for (int64_t w = (int64_t)blockIdx.x * kThreads + threadIdx.x; w < total;
       w += (int64_t)gridDim.x * kThreads) {
    const int64_t n = w / per_token;
    const int64_t e = w - n * per_token;
    const int32_t slot = slot_mapping[n];
    if (slot < 0 || slot >= num_slots) continue;
    if (e < row_elems)
      k_cache[(int64_t)slot * row_elems + e] = key[n * key_stride + e];
    else
      v_cache[(int64_t)slot * row_elems + (e - row_elems)] = value[n * value_stride + (e - row_elems)];
  }
}

}  // namespace
}  // namespace vlc

VLC_API int vlc_store_kvcache(const void* key, int64_t key_row_stride, const void* value,
                              int64_t value_row_stride, void* k_cache, void* v_cache,
                              int64_t num_slots, const int32_t* slot_mapping, int64_t num_tokens,
                              int64_t row_elems,
                              int elem_bytes, void* stream) {
  using namespace vlc;
  if (num_tokens < 0 || row_elems <= 0 || num_slots < 0 || (elem_bytes != 2 && elem_bytes != 4))
    return VLC_ERR_INVALID;
  if (key_row_stride < row_elems || value_row_stride < row_elems) return VLC_ERR_INVALID;
  if (num_tokens == 0) return VLC_OK;
  if (!key || !value || !k_cache || !v_cache || !slot_mapping) return VLC_ERR_INVALID;
  hipStream_t s = as_stream(stream);
  const int64_t row_bytes = row_elems * elem_bytes;
  const bool vec = (row_bytes % 16 == 0) && ((key_row_stride * elem_bytes) % 16 == 0) &&
                   ((value_row_stride * elem_bytes) % 16 == 0) && aligned16(key) &&
                   aligned16(value) && aligned16(k_cache) && aligned16(v_cache);
  if (vec) {
    const int cpr = (int)(row_bytes / 16);
    const int64_t total = num_tokens * cpr;
    if (total >= ((int64_t)1 << 32)) return VLC_ERR_UNSUPPORTED;  // 32-bit chunk index
    int64_t blocks = (total + kThreads - 1) / kThreads;
    if (blocks < 1) blocks = 1;
    if (blocks > (1 << 20)) blocks = 1 << 20;
    const int mode = store_mode_for(2 * num_tokens * row_bytes);
    auto kernel = mode == kStWt   ? store_kvcache_vec16<kStWt>
                  : mode == kStNt ? store_kvcache_vec16<kStNt>
                                  : store_kvcache_vec16<kStPlain>;
    hipLaunchKernelGGL(kernel, dim3((unsigned)blocks), dim3(kThreads), 0, s,
                       static_cast<const char*>(key), key_row_stride * elem_bytes,
                       static_cast<const char*>(value), value_row_stride * elem_bytes,
                       static_cast<char*>(k_cache), static_cast<char*>(v_cache), num_slots,
                       slot_mapping, num_tokens, cpr, row_bytes);
  } else {
    const int64_t total = num_tokens * 2 * row_elems;
    int64_t blocks = (total + kThreads - 1) / kThreads;
    if (blocks > (1 << 20)) blocks = 1 << 20;
    if (elem_bytes == 2)
      hipLaunchKernelGGL(store_kvcache_scalar<uint16_t>, dim3((unsigned)blocks), dim3(kThreads), 0,
                         s, static_cast<const uint16_t*>(key), key_row_stride,
                         static_cast<const uint16_t*>(value), value_row_stride,
                         static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache),
                         num_slots, slot_mapping, num_tokens, row_elems);
    else
      hipLaunchKernelGGL(store_kvcache_scalar<uint32_t>, dim3((unsigned)blocks), dim3(kThreads), 0,
                         s, static_cast<const uint32_t*>(key), key_row_stride,
                         static_cast<const uint32_t*>(value), value_row_stride,
                         static_cast<uint32_t*>(k_cache), static_cast<uint32_t*>(v_cache),
                         num_slots, slot_mapping, num_tokens, row_elems);
  }
  return launch_status();
}
