// Paged KV-cache scatter: the gfx950 replacement of the reference's Triton
// store_kvcache_kernel (layers/attention.py:10-30).
//
// Semantics (bit copy): for token n with slot = slot_mapping[n] >= 0, K row n and
// V row n (row_bytes each) go to row `slot` of k_cache / v_cache; slot < 0 skips.
//
// Layout of the work: one 16-byte chunk per lane.  A token owns 2*C chunks
// (C = row_bytes/16 for K, then C for V), so for Qwen2.5-VL-3B (2 kv heads x 128
// dims, 512 B per row) one wave64 moves exactly one token: lanes 0-31 carry K,
// lanes 32-63 carry V, each half a fully coalesced 512-byte read and write.
// Each thread handles VPT chunks strided by the grid so that several 16-byte
// loads are in flight before the first store.
#include "common.h"

namespace vlc {
namespace {

constexpr int kThreads = 256;
constexpr int kVPT = 1;  // chunks per thread

__global__ __launch_bounds__(kThreads) void store_kvcache_vec16(
    const char* __restrict__ key, int64_t key_stride_b, const char* __restrict__ value,
    int64_t value_stride_b, char* __restrict__ k_cache, char* __restrict__ v_cache,
    int64_t num_slots, const int32_t* __restrict__ slot_mapping, int64_t num_tokens,
    int chunks_per_row, int64_t row_bytes) {
  const int64_t chunks_per_token = 2 * (int64_t)chunks_per_row;
  const int64_t total = num_tokens * chunks_per_token;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  struct Chunk {
    u32x4 data;
    char* dst;  // nullptr = nothing to store
  };
  auto fetch = [&](int64_t w) -> Chunk {
    Chunk ch{{0u, 0u, 0u, 0u}, nullptr};
    if (w >= total) return ch;
    const int64_t n = w / chunks_per_token;
    const int c = (int)(w - n * chunks_per_token);
    const int32_t slot = slot_mapping[n];
    if (slot < 0 || slot >= num_slots) return ch;
    const bool is_v = c >= chunks_per_row;
    const int cc = is_v ? c - chunks_per_row : c;
    const char* src = is_v ? value + n * value_stride_b : key + n * key_stride_b;
    ch.data = *reinterpret_cast<const u32x4*>(src + (int64_t)cc * 16);
    ch.dst = (is_v ? v_cache : k_cache) + (int64_t)slot * row_bytes + (int64_t)cc * 16;
    return ch;
  };
  for (int64_t u = (int64_t)blockIdx.x * kThreads + threadIdx.x; u < total; u += stride * kVPT) {
    // All kVPT loads are issued before the first store.
    Chunk c[kVPT];
#pragma unroll
    for (int k = 0; k < kVPT; ++k) c[k] = fetch(u + k * stride);
#pragma unroll
    for (int k = 0; k < kVPT; ++k)
      if (c[k].dst) *reinterpret_cast<u32x4*>(c[k].dst) = c[k].data;
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
    const int64_t total = num_tokens * 2 * cpr;
    int64_t blocks = (total + (int64_t)kThreads * kVPT - 1) / ((int64_t)kThreads * kVPT);
    if (blocks < 1) blocks = 1;
    if (blocks > (1 << 20)) blocks = 1 << 20;
    hipLaunchKernelGGL(store_kvcache_vec16, dim3((unsigned)blocks), dim3(kThreads), 0, s,
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
