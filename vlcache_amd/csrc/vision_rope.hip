// 2-D rotary embedding of the vision tower's q and k, fused with the split of the
// QKV projection into head rows padded for the attention kernel.
//
// Replaces, per vision block, qkv.split + reshape + apply_rotary_pos_emb_vision
// of q and k (models/qwen2_5_vl.py:176-199).  The reference's cos/sin and q/k are
// bf16 tensors there, so every product and the sum round to bf16:
//   y[j] = bf16( bf16(x[j] * cos[j]) + bf16(r[j] * sin[j]) ),
//   r[j] = -x[j + D/2] for j < D/2, x[j - D/2] otherwise (rotate_half),
// where an fp32 product of two bf16 values is exact, so each term rounds once,
// and the sum is an fp32 add rounded to bf16: the same bits as the reference's
// three elementwise bf16 ops.  cos[j]/sin[j] of dim j come from the caller's
// bf16 tables [max_pos][D/4]: with a = j mod D/2, frequency a of the row axis
// (table row = patch row) for a < D/4, frequency a - D/4 of the column axis
// (table row = patch column) otherwise (the reference's cat(rpe, rpe) of the
// [h-axis | w-axis] angles, :452-462, :486-487).
//
// Output: [n][3][num_heads][padded_dim] bf16 (q, k, v), dims head_dim.. of each
// head zero, so the attention kernel (128-dim heads) computes the 80-dim
// attention exactly: zero dims add nothing to q.k, and the padded output dims
// are zero.  v is copied bit for bit.
//
// Work: a workgroup per (token, 16 of the 3 * num_heads head rows), a lane per
// 16-byte output chunk (16 chunks of 8 dims per 128-dim padded head), so a
// head row's lanes are adjacent and its loads and stores coalesce; no integer
// division.  A rotated chunk also reads the partner chunk D/2 away in the same
// head (L1 hit: the same head row), and its 8 cos and 8 sin values as 8-byte
// loads from the tables (L1/L2 hits: the tables are a few KB).
#include "common.h"

namespace vlc {
namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = kThreads / 16;  // head rows per workgroup (16 lanes each)

__device__ __forceinline__ float rbf(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }

// 4 consecutive bf16 table entries from an 8-byte aligned address.
__device__ __forceinline__ uint2 ld4(const uint16_t* p) { return *reinterpret_cast<const uint2*>(p); }

__global__ __launch_bounds__(kThreads) void vision_rope_pad_kernel(
    const char* __restrict__ qkv, int64_t qkv_stride_b, const int32_t* __restrict__ pos_hw,
    const uint16_t* __restrict__ cos_tab, const uint16_t* __restrict__ sin_tab, int max_pos, int num_heads,
    int head_dim, int chunks_per_head, char* __restrict__ out, int64_t out_stride_b) {
  const int c = threadIdx.x & 15;
  const int hp = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 4);  // part * num_heads + head
  if (hp >= 3 * num_heads || c >= chunks_per_head) return;
  const int64_t n = blockIdx.y;
  u32x4* dst = reinterpret_cast<u32x4*>(out + n * out_stride_b + ((int64_t)hp * chunks_per_head + c) * 16);
  const int d0 = c * 8;
  if (d0 >= head_dim) {
    *dst = u32x4{0u, 0u, 0u, 0u};
    return;
  }
  const char* row = qkv + n * qkv_stride_b + (int64_t)hp * head_dim * 2;
  const u32x4 xv = *reinterpret_cast<const u32x4*>(row + d0 * 2);
  if (hp >= 2 * num_heads) {  // v
    *dst = xv;
    return;
  }
  const int half = head_dim >> 1, quarter = head_dim >> 2;
  const bool lo = d0 < half;
  const u32x4 pv = *reinterpret_cast<const u32x4*>(row + (lo ? d0 + half : d0 - half) * 2);
  int ph = pos_hw[2 * n], pw = pos_hw[2 * n + 1];
  ph = ph < 0 ? 0 : (ph >= max_pos ? max_pos - 1 : ph);
  pw = pw < 0 ? 0 : (pw >= max_pos ? max_pos - 1 : pw);
  // Table entries of dims d0 .. d0+7, in two runs of 4 (a run never straddles the
  // row / column boundary at quarter, a multiple of 4): entry index a = j mod half.
  const int a0 = lo ? d0 : d0 - half;
  uint32_t cw[4], sw[4];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int a = a0 + 4 * r;
    const int t = a < quarter ? ph * quarter + a : pw * quarter + (a - quarter);
    const uint2 cv = ld4(cos_tab + t), sv = ld4(sin_tab + t);
    cw[2 * r] = cv.x, cw[2 * r + 1] = cv.y;
    sw[2 * r] = sv.x, sw[2 * r + 1] = sv.y;
  }
  const uint32_t xs[4] = {xv.x, xv.y, xv.z, xv.w};
  const uint32_t ps[4] = {pv.x, pv.y, pv.z, pv.w};
  uint32_t ys[4];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    uint32_t packed = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float cs = bf16_bits_to_f32((cw[w] >> (16 * h)) & 0xffffu);
      const float sn = bf16_bits_to_f32((sw[w] >> (16 * h)) & 0xffffu);
      const float x = bf16_bits_to_f32((xs[w] >> (16 * h)) & 0xffffu);
      const float p = bf16_bits_to_f32((ps[w] >> (16 * h)) & 0xffffu);
      const float y = rbf(x * cs) + rbf((lo ? -p : p) * sn);
      packed |= f32_to_bf16_bits(y) << (16 * h);
    }
    ys[w] = packed;
  }
  *dst = u32x4{ys[0], ys[1], ys[2], ys[3]};
}

}  // namespace
}  // namespace vlc

VLC_API int vlc_vision_rope_pad(const void* qkv, int64_t qkv_row_stride, const int32_t* pos_hw,
                                const void* cos_table, const void* sin_table, int64_t max_pos,
                                int64_t num_tokens, int num_heads, int head_dim, int padded_dim,
                                void* out, int64_t out_row_stride, void* stream) {
  using namespace vlc;
  if (num_tokens < 0 || num_heads <= 0 || head_dim <= 0 || head_dim % 16 != 0 ||
      padded_dim < head_dim || padded_dim % 8 != 0 || padded_dim > 128 || max_pos <= 0 || max_pos >= (1 << 24))
    return VLC_ERR_INVALID;
  if (qkv_row_stride < 3 * (int64_t)num_heads * head_dim ||
      out_row_stride < 3 * (int64_t)num_heads * padded_dim)
    return VLC_ERR_INVALID;
  if (num_tokens == 0) return VLC_OK;
  if (!qkv || !pos_hw || !cos_table || !sin_table || !out) return VLC_ERR_INVALID;
  if (!aligned16(qkv) || !aligned16(out) || (qkv_row_stride * 2) % 16 != 0 || (out_row_stride * 2) % 16 != 0 ||
      (reinterpret_cast<uintptr_t>(cos_table) & 7) || (reinterpret_cast<uintptr_t>(sin_table) & 7))
    return VLC_ERR_UNSUPPORTED;
  if ((int64_t)(head_dim / 4) * max_pos >= ((int64_t)1 << 31)) return VLC_ERR_UNSUPPORTED;
  if (num_tokens > 65535) {  // grid.y limit: launch in slices of tokens
    for (int64_t t0 = 0; t0 < num_tokens; t0 += 65535) {
      const int64_t nt = num_tokens - t0 < 65535 ? num_tokens - t0 : 65535;
      const int st = vlc_vision_rope_pad(static_cast<const char*>(qkv) + t0 * qkv_row_stride * 2, qkv_row_stride,
                                         pos_hw + 2 * t0, cos_table, sin_table, max_pos, nt, num_heads, head_dim,
                                         padded_dim, static_cast<char*>(out) + t0 * out_row_stride * 2,
                                         out_row_stride, stream);
      if (st != VLC_OK) return st;
    }
    return VLC_OK;
  }
  const int rows = 3 * num_heads;
  const dim3 grid((unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock), (unsigned)num_tokens);
  hipLaunchKernelGGL(vision_rope_pad_kernel, grid, dim3(kThreads), 0, as_stream(stream),
                     static_cast<const char*>(qkv), qkv_row_stride * 2, pos_hw,
                     static_cast<const uint16_t*>(cos_table), static_cast<const uint16_t*>(sin_table),
                     (int)max_pos, num_heads, head_dim, padded_dim / 8, static_cast<char*>(out), out_row_stride * 2);
  return launch_status();
}
