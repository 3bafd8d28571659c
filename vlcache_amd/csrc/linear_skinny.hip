// Skinny linear layer for decode steps: out[m][n] = bf16( sum_k x[m][k] * w[n][k] + bias[n] )
// for M <= 16 rows of x.
//
// In a decode step the projections of the decoder (models/qwen3.py: QKV, output,
// gate/up and down projections, and the LM head) multiply a handful of token rows by
// the whole weight matrix, so the work is streaming the weights from HBM once; the
// library GEMMs reach about 2-3 TB/s on these shapes with cold weights.  A wave
// owns a tile of 16 output features and a K range: it streams the range of the 16
// weight rows (16 bytes per lane per 32-k step, U steps in flight) and multiplies
// them with the matching x slice on the matrix pipe,
//   C (16 features x 16 rows) += W (16 x 32) . X^T (32 x 16)   v_mfma_f32_16x16x32_bf16,
// x rows >= M read as zero.  KS waves of a workgroup share a tile (K split KS ways);
// their partial C tiles are summed through LDS in a fixed order, the bias is added in
// fp32 and the result rounded to bf16 once.
#include "common.h"

namespace vlc {
namespace {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kMaxRows = 16;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8 ld16(const char* p) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4v*>(p));
}

// KS waves split K for each 16-feature tile; a workgroup holds kWaves / KS tiles.
template <int U, int KS>
__global__ __launch_bounds__(kThreads) void linear_skinny_kernel(const char* __restrict__ x, int64_t x_stride_b,
                                                                 int rows, int k_steps, int tiles,
                                                                 const char* __restrict__ w, int64_t w_stride_b,
                                                                 const uint16_t* __restrict__ bias,
                                                                 uint16_t* __restrict__ out, int64_t out_stride) {
  constexpr int kTiles = kWaves / KS;
  __shared__ f32x4 part[KS > 1 ? kWaves : 1][64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int tile = wave / KS, ks = wave % KS;
  const int r = lane & 15;              // A: feature row of the tile; B: row of x
  const int kq = (lane >> 4) * 16;      // byte offset of the lane's 8 k values in a 32-k step
  const int t = blockIdx.x * kTiles + tile;
  const bool live = t < tiles;          // the last workgroup's tiles past N do no work
  const int f0 = (live ? t : 0) * 16;
  const char* wp = w + (int64_t)(f0 + r) * w_stride_b + kq;
  const bool xr = r < rows;
  const char* xp = x + (int64_t)(xr ? r : 0) * x_stride_b + kq;
  // the wave's contiguous range of 32-k steps
  const int per = (k_steps + KS - 1) / KS;
  const int s0 = live ? min(k_steps, ks * per) : 0, s1 = live ? min(k_steps, s0 + per) : 0;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  const bf16x8 zero = __builtin_bit_cast(bf16x8, u32x4v{0u, 0u, 0u, 0u});
  int s = s0;
  for (; s + U <= s1; s += U) {
    bf16x8 a[U], b[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      a[u] = ld16(wp + (int64_t)(s + u) * 64);
      b[u] = xr ? ld16(xp + (int64_t)(s + u) * 64) : zero;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[u], b[u], acc, 0, 0, 0);
  }
  for (; s < s1; ++s) {
    const bf16x8 a = ld16(wp + (int64_t)s * 64);
    const bf16x8 b = xr ? ld16(xp + (int64_t)s * 64) : zero;
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
  }
  if constexpr (KS > 1) {
    if (ks > 0) part[wave][lane] = acc;
    __syncthreads();
    if (ks != 0) return;
#pragma unroll
    for (int v = 1; v < KS; ++v) {
      const f32x4 p = part[wave + v][lane];
      acc[0] += p[0], acc[1] += p[1], acc[2] += p[2], acc[3] += p[3];
    }
  }
  // lane holds C[feature 4 (lane / 16) + t][row lane % 16], t = 0..3
  const int m = lane & 15;
  if (m >= rows || !live) return;
  const int f = f0 + 4 * (lane >> 4);
  float y[4] = {acc[0], acc[1], acc[2], acc[3]};
  if (bias) {
    const uint2 bv = *reinterpret_cast<const uint2*>(bias + f);
    y[0] += bf16_bits_to_f32(bv.x & 0xffffu), y[1] += bf16_bits_to_f32(bv.x >> 16);
    y[2] += bf16_bits_to_f32(bv.y & 0xffffu), y[3] += bf16_bits_to_f32(bv.y >> 16);
  }
  const uint2 o = {f32_to_bf16_bits(y[0]) | (f32_to_bf16_bits(y[1]) << 16),
                   f32_to_bf16_bits(y[2]) | (f32_to_bf16_bits(y[3]) << 16)};
  *reinterpret_cast<uint2*>(out + (int64_t)m * out_stride + f) = o;
}

template <int U, int KS>
void launch_skinny(const void* x, int64_t xs, int64_t rows, int64_t k, const void* w, int64_t ws, int64_t n,
                   const void* bias, void* out, int64_t os, hipStream_t st) {
  const int64_t tiles = n / 16;
  constexpr int kTiles = kWaves / KS;
  hipLaunchKernelGGL((linear_skinny_kernel<U, KS>), dim3((unsigned)((tiles + kTiles - 1) / kTiles)), dim3(kThreads),
                     0, st, static_cast<const char*>(x), xs * 2, (int)rows, (int)(k / 32), (int)tiles,
                     static_cast<const char*>(w), ws * 2, static_cast<const uint16_t*>(bias),
                     static_cast<uint16_t*>(out), os);
}

}  // namespace
}  // namespace vlc

VLC_API int vlc_linear_skinny(const void* x, int64_t x_row_stride, int64_t rows, int64_t in_features,
                              const void* weight, int64_t w_row_stride, int64_t out_features, const void* bias,
                              void* out, int64_t out_row_stride, void* stream) {
  using namespace vlc;
  if (rows < 0 || rows > kMaxRows || in_features <= 0 || out_features <= 0) return VLC_ERR_INVALID;
  if (in_features % 32 != 0 || out_features % 16 != 0) return VLC_ERR_UNSUPPORTED;
  if (x_row_stride < in_features || w_row_stride < in_features || out_row_stride < out_features)
    return VLC_ERR_INVALID;
  if (rows == 0) return VLC_OK;
  if (!x || !weight || !out) return VLC_ERR_INVALID;
  if (!aligned16(x) || !aligned16(weight) || (x_row_stride % 8) || (w_row_stride % 8) ||
      (reinterpret_cast<uintptr_t>(out) & 7) || (out_row_stride % 4) || (bias && (reinterpret_cast<uintptr_t>(bias) & 7)))
    return VLC_ERR_UNSUPPORTED;
  if (out_features / 16 >= ((int64_t)1 << 30)) return VLC_ERR_UNSUPPORTED;
  // Measured on the decode projections of Qwen2.5-VL-7B with cold weights (batch 4):
  // 4 steps in flight per wave (U) beat 8 and 16 on every shape (fewer registers, more
  // resident waves); a 4-way K split (two tiles per workgroup) was fastest from 288
  // tiles up (QKV 11.8, gate/up 56.8, LM head 208.8 us) and an 8-way split for 224
  // tiles (output projection 8.1, down projection 29.8 us), against 12.4, 56.7, 235.6,
  // 12.1 and 48.2 us for the library GEMMs.
  const int64_t tiles = out_features / 16;
  hipStream_t st = as_stream(stream);
  if (tiles <= 256)
    launch_skinny<4, 8>(x, x_row_stride, rows, in_features, weight, w_row_stride, out_features, bias, out,
                        out_row_stride, st);
  else
    launch_skinny<4, 4>(x, x_row_stride, rows, in_features, weight, w_row_stride, out_features, bias, out,
                        out_row_stride, st);
  return launch_status();
}
