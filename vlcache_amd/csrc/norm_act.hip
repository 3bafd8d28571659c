// RMSNorm (with the fused residual add) and SiLU-and-multiply for the decoder
// and the vision tower: one launch each instead of torch's chain of eager
// elementwise and reduction kernels.
//
// rms_norm follows layers/layernorm.py:16-40 of the reference:
//   without residual: y = bf16( bf16(x * r) * w ),             r = rsqrt(mean(x^2) + eps)
//   with residual:    s = x + res (fp32); res_out = bf16(s);  y = bf16( bf16(s * r) * w ),
//                     r from the fp32 s (not the rounded res_out);
// statistics in fp32.  A wave owns a row: each lane holds its 16-byte chunks
// in registers between the sum of squares and the scaling, so a row is read
// once and written once.  The sum runs lane-serially over the lane's chunks,
// then across the wave by butterfly.
//
// silu_mul follows layers/activation.py:8-14 (SiluAndMul: chunk the last dim
// into gate and up, silu(gate) * up) with fp32 math and one rounding to bf16,
// as the reference's compiled kernel computes it.  A lane owns 4 elements.
#include "common.h"

namespace vlc {
namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = kThreads / 64;

__device__ __forceinline__ float lo16(uint32_t w) { return bf16_bits_to_f32(w & 0xffffu); }
__device__ __forceinline__ float hi16(uint32_t w) { return bf16_bits_to_f32(w >> 16); }
// fp32 -> bf16 with the hardware conversion (round to nearest even, v_cvt_pk_bf16_f32).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  const bf16x2_t v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ float rbf(float f) { return static_cast<float>(static_cast<__bf16>(f)); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// CPL = chunks (of 8 elements) per lane, rounded up: dim <= 64 * CPL * 8.
template <int CPL, bool kResidual>
__global__ __launch_bounds__(kThreads) void rms_norm_kernel(
    const char* x, int64_t x_stride_b, const char* res, int64_t res_stride_b, char* res_out,
    int64_t res_out_stride_b, const char* __restrict__ weight, float eps, int64_t rows, int chunks,
    float inv_dim, char* out, int64_t out_stride_b) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  // Every load of the row is issued before the first store: the new residual may be
  // written over x or the old residual, so a store ahead of a later chunk's load would
  // keep that load from being hoisted and serialise the row into CPL round trips.
  // The weight chunks are loaded with them, so the scaling does not wait for a second
  // round trip after the row's reduction.
  u32x4 xa[CPL], ra[CPL], wa[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = lane + 64 * i;
    if (c < chunks) {
      xa[i] = *reinterpret_cast<const u32x4*>(x + row * x_stride_b + c * 16);
      if constexpr (kResidual) ra[i] = *reinterpret_cast<const u32x4*>(res + row * res_stride_b + c * 16);
      wa[i] = *reinterpret_cast<const u32x4*>(weight + c * 16);
    }
  }
  float s[CPL][8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = lane + 64 * i;
    if (c < chunks) {
      const uint32_t aw[4] = {xa[i].x, xa[i].y, xa[i].z, xa[i].w};
      if constexpr (kResidual) {
        const uint32_t bw[4] = {ra[i].x, ra[i].y, ra[i].z, ra[i].w};
        uint32_t ro[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          s[i][2 * k] = lo16(aw[k]) + lo16(bw[k]);
          s[i][2 * k + 1] = hi16(aw[k]) + hi16(bw[k]);
          ro[k] = pack2(s[i][2 * k], s[i][2 * k + 1]);
        }
        *reinterpret_cast<u32x4*>(res_out + row * res_out_stride_b + c * 16) = u32x4{ro[0], ro[1], ro[2], ro[3]};
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          s[i][2 * k] = lo16(aw[k]);
          s[i][2 * k + 1] = hi16(aw[k]);
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += s[i][e] * s[i][e];
    }
  }
  ss = wave_sum(ss);
  const float r = rsqrtf(ss * inv_dim + eps);
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = lane + 64 * i;
    if (c < chunks) {
      const uint32_t ww[4] = {wa[i].x, wa[i].y, wa[i].z, wa[i].w};
      uint32_t o[4];
#pragma unroll
      for (int k = 0; k < 4; ++k)
        o[k] = pack2(rbf(s[i][2 * k] * r) * lo16(ww[k]), rbf(s[i][2 * k + 1] * r) * hi16(ww[k]));
      *reinterpret_cast<u32x4*>(out + row * out_stride_b + c * 16) = u32x4{o[0], o[1], o[2], o[3]};
    }
  }
}

template <int CPL>
int launch_rms(const void* x, int64_t xs, const void* res, int64_t rs, void* ro, int64_t ros, const void* w,
               float eps, int64_t rows, int dim, void* out, int64_t os, hipStream_t st) {
  const int64_t blocks = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  const float inv_dim = 1.0f / (float)dim;
  if (res)
    hipLaunchKernelGGL((rms_norm_kernel<CPL, true>), dim3((unsigned)blocks), dim3(kThreads), 0, st,
                       static_cast<const char*>(x), xs * 2, static_cast<const char*>(res), rs * 2,
                       static_cast<char*>(ro), ros * 2, static_cast<const char*>(w), eps, rows, dim / 8, inv_dim,
                       static_cast<char*>(out), os * 2);
  else
    hipLaunchKernelGGL((rms_norm_kernel<CPL, false>), dim3((unsigned)blocks), dim3(kThreads), 0, st,
                       static_cast<const char*>(x), xs * 2, nullptr, 0, nullptr, 0, static_cast<const char*>(w),
                       eps, rows, dim / 8, inv_dim, static_cast<char*>(out), os * 2);
  return launch_status();
}

// V = 8: 16-byte accesses (inter % 8 == 0), else 8-byte ones (V = 4).
template <int V>
__global__ __launch_bounds__(kThreads) void silu_mul_kernel(const char* __restrict__ gu, int64_t gu_stride_b,
                                                            int64_t rows, int groups, int64_t up_offset_b,
                                                            char* __restrict__ out, int64_t out_stride_b) {
  const int64_t u = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (u >= rows * groups) return;
  const int64_t row = u / groups;
  const int q = (int)(u - row * groups);
  const char* src = gu + row * gu_stride_b + (int64_t)q * (2 * V);
  uint32_t g[V / 2], p[V / 2];
  if constexpr (V == 8) {
    const u32x4 a = *reinterpret_cast<const u32x4*>(src);
    const u32x4 b = *reinterpret_cast<const u32x4*>(src + up_offset_b);
    g[0] = a.x, g[1] = a.y, g[2] = a.z, g[3] = a.w;
    p[0] = b.x, p[1] = b.y, p[2] = b.z, p[3] = b.w;
  } else {
    const uint2 a = *reinterpret_cast<const uint2*>(src);
    const uint2 b = *reinterpret_cast<const uint2*>(src + up_offset_b);
    g[0] = a.x, g[1] = a.y;
    p[0] = b.x, p[1] = b.y;
  }
  uint32_t o[V / 2];
#pragma unroll
  for (int k = 0; k < V / 2; ++k) {
    const float g0 = lo16(g[k]), g1 = hi16(g[k]);
    o[k] = pack2(g0 / (1.0f + expf(-g0)) * lo16(p[k]), g1 / (1.0f + expf(-g1)) * hi16(p[k]));
  }
  char* dst = out + row * out_stride_b + (int64_t)q * (2 * V);
  if constexpr (V == 8)
    *reinterpret_cast<u32x4*>(dst) = u32x4{o[0], o[1], o[2], o[3]};
  else
    *reinterpret_cast<uint2*>(dst) = uint2{o[0], o[1]};
}

}  // namespace
}  // namespace vlc

VLC_API int vlc_rms_norm(const void* x, int64_t x_row_stride, const void* residual, int64_t residual_row_stride,
                         void* residual_out, int64_t residual_out_row_stride, const void* weight, float eps,
                         int64_t num_rows, int64_t dim, void* out, int64_t out_row_stride, void* stream) {
  using namespace vlc;
  if (num_rows < 0 || dim <= 0 || dim % 8 != 0 || dim > 64 * 16 * 8 || !(eps >= 0.f)) return VLC_ERR_INVALID;
  if (x_row_stride < dim || out_row_stride < dim) return VLC_ERR_INVALID;
  if (residual && (residual_row_stride < dim || !residual_out || residual_out_row_stride < dim))
    return VLC_ERR_INVALID;
  if (num_rows == 0) return VLC_OK;
  if (!x || !weight || !out) return VLC_ERR_INVALID;
  if (!aligned16(x) || !aligned16(weight) || !aligned16(out) || (x_row_stride % 8) || (out_row_stride % 8))
    return VLC_ERR_UNSUPPORTED;
  if (residual && (!aligned16(residual) || !aligned16(residual_out) || (residual_row_stride % 8) ||
                   (residual_out_row_stride % 8)))
    return VLC_ERR_UNSUPPORTED;
  const int chunks = (int)(dim / 8);
  const int cpl = (chunks + 63) / 64;
  hipStream_t s = as_stream(stream);
#define VLC_RMS_CASE(N) \
  case N:               \
    return launch_rms<N>(x, x_row_stride, residual, residual_row_stride, residual_out, residual_out_row_stride, \
                         weight, eps, num_rows, (int)dim, out, out_row_stride, s);
  switch (cpl) {
    VLC_RMS_CASE(1) VLC_RMS_CASE(2) VLC_RMS_CASE(3) VLC_RMS_CASE(4) VLC_RMS_CASE(5) VLC_RMS_CASE(6)
    VLC_RMS_CASE(7) VLC_RMS_CASE(8)
    case 9: case 10: case 11: case 12:
      return launch_rms<12>(x, x_row_stride, residual, residual_row_stride, residual_out, residual_out_row_stride,
                            weight, eps, num_rows, (int)dim, out, out_row_stride, s);
    default:
      return launch_rms<16>(x, x_row_stride, residual, residual_row_stride, residual_out, residual_out_row_stride,
                            weight, eps, num_rows, (int)dim, out, out_row_stride, s);
  }
#undef VLC_RMS_CASE
}

VLC_API int vlc_silu_mul(const void* gate_up, int64_t gate_up_row_stride, int64_t num_rows, int64_t inter,
                         void* out, int64_t out_row_stride, void* stream) {
  using namespace vlc;
  if (num_rows < 0 || inter <= 0 || inter % 4 != 0) return VLC_ERR_INVALID;
  if (gate_up_row_stride < 2 * inter || out_row_stride < inter) return VLC_ERR_INVALID;
  if (num_rows == 0) return VLC_OK;
  if (!gate_up || !out) return VLC_ERR_INVALID;
  if ((reinterpret_cast<uintptr_t>(gate_up) & 7) || (reinterpret_cast<uintptr_t>(out) & 7) ||
      (gate_up_row_stride % 4) || (out_row_stride % 4))
    return VLC_ERR_UNSUPPORTED;
  // 16-byte accesses when the call is large enough to fill the device with half as
  // many lanes: 1247 x 11008 in 17.2 against 18.9 us, 10741 x 11008 in 125 against
  // 139 us; a decode step's 4 x 18944 measured 2.2 against 2.05 us with them.
  const bool v16 = inter % 8 == 0 && num_rows * inter >= ((int64_t)1 << 20) && aligned16(gate_up) &&
                   aligned16(out) && gate_up_row_stride % 8 == 0 && out_row_stride % 8 == 0;
  const int groups = (int)(inter / (v16 ? 8 : 4));
  const int64_t total = num_rows * groups;
  const int64_t blocks = (total + kThreads - 1) / kThreads;
  if (blocks >= ((int64_t)1 << 31)) return VLC_ERR_UNSUPPORTED;
  if (v16)
    hipLaunchKernelGGL(silu_mul_kernel<8>, dim3((unsigned)blocks), dim3(kThreads), 0, as_stream(stream),
                       static_cast<const char*>(gate_up), gate_up_row_stride * 2, num_rows, groups, inter * 2,
                       static_cast<char*>(out), out_row_stride * 2);
  else
    hipLaunchKernelGGL(silu_mul_kernel<4>, dim3((unsigned)blocks), dim3(kThreads), 0, as_stream(stream),
                       static_cast<const char*>(gate_up), gate_up_row_stride * 2, num_rows, groups, inter * 2,
                       static_cast<char*>(out), out_row_stride * 2);
  return launch_status();
}
