// Shared helpers for the gfx950 kernels behind include/vlc_capi.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vlc_capi.h"

#define VLC_API extern "C" __attribute__((visibility("default")))

namespace vlc {

// 16-byte vector used for every coalesced global load/store in the bandwidth kernels.
struct alignas(16) u32x4 {
  uint32_t x, y, z, w;
};

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? VLC_OK : static_cast<int>(e);
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// bf16 <-> fp32 by bit manipulation (round to nearest even, NaN kept quiet).
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return ((u >> 16) | 0x40u) & 0xffffu;  // NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

}  // namespace vlc
