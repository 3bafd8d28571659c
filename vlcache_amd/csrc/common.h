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

// bf16 <-> fp32.  bf16 -> fp32 is a shift; fp32 -> bf16 rounds to nearest even with
// the hardware conversion (v_cvt_pk_bf16_f32; NaN stays NaN), which measured about
// twice as fast as the same rounding done with integer operations in the
// instruction-bound RMSNorm and rotation kernels.
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

}  // namespace vlc
