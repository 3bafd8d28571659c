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

// 16-byte store with the nontemporal cache policy (streamed to HBM rather than kept in
// L2 and the MALL).  Inline assembly: the compiler folds the nontemporal builtin's
// store into a plain one where two branches store to different addresses.  The
// compiler does not count this store in its wait counters; stores never feed a
// register, and an extra memory operation in flight only makes its vmcnt waits stricter.
// It does not see the store's hazards either: a VALU write to the data registers of a
// store of more than 8 bytes needs two wait states after it (gfx940 and later), or the
// store can send the new values; the compiler reuses those registers at once.  Hence
// the s_nop 1 inside the statement.
typedef uint32_t u32x4_vec __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void st16_nt(void* p, const u32x4& v) {
  const u32x4_vec w = {v.x, v.y, v.z, v.w};
  asm volatile("global_store_dwordx4 %0, %1, off nt\n\ts_nop 1" : : "v"(p), "v"(w) : "memory");
}

// 16-byte store at agent scope (sc1): written through the XCD's L2 to the memory side,
// so it leaves no dirty line in L2.  Each kernel ends with a write-back of its XCDs'
// dirty L2 lines before the next kernel on the stream starts; a kernel whose output the
// next kernel reads spends that time after its last workgroup.  Measured on the warm
// attention call (main kernel, then the split-KV merge): the gap between the two
// kernels fell from 2.6 to 1.2 us with these stores for the outputs and partials
// (nontemporal stores, which still leave the lines dirty, changed nothing).  Same
// inline-assembly caveats as st16_nt.
__device__ __forceinline__ void st16_wt(void* p, const u32x4_vec& w) {
  asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1" : : "v"(p), "v"(w) : "memory");
}
// 8-byte store at agent scope: the compiler's relaxed atomic store (it tracks its hazards).
__device__ __forceinline__ void st8_wt(void* p, uint64_t bits) {
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Store policies of the bandwidth kernels' 16-byte stores.
enum StoreMode : int { kStPlain = 0, kStNt = 1, kStWt = 2 };

template <int kMode>
__device__ __forceinline__ void st16(void* p, const u32x4& v) {
  if constexpr (kMode == kStNt) {
    st16_nt(p, v);
  } else if constexpr (kMode == kStWt) {
    const u32x4_vec w = {v.x, v.y, v.z, v.w};
    st16_wt(p, w);
  } else {
    *reinterpret_cast<u32x4*>(p) = v;
  }
}

// Store policy by the bytes a call writes.  Agent-scope stores (no dirty L2 lines left
// for the write-back at the kernel's end) up to kWtMaxWriteBytes: the warm request's
// step (re-rotation, then per layer the fused RoPE + store and the attention) as one
// graph took 1.231 against 1.249 ms with them in the fused RoPE + store, and the scatter
// measured 0-7 % faster at 0.5-34 MB; at 168 MB the fused RoPE + store ran 9 % slower
// with them.  Nontemporal stores up to kNtMaxWriteBytes: they ran faster than plain
// ones for calls writing 1-170 MB (e.g. 22 MB of scatter in 3.16 against 4.29 us) and
// slower for larger writes (the 350 MB of K and V written by the re-rotation, the
// 594 MB of vision head rows).  Plain stores above.
constexpr int64_t kWtMaxWriteBytes = (int64_t)64 << 20;
constexpr int64_t kNtMaxWriteBytes = (int64_t)256 << 20;
inline int store_mode_for(int64_t written_bytes) {
  return written_bytes <= kWtMaxWriteBytes ? kStWt : written_bytes <= kNtMaxWriteBytes ? kStNt : kStPlain;
}

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
