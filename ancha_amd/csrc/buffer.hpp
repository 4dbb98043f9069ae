// Raw buffer access helpers shared by the gfx950 kernels: wave-uniform buffer descriptors whose
// hardware range check zero-fills loads past the end and drops stores there.
#pragma once
#include <hip/hip_runtime.h>

#include "common.hpp"

namespace ancha {

typedef __amdgpu_buffer_rsrc_t rsrc_t;

// Raw buffer over [base, base + bytes): loads past the end return 0, stores there are dropped.
// Callers pass wave-uniform values; readfirstlane states that, so the descriptor lives in SGPRs
// (a descriptor the compiler believes divergent costs a readfirstlane loop per access).
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, unsigned bytes) {
  const unsigned long long a = reinterpret_cast<unsigned long long>(base);
  const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)a);
  const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(a >> 32));
  void* uniform = reinterpret_cast<void*>(((unsigned long long)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(uniform, 0, __builtin_amdgcn_readfirstlane(bytes),
                                           0x00020000);
}

// Cache policy of a buffer access (gfx950): 0 = default; kStream = non-temporal, for data that
// is read or written exactly once (streamed past the caches' reuse).
constexpr int kStream = 2;

template <bool ALIGNED, int CP = 0>
__device__ __forceinline__ float4 bload4(rsrc_t r, unsigned off) {
  if constexpr (ALIGNED) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, CP));
  } else {
    return make_float4(__builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, CP)),
                       __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off + 4, 0, CP)),
                       __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off + 8, 0, CP)),
                       __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off + 12, 0, CP)));
  }
}

template <bool ALIGNED, int CP = 0>
__device__ __forceinline__ void bstore4(rsrc_t r, unsigned off, float4 v) {
  if constexpr (ALIGNED) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, CP);
  } else {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v.x), r, off, 0, CP);
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v.y), r, off + 4, 0, CP);
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v.z), r, off + 8, 0, CP);
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v.w), r, off + 12, 0, CP);
  }
}

__device__ __forceinline__ float bload1(rsrc_t r, unsigned off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

__device__ __forceinline__ float comp(float4 v, int j) {
  return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w;
}

}  // namespace ancha
