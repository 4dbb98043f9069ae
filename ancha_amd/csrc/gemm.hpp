// Tile constants and helpers shared by the projection GEMM kernels (linear.hip, gemm16.hip).
#pragma once
#include <hip/hip_runtime.h>

#include "buffer.hpp"
#include "common.hpp"

namespace ancha {
namespace gemm {

constexpr int kBM = 128;  // output rows per workgroup
constexpr int kBN = 128;  // output columns per workgroup
constexpr int kBK = 64;   // k per LDS stage
constexpr int kThreads = 256;
constexpr int kTileBytes = kBM * kBK * 2;  // one fp16 [128][64] tile

__device__ __forceinline__ int swz(int r) { return (r ^ (r >> 2)) & 7; }
// Byte offset of 16-byte chunk c (k = 8c..8c+7) of row r in a [128][64] fp16 tile.
__device__ __forceinline__ int tile_offset(int r, int c) { return r * 128 + ((c ^ swz(r)) << 4); }

__device__ __forceinline__ float gelu_erf(float x) {
  return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f));
}

// Four consecutive floats at element `col` of a row, zero for elements at or past `limit`
// (the unaligned path handles each element; the aligned path has limit % 4 == 0).
template <bool ALIGNED>
__device__ __forceinline__ float4 load_masked(rsrc_t r, unsigned off, int col, int limit) {
  float4 v = bload4<ALIGNED>(r, off);
  if constexpr (ALIGNED) {
    if (col >= limit) v = make_float4(0.f, 0.f, 0.f, 0.f);
  } else {
    if (col >= limit) v.x = 0.f;
    if (col + 1 >= limit) v.y = 0.f;
    if (col + 2 >= limit) v.z = 0.f;
    if (col + 3 >= limit) v.w = 0.f;
  }
  return v;
}

template <bool ALIGNED>
__device__ __forceinline__ void store_masked(rsrc_t r, unsigned off, int col, int limit, float4 v) {
  if constexpr (ALIGNED) {
    if (col < limit) bstore4<true>(r, off, v);
  } else {
    const u32x4 u = __builtin_bit_cast(u32x4, v);
    for (int j = 0; j < 4; j++)
      if (col + j < limit) __builtin_amdgcn_raw_buffer_store_b32(u[j], r, off + 4 * j, 0, 0);
  }
}

}  // namespace gemm
}  // namespace ancha
