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

// erf-GELU for epilogues whose result is rounded to fp16: erfc(z) from Abramowitz & Stegun,
// Handbook of Mathematical Functions, formula 7.1.26 (Hastings' rational approximation,
// |error| <= 1.5e-7 in erf), with t = 1 / (1 + p z) and exp(-z^2) on the hardware exp2 and
// reciprocal. GELU(x) = x - x/2 erfc(x/sqrt2) for x >= 0 and x/2 erfc(-x/sqrt2) below, so the
// negative tail keeps its relative accuracy.
// The constants are folded for the VALU: p / sqrt2 multiplies |x| directly, the polynomial
// carries the factor 1/2 (so q = erfc(|x|/sqrt2) / 2 is two multiplies), and
// exp(-z^2) = exp2(x^2 * (-log2(e) / 2)). Both branches are max(x, 0) - |x| q: x - x q for
// x >= 0, x q below; one fused multiply-add with the sign and magnitude as operand modifiers.
__device__ __forceinline__ float gelu_fast(float x) {
  const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f * 0.70710678118654752f, fabsf(x), 1.0f));
  float poly = fmaf(t, 0.5f * 1.061405429f, 0.5f * -1.453152027f);
  poly = fmaf(t, poly, 0.5f * 1.421413741f);
  poly = fmaf(t, poly, 0.5f * -0.284496736f);
  poly = fmaf(t, poly, 0.5f * 0.254829592f);
  const float e = __builtin_amdgcn_exp2f(x * -0.72134752044448170f * x);
  return fmaf(-fabsf(x), poly * t * e, fmaxf(x, 0.0f));
}

// tanh as 1 - 2 / (e^{2|x|} + 1) with the sign restored; below |x| = 2^-8 the series
// x (1 - x^2/3) (the cancellation in the first form would cost relative accuracy there).
__device__ __forceinline__ float tanh_fast(float x) {
  const float a = fabsf(x);
  const float e = __builtin_amdgcn_exp2f(a * 2.88539008177792682f);
  const float r = 1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f);
  const float small = x * fmaf(x * x, -0.333333333f, 1.0f);
  return a < 0.00390625f ? small : copysignf(r, x);
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
