// Device helpers shared by the CDNA4 (gfx950) kernels: fp16 operand packing, the 16x16x32 fp16
// MFMA with its register fragments, wave reductions and the XCD-aware block remap.
//
// MFMA operands are IEEE fp16 (11-bit significand, 8x finer than bf16 at the same MFMA rate),
// products accumulate in fp32. Operand values must stay below 65504 in magnitude.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ancha {

typedef _Float16 h16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 h16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
// Finite stand-in for -inf in the log2-domain softmax: exp2(kMasked - m) is exactly 0.
constexpr float kMasked = -1.0e30f;
// MI355X has 8 XCDs; consecutive workgroup ids are dealt round-robin across them.
constexpr int kXcds = 8;

// Two fp32 -> one dword of two fp16 (round to nearest even; v_cvt_pk_f16_f32).
__device__ __forceinline__ unsigned pack_h2(float a, float b) {
  h16x2 r;
  r[0] = (_Float16)a;
  r[1] = (_Float16)b;
  return __builtin_bit_cast(unsigned, r);
}

// D(16x16 fp32) += A(16x32 fp16) . B(32x16 fp16).
// Lane l holds A[row l%16][k 8*(l/16)..+7], B[k 8*(l/16)..+7][col l%16] and
// D[rows 4*(l/16)..+3][col l%16].
__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h16x8, a),
                                                __builtin_bit_cast(h16x8, b), c, 0, 0, 0);
}

typedef float f32x16 __attribute__((ext_vector_type(16)));

// D(32x32 fp32) += A(32x16 fp16) . B(16x32 fp16).
// Lane l holds A[row l%32][k 8*(l/32)..+7], B[k 8*(l/32)..+7][col l%32] and, in element
// 4q + e, D[row 8q + 4*(l/32) + e][col l%32].
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h16x8, a),
                                                __builtin_bit_cast(h16x8, b), c, 0, 0, 0);
}

// Zero accumulator for the first mfma32 of a chain, built in registers behind an empty asm so
// that the compiler cannot fold it into the MFMA's inline-constant C operand. In that form the
// compiler may give the MFMA a destination overlapping its A or B registers, and the 8-pass
// MFMA then overwrites operand registers it has not finished reading (wrong products, varying
// from run to run). A register C is tied to the destination, which keeps it apart from A and B.
__device__ __forceinline__ f32x16 mfma32_zero() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; i++) z[i] = 0.f;
  asm volatile("" : "+v"(z));
  return z;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// True for +-inf and NaN. The library is compiled with -fno-honor-nans, under which the
// compiler folds isfinite() and even an exponent bit test on a float to an infinity compare
// (NaN assumed absent); the empty asm hides the value's float origin, so the bit test stays.
__device__ __forceinline__ bool non_finite(float x) {
  unsigned bits = __builtin_bit_cast(unsigned, x);
  asm volatile("" : "+v"(bits));
  return (bits & 0x7f800000u) == 0x7f800000u;
}

// ORs `bit` into the device check word (a vector-memory atomic).
__device__ __forceinline__ void raise_flag(unsigned* flags, unsigned bit) {
  __hip_atomic_fetch_or(flags, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Maximum over the four lanes {l, l^16, l^32, l^48} that share a column of an MFMA tile.
__device__ __forceinline__ float max_over_rows(float x) {
  x = fmaxf(x, __shfl_xor(x, 16));
  return fmaxf(x, __shfl_xor(x, 32));
}

// Bijection from the hardware workgroup id to a logical id such that each XCD runs one
// contiguous range of logical ids (so blocks that share inputs share that XCD's L2).
__device__ __forceinline__ int xcd_remap(int b, int n) {
  const int per = n / kXcds, rem = n % kXcds;
  const int xcd = b % kXcds, idx = b / kXcds;
  return xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
}

// Interleaved-pair rotation of 4 consecutive channels (two pairs):
// y = x*cos + swap_pairs(x)*sin, the pair sign folded into sin. The fused multiply-add is
// written out, so every call site rounds the same way (left to the compiler, the contraction of
// the two products can differ between inlined copies and move a rotated value by one ulp).
__device__ __forceinline__ float4 rotate4(float4 x, float4 c, float4 s) {
  float4 y;
  y.x = __builtin_fmaf(x.x, c.x, x.y * s.x);
  y.y = __builtin_fmaf(x.y, c.y, x.x * s.y);
  y.z = __builtin_fmaf(x.z, c.z, x.w * s.z);
  y.w = __builtin_fmaf(x.w, c.w, x.z * s.w);
  return y;
}

__device__ __forceinline__ float4 scale4(float4 x, float s) {
  return make_float4(x.x * s, x.y * s, x.z * s, x.w * s);
}

}  // namespace ancha
