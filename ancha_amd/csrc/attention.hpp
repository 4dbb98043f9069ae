// Shared pieces of the fused attention kernels (attention.hip: short sequences and the
// 16x16x32 long-sequence kernel; attention_long.hip: the 32x32x16 long-sequence kernel).
#pragma once
#include "buffer.hpp"
#include "common.hpp"
#include "kernels.hpp"

namespace ancha {

// Lazy-rescale threshold in log2 units: unnormalised probabilities stay below 2^kTau (fp16-safe).
constexpr float kTau = 8.0f;
// s_waitcnt operand (GFX9 encoding) waiting for all vector memory operations: vmcnt(0),
// expcnt and lgkmcnt left at their maxima.
constexpr int kWaitVmem = 0x0F70;

// Byte offset of 16-byte chunk c (8 fp16 channels) of K row r in a [64][64] fp16 tile.
__device__ __forceinline__ int k_offset(int r, int c) { return r * 128 + ((c ^ (r & 7)) << 4); }

// First row of group g (token 0) in q/k/v/gate/out; token t adds t * p.tstep rows.
__device__ __forceinline__ long group_row(const AttnParams& p, int g) {
  return (long)(g / p.gsplit) * p.gouter + (long)(g % p.gsplit) * p.gstep;
}

// Output rows of one (group, head): [tokens, heads*64] starting at channel 64*h.
struct OutRows {
  rsrc_t out, gate;
  unsigned ld4, ldg4;
  bool half, gate_half;
};

__device__ __forceinline__ OutRows out_rows(const AttnParams& p, int g, int h) {
  const int T = p.tokens;
  const long row = group_row(p, g);
  OutRows o;
  o.half = p.out_half != 0;
  const unsigned esize = o.half ? 2 : 4;
  o.ld4 = (unsigned)(p.tstep * p.heads * 64 * esize);
  o.out = make_rsrc(reinterpret_cast<unsigned char*>(p.out) + (row * p.heads + h) * 64 * esize,
                    (unsigned)(T - 1) * o.ld4 + 64 * esize);
  o.gate_half = p.in_half != 0;
  const unsigned gsize = o.gate_half ? 2 : 4;
  o.ldg4 = (unsigned)(p.tstep * p.ldg * gsize);
  o.gate = make_rsrc(p.gate ? reinterpret_cast<const unsigned char*>(p.gate) +
                                  (row * p.ldg + h) * gsize
                            : reinterpret_cast<const unsigned char*>(p.out),
                     p.gate ? (unsigned)(T - 1) * o.ldg4 + gsize : 0);
  return o;
}

// Long sequences (T > 64) on v_mfma_f32_32x32x16_f16: 16 waves x 32 queries per workgroup.
// fp32 q / k / v (`aligned`: rows, table and output 16-byte aligned; otherwise 4-byte accesses),
// or the block's fp16 projection (in_half, aligned only).
hipError_t launch_attention_long(const AttnParams& p, bool gated, bool rope, bool aligned,
                                 hipStream_t stream);

}  // namespace ancha
