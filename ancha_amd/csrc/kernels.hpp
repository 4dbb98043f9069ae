// Kernel parameter blocks and host launchers of the HIP kernels (internal to the library; the
// public surface is the C ABI in include/ancha_hip.h).
#pragma once
#include <hip/hip_runtime.h>

namespace ancha {

// softmax(q.k^T).v per (group, head). q/k/v/gate point at the column of head 0 inside
// row-major buffers (head h at +64h). Token t of group g sits in row
//   (g / gsplit) * gouter + (g % gsplit) * gstep + t * tstep
// of q/k/v/gate (row stride ld*) and of out (row stride heads*64): gsplit 1, gouter tokens,
// gstep 0, tstep 1 for groups of contiguous tokens ([groups, tokens, ...]); gsplit frames,
// gouter bands*frames, gstep 1, tstep frames for the band axis of a [batch, bands, frames, ...]
// buffer (group = batch*frames + frame, token = band). gsplit 0 means contiguous groups.
struct AttnParams {
  const float* q;
  const float* k;
  const float* v;
  const float* gate;  // per-head gate logits (head h at +h), or null
  const float* rope;  // packed [4, tokens, 64] table, or null (q/k already rotated, q scaled)
  float* out;         // [groups, tokens, heads, 64] contiguous (fp16 values if out_half)
  long ldq, ldk, ldv, ldg;
  int groups, tokens, heads;
  int out_half;       // store the output as fp16 (the block's internal activation)
  int gsplit;
  long gouter, gstep, tstep;
};

// `aligned`: every float4 access is 16-byte aligned (base pointers and row strides).
hipError_t launch_attention(const AttnParams& p, bool aligned, hipStream_t stream);

// out = epilogue(x . w): x [n, k] (row stride ldx), w [k, m] row-major (the reference's
// [in, out] Linear layout), out [n, m] contiguous. Epilogue, in order: optional input row norm
// (the product of row r scaled by 1 / max(||x_r||, 1e-12)), bias [m], erf-GELU, interleaved
// rotary on columns [0, 2*width) (queries then keys of token r % tokens, packed [4, tokens, 64]
// table), residual [n, m] contiguous.
struct LinearParams {
  const float* x;
  const float* w;
  const float* bias;      // or null
  const float* rope;      // or null
  const float* residual;  // or null (may alias out)
  float* out;
  long ldx;
  int n, k, m;
  int tokens, width;
  int gelu;
  int norm;
};

// `aligned`: x, w, out (and bias / residual / rope when present) are 16-byte aligned, ldx and m
// are multiples of 4.
hipError_t launch_linear(const LinearParams& p, bool aligned, hipStream_t stream);

// out[r] = x[r] / max(||x[r]||, 1e-12) * scale (scale [dim] or null): x [rows, dim] with row
// stride ldx, out [rows, dim] contiguous; out may alias x when ldx == dim.
struct NormParams {
  const float* x;
  const float* scale;
  float* out;
  long ldx;
  int rows, dim;
};

hipError_t launch_unit_norm(const NormParams& p, bool aligned, hipStream_t stream);

// The block's projection GEMM on load-time fp16 weights: out = epilogue(x . W) with W^T fp16
// [m][k] (k contiguous, the PyTorch [out, in] layout), x fp32 or fp16 (x_half) [n][k] with row
// stride ldx, out fp32 or fp16 (out_half) [n][m] contiguous; bias, rope, residual (fp32) and
// the row norm as in LinearParams. Requires m % 128 == 0, k % 8 == 0, 16-byte aligned rows.
struct Gemm16Params {
  const void* x;
  const _Float16* wt;
  const float* bias;
  const float* rope;
  const float* residual;
  void* out;
  long ldx;
  int n, k, m;
  int tokens, width;
  int token_div;  // rotary position of row r: (r / token_div) % tokens
  int gelu, norm, x_half, out_half;
};

hipError_t launch_gemm16(const Gemm16Params& p, hipStream_t stream);

// out [batch, b, a, dim] = x [batch, a, b, dim] with axes 1 and 2 swapped (both contiguous).
struct SwapParams {
  const float* x;
  float* out;
  int batch, a, b, dim;
};

hipError_t launch_swap_axes(const SwapParams& p, bool aligned, hipStream_t stream);

}  // namespace ancha
