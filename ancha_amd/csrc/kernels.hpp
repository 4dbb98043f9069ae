// Kernel parameter blocks and host launchers of the HIP kernels (internal to the library; the
// public surface is the C ABI in include/ancha_hip.h).
#pragma once
#include <hip/hip_runtime.h>

namespace ancha {

// softmax(q.k^T).v per (group, head). q/k/v/gate point at the column of head 0 inside
// [groups, tokens, ld*] row-major buffers (head h at +64h, group stride tokens*ld).
struct AttnParams {
  const float* q;
  const float* k;
  const float* v;
  const float* gate;  // per-head gate logits (head h at +h), or null
  const float* rope;  // packed [4, tokens, 64] table, or null (q/k already rotated, q scaled)
  float* out;         // [groups, tokens, heads, 64] contiguous
  long ldq, ldk, ldv, ldg;
  int groups, tokens, heads;
};

// `aligned`: every float4 access is 16-byte aligned (base pointers and row strides).
hipError_t launch_attention(const AttnParams& p, bool aligned, hipStream_t stream);

}  // namespace ancha
