// Row L2 normalisation for CDNA4 (gfx950): out[r] = x[r] / max(||x[r]||_2, 1e-12) * scale.
// Replaces `unit_norm` (crates/ancha-models/src/roformer.rs:16-24) and `SourceNorm::forward`
// (:43-54, scale = sqrt(dim) * gamma) on the GPU path, where the reference runs them as
// separate Burn ops (roformer.rs:478,497,516-519).
//
// One wave per row. Pass 1 sums squares (fp32, per-lane partials then a wave reduction);
// pass 2 re-reads the row (from L2: a row is at most a few KB), scales and writes it. Each lane
// reads and writes the same elements in both passes, so out may alias x. HBM-bound: one read
// and one write of the row.
#include "buffer.hpp"
#include "common.hpp"
#include "kernels.hpp"

namespace ancha {
namespace {

constexpr int kRowsPerBlock = 4;

template <bool ALIGNED>
__global__ __launch_bounds__(256) void unit_norm_kernel(NormParams p) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= p.rows) return;
  const int dim = p.dim;
  const rsrc_t xr = make_rsrc(p.x + (long)row * p.ldx, (unsigned)dim * 4);
  const rsrc_t outr = make_rsrc(p.out + (long)row * dim, (unsigned)dim * 4);
  const rsrc_t sr = make_rsrc(p.scale ? p.scale : p.out, p.scale ? (unsigned)dim * 4 : 0u);
  float ss = 0.f;
  if constexpr (ALIGNED) {
    for (int c = 4 * lane; c < dim; c += 256) {
      const float4 v = bload4<true>(xr, c * 4);
      ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
  } else {
    for (int c = lane; c < dim; c += 64) {
      const float v = bload1(xr, c * 4);
      ss += v * v;
    }
  }
  for (int o = 1; o < 64; o <<= 1) ss += __shfl_xor(ss, o);
  const float inv = 1.0f / fmaxf(sqrtf(ss), 1e-12f);
  if constexpr (ALIGNED) {
    for (int c = 4 * lane; c < dim; c += 256) {
      float4 v = scale4(bload4<true>(xr, c * 4), inv);
      if (p.scale) {
        const float4 s = bload4<true>(sr, c * 4);
        v = make_float4(v.x * s.x, v.y * s.y, v.z * s.z, v.w * s.w);
      }
      bstore4<true>(outr, c * 4, v);
    }
  } else {
    for (int c = lane; c < dim; c += 64) {
      float v = bload1(xr, c * 4) * inv;
      if (p.scale) v *= bload1(sr, c * 4);
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), outr, c * 4, 0, 0);
    }
  }
}

}  // namespace

hipError_t launch_unit_norm(const NormParams& p, bool aligned, hipStream_t stream) {
  const dim3 grid((p.rows + kRowsPerBlock - 1) / kRowsPerBlock), block(64 * kRowsPerBlock);
  if (aligned)
    hipLaunchKernelGGL(unit_norm_kernel<true>, grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL(unit_norm_kernel<false>, grid, block, 0, stream, p);
  return hipGetLastError();
}

}  // namespace ancha
