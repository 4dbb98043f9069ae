// Axis swap of a [batch, a, b, dim] fp32 tensor into [batch, b, a, dim] for CDNA4 (gfx950):
// the dense `x.swap_dims(..)` copy between the time and band passes of the RoFormer axis loop
// (crates/ancha-models/src/network.rs:336-338, `dense` roformer.rs:57-70). HBM-bound: each
// thread moves 16-byte vectors of one dim-row; rows are contiguous in both layouts.
#include "buffer.hpp"
#include "common.hpp"
#include "kernels.hpp"

namespace ancha {
namespace {

// One block per 4 output rows (one wave each): out row (n, j, i) <- in row (n, i, j).
template <bool ALIGNED>
__global__ __launch_bounds__(256) void swap_axes_kernel(SwapParams p) {
  const long orow = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const long rows = (long)p.batch * p.a * p.b;
  if (orow >= rows) return;
  const int lane = threadIdx.x & 63;
  const long n = orow / ((long)p.a * p.b), rem = orow % ((long)p.a * p.b);
  const long j = rem / p.a, i = rem % p.a;  // output row index (n, j, i) of [batch, b, a]
  const long irow = (n * p.a + i) * p.b + j;
  const rsrc_t src = make_rsrc(p.x + irow * p.dim, (unsigned)p.dim * 4);
  const rsrc_t dst = make_rsrc(p.out + orow * p.dim, (unsigned)p.dim * 4);
  if constexpr (ALIGNED) {
    for (int c = 4 * lane; c < p.dim; c += 256) bstore4<true>(dst, c * 4, bload4<true>(src, c * 4));
  } else {
    for (int c = lane; c < p.dim; c += 64)
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_amdgcn_raw_buffer_load_b32(src, c * 4, 0, 0),
                                            dst, c * 4, 0, 0);
  }
}

}  // namespace

hipError_t launch_swap_axes(const SwapParams& p, bool aligned, hipStream_t stream) {
  const long rows = (long)p.batch * p.a * p.b;
  const dim3 grid((unsigned)((rows + 3) / 4)), block(256);
  if (aligned)
    hipLaunchKernelGGL(swap_axes_kernel<true>, grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL(swap_axes_kernel<false>, grid, block, 0, stream, p);
  return hipGetLastError();
}

}  // namespace ancha
