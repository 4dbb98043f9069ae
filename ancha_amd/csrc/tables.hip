// Small per-forward tables built on the device, so that a forward over a frame count the model
// was not created for allocates nothing and does not wait on the host: the packed rotary
// tables of each axis layer and the tile tables of the mask heads' grouped product.
#include "kernels.hpp"

namespace ancha {
namespace {

// AxisRope::new (crates/ancha-models/src/roformer.rs:282-302): one thread per (set, t, i),
// writing entry i of token t in all four tables: query cos and signed sin (times 1/sqrt(64)),
// key cos and signed sin. Channel pairs (2j, 2j+1) share the angle f32(t) * freqs[j]; the
// first channel of a pair carries -sin, the second +sin.
__global__ void axis_rope_kernel(const float* freqs, int sets, int tokens, float* out) {
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long per_set = (long)tokens * 64;
  if (idx >= per_set * sets) return;
  const int set = (int)(idx / per_set);
  const int t = (int)((idx % per_set) / 64), i = (int)(idx % 64);
  const float angle = (float)t * freqs[set * 32 + i / 2];
  float s, c;
  sincosf(angle, &s, &c);
  const float sn = (i & 1) ? s : -s;
  float* o = out + (long)set * 4 * per_set + (long)t * 64 + i;
  o[0] = c * 0.125f;
  o[per_set] = sn * 0.125f;
  o[2 * per_set] = c;
  o[3 * per_set] = sn;
}

// first[b] = row_tiles * col0[b] / 128 for b <= bands; of_tile[t] = the band whose range holds
// tile t.
__global__ void group_tiles_kernel(const long* col0, int bands, int row_tiles, int* of_tile,
                                   int* first) {
  const long total = (long)row_tiles * (col0[bands] / 128);
  const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (t <= bands) first[t] = (int)((long)row_tiles * (col0[t] / 128));
  if (t >= total) return;
  int b = 0;
  while (b + 1 < bands && (long)row_tiles * (col0[b + 1] / 128) <= t) b++;
  of_tile[t] = b;
}

}  // namespace

hipError_t launch_axis_rope(const float* freqs, int sets, int tokens, float* out,
                            hipStream_t stream) {
  const long n = (long)sets * tokens * 64;
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(axis_rope_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                     freqs, sets, tokens, out);
  return hipGetLastError();
}

hipError_t launch_group_tiles(const long* col0, int bands, int row_tiles, long total,
                              int* of_tile, int* first, hipStream_t stream) {
  const long n = total > bands + 1 ? total : bands + 1;
  hipLaunchKernelGGL(group_tiles_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                     col0, bands, row_tiles, of_tile, first);
  return hipGetLastError();
}

}  // namespace ancha
