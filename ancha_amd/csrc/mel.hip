// Band split and mask-estimator output of the Mel/BS-RoFormer (gfx950): the two ends of the
// network around the axis loop of transformer blocks (crates/ancha-models/src/network.rs).
//
//  * band_split_kernel (network.rs:316-323): for band b and a tile of frames, gather the
//    band's 4 columns per FFT bin from the packed spectrum [frames][cols] into LDS, take each
//    frame's 1 / max(||z||, 1e-12) (unit_norm, roformer.rs:16-24) and project with the folded
//    weight (sqrt(width)*gamma already in its rows, network.rs:104-110) in fp32:
//    x[b][t][d] = inv_t * sum_c W'[c][d] z[t][c] + bias[b][d]. W' is stored [width][dim] so
//    the threads of a workgroup (one output channel d each) read consecutive addresses.
//  * glu_gather_kernel (network.rs:381-396): mask = value * sigmoid(gate) from the per-band
//    output projections, summed over the bands that cover each FFT bin and divided by their
//    number, written in the reference's [row = 2*bin + channel][re, im][frame] layout.
//    Each output gathers its 1..k covering bands from a host-built table (no atomics, the
//    summation order is the band order).
#include "kernels.hpp"

namespace ancha {
namespace {

constexpr int kSplitFrames = 16;     // frames per workgroup at most
constexpr int kSplitThreads = 256;
constexpr int kSplitLds = 48 * 1024;  // LDS for the gathered features

__global__ __launch_bounds__(kSplitThreads) void band_split_kernel(BandSplitParams p) {
  extern __shared__ float z[];  // [tile][max_width] then inv[tile]
  const int tile = p.tile;     // frames per workgroup: kSplitLds / (4 * max_width), <= 16
  const int b = blockIdx.x, t0 = blockIdx.y * tile;
  const int q0 = p.offsets[b], nb = p.offsets[b + 1] - q0, width = 4 * nb;
  const int frames = min(tile, p.frames - t0);
  float* inv = z + tile * p.max_width;
  // Gather: one float4 (the bin's 4 columns) per (frame, bin).
  for (int e = threadIdx.x; e < frames * nb; e += kSplitThreads) {
    const int tt = e / nb, q = e % nb;
    const float4 v = *reinterpret_cast<const float4*>(
        p.spectrum + (long)(t0 + tt) * p.cols + 4 * p.bins[q0 + q]);
    *reinterpret_cast<float4*>(z + tt * p.max_width + 4 * q) = v;
  }
  __syncthreads();
  // Row norms: wave w takes frames w, w + 4, ...
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int tt = wave; tt < frames; tt += kSplitThreads / 64) {
    float s = 0.0f;
    for (int c = lane; c < width; c += 64) s += z[tt * p.max_width + c] * z[tt * p.max_width + c];
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    if (lane == 0) inv[tt] = 1.0f / fmaxf(sqrtf(s), 1e-12f);
  }
  __syncthreads();
  const float* w = p.weight + (long)p.wofs[b] * p.dim;
  for (int d = threadIdx.x; d < p.dim; d += kSplitThreads) {
    float acc[kSplitFrames];
#pragma unroll
    for (int tt = 0; tt < kSplitFrames; tt++) acc[tt] = 0.0f;
    for (int c = 0; c < width; c++) {
      const float wc = w[(long)c * p.dim + d];
#pragma unroll
      for (int tt = 0; tt < kSplitFrames; tt++)
        if (tt < frames) acc[tt] += wc * z[tt * p.max_width + c];
    }
    const float bias = p.bias[(long)b * p.dim + d];
    for (int tt = 0; tt < frames; tt++)
      p.x[((long)b * p.frames + t0 + tt) * p.dim + d] = acc[tt] * inv[tt] + bias;
  }
}

__global__ void glu_gather_kernel(GluParams p) {
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long total = (long)p.outputs * p.frames;
  if (idx >= total) return;
  const int t = (int)(idx % p.frames), o = (int)(idx / p.frames);
  const int f = o >> 2, within = o & 3;  // column 2*channel + re/im of bin f
  const int e0 = p.cover_start[f], e1 = p.cover_start[f + 1];
  float sum = 0.0f;
  for (int e = e0; e < e1; e++) {
    const int b = p.cover_band[e], col = 4 * p.cover_local[e] + within;
    const float* row = p.glu + p.band_base[b] * p.frames + (long)t * p.band_stride[b];
    const float value = row[col], gate = row[p.band_width[b] + col];
    sum += value * (1.0f / (1.0f + expf(-gate)));
  }
  p.masks[(long)o * p.frames + t] = sum / (float)(e1 - e0);
}

}  // namespace

hipError_t launch_band_split(const BandSplitParams& params, hipStream_t stream) {
  BandSplitParams p = params;
  if (p.max_width <= 0 || 4 * p.max_width > kSplitLds) return hipErrorInvalidValue;
  p.tile = min(kSplitFrames, kSplitLds / (4 * p.max_width));
  const dim3 grid(p.bands, (p.frames + p.tile - 1) / p.tile);
  const size_t lds = sizeof(float) * ((size_t)p.tile * p.max_width + p.tile);
  hipLaunchKernelGGL(band_split_kernel, grid, dim3(kSplitThreads), lds, stream, p);
  return hipGetLastError();
}

hipError_t launch_glu_gather(const GluParams& p, hipStream_t stream) {
  const long total = (long)p.outputs * p.frames;
  hipLaunchKernelGGL(glu_gather_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     stream, p);
  return hipGetLastError();
}

}  // namespace ancha
