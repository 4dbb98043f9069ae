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
#include "common.hpp"
#include "kernels.hpp"

namespace ancha {
namespace {

constexpr int kSplitFrames = 32;   // frames per workgroup
constexpr int kSplitThreads = 256;
constexpr int kSplitCols = 256;    // feature columns staged per pass (32 KB of LDS)
constexpr int kSplitDims = 4;      // output channels per thread (one float4 of W')
constexpr int kSplitHalf = kSplitFrames / 2;  // frames per thread job
constexpr int kSplitJobs = 2 * 512 / kSplitDims;  // (channel group, frame half) pairs, dim <= 512

// Thread job (dg, half): channels 4*dg .. 4*dg+3 for frames 16*half .. 16*half+15 of the tile.
// The band's features pass through LDS transposed, zt[column][frame], kSplitCols columns at a
// time, so a thread reads its 16 frames of a column as four 16-byte words and its 4 weights as
// one: 64 FMAs per 5 loads. Squared norms accumulate over the passes; 1/norm is applied last.
// 32 frames per workgroup amortise the gather of the band's spectrum columns (two dependent
// global reads) over twice the arithmetic of a 16-frame tile; the workgroup has one thread per
// job (192 at dim 384).
__global__ __launch_bounds__(kSplitThreads) void band_split_kernel(BandSplitParams p) {
  __shared__ __attribute__((aligned(16))) float zt[kSplitCols * kSplitFrames];
  __shared__ float sq[kSplitFrames];
  // Bands run high to low: both band layouts list them by frequency, so the widest (the
  // longest workgroups) are dispatched first and the narrow ones fill in behind them.
  const int b = p.bands - 1 - (int)blockIdx.y, t0 = blockIdx.x * kSplitFrames;
  const int q0 = p.offsets[b], nb = p.offsets[b + 1] - q0, width = 4 * nb;
  const int frames = min(kSplitFrames, p.frames - t0);
  const float* w = p.weight + (long)p.wofs[b] * p.dim;
  const int groups = p.dim / kSplitDims;
  const int job = threadIdx.x;
  const bool active = job < 2 * groups;
  const int dg = job % groups, half = job / groups, d0 = kSplitDims * dg;
  if (threadIdx.x < kSplitFrames) sq[threadIdx.x] = 0.0f;
  float acc[kSplitHalf][kSplitDims];
#pragma unroll
  for (int i = 0; i < kSplitHalf; i++)
#pragma unroll
    for (int j = 0; j < kSplitDims; j++) acc[i][j] = 0.0f;
  for (int c0 = 0; c0 < width; c0 += kSplitCols) {
    const int cols = min(kSplitCols, width - c0), bins = cols / 4;
    __syncthreads();  // the previous pass is done with zt
    for (int e = threadIdx.x; e < kSplitFrames * bins; e += blockDim.x) {
      const int tt = e % kSplitFrames, q = e / kSplitFrames;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (tt < frames)
        v = *reinterpret_cast<const float4*>(p.spectrum + (long)(t0 + tt) * p.cols +
                                             4 * p.bins[q0 + c0 / 4 + q]);
      zt[(4 * q + 0) * kSplitFrames + tt] = v.x;
      zt[(4 * q + 1) * kSplitFrames + tt] = v.y;
      zt[(4 * q + 2) * kSplitFrames + tt] = v.z;
      zt[(4 * q + 3) * kSplitFrames + tt] = v.w;
    }
    __syncthreads();
    // squared norms: 16 lanes per frame
    for (int tt = threadIdx.x >> 4; tt < kSplitFrames; tt += blockDim.x / 16) {
      const int l = threadIdx.x & 15;
      float s = 0.0f;
      for (int c = l; c < cols; c += 16) s += zt[c * kSplitFrames + tt] * zt[c * kSplitFrames + tt];
      for (int o = 8; o > 0; o >>= 1) s += __shfl_xor(s, o);
      if (l == 0) sq[tt] += s;
    }
    if (active) {
      const float* zc = zt + half * kSplitHalf;
      const float* wc = w + (long)c0 * p.dim + d0;
      // Weight rows stream through a ring of kRing registers, kRing columns ahead of their FMAs.
      constexpr int kRing = 8;
      float4 ring[kRing];
#pragma unroll
      for (int u = 0; u < kRing; u++)
        if (u < cols) ring[u] = *reinterpret_cast<const float4*>(wc + (long)u * p.dim);
      for (int cb = 0; cb < cols; cb += kRing) {
#pragma unroll
        for (int u = 0; u < kRing; u++) {
          const int c = cb + u;
          if (c >= cols) break;
          const float4 wv = ring[u];
          if (c + kRing < cols)
            ring[u] = *reinterpret_cast<const float4*>(wc + (long)(c + kRing) * p.dim);
          float zz[kSplitHalf];
#pragma unroll
          for (int k = 0; k < kSplitHalf / 4; k++) {
            const float4 z = *reinterpret_cast<const float4*>(zc + c * kSplitFrames + 4 * k);
            zz[4 * k] = z.x;
            zz[4 * k + 1] = z.y;
            zz[4 * k + 2] = z.z;
            zz[4 * k + 3] = z.w;
          }
          const float ww[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
          for (int i = 0; i < kSplitHalf; i++)
#pragma unroll
            for (int j = 0; j < kSplitDims; j++) acc[i][j] += ww[j] * zz[i];
        }
      }
    }
  }
  __syncthreads();
  if (active) {
    const float4 bias = *reinterpret_cast<const float4*>(p.bias + (long)b * p.dim + d0);
    for (int i = 0; i < kSplitHalf; i++) {
      const int tt = half * kSplitHalf + i;
      if (tt >= frames) break;
      const float s = 1.0f / fmaxf(sqrtf(sq[tt]), 1e-12f);
      *reinterpret_cast<float4*>(p.x + ((long)b * p.frames + t0 + tt) * p.dim + d0) =
          make_float4(acc[i][0] * s + bias.x, acc[i][1] * s + bias.y, acc[i][2] * s + bias.z,
                      acc[i][3] * s + bias.w);
    }
  }
}

// One workgroup per tile of 64 outputs x 64 frames. Lanes run along the outputs, so a wave
// reads consecutive columns of one band row (the rows are frame-major); the tile is transposed
// through LDS and written frame-contiguous, each wave storing whole 256-byte rows.
constexpr int kGluTile = 64;
__global__ __launch_bounds__(256) void glu_gather_kernel(GluParams p) {
  __shared__ float tile[kGluTile][kGluTile + 1];
  const int o0 = blockIdx.x * kGluTile, t0 = blockIdx.y * kGluTile;
  const int lane = threadIdx.x & 63, sub = threadIdx.x >> 6;
  const int o = o0 + lane;
  if (o < p.outputs) {
    const int f = o >> 2, within = o & 3;  // column 2*channel + re/im of bin f
    const int e0 = p.cover_start[f], e1 = p.cover_start[f + 1];
    const int nt = min(kGluTile / 4, (p.frames - t0 - sub + 3) / 4);  // frames t0 + sub + 4 i
    float sum[kGluTile / 4];
#pragma unroll
    for (int i = 0; i < kGluTile / 4; i++) sum[i] = 0.0f;
    // Covering bands in order (the summation order of the reference), each band's row pointer
    // and gate offset read once for the tile's 16 frames of this thread.
    for (int e = e0; e < e1; e++) {
      const int b = p.cover_band[e], col = 4 * p.cover_local[e] + within;
      const long stride = p.band_stride[b];
      const float* row = p.glu + p.band_base[b] * p.frames + (long)(t0 + sub) * stride + col;
      const int gate = p.band_width[b];
#pragma unroll
      for (int i = 0; i < kGluTile / 4; i++)
        if (i < nt) {
          const float* r = row + (long)(4 * i) * stride;
          sum[i] += r[0] * (1.0f / (1.0f + expf(-r[gate])));
        }
    }
    const float count = (float)(e1 - e0);
#pragma unroll
    for (int i = 0; i < kGluTile / 4; i++)
      if (i < nt) {
        const float mask = sum[i] / count;
        if (p.flags && non_finite(mask)) raise_flag(p.flags, kFlagMasks);
        tile[lane][sub + 4 * i] = mask;
      }
  }
  __syncthreads();
  for (int r = sub; r < kGluTile; r += 4) {
    const int oo = o0 + r, t = t0 + lane;
    if (oo < p.outputs && t < p.frames) p.masks[(long)oo * p.frames + t] = tile[r][lane];
  }
}

}  // namespace

hipError_t launch_band_split(const BandSplitParams& params, hipStream_t stream) {
  BandSplitParams p = params;
  if (p.dim % kSplitDims || 2 * p.dim / kSplitDims > kSplitJobs) return hipErrorInvalidValue;
  p.tile = kSplitFrames;
  const dim3 grid((p.frames + kSplitFrames - 1) / kSplitFrames, p.bands);
  // One thread per (channel group, frame half) job: 192 threads at dim 384, 256 at 512.
  hipLaunchKernelGGL(band_split_kernel, grid, dim3(2 * p.dim / kSplitDims), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_glu_gather(const GluParams& p, hipStream_t stream) {
  const dim3 grid((p.outputs + kGluTile - 1) / kGluTile, (p.frames + kGluTile - 1) / kGluTile);
  hipLaunchKernelGGL(glu_gather_kernel, grid, dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace ancha
