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

// One wave per row: sum of squares, optional scaled unit norm written back, second norm of that
// result, fp16 normalised copy. The fp16 row is the operand every block GEMM would round its
// input to, so the GEMM then runs on fp16 x without a norm of its own. Rows of up to 512
// channels stay in registers (two float4 per lane); longer rows are read again per pass.
__device__ __forceinline__ float wave_sum(float s) {
  for (int o = 1; o < 64; o <<= 1) s += __shfl_xor(s, o);
  return s;
}

__device__ __forceinline__ float sumsq(float4 v) {
  return v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
}

__device__ __forceinline__ float4 mul4(float4 v, float a, float4 s) {
  return make_float4(v.x * a * s.x, v.y * a * s.y, v.z * a * s.z, v.w * a * s.w);
}

__device__ __forceinline__ void store_h4(rsrc_t hr, unsigned chunk, float4 v, float inv) {
  const u32x2 pk = {pack_h2(v.x * inv, v.y * inv), pack_h2(v.z * inv, v.w * inv)};
  __builtin_amdgcn_raw_buffer_store_b64(pk, hr, chunk * 8, 0, 0);
}

template <bool SHORT>
__global__ __launch_bounds__(256) void norm_half_kernel(const float* x, int rows, int dim,
                                                        const float* scale, float* y,
                                                        _Float16* h) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const unsigned bytes = (unsigned)dim * 4;
  const rsrc_t xr = make_rsrc(x + (long)row * dim, bytes);
  const rsrc_t hr = make_rsrc(h + (long)row * dim, (unsigned)dim * 2);
  const rsrc_t sr = make_rsrc(scale ? scale : x, scale ? bytes : 0u);
  const rsrc_t yr = make_rsrc(y ? y + (long)row * dim : x, y ? bytes : 0u);
  const int chunks = dim / 4;  // float4 chunks; lanes past the end read 0 and store nothing
  if constexpr (SHORT) {
    float4 v[2];
    float ss = 0.f;
    for (int i = 0; i < 2; i++) {
      v[i] = bload4<true>(xr, (lane + 64 * i) * 16);
      ss += sumsq(v[i]);
    }
    ss = wave_sum(ss);
    if (scale) {
      const float inv = 1.0f / fmaxf(sqrtf(ss), 1e-12f);
      ss = 0.f;
      for (int i = 0; i < 2; i++) {
        v[i] = mul4(v[i], inv, bload4<true>(sr, (lane + 64 * i) * 16));
        ss += sumsq(v[i]);
        if (y) bstore4<true>(yr, (lane + 64 * i) * 16, v[i]);
      }
      ss = wave_sum(ss);
    }
    const float inv = 1.0f / fmaxf(sqrtf(ss), 1e-12f);
    for (int i = 0; i < 2; i++) store_h4(hr, lane + 64 * i, v[i], inv);
  } else {
    float ss = 0.f;
    for (int c = lane; c < chunks; c += 64) ss += sumsq(bload4<true>(xr, c * 16));
    ss = wave_sum(ss);
    float inv = 1.0f / fmaxf(sqrtf(ss), 1e-12f);
    if (scale) {
      // y (or, without y, only its norm) first; the fp16 pass recomputes it from x (y does
      // not alias x here).
      const float inv1 = inv;
      ss = 0.f;
      for (int c = lane; c < chunks; c += 64) {
        const float4 v = mul4(bload4<true>(xr, c * 16), inv1, bload4<true>(sr, c * 16));
        ss += sumsq(v);
        if (y) bstore4<true>(yr, c * 16, v);
      }
      ss = wave_sum(ss);
      inv = 1.0f / fmaxf(sqrtf(ss), 1e-12f);
      for (int c = lane; c < chunks; c += 64) {
        store_h4(hr, c, mul4(bload4<true>(xr, c * 16), inv1, bload4<true>(sr, c * 16)), inv);
      }
    } else {
      for (int c = lane; c < chunks; c += 64) store_h4(hr, c, bload4<true>(xr, c * 16), inv);
    }
  }
}

// fp16 copy of n floats, 8 per thread (n % 8 == 0), rounded to nearest even as the GEMMs
// round their fp32 operands.
__global__ __launch_bounds__(256) void cast_half_kernel(const float4* x, long n8, u32x4* h) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  const float4 a = x[2 * i], b = x[2 * i + 1];
  h[i] = u32x4{pack_h2(a.x, a.y), pack_h2(a.z, a.w), pack_h2(b.x, b.y), pack_h2(b.z, b.w)};
}

}  // namespace

hipError_t launch_cast_half(const float* x, long n, _Float16* h, hipStream_t stream) {
  if (n < 0 || n % 8 || (reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(h) & 15))
    return hipErrorInvalidValue;
  if (n == 0) return hipSuccess;
  const long n8 = n / 8;
  hipLaunchKernelGGL(cast_half_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, stream,
                     reinterpret_cast<const float4*>(x), n8, reinterpret_cast<u32x4*>(h));
  return hipGetLastError();
}

hipError_t launch_norm_half(const float* x, int rows, int dim, const float* scale, float* y,
                            _Float16* h, hipStream_t stream) {
  if (dim <= 0 || dim % 4 || (dim > 512 && scale && y == x)) return hipErrorInvalidValue;
  if (rows <= 0) return hipSuccess;
  const dim3 grid((rows + kRowsPerBlock - 1) / kRowsPerBlock), block(64 * kRowsPerBlock);
  if (dim <= 512)
    hipLaunchKernelGGL(norm_half_kernel<true>, grid, block, 0, stream, x, rows, dim, scale, y, h);
  else
    hipLaunchKernelGGL(norm_half_kernel<false>, grid, block, 0, stream, x, rows, dim, scale, y, h);
  return hipGetLastError();
}

hipError_t launch_unit_norm(const NormParams& p, bool aligned, hipStream_t stream) {
  const dim3 grid((p.rows + kRowsPerBlock - 1) / kRowsPerBlock), block(64 * kRowsPerBlock);
  if (aligned)
    hipLaunchKernelGGL(unit_norm_kernel<true>, grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL(unit_norm_kernel<false>, grid, block, 0, stream, p);
  return hipGetLastError();
}

}  // namespace ancha
