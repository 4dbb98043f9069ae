// STFT / iSTFT and chunk bookkeeping of the separation runtime on the GPU (gfx950).
//
// The reference's Stft (crates/ancha-audio/src/dsp.rs:29-134) is PyTorch's center=true STFT:
// periodic Hann window, reflect padding, unnormalised FFT of n_fft = 2048 (the only size the
// model schema allows, config.rs:58-61). Both channels of a frame go through ONE complex FFT
// (channel 0 as the real part, channel 1 as the imaginary part) and are separated with the
// conjugate symmetry of real spectra; the inverse packs them the same way. The FFT is an
// in-LDS iterative radix-2 transform in fp32 (bit-reversed load, 11 butterfly stages), one
// workgroup per frame, twiddles from sincospif.
//
// Layouts: audio / chunks [2][samples]; the model spectrum [frames][bins][channel][re, im]
// (runtime.rs:161-172, the band-split input); masks [rows = 2*bins][re, im][frames] per stem
// (network.rs Roformer::forward output); frames scratch [frames][2][n_fft].
#include "common.hpp"
#include "kernels.hpp"

namespace ancha {
namespace {

constexpr int kN = 2048;             // FFT size
constexpr int kLog2N = 11;
constexpr int kBins = kN / 2 + 1;
constexpr int kFftThreads = 256;

__device__ __forceinline__ long reflect(long index, long length) {
  if (length <= 1) return 0;
  const long period = 2 * (length - 1);
  long i = index % period;
  if (i < 0) i += period;
  return i < length ? i : period - i;
}

// Periodic Hann, formed in f32 as Stft::new does (dsp.rs:31-33).
__device__ __forceinline__ float hann(int i) {
  return 0.5f - 0.5f * cosf(6.28318530717958647692f * (float)i / (float)kN);
}

__device__ __forceinline__ int bit_reverse(int i) { return (int)(__brev((unsigned)i) >> (32 - kLog2N)); }

// In-place radix-2 FFT of the bit-reverse-ordered values in re/im (LDS); sign -1 forward,
// +1 inverse (unnormalised). Called by all kFftThreads threads; ends with a barrier.
__device__ void fft_lds(float* re, float* im, float sign) {
  __syncthreads();
  for (int s = 1; s <= kLog2N; s++) {
    const int half = 1 << (s - 1);
    for (int b = threadIdx.x; b < kN / 2; b += kFftThreads) {
      const int k = b & (half - 1), i0 = ((b >> (s - 1)) << s) + k, i1 = i0 + half;
      float sn, cs;
      sincospif(sign * (float)k / (float)half, &sn, &cs);
      const float xr = re[i1], xi = im[i1];
      const float vr = xr * cs - xi * sn, vi = xr * sn + xi * cs;
      const float ur = re[i0], ui = im[i0];
      re[i0] = ur + vr;
      im[i0] = ui + vi;
      re[i1] = ur - vr;
      im[i1] = ui - vi;
    }
    __syncthreads();
  }
}

// Stft::forward for both channels of one frame (dsp.rs:46-84): spectrum packed
// [frame][bin][channel][re, im].
__global__ __launch_bounds__(kFftThreads) void stft_kernel(const float* chunk, long samples,
                                                           int hop, float* spectrum) {
  __shared__ float re[kN], im[kN];
  const int t = blockIdx.x;
  const float* x0 = chunk;
  const float* x1 = chunk + samples;
  for (int i = threadIdx.x; i < kN; i += kFftThreads) {
    const long src = reflect((long)t * hop + i - kN / 2, samples);
    const float w = hann(i);
    const int j = bit_reverse(i);
    re[j] = x0[src] * w;
    im[j] = x1[src] * w;
  }
  fft_lds(re, im, -1.0f);
  float* out = spectrum + (long)t * kBins * 4;
  for (int k = threadIdx.x; k < kBins; k += kFftThreads) {
    const int n = (kN - k) & (kN - 1);
    const float a = re[k], b = im[k], c = re[n], d = -im[n];  // Z[k], conj(Z[N-k])
    float4 v;
    v.x = 0.5f * (a + c);  // channel 0: (Z[k] + conj(Z[N-k])) / 2
    v.y = 0.5f * (b + d);
    v.z = 0.5f * (b - d);  // channel 1: (Z[k] - conj(Z[N-k])) / 2i
    v.w = -0.5f * (a - c);
    *reinterpret_cast<float4*>(out + k * 4) = v;
  }
}

// Masked spectrum of one stem -> windowed inverse frames (Stft::inverse, dsp.rs:100-125,
// with the complex mask multiply of runtime.rs:190-196 first): frames [frame][channel][n].
__global__ __launch_bounds__(kFftThreads) void istft_frames_kernel(const float* spectrum,
                                                                   const float* masks,
                                                                   int frames, int zero_dc,
                                                                   float* out) {
  __shared__ float re[kN], im[kN];
  const int t = blockIdx.x;
  const float* s = spectrum + (long)t * kBins * 4;
  for (int k = threadIdx.x; k < kBins; k += kFftThreads) {
    float xr[2], xi[2];
    for (int c = 0; c < 2; c++) {
      const long row = 2 * k + c;
      const float mr = masks[(row * 2) * frames + t], mi = masks[(row * 2 + 1) * frames + t];
      const float ar = s[k * 4 + c * 2], ai = s[k * 4 + c * 2 + 1];
      xr[c] = ar * mr - ai * mi;
      xi[c] = ar * mi + ai * mr;
      if (k == 0 || k == kBins - 1) xi[c] = 0.0f;
      if (k == 0 && zero_dc) xr[c] = 0.0f;
    }
    // Z = X0 + i X1 at k and, by conjugate symmetry of X0 and X1, at N - k.
    const int j = bit_reverse(k);
    re[j] = xr[0] - xi[1];
    im[j] = xi[0] + xr[1];
    if (k > 0 && k < kN / 2) {
      const int jn = bit_reverse(kN - k);
      re[jn] = xr[0] + xi[1];
      im[jn] = -xi[0] + xr[1];
    }
  }
  fft_lds(re, im, 1.0f);
  const float scale = 1.0f / (float)kN;
  float* o = out + (long)t * 2 * kN;
  for (int i = threadIdx.x; i < kN; i += kFftThreads) {
    const float w = hann(i);
    o[i] = re[i] * scale * w;
    o[kN + i] = im[i] * scale * w;
  }
}

// Overlap-add of the inverse frames divided by the summed squared window (dsp.rs:118-132),
// samples [n/2, n/2 + length) of the chunk, then the fade-weighted accumulation of the chunk
// into the clip sums (ChunkPlan::weight + Accumulator::add, chunk.rs:27-73).
// sums [2][total], weights [total] (updated only when `count_weight`).
__global__ void ola_accumulate_kernel(const float* frames_buf, int frames, int hop,
                                      long length, long start, long total, int first, int last,
                                      int count_weight, float* sums, float* weights,
                                      unsigned* flags) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= length) return;
  const long pos = start + i;
  const long j = i + kN / 2;
  long t0 = j - kN + 1 > 0 ? (j - kN + 1 + hop - 1) / hop : 0;
  long t1 = j / hop;
  if (t1 > frames - 1) t1 = frames - 1;
  float a0 = 0.0f, a1 = 0.0f, den = 0.0f;
  for (long t = t0; t <= t1; t++) {
    const int o = (int)(j - t * hop);
    const float w = hann(o);
    a0 += frames_buf[t * 2 * kN + o];
    a1 += frames_buf[t * 2 * kN + kN + o];
    den += w * w;
  }
  const float y0 = a0 / den, y1 = a1 / den;
  // Every sample of the chunk is checked, also those past the clip's end, which are not
  // accumulated (Stft::inverse and Accumulator::add check whole planes).
  if (flags) {
    if (!(den > 1e-11f)) raise_flag(flags, kFlagIstftUncovered);
    if (non_finite(y0) || non_finite(y1)) raise_flag(flags, kFlagChunk);
  }
  if (pos >= total) return;
  const long fade = length / 10 > 1 ? length / 10 : 1;
  float wt = 1.0f;
  if (!first && i < fade) wt = (float)(i + 1) / (float)fade;
  if (!last && i >= length - fade) wt = (float)(length - i) / (float)fade;
  sums[pos] += wt * y0;
  sums[total + pos] += wt * y1;
  if (count_weight) weights[pos] += wt;
}

// Chunk extraction of runtime.rs:118-136: reflect-bordered samples of the clip.
__global__ void chunk_gather_kernel(const float* audio, long n, long start, long border,
                                    long remaining, long samples, float* chunk,
                                    unsigned* flags) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= samples) return;
  float v0 = 0.0f, v1 = 0.0f;
  if (!(i >= remaining && remaining <= samples / 2)) {
    const long local = i < remaining ? i : reflect(i, remaining);
    const long src = reflect(start + local - border, n);
    v0 = audio[src];
    v1 = audio[n + src];
  }
  if (flags && (non_finite(v0) || non_finite(v1))) raise_flag(flags, kFlagInput);
  chunk[i] = v0;
  chunk[samples + i] = v1;
}

// Accumulator::finish + border crop (chunk.rs:75-88, runtime.rs:215-223); optionally the
// residual input - stem (runtime.rs:403-420).
__global__ void finish_kernel(const float* sums, const float* weights, long total, long border,
                              long n, const float* audio, float* out, float* residual,
                              unsigned* flags) {
  // One thread per accumulator sample: every weight is checked (Accumulator::finish), the
  // samples of the cropped clip [border, border + n) are written.
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const float w = weights[idx];
  if (flags && !(w > 0.0f)) raise_flag(flags, kFlagOlaUncovered);
  const long i = idx - border;
  if (i < 0 || i >= n) return;
  for (int c = 0; c < 2; c++) {
    const float y = sums[c * total + border + i] / w;
    out[c * n + i] = y;
    if (residual) residual[c * n + i] = audio[c * n + i] - y;
  }
}

__global__ void zero_kernel(float* p, long n) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.0f;
}

inline unsigned blocks_for(long n, int threads) { return (unsigned)((n + threads - 1) / threads); }

}  // namespace

hipError_t launch_stft(const float* chunk, long samples, int hop, float* spectrum,
                       hipStream_t stream) {
  const int frames = (int)(samples / hop + 1);
  hipLaunchKernelGGL(stft_kernel, dim3(frames), dim3(kFftThreads), 0, stream, chunk, samples, hop,
                     spectrum);
  return hipGetLastError();
}

hipError_t launch_istft_frames(const float* spectrum, const float* masks, int frames, int zero_dc,
                               float* frames_buf, hipStream_t stream) {
  hipLaunchKernelGGL(istft_frames_kernel, dim3(frames), dim3(kFftThreads), 0, stream, spectrum,
                     masks, frames, zero_dc, frames_buf);
  return hipGetLastError();
}

hipError_t launch_ola_accumulate(const float* frames_buf, int frames, int hop, long length,
                                 long start, long total, bool first, bool last, bool count_weight,
                                 float* sums, float* weights, unsigned* flags,
                                 hipStream_t stream) {
  hipLaunchKernelGGL(ola_accumulate_kernel, dim3(blocks_for(length, 256)), dim3(256), 0, stream,
                     frames_buf, frames, hop, length, start, total, (int)first, (int)last,
                     (int)count_weight, sums, weights, flags);
  return hipGetLastError();
}

hipError_t launch_chunk_gather(const float* audio, long n, long start, long border,
                               long remaining, long samples, float* chunk, unsigned* flags,
                               hipStream_t stream) {
  hipLaunchKernelGGL(chunk_gather_kernel, dim3(blocks_for(samples, 256)), dim3(256), 0, stream,
                     audio, n, start, border, remaining, samples, chunk, flags);
  return hipGetLastError();
}

hipError_t launch_finish(const float* sums, const float* weights, long total, long border, long n,
                         const float* audio, float* out, float* residual, unsigned* flags,
                         hipStream_t stream) {
  hipLaunchKernelGGL(finish_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, stream, sums, weights,
                     total, border, n, audio, out, residual, flags);
  return hipGetLastError();
}

hipError_t launch_zero(float* p, long n, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(zero_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, stream, p, n);
  return hipGetLastError();
}

}  // namespace ancha
