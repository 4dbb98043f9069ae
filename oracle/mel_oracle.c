/*
 * CPU restatement of the Mel/BS-RoFormer front end, mask estimator and STFT of Ancha:
 * TEST INFRASTRUCTURE ONLY (see ancha_oracle.h). Only tests, the smoke check and the
 * benchmark's CPU-baseline leg load it.
 *
 * Sources followed (paths relative to the Ancha repository root):
 *   crates/ancha-audio/src/dsp.rs:29-147      Stft::{new, forward, inverse}, reflect_index
 *   crates/ancha-models/src/network.rs:18-35   BandAffine (W.x + b per band)
 *   crates/ancha-models/src/network.rs:96-121  band projections with sqrt(width)*gamma folded
 *   crates/ancha-models/src/network.rs:316-323 band split: gather, unit_norm, projection
 *   crates/ancha-models/src/network.rs:138-177 mask heads: tanh hidden layers, GLU output
 *   crates/ancha-models/src/network.rs:365-398 GLU mask, overlap scatter-add / coverage
 *
 * The reference's FFT is realfft 3.5.0 / rustfft 6.4.1 (not under the reference tree); the
 * restatement computes the same unnormalised DFT with an iterative radix-2 FFT in double
 * precision and rounds the result to f32.
 */
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#include "ancha_oracle.h"

/* dsp.rs:139-147: reflection without repeating the edge sample, any number of periods. */
size_t anc_reflect_index(long index, size_t length) {
  if (length <= 1) return 0;
  long period = 2 * ((long)length - 1);
  long i = index % period;
  if (i < 0) i += period;
  return i < (long)length ? (size_t)i : (size_t)(period - i);
}

/* In-place iterative radix-2 complex FFT of size n (a power of two), sign -1 forward. */
static void fft(double *re, double *im, size_t n, int sign) {
  for (size_t i = 1, j = 0; i < n; i++) {
    size_t bit = n >> 1;
    for (; j & bit; bit >>= 1) j ^= bit;
    j ^= bit;
    if (i < j) {
      double t = re[i];
      re[i] = re[j];
      re[j] = t;
      t = im[i];
      im[i] = im[j];
      im[j] = t;
    }
  }
  for (size_t len = 2; len <= n; len <<= 1) {
    double ang = sign * 6.283185307179586476925 / (double)len;
    for (size_t i = 0; i < n; i += len)
      for (size_t k = 0; k < len / 2; k++) {
        double wr = cos(ang * (double)k), wi = sin(ang * (double)k);
        double ur = re[i + k], ui = im[i + k];
        double xr = re[i + k + len / 2], xi = im[i + k + len / 2];
        double vr = xr * wr - xi * wi, vi = xr * wi + xi * wr;
        re[i + k] = ur + vr;
        im[i + k] = ui + vi;
        re[i + k + len / 2] = ur - vr;
        im[i + k + len / 2] = ui - vi;
      }
  }
}

/* Stft::new (dsp.rs:23-44): periodic Hann window, computed in f32 like the reference. */
static float *hann(size_t n_fft) {
  float *w = malloc(sizeof(float) * n_fft);
  const float tau = 6.28318530717958647692f;
  for (size_t i = 0; i < n_fft; i++) w[i] = 0.5f - 0.5f * cosf(tau * (float)i / (float)n_fft);
  return w;
}

static int valid_fft(size_t n_fft, size_t hop) {
  return n_fft >= 2 && (n_fft & (n_fft - 1)) == 0 && hop > 0 && hop <= n_fft / 2;
}

/* Stft::forward (dsp.rs:46-84): frames = n / hop + 1, centred frames with reflect padding,
 * windowed, unnormalised real FFT; out [frames][n_fft/2 + 1][re, im]. */
int anc_stft(const float *signal, size_t n, size_t n_fft, size_t hop, float *out) {
  if (!valid_fft(n_fft, hop)) return ANC_E_SHAPE;
  if (n <= n_fft / 2) return ANC_E_SHAPE;
  for (size_t i = 0; i < n; i++)
    if (!isfinite(signal[i])) return ANC_E_NONFINITE_IN;
  const size_t frames = n / hop + 1, bins = n_fft / 2 + 1;
  float *w = hann(n_fft);
  double *re = malloc(sizeof(double) * n_fft), *im = malloc(sizeof(double) * n_fft);
  for (size_t t = 0; t < frames; t++) {
    for (size_t i = 0; i < n_fft; i++) {
      const long index = (long)(t * hop + i) - (long)(n_fft / 2);
      re[i] = (double)(signal[anc_reflect_index(index, n)] * w[i]);
      im[i] = 0.0;
    }
    fft(re, im, n_fft, -1);
    for (size_t f = 0; f < bins; f++) {
      out[(t * bins + f) * 2] = (float)re[f];
      out[(t * bins + f) * 2 + 1] = (float)im[f];
    }
  }
  free(w);
  free(re);
  free(im);
  return ANC_OK;
}

/* Stft::inverse (dsp.rs:86-134): imaginary parts of the DC and Nyquist bins dropped, DC
 * zeroed when zero_dc, unnormalised inverse real FFT times 1/n_fft and the window, overlap-add
 * divided by the summed squared window; samples [n_fft/2, n_fft/2 + length). */
int anc_istft(const float *spectrum, size_t frames, size_t n_fft, size_t hop, size_t length,
              int zero_dc, float *out) {
  if (!valid_fft(n_fft, hop) || frames == 0) return ANC_E_SHAPE;
  const size_t bins = n_fft / 2 + 1, total = (frames - 1) * hop + n_fft, pad = n_fft / 2;
  if (length + pad > total) return ANC_E_SHAPE;
  float *w = hann(n_fft);
  float *acc = calloc(total, sizeof(float)), *den = calloc(total, sizeof(float));
  double *re = malloc(sizeof(double) * n_fft), *im = malloc(sizeof(double) * n_fft);
  const float scale = 1.0f / (float)n_fft;
  for (size_t t = 0; t < frames; t++) {
    const float *s = spectrum + t * bins * 2;
    for (size_t f = 0; f < bins; f++) {
      re[f] = s[2 * f];
      im[f] = s[2 * f + 1];
    }
    im[0] = 0.0;
    im[bins - 1] = 0.0;
    if (zero_dc) re[0] = 0.0;
    for (size_t f = bins; f < n_fft; f++) {  // Hermitian extension
      re[f] = re[n_fft - f];
      im[f] = -im[n_fft - f];
    }
    fft(re, im, n_fft, +1);
    for (size_t i = 0; i < n_fft; i++) {
      acc[t * hop + i] += (float)re[i] * scale * w[i];
      den[t * hop + i] += w[i] * w[i];
    }
  }
  int rc = ANC_OK;
  for (size_t i = 0; i < length; i++) {
    if (!(den[pad + i] > 1e-11f)) {
      rc = ANC_E_SHAPE;
      break;
    }
    out[i] = acc[pad + i] / den[pad + i];
  }
  free(w);
  free(acc);
  free(den);
  free(re);
  free(im);
  return rc;
}

/* ---- band split --------------------------------------------------------------------------- */

typedef struct {
  const float *spectrum;
  size_t t, cols, dim;
  const size_t *offsets, *bins;
  const float *gamma, *weight, *bias;
  size_t b0, b1;
  const size_t *wofs; /* per band: first gamma element; weight offset is dim * wofs[b] */
  float *x;
} split_job;

static void *split_worker(void *arg) {
  const split_job *j = (const split_job *)arg;
  for (size_t b = j->b0; b < j->b1; b++) {
    const size_t nb = j->offsets[b + 1] - j->offsets[b], width = 4 * nb;
    const size_t *fb = j->bins + j->offsets[b];
    const float *g = j->gamma + j->wofs[b];
    const float *wt = j->weight + j->dim * j->wofs[b];
    /* SourceNorm::scale (roformer.rs:43-51): sqrt(width) * gamma, folded into the columns. */
    float *wf = malloc(sizeof(float) * j->dim * width);
    const float root = sqrtf((float)width);
    for (size_t d = 0; d < j->dim; d++)
      for (size_t c = 0; c < width; c++) wf[d * width + c] = wt[d * width + c] * (g[c] * root);
    float *z = malloc(sizeof(float) * width);
    for (size_t t = 0; t < j->t; t++) {
      const float *row = j->spectrum + t * j->cols;
      for (size_t q = 0; q < nb; q++)
        for (size_t k = 0; k < 4; k++) z[4 * q + k] = row[4 * fb[q] + k];
      anc_unit_norm_f32(z, 1, width, NULL, z);
      float *o = j->x + (b * j->t + t) * j->dim;
      for (size_t d = 0; d < j->dim; d++) {
        float s = 0.0f;
        for (size_t c = 0; c < width; c++) s += wf[d * width + c] * z[c];
        o[d] = s + j->bias[b * j->dim + d];
      }
    }
    free(z);
    free(wf);
  }
  return NULL;
}

static size_t *band_offsets(size_t bands, const size_t *offsets) {
  size_t *w = malloc(sizeof(size_t) * (bands + 1));
  w[0] = 0;
  for (size_t b = 0; b < bands; b++) w[b + 1] = w[b] + 4 * (offsets[b + 1] - offsets[b]);
  return w;
}

/* Band split (network.rs:316-323): spectrum [t][cols] packed (frame, bin*2 + channel,
 * re/im), band b = FFT bins bins[offsets[b] .. offsets[b+1]); its features are the columns
 * 4f .. 4f+3 of each bin f, row-normalised (unit_norm) and projected with W_b [dim][width]
 * (sqrt(width)*gamma_b folded into the columns, network.rs:104-110) plus bias_b.
 * gamma / weight are the bands' tensors concatenated in band order. x [bands][t][dim]. */
int anc_band_split(const float *spectrum, size_t t, size_t cols, size_t bands,
                   const size_t *offsets, const size_t *bins, size_t dim, const float *gamma,
                   const float *weight, const float *bias, size_t threads, float *x) {
  if (!t || !bands || !dim) return ANC_E_ZERO_DIM;
  for (size_t b = 0; b < bands; b++) {
    if (offsets[b + 1] <= offsets[b]) return ANC_E_SHAPE;
    for (size_t i = offsets[b]; i < offsets[b + 1]; i++)
      if (4 * bins[i] + 3 >= cols) return ANC_E_SHAPE;
  }
  size_t *wofs = band_offsets(bands, offsets);
  if (threads < 1) threads = 1;
  if (threads > bands) threads = bands;
  pthread_t *tid = malloc(sizeof(pthread_t) * threads);
  split_job *jobs = malloc(sizeof(split_job) * threads);
  for (size_t i = 0; i < threads; i++) {
    jobs[i] = (split_job){spectrum, t, cols, dim, offsets, bins, gamma, weight, bias,
                          bands * i / threads, bands * (i + 1) / threads, wofs, x};
    pthread_create(&tid[i], NULL, split_worker, &jobs[i]);
  }
  for (size_t i = 0; i < threads; i++) pthread_join(tid[i], NULL);
  free(tid);
  free(jobs);
  free(wofs);
  return ANC_OK;
}

/* ---- mask estimator ----------------------------------------------------------------------- */

typedef struct {
  const float *x;
  size_t t, dim, hidden, layers;
  const size_t *offsets;
  const float *const *hw;
  const float *const *hb;
  const float *ow, *ob;
  const size_t *wofs;
  size_t b0, b1;
  float *glu; /* [total width][t] per band at 2 * wofs[b] ... (value * sigmoid(gate)) */
} head_job;

/* [out][in] -> [in][out] (the [k][m] layout of anc_linear_f32). */
static float *transpose(const float *w, size_t out, size_t in) {
  float *t = malloc(sizeof(float) * out * in);
  for (size_t o = 0; o < out; o++)
    for (size_t i = 0; i < in; i++) t[i * out + o] = w[o * in + i];
  return t;
}

static void *head_worker(void *arg) {
  const head_job *j = (const head_job *)arg;
  const size_t widest = j->hidden > j->dim ? j->hidden : j->dim;
  float *a = malloc(sizeof(float) * j->t * widest), *c = malloc(sizeof(float) * j->t * widest);
  for (size_t b = j->b0; b < j->b1; b++) {
    const size_t width = j->wofs[b + 1] - j->wofs[b];
    memcpy(a, j->x + b * j->t * j->dim, sizeof(float) * j->t * j->dim);
    size_t in = j->dim;
    for (size_t l = 0; l < j->layers; l++) {
      const size_t out = j->hidden;
      float *wt = transpose(j->hw[l] + b * out * in, out, in);
      anc_linear_f32(a, j->t, in, in, wt, out, j->hb[l] + b * out, 0, NULL, 1, 0, NULL, c);
      for (size_t e = 0; e < j->t * out; e++) a[e] = tanhf(c[e]);
      free(wt);
      in = out;
    }
    /* Last projection [2*width, hidden]: value rows then gate rows (network.rs:162-169). */
    float *vg = malloc(sizeof(float) * j->t * 2 * width);
    float *wt = transpose(j->ow + 2 * j->wofs[b] * in, 2 * width, in);
    anc_linear_f32(a, j->t, in, in, wt, 2 * width, j->ob + 2 * j->wofs[b], 0, NULL, 1, 0, NULL, vg);
    for (size_t t = 0; t < j->t; t++)
      for (size_t r = 0; r < width; r++) {
        const float gate = 1.0f / (1.0f + expf(-vg[t * 2 * width + width + r]));
        j->glu[(j->wofs[b] + r) * j->t + t] = vg[t * 2 * width + r] * gate;
      }
    free(wt);
    free(vg);
  }
  free(a);
  free(c);
  return NULL;
}

/* One stem's mask head (network.rs:374-398): per band, `layers` hidden layers
 * h = tanh(W h + b) (dim -> hidden -> ... -> hidden; hw[l] / hb[l] hold the bands' [out][in]
 * weights and [out] biases back to back), then value / gate = W_v h + b_v, W_g h + b_g with
 * the band's [2*width][hidden] output weight (value rows first) and [2*width] bias,
 * mask = value * sigmoid(gate) over the band's 4 columns per bin (channel 0 re, im, channel 1
 * re, im). Masks of overlapping bands are summed into spectrum rows (bin f, channel c) ->
 * row 2f + c and divided by the number of bands covering f (network.rs:248-263, :384-396).
 * x [bands][t][dim] -> masks [2 * fft_bins][2][t] (row, re/im, frame). */
int anc_mask_head(const float *x, size_t t, size_t bands, const size_t *offsets,
                  const size_t *bins, size_t fft_bins, size_t dim, size_t hidden, size_t layers,
                  const float *const *hw, const float *const *hb, const float *ow,
                  const float *ob, size_t threads, float *masks) {
  if (!t || !bands || !dim || !hidden) return ANC_E_ZERO_DIM;
  size_t *wofs = band_offsets(bands, offsets);
  float *glu = malloc(sizeof(float) * wofs[bands] * t);
  if (threads < 1) threads = 1;
  if (threads > bands) threads = bands;
  pthread_t *tid = malloc(sizeof(pthread_t) * threads);
  head_job *jobs = malloc(sizeof(head_job) * threads);
  for (size_t i = 0; i < threads; i++) {
    jobs[i] = (head_job){x, t, dim, hidden, layers, offsets, hw, hb, ow, ob, wofs,
                         bands * i / threads, bands * (i + 1) / threads, glu};
    pthread_create(&tid[i], NULL, head_worker, &jobs[i]);
  }
  for (size_t i = 0; i < threads; i++) pthread_join(tid[i], NULL);
  const size_t rows = 2 * fft_bins;
  float *coverage = calloc(rows, sizeof(float));
  memset(masks, 0, sizeof(float) * rows * 2 * t);
  for (size_t b = 0; b < bands; b++)
    for (size_t q = offsets[b]; q < offsets[b + 1]; q++) {
      const size_t f = bins[q], j = q - offsets[b];
      for (size_t ch = 0; ch < 2; ch++) {
        const size_t row = 2 * f + ch;
        coverage[row] += 1.0f;
        for (size_t ri = 0; ri < 2; ri++) {
          const float *src = glu + (wofs[b] + 4 * j + 2 * ch + ri) * t;
          float *dst = masks + (row * 2 + ri) * t;
          for (size_t k = 0; k < t; k++) dst[k] += src[k];
        }
      }
    }
  for (size_t row = 0; row < rows; row++)
    for (size_t k = 0; k < 2 * t; k++) masks[row * 2 * t + k] /= coverage[row];
  free(coverage);
  free(tid);
  free(jobs);
  free(glu);
  free(wofs);
  return ANC_OK;
}
