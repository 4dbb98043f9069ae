/*
 * CPU restatement of Ancha's fused RoFormer attention path: TEST INFRASTRUCTURE ONLY.
 * See ancha_oracle.h. Built by oracle/Makefile into oracle/_build/libancha_oracle.so.
 */
#include "ancha_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define R float
#define S f32
#define SQRT sqrtf
#define EXP expf
#define ERF erff
#define FMAX fmaxf
#include "oracle_impl.h"
#undef R
#undef S
#undef SQRT
#undef EXP
#undef ERF
#undef FMAX

#define R double
#define S f64
#define SQRT sqrt
#define EXP exp
#define ERF erf
#define FMAX fmax
#include "oracle_impl.h"
#undef R
#undef S
#undef SQRT
#undef EXP
#undef ERF
#undef FMAX

static uint64_t splitmix64_at(uint64_t seed, uint64_t index) {
  /* Output `index` (0-based) of the splitmix64 sequence started at state `seed`. */
  uint64_t z = seed + (index + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

void anc_fill_normal(float *out, size_t n, uint64_t seed, double scale, size_t first) {
  const double two_pi = 6.283185307179586476925286766559;
  for (size_t o = 0; o < n; o++) {
    size_t i = first + o;
    size_t pair = i / 2;
    double u1 = 1.0 - (double)(splitmix64_at(seed, 2 * pair) >> 11) * 0x1.0p-53;
    double u2 = (double)(splitmix64_at(seed, 2 * pair + 1) >> 11) * 0x1.0p-53;
    double r = sqrt(-2.0 * log(u1));
    double z = (i & 1) ? r * sin(two_pi * u2) : r * cos(two_pi * u2);
    out[o] = (float)(z * scale);
  }
}

void anc_axis_rope_packed(const float *freqs, size_t nf, size_t tokens, float *out) {
  size_t width = nf * 2;
  float scale = 1.0f / sqrtf((float)width);
  size_t p = 0;
  for (int table = 0; table < 2; table++) {
    float s_ = table == 0 ? scale : 1.0f;
    for (int sine = 0; sine < 2; sine++)
      for (size_t t = 0; t < tokens; t++)
        for (size_t i = 0; i < nf; i++) {
          float angle = (float)t * freqs[i];
          float s = sinf(angle), c = cosf(angle);
          if (sine) {
            out[p++] = -s * s_;
            out[p++] = s * s_;
          } else {
            out[p++] = c * s_;
            out[p++] = c * s_;
          }
        }
  }
}

void anc_rope_tables(const float *freqs, size_t nf, size_t tokens, size_t heads, float scale,
                     float *cos_out, float *sin_out) {
  size_t p = 0;
  for (size_t t = 0; t < tokens; t++)
    for (size_t h = 0; h < heads; h++)
      for (size_t i = 0; i < nf; i++) {
        float angle = (float)t * freqs[i];
        float s = sinf(angle), c = cosf(angle);
        cos_out[p] = c * scale;
        cos_out[p + 1] = c * scale;
        sin_out[p] = -s * scale;
        sin_out[p + 1] = s * scale;
        p += 2;
      }
}

int anc_residual_l2norm(const float *x, const float *residual, const float *gamma, size_t rows,
                        size_t dim, float eps, float *sum, float *norm) {
  if (!rows || !dim || !(eps > 0.0f) || !isfinite(eps)) return ANC_E_SHAPE;
  size_t n = rows * dim;
  for (size_t i = 0; i < n; i++)
    if (!isfinite(x[i]) || !isfinite(residual[i])) return ANC_E_NONFINITE_IN;
  for (size_t i = 0; i < dim; i++)
    if (!isfinite(gamma[i])) return ANC_E_NONFINITE_IN;
  for (size_t r = 0; r < rows; r++) {
    float sq = 0.0f;
    for (size_t d = 0; d < dim; d++) {
      float y = x[r * dim + d] + residual[r * dim + d];
      sum[r * dim + d] = y;
      sq += y * y;
    }
    if (!isfinite(sq)) return ANC_E_NORM_OVERFLOW;
    float scale = sqrtf((float)dim) / fmaxf(sqrtf(sq), eps);
    for (size_t d = 0; d < dim; d++) norm[r * dim + d] = sum[r * dim + d] * scale * gamma[d];
  }
  for (size_t i = 0; i < n; i++)
    if (!isfinite(norm[i])) return ANC_E_OUTPUT_OVERFLOW;
  return ANC_OK;
}

int anc_pack_qkv_gate(const float *qkv, size_t qkv_len, const float *gate, size_t gate_len,
                      const float *gate_bias, size_t heads, size_t dim, float *w_out,
                      float *b_out) {
  if (!dim || qkv_len % dim || gate_len != heads * dim) return ANC_E_SHAPE;
  memcpy(w_out, qkv, sizeof(float) * qkv_len);
  memcpy(w_out + qkv_len, gate, sizeof(float) * gate_len);
  size_t zeros = qkv_len / dim;
  for (size_t i = 0; i < zeros; i++) b_out[i] = 0.0f;
  memcpy(b_out + zeros, gate_bias, sizeof(float) * heads);
  return ANC_OK;
}

int anc_fold_norm_scale(const float *weights, size_t len, const float *gamma, size_t dim,
                        float *out) {
  if (!dim || len % dim) return ANC_E_SHAPE;
  float root = sqrtf((float)dim);
  for (size_t i = 0; i < len; i++) out[i] = weights[i] * gamma[i % dim] * root;
  return ANC_OK;
}

void anc_folded_linear(const float *weight, size_t input, size_t row0, size_t row1,
                       const float *input_scale, float output_scale, const float *bias,
                       float *w_out, float *b_out) {
  size_t output = row1 - row0;
  for (size_t o = 0; o < output; o++)
    for (size_t i = 0; i < input; i++)
      w_out[i * output + o] = weight[(row0 + o) * input + i] * input_scale[i] * output_scale;
  if (bias && b_out)
    for (size_t o = 0; o < output; o++) b_out[o] = bias[row0 + o] * output_scale;
}

/* PyTorch [out, in] -> Burn [in, out] (weights.rs Weights::linear). */
static float *transposed(const float *w, size_t out, size_t in) {
  float *t = (float *)malloc(sizeof(float) * out * in);
  for (size_t o = 0; o < out; o++)
    for (size_t i = 0; i < in; i++) t[i * out + o] = w[o * in + i];
  return t;
}

/* anc_linear_f32 with its rows split over `threads` pthreads (the reference's Burn GEMMs run
 * multi-threaded); slices start at multiples of `tokens` so the rotary token index r % tokens is
 * unchanged. Every row's arithmetic is the same as in one call. */
typedef struct {
  const float *x, *w, *bias, *rope, *residual;
  float *out;
  size_t n, k, ldx, m, tokens, width;
  int gelu;
} lin_job;

static void *lin_worker(void *arg) {
  lin_job *j = (lin_job *)arg;
  anc_linear_f32(j->x, j->n, j->k, j->ldx, j->w, j->m, j->bias, j->gelu, j->rope, j->tokens,
                 j->width, j->residual, j->out);
  return NULL;
}

static void par_linear(size_t threads, const float *x, size_t n, size_t k, size_t ldx,
                       const float *w, size_t m, const float *bias, int gelu, const float *rope,
                       size_t tokens, size_t width, const float *residual, float *out) {
  size_t unit = rope ? tokens : 1;
  size_t units = (n + unit - 1) / unit;
  size_t parts = threads < 1 ? 1 : threads;
  if (parts > units) parts = units;
  if (parts <= 1) {
    anc_linear_f32(x, n, k, ldx, w, m, bias, gelu, rope, tokens, width, residual, out);
    return;
  }
  size_t per = (units + parts - 1) / parts * unit;
  lin_job jobs[256];
  pthread_t tids[256];
  size_t nj = 0;
  for (size_t r0 = 0; r0 < n && nj < 256; r0 += per, nj++) {
    size_t rows = n - r0 < per ? n - r0 : per;
    lin_job j = {x + r0 * ldx, w, bias, rope, residual ? residual + r0 * m : NULL, out + r0 * m,
                 rows, k, ldx, m, tokens, width, gelu};
    jobs[nj] = j;
  }
  for (size_t i = 0; i < nj; i++) pthread_create(&tids[i], NULL, lin_worker, &jobs[i]);
  for (size_t i = 0; i < nj; i++) pthread_join(tids[i], NULL);
}

static float *source_scale(const float *gamma, size_t dim) {
  float *s = (float *)malloc(sizeof(float) * dim);
  float root = sqrtf((float)dim);
  for (size_t i = 0; i < dim; i++) s[i] = gamma[i] * root;
  return s;
}

int anc_transformer_forward(const anc_block_weights *w, const float *x, size_t groups,
                            size_t tokens, int kernels, size_t threads, float *out) {
  size_t dim = w->dim, heads = w->heads, hd = w->head_dim, inner = heads * hd, hidden = w->hidden;
  size_t rows = groups * tokens, nf = hd / 2;
  if (!rows || !dim || hd != 64) return ANC_E_SHAPE;
  float *norm = source_scale(w->attn_gamma, dim);
  float *ffs = source_scale(w->ff_gamma, dim);
  /* Load-time folding (roformer.rs:205-244, :388-395). */
  float *wq = malloc(sizeof(float) * dim * inner), *wk = malloc(sizeof(float) * dim * inner);
  float *wv = malloc(sizeof(float) * dim * inner), *wg = malloc(sizeof(float) * dim * heads);
  float *bg = malloc(sizeof(float) * heads);
  anc_folded_linear(w->to_qkv, dim, 0, inner, norm, 1.0f, NULL, wq, NULL);
  anc_folded_linear(w->to_qkv, dim, inner, 2 * inner, norm, 1.0f, NULL, wk, NULL);
  anc_folded_linear(w->to_qkv, dim, 2 * inner, 3 * inner, norm, 1.0f, NULL, wv, NULL);
  anc_folded_linear(w->to_gates, dim, 0, heads, norm, 1.0f, w->to_gates_bias, wg, bg);
  float *w1 = malloc(sizeof(float) * dim * hidden), *b1 = malloc(sizeof(float) * hidden);
  anc_folded_linear(w->ff_in, dim, 0, hidden, ffs, 1.0f, w->ff_in_bias, w1, b1);
  float *wo = transposed(w->to_out, dim, inner);
  float *w2 = transposed(w->ff_out, dim, hidden);
  float *table = malloc(sizeof(float) * 4 * tokens * hd);
  anc_axis_rope_packed(w->freqs, nf, tokens, table);

  float *xn = malloc(sizeof(float) * rows * dim);
  float *attended = malloc(sizeof(float) * rows * inner);
  float *x1 = malloc(sizeof(float) * rows * dim);
  float *h = malloc(sizeof(float) * rows * hidden);
  int rc = ANC_OK;
  anc_unit_norm_f32(x, rows, dim, NULL, xn);
  if (kernels) {
    /* forward_kernels (roformer.rs:464-520): packed q|k|v|gates|pad GEMM, RoPE epilogue. */
    size_t used = 3 * inner + heads, columns = (used + 127) / 128 * 128;
    float *wp = calloc(dim * columns, sizeof(float)), *bp = calloc(columns, sizeof(float));
    for (size_t i = 0; i < dim; i++) {
      memcpy(wp + i * columns, wq + i * inner, sizeof(float) * inner);
      memcpy(wp + i * columns + inner, wk + i * inner, sizeof(float) * inner);
      memcpy(wp + i * columns + 2 * inner, wv + i * inner, sizeof(float) * inner);
      memcpy(wp + i * columns + 3 * inner, wg + i * heads, sizeof(float) * heads);
    }
    memcpy(bp + 3 * inner, bg, sizeof(float) * heads);
    float *packed = malloc(sizeof(float) * rows * columns);
    par_linear(threads, xn, rows, dim, dim, wp, columns, bp, 0, table, tokens, inner, NULL, packed);
    rc = anc_gated_attention_f32(packed, groups, tokens, columns, heads, NULL, attended);
    free(packed);
    free(wp);
    free(bp);
  } else {
    /* Attention::forward (roformer.rs:258-270): separate projections, RopeTables, Burn attention. */
    float *q = malloc(sizeof(float) * rows * inner), *k = malloc(sizeof(float) * rows * inner);
    float *v = malloc(sizeof(float) * rows * inner), *gt = malloc(sizeof(float) * rows * heads);
    float *cq = malloc(sizeof(float) * tokens * inner), *sq = malloc(sizeof(float) * tokens * inner);
    float *ck = malloc(sizeof(float) * tokens * inner), *sk = malloc(sizeof(float) * tokens * inner);
    anc_rope_tables(w->freqs, nf, tokens, heads, 1.0f / sqrtf((float)hd), cq, sq);
    anc_rope_tables(w->freqs, nf, tokens, heads, 1.0f, ck, sk);
    par_linear(threads, xn, rows, dim, dim, wq, inner, NULL, 0, NULL, 1, 0, NULL, q);
    par_linear(threads, xn, rows, dim, dim, wk, inner, NULL, 0, NULL, 1, 0, NULL, k);
    par_linear(threads, xn, rows, dim, dim, wv, inner, NULL, 0, NULL, 1, 0, NULL, v);
    par_linear(threads, xn, rows, dim, dim, wg, heads, bg, 0, NULL, 1, 0, NULL, gt);
    /* RopeTables::apply (roformer.rs:177-186): x*cos + x[i^1]*sin */
    for (size_t r = 0; r < rows; r++) {
      size_t t = r % tokens;
      float *qr = q + r * inner, *kr = k + r * inner;
      for (size_t c = 0; c < inner; c += 2) {
        size_t p = t * inner + c;
        float a = qr[c], b = qr[c + 1];
        qr[c] = a * cq[p] + b * sq[p];
        qr[c + 1] = b * cq[p + 1] + a * sq[p + 1];
        a = kr[c];
        b = kr[c + 1];
        kr[c] = a * ck[p] + b * sk[p];
        kr[c + 1] = b * ck[p + 1] + a * sk[p + 1];
      }
    }
    rc = anc_token_major_attention_f32(q, k, v, groups, tokens, heads, hd, inner, inner, inner,
                                       groups, tokens, threads, attended);
    for (size_t r = 0; r < rows; r++)
      for (size_t hh = 0; hh < heads; hh++) {
        float s = 1.0f / (1.0f + expf(-gt[r * heads + hh]));
        for (size_t e = 0; e < hd; e++) attended[r * inner + hh * hd + e] *= s;
      }
    free(q);
    free(k);
    free(v);
    free(gt);
    free(cq);
    free(sq);
    free(ck);
    free(sk);
  }
  if (!rc) {
    par_linear(threads, attended, rows, inner, inner, wo, dim, NULL, 0, NULL, 1, 0, x, x1);
    anc_unit_norm_f32(x1, rows, dim, NULL, xn);
    par_linear(threads, xn, rows, dim, dim, w1, hidden, b1, 1, NULL, 1, 0, NULL, h);
    par_linear(threads, h, rows, hidden, hidden, w2, dim, w->ff_out_bias, 0, NULL, 1, 0, x1, out);
    if (w->output_gamma) {
      float *os = source_scale(w->output_gamma, dim);
      memcpy(x1, out, sizeof(float) * rows * dim);
      anc_unit_norm_f32(x1, rows, dim, os, out);
      free(os);
    }
  }
  free(norm);
  free(ffs);
  free(wq);
  free(wk);
  free(wv);
  free(wg);
  free(bg);
  free(w1);
  free(b1);
  free(wo);
  free(w2);
  free(table);
  free(xn);
  free(attended);
  free(x1);
  free(h);
  return rc;
}
