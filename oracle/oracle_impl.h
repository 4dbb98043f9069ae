/*
 * Oracle body, included twice by ancha_oracle.c: once with R=float (S=f32), once with
 * R=double (S=f64). TEST INFRASTRUCTURE ONLY (see ancha_oracle.h).
 */
#define CAT_(a, b) a##_##b
#define CAT(a, b) CAT_(a, b)
#define FN(name) CAT(name, S)

/* ancha-kernels/src/attention.rs:47-55 */
static R FN(score)(const R *q, const R *k, size_t queries, size_t keys, size_t head_dim,
                   size_t g, size_t i, size_t j) {
  size_t qi = (g * queries + i) * head_dim;
  size_t kj = (g * keys + j) * head_dim;
  R dot = 0;
  for (size_t d = 0; d < head_dim; d++) dot += q[qi + d] * k[kj + d];
  return dot / SQRT((R)head_dim);
}

static int FN(all_finite)(const R *x, size_t n) {
  for (size_t i = 0; i < n; i++)
    if (!isfinite(x[i])) return 0;
  return 1;
}

/* ancha-kernels/src/attention.rs:10-44 */
static int FN(validate)(const R *q, const R *k, const R *v, size_t groups, size_t queries,
                        size_t keys, size_t head_dim, size_t value_dim) {
  if (!groups || !queries || !keys || !head_dim || !value_dim) return ANC_E_ZERO_DIM;
  if (!FN(all_finite)(q, groups * queries * head_dim) ||
      !FN(all_finite)(k, groups * keys * head_dim) ||
      !FN(all_finite)(v, groups * keys * value_dim))
    return ANC_E_NONFINITE_IN;
  return ANC_OK;
}

int FN(anc_attention_dense)(const R *q, const R *k, const R *v, size_t groups, size_t queries,
                            size_t keys, size_t head_dim, size_t value_dim, R *out) {
  int rc = FN(validate)(q, k, v, groups, queries, keys, head_dim, value_dim);
  if (rc) return rc;
  R *scores = (R *)malloc(sizeof(R) * keys);
  memset(out, 0, sizeof(R) * groups * queries * value_dim);
  for (size_t g = 0; g < groups; g++) {
    for (size_t i = 0; i < queries; i++) {
      for (size_t j = 0; j < keys; j++) scores[j] = FN(score)(q, k, queries, keys, head_dim, g, i, j);
      R max = -INFINITY;
      for (size_t j = 0; j < keys; j++) max = FMAX(max, scores[j]);
      if (!isfinite(max)) {
        free(scores);
        return ANC_E_SCORE_OVERFLOW;
      }
      R denom = 0;
      for (size_t j = 0; j < keys; j++) {
        scores[j] = EXP(scores[j] - max);
        denom += scores[j];
      }
      R *o = out + (g * queries + i) * value_dim;
      for (size_t j = 0; j < keys; j++) {
        R p = scores[j] / denom;
        const R *vj = v + (g * keys + j) * value_dim;
        for (size_t d = 0; d < value_dim; d++) o[d] += p * vj[d];
      }
    }
  }
  free(scores);
  return FN(all_finite)(out, groups * queries * value_dim) ? ANC_OK : ANC_E_OUTPUT_OVERFLOW;
}

int FN(anc_attention_tiled)(const R *q, const R *k, const R *v, size_t groups, size_t queries,
                            size_t keys, size_t head_dim, size_t value_dim, size_t query_tile,
                            size_t key_tile, R *out) {
  int rc = FN(validate)(q, k, v, groups, queries, keys, head_dim, value_dim);
  if (rc) return rc;
  if (!query_tile || !key_tile) return ANC_E_TILE;
  size_t qt = query_tile < queries ? query_tile : queries;
  size_t kt = key_tile < keys ? key_tile : keys;
  R *scores = (R *)malloc(sizeof(R) * qt * kt);
  R *num = (R *)malloc(sizeof(R) * qt * value_dim);
  R *maxima = (R *)malloc(sizeof(R) * qt);
  R *denoms = (R *)malloc(sizeof(R) * qt);
  rc = ANC_OK;
  for (size_t g = 0; g < groups && !rc; g++) {
    for (size_t q0 = 0; q0 < queries && !rc; q0 += qt) {
      size_t nq = qt < queries - q0 ? qt : queries - q0;
      for (size_t i = 0; i < qt * value_dim; i++) num[i] = 0;
      for (size_t i = 0; i < qt; i++) {
        maxima[i] = -INFINITY;
        denoms[i] = 0;
      }
      for (size_t k0 = 0; k0 < keys && !rc; k0 += kt) {
        size_t nk = kt < keys - k0 ? kt : keys - k0;
        for (size_t i = 0; i < nq && !rc; i++) {
          R tile_max = -INFINITY;
          for (size_t j = 0; j < nk; j++) {
            R value = FN(score)(q, k, queries, keys, head_dim, g, q0 + i, k0 + j);
            if (!isfinite(value)) {
              rc = ANC_E_SCORE_OVERFLOW;
              break;
            }
            scores[i * kt + j] = value;
            tile_max = FMAX(tile_max, value);
          }
          if (rc) break;
          R new_max = FMAX(maxima[i], tile_max);
          R alpha = EXP(maxima[i] - new_max);
          denoms[i] *= alpha;
          for (size_t d = 0; d < value_dim; d++) num[i * value_dim + d] *= alpha;
          for (size_t j = 0; j < nk; j++) {
            R p = EXP(scores[i * kt + j] - new_max);
            denoms[i] += p;
            const R *vj = v + (g * keys + k0 + j) * value_dim;
            for (size_t d = 0; d < value_dim; d++) num[i * value_dim + d] += p * vj[d];
          }
          maxima[i] = new_max;
        }
      }
      for (size_t i = 0; i < nq && !rc; i++)
        for (size_t d = 0; d < value_dim; d++)
          out[(g * queries + q0 + i) * value_dim + d] = num[i * value_dim + d] / denoms[i];
    }
  }
  free(scores);
  free(num);
  free(maxima);
  free(denoms);
  if (rc) return rc;
  return FN(all_finite)(out, groups * queries * value_dim) ? ANC_OK : ANC_E_OUTPUT_OVERFLOW;
}

/* ---- token-major materialized attention (roformer.rs:324-363), the Flex CPU path ---- */
typedef struct {
  const R *q, *k, *v;
  R *out;
  size_t g0, g1, tokens, heads, d, ldq, ldk, ldv, query_tile;
} FN(tm_job);

static void *FN(tm_worker)(void *arg) {
  FN(tm_job) *job = (FN(tm_job) *)arg;
  size_t T = job->tokens, H = job->heads, D = job->d;
  size_t qt = job->query_tile < T ? job->query_tile : T;
  /* Heads-major dense copies (roformer.rs:335) of one (group, head) at a time; the key copy is
   * stored transposed so the q.k^T product streams along keys. */
  R *qh = (R *)malloc(sizeof(R) * T * D);
  R *kt = (R *)malloc(sizeof(R) * T * D);
  R *vh = (R *)malloc(sizeof(R) * T * D);
  R *scores = (R *)malloc(sizeof(R) * qt * T);
  for (size_t g = job->g0; g < job->g1; g++) {
    for (size_t h = 0; h < H; h++) {
      for (size_t t = 0; t < T; t++) {
        const R *qs = job->q + (g * T + t) * job->ldq + h * D;
        const R *ks = job->k + (g * T + t) * job->ldk + h * D;
        const R *vs = job->v + (g * T + t) * job->ldv + h * D;
        for (size_t e = 0; e < D; e++) {
          qh[t * D + e] = qs[e];
          kt[e * T + t] = ks[e];
          vh[t * D + e] = vs[e];
        }
      }
      for (size_t i0 = 0; i0 < T; i0 += qt) {
        size_t nq = qt < T - i0 ? qt : T - i0;
        /* scores = q . k^T (roformer.rs:357) */
        for (size_t i = 0; i < nq; i++) {
          R *row = scores + i * T;
          for (size_t j = 0; j < T; j++) row[j] = 0;
          for (size_t e = 0; e < D; e++) {
            R a = qh[(i0 + i) * D + e];
            const R *kr = kt + e * T;
            for (size_t j = 0; j < T; j++) row[j] += a * kr[j];
          }
          /* softmax(dim 3): exp(x - max) / sum (roformer.rs:358) */
          R max = -INFINITY;
          for (size_t j = 0; j < T; j++) max = FMAX(max, row[j]);
          R sum = 0;
          for (size_t j = 0; j < T; j++) {
            row[j] = EXP(row[j] - max);
            sum += row[j];
          }
          for (size_t j = 0; j < T; j++) row[j] = row[j] / sum;
          /* . v, written back token-major (roformer.rs:336 swap_dims) */
          R *o = job->out + ((g * T + i0 + i) * H + h) * D;
          for (size_t e = 0; e < D; e++) o[e] = 0;
          for (size_t j = 0; j < T; j++) {
            R p = row[j];
            const R *vr = vh + j * D;
            for (size_t e = 0; e < D; e++) o[e] += p * vr[e];
          }
        }
      }
    }
  }
  free(qh);
  free(kt);
  free(vh);
  free(scores);
  return NULL;
}

int FN(anc_token_major_attention)(const R *q, const R *k, const R *v, size_t groups,
                                  size_t tokens, size_t heads, size_t head_dim, size_t ldq,
                                  size_t ldk, size_t ldv, size_t group_tile, size_t query_tile,
                                  size_t threads, R *out) {
  (void)group_tile; /* group tiles bound memory only; the arithmetic per group is identical */
  if (!groups || !tokens || !heads || !head_dim) return ANC_E_ZERO_DIM;
  if (!query_tile) return ANC_E_TILE;
  size_t parts = threads < 1 ? 1 : threads;
  if (parts > groups) parts = groups;
  size_t size = (groups + parts - 1) / parts;
  size_t njobs = (groups + size - 1) / size;
  FN(tm_job) *jobs = (FN(tm_job) *)calloc(njobs, sizeof(FN(tm_job)));
  pthread_t *tids = (pthread_t *)calloc(njobs, sizeof(pthread_t));
  for (size_t j = 0; j < njobs; j++) {
    FN(tm_job) job = {q, k, v, out, j * size, (j + 1) * size < groups ? (j + 1) * size : groups,
                      tokens, heads, head_dim, ldq, ldk, ldv, query_tile};
    jobs[j] = job;
  }
  if (njobs == 1) {
    FN(tm_worker)(&jobs[0]);
  } else {
    for (size_t j = 0; j < njobs; j++) pthread_create(&tids[j], NULL, FN(tm_worker), &jobs[j]);
    for (size_t j = 0; j < njobs; j++) pthread_join(tids[j], NULL);
  }
  free(jobs);
  free(tids);
  return ANC_OK;
}

/* Rotate one head's 64-wide row in place: x*cos + swap_pairs(x)*sin (fused/gemm.rs:30-41). */
static void FN(rotate_row)(R *x, const float *cos, const float *sin, size_t width) {
  for (size_t d = 0; d < width; d += 2) {
    R a = x[d], b = x[d + 1];
    x[d] = a * (R)cos[d] + b * (R)sin[d];
    x[d + 1] = b * (R)cos[d + 1] + a * (R)sin[d + 1];
  }
}

int FN(anc_attention_op)(const R *q, const R *k, const R *v, size_t groups, size_t tokens,
                         size_t heads, size_t ldq, size_t ldk, size_t ldv, const float *rope,
                         R *out) {
  const size_t D = 64;
  if (!groups || !tokens || !heads) return ANC_E_ZERO_DIM;
  size_t n = groups * heads * tokens * D;
  R *qh = (R *)malloc(sizeof(R) * n), *kh = (R *)malloc(sizeof(R) * n);
  R *vh = (R *)malloc(sizeof(R) * n), *oh = (R *)malloc(sizeof(R) * n);
  for (size_t g = 0; g < groups; g++)
    for (size_t h = 0; h < heads; h++)
      for (size_t t = 0; t < tokens; t++) {
        size_t dst = ((g * heads + h) * tokens + t) * D;
        for (size_t e = 0; e < D; e++) {
          qh[dst + e] = q[(g * tokens + t) * ldq + h * D + e];
          kh[dst + e] = k[(g * tokens + t) * ldk + h * D + e];
          vh[dst + e] = v[(g * tokens + t) * ldv + h * D + e];
        }
        if (rope) {
          FN(rotate_row)(qh + dst, rope + t * D, rope + (tokens + t) * D, D);
          FN(rotate_row)(kh + dst, rope + (2 * tokens + t) * D, rope + (3 * tokens + t) * D, D);
        }
        /* dense() divides by sqrt(d); the op's q is pre-scaled, so undo that here. */
        for (size_t e = 0; e < D; e++) qh[dst + e] *= (R)8;
      }
  int rc = FN(anc_attention_dense)(qh, kh, vh, groups * heads, tokens, tokens, D, D, oh);
  if (!rc)
    for (size_t g = 0; g < groups; g++)
      for (size_t h = 0; h < heads; h++)
        for (size_t t = 0; t < tokens; t++)
          memcpy(out + ((g * tokens + t) * heads + h) * D, oh + ((g * heads + h) * tokens + t) * D,
                 sizeof(R) * D);
  free(qh);
  free(kh);
  free(vh);
  free(oh);
  return rc;
}

int FN(anc_gated_attention)(const R *packed, size_t groups, size_t tokens, size_t columns,
                            size_t heads, const float *rope, R *out) {
  size_t inner = heads * 64;
  if (columns < heads * (3 * 64 + 1)) return ANC_E_SHAPE;
  int rc = FN(anc_attention_op)(packed, packed + inner, packed + 2 * inner, groups, tokens, heads,
                                columns, columns, columns, rope, out);
  if (rc) return rc;
  for (size_t g = 0; g < groups; g++)
    for (size_t t = 0; t < tokens; t++)
      for (size_t h = 0; h < heads; h++) {
        R gate = packed[(g * tokens + t) * columns + 3 * inner + h];
        R s = (R)1 / ((R)1 + EXP(-gate));
        R *o = out + ((g * tokens + t) * heads + h) * 64;
        for (size_t e = 0; e < 64; e++) o[e] *= s;
      }
  return ANC_OK;
}

void FN(anc_unit_norm)(const R *x, size_t rows, size_t dim, const R *scale, R *out) {
  for (size_t r = 0; r < rows; r++) {
    const R *xr = x + r * dim;
    R sq = 0;
    for (size_t d = 0; d < dim; d++) sq += xr[d] * xr[d];
    R den = FMAX(SQRT(sq), (R)1e-12);
    for (size_t d = 0; d < dim; d++) {
      R y = xr[d] / den;
      out[r * dim + d] = scale ? y * scale[d] : y;
    }
  }
}

void FN(anc_linear)(const R *x, size_t n, size_t k, size_t ldx, const R *w, size_t m,
                    const R *bias, int gelu, const float *rope, size_t tokens, size_t width,
                    const R *residual, R *out) {
  R *acc = (R *)malloc(sizeof(R) * m);
  for (size_t r = 0; r < n; r++) {
    for (size_t c = 0; c < m; c++) acc[c] = 0;
    for (size_t i = 0; i < k; i++) {
      R a = x[r * ldx + i];
      const R *wr = w + i * m;
      for (size_t c = 0; c < m; c++) acc[c] += a * wr[c];
    }
    for (size_t c = 0; c < m; c++) {
      R v = acc[c];
      if (bias) v += bias[c];
      if (gelu) v = v * (R)0.5 * ((R)1 + ERF(v * (R)0.70710678118654752440));
      acc[c] = v;
    }
    if (rope) {
      size_t t = r % tokens;
      for (size_t c = 0; c < 2 * width; c += 64) {
        size_t table = c >= width ? 2 : 0;
        FN(rotate_row)(acc + c, rope + (table * tokens + t) * 64, rope + ((table + 1) * tokens + t) * 64,
                       64);
      }
    }
    for (size_t c = 0; c < m; c++) out[r * m + c] = residual ? acc[c] + residual[r * m + c] : acc[c];
  }
  free(acc);
}

#undef FN
#undef CAT
#undef CAT_
