/*
 * CPU restatement of Ancha's fused RoFormer attention path: TEST INFRASTRUCTURE ONLY.
 *
 * This library is the oracle that the HIP kernels are checked against. Only tests,
 * the smoke check and the benchmark's CPU-baseline leg load it; the product path
 * (ancha_amd/) never links, loads or calls it.
 *
 * Every function exists twice: `_f32` follows the reference's fp32 operation order
 * (the "reference CPU path"), `_f64` runs the same steps in double precision and is
 * used to write golden vectors. Layouts and argument meanings follow the reference
 * functions cited on each declaration (paths relative to the Ancha repository root).
 *
 * Return codes: 0 ok, ANC_E_* (< 0) mirror the reference's `Err(..)` strings.
 */
#ifndef ANCHA_ORACLE_H
#define ANCHA_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  ANC_OK = 0,
  ANC_E_ZERO_DIM = -1,       /* "all dimensions must be positive" */
  ANC_E_NONFINITE_IN = -3,   /* "non-finite input" */
  ANC_E_SCORE_OVERFLOW = -4, /* "score overflow" */
  ANC_E_OUTPUT_OVERFLOW = -5,/* "output overflow" */
  ANC_E_TILE = -6,           /* "tiles must be positive" */
  ANC_E_SHAPE = -7,          /* "invalid projection shape" / "invalid dimensions/epsilon" */
  ANC_E_NORM_OVERFLOW = -8,  /* "norm overflow" */
};

/* splitmix64 -> 53-bit uniform -> Box-Muller normal, times `scale`. Element i of the
 * stream uses splitmix outputs 2*(i/2) and 2*(i/2)+1 (cosine branch for even i, sine
 * branch for odd i), so any slice can be generated independently. */
void anc_fill_normal(float *out, size_t n, uint64_t seed, double scale, size_t first);

/* Interleaved-pair RoPE tables in the packed `[4, tokens, 2*nf]` layout of
 * crates/ancha-models/src/roformer.rs:282-302 (AxisRope::new): query cos, query signed
 * sin (both times 1/sqrt(2*nf)), key cos, key signed sin. Angles are f32 `t*f`. */
void anc_axis_rope_packed(const float *freqs, size_t nf, size_t tokens, float *out);

/* RopeTables::new (roformer.rs:156-175): cos / signed-sin rows of width heads*2*nf, times scale. */
void anc_rope_tables(const float *freqs, size_t nf, size_t tokens, size_t heads, float scale,
                     float *cos_out, float *sin_out);

#define ANC_DECLARE(R, S)                                                                      \
  /* ancha-kernels/src/attention.rs:58-98: softmax(q.k^T / sqrt(d)).v, [group, token, dim]. */ \
  int anc_attention_dense_##S(const R *q, const R *k, const R *v, size_t groups,              \
                              size_t queries, size_t keys, size_t head_dim, size_t value_dim,  \
                              R *out);                                                         \
  /* ancha-kernels/src/attention.rs:103-169: the online-softmax recurrence. */                 \
  int anc_attention_tiled_##S(const R *q, const R *k, const R *v, size_t groups,              \
                              size_t queries, size_t keys, size_t head_dim, size_t value_dim,  \
                              size_t query_tile, size_t key_tile, R *out);                     \
  /* roformer.rs:324-363 (token_major_attention -> prescaled_attention): q already scaled,    \
   * token-major [G, T, H, d] rows with element row strides ld*, heads-major copy, score tiles \
   * of group_tile x query_tile, groups split over `threads` contiguous slices              \
   * (roformer.rs:410-438). Output [G, T, H, d] contiguous. */                                 \
  int anc_token_major_attention_##S(const R *q, const R *k, const R *v, size_t groups,        \
                                    size_t tokens, size_t heads, size_t head_dim, size_t ldq,  \
                                    size_t ldk, size_t ldv, size_t group_tile,                 \
                                    size_t query_tile, size_t threads, R *out);                \
  /* The fused-op contract of crates/ancha-models/src/fused/mod.rs:22-41 (attention) with an \
   * optional packed rope table applied to q and k first (q tables carry 1/sqrt(d)). */        \
  int anc_attention_op_##S(const R *q, const R *k, const R *v, size_t groups, size_t tokens,  \
                           size_t heads, size_t ldq, size_t ldk, size_t ldv,                   \
                           const float *rope, R *out);                                         \
  /* fused/mod.rs:47-55 + fused/attention.rs:208-226: packed [G, T, C] holding q | k | v |    \
   * per-head gate logits; out = softmax(q.k^T).v * sigmoid(gate), [G, T, H, 64]. */            \
  int anc_gated_attention_##S(const R *packed, size_t groups, size_t tokens, size_t columns,  \
                              size_t heads, const float *rope, R *out);                        \
  /* roformer.rs:16-24 unit_norm and :52-54 SourceNorm::forward (scale may be NULL). */        \
  void anc_unit_norm_##S(const R *x, size_t rows, size_t dim, const R *scale, R *out);        \
  /* fused/mod.rs:94-176 + fused/gemm.rs:46-82: out = x[n,k].w[k,m] then bias, erf-GELU,      \
   * interleaved RoPE on columns [0, 2*width) for token row % tokens, residual. */             \
  void anc_linear_##S(const R *x, size_t n, size_t k, size_t ldx, const R *w, size_t m,       \
                      const R *bias, int gelu, const float *rope, size_t tokens, size_t width, \
                      const R *residual, R *out);

ANC_DECLARE(float, f32)
ANC_DECLARE(double, f64)
#undef ANC_DECLARE

/* ancha-kernels/src/fusion.rs:3-46 */
int anc_residual_l2norm(const float *x, const float *residual, const float *gamma, size_t rows,
                        size_t dim, float eps, float *sum, float *norm);
/* ancha-kernels/src/fusion.rs:50-67; w_out holds qkv then gate, b_out zeros then gate_bias. */
int anc_pack_qkv_gate(const float *qkv, size_t qkv_len, const float *gate, size_t gate_len,
                      const float *gate_bias, size_t heads, size_t dim, float *w_out,
                      float *b_out);
/* ancha-kernels/src/fusion.rs:71-81 */
int anc_fold_norm_scale(const float *weights, size_t len, const float *gamma, size_t dim,
                        float *out);
/* crates/ancha-models/src/weights.rs:149-176: W'[i][o] = W[row0+o][i]*input_scale[i]*s. */
void anc_folded_linear(const float *weight, size_t input, size_t row0, size_t row1,
                       const float *input_scale, float output_scale, const float *bias,
                       float *w_out, float *b_out);

/* One RoFormer transformer block (roformer.rs:374-520) on [groups, tokens, dim]. Weights in
 * PyTorch checkpoint layout; `kernels` selects forward_kernels (packed GEMM + gated
 * attention, :464-520) or forward_groups' Burn path (:451-458, Attention::forward
 * :258-270). output_gamma NULL means no per-axis output norm (BS-RoFormer). */
typedef struct {
  size_t dim, heads, head_dim, hidden;
  const float *attn_gamma;    /* [dim] layers.0.0.norm.gamma */
  const float *to_qkv;        /* [3*inner, dim] */
  const float *to_gates;      /* [heads, dim] */
  const float *to_gates_bias; /* [heads] */
  const float *to_out;        /* [dim, inner] */
  const float *freqs;         /* [head_dim/2] */
  const float *ff_gamma;      /* [dim] layers.0.1.net.0.gamma */
  const float *ff_in;         /* [hidden, dim] */
  const float *ff_in_bias;    /* [hidden] */
  const float *ff_out;        /* [dim, hidden] */
  const float *ff_out_bias;   /* [dim] */
  const float *output_gamma;  /* [dim] or NULL */
} anc_block_weights;

int anc_transformer_forward(const anc_block_weights *w, const float *x, size_t groups,
                            size_t tokens, int kernels, size_t threads, float *out);

/* ---- mel_oracle.c: Mel/BS-RoFormer front end, mask estimator and STFT ---- */

/* crates/ancha-audio/src/dsp.rs:139-147 */
size_t anc_reflect_index(long index, size_t length);
/* dsp.rs:46-84 Stft::forward: out [n / hop + 1][n_fft / 2 + 1][re, im]. */
int anc_stft(const float *signal, size_t n, size_t n_fft, size_t hop, float *out);
/* dsp.rs:86-134 Stft::inverse: spectrum [frames][n_fft / 2 + 1][re, im] -> out [length]. */
int anc_istft(const float *spectrum, size_t frames, size_t n_fft, size_t hop, size_t length,
              int zero_dc, float *out);
/* crates/ancha-models/src/network.rs:316-323 (+ :96-121 folding): x [bands][t][dim]. */
int anc_band_split(const float *spectrum, size_t t, size_t cols, size_t bands,
                   const size_t *offsets, const size_t *bins, size_t dim, const float *gamma,
                   const float *weight, const float *bias, size_t threads, float *x);
/* network.rs:138-177 + :365-398: one stem's masks [2 * fft_bins][2][t]. */
int anc_mask_head(const float *x, size_t t, size_t bands, const size_t *offsets,
                  const size_t *bins, size_t fft_bins, size_t dim, size_t hidden, size_t layers,
                  const float *const *hw, const float *const *hb, const float *ow,
                  const float *ob, size_t threads, float *masks);

#ifdef __cplusplus
}
#endif
#endif
