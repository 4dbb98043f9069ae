/*
 * ancha_hip.h - C ABI of the MI355X (gfx950) fused RoFormer attention path.
 *
 * Drop-in replacement for the CUDA-only entry points of Ancha's op boundary
 * `ancha_models::fused` (crates/ancha-models/src/fused/mod.rs). Each function below names the
 * reference item it replaces. All tensors are caller-owned device buffers of fp32 values,
 * row-major, with explicit row strides in elements; the library writes only `out` (and the
 * caller's workspace) and allocates no device memory per call (the *_create calls allocate
 * a model's weights once). Every call is stream-ordered on `stream` (0 = the null stream),
 * does not synchronise the host (except ancha_hip_separate, once at its end, and *_create)
 * and is safe to call from several host threads on different streams.
 *
 * Return codes:
 *   ANCHA_HIP_OK (0)            success (launched on `stream`).
 *   ANCHA_HIP_UNSUPPORTED (1)   shape / option outside what the kernels cover; nothing was
 *                               launched. This is the reference's `None`: the caller keeps its
 *                               own implementation as the fallback.
 *   ANCHA_HIP_INVALID (2)       arguments break the op contract (the reference's `assert!`
 *                               panics inside `launch`): null pointers, column ranges that do
 *                               not fit the row stride, ...; nothing was launched.
 *   ANCHA_HIP_CANCELLED (3)     the caller's cancellation flag was set (the reference's "task
 *                               cancelled", src/runtime.rs:118; network.rs:334,367).
 *   < 0                         a HIP runtime error, -(hipError_t). The failure is sticky, like
 *                               the reference's `device::check` (src/device.rs:11-41): every
 *                               later call of any entry point returns it again without
 *                               launching anything.
 * ancha_hip_last_error() describes the most recent non-zero return of the calling thread.
 */
#ifndef ANCHA_HIP_H
#define ANCHA_HIP_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The HIP runtime's stream handle (same definition as <hip/hip_runtime_api.h>). */
typedef struct ihipStream_t *hipStream_t;

#define ANCHA_HIP_OK 0
#define ANCHA_HIP_UNSUPPORTED 1
#define ANCHA_HIP_INVALID 2
#define ANCHA_HIP_CANCELLED 3

/* Head width the attention kernels are specialised for.
 * Replaces `pub const ATTENTION_HEAD_DIM: usize = 64` (fused/mod.rs:18). */
#define ANCHA_ATTENTION_HEAD_DIM 64

/* 1 when a gfx950 device is present and the kernels can run on the current device, else 0.
 * Replaces `fused::available::<B>()` (fused/mod.rs:250-255). */
int ancha_hip_available(void);

/* softmax(q.k^T).v per (group, head), q pre-scaled, scores never materialised.
 * q, k, v: [groups, tokens, heads*64] with row strides ldq, ldk, ldv (>= heads*64; the group
 * stride is tokens*ld); out: [groups, tokens, heads, 64] contiguous.
 * rope: NULL (q and k already rotated, q scaled by 1/sqrt(64): exactly the reference op), or
 * the packed [4, tokens, 64] table of AxisRope::packed (roformer.rs:282-302: query cos and
 * signed sin carrying 1/sqrt(64), key cos and signed sin), applied to q and k as they load.
 * Replaces `fused::attention(q, k, v)` (fused/mod.rs:22-41; kernel fused/attention.rs:26-298);
 * a head width other than 64 is the caller-side `None` of :27. */
int ancha_hip_attention(const float *q, const float *k, const float *v, size_t groups,
                        size_t tokens, size_t heads, size_t ldq, size_t ldk, size_t ldv,
                        const float *rope, float *out, hipStream_t stream);

/* The RoFormer attention core from one packed projection: packed [groups, tokens, columns]
 * holds q | k | v (heads*64 columns each, from column 0) and the per-head gate logits after
 * them; out = softmax(q.k^T).v * sigmoid(gate), [groups, tokens, heads, 64] contiguous.
 * `rope` as in ancha_hip_attention. Returns ANCHA_HIP_UNSUPPORTED when
 * columns < heads*(3*64+1), like the reference's `None`.
 * Replaces `fused::gated_attention(packed, heads)` (fused/mod.rs:47-55, kernel columns
 * fused/mod.rs:342-352). */
int ancha_hip_gated_attention(const float *packed, size_t groups, size_t tokens, size_t columns,
                              size_t heads, const float *rope, float *out, hipStream_t stream);

/* Whether the projection GEMM covers [n, k].[k, m] with its full 128-column tile:
 * k % 8 == 0 and m % 128 == 0 (both > 0). Other positive m still run as bare products.
 * Replaces `fused::linear_supported(k, m)` (fused/mod.rs:83-85). */
int ancha_hip_linear_supported(size_t k, size_t m);

/* out [n, m] = epilogue(x . w): x [n, k] with row stride ldx, w [k, m] row-major (the
 * reference's Burn `Linear` [in, out] layout), out [n, m] contiguous. Epilogue applied in the
 * reference's order (fused/gemm.rs:46-82): bias [m] (or NULL); erf-GELU if gelu != 0; rotary if
 * rope != NULL: the packed [4, tokens, 64] AxisRope table, columns [0, width) of row r rotated
 * as queries and [width, 2*width) as keys of token r % tokens; residual [n, m] contiguous (or
 * NULL; may alias out). fp16 MFMA operands, fp32 accumulation.
 * Returns ANCHA_HIP_UNSUPPORTED where the reference returns `None`: k == 0, k % 8 != 0, m == 0;
 * an epilogue with m % 128 != 0; rotary with tokens == 0, n % tokens != 0, width % 64 != 0 or
 * 2*width > m.
 * Replaces `fused::linear(x, weight, Epilogue{bias, gelu, rotary, residual})`
 * (fused/mod.rs:58-176; kernel fused/gemm.rs:86-311). */
int ancha_hip_linear(const float *x, size_t n, size_t k, size_t ldx, const float *w, size_t m,
                     const float *bias, int gelu, const float *rope, size_t tokens, size_t width,
                     const float *residual, float *out, hipStream_t stream);

/* ancha_hip_linear applied to unit_norm(x) without materialising it: each row's product is
 * scaled by 1 / max(||x_r||_2, 1e-12) before the epilogue. Same arguments and return codes.
 * Replaces the pair `fused::linear(&unit_norm(x), weight, epilogue)` of
 * Transformer::forward_kernels (roformer.rs:477-485 and :497-505; unit_norm :16-24). */
int ancha_hip_norm_linear(const float *x, size_t n, size_t k, size_t ldx, const float *w,
                          size_t m, const float *bias, int gelu, const float *rope,
                          size_t tokens, size_t width, const float *residual, float *out,
                          hipStream_t stream);

/* out[r] = x[r] / max(||x[r]||_2, 1e-12) * scale: x [rows, dim] with row stride ldx, scale
 * [dim] or NULL, out [rows, dim] contiguous (may alias x when ldx == dim).
 * Replaces `unit_norm` (roformer.rs:16-24) and, with scale = sqrt(dim)*gamma,
 * `SourceNorm::forward` (roformer.rs:43-54). */
int ancha_hip_unit_norm(const float *x, size_t rows, size_t dim, size_t ldx, const float *scale,
                        float *out, hipStream_t stream);

/* One RoFormer transformer block on the kernels above (opaque handle, device-resident
 * packed weights). */
typedef struct ancha_hip_block ancha_hip_block;

/* Load-time packing of one block from host fp32 weights in PyTorch nn.Linear layout
 * ([out, in]): attn_gamma [dim], to_qkv [3*heads*64, dim], to_gates [heads, dim],
 * to_gates_bias [heads], to_out [dim, heads*64], ff_gamma [dim], ff_in [hidden, dim],
 * ff_in_bias [hidden], ff_out [dim, hidden], ff_out_bias [dim], output_gamma [dim] or NULL.
 * sqrt(dim)*gamma folds into the following projections' input rows and q | k | v | gates are
 * packed side by side, zero-padded to a multiple of 128 columns. Allocates the device weights
 * on the current device. UNSUPPORTED when a projection shape fails ancha_hip_linear_supported.
 * Replaces `Transformer::load` + `Attention::load` (roformer.rs:381-409, :205-244; folding
 * weights.rs:149-176). */
int ancha_hip_block_create(size_t dim, size_t heads, size_t hidden, const float *attn_gamma,
                           const float *to_qkv, const float *to_gates,
                           const float *to_gates_bias, const float *to_out,
                           const float *ff_gamma, const float *ff_in, const float *ff_in_bias,
                           const float *ff_out, const float *ff_out_bias,
                           const float *output_gamma, ancha_hip_block **block);

/* Device bytes of the workspace ancha_hip_block_forward needs for `rows` = groups*tokens. */
size_t ancha_hip_block_workspace(const ancha_hip_block *block, size_t rows);

/* y = block(x): x, out [groups, tokens, dim] contiguous (out may alias x); rope the packed
 * [4, tokens, 64] AxisRope table of this axis; workspace >= ancha_hip_block_workspace bytes.
 * x + gated attention(unit_norm x) -> x + FF(unit_norm x) -> optional output norm, on the
 * packed-projection path with RoPE in the QKV epilogue. Allocates nothing.
 * Replaces `Transformer::forward_kernels` (roformer.rs:464-520). */
int ancha_hip_block_forward(const ancha_hip_block *block, const float *x, size_t groups,
                            size_t tokens, const float *rope, void *workspace,
                            size_t workspace_bytes, float *out, hipStream_t stream);

void ancha_hip_block_destroy(ancha_hip_block *block);

/* out [batch, b, a, dim] = x [batch, a, b, dim] with axes 1 and 2 swapped (contiguous; out
 * must not alias x). Replaces the dense `swap_dims` copies between the time and band passes
 * (network.rs:336-338; `dense` roformer.rs:57-70). */
int ancha_hip_swap_axes(const float *x, size_t batch, size_t a, size_t b, size_t dim, float *out,
                        hipStream_t stream);

/* Device bytes of the workspace ancha_hip_axis_pair_forward needs for
 * rows = batch*bands*frames. */
size_t ancha_hip_axis_pair_workspace(const ancha_hip_block *time, const ancha_hip_block *band,
                                     size_t rows);

/* One time pass + band pass of the RoFormer axis loop: x, out [batch, bands, frames, dim]
 * contiguous (out may alias x); the time block runs on groups = batch*bands with sequence
 * frames, then the band block on groups = batch*frames with sequence bands, in place on the
 * same rows: its attention reads each band sequence with a row stride of `frames` and its
 * rotary epilogue takes the band index (row / frames) % bands, so no transposed copy is made.
 * time_rope [4, frames, 64], band_rope [4, bands, 64]. Allocates nothing. Replaces one
 * iteration of the axis loop of the RoFormer networks (network.rs:333-339), whose two dense
 * `swap_dims` copies it removes. */
int ancha_hip_axis_pair_forward(const ancha_hip_block *time, const ancha_hip_block *band,
                                const float *x, size_t batch, size_t bands, size_t frames,
                                const float *time_rope, const float *band_rope, void *workspace,
                                size_t workspace_bytes, float *out, hipStream_t stream);

/* ---- Mel/BS-RoFormer network and separation runtime around the attention path ---- */

/* Model configuration: the fields of ModelConfig (crates/ancha-models/src/config.rs:14-32).
 * Band b covers FFT bins band_bins[band_offsets[b] .. band_offsets[b+1]) (strictly increasing
 * within a band; every bin covered). n_fft must be 2048 and head_dim 64. */
typedef struct {
  int mel;               /* 1: Mel-Band-RoFormer (per-block output norms), 0: BS-RoFormer */
  size_t dim, depth, heads, head_dim, ff_mult, mask_depth, mask_expansion;
  size_t n_fft, hop, chunk_samples, overlap;
  int zero_dc;
  size_t stems, bands;
  const size_t *band_offsets; /* [bands + 1] */
  const size_t *band_bins;    /* [band_offsets[bands]] */
} ancha_hip_roformer_config;

/* Serves the checkpoint tensor `name` (the reference's safetensors names, e.g.
 * "band_split.to_features.3.1.weight") as `numel` host fp32 values, or NULL when absent. The
 * pointer must stay valid until ancha_hip_roformer_create returns. */
typedef const float *(*ancha_hip_tensor_fn)(void *ctx, const char *name, size_t numel);

typedef struct ancha_hip_roformer ancha_hip_roformer;

/* Loads the network on the current device: band-split projections (sqrt(width)*gamma folded),
 * depth x (time, frequency) blocks, BS final norm, per-stem mask heads (fp16 weights, output
 * projections padded to multiples of 128 columns). INVALID for a config the schema rejects or
 * a missing tensor, UNSUPPORTED for shapes outside the kernels.
 * Replaces `Roformer::load` / `Roformer::build` (crates/ancha-models/src/network.rs:79-278). */
int ancha_hip_roformer_create(const ancha_hip_roformer_config *config, ancha_hip_tensor_fn get,
                              void *ctx, ancha_hip_roformer **model);

/* Device bytes of the workspace ancha_hip_roformer_forward needs for `frames` frames. */
size_t ancha_hip_roformer_workspace(const ancha_hip_roformer *model, size_t frames);

/* masks [stems][2 * 1025][re, im][frames] = model(spectrum [frames][1025][channel][re, im]):
 * band split -> axis loop (the frequency pass reads the time layout in place) -> mask heads
 * (tanh hidden layers, GLU, overlapping-band average). Allocates nothing and does not wait:
 * the rotary tables of the chunk's frame count are built at create time, those of any other
 * frame count in the workspace by the call itself. Calls sharing a model may run concurrently
 * on different streams with different workspaces.
 * `cancelled` (or NULL): checked before each layer pair and each mask head like the reference's
 * `&AtomicBool`; a set flag returns ANCHA_HIP_CANCELLED, and the work already enqueued on
 * `stream` still runs (synchronise it before releasing the buffers).
 * Replaces `Roformer::forward` (network.rs:303-400). */
int ancha_hip_roformer_forward(ancha_hip_roformer *model, const float *spectrum, size_t frames,
                               void *workspace, size_t workspace_bytes, float *masks,
                               const volatile int *cancelled, hipStream_t stream);

/* The chunk plan ancha_hip_separate runs for a clip of `samples` samples per channel: chunks
 * of `chunk_samples` start every chunk_samples / overlap samples across the clip plus a
 * reflected border of chunk_samples - step samples on each side (0 when the clip is not longer
 * than two borders). Writes the chunk count (the reference's `report.chunks`, 0 for an empty
 * clip) and the border to the non-NULL pointers. Host only. ANCHA_HIP_INVALID for a zero chunk,
 * a zero overlap or overlap > chunk_samples ("invalid chunk or overlap divisor").
 * Replaces `ChunkPlan::new` / `ChunkPlan::starts` (crates/ancha-audio/src/chunk.rs:9-24) and the
 * border rule of src/runtime.rs:103-111. */
int ancha_hip_chunk_plan(size_t chunk_samples, size_t overlap, size_t samples, size_t *chunks,
                         size_t *border);

/* Device bytes of the workspace ancha_hip_separate needs for a clip of `samples` samples. */
size_t ancha_hip_separate_workspace(const ancha_hip_roformer *model, size_t samples);

/* stems [stems][2][samples] (and, for one-stem models, residual [2][samples] = audio - stem, or
 * NULL) from stereo audio [2][samples], all device memory: reflect-bordered chunks every
 * chunk_samples / overlap samples, STFT, forward, complex masks, iSTFT, fade-weighted
 * overlap-add, border crop. Allocates nothing. The reference runtime's checks run on the
 * device and are read back once, at the end (the call waits for `stream` there): a
 * non-finite input sample, model output or chunk output, or an uncovered iSTFT / overlap-add
 * sample returns ANCHA_HIP_INVALID with the reference's message (runtime.rs:172-176;
 * crates/ancha-audio/src/dsp.rs:57-60,126-131; chunk.rs:57-60,76-79); the stems are then not
 * valid. `cancelled` (or NULL) is checked before each pair of chunks, each layer pair and each
 * mask head; a set flag returns ANCHA_HIP_CANCELLED after the enqueued work has finished.
 * Replaces the chunk loop of src/runtime.rs:103-238 (+ residual_audio, :403-420). */
int ancha_hip_separate(ancha_hip_roformer *model, const float *audio, size_t samples,
                       void *workspace, size_t workspace_bytes, float *stems, float *residual,
                       const volatile int *cancelled, hipStream_t stream);

void ancha_hip_roformer_destroy(ancha_hip_roformer *model);

/* Stft::forward (crates/ancha-audio/src/dsp.rs:46-84) of both channels of signal
 * [2][samples]: spectrum [samples / hop + 1][1025][channel][re, im] (n_fft 2048, periodic
 * Hann, reflect padding, unnormalised). */
int ancha_hip_stft(const float *signal, size_t samples, size_t hop, float *spectrum,
                   hipStream_t stream);

size_t ancha_hip_istft_workspace(size_t frames);

/* Stft::inverse (dsp.rs:86-134) of spectrum * masks for both channels: spectrum as above,
 * masks [2 * 1025][re, im][frames] (complex, per row 2*bin + channel), out [2][length]. */
int ancha_hip_istft(const float *spectrum, const float *masks, size_t frames, size_t hop,
                    size_t length, int zero_dc, void *workspace, size_t workspace_bytes,
                    float *out, hipStream_t stream);

/* ancha_hip_istft without a workspace argument, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops). No counterpart in the reference.
 * The inverse frames go to a static device array of the library (24 MiB per GPU, held until
 * the process ends), so `frames` is at most 1536 (ANCHA_HIP_UNSUPPORTED beyond, with a
 * message). Allocates nothing. Calls that overlap on one GPU (other streams or threads) share
 * that array and race: serialise them. Results equal ancha_hip_istft's. */
int ancha_hip_istft_noalloc(const float *spectrum, const float *masks, size_t frames, size_t hop,
                            size_t length, int zero_dc, float *out, hipStream_t stream);

/* Sticky device-failure check: 0, or the first HIP error (< 0) any call has met.
 * Replaces `device::check()` (src/device.rs:30-41) for this path. */
int ancha_hip_check(void);

/* Human-readable description of the calling thread's last non-zero return. */
const char *ancha_hip_last_error(void);

#ifdef __cplusplus
}
#endif
#endif /* ANCHA_HIP_H */
