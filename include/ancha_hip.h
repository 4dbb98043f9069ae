/*
 * ancha_hip.h - C ABI of the MI355X (gfx950) fused RoFormer attention path.
 *
 * Drop-in replacement for the CUDA-only entry points of Ancha's op boundary
 * `ancha_models::fused` (crates/ancha-models/src/fused/mod.rs). Each function below names the
 * reference item it replaces. All tensors are caller-owned device buffers of fp32 values,
 * row-major, with explicit row strides in elements; the library writes only `out` and
 * allocates no device memory per call. Every call is stream-ordered on `stream` (0 = the
 * null stream), does not synchronise the host and is safe to call from several host threads
 * on different streams.
 *
 * Return codes:
 *   ANCHA_HIP_OK (0)            success (launched on `stream`).
 *   ANCHA_HIP_UNSUPPORTED (1)   shape / option outside what the kernels cover; nothing was
 *                               launched. This is the reference's `None`: the caller keeps its
 *                               own implementation as the fallback.
 *   ANCHA_HIP_INVALID (2)       arguments break the op contract (the reference's `assert!`
 *                               panics inside `launch`): null pointers, column ranges that do
 *                               not fit the row stride, ...; nothing was launched.
 *   < 0                         a HIP runtime error, -(hipError_t). The failure is sticky, like
 *                               the reference's `device::check` (src/device.rs:11-41): every
 *                               later call returns it again without launching anything.
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

/* Sticky device-failure check: 0, or the first HIP error (< 0) any call has met.
 * Replaces `device::check()` (src/device.rs:30-41) for this path. */
int ancha_hip_check(void);

/* Human-readable description of the calling thread's last non-zero return. */
const char *ancha_hip_last_error(void);

#ifdef __cplusplus
}
#endif
#endif /* ANCHA_HIP_H */
