// One RoFormer transformer block on the gfx950 kernels (C ABI of include/ancha_hip.h):
// load-time weight packing and the forward pass, host code only.
//
// Mirrors crates/ancha-models/src/roformer.rs: `Attention::load` (:205-244) folds sqrt(dim)*gamma
// of the pre-attention norm into the q / k / v / gate projections and packs them side by side
// (zero-padded to a multiple of 128 columns, gate bias in the packed bias); `Transformer::load`
// (:381-409) folds the feed-forward norm into ff_in; `Transformer::forward_kernels` (:464-520)
// runs packed GEMM (RoPE epilogue) -> gated attention -> out GEMM (+x) -> ff_in GEMM (bias,
// GELU) -> ff_out GEMM (bias, +x) -> optional output norm. Here the two unit_norm calls are
// fused into the GEMMs that consume them (ancha_hip_norm_linear).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <new>
#include <vector>

#include "../../include/ancha_hip.h"

struct ancha_hip_block {
  size_t dim, heads, hidden, inner, columns;
  int device;
  float* packed_w;    // [dim, columns]
  float* packed_b;    // [columns]
  float* out_w;       // [inner, dim]
  float* ff_in_w;     // [dim, hidden]
  float* ff_in_b;     // [hidden]
  float* ff_out_w;    // [hidden, dim]
  float* ff_out_b;    // [dim]
  float* out_scale;   // [dim] sqrt(dim)*output_gamma, or null
};

namespace {

constexpr size_t kHeadDim = ANCHA_ATTENTION_HEAD_DIM;

// sqrt(dim) * gamma, with the root formed in fp32 like the reference (SourceNorm::scale).
std::vector<float> source_scale(const float* gamma, size_t dim) {
  const float root = std::sqrt(static_cast<float>(dim));
  std::vector<float> s(dim);
  for (size_t i = 0; i < dim; i++) s[i] = gamma[i] * root;
  return s;
}

// W'[i][c0 + o] = W[row0 + o][i] * scale[i] for o < outs: a PyTorch [out, in] block written
// transposed into columns [c0, c0 + outs) of a row-major [in, ld] matrix
// (folded_linear, weights.rs:149-176).
void fold_into(const float* w, size_t in, size_t row0, size_t outs, const float* scale,
               float* dst, size_t ld, size_t c0) {
  for (size_t o = 0; o < outs; o++)
    for (size_t i = 0; i < in; i++)
      dst[i * ld + c0 + o] = w[(row0 + o) * in + i] * (scale ? scale[i] : 1.0f);
}

int upload(const std::vector<float>& host, float** dev) {
  *dev = nullptr;
  if (host.empty()) return 0;
  hipError_t e = hipMalloc(reinterpret_cast<void**>(dev), host.size() * sizeof(float));
  if (e == hipSuccess)
    e = hipMemcpy(*dev, host.data(), host.size() * sizeof(float), hipMemcpyHostToDevice);
  return e == hipSuccess ? 0 : -static_cast<int>(e);
}

size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

}  // namespace

extern "C" {

int ancha_hip_block_create(size_t dim, size_t heads, size_t hidden, const float* attn_gamma,
                           const float* to_qkv, const float* to_gates,
                           const float* to_gates_bias, const float* to_out,
                           const float* ff_gamma, const float* ff_in, const float* ff_in_bias,
                           const float* ff_out, const float* ff_out_bias,
                           const float* output_gamma, ancha_hip_block** block) {
  if (!block) return ANCHA_HIP_INVALID;
  *block = nullptr;
  if (!attn_gamma || !to_qkv || !to_gates || !to_gates_bias || !to_out || !ff_gamma || !ff_in ||
      !ff_in_bias || !ff_out || !ff_out_bias || dim == 0 || heads == 0 || hidden == 0)
    return ANCHA_HIP_INVALID;
  const size_t inner = heads * kHeadDim;
  const size_t columns = round_up(3 * inner + heads, 128);
  // forward_kernels' shape gate (roformer.rs:471-475).
  if (!ancha_hip_linear_supported(dim, columns) || !ancha_hip_linear_supported(inner, dim) ||
      !ancha_hip_linear_supported(dim, hidden) || !ancha_hip_linear_supported(hidden, dim))
    return ANCHA_HIP_UNSUPPORTED;

  const std::vector<float> norm = source_scale(attn_gamma, dim);
  const std::vector<float> ffs = source_scale(ff_gamma, dim);
  std::vector<float> pw(dim * columns, 0.0f), pb(columns, 0.0f);
  fold_into(to_qkv, dim, 0, inner, norm.data(), pw.data(), columns, 0);
  fold_into(to_qkv, dim, inner, inner, norm.data(), pw.data(), columns, inner);
  fold_into(to_qkv, dim, 2 * inner, inner, norm.data(), pw.data(), columns, 2 * inner);
  fold_into(to_gates, dim, 0, heads, norm.data(), pw.data(), columns, 3 * inner);
  for (size_t h = 0; h < heads; h++) pb[3 * inner + h] = to_gates_bias[h];
  std::vector<float> ow(inner * dim), w1(dim * hidden), w2(hidden * dim);
  fold_into(to_out, inner, 0, dim, nullptr, ow.data(), dim, 0);
  fold_into(ff_in, dim, 0, hidden, ffs.data(), w1.data(), hidden, 0);
  fold_into(ff_out, hidden, 0, dim, nullptr, w2.data(), dim, 0);
  const std::vector<float> b1(ff_in_bias, ff_in_bias + hidden), b2(ff_out_bias, ff_out_bias + dim);
  std::vector<float> os;
  if (output_gamma) os = source_scale(output_gamma, dim);

  auto* b = new (std::nothrow) ancha_hip_block{};
  if (!b) return ANCHA_HIP_INVALID;
  b->dim = dim;
  b->heads = heads;
  b->hidden = hidden;
  b->inner = inner;
  b->columns = columns;
  if (hipGetDevice(&b->device) != hipSuccess) b->device = 0;
  int rc = 0;
  if (!rc) rc = upload(pw, &b->packed_w);
  if (!rc) rc = upload(pb, &b->packed_b);
  if (!rc) rc = upload(ow, &b->out_w);
  if (!rc) rc = upload(w1, &b->ff_in_w);
  if (!rc) rc = upload(b1, &b->ff_in_b);
  if (!rc) rc = upload(w2, &b->ff_out_w);
  if (!rc) rc = upload(b2, &b->ff_out_b);
  if (!rc) rc = upload(os, &b->out_scale);
  if (rc) {
    ancha_hip_block_destroy(b);
    return rc;
  }
  *block = b;
  return ANCHA_HIP_OK;
}

size_t ancha_hip_block_workspace(const ancha_hip_block* b, size_t rows) {
  if (!b) return 0;
  // packed projection (later reused for the FF hidden activation), attention output, x + attn.
  const size_t first = b->columns > b->hidden ? b->columns : b->hidden;
  return rows * (round_up(first, 64) + b->inner + b->dim) * sizeof(float);
}

int ancha_hip_block_forward(const ancha_hip_block* b, const float* x, size_t groups,
                            size_t tokens, const float* rope, void* workspace,
                            size_t workspace_bytes, float* out, hipStream_t stream) {
  if (!b) return ANCHA_HIP_INVALID;
  const size_t rows = groups * tokens;
  if (rows == 0) return ANCHA_HIP_OK;
  if (!x || !out || !rope || !workspace) return ANCHA_HIP_INVALID;
  if (workspace_bytes < ancha_hip_block_workspace(b, rows)) return ANCHA_HIP_INVALID;
  const size_t first = b->columns > b->hidden ? b->columns : b->hidden;
  float* packed = static_cast<float*>(workspace);       // [rows, columns], then [rows, hidden]
  float* attended = packed + rows * round_up(first, 64);  // [rows, inner]
  float* x1 = attended + rows * b->inner;                // [rows, dim]
  const size_t dim = b->dim, inner = b->inner;
  int rc = ancha_hip_norm_linear(x, rows, dim, dim, b->packed_w, b->columns, b->packed_b, 0, rope,
                                 tokens, inner, nullptr, packed, stream);
  if (rc) return rc;
  rc = ancha_hip_gated_attention(packed, groups, tokens, b->columns, b->heads, nullptr, attended,
                                 stream);
  if (rc) return rc;
  rc = ancha_hip_linear(attended, rows, inner, inner, b->out_w, dim, nullptr, 0, nullptr, 0, 0, x,
                        x1, stream);
  if (rc) return rc;
  float* hidden = packed;
  rc = ancha_hip_norm_linear(x1, rows, dim, dim, b->ff_in_w, b->hidden, b->ff_in_b, 1, nullptr, 0,
                             0, nullptr, hidden, stream);
  if (rc) return rc;
  rc = ancha_hip_linear(hidden, rows, b->hidden, b->hidden, b->ff_out_w, dim, b->ff_out_b, 0,
                        nullptr, 0, 0, x1, out, stream);
  if (rc) return rc;
  if (b->out_scale) rc = ancha_hip_unit_norm(out, rows, dim, dim, b->out_scale, out, stream);
  return rc;
}

size_t ancha_hip_axis_pair_workspace(const ancha_hip_block* time, const ancha_hip_block* band,
                                     size_t rows) {
  if (!time || !band || time->dim != band->dim) return 0;
  const size_t a = ancha_hip_block_workspace(time, rows), c = ancha_hip_block_workspace(band, rows);
  return (a > c ? a : c) + 2 * rows * time->dim * sizeof(float);
}

int ancha_hip_axis_pair_forward(const ancha_hip_block* time, const ancha_hip_block* band,
                                const float* x, size_t batch, size_t bands, size_t frames,
                                const float* time_rope, const float* band_rope, void* workspace,
                                size_t workspace_bytes, float* out, hipStream_t stream) {
  if (!time || !band || time->dim != band->dim) return ANCHA_HIP_INVALID;
  const size_t rows = batch * bands * frames, dim = time->dim;
  if (rows == 0) return ANCHA_HIP_OK;
  if (!x || !out || !time_rope || !band_rope || !workspace) return ANCHA_HIP_INVALID;
  const size_t need = ancha_hip_axis_pair_workspace(time, band, rows);
  if (workspace_bytes < need) return ANCHA_HIP_INVALID;
  float* a = static_cast<float*>(workspace);
  float* c = a + rows * dim;
  void* inner = c + rows * dim;
  const size_t inner_bytes = need - 2 * rows * dim * sizeof(float);
  // Time pass: groups = batch * bands, sequence = frames.
  int rc = ancha_hip_block_forward(time, x, batch * bands, frames, time_rope, inner, inner_bytes,
                                   a, stream);
  if (!rc) rc = ancha_hip_swap_axes(a, batch, bands, frames, dim, c, stream);
  // Band pass: groups = batch * frames, sequence = bands.
  if (!rc) rc = ancha_hip_block_forward(band, c, batch * frames, bands, band_rope, inner,
                                        inner_bytes, a, stream);
  if (!rc) rc = ancha_hip_swap_axes(a, batch, frames, bands, dim, out, stream);
  return rc;
}

void ancha_hip_block_destroy(ancha_hip_block* b) {
  if (!b) return;
  for (float* p : {b->packed_w, b->packed_b, b->out_w, b->ff_in_w, b->ff_in_b, b->ff_out_w,
                   b->ff_out_b, b->out_scale})
    if (p) (void)hipFree(p);
  delete b;
}

}  // extern "C"
