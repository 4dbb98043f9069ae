// One RoFormer transformer block on the gfx950 kernels (C ABI of include/ancha_hip.h):
// load-time weight packing and the forward pass, host code only.
//
// Mirrors crates/ancha-models/src/roformer.rs: `Attention::load` (:205-244) folds sqrt(dim)*gamma
// of the pre-attention norm into the q / k / v / gate projections and packs them side by side
// (zero-padded to a multiple of 128 columns, gate bias in the packed bias); `Transformer::load`
// (:381-409) folds the feed-forward norm into ff_in; `Transformer::forward_kernels` (:464-520)
// runs packed GEMM (RoPE epilogue) -> gated attention -> out GEMM (+x) -> ff_in GEMM (bias,
// GELU) -> ff_out GEMM (bias, +x) -> optional output norm. Here each unit_norm writes the fp16
// row its GEMM rounds its operand to (norm_half), and the packed projection, the attention
// output and the feed-forward hidden activation stay fp16.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>
#include <new>
#include <vector>

#include "../../include/ancha_hip.h"
#include "kernels.hpp"
#include "status.hpp"

// Weights are stored as fp16 W^T [out][in] (the PyTorch layout, folded scales applied before
// rounding): the GEMMs round every operand to fp16 anyway, so converting once at load time
// changes no result and halves the weight bytes each GEMM tile reads.
struct ancha_hip_block {
  size_t dim, heads, hidden, inner, columns;
  int device;
  _Float16* packed_w;  // [columns, dim]: q | k | v | gates | zero rows
  float* packed_b;     // [columns]
  _Float16* out_w;     // [dim, inner]
  _Float16* ff_in_w;   // [hidden, dim]
  float* ff_in_b;      // [hidden]
  _Float16* ff_out_w;  // [dim, hidden]
  float* ff_out_b;     // [dim]
  float* out_scale;    // [dim] sqrt(dim)*output_gamma, or null
  // Fragment-major copies for the fused tail (tail.hip), or null where it does not apply:
  // W_out^T, W1'^T and W2^T (the last two with their k axis in kPerm16 order).
  _Float16 *wo_frag = nullptr, *w1_frag = nullptr, *w2_frag = nullptr;
  // Fragment-major copy of the packed projection for qkv.hip, or null.
  _Float16* packed_frag = nullptr;
};

namespace ancha {

// Fragment-major copy of W^T [rows][k] (k contiguous) for the A operand of the 32x32x16 MFMA
// in tail.hip: fragment (b, s) is 512 halves at (b * (k / 16) + s) * 512, lane l's 8 at 8 l,
// holding W^T[32 b + l % 32][16 s + perm(8 (l / 32) + t)] for t < 8, perm = kPerm16 (or the
// identity). rows % 32 == 0, k % 16 == 0.
std::vector<_Float16> fragment_major(const std::vector<_Float16>& wt, size_t rows, size_t k,
                                     bool permute) {
  std::vector<_Float16> out(rows * k);
  const size_t steps = k / 16;
  for (size_t b = 0; b < rows / 32; b++)
    for (size_t s = 0; s < steps; s++)
      for (size_t l = 0; l < 64; l++)
        for (size_t t = 0; t < 8; t++) {
          const size_t kk = 8 * (l / 32) + t;
          const size_t src = 16 * s + (permute ? static_cast<size_t>(ancha::kPerm16[kk]) : kk);
          out[((b * steps + s) * 64 + l) * 8 + t] = wt[(32 * b + l % 32) * k + src];
        }
  return out;
}

}  // namespace ancha

namespace {

constexpr size_t kHeadDim = ANCHA_ATTENTION_HEAD_DIM;

// sqrt(dim) * gamma, with the root formed in fp32 like the reference (SourceNorm::scale).
std::vector<float> source_scale(const float* gamma, size_t dim) {
  const float root = std::sqrt(static_cast<float>(dim));
  std::vector<float> s(dim);
  for (size_t i = 0; i < dim; i++) s[i] = gamma[i] * root;
  return s;
}

// dst[(r0 + o)][i] = fp16(W[row0 + o][i] * scale[i]) for o < outs: rows of a PyTorch
// [out, in] matrix with the folded input scale (folded_linear's W'[i][o] = W[o][i]*scale[i],
// weights.rs:149-176, kept in [out][in] order), rounded to fp16 (round to nearest even).
void fold_rows(const float* w, size_t in, size_t row0, size_t outs, const float* scale,
               _Float16* dst, size_t r0) {
  for (size_t o = 0; o < outs; o++)
    for (size_t i = 0; i < in; i++)
      dst[(r0 + o) * in + i] = static_cast<_Float16>(w[(row0 + o) * in + i] * (scale ? scale[i] : 1.0f));
}

template <typename T>
int upload(const std::vector<T>& host, T** dev) {
  *dev = nullptr;
  if (host.empty()) return 0;
  hipError_t e = hipMalloc(reinterpret_cast<void**>(dev), host.size() * sizeof(T));
  if (e == hipSuccess)
    e = hipMemcpy(*dev, host.data(), host.size() * sizeof(T), hipMemcpyHostToDevice);
  return ancha::hip_status(e, "ancha_hip_block_create: weight upload");
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// One block GEMM through the fp16-weight kernel.
int gemm(const void* x, bool x_half, size_t n, size_t k, const _Float16* wt, size_t m,
         const float* bias, bool gelu, const float* rope, size_t tokens, size_t token_div,
         size_t width, const float* residual, void* out, bool out_half, bool norm,
         hipStream_t stream, float q_scale = 0.0f) {
  ancha::Gemm16Params p{};
  p.x = x;
  p.wt = wt;
  p.bias = bias;
  p.rope = rope;
  p.residual = residual;
  p.out = out;
  p.ldx = static_cast<long>(k);
  p.n = static_cast<int>(n);
  p.k = static_cast<int>(k);
  p.m = static_cast<int>(m);
  p.tokens = rope ? static_cast<int>(tokens) : 1;
  p.token_div = rope ? static_cast<int>(token_div) : 1;
  p.width = rope ? static_cast<int>(width) : 0;
  p.gelu = gelu;
  p.norm = norm;
  p.x_half = x_half;
  p.out_half = out_half;
  p.q_scale = q_scale;
  return ancha::hip_status(ancha::launch_gemm16(p, stream), "block GEMM");
}

size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

constexpr float kLog2eHost = 1.4426950408889634f;

}  // namespace

// Workspace regions: the packed projection (fp16 [rows, columns]; later the fp16 FF hidden
// activation [rows, hidden]), the fp16 attention output [rows, inner], x + attention (fp32),
// the fp16 normalised GEMM operand [rows, dim].
static size_t region_packed(const ancha_hip_block* b, size_t rows) {
  const size_t p = rows * b->columns * 2, h = rows * b->hidden * 2;
  return round_up(p > h ? p : h, 256);
}

// Forward of one block over `groups` sequences of `tokens` rows. split 0: sequence g is rows
// g*tokens .. g*tokens + tokens - 1. split > 0: the rows are a [batch, tokens, split] grid (the
// time layout [batch, bands, frames] with tokens = bands, split = frames) and sequence
// g = b*split + f is rows (b*tokens + t)*split + f: the band pass runs on the time layout, with
// no transposed copy. Every stage but attention and the rotary epilogue is row-wise, so only
// those two see the layout. out may be x (x is last read before out is first written).
// xh_in: the workspace already holds fp16(unit_norm(x)) (the previous block's xh_out).
// xh_out: also write fp16(unit_norm(out)) there for the next block (dim <= 512 and a next block
// of the same shape; see block_chainable).
static int block_forward(const ancha_hip_block* b, const float* x, size_t groups, size_t tokens,
                         size_t split, const float* rope, void* workspace,
                         size_t workspace_bytes, float* out, hipStream_t stream,
                         bool xh_in = false, bool xh_out = false) {
  static const std::string kWhere = "ancha_hip_block_forward: ";
  auto invalid = [](const char* why) { return ancha::fail(ANCHA_HIP_INVALID, kWhere + why); };
  if (!b) return invalid("null block");
  const size_t rows = groups * tokens;
  if (rows == 0) return ANCHA_HIP_OK;
  if (!x || !out || !rope || !workspace) return invalid("null buffer");
  if (workspace_bytes < ancha_hip_block_workspace(b, rows)) return invalid("workspace too small");
  if (!aligned16(x) || !aligned16(out) || !aligned16(rope) || !aligned16(workspace))
    return invalid("buffer not 16-byte aligned");
  if (split && groups % split) return invalid("groups not a multiple of the frame count");
  // Attention addresses one sequence with 32-bit offsets from its first row.
  if (rows > 0x7fffffff || rows * b->columns * 4 >= (size_t(1) << 40) ||
      tokens * (split ? split : 1) * b->columns * 2 >= (size_t(1) << 31) ||
      !ancha::attention_grid_fits(groups, tokens, b->heads))
    return ancha::fail(ANCHA_HIP_UNSUPPORTED, kWhere + "rows exceed the kernels' ranges");
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev != b->device)
    return invalid("called on another device than the block's");
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  _Float16* packed = reinterpret_cast<_Float16*>(ws);                // [rows, columns] fp16
  _Float16* hidden = reinterpret_cast<_Float16*>(ws);                // [rows, hidden] fp16
  _Float16* attended = reinterpret_cast<_Float16*>(ws + region_packed(b, rows));
  float* x1 = reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(attended) +
                                       round_up(rows * b->inner * 2, 256));
  _Float16* xh = reinterpret_cast<_Float16*>(reinterpret_cast<unsigned char*>(x1) +
                                             round_up(rows * b->dim * 4, 256));
  const size_t dim = b->dim, inner = b->inner;
  // xh = fp16(unit_norm(x)); packed = xh . [Wq|Wk|Wv|Wg|0] + [0|0|0|bg|0], RoPE on the q / k
  // columns, q times log2(e) for the exp2-based softmax.
  hipError_t e = hipSuccess;
  if (!xh_in)
    e = ancha::launch_norm_half(x, static_cast<int>(rows), static_cast<int>(dim), nullptr,
                                nullptr, xh, stream);
  if (e != hipSuccess) return ancha::hip_fail(e, "ancha_hip_block_forward");
  int rc = 0;
  if (b->packed_frag) {
    ancha::QkvParams qp{};
    qp.xh = xh;
    qp.w = b->packed_frag;
    qp.bias = b->packed_b;
    qp.rope = rope;
    qp.out = packed;
    qp.rows = static_cast<int>(rows);
    qp.dim = static_cast<int>(dim);
    qp.cols = static_cast<int>(b->columns);
    qp.tokens = static_cast<int>(tokens);
    qp.token_div = static_cast<int>(split ? split : 1);
    qp.width = static_cast<int>(inner);
    qp.q_scale = kLog2eHost;
    rc = ancha::hip_status(ancha::launch_qkv(qp, stream), "ancha_hip_block_forward");
  } else {
    rc = gemm(xh, true, rows, dim, b->packed_w, b->columns, b->packed_b, false, rope, tokens,
              split ? split : 1, inner, nullptr, packed, true, false, stream, kLog2eHost);
  }
  if (rc) return rc;
  // attended = softmax(q k^T) v * sigmoid(gate), stored fp16.
  ancha::AttnParams ap{};
  ap.q = reinterpret_cast<const float*>(packed);
  ap.k = reinterpret_cast<const float*>(packed + inner);
  ap.v = reinterpret_cast<const float*>(packed + 2 * inner);
  ap.gate = reinterpret_cast<const float*>(packed + 3 * inner);
  ap.in_half = 1;
  ap.out = reinterpret_cast<float*>(attended);
  ap.ldq = ap.ldk = ap.ldv = ap.ldg = static_cast<long>(b->columns);
  ap.groups = static_cast<int>(groups);
  ap.tokens = static_cast<int>(tokens);
  ap.heads = static_cast<int>(b->heads);
  ap.out_half = 1;
  if (split) {
    ap.gsplit = static_cast<int>(split);
    ap.gouter = static_cast<long>(tokens * split);
    ap.gstep = 1;
    ap.tstep = static_cast<long>(split);
  } else {
    ap.gsplit = 1;
    ap.gouter = static_cast<long>(tokens);
    ap.gstep = 0;
    ap.tstep = 1;
  }
  e = ancha::launch_attention(ap, true, stream);
  if (e != hipSuccess) return ancha::hip_fail(e, "ancha_hip_block_forward");
  if (b->w1_frag) {
    // Out projection, residual, norm, feed-forward (hidden activation on chip), residual and
    // the optional output norm in one kernel.
    ancha::TailParams tp{};
    tp.attended = attended;
    tp.x = x;
    tp.wo = b->wo_frag;
    tp.w1 = b->w1_frag;
    tp.b1 = b->ff_in_b;
    tp.w2 = b->w2_frag;
    tp.b2 = b->ff_out_b;
    tp.out_scale = b->out_scale;
    tp.out = out;
    tp.xh = xh_out ? xh : nullptr;
    tp.rows = static_cast<int>(rows);
    tp.dim = static_cast<int>(dim);
    tp.inner = static_cast<int>(inner);
    tp.hidden = static_cast<int>(b->hidden);
    return ancha::hip_status(ancha::launch_block_tail(tp, stream), "ancha_hip_block_forward");
  }
  // x1 = x + attended . W_out
  rc = gemm(attended, true, rows, inner, b->out_w, dim, nullptr, false, nullptr, 0, 1, 0, x, x1,
            false, false, stream);
  if (rc) return rc;
  // hidden = GELU(fp16(unit_norm(x1)) . W1' + b1), stored fp16.
  e = ancha::launch_norm_half(x1, static_cast<int>(rows), static_cast<int>(dim), nullptr, nullptr,
                              xh, stream);
  if (e != hipSuccess) return ancha::hip_fail(e, "ancha_hip_block_forward");
  rc = gemm(xh, true, rows, dim, b->ff_in_w, b->hidden, b->ff_in_b, true, nullptr, 0, 1, 0,
            nullptr, hidden, true, false, stream);
  if (rc) return rc;
  // out = x1 + hidden . W2 + b2
  rc = gemm(hidden, true, rows, b->hidden, b->ff_out_w, dim, b->ff_out_b, false, nullptr, 0, 1, 0,
            x1, out, false, false, stream);
  if (rc) return rc;
  if (xh_out) {
    // [out = unit_norm(out) * scale in place, and] the next block's fp16 operand in one pass.
    e = ancha::launch_norm_half(out, static_cast<int>(rows), static_cast<int>(dim), b->out_scale,
                                b->out_scale ? out : nullptr, xh, stream);
    if (e != hipSuccess) return ancha::hip_fail(e, "ancha_hip_block_forward");
  } else if (b->out_scale) {
    rc = ancha_hip_unit_norm(out, rows, dim, dim, b->out_scale, out, stream);
  }
  return rc;
}

namespace ancha {

bool block_chainable(const ancha_hip_block* a, const ancha_hip_block* b) {
  return a && b && a->dim <= 512 && a->dim == b->dim && a->inner == b->inner &&
         a->columns == b->columns && a->hidden == b->hidden;
}

int axis_pair_forward_chained(const ancha_hip_block* time, const ancha_hip_block* band,
                              const float* x, size_t batch, size_t bands, size_t frames,
                              const float* time_rope, const float* band_rope, void* workspace,
                              size_t workspace_bytes, float* out, hipStream_t stream, bool xh_in,
                              bool xh_out) {
  static const std::string kWhere = "ancha_hip_axis_pair_forward: ";
  if (!time || !band || time->dim != band->dim)
    return ancha::fail(ANCHA_HIP_INVALID, kWhere + "null blocks or blocks of different dim");
  const size_t rows = batch * bands * frames;
  if (rows == 0) return ANCHA_HIP_OK;
  if (!x || !out || !time_rope || !band_rope || !workspace)
    return ancha::fail(ANCHA_HIP_INVALID, kWhere + "null buffer");
  if (workspace_bytes < ancha_hip_axis_pair_workspace(time, band, rows))
    return ancha::fail(ANCHA_HIP_INVALID, kWhere + "workspace too small");
  const bool inner = block_chainable(time, band);
  // Time pass: groups = batch * bands, sequence = frames, x -> out.
  int rc = block_forward(time, x, batch * bands, frames, 0, time_rope, workspace, workspace_bytes,
                         out, stream, xh_in, inner);
  // Band pass in place on the same [batch, bands, frames, dim] rows: groups = batch * frames,
  // sequence = bands (network.rs:336-338 transposes instead).
  if (!rc) rc = block_forward(band, out, batch * frames, bands, frames, band_rope, workspace,
                              workspace_bytes, out, stream, inner, xh_out);
  return rc;
}

}  // namespace ancha

extern "C" {

int ancha_hip_block_create(size_t dim, size_t heads, size_t hidden, const float* attn_gamma,
                           const float* to_qkv, const float* to_gates,
                           const float* to_gates_bias, const float* to_out,
                           const float* ff_gamma, const float* ff_in, const float* ff_in_bias,
                           const float* ff_out, const float* ff_out_bias,
                           const float* output_gamma, ancha_hip_block** block) {
  static const std::string kWhere = "ancha_hip_block_create: ";
  if (const int s = ancha::sticky()) return s;
  if (!block) return ancha::fail(ANCHA_HIP_INVALID, kWhere + "null block out-pointer");
  *block = nullptr;
  if (!attn_gamma || !to_qkv || !to_gates || !to_gates_bias || !to_out || !ff_gamma || !ff_in ||
      !ff_in_bias || !ff_out || !ff_out_bias || dim == 0 || heads == 0 || hidden == 0)
    return ancha::fail(ANCHA_HIP_INVALID, kWhere + "null weight or zero size");
  const size_t inner = heads * kHeadDim;
  const size_t columns = round_up(3 * inner + heads, 128);
  // forward_kernels' shape gate (roformer.rs:471-475).
  if (!ancha_hip_linear_supported(dim, columns) || !ancha_hip_linear_supported(inner, dim) ||
      !ancha_hip_linear_supported(dim, hidden) || !ancha_hip_linear_supported(hidden, dim))
    return ancha::fail(ANCHA_HIP_UNSUPPORTED, kWhere + "a projection fails linear_supported");

  if (!ancha_hip_available())
    return ancha::fail(ANCHA_HIP_UNSUPPORTED, kWhere + "not a gfx950 device");
  if (dim * 4 * 128 >= (size_t(1) << 31) || hidden * 4 * 128 >= (size_t(1) << 31) ||
      columns * 4 * 128 >= (size_t(1) << 31))
    return ancha::fail(ANCHA_HIP_UNSUPPORTED, kWhere + "widths exceed the kernels' ranges");

  const std::vector<float> norm = source_scale(attn_gamma, dim);
  const std::vector<float> ffs = source_scale(ff_gamma, dim);
  std::vector<_Float16> pw(columns * dim, static_cast<_Float16>(0.0f));
  std::vector<float> pb(columns, 0.0f);
  fold_rows(to_qkv, dim, 0, 3 * inner, norm.data(), pw.data(), 0);
  fold_rows(to_gates, dim, 0, heads, norm.data(), pw.data(), 3 * inner);
  for (size_t h = 0; h < heads; h++) pb[3 * inner + h] = to_gates_bias[h];
  std::vector<_Float16> ow(dim * inner), w1(hidden * dim), w2(dim * hidden);
  fold_rows(to_out, inner, 0, dim, nullptr, ow.data(), 0);
  fold_rows(ff_in, dim, 0, hidden, ffs.data(), w1.data(), 0);
  fold_rows(ff_out, hidden, 0, dim, nullptr, w2.data(), 0);
  const std::vector<float> b1(ff_in_bias, ff_in_bias + hidden), b2(ff_out_bias, ff_out_bias + dim);
  std::vector<float> os;
  if (output_gamma) os = source_scale(output_gamma, dim);

  auto* b = new (std::nothrow) ancha_hip_block{};
  if (!b) return ancha::fail(ANCHA_HIP_INVALID, kWhere + "out of host memory");
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
  if (!rc && ancha::block_tail_supported(static_cast<int>(dim), static_cast<int>(inner),
                                         static_cast<int>(hidden))) {
    rc = upload(ancha::fragment_major(ow, dim, inner, false), &b->wo_frag);
    if (!rc) rc = upload(ancha::fragment_major(w1, hidden, dim, true), &b->w1_frag);
    if (!rc) rc = upload(ancha::fragment_major(w2, dim, hidden, true), &b->w2_frag);
  }
  if (!rc && ancha::qkv_supported(static_cast<int>(dim), static_cast<int>(columns)))
    rc = upload(ancha::fragment_major(pw, columns, dim, false), &b->packed_frag);
  if (rc) {
    ancha_hip_block_destroy(b);
    return rc;
  }
  *block = b;
  return ANCHA_HIP_OK;
}

size_t ancha_hip_block_workspace(const ancha_hip_block* b, size_t rows) {
  if (!b) return 0;
  return region_packed(b, rows) + round_up(rows * b->inner * 2, 256) +
         round_up(rows * b->dim * 4, 256) + rows * b->dim * 2;
}

int ancha_hip_block_forward(const ancha_hip_block* b, const float* x, size_t groups,
                            size_t tokens, const float* rope, void* workspace,
                            size_t workspace_bytes, float* out, hipStream_t stream) {
  if (const int s = ancha::sticky()) return s;
  return block_forward(b, x, groups, tokens, 0, rope, workspace, workspace_bytes, out, stream);
}

size_t ancha_hip_axis_pair_workspace(const ancha_hip_block* time, const ancha_hip_block* band,
                                     size_t rows) {
  if (!time || !band || time->dim != band->dim) return 0;
  const size_t a = ancha_hip_block_workspace(time, rows), c = ancha_hip_block_workspace(band, rows);
  return a > c ? a : c;
}

int ancha_hip_axis_pair_forward(const ancha_hip_block* time, const ancha_hip_block* band,
                                const float* x, size_t batch, size_t bands, size_t frames,
                                const float* time_rope, const float* band_rope, void* workspace,
                                size_t workspace_bytes, float* out, hipStream_t stream) {
  if (const int s = ancha::sticky()) return s;
  return ancha::axis_pair_forward_chained(time, band, x, batch, bands, frames, time_rope,
                                          band_rope, workspace, workspace_bytes, out, stream,
                                          false, false);
}

void ancha_hip_block_destroy(ancha_hip_block* b) {
  if (!b) return;
  for (void* p : {static_cast<void*>(b->packed_w), static_cast<void*>(b->packed_b),
                  static_cast<void*>(b->out_w), static_cast<void*>(b->ff_in_w),
                  static_cast<void*>(b->ff_in_b), static_cast<void*>(b->ff_out_w),
                  static_cast<void*>(b->ff_out_b), static_cast<void*>(b->out_scale),
                  static_cast<void*>(b->wo_frag), static_cast<void*>(b->w1_frag),
                  static_cast<void*>(b->w2_frag), static_cast<void*>(b->packed_frag)})
    if (p) (void)hipFree(p);
  delete b;
}

}  // extern "C"
