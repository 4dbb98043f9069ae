// Kernel parameter blocks and host launchers of the HIP kernels (internal to the library; the
// public surface is the C ABI in include/ancha_hip.h).
#pragma once
#include <hip/hip_runtime.h>

#include <vector>

#include "../../include/ancha_hip.h"

namespace ancha {

// softmax(q.k^T).v per (group, head). q/k/v/gate point at the column of head 0 inside
// row-major buffers (head h at +64h). Token t of group g sits in row
//   (g / gsplit) * gouter + (g % gsplit) * gstep + t * tstep
// of q/k/v/gate (row stride ld*) and of out (row stride heads*64): gsplit 1, gouter tokens,
// gstep 0, tstep 1 for groups of contiguous tokens ([groups, tokens, ...]); gsplit frames,
// gouter bands*frames, gstep 1, tstep frames for the band axis of a [batch, bands, frames, ...]
// buffer (group = batch*frames + frame, token = band). gsplit 0 means contiguous groups.
struct AttnParams {
  const float* q;
  const float* k;
  const float* v;
  const float* gate;  // per-head gate logits (head h at +h), or null
  const float* rope;  // packed [4, tokens, 64] table, or null (q/k already rotated, q scaled)
  float* out;         // [groups, tokens, heads, 64] contiguous (fp16 values if out_half)
  long ldq, ldk, ldv, ldg;
  int groups, tokens, heads;
  int out_half;       // store the output as fp16 (the block's internal activation); set with in_half
  // q / k / v / gate are fp16 (ld* in fp16 elements) and q already carries log2(e) with the
  // softmax scale: the block's packed projection. Gated, rope-free, 16-byte aligned calls only.
  int in_half;
  int gsplit;
  long gouter, gstep, tstep;
};

// Compute units of the current device (looked up once per device; 256 if the query fails).
int device_cus();

// `aligned`: every float4 access is 16-byte aligned (base pointers and row strides).
hipError_t launch_attention(const AttnParams& p, bool aligned, hipStream_t stream);

// Whether the launch launch_attention picks for this shape fits HIP's grid limits (workgroup
// count below 2^31 and total thread count below 2^32).
bool attention_grid_fits(size_t groups, size_t tokens, size_t heads);

// out = epilogue(x . w): x [n, k] (row stride ldx), w [k, m] row-major (the reference's
// [in, out] Linear layout), out [n, m] contiguous. Epilogue, in order: optional input row norm
// (the product of row r scaled by 1 / max(||x_r||, 1e-12)), bias [m], erf-GELU, interleaved
// rotary on columns [0, 2*width) (queries then keys of token r % tokens, packed [4, tokens, 64]
// table), residual [n, m] contiguous.
struct LinearParams {
  const float* x;
  const float* w;
  const float* bias;      // or null
  const float* rope;      // or null
  const float* residual;  // or null (may alias out)
  float* out;
  long ldx;
  int n, k, m;
  int tokens, width;
  int gelu;
  int norm;
};

// `aligned`: x, w, out (and bias / residual / rope when present) are 16-byte aligned, ldx and m
// are multiples of 4.
hipError_t launch_linear(const LinearParams& p, bool aligned, hipStream_t stream);

// out[r] = x[r] / max(||x[r]||, 1e-12) * scale (scale [dim] or null): x [rows, dim] with row
// stride ldx, out [rows, dim] contiguous; out may alias x when ldx == dim.
struct NormParams {
  const float* x;
  const float* scale;
  float* out;
  long ldx;
  int rows, dim;
};

hipError_t launch_unit_norm(const NormParams& p, bool aligned, hipStream_t stream);

// Normalised fp16 operand of the block GEMMs (norm.hip), x [rows, dim] contiguous fp32,
// 16-byte aligned, dim % 4 == 0: y = scale ? unit_norm(x) * scale : x (written to y when y is
// not null; y may alias x only for dim <= 512), h = fp16(unit_norm(y)) [rows, dim].
// h = fp16(x) for n floats (n % 8 == 0, 16-byte aligned), round to nearest even.
hipError_t launch_cast_half(const float* x, long n, _Float16* h, hipStream_t stream);
hipError_t launch_norm_half(const float* x, int rows, int dim, const float* scale, float* y,
                            _Float16* h, hipStream_t stream);

// The block's projection GEMM on load-time fp16 weights: out = epilogue(x . W) with W^T fp16
// [m][k] (k contiguous, the PyTorch [out, in] layout), x fp32 or fp16 (x_half) [n][k] with row
// stride ldx, out fp32 or fp16 (out_half) [n][m] contiguous; bias, rope, residual (fp32) and
// the row norm as in LinearParams. Requires m % 128 == 0, k % 8 == 0, 16-byte aligned rows.
struct Gemm16Params {
  const void* x;
  const _Float16* wt;
  const float* bias;
  const float* rope;
  const float* residual;
  void* out;
  long ldx;
  int n, k, m;
  int tokens, width;
  int token_div;  // rotary position of row r: (r / token_div) % tokens
  int gelu, norm, x_half, out_half;
  int tanh_act;   // tanh after the bias (the mask estimator's hidden layers)
  float q_scale;  // factor on the rotated query columns [0, width) (0: none)
  // Batched products (batch > 1): product b reads x + b*x_bstride, wt + b*w_bstride,
  // bias + b*bias_bstride and writes out (and reads residual) at + b*out_bstride (elements).
  // Rotary epilogues are for unbatched calls.
  int batch;
  long x_bstride, w_bstride, bias_bstride, out_bstride;
  // Grouped products (group_of_tile not null; batch products, group_tiles tiles in all): tile t
  // belongs to product b = group_of_tile[t], whose tiles start at group_first_tile[b]; product b
  // reads x + b*x_bstride and W^T rows from group_col0[b] on, its output is [n][group_cols[b]]
  // at element group_col0[b]*n, its bias starts at element group_col0[b] (group_cols[b] a
  // multiple of 128; w_bstride, bias_bstride and out_bstride are not used).
  const int* group_of_tile;
  const int* group_first_tile;
  const int* group_cols;
  const long* group_col0;
  int group_tiles;
};

hipError_t launch_gemm16(const Gemm16Params& p, hipStream_t stream);

// Fused tail of the RoFormer block (tail.hip), 128 rows per workgroup step:
//   x1 = x + attended . W_out; h = fp16(GELU(fp16(unit_norm(x1)) . W1' + b1));
//   out = x1 + h . W2 + b2; with out_scale: out = unit_norm(out) * out_scale and, with xh,
//   xh = fp16(unit_norm(out)).
// attended fp16 [rows][inner]; x, out fp32 [rows][dim] (out may be x); xh fp16 [rows][dim].
// wo, w1, w2: fp16 fragment-major copies of W_out^T [dim][inner], W1'^T [hidden][dim] and
// W2^T [dim][hidden] (tail_fragments), the last two with their k axis in kPerm16 order.
struct TailParams {
  const _Float16* attended;
  const float* x;
  const _Float16* wo;
  const _Float16* w1;
  const float* b1;
  const _Float16* w2;
  const float* b2;
  const float* out_scale;  // [dim] or null
  float* out;
  _Float16* xh;            // or null (needs out_scale)
  int rows, dim, inner, hidden;
};
bool block_tail_supported(int dim, int inner, int hidden);
hipError_t launch_block_tail(const TailParams& p, hipStream_t stream);

// Packed q | k | v | gate projection of the block (qkv.hip): out fp16 [rows][cols] =
// bias + xh . W with the rotary epilogue on columns [0, 2 width) (token of row r:
// (r / token_div) % tokens; the packed [4, tokens, 64] table's key half is read, the query half
// being it times 1/8) and the query columns times q_scale. xh fp16 [rows][dim]; w: fp16
// fragment-major W^T [cols][dim] (natural k order, tail_fragments layout).
struct QkvParams {
  const _Float16* xh;
  const _Float16* w;
  const float* bias;   // [cols]
  const float* rope;   // or null
  _Float16* out;
  int rows, dim, cols;
  int tokens, token_div, width;
  float q_scale;
  // launch_mask_hidden only: `batch` products, product b reading xh + b * x_bstride, w +
  // b * w_bstride, bias + b * b_bstride and writing out + b * out_bstride (elements).
  int batch;
  long x_bstride, w_bstride, b_bstride, out_bstride;
};
bool qkv_supported(int dim, int cols);
hipError_t launch_qkv(const QkvParams& p, hipStream_t stream);
// The mask heads' first hidden layer on the same kernel: out = fp16(tanh(xh . W^T + bias)) for
// every column (cols % 64 == 0), per band product, W^T fragment-major as in the block.
bool mask_hidden_supported(int dim, int cols);
// Fragment-major copy of W^T [rows][k] (host side, at weight load): fragment (b, s) = 512
// halves at (b * (k / 16) + s) * 512, lane l's 8 at 8 l, holding W^T[32 b + l % 32][16 s +
// perm(8 (l / 32) + t)], perm = kPerm16 (permute) or the identity. rows % 32 == 0, k % 16 == 0.
std::vector<_Float16> fragment_major(const std::vector<_Float16>& wt, size_t rows, size_t k,
                                     bool permute);
hipError_t launch_mask_hidden(const QkvParams& p, hipStream_t stream);

// Order of k within each 16-block of a fragment-major weight whose B operand comes straight
// from another product's accumulators (tail.hip): B k-slot 8h + t holds feature kPerm16[8h + t].
constexpr int kPerm16[16] = {0, 1, 2, 3, 8, 9, 10, 11, 4, 5, 6, 7, 12, 13, 14, 15};

// Axis pair of two blocks (block.hip) where each block hands the next its fp16 operand:
// xh_in, the workspace holds fp16(unit_norm(x)) from the previous pair; xh_out, the band block
// leaves fp16(unit_norm(out)) there for the next pair (which must satisfy block_chainable with
// it). Between the two blocks of the pair the same hand-over happens when they allow it.
bool block_chainable(const ancha_hip_block* a, const ancha_hip_block* b);
int axis_pair_forward_chained(const ancha_hip_block* time, const ancha_hip_block* band,
                              const float* x, size_t batch, size_t bands, size_t frames,
                              const float* time_rope, const float* band_rope, void* workspace,
                              size_t workspace_bytes, float* out, hipStream_t stream, bool xh_in,
                              bool xh_out);

// Check flags of one separation: the kernels below OR these bits into a device word (`flags`,
// or null for no checks) where they meet what the reference runtime rejects.
enum : unsigned {
  kFlagInput = 1u,          // non-finite STFT input (dsp.rs:57-60)
  kFlagMasks = 2u,          // non-finite model output (runtime.rs:173-176)
  kFlagIstftUncovered = 4u, // iSTFT window sum <= 1e-11 at an output sample (dsp.rs:126)
  kFlagChunk = 8u,          // non-finite iSTFT / chunk output (dsp.rs:128-131, chunk.rs:57-60)
  kFlagOlaUncovered = 16u,  // overlap-add weight <= 0 at an output sample (chunk.rs:76-79)
};

// Separation runtime (dsp.hip), n_fft = 2048. chunk / audio [2][samples]; spectrum
// [frames][1025][channel][re, im]; masks [2050][re, im][frames] (one stem); frames_buf
// [frames][2][2048]; sums [2][total], weights [total].
hipError_t launch_stft(const float* chunk, long samples, int hop, float* spectrum,
                       hipStream_t stream);
hipError_t launch_istft_frames(const float* spectrum, const float* masks, int frames, int zero_dc,
                               float* frames_buf, hipStream_t stream);
hipError_t launch_ola_accumulate(const float* frames_buf, int frames, int hop, long length,
                                 long start, long total, bool first, bool last, bool count_weight,
                                 float* sums, float* weights, unsigned* flags, hipStream_t stream);
hipError_t launch_chunk_gather(const float* audio, long n, long start, long border,
                               long remaining, long samples, float* chunk, unsigned* flags,
                               hipStream_t stream);
hipError_t launch_finish(const float* sums, const float* weights, long total, long border, long n,
                         const float* audio, float* out, float* residual, unsigned* flags,
                         hipStream_t stream);
hipError_t launch_zero(float* p, long n, hipStream_t stream);

// Packed rotary tables of AxisRope::new (roformer.rs:282-302) for `sets` frequency sets, built
// on the device: freqs [sets][32] -> out [sets][4][tokens][64] (query cos and signed sin times
// 1/8, key cos and signed sin; angle = f32(t) * f).
hipError_t launch_axis_rope(const float* freqs, int sets, int tokens, float* out,
                            hipStream_t stream);
// Tile tables of the mask heads' grouped product (Gemm16Params::group_*) for `row_tiles` row
// tiles per band: band b owns tiles [first[b], first[b+1]) with first[b] = row_tiles *
// col0[b] / 128; of_tile[t] = the band of tile t (total = row_tiles * col0[bands] / 128 tiles;
// first has bands + 1 entries).
hipError_t launch_group_tiles(const long* col0, int bands, int row_tiles, long total,
                              int* of_tile, int* first, hipStream_t stream);

// Band split (mel.hip): spectrum [frames][cols]; band b = FFT bins bins[offsets[b] ..
// offsets[b+1]), feature columns 4*bin .. 4*bin+3; weight: per band [width][dim] fp32 (folded
// scale applied) starting at element wofs[b] * dim; bias [bands][dim]; x [bands][frames][dim].
struct BandSplitParams {
  const float* spectrum;
  const int* offsets;
  const int* bins;
  const int* wofs;
  const float* weight;
  const float* bias;
  float* x;
  int bands, frames, cols, dim, max_width;
  int tile;  // frames per workgroup (set by the launcher)
};
hipError_t launch_band_split(const BandSplitParams& p, hipStream_t stream);

// GLU masks (mel.hip): glu holds, per band b at band_base[b] * frames, [frames][band_stride[b]] fp32
// rows whose first band_width[b] columns are the values and next band_width[b] the gates.
// FFT bin f is covered by entries cover_start[f] .. cover_start[f+1] (band, local bin).
// masks [outputs = 4 * bins][frames] with output 4f + 2*channel + re/im.
struct GluParams {
  const float* glu;
  const long* band_base;
  const int* band_stride;
  const int* band_width;
  const int* cover_start;
  const int* cover_band;
  const int* cover_local;
  float* masks;
  unsigned* flags;  // kFlagMasks on a non-finite mask value (or null)
  int outputs, frames;
};
hipError_t launch_glu_gather(const GluParams& p, hipStream_t stream);

// out [batch, b, a, dim] = x [batch, a, b, dim] with axes 1 and 2 swapped (both contiguous).
struct SwapParams {
  const float* x;
  float* out;
  int batch, a, b, dim;
};

hipError_t launch_swap_axes(const SwapParams& p, bool aligned, hipStream_t stream);

}  // namespace ancha
