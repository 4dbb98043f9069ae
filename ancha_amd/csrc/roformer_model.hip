// The Mel/BS-RoFormer network and the chunked separation runtime on the gfx950 kernels (C ABI
// of include/ancha_hip.h), host code only.
//
// Mirrors crates/ancha-models/src/network.rs (Roformer::build :89-278, forward :303-400) and
// the chunk loop of src/runtime.rs:103-238:
//   spectrum -> band split (mel.hip) -> depth x [time block, frequency block] (block.hip, the
//   frequency block reading the time layout in place) -> [BS: final norm] -> per stem: tanh
//   hidden layers and the value|gate output projection as batched fp16 GEMMs (gemm16.hip),
//   GLU + overlap gather (mel.hip) -> masks [stems][2*bins][re, im][frames].
//   separate: per chunk gather -> STFT -> forward -> per stem masked iSTFT + overlap-add into
//   the clip accumulators (dsp.hip); finally the accumulator division and border crop.
// Weights come from a callback that serves the reference checkpoint's tensors by name.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "../../include/ancha_hip.h"
#include "kernels.hpp"
#include "status.hpp"

namespace {

constexpr size_t kFft = 2048;
constexpr size_t kHeadDim = ANCHA_ATTENTION_HEAD_DIM;

size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

template <typename T>
int upload(const std::vector<T>& host, T** dev) {
  *dev = nullptr;
  if (host.empty()) return 0;
  hipError_t e = hipMalloc(reinterpret_cast<void**>(dev), host.size() * sizeof(T));
  if (e == hipSuccess)
    e = hipMemcpy(*dev, host.data(), host.size() * sizeof(T), hipMemcpyHostToDevice);
  return ancha::hip_status(e, "ancha_hip_roformer_create: weight upload");
}

template <typename T>
int alloc(size_t count, T** dev) {
  *dev = nullptr;
  return ancha::hip_status(hipMalloc(reinterpret_cast<void**>(dev), count * sizeof(T)),
                           "ancha_hip_roformer_create: table allocation");
}

constexpr size_t kRopeFloats = 4 * kHeadDim;  // per token of one packed rotary table

}  // namespace

struct ancha_hip_roformer {
  bool mel, zero_dc;
  size_t dim, depth, heads, ff_hidden, mask_hidden, mask_layers, hop, chunk, overlap, stems;
  size_t bands, fft_bins, max_width;
  std::vector<size_t> offsets, bins, widths, wofs;
  int device;
  int *d_offsets = nullptr, *d_bins = nullptr, *d_wofs = nullptr;
  float *split_w = nullptr, *split_b = nullptr;
  std::vector<ancha_hip_block*> blocks;  // time, frequency per depth
  std::vector<std::vector<float>> freqs;
  float* final_scale = nullptr;
  struct Head {
    std::vector<_Float16*> hw;
    std::vector<float*> hb;
    bool frag0 = false;  // hw[0] fragment-major per band (launch_mask_hidden)
    _Float16* ow = nullptr;
    float* ob = nullptr;
  };
  std::vector<Head> mask_heads;
  std::vector<size_t> mpad, colprefix;  // per band padded output width, prefix (columns)
  long* d_band_base = nullptr;
  int *d_band_stride = nullptr, *d_band_width = nullptr;
  int *d_cover_start = nullptr, *d_cover_band = nullptr, *d_cover_local = nullptr;
  // Rotary frequencies [2 * depth][32] (the time sets, then the frequency sets) and the packed
  // rotary tables built from them at load time: time [depth][4][frames][64] for the chunk's
  // frame count, frequency [depth][4][bands][64]. A forward over another frame count builds its
  // time tables in its workspace instead.
  size_t frames = 0;
  float* d_freqs = nullptr;
  float *time_rope = nullptr, *band_rope = nullptr;
  // The value|gate projections of all bands as one grouped product: per band output width and
  // first column (bands + 1 entries); for the chunk's frame count, the band of each tile and
  // each band's first tile.
  int* d_group_cols = nullptr;
  long* d_group_col0 = nullptr;
  int *d_group_of_tile = nullptr, *d_group_first = nullptr;
};

namespace {

void free_all(ancha_hip_roformer* m) {
  if (!m) return;
  for (void* p : {static_cast<void*>(m->d_offsets), static_cast<void*>(m->d_bins),
                  static_cast<void*>(m->d_wofs), static_cast<void*>(m->split_w),
                  static_cast<void*>(m->split_b), static_cast<void*>(m->final_scale),
                  static_cast<void*>(m->d_band_base), static_cast<void*>(m->d_band_stride),
                  static_cast<void*>(m->d_band_width), static_cast<void*>(m->d_cover_start),
                  static_cast<void*>(m->d_cover_band), static_cast<void*>(m->d_cover_local),
                  static_cast<void*>(m->d_group_cols), static_cast<void*>(m->d_group_col0),
                  static_cast<void*>(m->d_group_of_tile), static_cast<void*>(m->d_group_first),
                  static_cast<void*>(m->d_freqs), static_cast<void*>(m->time_rope),
                  static_cast<void*>(m->band_rope)})
    if (p) (void)hipFree(p);
  for (auto* b : m->blocks) ancha_hip_block_destroy(b);
  for (auto& h : m->mask_heads) {
    for (auto* p : h.hw) (void)hipFree(p);
    for (auto* p : h.hb) (void)hipFree(p);
    if (h.ow) (void)hipFree(h.ow);
    if (h.ob) (void)hipFree(h.ob);
  }
  delete m;
}

// One (batched) product through the block GEMM: out = act(x . W^T + bias).
int gemm(const void* x, bool x_half, size_t n, size_t k, const _Float16* wt, size_t m,
         const float* bias, bool tanh_act, void* out, bool out_half, size_t batch,
         long x_bstride, long w_bstride, long bias_bstride, long out_bstride,
         hipStream_t stream) {
  ancha::Gemm16Params p{};
  p.x = x;
  p.wt = wt;
  p.bias = bias;
  p.out = out;
  p.ldx = static_cast<long>(k);
  p.n = static_cast<int>(n);
  p.k = static_cast<int>(k);
  p.m = static_cast<int>(m);
  p.tokens = 1;
  p.token_div = 1;
  p.x_half = x_half;
  p.out_half = out_half;
  p.tanh_act = tanh_act;
  p.batch = static_cast<int>(batch);
  p.x_bstride = x_bstride;
  p.w_bstride = w_bstride;
  p.bias_bstride = bias_bstride;
  p.out_bstride = out_bstride;
  return ancha::hip_status(ancha::launch_gemm16(p, stream), "mask head GEMM");
}

// Tiles of the grouped value|gate product over `frames` frames: band b has row tiles x
// (mpad[b] / 128) of them.
size_t group_tiles(const ancha_hip_roformer* m, size_t frames) {
  return (frames + 127) / 128 * (m->colprefix.back() / 128);
}

// Workspace regions of a forward over `frames` frames.
struct Layout {
  size_t tables, x, inner, h1, h2, glu, xh, total;
};
// nch chunks share the axis loop (x [nch][bands][frames][dim]); the mask heads run one chunk
// at a time in the same head buffers. A frame count other than the chunk's first gets its
// rotary and tile tables (region `tables`, rebuilt on the device by every forward).
Layout forward_layout(const ancha_hip_roformer* m, size_t frames, size_t nch = 1) {
  Layout l{};
  const size_t rows = m->bands * frames;
  size_t tables = 0;
  if (frames != m->frames)
    tables = round_up(m->depth * frames * kRopeFloats * 4, 256) +
             round_up((group_tiles(m, frames) + m->bands + 1) * 4, 256);
  l.tables = 0;
  l.x = tables;
  const size_t block_ws =
      ancha_hip_axis_pair_workspace(m->blocks[0], m->blocks[1], nch * rows);
  l.inner = l.x + round_up(nch * rows * m->dim * 4, 256);
  l.h1 = l.inner;
  l.h2 = l.h1 + round_up(rows * m->mask_hidden * 2, 256);
  l.glu = l.h2 + round_up(rows * m->mask_hidden * 2, 256);
  // fp16 copy of x for the first mask layer, past the head buffers.
  l.xh = l.glu + round_up(frames * m->colprefix.back() * 4, 256);
  const size_t heads_end = l.xh + round_up(nch * rows * m->dim * 2, 256);
  const size_t blocks_end = l.inner + round_up(block_ws, 256);
  l.total = heads_end > blocks_end ? heads_end : blocks_end;
  return l;
}

bool cancel_requested(const volatile int* cancelled) { return cancelled && *cancelled != 0; }

int cancelled_rc() { return ancha::fail(ANCHA_HIP_CANCELLED, "task cancelled"); }

// Forward of nch chunks' spectra (1 or 2) into their masks. `flags` (or null) collects the
// non-finite mask check of the separation runtime. Returns ANCHA_HIP_CANCELLED when
// *cancelled is set at a layer pair or a mask head (network.rs:334,367); what was enqueued
// before still runs.
int forward_impl(ancha_hip_roformer* m, const float* const* spectra, size_t nch, size_t frames,
                 void* workspace, float* const* masks_of, const volatile int* cancelled,
                 unsigned* flags, hipStream_t stream) {
  static const char* kWhere = "ancha_hip_roformer_forward";
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  const Layout l = forward_layout(m, frames, nch);
  float* x = reinterpret_cast<float*>(ws + l.x);
  const size_t rows = m->bands * frames;
  const size_t table_floats = frames * kRopeFloats;
  // Rotary and tile tables: the model's own for the chunk's frame count, else built here.
  const float* time_rope = m->time_rope;
  const int* of_tile = m->d_group_of_tile;
  const int* first_tile = m->d_group_first;
  if (frames != m->frames) {
    float* rope = reinterpret_cast<float*>(ws + l.tables);
    int* tiles = reinterpret_cast<int*>(ws + l.tables +
                                        round_up(m->depth * table_floats * 4, 256));
    const size_t ntiles = group_tiles(m, frames);
    if (frames * kRopeFloats * m->depth > 0x7fffffff || ntiles > 0x7fffffff)
      return ancha::fail(ANCHA_HIP_UNSUPPORTED, "ancha_hip_roformer_forward: too many frames");
    hipError_t e = ancha::launch_axis_rope(m->d_freqs, static_cast<int>(m->depth),
                                           static_cast<int>(frames), rope, stream);
    if (e == hipSuccess)
      e = ancha::launch_group_tiles(m->d_group_col0, static_cast<int>(m->bands),
                                    static_cast<int>((frames + 127) / 128),
                                    static_cast<long>(ntiles), tiles, tiles + ntiles, stream);
    if (e != hipSuccess) return ancha::hip_fail(e, kWhere);
    time_rope = rope;
    of_tile = tiles;
    first_tile = tiles + ntiles;
  }
  ancha::BandSplitParams bp{};
  bp.offsets = m->d_offsets;
  bp.bins = m->d_bins;
  bp.wofs = m->d_wofs;
  bp.weight = m->split_w;
  bp.bias = m->split_b;
  bp.x = x;
  bp.bands = static_cast<int>(m->bands);
  bp.frames = static_cast<int>(frames);
  bp.cols = static_cast<int>(4 * m->fft_bins);
  bp.dim = static_cast<int>(m->dim);
  bp.max_width = static_cast<int>(m->max_width);
  for (size_t c = 0; c < nch; c++) {
    bp.spectrum = spectra[c];
    bp.x = x + c * rows * m->dim;
    if (const int rc = ancha::hip_status(ancha::launch_band_split(bp, stream), kWhere)) return rc;
  }
  // Axis loop (network.rs:333-339): x [nch][bands][frames][dim] is the time layout with batch
  // nch.
  const size_t block_bytes = l.total - l.inner;
  // Each block also writes the next block's fp16 operand where the blocks allow.
  bool xh_in = false;
  for (size_t i = 0; i < m->depth; i++) {
    if (cancel_requested(cancelled)) return cancelled_rc();
    const bool xh_out =
        i + 1 < m->depth && ancha::block_chainable(m->blocks[2 * i + 1], m->blocks[2 * i + 2]);
    const int rc = ancha::axis_pair_forward_chained(
        m->blocks[2 * i], m->blocks[2 * i + 1], x, nch, m->bands, frames,
        time_rope + i * table_floats, m->band_rope + i * m->bands * kRopeFloats, ws + l.inner,
        block_bytes, x, stream, xh_in, xh_out);
    if (rc) return rc;
    xh_in = xh_out;
  }
  if (m->final_scale) {
    const int rc = ancha_hip_unit_norm(x, nch * rows, m->dim, m->dim, m->final_scale, x, stream);
    if (rc) return rc;
  }
  _Float16* h[2] = {reinterpret_cast<_Float16*>(ws + l.h1), reinterpret_cast<_Float16*>(ws + l.h2)};
  // The first mask layer reads x as fp16, the operand the fp32-input GEMM would round to.
  _Float16* xh = reinterpret_cast<_Float16*>(ws + l.xh);
  const bool cast = m->dim % 8 == 0;
  if (cast) {
    const int rc = ancha::hip_status(
        ancha::launch_cast_half(x, static_cast<long>(nch * rows * m->dim), xh, stream), kWhere);
    if (rc) return rc;
  }
  float* glu = reinterpret_cast<float*>(ws + l.glu);
  const size_t mh = m->mask_hidden;
  for (size_t c = 0; c < nch; c++)
  for (size_t s = 0; s < m->stems; s++) {
    if (cancel_requested(cancelled)) return cancelled_rc();
    const ancha_hip_roformer::Head& head = m->mask_heads[s];
    // Hidden layers (network.rs:377-379): h = tanh(W h + b) per band, fp16 between layers.
    const void* in = cast ? static_cast<const void*>(xh + c * rows * m->dim)
                          : static_cast<const void*>(x + c * rows * m->dim);
    bool in_half = cast;
    size_t in_dim = m->dim;
    for (size_t layer = 0; layer < m->mask_layers; layer++) {
      _Float16* out = h[layer & 1];
      int rc = 0;
      if (layer == 0 && head.frag0 && in_half) {
        ancha::QkvParams qp{};
        qp.xh = static_cast<const _Float16*>(in);
        qp.w = head.hw[0];
        qp.bias = head.hb[0];
        qp.out = out;
        qp.rows = static_cast<int>(frames);
        qp.dim = static_cast<int>(in_dim);
        qp.cols = static_cast<int>(mh);
        qp.batch = static_cast<int>(m->bands);
        qp.x_bstride = static_cast<long>(frames * in_dim);
        qp.w_bstride = static_cast<long>(mh * in_dim);
        qp.b_bstride = static_cast<long>(mh);
        qp.out_bstride = static_cast<long>(frames * mh);
        rc = ancha::hip_status(ancha::launch_mask_hidden(qp, stream), kWhere);
      } else {
        rc = gemm(in, in_half, frames, in_dim, head.hw[layer], mh, head.hb[layer], true, out,
                  true, m->bands, static_cast<long>(frames * in_dim),
                  static_cast<long>(mh * in_dim), static_cast<long>(mh),
                  static_cast<long>(frames * mh), stream);
      }
      if (rc) return rc;
      in = out;
      in_half = true;
      in_dim = mh;
    }
    // Output projection, value and gate halves side by side: one grouped product over the
    // bands (band b: [frames, mh] x [mh, mpad[b]] into glu + colprefix[b] * frames).
    ancha::Gemm16Params gp16{};
    gp16.x = in;
    gp16.wt = head.ow;
    gp16.bias = head.ob;
    gp16.out = glu;
    gp16.ldx = static_cast<long>(mh);
    gp16.n = static_cast<int>(frames);
    gp16.k = static_cast<int>(mh);
    gp16.m = 128;
    gp16.tokens = 1;
    gp16.token_div = 1;
    gp16.x_half = 1;
    gp16.batch = static_cast<int>(m->bands);
    gp16.x_bstride = static_cast<long>(frames * mh);
    gp16.group_of_tile = of_tile;
    gp16.group_first_tile = first_tile;
    gp16.group_cols = m->d_group_cols;
    gp16.group_col0 = m->d_group_col0;
    gp16.group_tiles = static_cast<int>(group_tiles(m, frames));
    if (const int rc = ancha::hip_status(ancha::launch_gemm16(gp16, stream), kWhere)) return rc;
    ancha::GluParams gp{};
    gp.glu = glu;
    gp.band_base = m->d_band_base;
    gp.band_stride = m->d_band_stride;
    gp.band_width = m->d_band_width;
    gp.cover_start = m->d_cover_start;
    gp.cover_band = m->d_cover_band;
    gp.cover_local = m->d_cover_local;
    gp.masks = masks_of[c] + s * 4 * m->fft_bins * frames;
    gp.flags = flags;
    gp.outputs = static_cast<int>(4 * m->fft_bins);
    gp.frames = static_cast<int>(frames);
    if (const int rc = ancha::hip_status(ancha::launch_glu_gather(gp, stream), kWhere)) return rc;
  }
  return 0;
}

// Chunk plan of src/runtime.rs:103-116 and ChunkPlan (chunk.rs:1-25): chunks start every
// chunk / overlap samples over the clip plus a reflected border of chunk - step samples on
// each side (no border when the clip is not longer than two borders).
struct Plan {
  size_t step, border, length, frames;
  std::vector<size_t> starts;
};
Plan plan_of(size_t chunk, size_t overlap, size_t samples) {
  Plan p{};
  p.step = chunk / overlap;
  p.border = chunk - p.step;
  if (!(samples > 2 * p.border)) p.border = 0;
  p.length = samples + 2 * p.border;
  for (size_t s = 0; s < p.length; s += p.step) p.starts.push_back(s);
  return p;
}
Plan plan_for(const ancha_hip_roformer* m, size_t samples) {
  Plan p = plan_of(m->chunk, m->overlap, samples);
  p.frames = m->chunk / m->hop + 1;
  return p;
}

struct SepLayout {
  size_t flags, chunk, spectrum, masks, frames_buf, sums, weights, model, total;
};
SepLayout separate_layout(const ancha_hip_roformer* m, size_t samples) {
  const Plan p = plan_for(m, samples);
  SepLayout l{};
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += round_up(bytes, 256);
    return at;
  };
  l.flags = take(4);
  // Two chunks at a time go through the model together.
  l.chunk = take(2 * 2 * m->chunk * 4);
  l.spectrum = take(2 * p.frames * 4 * m->fft_bins * 4);
  l.masks = take(2 * m->stems * 4 * m->fft_bins * p.frames * 4);
  l.frames_buf = take(p.frames * 2 * kFft * 4);
  l.sums = take(m->stems * 2 * p.length * 4);
  l.weights = take(p.length * 4);
  l.model = take(forward_layout(m, p.frames, p.starts.size() > 1 ? 2 : 1).total);
  l.total = o;
  return l;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" {

int ancha_hip_roformer_create(const ancha_hip_roformer_config* c, ancha_hip_tensor_fn get,
                              void* ctx, ancha_hip_roformer** model) {
  static const char* kWhere = "ancha_hip_roformer_create: ";
  auto invalid = [&](const char* why) {
    return ancha::fail(ANCHA_HIP_INVALID, std::string(kWhere) + why);
  };
  if (const int s = ancha::sticky()) return s;
  if (!model) return invalid("null model out-pointer");
  *model = nullptr;
  if (!c || !get || !c->band_offsets || !c->band_bins) return invalid("null config or callback");
  if (!ancha_hip_available())
    return ancha::fail(ANCHA_HIP_UNSUPPORTED, std::string(kWhere) + "not a gfx950 device");
  // Schema checks (config.rs:36-121) plus what the kernels cover.
  if (c->n_fft != kFft || c->head_dim != kHeadDim || c->hop == 0 || c->hop > kFft / 2 ||
      c->dim == 0 || c->depth == 0 || c->heads == 0 || c->ff_mult == 0 || c->mask_depth == 0 ||
      c->mask_expansion == 0 || c->stems == 0 || c->stems > 2 || c->bands < 2 ||
      c->chunk_samples <= kFft / 2 || c->overlap == 0 || c->overlap > c->chunk_samples ||
      (!c->mel && c->mask_depth < 2))
    return invalid("config outside the model schema");
  const size_t fft_bins = kFft / 2 + 1;
  std::vector<int> coverage(fft_bins, 0);
  for (size_t b = 0; b < c->bands; b++) {
    if (c->band_offsets[b + 1] <= c->band_offsets[b]) return invalid("empty band");
    for (size_t q = c->band_offsets[b]; q < c->band_offsets[b + 1]; q++) {
      if (c->band_bins[q] >= fft_bins) return invalid("band bin past the FFT bins");
      if (q > c->band_offsets[b] && c->band_bins[q] <= c->band_bins[q - 1])
        return invalid("band bins not strictly increasing");
      coverage[c->band_bins[q]]++;
    }
  }
  for (int n : coverage)
    if (n == 0) return invalid("bands leave uncovered FFT bins");
  const size_t dim = c->dim, mh = c->dim * c->mask_expansion;
  // (the band-split kernel covers dim <= 512)
  if (!ancha_hip_linear_supported(dim, mh) || !ancha_hip_linear_supported(mh, mh) || dim > 512)
    return ancha::fail(ANCHA_HIP_UNSUPPORTED,
                       std::string(kWhere) + "dim or mask width outside the kernels");

  auto* m = new (std::nothrow) ancha_hip_roformer{};
  if (!m) return invalid("out of host memory");
  m->mel = c->mel != 0;
  m->zero_dc = c->zero_dc != 0;
  m->dim = dim;
  m->depth = c->depth;
  m->heads = c->heads;
  m->ff_hidden = dim * c->ff_mult;
  m->mask_hidden = mh;
  // BS depth counts all Linears, Mel depth counts hidden layers (network.rs:138-144).
  m->mask_layers = m->mel ? c->mask_depth : c->mask_depth - 1;
  m->hop = c->hop;
  m->chunk = c->chunk_samples;
  m->overlap = c->overlap;
  m->stems = c->stems;
  m->bands = c->bands;
  m->fft_bins = fft_bins;
  if (hipGetDevice(&m->device) != hipSuccess) m->device = 0;
  m->offsets.assign(c->band_offsets, c->band_offsets + c->bands + 1);
  m->bins.assign(c->band_bins, c->band_bins + m->offsets.back());
  m->wofs.assign(c->bands + 1, 0);
  m->max_width = 0;
  for (size_t b = 0; b < c->bands; b++) {
    const size_t w = 4 * (m->offsets[b + 1] - m->offsets[b]);
    m->widths.push_back(w);
    m->wofs[b + 1] = m->wofs[b] + w;
    if (w > m->max_width) m->max_width = w;
  }
  int rc = 0;
  auto abandon = [&](int code) {
    free_all(m);
    return code;
  };
  auto missing = [&](const std::string& name) {
    return abandon(ancha::fail(ANCHA_HIP_INVALID,
                               "ancha_hip_roformer_create: missing or mis-shaped tensor " + name));
  };
  auto tensor = [&](const std::string& name, size_t numel) -> const float* {
    return get(ctx, name.c_str(), numel);
  };
  // Band split (network.rs:96-121): W'[c][d] = W[d][c] * sqrt(width) * gamma[c], [width][dim].
  {
    std::vector<float> w(m->wofs.back() * dim), bias(c->bands * dim);
    for (size_t b = 0; b < c->bands; b++) {
      const size_t width = m->widths[b];
      const std::string p = "band_split.to_features." + std::to_string(b);
      const float* g = tensor(p + ".0.gamma", width);
      const float* wt = tensor(p + ".1.weight", dim * width);
      const float* bs = tensor(p + ".1.bias", dim);
      if (!g || !wt || !bs) return missing(p + ".*");
      const float root = std::sqrt(static_cast<float>(width));
      for (size_t d = 0; d < dim; d++)
        for (size_t col = 0; col < width; col++)
          w[(m->wofs[b] + col) * dim + d] = wt[d * width + col] * (g[col] * root);
      for (size_t d = 0; d < dim; d++) bias[b * dim + d] = bs[d];
    }
    std::vector<int> off(m->offsets.begin(), m->offsets.end()), bins(m->bins.begin(), m->bins.end());
    std::vector<int> wofs(m->wofs.begin(), m->wofs.end());
    if (!rc) rc = upload(w, &m->split_w);
    if (!rc) rc = upload(bias, &m->split_b);
    if (!rc) rc = upload(off, &m->d_offsets);
    if (!rc) rc = upload(bins, &m->d_bins);
    if (!rc) rc = upload(wofs, &m->d_wofs);
    if (rc) return abandon(rc);
  }
  // Transformer blocks (network.rs:122-137; Transformer::load, roformer.rs:381-409).
  for (size_t i = 0; i < c->depth; i++)
    for (int axis = 0; axis < 2; axis++) {
      const std::string p = "layers." + std::to_string(i) + "." + std::to_string(axis);
      const size_t inner = c->heads * kHeadDim, hidden = m->ff_hidden;
      const std::string a = p + ".layers.0.0", f = p + ".layers.0.1.net";
      const float* t[11] = {
          tensor(a + ".norm.gamma", dim),         tensor(a + ".to_qkv.weight", 3 * inner * dim),
          tensor(a + ".to_gates.weight", c->heads * dim), tensor(a + ".to_gates.bias", c->heads),
          tensor(a + ".to_out.0.weight", dim * inner),    tensor(f + ".0.gamma", dim),
          tensor(f + ".1.weight", hidden * dim),          tensor(f + ".1.bias", hidden),
          tensor(f + ".4.weight", dim * hidden),          tensor(f + ".4.bias", dim),
          m->mel ? tensor(p + ".norm.gamma", dim) : nullptr};
      const float* fr = tensor(a + ".rotary_embed.freqs", kHeadDim / 2);
      for (int j = 0; j < 10; j++)
        if (!t[j]) return missing(p + ".*");
      if (!fr || (m->mel && !t[10])) return missing(p + ".*");
      ancha_hip_block* blk = nullptr;
      rc = ancha_hip_block_create(dim, c->heads, hidden, t[0], t[1], t[2], t[3], t[4], t[5], t[6],
                                  t[7], t[8], t[9], t[10], &blk);
      if (rc) return abandon(rc);
      m->blocks.push_back(blk);
      m->freqs.emplace_back(fr, fr + kHeadDim / 2);
    }
  if (!m->mel) {  // final_norm (network.rs:138-142, :340-342)
    const float* g = tensor("final_norm.gamma", dim);
    if (!g) return missing("final_norm.gamma");
    std::vector<float> s(dim);
    const float root = std::sqrt(static_cast<float>(dim));
    for (size_t d = 0; d < dim; d++) s[d] = g[d] * root;
    rc = upload(s, &m->final_scale);
    if (rc) return abandon(rc);
  }
  // Value|gate output width of each band, padded to a multiple of 128, and its first column.
  m->mpad.resize(c->bands);
  m->colprefix.assign(c->bands + 1, 0);
  for (size_t b = 0; b < c->bands; b++) {
    m->mpad[b] = round_up(2 * m->widths[b], 128);
    m->colprefix[b + 1] = m->colprefix[b] + m->mpad[b];
  }
  {
    std::vector<int> cols(c->bands);
    std::vector<long> col0(c->bands + 1);
    for (size_t b = 0; b < c->bands; b++) cols[b] = static_cast<int>(m->mpad[b]);
    for (size_t b = 0; b <= c->bands; b++) col0[b] = static_cast<long>(m->colprefix[b]);
    rc = upload(cols, &m->d_group_cols);
    if (!rc) rc = upload(col0, &m->d_group_col0);
    if (rc) return abandon(rc);
  }
  // Mask heads (network.rs:143-177): hidden layers [bands][out][in] fp16, output [m_pad][mh].
  for (size_t s = 0; s < c->stems; s++) {
    ancha_hip_roformer::Head head;
    m->mask_heads.push_back(head);
    ancha_hip_roformer::Head& h = m->mask_heads.back();
    auto key = [&](size_t b, size_t layer) {
      return "mask_estimators." + std::to_string(s) + ".to_freqs." + std::to_string(b) + ".0." +
             std::to_string(2 * layer);
    };
    size_t in = dim;
    for (size_t layer = 0; layer < m->mask_layers; layer++) {
      std::vector<_Float16> w(c->bands * mh * in);
      std::vector<float> bias(c->bands * mh);
      for (size_t b = 0; b < c->bands; b++) {
        const float* wt = tensor(key(b, layer) + ".weight", mh * in);
        const float* bs = tensor(key(b, layer) + ".bias", mh);
        if (!wt || !bs) return missing(key(b, layer) + ".*");
        for (size_t e = 0; e < mh * in; e++) w[b * mh * in + e] = static_cast<_Float16>(wt[e]);
        for (size_t o = 0; o < mh; o++) bias[b * mh + o] = bs[o];
      }
      _Float16* dw = nullptr;
      float* db = nullptr;
      // The first hidden layer (fp16 input, dim 384 / 512) runs on the projection kernel, which
      // takes W^T fragment-major per band.
      if (layer == 0 && ancha::mask_hidden_supported(static_cast<int>(in), static_cast<int>(mh))) {
        std::vector<_Float16> f(w.size());
        for (size_t b = 0; b < c->bands; b++) {
          const std::vector<_Float16> one(w.begin() + b * mh * in, w.begin() + (b + 1) * mh * in);
          const std::vector<_Float16> fm = ancha::fragment_major(one, mh, in, false);
          std::copy(fm.begin(), fm.end(), f.begin() + b * mh * in);
        }
        w.swap(f);
        h.frag0 = true;
      }
      rc = upload(w, &dw);
      h.hw.push_back(dw);
      if (!rc) rc = upload(bias, &db);
      h.hb.push_back(db);
      if (rc) return abandon(rc);
      in = mh;
    }
    std::vector<_Float16> ow(m->colprefix.back() * mh, static_cast<_Float16>(0.0f));
    std::vector<float> ob(m->colprefix.back(), 0.0f);
    for (size_t b = 0; b < c->bands; b++) {
      const size_t w2 = 2 * m->widths[b];
      const float* wt = tensor(key(b, m->mask_layers) + ".weight", w2 * mh);
      const float* bs = tensor(key(b, m->mask_layers) + ".bias", w2);
      if (!wt || !bs) return missing(key(b, m->mask_layers) + ".*");
      for (size_t r = 0; r < w2; r++) {
        for (size_t e = 0; e < mh; e++)
          ow[(m->colprefix[b] + r) * mh + e] = static_cast<_Float16>(wt[r * mh + e]);
        ob[m->colprefix[b] + r] = bs[r];
      }
    }
    rc = upload(ow, &h.ow);
    if (!rc) rc = upload(ob, &h.ob);
    if (rc) return abandon(rc);
  }
  // GLU gather tables (network.rs:248-263): covering (band, local bin) entries per FFT bin.
  {
    std::vector<std::vector<std::pair<int, int>>> cover(fft_bins);
    for (size_t b = 0; b < c->bands; b++)
      for (size_t q = m->offsets[b]; q < m->offsets[b + 1]; q++)
        cover[m->bins[q]].push_back({static_cast<int>(b), static_cast<int>(q - m->offsets[b])});
    std::vector<int> start(fft_bins + 1, 0), band, local;
    for (size_t f = 0; f < fft_bins; f++) {
      for (auto& e : cover[f]) {
        band.push_back(e.first);
        local.push_back(e.second);
      }
      start[f + 1] = static_cast<int>(band.size());
    }
    std::vector<long> base(c->bands);
    std::vector<int> stride(c->bands), width(c->bands);
    for (size_t b = 0; b < c->bands; b++) {
      base[b] = static_cast<long>(m->colprefix[b]);
      stride[b] = static_cast<int>(m->mpad[b]);
      width[b] = static_cast<int>(m->widths[b]);
    }
    rc = upload(start, &m->d_cover_start);
    if (!rc) rc = upload(band, &m->d_cover_band);
    if (!rc) rc = upload(local, &m->d_cover_local);
    if (!rc) rc = upload(base, &m->d_band_base);
    if (!rc) rc = upload(stride, &m->d_band_stride);
    if (!rc) rc = upload(width, &m->d_band_width);
    if (rc) return abandon(rc);
  }
  // Rotary and tile tables for the chunk's frame count (network.rs:280-299,331-332), built on
  // the device from the checkpoint's frequencies.
  {
    m->frames = c->chunk_samples / c->hop + 1;
    std::vector<float> freqs;
    for (int axis = 0; axis < 2; axis++)
      for (size_t i = 0; i < m->depth; i++) {
        const std::vector<float>& f = m->freqs[2 * i + axis];
        freqs.insert(freqs.end(), f.begin(), f.end());
      }
    const size_t ntiles = group_tiles(m, m->frames);
    if (m->frames * kRopeFloats * m->depth > 0x7fffffff || ntiles > 0x7fffffff)
      return abandon(ancha::fail(ANCHA_HIP_UNSUPPORTED, "ancha_hip_roformer_create: chunk too long"));
    rc = upload(freqs, &m->d_freqs);
    if (!rc) rc = alloc(m->depth * m->frames * kRopeFloats, &m->time_rope);
    if (!rc) rc = alloc(m->depth * m->bands * kRopeFloats, &m->band_rope);
    if (!rc) rc = alloc(ntiles, &m->d_group_of_tile);
    if (!rc) rc = alloc(m->bands + 1, &m->d_group_first);
    if (rc) return abandon(rc);
    hipError_t e = ancha::launch_axis_rope(m->d_freqs, static_cast<int>(m->depth),
                                           static_cast<int>(m->frames), m->time_rope, nullptr);
    if (e == hipSuccess)
      e = ancha::launch_axis_rope(m->d_freqs + m->depth * kHeadDim / 2,
                                  static_cast<int>(m->depth), static_cast<int>(m->bands),
                                  m->band_rope, nullptr);
    if (e == hipSuccess)
      e = ancha::launch_group_tiles(m->d_group_col0, static_cast<int>(m->bands),
                                    static_cast<int>((m->frames + 127) / 128),
                                    static_cast<long>(ntiles), m->d_group_of_tile,
                                    m->d_group_first, nullptr);
    if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
    if (e != hipSuccess) return abandon(ancha::hip_fail(e, "ancha_hip_roformer_create"));
  }
  *model = m;
  return ANCHA_HIP_OK;
}

size_t ancha_hip_roformer_workspace(const ancha_hip_roformer* m, size_t frames) {
  if (!m || frames == 0) return 0;
  return forward_layout(m, frames).total;
}

int ancha_hip_roformer_forward(ancha_hip_roformer* m, const float* spectrum, size_t frames,
                               void* workspace, size_t workspace_bytes, float* masks,
                               const volatile int* cancelled, hipStream_t stream) {
  static const std::string kWhere = "ancha_hip_roformer_forward: ";
  if (const int s = ancha::sticky()) return s;
  if (!m) return ancha::fail(ANCHA_HIP_INVALID, kWhere + "null model");
  if (frames == 0) return ANCHA_HIP_OK;
  if (!spectrum || !workspace || !masks || !aligned16(spectrum) || !aligned16(workspace) ||
      !aligned16(masks))
    return ancha::fail(ANCHA_HIP_INVALID, kWhere + "null or unaligned buffer");
  if (frames > 0x7fffffff)
    return ancha::fail(ANCHA_HIP_UNSUPPORTED, kWhere + "too many frames");
  if (workspace_bytes < ancha_hip_roformer_workspace(m, frames))
    return ancha::fail(ANCHA_HIP_INVALID, kWhere + "workspace too small");
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev != m->device)
    return ancha::fail(ANCHA_HIP_INVALID, kWhere + "called on another device than the model's");
  return forward_impl(m, &spectrum, 1, frames, workspace, &masks, cancelled, nullptr, stream);
}

int ancha_hip_chunk_plan(size_t chunk_samples, size_t overlap, size_t samples, size_t* chunks,
                         size_t* border) {
  if (chunk_samples == 0 || overlap == 0 || overlap > chunk_samples)
    return ancha::fail(ANCHA_HIP_INVALID, "ancha_hip_chunk_plan: invalid chunk or overlap divisor");
  if (samples > (size_t(1) << 40))
    return ancha::fail(ANCHA_HIP_UNSUPPORTED, "ancha_hip_chunk_plan: clip too long");
  const size_t step = chunk_samples / overlap;
  const size_t b = 2 * (chunk_samples - step) < samples ? chunk_samples - step : 0;
  // starts = 0, step, ... below samples + 2 * border: the count plan_of's loop produces.
  if (chunks) *chunks = (samples + 2 * b + step - 1) / step;
  if (border) *border = b;
  return ANCHA_HIP_OK;
}

size_t ancha_hip_separate_workspace(const ancha_hip_roformer* m, size_t samples) {
  if (!m || samples == 0) return 0;
  return separate_layout(m, samples).total;
}

namespace {

// The first check flag in the order the reference runtime meets them within one chunk, as its
// message: Stft::forward's input check, the model output check of runtime.rs:172-176, then
// Stft::inverse's coverage and output checks (dsp.rs:126-133; they fire before
// Accumulator::add's "non-finite chunk output", which can then never be reached), and
// Accumulator::finish. The flags are ORed over the whole clip, so when two chunks fail in
// different ways the message is that of the earlier kind here, not of the earlier chunk.
const char* flag_message(unsigned flags) {
  if (flags & ancha::kFlagInput) return "non-finite STFT input";
  if (flags & ancha::kFlagMasks) return "non-finite model output";
  if (flags & ancha::kFlagIstftUncovered) return "iSTFT has an uncovered sample";
  if (flags & ancha::kFlagChunk) return "non-finite iSTFT output";
  return "uncovered overlap-add sample";
}

}  // namespace

int ancha_hip_separate(ancha_hip_roformer* m, const float* audio, size_t samples, void* workspace,
                       size_t workspace_bytes, float* stems, float* residual,
                       const volatile int* cancelled, hipStream_t stream) {
  static const std::string kWhere = "ancha_hip_separate: ";
  if (const int s = ancha::sticky()) return s;
  if (!m) return ancha::fail(ANCHA_HIP_INVALID, kWhere + "null model");
  if (samples == 0) return ANCHA_HIP_OK;
  if (!audio || !workspace || !stems || !aligned16(workspace))
    return ancha::fail(ANCHA_HIP_INVALID, kWhere + "null or unaligned buffer");
  if (residual && m->stems != 1)
    return ancha::fail(ANCHA_HIP_INVALID, kWhere + "a residual needs a one-stem model");
  if (samples > (size_t(1) << 40))
    return ancha::fail(ANCHA_HIP_UNSUPPORTED, kWhere + "clip too long");
  if (workspace_bytes < ancha_hip_separate_workspace(m, samples))
    return ancha::fail(ANCHA_HIP_INVALID, kWhere + "workspace too small");
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev != m->device)
    return ancha::fail(ANCHA_HIP_INVALID, kWhere + "called on another device than the model's");
  const Plan p = plan_for(m, samples);
  const SepLayout l = separate_layout(m, samples);
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  unsigned* flags = reinterpret_cast<unsigned*>(ws + l.flags);
  float* chunk = reinterpret_cast<float*>(ws + l.chunk);
  float* spectrum = reinterpret_cast<float*>(ws + l.spectrum);
  float* masks = reinterpret_cast<float*>(ws + l.masks);
  float* frames_buf = reinterpret_cast<float*>(ws + l.frames_buf);
  float* sums = reinterpret_cast<float*>(ws + l.sums);
  float* weights = reinterpret_cast<float*>(ws + l.weights);
  const long length = static_cast<long>(p.length), cs = static_cast<long>(m->chunk);
  // On cancellation the work already enqueued still reads and writes the caller's buffers:
  // wait for it, so the caller may release them on return.
  auto cancel = [&]() {
    (void)hipStreamSynchronize(stream);
    return ancha::fail(ANCHA_HIP_CANCELLED, "task cancelled");
  };
  auto device_error = [&](hipError_t e) { return ancha::hip_fail(e, "ancha_hip_separate"); };
  hipError_t e = ancha::launch_zero(reinterpret_cast<float*>(flags), 1, stream);
  if (e == hipSuccess) e = ancha::launch_zero(sums, static_cast<long>(m->stems) * 2 * length, stream);
  if (e == hipSuccess) e = ancha::launch_zero(weights, length, stream);
  if (e != hipSuccess) return device_error(e);
  const size_t mask_stride = 4 * m->fft_bins * p.frames;
  const size_t chunk_floats = 2 * m->chunk, spectrum_floats = p.frames * 4 * m->fft_bins;
  for (size_t i = 0; i < p.starts.size(); i += 2) {
    if (cancel_requested(cancelled)) return cancel();  // runtime.rs:118
    const size_t nch = std::min<size_t>(2, p.starts.size() - i);
    const float* spectra[2];
    float* masks_of[2];
    for (size_t c = 0; c < nch; c++) {
      const size_t start = p.starts[i + c];
      const long remaining = std::min<long>(length - static_cast<long>(start), cs);
      float* chunk_c = chunk + c * chunk_floats;
      float* spectrum_c = spectrum + c * spectrum_floats;
      e = ancha::launch_chunk_gather(audio, static_cast<long>(samples), static_cast<long>(start),
                                     static_cast<long>(p.border), remaining, cs, chunk_c, flags,
                                     stream);
      if (e == hipSuccess)
        e = ancha::launch_stft(chunk_c, cs, static_cast<int>(m->hop), spectrum_c, stream);
      if (e != hipSuccess) return device_error(e);
      spectra[c] = spectrum_c;
      masks_of[c] = masks + c * m->stems * mask_stride;
    }
    const int rc = forward_impl(m, spectra, nch, p.frames, ws + l.model, masks_of, cancelled,
                                flags, stream);
    if (rc == ANCHA_HIP_CANCELLED) return cancel();
    if (rc) return rc;
    // Overlap-add in chunk order, as one chunk at a time would.
    for (size_t c = 0; c < nch; c++) {
      const size_t start = p.starts[i + c];
      const bool first = start == 0, last = static_cast<long>(start) + cs >= length;
      for (size_t s = 0; s < m->stems; s++) {
        e = ancha::launch_istft_frames(spectra[c], masks_of[c] + s * mask_stride,
                                       static_cast<int>(p.frames), m->zero_dc ? 1 : 0,
                                       frames_buf, stream);
        if (e == hipSuccess)
          e = ancha::launch_ola_accumulate(frames_buf, static_cast<int>(p.frames),
                                           static_cast<int>(m->hop), cs,
                                           static_cast<long>(start), length, first, last, s == 0,
                                           sums + s * 2 * length, weights, flags, stream);
        if (e != hipSuccess) return device_error(e);
      }
    }
  }
  for (size_t s = 0; s < m->stems; s++) {
    e = ancha::launch_finish(sums + s * 2 * length, weights, length, static_cast<long>(p.border),
                             static_cast<long>(samples), audio, stems + s * 2 * samples,
                             s == 0 ? residual : nullptr, flags, stream);
    if (e != hipSuccess) return device_error(e);
  }
  // The reference checks every chunk's model output and audio as it goes (runtime.rs:172-176,
  // chunk.rs:57-60,76-79); here the kernels set flags and the clip's one read-back reports them.
  unsigned host_flags = 0;
  e = hipMemcpyAsync(&host_flags, flags, sizeof(host_flags), hipMemcpyDeviceToHost, stream);
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  if (e != hipSuccess) return device_error(e);
  if (host_flags) return ancha::fail(ANCHA_HIP_INVALID, flag_message(host_flags));
  if (cancel_requested(cancelled)) return ancha::fail(ANCHA_HIP_CANCELLED, "task cancelled");
  return ANCHA_HIP_OK;
}

void ancha_hip_roformer_destroy(ancha_hip_roformer* m) { free_all(m); }

int ancha_hip_stft(const float* signal, size_t samples, size_t hop, float* spectrum,
                   hipStream_t stream) {
  static const std::string kWhere = "ancha_hip_stft: ";
  if (const int s = ancha::sticky()) return s;
  if (samples == 0) return ANCHA_HIP_OK;
  if (!signal || !spectrum || !aligned16(spectrum))
    return ancha::fail(ANCHA_HIP_INVALID, kWhere + "null or unaligned buffer");
  if (hop == 0 || hop > kFft / 2 || samples <= kFft / 2)
    return ancha::fail(ANCHA_HIP_INVALID,
                       kWhere + "hop outside (0, 1024] or input not longer than FFT/2");
  if (samples / hop + 1 > 0x7fffffff || samples > (size_t(1) << 40))
    return ancha::fail(ANCHA_HIP_UNSUPPORTED, kWhere + "too many frames");
  return ancha::hip_status(ancha::launch_stft(signal, static_cast<long>(samples),
                                              static_cast<int>(hop), spectrum, stream),
                           "ancha_hip_stft");
}

size_t ancha_hip_istft_workspace(size_t frames) { return frames * 2 * kFft * sizeof(float); }

int ancha_hip_istft(const float* spectrum, const float* masks, size_t frames, size_t hop,
                    size_t length, int zero_dc, void* workspace, size_t workspace_bytes,
                    float* out, hipStream_t stream) {
  static const std::string kWhere = "ancha_hip_istft: ";
  if (const int s = ancha::sticky()) return s;
  if (frames == 0 || length == 0) return ANCHA_HIP_OK;
  if (!spectrum || !masks || !workspace || !out)
    return ancha::fail(ANCHA_HIP_INVALID, kWhere + "null buffer");
  if (hop == 0 || hop > kFft / 2) return ancha::fail(ANCHA_HIP_INVALID, kWhere + "hop outside (0, 1024]");
  if (frames > 0x7fffffff || length > (size_t(1) << 40))
    return ancha::fail(ANCHA_HIP_UNSUPPORTED, kWhere + "too many frames");
  if (length + kFft / 2 > (frames - 1) * hop + kFft)
    return ancha::fail(ANCHA_HIP_INVALID, kWhere + "requested length exceeds frame support");
  if (workspace_bytes < ancha_hip_istft_workspace(frames) || !aligned16(workspace))
    return ancha::fail(ANCHA_HIP_INVALID, kWhere + "workspace too small or unaligned");
  float* frames_buf = static_cast<float*>(workspace);
  const long n = static_cast<long>(length);
  hipError_t e = ancha::launch_zero(out, 2 * n, stream);
  if (e == hipSuccess)
    e = ancha::launch_istft_frames(spectrum, masks, static_cast<int>(frames), zero_dc ? 1 : 0,
                                   frames_buf, stream);
  // One chunk covering the whole output: unit fade weights (first and last).
  if (e == hipSuccess)
    e = ancha::launch_ola_accumulate(frames_buf, static_cast<int>(frames), static_cast<int>(hop),
                                     n, 0, n, true, true, false, out, nullptr, nullptr, stream);
  return ancha::hip_status(e, "ancha_hip_istft");
}

// ------------------------------------------------------------------------------------------
// Allocation-free iSTFT: ancha_hip_istft with its frame workspace in a static device array.
// ------------------------------------------------------------------------------------------

}  // extern "C"

namespace {

// The windowed inverse frames [frames][2][2048] of one ancha_hip_istft_noalloc call. Every GPU
// the library runs on holds its own copy (24 MiB) until the process ends. Host code uses only
// the per-device address from hipGetSymbolAddress, never this name.
constexpr size_t kIstftScratchFrames = 1536;
__device__ __align__(256) float scratch[kIstftScratchFrames * 2 * kFft];

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mutex;
float* g_scratch[kScratchDevices] = {};

// The current device's address of `scratch`, looked up on the first call on that device.
int scratch_address(float** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return ancha::hip_fail(e, "ancha_hip_istft_noalloc: hipGetDevice");
  if (dev < 0 || dev >= kScratchDevices)
    return ancha::fail(ANCHA_HIP_UNSUPPORTED, "ancha_hip_istft_noalloc: device index >= 64");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return ancha::hip_fail(e, "ancha_hip_istft_noalloc: hipGetSymbolAddress");
    g_scratch[dev] = static_cast<float*>(ptr);
  }
  *out = g_scratch[dev];
  return 0;
}

}  // namespace

extern "C" {

int ancha_hip_istft_noalloc(const float* spectrum, const float* masks, size_t frames, size_t hop,
                            size_t length, int zero_dc, float* out, hipStream_t stream) {
  static const std::string kWhere = "ancha_hip_istft_noalloc: ";
  if (const int s = ancha::sticky()) return s;
  if (frames == 0 || length == 0) return ANCHA_HIP_OK;
  if (frames > kIstftScratchFrames)
    return ancha::fail(ANCHA_HIP_UNSUPPORTED,
                       kWhere + "more than 1536 frames (the static scratch holds 1536)");
  float* ws = nullptr;
  if (const int rc = scratch_address(&ws)) return rc;
  return ancha_hip_istft(spectrum, masks, frames, hop, length, zero_dc, ws,
                         ancha_hip_istft_workspace(frames), out, stream);
}

}  // extern "C"
