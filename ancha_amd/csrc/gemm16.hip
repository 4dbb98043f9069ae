// Projection GEMM of the RoFormer block on load-time fp16 weights (gfx950):
// out = epilogue(x . W) with W stored once, at block load, as fp16 W^T [m][k] (k contiguous),
// x fp32 or fp16 [n][k], out fp32 or fp16 [n][m]. The arithmetic is that of linear.hip (every
// operand rounded to fp16 once, fp32 accumulation, the same epilogue), so an fp16 activation
// written by one GEMM and read by the next is bit-for-bit the operand the next GEMM would
// round to; only the bytes moved change.
//
// Persistent workgroups (two per CU) walk 128 x 128 output tiles; each XCD takes one
// contiguous range of tiles, column tiles of a row block next to each other, so a row block of
// x is read from HBM once and re-read from that XCD's L2. Per tile: 4 waves of 64 x 64 (fp16 x)
// or 8 waves of 64 x 32 (fp32 x) in MFMA 16x16x32 tiles, K in 64-wide steps through a
// double-buffered LDS tile, global loads one step ahead in registers. After the last K step the
// accumulators go to LDS, and the loads of the next tile's first step are issued before the
// epilogue, so they travel while the epilogue reads the tile back row-wise (bias, GELU / tanh,
// rotary, residual: 512-byte coalesced rows) and stores it. (Stores straight from the
// accumulators, 16 rows x 32-64 bytes per instruction, measured slower.) The epilogue's kind is
// a template parameter for the combinations the block and the mask estimator use. Loads past
// the end of K or of the rows get an offset outside the buffer: they return 0 without touching
// memory.
#include "buffer.hpp"
#include "common.hpp"
#include "gemm.hpp"
#include "kernels.hpp"

namespace ancha {
namespace {

using namespace gemm;

// Offset added to a load that must read 0 (beyond every buffer range used here: < 2^31).
constexpr unsigned kNowhere = 0x80000000u;
constexpr int kStageFloats = kBM * kBN;  // epilogue staging: the fp32 output tile (64 KB)

// Registers of one 128 x 64 x tile and one 128 x 64 W^T tile, spread over NT threads: fp32 x
// as float4 (16 threads per row), fp16 x and W^T as 8 halves (8 threads per row).
template <bool XH, int NT>
struct XStage;
template <int NT>
struct XStage<false, NT> {
  float4 v[2048 / NT];
};
template <int NT>
struct XStage<true, NT> {
  u32x4 v[1024 / NT];
};
template <int NT>
struct WStage {
  u32x4 v[1024 / NT];
};

// Byte offset of float4 chunk c (columns 4c..4c+3) of row r in the [128][128] fp32 staging tile;
// chunks are XOR-swizzled by r & 7 so 16 rows written at one chunk hit distinct banks.
__device__ __forceinline__ int stage_offset(int r, int c) { return r * 512 + ((c ^ (r & 7)) << 4); }

// Epilogue kinds fixed at compile time (the block's and the mask estimator's products: straight
// code per row, no flag tests); kEpiRuntime reads the flags of Gemm16Params.
constexpr int kEpiGelu = 1, kEpiTanh = 2, kEpiRope = 4, kEpiResidual = 8, kEpiRuntime = -1;

// WAVES = 4 (64 x 64 per wave) or 8 (64 x 32 per wave: half the accumulators and staging
// registers per thread, which the fp32-input variants need to stay within 128 registers).
template <bool XH, bool OH, bool NORM, int WAVES, int EPI>
__global__ __launch_bounds__(WAVES * 64, 2) void gemm16_kernel(Gemm16Params p, int col_tiles,
                                                               int tiles) {
  constexpr int NT = WAVES * 64;
  constexpr int XP = XH ? 1024 / NT : 2048 / NT;  // x rows per thread per K step
  constexpr int WP = 1024 / NT;                   // W^T rows per thread per K step
  constexpr int CB = WAVES == 4 ? 4 : 2;          // 16-column MFMA blocks per wave
  constexpr int XROWS = XH ? NT / 8 : NT / 16;    // x rows covered per pass
  constexpr int WROWS = NT / 8;
  static_assert(4 * kTileBytes == kStageFloats * 4, "staging tile must fit the LDS pool");
  __shared__ __attribute__((aligned(16))) unsigned char lds[4 * kTileBytes];
  __shared__ float lds_inv[kBM];
  __shared__ int lds_tok[kBM];
  // K-step buffers: x tile b at lds + b*kTileBytes, W^T tile b at lds + (2+b)*kTileBytes.

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = p.n, k = p.k;
  constexpr int xbytes = XH ? 2 : 4;
  const unsigned ldx_b = (unsigned)p.ldx * xbytes, k2 = (unsigned)k * 2;
  const int ktiles = (k + kBK - 1) / kBK;
  const int batch_tiles = ((n + kBM - 1) / kBM) * col_tiles;  // tiles of one product
  // Tile t -> product, row / column origin, output width, and the product's offsets of W^T
  // (elements), bias and output.
  struct TileAt {
    int bt, r0, c0, m;
    long wofs, bofs, oofs;
  };
  auto decode = [&](int tile) {
    TileAt d;
    if (p.group_of_tile) {
      const int b = p.group_of_tile[tile];
      const int rt = tile - p.group_first_tile[b], ct = p.group_cols[b] / kBN;
      const long c0 = p.group_col0[b];
      d.bt = b;
      d.r0 = (rt / ct) * kBM;
      d.c0 = (rt % ct) * kBN;
      d.m = p.group_cols[b];
      d.wofs = c0 * k;
      d.bofs = c0;
      d.oofs = c0 * n;
    } else {
      const int rt = tile % batch_tiles;
      d.bt = tile / batch_tiles;
      d.r0 = (rt / col_tiles) * kBM;
      d.c0 = (rt % col_tiles) * kBN;
      d.m = p.m;
      d.wofs = d.bt * p.w_bstride;
      d.bofs = d.bt * p.bias_bstride;
      d.oofs = d.bt * p.out_bstride;
    }
    return d;
  };

  // Tiles of this workgroup: XCD x (= blockIdx % 8) owns tiles [x*per, (x+1)*per); its
  // workgroups take every (gridDim/8)-th tile of that range.
  const int xcd = blockIdx.x % kXcds, slot = blockIdx.x / kXcds, slots = gridDim.x / kXcds;
  const int per = (tiles + kXcds - 1) / kXcds;
  const int first = xcd * per + slot, last = min((xcd + 1) * per, tiles);

  // Staging roles: fp32 x: 16 lanes per row (float4), rows xr32 + XROWS*i; fp16 x and W^T:
  // 8 lanes per row (8 halves), rows r16 + XROWS*i (x) or r16 + WROWS*i (W^T).
  const int x4 = tid & 15, xr32 = tid >> 4;
  const int c8 = tid & 7, r16 = tid >> 3;

  float ss[XP];
  XStage<XH, NT> xs;
  WStage<NT> ws;
  // Loads K step t of tile `tile` (tile >= last: nothing; every load returns 0).
  auto load = [&](int tile, int t) {
    const bool live = tile < last;
    TileAt d{};
    if (live) d = decode(tile);
    const int bt = d.bt, r0 = d.r0, c0 = d.c0;
    const int rows = live ? min(kBM, n - r0) : 0;
    const rsrc_t xr = make_rsrc(static_cast<const unsigned char*>(p.x) +
                                    (bt * p.x_bstride + (long)r0 * p.ldx) * xbytes,
                                rows ? (unsigned)(((long)(rows - 1) * p.ldx + k) * xbytes) : 0u);
    const rsrc_t wr = make_rsrc(p.wt + d.wofs + (long)c0 * k,
                                live ? (unsigned)((long)kBN * k * 2) : 0u);
    const int k0 = t * kBK;
    if constexpr (XH) {
      const int kc = k0 + 8 * c8;
      const unsigned skip = kc < k ? 0u : kNowhere;
      for (int i = 0; i < XP; i++)
        xs.v[i] = __builtin_amdgcn_raw_buffer_load_b128(
            xr, ((unsigned)(r16 + XROWS * i) * ldx_b + kc * 2) | skip, 0, 0);
    } else {
      const int kc = k0 + 4 * x4;
      const unsigned skip = kc < k ? 0u : kNowhere;
      for (int i = 0; i < XP; i++)
        xs.v[i] = __builtin_bit_cast(
            float4, __builtin_amdgcn_raw_buffer_load_b128(
                        xr, ((unsigned)(xr32 + XROWS * i) * ldx_b + kc * 4) | skip, 0, 0));
    }
    const int kc = k0 + 8 * c8;
    const unsigned skip = kc < k ? 0u : kNowhere;
    for (int i = 0; i < WP; i++)
      ws.v[i] = __builtin_amdgcn_raw_buffer_load_b128(
          wr, ((unsigned)(r16 + WROWS * i) * k2 + kc * 2) | skip, 0, 0);
  };
  auto store = [&](int buf) {
    unsigned char* X = lds + buf * kTileBytes;
    unsigned char* Wt = lds + (2 + buf) * kTileBytes;
    if constexpr (XH) {
      for (int i = 0; i < XP; i++) {
        if constexpr (NORM) {
          const h16x8 h = __builtin_bit_cast(h16x8, xs.v[i]);
          float s = 0.f;
          for (int j = 0; j < 8; j++) s += (float)h[j] * (float)h[j];
          ss[i] += s;
        }
        *reinterpret_cast<u32x4*>(X + tile_offset(r16 + XROWS * i, c8)) = xs.v[i];
      }
    } else {
      for (int i = 0; i < XP; i++) {
        const float4 v = xs.v[i];
        if constexpr (NORM) ss[i] += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        const u32x2 h = {pack_h2(v.x, v.y), pack_h2(v.z, v.w)};
        *reinterpret_cast<u32x2*>(X + tile_offset(xr32 + XROWS * i, x4 >> 1) + ((x4 & 1) << 3)) =
            h;
      }
    }
    for (int i = 0; i < WP; i++)
      *reinterpret_cast<u32x4*>(Wt + tile_offset(r16 + WROWS * i, c8)) = ws.v[i];
  };

  const int qr = (wave & 1) * 64, qc = (wave >> 1) * 16 * CB;
  const int lr = lane & 15, lk = lane >> 4;
  f32x4 acc[CB][4];
  auto compute = [&](int buf) {
    const unsigned char* X = lds + buf * kTileBytes;
    const unsigned char* Wt = lds + (2 + buf) * kTileBytes;
    for (int kk = 0; kk < 2; kk++) {
      u32x4 a[CB], b[4];
      for (int cb = 0; cb < CB; cb++)
        a[cb] = *reinterpret_cast<const u32x4*>(Wt + tile_offset(qc + cb * 16 + lr, kk * 4 + lk));
      for (int rb = 0; rb < 4; rb++)
        b[rb] = *reinterpret_cast<const u32x4*>(X + tile_offset(qr + rb * 16 + lr, kk * 4 + lk));
      for (int cb = 0; cb < CB; cb++)
        for (int rb = 0; rb < 4; rb++) acc[cb][rb] = mfma16x16x32(a[cb], b[rb], acc[cb][rb]);
    }
  };

  // Epilogue constants: this thread's 4 output columns (c4) in the row-wise pass.
  const int c4 = tid & 31, erow = tid >> 5;
  const void* any = p.wt;  // base of the empty descriptors of absent operands
  const rsrc_t roper = make_rsrc(p.rope ? static_cast<const void*>(p.rope) : any,
                                 p.rope ? (unsigned)(4 * p.tokens * 64 * 4) : 0u);

  load(first, 0);
  for (int tile = first; tile < last; tile += slots) {
    const TileAt d = decode(tile);
    const int r0 = d.r0, c0 = d.c0, m = d.m;
    const int rows = min(kBM, n - r0);
    if constexpr (NORM)
      for (int i = 0; i < XP; i++) ss[i] = 0.f;
    for (int a = 0; a < CB; a++)
      for (int b = 0; b < 4; b++) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
    store(0);
    __syncthreads();
    for (int t = 0; t < ktiles; t++) {
      // Next step of this tile, or the first step of the next tile (in flight over the epilogue).
      if (t + 1 < ktiles)
        load(tile, t + 1);
      else
        load(tile + slots, 0);
      compute(t & 1);
      if (t + 1 < ktiles) store((t + 1) & 1);
      __syncthreads();
    }
    if constexpr (NORM) {
      // Per-row sums of squares: partials of the lanes sharing a row, then one value per row.
      constexpr int kLanesPerRow = XH ? 8 : 16;
      for (int i = 0; i < XP; i++) {
        float s = ss[i];
        for (int o = 1; o < kLanesPerRow; o <<= 1) s += __shfl_xor(s, o);
        const int row = XH ? r16 + XROWS * i : xr32 + XROWS * i;
        if ((XH ? c8 : x4) == 0) lds_inv[row] = 1.0f / fmaxf(sqrtf(s), 1e-12f);
      }
    }
    // Token index of each tile row for the rotary epilogue (read after the barrier below).
    if ((EPI == kEpiRuntime ? p.rope != nullptr : (EPI & kEpiRope) != 0) && tid < kBM)
      lds_tok[tid] = ((r0 + tid) / p.token_div) % p.tokens;
    // Accumulators -> LDS (the K-step buffers are free after the barrier above).
    for (int rb = 0; rb < 4; rb++)
      for (int cb = 0; cb < CB; cb++)
        *reinterpret_cast<f32x4*>(lds + stage_offset(qr + rb * 16 + lr, (qc + cb * 16) / 4 + lk)) =
            acc[cb][rb];
    __syncthreads();

    // Row-wise epilogue: bias -> GELU -> rotary -> residual (fused/gemm.rs:46-82 order).
    constexpr int obytes = OH ? 2 : 4;
    const long orow = d.oofs + (long)r0 * m;
    const rsrc_t outr = make_rsrc(static_cast<unsigned char*>(p.out) + orow * obytes,
                                  (unsigned)((long)rows * m * obytes));
    const rsrc_t resr = make_rsrc(p.residual ? static_cast<const void*>(p.residual + orow) : any,
                                  p.residual ? (unsigned)((long)rows * m * 4) : 0u);
    const int col = c0 + 4 * c4;
    float4 bias = make_float4(0.f, 0.f, 0.f, 0.f);
    if (p.bias) bias = *reinterpret_cast<const float4*>(p.bias + d.bofs + col);
    constexpr bool RT = EPI == kEpiRuntime;
    const bool gelu = RT ? p.gelu != 0 : (EPI & kEpiGelu) != 0;
    const bool tanh_act = RT ? p.tanh_act != 0 : (EPI & kEpiTanh) != 0;
    const bool residual = RT ? p.residual != nullptr : (EPI & kEpiResidual) != 0;
    const bool rope_any = RT ? p.rope != nullptr : (EPI & kEpiRope) != 0;
    const bool rot = rope_any && col < 2 * p.width;
    const int table = col < p.width ? 0 : 2;
    // Global inputs of one row (rotary table rows, residual), fetched one row ahead: the wait
    // for a row's inputs then never covers the stores of the rows before it (the vector
    // memory counter retires in order).
    struct RowIn {
      float4 c, s, r;
    };
    // The table rows are read for every column of a rotary product (rows of the v / gate
    // columns go unused), so the loads sit outside the per-lane rotation test.
    auto fetch = [&](int i) {
      const int lrow = erow + (NT / 32) * i;
      RowIn in;
      if (rope_any) {
        const unsigned c = ((unsigned)(table * p.tokens + lds_tok[lrow]) * 64 + (col & 63)) * 4;
        in.c = bload4<true>(roper, c);
        in.s = bload4<true>(roper, c + (unsigned)p.tokens * 256);
      }
      if (residual) in.r = bload4<true>(resr, ((unsigned)lrow * m + col) * 4);
      return in;
    };
    constexpr int kRows = kBM / (NT / 32);
    RowIn cur = fetch(0);
    // Rows past the tile's end are computed too (from zero x rows) and their stores fall
    // outside the output descriptor, so the loop has no exit test and unrolls.
#pragma unroll
    for (int i = 0; i < kRows; i++) {
      const int lrow = erow + (NT / 32) * i;
      const RowIn in = cur;
      if (i + 1 < kRows) cur = fetch(i + 1);
      const float4 a = *reinterpret_cast<const float4*>(lds + stage_offset(lrow, c4));
      const float inv = NORM ? lds_inv[lrow] : 1.0f;
      float4 v = make_float4(a.x * inv + bias.x, a.y * inv + bias.y, a.z * inv + bias.z,
                             a.w * inv + bias.w);
      if (gelu) v = make_float4(gelu_fast(v.x), gelu_fast(v.y), gelu_fast(v.z), gelu_fast(v.w));
      if (tanh_act) v = make_float4(tanh_fast(v.x), tanh_fast(v.y), tanh_fast(v.z), tanh_fast(v.w));
      if (rot) {
        v = rotate4(v, in.c, in.s);
        if (table == 0 && p.q_scale != 0.f)
          v = make_float4(v.x * p.q_scale, v.y * p.q_scale, v.z * p.q_scale, v.w * p.q_scale);
      }
      const unsigned off = (unsigned)lrow * m + col;
      if (residual) v = make_float4(v.x + in.r.x, v.y + in.r.y, v.z + in.r.z, v.w + in.r.w);
      if constexpr (OH) {
        const u32x2 h = {pack_h2(v.x, v.y), pack_h2(v.z, v.w)};
        __builtin_amdgcn_raw_buffer_store_b64(h, outr, off * 2, 0, 0);
      } else {
        bstore4<true>(outr, off * 4, v);
      }
    }
    __syncthreads();  // the staging tile is the next tile's K-step buffers
  }
}

template <bool XH, bool OH, bool NORM, int EPI>
void launch_epi(const Gemm16Params& p, int grid, int col_tiles, int tiles, hipStream_t stream) {
  constexpr int waves = XH ? 4 : 8;
  hipLaunchKernelGGL((gemm16_kernel<XH, OH, NORM, waves, EPI>), dim3(grid), dim3(waves * 64), 0,
                     stream, p, col_tiles, tiles);
}

// Compile-time epilogues for the combinations the block and the mask estimator run; any other
// flag set takes the runtime-flag kernel.
template <bool XH, bool OH, bool NORM>
void launch(const Gemm16Params& p, int grid, int col_tiles, int tiles, hipStream_t stream) {
  const int epi = (p.gelu ? kEpiGelu : 0) | (p.tanh_act ? kEpiTanh : 0) |
                  (p.rope ? kEpiRope : 0) | (p.residual ? kEpiResidual : 0);
  if constexpr (!NORM && OH) {
    if (epi == kEpiGelu) return launch_epi<XH, OH, NORM, kEpiGelu>(p, grid, col_tiles, tiles, stream);
    if (epi == kEpiTanh) return launch_epi<XH, OH, NORM, kEpiTanh>(p, grid, col_tiles, tiles, stream);
    if (XH && epi == kEpiRope)
      return launch_epi<XH, OH, NORM, kEpiRope>(p, grid, col_tiles, tiles, stream);
  }
  if constexpr (XH && !NORM && !OH) {
    if (epi == 0) return launch_epi<XH, OH, NORM, 0>(p, grid, col_tiles, tiles, stream);
    if (epi == kEpiResidual)
      return launch_epi<XH, OH, NORM, kEpiResidual>(p, grid, col_tiles, tiles, stream);
  }
  launch_epi<XH, OH, NORM, kEpiRuntime>(p, grid, col_tiles, tiles, stream);
}

}  // namespace

int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

hipError_t launch_gemm16(const Gemm16Params& p, hipStream_t stream) {
  const int row_tiles = (p.n + kBM - 1) / kBM, col_tiles = p.m / kBN;
  const int tiles = p.group_of_tile ? p.group_tiles
                                    : row_tiles * col_tiles * (p.batch > 1 ? p.batch : 1);
  // Resident workgroups only (two 4-wave ones per CU for fp16 x; one 8-wave one for fp32 x,
  // whose registers allow three waves per SIMD), a multiple of the XCD count, no more than the
  // tiles need.
  int grid = (p.x_half ? 2 : 1) * device_cus();
  const int need = (tiles + kXcds - 1) / kXcds * kXcds;
  grid = (grid < need ? grid : need) / kXcds * kXcds;
  if (grid < kXcds) grid = kXcds;
  const int key = (p.x_half ? 4 : 0) | (p.out_half ? 2 : 0) | (p.norm ? 1 : 0);
  switch (key) {
    case 0: launch<false, false, false>(p, grid, col_tiles, tiles, stream); break;
    case 1: launch<false, false, true>(p, grid, col_tiles, tiles, stream); break;
    case 2: launch<false, true, false>(p, grid, col_tiles, tiles, stream); break;
    case 3: launch<false, true, true>(p, grid, col_tiles, tiles, stream); break;
    case 4: launch<true, false, false>(p, grid, col_tiles, tiles, stream); break;
    case 5: launch<true, false, true>(p, grid, col_tiles, tiles, stream); break;
    case 6: launch<true, true, false>(p, grid, col_tiles, tiles, stream); break;
    default: launch<true, true, true>(p, grid, col_tiles, tiles, stream); break;
  }
  return hipGetLastError();
}

}  // namespace ancha
