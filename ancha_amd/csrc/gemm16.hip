// Projection GEMM of the RoFormer block on load-time fp16 weights (gfx950):
// out = epilogue(x . W) with W stored once, at block load, as fp16 W^T [m][k] (k contiguous),
// x fp32 or fp16 [n][k], out fp32 or fp16 [n][m]. The arithmetic is that of linear.hip (every
// operand rounded to fp16 once, fp32 accumulation, the same epilogue), so an fp16 activation
// written by one GEMM and read by the next is bit-for-bit the operand the next GEMM would
// round to; only the bytes moved change.
//
// Workgroup = 4 waves, 128 x 128 output tile, 64 x 64 per wave (4 x 4 MFMA 16x16x32 tiles),
// K in 64-wide steps through a double-buffered LDS tile, as in linear.hip. With fp16 x, global
// loads run two K steps ahead (two register sets, used alternately), so each load has two steps
// of MFMA work and barriers to arrive before it is needed; fp32 x keeps one step (its tiles
// need twice the registers, and two workgroups per CU hide more than a second set would). Loads past the end of K or of the rows are given
// an offset outside the buffer: they return 0 without touching memory, and the loop issues the
// same loads every step (no conditional loads, so the compiler's wait counts stay exact).
#include "buffer.hpp"
#include "common.hpp"
#include "gemm.hpp"
#include "kernels.hpp"

namespace ancha {
namespace {

using namespace gemm;

// Offset added to a load that must read 0 (beyond every buffer range used here: < 2^31).
constexpr unsigned kNowhere = 0x80000000u;

template <bool XH>
struct XStage;  // registers holding one 128 x 64 x tile

template <>
struct XStage<false> {  // fp32 x: 8 rows x float4 per thread
  float4 v[8];
};
template <>
struct XStage<true> {  // fp16 x: 4 rows x 8 halves per thread
  u32x4 v[4];
};

struct WStage {  // fp16 W^T: 4 rows (output columns) x 8 halves per thread
  u32x4 v[4];
};

template <bool XH, bool OH, bool NORM>
__global__ __launch_bounds__(kThreads, XH ? 1 : 2) void gemm16_kernel(Gemm16Params p, int col_tiles) {
  __shared__ __attribute__((aligned(16))) unsigned char lds_x[2][kTileBytes];
  __shared__ __attribute__((aligned(16))) unsigned char lds_w[2][kTileBytes];
  __shared__ float lds_inv[kBM];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  const int r0 = (tile / col_tiles) * kBM, c0 = (tile % col_tiles) * kBN;
  const int rows = min(kBM, p.n - r0);
  const int n = p.n, k = p.k, m = p.m;
  constexpr int xbytes = XH ? 2 : 4;

  const rsrc_t xr = make_rsrc(static_cast<const unsigned char*>(p.x) + (long)r0 * p.ldx * xbytes,
                              (unsigned)(((long)(rows - 1) * p.ldx + k) * xbytes));
  const rsrc_t wr = make_rsrc(p.wt + (long)c0 * k, (unsigned)((long)min(kBN, m - c0) * k * 2));
  const unsigned ldx_b = (unsigned)p.ldx * xbytes, k2 = (unsigned)k * 2;
  const int ktiles = (k + kBK - 1) / kBK;

  // Staging roles: fp32 x: 16 lanes per row (float4), rows xr32 + 16i; fp16 x and W^T: 8 lanes
  // per row (8 halves), rows r16 + 32i.
  const int x4 = tid & 15, xr32 = tid >> 4;
  const int c8 = tid & 7, r16 = tid >> 3;

  float ss[8];
  if constexpr (NORM)
    for (int i = 0; i < 8; i++) ss[i] = 0.f;

  auto load = [&](XStage<XH>& xs, WStage& ws, int t) {
    const int k0 = t * kBK;
    if constexpr (XH) {
      const int kc = k0 + 8 * c8;
      const unsigned skip = (t < ktiles && kc < k) ? 0u : kNowhere;
      for (int i = 0; i < 4; i++)
        xs.v[i] = __builtin_amdgcn_raw_buffer_load_b128(
            xr, ((unsigned)(r16 + 32 * i) * ldx_b + kc * 2) | skip, 0, 0);
    } else {
      const int kc = k0 + 4 * x4;
      const unsigned skip = (t < ktiles && kc < k) ? 0u : kNowhere;
      for (int i = 0; i < 8; i++)
        xs.v[i] = __builtin_bit_cast(
            float4, __builtin_amdgcn_raw_buffer_load_b128(
                        xr, ((unsigned)(xr32 + 16 * i) * ldx_b + kc * 4) | skip, 0, 0));
    }
    const int kc = k0 + 8 * c8;
    const unsigned skip = (t < ktiles && kc < k) ? 0u : kNowhere;
    for (int i = 0; i < 4; i++)
      ws.v[i] = __builtin_amdgcn_raw_buffer_load_b128(
          wr, ((unsigned)(r16 + 32 * i) * k2 + kc * 2) | skip, 0, 0);
  };
  auto store = [&](const XStage<XH>& xs, const WStage& ws, int buf) {
    unsigned char* X = lds_x[buf];
    unsigned char* Wt = lds_w[buf];
    if constexpr (XH) {
      for (int i = 0; i < 4; i++) {
        if constexpr (NORM) {
          const h16x8 h = __builtin_bit_cast(h16x8, xs.v[i]);
          float s = 0.f;
          for (int j = 0; j < 8; j++) s += (float)h[j] * (float)h[j];
          ss[i] += s;
        }
        *reinterpret_cast<u32x4*>(X + tile_offset(r16 + 32 * i, c8)) = xs.v[i];
      }
    } else {
      for (int i = 0; i < 8; i++) {
        const float4 v = xs.v[i];
        if constexpr (NORM) ss[i] += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        const u32x2 h = {pack_h2(v.x, v.y), pack_h2(v.z, v.w)};
        *reinterpret_cast<u32x2*>(X + tile_offset(xr32 + 16 * i, x4 >> 1) + ((x4 & 1) << 3)) = h;
      }
    }
    for (int i = 0; i < 4; i++)
      *reinterpret_cast<u32x4*>(Wt + tile_offset(r16 + 32 * i, c8)) = ws.v[i];
  };

  const int qr = (wave & 1) * 64, qc = (wave >> 1) * 64;
  const int lr = lane & 15, lk = lane >> 4;
  f32x4 acc[4][4];
  for (int a = 0; a < 4; a++)
    for (int b = 0; b < 4; b++) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int buf) {
    const unsigned char* X = lds_x[buf];
    const unsigned char* Wt = lds_w[buf];
    for (int kk = 0; kk < 2; kk++) {
      u32x4 a[4], b[4];
      for (int cb = 0; cb < 4; cb++)
        a[cb] = *reinterpret_cast<const u32x4*>(Wt + tile_offset(qc + cb * 16 + lr, kk * 4 + lk));
      for (int rb = 0; rb < 4; rb++)
        b[rb] = *reinterpret_cast<const u32x4*>(X + tile_offset(qr + rb * 16 + lr, kk * 4 + lk));
      for (int cb = 0; cb < 4; cb++)
        for (int rb = 0; rb < 4; rb++) acc[cb][rb] = mfma16x16x32(a[cb], b[rb], acc[cb][rb]);
    }
  };

  XStage<XH> x0;
  WStage w0;
  load(x0, w0, 0);
  if constexpr (XH) {
    // fp16 x: two register sets, loads two K steps ahead.
    XStage<XH> x1;
    WStage w1;
    load(x1, w1, 1);
    store(x0, w0, 0);
    __syncthreads();
    load(x0, w0, 2);
    for (int t = 0; t < ktiles; t += 2) {
      // Tile t is in LDS buffer 0; registers: set 1 = tile t+1, set 0 = tile t+2 (in flight).
      compute(0);
      store(x1, w1, 1);
      __syncthreads();
      load(x1, w1, t + 3);
      if (t + 1 >= ktiles) break;
      compute(1);
      store(x0, w0, 0);
      __syncthreads();
      load(x0, w0, t + 4);
    }
  } else {
    // fp32 x (twice the register bytes per tile): one register set, loads one K step ahead,
    // which keeps two workgroups per CU.
    store(x0, w0, 0);
    __syncthreads();
    load(x0, w0, 1);
    for (int t = 0; t < ktiles; t++) {
      compute(t & 1);
      store(x0, w0, (t + 1) & 1);
      __syncthreads();
      load(x0, w0, t + 2);
    }
  }

  if constexpr (NORM) {
    // Per-row sums of squares: partials of the lanes sharing a row, then one value per row.
    constexpr int kRowsPerThread = XH ? 4 : 8;
    constexpr int kLanesPerRow = XH ? 8 : 16;
    for (int i = 0; i < kRowsPerThread; i++) {
      float s = ss[i];
      for (int o = 1; o < kLanesPerRow; o <<= 1) s += __shfl_xor(s, o);
      const int row = XH ? r16 + 32 * i : xr32 + 16 * i;
      if ((XH ? c8 : x4) == 0) lds_inv[row] = 1.0f / fmaxf(sqrtf(s), 1e-12f);
    }
    __syncthreads();
  }

  // Epilogue: bias -> GELU -> rotary -> residual (fused/gemm.rs:46-82 order).
  constexpr int obytes = OH ? 2 : 4;
  const rsrc_t outr = make_rsrc(static_cast<unsigned char*>(p.out) + (long)r0 * m * obytes,
                                (unsigned)((long)rows * m * obytes));
  const rsrc_t resr = make_rsrc(p.residual ? p.residual + (long)r0 * m : p.bias,
                                p.residual ? (unsigned)((long)rows * m * 4) : 0u);
  const rsrc_t biasr = make_rsrc(p.bias ? p.bias : p.residual, p.bias ? (unsigned)m * 4 : 0u);
  const rsrc_t roper = make_rsrc(p.rope ? p.rope : p.bias,
                                 p.rope ? (unsigned)(4 * p.tokens * 64 * 4) : 0u);
  for (int rb = 0; rb < 4; rb++) {
    const int lrow = qr + rb * 16 + lr;
    const int row = r0 + lrow;
    const float inv = NORM ? lds_inv[lrow] : 1.0f;
    const int tok = p.rope ? row % p.tokens : 0;
    for (int cb = 0; cb < 4; cb++) {
      const int col = c0 + qc + cb * 16 + 4 * lk;
      if (row >= n) continue;
      const f32x4 a = acc[cb][rb];
      float4 v = make_float4(a[0] * inv, a[1] * inv, a[2] * inv, a[3] * inv);
      if (p.bias) {
        const float4 b = bload4<true>(biasr, col * 4);
        v = make_float4(v.x + b.x, v.y + b.y, v.z + b.z, v.w + b.w);
      }
      if (p.gelu) v = make_float4(gelu_erf(v.x), gelu_erf(v.y), gelu_erf(v.z), gelu_erf(v.w));
      if (p.rope && col < 2 * p.width) {
        const int table = col < p.width ? 0 : 2;
        const unsigned c = ((unsigned)(table * p.tokens + tok) * 64 + (col & 63)) * 4;
        v = rotate4(v, bload4<true>(roper, c), bload4<true>(roper, c + (unsigned)p.tokens * 256));
      }
      const unsigned off = (unsigned)lrow * m + col;  // element offset inside the tile rows
      if (p.residual) {
        const float4 r = bload4<true>(resr, off * 4);
        v = make_float4(v.x + r.x, v.y + r.y, v.z + r.z, v.w + r.w);
      }
      if constexpr (OH) {
        const u32x2 h = {pack_h2(v.x, v.y), pack_h2(v.z, v.w)};
        __builtin_amdgcn_raw_buffer_store_b64(h, outr, off * 2, 0, 0);
      } else {
        bstore4<true>(outr, off * 4, v);
      }
    }
  }
}

template <bool XH, bool OH, bool NORM>
void launch(const Gemm16Params& p, dim3 grid, int col_tiles, hipStream_t stream) {
  hipLaunchKernelGGL((gemm16_kernel<XH, OH, NORM>), grid, dim3(kThreads), 0, stream, p,
                     col_tiles);
}

}  // namespace

hipError_t launch_gemm16(const Gemm16Params& p, hipStream_t stream) {
  const int row_tiles = (p.n + kBM - 1) / kBM, col_tiles = p.m / kBN;
  const dim3 grid(row_tiles * col_tiles);
  const int key = (p.x_half ? 4 : 0) | (p.out_half ? 2 : 0) | (p.norm ? 1 : 0);
  switch (key) {
    case 0: launch<false, false, false>(p, grid, col_tiles, stream); break;
    case 1: launch<false, false, true>(p, grid, col_tiles, stream); break;
    case 2: launch<false, true, false>(p, grid, col_tiles, stream); break;
    case 3: launch<false, true, true>(p, grid, col_tiles, stream); break;
    case 4: launch<true, false, false>(p, grid, col_tiles, stream); break;
    case 5: launch<true, false, true>(p, grid, col_tiles, stream); break;
    case 6: launch<true, true, false>(p, grid, col_tiles, stream); break;
    default: launch<true, true, true>(p, grid, col_tiles, stream); break;
  }
  return hipGetLastError();
}

}  // namespace ancha
