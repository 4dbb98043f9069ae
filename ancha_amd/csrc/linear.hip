// Projection GEMM with the RoFormer epilogues for CDNA4 (gfx950): out = epilogue(x . w) with
// fp32 operands in HBM, fp16 MFMA operands and fp32 accumulation. Replaces the CubeCL GEMM of
// crates/ancha-models/src/fused/gemm.rs:86-211 (launch :242-311, epilogue :46-82) behind
// `fused::linear` (fused/mod.rs:100-176).
//
// One workgroup (4 waves) computes a 128-row x 128-column output tile; each wave owns a
// 64 x 64 quadrant as 4 x 4 MFMA tiles. The product is formed transposed, out^T = w^T . x^T
// (A operand = 16 output columns of w^T, B operand = 16 rows of x^T), so every lane ends with
// four consecutive output columns of one row: the epilogue reads bias / residual / rotary table
// and writes the output as 16-byte vectors, and each rotary pair sits inside one lane.
//
// K advances in 64-wide steps. x and w tiles are loaded from HBM as fp32 one step ahead into
// registers, converted to fp16 and written to a double-buffered LDS tile ([row][k] for x,
// [column][k] for w, so both MFMA operands are single 16-byte LDS reads); rows of 64 fp16 are
// 8 chunks of 16 bytes, XOR-swizzled by (r ^ r>>2) & 7 so the transposing w writes and the
// operand reads of 16 consecutive rows hit distinct banks.
//
// The shapes are HBM-bound at fp32 I/O (K = 384..1536): the tile order is XCD-aware so the
// column tiles of one row block run on one XCD and re-read that row block from its L2.
#include "buffer.hpp"
#include "common.hpp"
#include "gemm.hpp"
#include "kernels.hpp"

namespace ancha {
namespace {

using namespace gemm;

template <bool ALIGNED, bool NORM>
__global__ __launch_bounds__(kThreads) void linear_kernel(LinearParams p, int col_tiles) {
  __shared__ __attribute__((aligned(16))) unsigned char lds_x[2][kTileBytes];
  __shared__ __attribute__((aligned(16))) unsigned char lds_w[2][kTileBytes];
  __shared__ float lds_inv[kBM];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  const int r0 = (tile / col_tiles) * kBM, c0 = (tile % col_tiles) * kBN;
  const int rows = min(kBM, p.n - r0);
  const int n = p.n, k = p.k, m = p.m;

  // Per-workgroup descriptors: offsets stay small whatever n is; rows past n read as 0.
  const rsrc_t xr = make_rsrc(p.x + (long)r0 * p.ldx,
                              (unsigned)(((long)(rows - 1) * p.ldx + k) * 4));
  const rsrc_t wr = make_rsrc(p.w, (unsigned)((long)k * m * 4));

  // Staging roles. x: 16 lanes per row (float4 each), rows xrow + 16i. w: 32 lanes per k row
  // (4 columns each), 8 consecutive k rows per lane.
  const int xk = tid & 15, xrow = tid >> 4;
  const int wc = tid & 31, wk = tid >> 5;
  const unsigned ldx4 = (unsigned)p.ldx * 4, m4 = (unsigned)m * 4;

  float4 xv[8], wv[8];
  float ss[8];
  if constexpr (NORM)
    for (int i = 0; i < 8; i++) ss[i] = 0.f;

  auto load = [&](int k0) {
    const int kx = k0 + 4 * xk;
    for (int i = 0; i < 8; i++)
      xv[i] = load_masked<ALIGNED>(xr, (unsigned)(xrow + 16 * i) * ldx4 + kx * 4, kx, k);
    const int col = c0 + 4 * wc;
    for (int j = 0; j < 8; j++)
      wv[j] = load_masked<ALIGNED>(wr, (unsigned)(k0 + 8 * wk + j) * m4 + col * 4, col, m);
  };
  auto store = [&](int buf) {
    unsigned char* X = lds_x[buf];
    unsigned char* Wt = lds_w[buf];
    for (int i = 0; i < 8; i++) {
      const int r = xrow + 16 * i;
      if constexpr (NORM)
        ss[i] += xv[i].x * xv[i].x + xv[i].y * xv[i].y + xv[i].z * xv[i].z + xv[i].w * xv[i].w;
      const u32x2 h = {pack_h2(xv[i].x, xv[i].y), pack_h2(xv[i].z, xv[i].w)};
      *reinterpret_cast<u32x2*>(X + tile_offset(r, xk >> 1) + ((xk & 1) << 3)) = h;
    }
    for (int c = 0; c < 4; c++) {
      const u32x4 h = {pack_h2(comp(wv[0], c), comp(wv[1], c)), pack_h2(comp(wv[2], c), comp(wv[3], c)),
                       pack_h2(comp(wv[4], c), comp(wv[5], c)), pack_h2(comp(wv[6], c), comp(wv[7], c))};
      *reinterpret_cast<u32x4*>(Wt + tile_offset(4 * wc + c, wk)) = h;
    }
  };

  // Quadrant of this wave and its operand rows.
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

  const int ktiles = (k + kBK - 1) / kBK;
  load(0);
  store(0);
  __syncthreads();
  for (int t = 0; t < ktiles; t++) {
    const bool more = t + 1 < ktiles;
    if (more) load((t + 1) * kBK);
    compute(t & 1);
    if (more) store((t + 1) & 1);
    __syncthreads();
  }

  if constexpr (NORM) {
    for (int i = 0; i < 8; i++) {
      float s = ss[i];
      s += __shfl_xor(s, 1);
      s += __shfl_xor(s, 2);
      s += __shfl_xor(s, 4);
      s += __shfl_xor(s, 8);
      if (xk == 0) lds_inv[xrow + 16 * i] = 1.0f / fmaxf(sqrtf(s), 1e-12f);
    }
    __syncthreads();
  }

  // Epilogue: bias -> GELU -> rotary -> residual, as the reference orders them.
  const rsrc_t outr = make_rsrc(p.out + (long)r0 * m, (unsigned)((long)rows * m * 4));
  const rsrc_t resr = make_rsrc(p.residual ? p.residual + (long)r0 * m : p.out,
                                p.residual ? (unsigned)((long)rows * m * 4) : 0u);
  const rsrc_t biasr = make_rsrc(p.bias ? p.bias : p.out, p.bias ? (unsigned)m4 : 0u);
  const rsrc_t roper = make_rsrc(p.rope ? p.rope : p.out,
                                 p.rope ? (unsigned)(4 * p.tokens * 64 * 4) : 0u);
  for (int rb = 0; rb < 4; rb++) {
    const int lrow = qr + rb * 16 + lr;  // row inside the tile
    const int row = r0 + lrow;
    const float inv = NORM ? lds_inv[lrow] : 1.0f;
    const int t = p.rope ? row % p.tokens : 0;
    for (int cb = 0; cb < 4; cb++) {
      const int col = c0 + qc + cb * 16 + 4 * lk;
      if (row >= n || col >= m) continue;
      const unsigned off = (unsigned)lrow * m4 + col * 4;
      f32x4 a = acc[cb][rb];
      float4 v = make_float4(a[0] * inv, a[1] * inv, a[2] * inv, a[3] * inv);
      if (p.bias) {
        const float4 b = load_masked<ALIGNED>(biasr, col * 4, col, m);
        v = make_float4(v.x + b.x, v.y + b.y, v.z + b.z, v.w + b.w);
      }
      if (p.gelu) v = make_float4(gelu_erf(v.x), gelu_erf(v.y), gelu_erf(v.z), gelu_erf(v.w));
      if (p.rope && col < 2 * p.width) {
        const int table = col < p.width ? 0 : 2;
        const unsigned c = ((unsigned)(table * p.tokens + t) * 64 + (col & 63)) * 4;
        const float4 cs = bload4<ALIGNED>(roper, c);
        const float4 sn = bload4<ALIGNED>(roper, c + (unsigned)p.tokens * 256);
        v = rotate4(v, cs, sn);
      }
      if (p.residual) {
        const float4 r = load_masked<ALIGNED>(resr, off, col, m);
        v = make_float4(v.x + r.x, v.y + r.y, v.z + r.z, v.w + r.w);
      }
      store_masked<ALIGNED>(outr, off, col, m, v);
    }
  }
}

}  // namespace

hipError_t launch_linear(const LinearParams& p, bool aligned, hipStream_t stream) {
  const int row_tiles = (p.n + kBM - 1) / kBM, col_tiles = (p.m + kBN - 1) / kBN;
  const dim3 grid(row_tiles * col_tiles), block(kThreads);
  if (aligned) {
    if (p.norm)
      hipLaunchKernelGGL((linear_kernel<true, true>), grid, block, 0, stream, p, col_tiles);
    else
      hipLaunchKernelGGL((linear_kernel<true, false>), grid, block, 0, stream, p, col_tiles);
  } else {
    if (p.norm)
      hipLaunchKernelGGL((linear_kernel<false, true>), grid, block, 0, stream, p, col_tiles);
    else
      hipLaunchKernelGGL((linear_kernel<false, false>), grid, block, 0, stream, p, col_tiles);
  }
  return hipGetLastError();
}

}  // namespace ancha
