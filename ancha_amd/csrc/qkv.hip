// Packed q | k | v | gate projection of the RoFormer block on gfx950 (crates/ancha-models/src/
// roformer.rs:477-485: fused::linear with the bias + rotary epilogue of fused/gemm.rs:46-82):
//   out[r][c] = epilogue(sum_k xh[r][k] W^T[c][k] + bias[c]), fp16,
// with the interleaved rotary embedding on columns [0, 2 width) (queries, then keys, of token
// (r / token_div) % tokens) and the queries also times q_scale (log2 e for the exp2 softmax).
// Only the columns that hold values are computed and written: q, k, v and the heads' gate
// logits, 3 width + width / 64 of them, rounded up to a 32-column block; the packed layout's
// zero padding after them is never read by the attention kernels and is left as it is.
//
// 128 rows per workgroup (96 at dim 512): their fp16 operand rows sit in LDS for the whole block
// as B fragments of v_mfma_f32_32x32x16_f16 (straight from HBM with direct-to-LDS loads), with the
// rows' rotary cos / sin (32 + 32 per row) next to them. The 8 waves walk the output in pairs of
// 32-column blocks (pair p on SIMD p % 4, so the SIMDs get the same count); per pair a wave
// accumulates all its rows (4 or 3 32-row MFMA tiles per block) over K, so each operand B
// fragment read from LDS feeds two MFMAs and each weight A fragment (a contiguous kilobyte of the
// fragment-major W^T) four (three). The epilogue takes one 32-row tile of the pair at a time: bias,
// rotary and query scale on the accumulators (lane l owns row l % 32, columns 8q + 4(l/32) .. +3
// of each block: both members of every rotary pair), fp16 into a 4 KB staging area of the wave,
// read back so that each store covers 8 whole rows of the pair, i.e. whole 128-byte lines,
// written non-temporally (the projection is read once, by the next kernel). Measured against
// stores of 32-byte row pieces from the accumulators: the 320 MB output costs ~26 % of the
// kernel that way, whole lines through the caches save 10 % of it, non-temporal whole lines 17 %.
// The same kernel (TANH) runs the mask heads' first hidden layer: bias + tanh on every column,
// per-band products of `rows` rows, a band's row blocks on one XCD.
// An odd last block is split by row tile over the first four (three) waves, its first weight
// steps loaded by the ring of each wave's last pair. No
// barriers inside the column walk, so the two waves of a SIMD drift apart and one's epilogue
// runs beside the other's MFMAs. At dim 512 the operand rows, tables and staging areas of 96
// rows fill 152 KB of the LDS.
#include "buffer.hpp"
#include "common.hpp"
#include "gemm.hpp"
#include "kernels.hpp"

namespace ancha {
namespace {

constexpr int kWaves = 8;
constexpr int kFrag = 1024;

// SD = dim / 16 k steps (dims 128 - 512); NR 32-row tiles per row block (4; 3 at dim 512).
// TANH: the mask heads' hidden layer (bias + tanh on every column, no rotary table, p.batch
// products of p.rows rows each).
template <int SD, int NR, bool TANH = false>
__global__ __launch_bounds__(kWaves * 64, 1) void qkv_kernel(QkvParams p) {
  constexpr int kRows = 32 * NR;
  constexpr int kX = kRows * SD * 16 * 2;      // operand fragments
  // Per row: 16 chunks of (cos, sin) for two rotary pairs, chunk c at position c ^ (row & 15)
  // (rows 256 bytes apart would otherwise put one column's reads of 32 rows in one bank).
  constexpr int kT = kRows * 64 * 4;
  __shared__ __attribute__((aligned(16))) unsigned char lds[kX + kT];
  float* const cs = reinterpret_cast<float*>(lds + kX);
  // Per wave: one row tile of a pair's output, 32 rows x 128 bytes, 16-byte chunk c of row r at
  // position c ^ ((r >> 1) & 7), so a wave's stores leave as whole 128-byte lines (8 rows per
  // store). Two rows share a 256-byte line of the 64 banks: with that swizzle the 16 chunks of
  // two rows that one LDS cycle of the 16-byte reads serves fall on 16 bank groups, and with the
  // two 8-byte halves of every chunk swapped in rows 16-31 the 32 lanes (rows) that one cycle of
  // the 8-byte accumulator writes serves cover all 64 banks.
  __shared__ __attribute__((aligned(16))) unsigned char stage[kWaves][32 * 128];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, col = lane & 31;
  const unsigned lane16 = (unsigned)lane * 16;
  const int dim = SD * 16;
  // q, k, v and one gate column per head (all columns for TANH)
  const int used = TANH ? p.cols : 3 * p.width + p.width / 64;
  const int blocks = (used + 31) / 32;
  const int pairs = blocks / 2;
  const bool odd = (blocks & 1) != 0;
  rsrc_t wr = make_rsrc(p.w, (unsigned)(p.cols * dim * 2));
  rsrc_t br = make_rsrc(p.bias, (unsigned)(p.cols * 4));
  const rsrc_t tr = make_rsrc(TANH ? p.bias : p.rope, TANH ? 0u : (unsigned)(4 * p.tokens * 256));

  auto load_bias = [&](int b, float4 (&bias)[4]) {
#pragma unroll
    for (int q = 0; q < 4; q++)
      bias[q] = __builtin_bit_cast(
          float4, __builtin_amdgcn_raw_buffer_load_b128(br, 16 * half,
                                                        (unsigned)(32 * b + 8 * q) * 4, 0));
  };
  // Bias -> rotary -> query scale (fused/gemm.rs:46-82 order) of row tile j of output block b,
  // as fp16: packed[q] holds this lane's row 32 j + l % 32, columns 8 q + 4 (l / 32) .. + 3.
  auto tile_values = [&](const f32x16& acc, int b, int j, const float4 (&bias)[4],
                         u32x2 (&packed)[4]) {
    const bool rq = 32 * b < p.width, rk = !rq && 32 * b < 2 * p.width;
    const int r = 32 * j + col;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int pair = ((32 * b + 8 * q + 4 * half) & 63) >> 1;
      float4 v = make_float4(acc[4 * q] + bias[q].x, acc[4 * q + 1] + bias[q].y,
                             acc[4 * q + 2] + bias[q].z, acc[4 * q + 3] + bias[q].w);
      if constexpr (TANH) {
        v = make_float4(gemm::tanh_fast(v.x), gemm::tanh_fast(v.y), gemm::tanh_fast(v.z),
                        gemm::tanh_fast(v.w));
      } else if (rq || rk) {
        // (cos, sin) of pairs `pair` and `pair` + 1 (one 16-byte chunk).
        const float4 t = *reinterpret_cast<const float4*>(
            cs + r * 64 + (((pair >> 1) ^ (r & 15)) << 2));
        // Pair (c, c+1): y_c = x_c cos - x_{c+1} sin, y_{c+1} = x_{c+1} cos + x_c sin.
        float4 y = make_float4(v.x * t.x - v.y * t.y, v.y * t.x + v.x * t.y,
                               v.z * t.z - v.w * t.w, v.w * t.z + v.z * t.w);
        if (rq) {
          const float s = 0.125f * p.q_scale;
          y = make_float4(y.x * s, y.y * s, y.z * s, y.w * s);
        }
        v = y;
      }
      packed[q] = u32x2{pack_h2(v.x, v.y), pack_h2(v.z, v.w)};
    }
  };

  // Pairs of this wave: wave + 8 n (n < mine); pair index % 4 = wave % 4 = its SIMD.
  const int mine = pairs > wave ? (pairs - wave + kWaves - 1) / kWaves : 0;
  // k steps of weight fragments in flight (two fragments each): four at dims 384 (255 registers,
  // QKV 156 -> 150 us at 96 120 rows against two) and 512, two at dims 128 and 256.
  constexpr int PD = SD % 4 == 0 && SD > 16 ? 4 : 2;
  static_assert(SD % PD == 0 && SD >= PD, "K steps come in groups of PD");

  // Row blocks of each product (one product unless TANH).
  const int bpi = (p.rows + kRows - 1) / kRows;
  const int total = TANH ? bpi * p.batch : bpi;
  // TANH: each product has weights of its own, so the row blocks of one product are kept on one
  // XCD (consecutive logical ids share an XCD) and its weights come into that XCD's L2 once.
  const int first = TANH ? xcd_remap(blockIdx.x, gridDim.x) : (int)blockIdx.x;
  for (int blk = first; blk < total; blk += gridDim.x) {
    const int item = TANH ? blk / bpi : 0;
    const int row0 = (blk - item * bpi) * kRows;
    const int nrows = min(kRows, p.rows - row0);
    const rsrc_t xr = make_rsrc(p.xh + item * p.x_bstride + (long)row0 * dim,
                                (unsigned)(nrows * dim * 2));
    const rsrc_t outr = make_rsrc(p.out + item * p.out_bstride + (long)row0 * p.cols,
                                  (unsigned)(nrows * p.cols * 2));
    if constexpr (TANH) {
      wr = make_rsrc(p.w + item * p.w_bstride, (unsigned)(p.cols * dim * 2));
      br = make_rsrc(p.bias + item * p.b_bstride, (unsigned)(p.cols * 4));
    }
    // Operand rows as B fragments: fragment (jb, s) = rows 32 jb + (l % 32), k 16 s + 8 (l / 32).
    for (int f = wave; f < NR * SD; f += kWaves) {
      const int jb = f / SD, s = f % SD;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          xr, (__attribute__((address_space(3))) void*)(lds + f * kFrag), 16,
          ((unsigned)(32 * jb + col) * dim + 16 * s + 8 * half) * 2, 0, 0, 0);
    }
    // Key-table cos / sin of each row's token (the query tables are these times 1/8).
    for (int e = tid; e < (TANH ? 0 : kRows * 32); e += kWaves * 64) {
      const int r = e >> 5, i = e & 31;
      const int tok = ((row0 + r) / p.token_div) % p.tokens;
      float* slot = cs + r * 64 + (((i >> 1) ^ (r & 15)) << 2) + 2 * (i & 1);
      slot[0] = bload1(tr, (unsigned)((2 * p.tokens + tok) * 64 + 2 * i) * 4);
      slot[1] = bload1(tr, (unsigned)((3 * p.tokens + tok) * 64 + 2 * i + 1) * 4);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    // The A fragments of block 2 pr (x = 0) and 2 pr + 1 (x = 1) stream through the ring across
    // the wave's pairs; the last pair's last steps load the first steps of the odd block's tile
    // where the wave has one.
    const bool tile_odd = odd && wave < NR;
    u32x4 a[PD][2];
    if (mine > 0) {
#pragma unroll
      for (int i = 0; i < PD; i++)
#pragma unroll
        for (int x = 0; x < 2; x++)
          a[i][x] = __builtin_amdgcn_raw_buffer_load_b128(
              wr, lane16, (unsigned)(((2 * wave + x) * SD + i) * kFrag), 0);
      for (int n = 0; n < mine; n++) {
        const int pr = wave + kWaves * n;
        // The operand fragments are the same for every pair; an opaque per-pair offset keeps
        // the compiler from hoisting all their LDS reads (NR * SD fragments) out of the loop.
        int opaque = 0;
        asm volatile("" : "+s"(opaque));
        const unsigned char* X = lds + opaque;
        f32x16 acc[2][NR];
#pragma unroll
        for (int x = 0; x < 2; x++)
#pragma unroll
          for (int j = 0; j < NR; j++) acc[x][j] = mfma32_zero();
        // Fragment offsets of this pair's first block and of what follows it (x = 0, 1): the
        // next pair's two blocks, the odd block (both streams: the second is not used) after
        // the last pair, or else the last pair itself again (unconditional loads keep the ring in
        // fixed registers).
        const unsigned here = (unsigned)(2 * pr * SD * kFrag);
        const bool last = n == mine - 1;
        const unsigned next0 = !last      ? (unsigned)(2 * (pr + kWaves) * SD * kFrag)
                               : tile_odd ? (unsigned)((blocks - 1) * SD * kFrag)
                                          : here;
        const unsigned next1 = last && tile_odd ? next0 : next0 + (unsigned)(SD * kFrag);
#pragma unroll
        for (int s = 0; s < SD; s++) {
          u32x4 cur[2];
#pragma unroll
          for (int x = 0; x < 2; x++) {
            cur[x] = a[s % PD][x];
            const unsigned off = s + PD < SD ? here + (x * SD + s + PD) * kFrag
                                             : (x ? next1 : next0) + (s + PD - SD) * kFrag;
            a[s % PD][x] = __builtin_amdgcn_raw_buffer_load_b128(wr, lane16, off, 0);
          }
          // Operand reads and MFMAs of one step; the scheduling barrier keeps the compiler from
          // pulling later steps' LDS reads forward.
#pragma unroll
          for (int j = 0; j < NR; j++) {
            const u32x4 bf = *reinterpret_cast<const u32x4*>(X + (j * SD + s) * kFrag + lane16);
#pragma unroll
            for (int x = 0; x < 2; x++) acc[x][j] = mfma32(cur[x], bf, acc[x][j]);
          }
          if (s % 2 == 1) __builtin_amdgcn_sched_barrier(0);
        }
        float4 bias[2][4];
#pragma unroll
        for (int x = 0; x < 2; x++) load_bias(2 * pr + x, bias[x]);
        unsigned char* const st = stage[wave];
#pragma unroll
        for (int j = 0; j < NR; j++) {
#pragma unroll
          for (int x = 0; x < 2; x++) {
            u32x2 packed[4];
            tile_values(acc[x][j], 2 * pr + x, j, bias[x], packed);
#pragma unroll
            for (int q = 0; q < 4; q++)
              *reinterpret_cast<u32x2*>(st + col * 128 + (((4 * x + q) ^ ((col >> 1) & 7)) << 4) +
                                        8 * (half ^ (col >> 4))) = packed[q];
          }
          // Rows 8 k + l / 8 of the tile, 16-byte chunk l % 8: whole 128-byte lines. Rows 16-31
          // (k = 2, 3) hold their chunks' 8-byte halves swapped.
#pragma unroll
          for (int k = 0; k < 4; k++) {
            const int rr = 8 * k + (lane >> 3);
            u32x4 w = *reinterpret_cast<const u32x4*>(
                st + rr * 128 + (((lane & 7) ^ ((rr >> 1) & 7)) << 4));
            if (k >= 2) w = u32x4{w[2], w[3], w[0], w[1]};
            __builtin_amdgcn_raw_buffer_store_b128(
                w, outr, ((unsigned)(32 * j + rr) * p.cols + 8 * (lane & 7)) * 2,
                (unsigned)(64 * pr) * 2, kStream);
          }
        }
      }
    }
    if (tile_odd) {
      // The last block: row tile `wave` of it (one MFMA per k step), its first PD steps already
      // in the ring when the wave had pairs.
      const int b = blocks - 1, j = wave;
      f32x16 acc = mfma32_zero();
      if (mine == 0) {
#pragma unroll
        for (int i = 0; i < PD; i++)
          a[i][0] = __builtin_amdgcn_raw_buffer_load_b128(wr, lane16,
                                                          (unsigned)((b * SD + i) * kFrag), 0);
      }
      float4 bias[4];
      load_bias(b, bias);
#pragma unroll
      for (int s = 0; s < SD; s++) {
        const u32x4 cur = a[s % PD][0];
        if (s + PD < SD)
          a[s % PD][0] = __builtin_amdgcn_raw_buffer_load_b128(
              wr, lane16, (unsigned)((b * SD + s + PD) * kFrag), 0);
        const u32x4 bf = *reinterpret_cast<const u32x4*>(lds + (j * SD + s) * kFrag + lane16);
        acc = mfma32(cur, bf, acc);
      }
      u32x2 packed[4];
      tile_values(acc, b, j, bias, packed);
      // Lanes l and l + 32 trade halves (v_permlane32_swap) so each holds 8 consecutive columns
      // of its row: one 16-byte store per lane covers 16 columns of 32 rows.
      const int r = 32 * j + col;
#pragma unroll
      for (int qq = 0; qq < 4; qq += 2) {
        // Low lanes: own columns 8(qq+1) .. +3 and the partner's 8(qq+1) + 4 .. +7; high lanes:
        // the partner's 8 qq .. +3 and own 8 qq + 4 .. +7.
        u32x4 w;
#pragma unroll
        for (int d = 0; d < 2; d++) {
          const auto sw = __builtin_amdgcn_permlane32_swap(packed[qq + 1][d], packed[qq][d],
                                                           false, false);
          const unsigned lo = sw[0], hi = sw[1];
          w[d] = lo;
          w[2 + d] = hi;
        }
        __builtin_amdgcn_raw_buffer_store_b128(
            w, outr, ((unsigned)r * p.cols + 8 * (1 - half)) * 2, (unsigned)(32 * b + 8 * qq) * 2,
            0);
      }
    }
    __syncthreads();  // the next row block rewrites LDS
  }
}

template <int SD, int NR = 4, bool TANH = false>
hipError_t launch_t(const QkvParams& p, hipStream_t stream) {
  const int cus = device_cus();
  const int blocks = (p.rows + 32 * NR - 1) / (32 * NR) * (TANH ? p.batch : 1);
  const int grid = blocks < cus ? blocks : cus;
  hipLaunchKernelGGL((qkv_kernel<SD, NR, TANH>), dim3(grid), dim3(kWaves * 64), 0, stream, p);
  return hipGetLastError();
}

}  // namespace

bool qkv_supported(int dim, int cols) {
  return (dim == 128 || dim == 256 || dim == 384 || dim == 512) && cols > 0 && cols % 32 == 0;
}

hipError_t launch_qkv(const QkvParams& p, hipStream_t stream) {
  // The query scaling rides on the rotary epilogue: a table is required (the block always
  // passes one; without it the query columns would come out unscaled).
  if (!qkv_supported(p.dim, p.cols) || !p.rope || p.tokens <= 0 || p.token_div <= 0 ||
      p.width <= 0 || p.width % 64 != 0 || 3 * p.width + p.width / 64 > p.cols)
    return hipErrorInvalidValue;
  if (p.rows <= 0) return hipSuccess;
  switch (p.dim) {
    case 128: return launch_t<8>(p, stream);
    case 256: return launch_t<16>(p, stream);
    case 384: return launch_t<24>(p, stream);
    default: return launch_t<32, 3>(p, stream);
  }
}

bool mask_hidden_supported(int dim, int cols) {
  return (dim == 384 || dim == 512) && cols > 0 && cols % 64 == 0;
}

hipError_t launch_mask_hidden(const QkvParams& p, hipStream_t stream) {
  if (!mask_hidden_supported(p.dim, p.cols) || p.batch <= 0 || !p.bias)
    return hipErrorInvalidValue;
  if (p.rows <= 0) return hipSuccess;
  return p.dim == 384 ? launch_t<24, 4, true>(p, stream) : launch_t<32, 3, true>(p, stream);
}

}  // namespace ancha
