// Packed q | k | v | gate projection of the RoFormer block on gfx950 (crates/ancha-models/src/
// roformer.rs:477-485: fused::linear with the bias + rotary epilogue of fused/gemm.rs:46-82):
//   out[r][c] = epilogue(sum_k xh[r][k] W^T[c][k] + bias[c]), fp16,
// with the interleaved rotary embedding on columns [0, 2 width) (queries, then keys, of token
// (r / token_div) % tokens) and the queries also times q_scale (log2 e for the exp2 softmax).
//
// 128 rows per workgroup: their fp16 operand rows sit in LDS for the whole block as B
// fragments of v_mfma_f32_32x32x16_f16 (straight from HBM with direct-to-LDS loads), with the
// rows' rotary cos / sin (32 + 32 per row) next to them. The 8 waves walk the output in 32-column
// blocks (wave w takes blocks w, w + 8, ..., so each SIMD gets the same count); per block a wave
// accumulates all 128 rows (4 x 32-row MFMA tiles) over K, reading each weight A fragment once
// (a contiguous kilobyte of the fragment-major W^T) for four MFMAs, then rotates and stores its
// 32 x 128 tile straight from the accumulators (lane l owns row l % 32, columns 8q + 4(l/32) ..
// +3: both members of every rotary pair). No barriers inside the column walk, so the two waves
// of a SIMD drift apart and one's epilogue runs beside the other's MFMAs.
#include "buffer.hpp"
#include "common.hpp"
#include "kernels.hpp"

namespace ancha {
namespace {

constexpr int kRows = 128;
constexpr int kWaves = 8;
constexpr int kFrag = 1024;

// SD = dim / 16 k steps.
template <int SD>
__global__ __launch_bounds__(kWaves * 64, 1) void qkv_kernel(QkvParams p) {
  constexpr int kX = kRows * SD * 16 * 2;      // operand fragments
  // Per row: 16 chunks of (cos, sin) for two rotary pairs, chunk c at position c ^ (row & 15)
  // (rows 256 bytes apart would otherwise put one column's reads of 32 rows in one bank).
  constexpr int kT = kRows * 64 * 4;
  __shared__ __attribute__((aligned(16))) unsigned char lds[kX + kT];
  float* const cs = reinterpret_cast<float*>(lds + kX);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, col = lane & 31;
  const unsigned lane16 = (unsigned)lane * 16;
  const int blocks = p.cols / 32;
  const int dim = SD * 16;
  const rsrc_t wr = make_rsrc(p.w, (unsigned)(p.cols * dim * 2));
  const rsrc_t br = make_rsrc(p.bias, (unsigned)(p.cols * 4));
  const bool rot = p.rope != nullptr;
  const rsrc_t tr = make_rsrc(rot ? p.rope : p.bias, rot ? (unsigned)(4 * p.tokens * 256) : 0u);

  for (int blk = blockIdx.x; blk * kRows < p.rows; blk += gridDim.x) {
    const int row0 = blk * kRows;
    const int nrows = min(kRows, p.rows - row0);
    const rsrc_t xr = make_rsrc(p.xh + (long)row0 * dim, (unsigned)(nrows * dim * 2));
    const rsrc_t outr = make_rsrc(p.out + (long)row0 * p.cols, (unsigned)(nrows * p.cols * 2));
    // Operand rows as B fragments: fragment (jb, s) = rows 32 jb + (l % 32), k 16 s + 8 (l / 32).
    for (int f = wave; f < 4 * SD; f += kWaves) {
      const int jb = f / SD, s = f % SD;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          xr, (__attribute__((address_space(3))) void*)(lds + f * kFrag), 16,
          ((unsigned)(32 * jb + col) * dim + 16 * s + 8 * half) * 2, 0, 0, 0);
    }
    // Key-table cos / sin of each row's token (the query tables are these times 1/8).
    if (rot)
      for (int e = tid; e < kRows * 32; e += kWaves * 64) {
        const int r = e >> 5, i = e & 31;
        const int tok = ((row0 + r) / p.token_div) % p.tokens;
        float* slot = cs + r * 64 + (((i >> 1) ^ (r & 15)) << 2) + 2 * (i & 1);
        slot[0] = bload1(tr, (unsigned)((2 * p.tokens + tok) * 64 + 2 * i) * 4);
        slot[1] = bload1(tr, (unsigned)((3 * p.tokens + tok) * 64 + 2 * i + 1) * 4);
      }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    constexpr int PD = 8;  // weight fragments in flight
    static_assert(SD % PD == 0 && SD >= PD, "K steps come in groups of PD");
    u32x4 a[PD];
    // The wave's blocks b = wave + 8 n; its A fragments stream through the ring across blocks.
    const int mine = (blocks - wave + kWaves - 1) / kWaves;
#pragma unroll
    for (int i = 0; i < PD; i++)
      a[i] = __builtin_amdgcn_raw_buffer_load_b128(wr, lane16, (unsigned)((wave * SD + i) * kFrag),
                                                   0);
    for (int n = 0; n < mine; n++) {
      const int b = wave + kWaves * n;
      // The operand fragments are the same for every column block; an opaque per-block offset
      // keeps the compiler from hoisting all their LDS reads (4 * SD fragments) out of the loop.
      int opaque = 0;
      asm volatile("" : "+s"(opaque));
      const unsigned char* X = lds + opaque;
      f32x16 acc[4];
#pragma unroll
      for (int j = 0; j < 4; j++) acc[j] = mfma32_zero();
      // This block's bias columns (used after the K loop).
      float4 bias[4];
#pragma unroll
      for (int q = 0; q < 4; q++)
        bias[q] = __builtin_bit_cast(
            float4, __builtin_amdgcn_raw_buffer_load_b128(br, 16 * half,
                                                          (unsigned)(32 * b + 8 * q) * 4, 0));
      // Fragment offsets of this block and of the next one (the last block reloads itself:
      // unconditional loads keep the ring in fixed registers).
      const unsigned here = (unsigned)(b * SD * kFrag);
      const unsigned next = (unsigned)(min(b + kWaves, wave + kWaves * (mine - 1)) * SD * kFrag);
#pragma unroll
      for (int s = 0; s < SD; s++) {
        const u32x4 cur = a[s % PD];
        a[s % PD] = __builtin_amdgcn_raw_buffer_load_b128(
            wr, lane16, s + PD < SD ? here + (s + PD) * kFrag : next + (s + PD - SD) * kFrag, 0);
        // Operand reads and MFMAs of one step; the scheduling barrier keeps the compiler from
        // pulling later steps' LDS reads forward (all 4 * SD would not fit in registers).
#pragma unroll
        for (int j = 0; j < 4; j++)
          acc[j] = mfma32(cur, *reinterpret_cast<const u32x4*>(X + (j * SD + s) * kFrag + lane16),
                          acc[j]);
        if (s % 4 == 3) __builtin_amdgcn_sched_barrier(0);
      }
      // Epilogue: bias -> rotary -> query scale (fused/gemm.rs:46-82 order), fp16. Lanes l and
      // l + 32 then trade halves (v_permlane32_swap) so each holds 8 consecutive columns of its
      // row: one 16-byte store per lane covers 16 columns of 32 rows.
      u32x2 packed[4][4];  // [q][j]
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int c = 32 * b + 8 * q + 4 * half;  // this lane's 4 columns c .. c + 3
        const bool rq = rot && c < p.width, rk = rot && c >= p.width && c < 2 * p.width;
        const int pair = (c & 63) >> 1;
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int r = 32 * j + col;
          float4 v = make_float4(acc[j][4 * q] + bias[q].x, acc[j][4 * q + 1] + bias[q].y,
                                 acc[j][4 * q + 2] + bias[q].z, acc[j][4 * q + 3] + bias[q].w);
          if (rq || rk) {
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
          packed[q][j] = u32x2{pack_h2(v.x, v.y), pack_h2(v.z, v.w)};
        }
      }
#pragma unroll
      for (int qq = 0; qq < 4; qq += 2)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          // Low lanes: own columns 8(qq+1) .. +3 and the partner's 8(qq+1) + 4 .. +7; high lanes:
          // the partner's 8 qq .. +3 and own 8 qq + 4 .. +7.
          u32x4 w;
#pragma unroll
          for (int d = 0; d < 2; d++) {
            const auto sw = __builtin_amdgcn_permlane32_swap(packed[qq + 1][j][d],
                                                             packed[qq][j][d], false, false);
            const unsigned lo = sw[0], hi = sw[1];
            w[d] = lo;
            w[2 + d] = hi;
          }
          const int r = 32 * j + col;
          __builtin_amdgcn_raw_buffer_store_b128(
              w, outr, ((unsigned)r * p.cols + 8 * (1 - half)) * 2, (unsigned)(32 * b + 8 * qq) * 2,
              0);
        }
    }
    __syncthreads();  // the next row block rewrites LDS
  }
}

template <int SD>
hipError_t launch_t(const QkvParams& p, int grid, hipStream_t stream) {
  hipLaunchKernelGGL((qkv_kernel<SD>), dim3(grid), dim3(kWaves * 64), 0, stream, p);
  return hipGetLastError();
}

}  // namespace

bool qkv_supported(int dim, int cols) {
  return (dim == 128 || dim == 256 || dim == 384 || dim == 512) && cols > 0 && cols % 32 == 0;
}

hipError_t launch_qkv(const QkvParams& p, hipStream_t stream) {
  // The query scaling rides on the rotary epilogue: a table is required (the block always
  // passes one; without it the query columns would come out unscaled).
  if (!qkv_supported(p.dim, p.cols) || !p.rope || p.tokens <= 0 || p.token_div <= 0)
    return hipErrorInvalidValue;
  if (p.rows <= 0) return hipSuccess;
  const int cus = device_cus();
  const int blocks = (p.rows + kRows - 1) / kRows;
  const int grid = blocks < cus ? blocks : cus;
  switch (p.dim) {
    case 128: return launch_t<8>(p, grid, stream);
    case 256: return launch_t<16>(p, grid, stream);
    case 384: return launch_t<24>(p, grid, stream);
    default: return launch_t<32>(p, grid, stream);
  }
}

}  // namespace ancha
