// Fused tail of the RoFormer block on gfx950: everything after the attention core, 64 rows at
// a time, with the feed-forward hidden activation kept on chip (crates/ancha-models/src/
// roformer.rs:487-519, Transformer::forward_kernels after its gated_attention call):
//   x1 = x + attended . W_out                          out projection + residual
//   h  = fp16(GELU(fp16(unit_norm(x1)) . W1' + b1))    FF in (sqrt(dim)*gamma folded into W1')
//   y  = x1 + h . W2 + b2                              FF out + bias + residual
//   [y = unit_norm(y) * scale]                          output norm (Mel-RoFormer blocks)
//   [xh = fp16(unit_norm(y))]                           the next block's operand
// The rounding points are those of the unfused path (block.hip): fp16 normalised operand, fp16
// hidden activation, fp32 accumulation and fp32 residual stream.
//
// MFMA v_mfma_f32_32x32x16_f16 computes D[feature][row] = W^T . act^T: A fragments (32 output
// features x 16 k) come from the weights, stored at block load in a fragment-major layout (one
// 1 KB fragment per (32-feature block, 16-k step), lane-ordered, so a wave's A load is one
// contiguous kilobyte); B fragments (16 k x 32 rows) come from LDS in the same fragment-major
// order. Lane l holds D rows (features) 8q + 4(l/32) + e (q, e < 4) of row l % 32. A lane's 8
// values of one 16-feature step are thus features {4h..4h+3, 8+4h..8+4h+3} (h = l/32): written
// as fp16 they are directly lane l's B fragment of the next product if the next product's
// weights take their k (= feature) axis in that order, i.e. permuted within each 16-block by
// kPerm16 at load time. So x1 -> unit_norm -> fp16 and h -> fp16 go from accumulators to B
// fragments in LDS with one 16-byte store per lane and no shuffles.
//
// Workgroup: 64 rows, 4 waves, one per feature quarter (and SIMD); two workgroups per CU, whose
// phases drift apart, so one's GELU / norm VALU work runs beside the other's MFMAs. The out
// accumulator (64 rows x dim) stays in registers from the residual load to the final store; the
// hidden dimension runs in chunks of 256 units up to dim 384, 128 at dim 512 (per chunk: FF-in
// for 64 or 32 hidden units per wave, GELU, the chunk's fp16 activation to LDS, then its FF-out
// contribution).
#include "buffer.hpp"
#include "common.hpp"
#include "gemm.hpp"
#include "kernels.hpp"

namespace ancha {
namespace {


constexpr int kRows = 64;         // rows per workgroup step
constexpr int kChunk = 128;       // hidden units of one 32-unit block per wave (4 waves)
constexpr int kWaves = 4;         // one per feature quarter (and per SIMD)
constexpr int kFrag = 1024;       // bytes of one 32 x 16 fp16 fragment
// B fragments are read from LDS this many k steps ahead of their MFMAs (a scheduling barrier
// per step keeps the reads there), so an MFMA never waits on a read issued just before it.
constexpr int kBD = 2;

// Lane l's B fragment (8 halves) from accumulator values 8 sub .. 8 sub + 7 (q = 2 sub, 2 sub + 1).
__device__ __forceinline__ u32x4 pack_frag(const f32x16& d, int sub, float s) {
  const int o = 8 * sub;
  return u32x4{pack_h2(d[o] * s, d[o + 1] * s), pack_h2(d[o + 2] * s, d[o + 3] * s),
               pack_h2(d[o + 4] * s, d[o + 5] * s), pack_h2(d[o + 6] * s, d[o + 7] * s)};
}

// Sum over the 4 feature-quarter waves of per-row partials (red: [4][128] floats in LDS).
// Every wave calls it; it ends with the totals of this lane's rows in tot[].
template <int NJ>
__device__ __forceinline__ void row_totals(float* red, const float (&part)[NJ], float (&tot)[NJ],
                                           int fq, int rh, int lane) {
  if (lane < 32)
#pragma unroll
    for (int j = 0; j < NJ; j++) red[fq * kRows + 32 * (2 * rh + j) + lane] = part[j];
  __syncthreads();
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    const int row = 32 * (2 * rh + j) + (lane & 31);
    tot[j] = red[row] + red[kRows + row] + red[2 * kRows + row] + red[3 * kRows + row];
  }
  __syncthreads();
}

// DIM = 128 * NI features, INNER = heads * 64.
template <int NI, int INNER>
__global__ __launch_bounds__(kWaves * 64, 2) void block_tail_kernel(TailParams p) {
  constexpr int DIM = 128 * NI;
  constexpr int S0 = INNER / 16;   // k steps of the out projection
  constexpr int SD = DIM / 16;     // k steps of FF in
  constexpr int kX = kRows * DIM * 2;                                   // xh1 fragments
  // Hidden blocks of 32 units per wave and chunk: two where the chunk's activation (32 KB) still
  // leaves two workgroups a CU (dim <= 384), so each X fragment feeds two MFMAs of FF in.
  constexpr int NB = NI <= 3 ? 2 : 1;
  constexpr int kCH = kChunk * NB;  // hidden units per chunk
  constexpr int kSC = kCH / 16;     // k steps of FF out per chunk
  constexpr int kLds = (kRows * INNER * 2 > kX + kRows * kCH * 2) ? kRows * INNER * 2
                                                                   : kX + kRows * kCH * 2;
  static_assert(kLds <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(16))) unsigned char lds[kLds];
  unsigned char* const X = lds;         // xh1: fragment (jb, s) at (jb * SD + s) * 1 KB
  unsigned char* const H = lds + kX;    // hidden chunk: fragment (jb, s) at (jb * kSC + s) * 1 KB
  float* const red = reinterpret_cast<float*>(H);  // [4][128] row partials (aliases H)

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  constexpr int rh = 0;  // the workgroup's 64 rows are one pair of 32-row blocks
  const int fq = wave;
  const int half = lane >> 5, col = lane & 31;
  const int hidden = p.hidden;
  const unsigned lane16 = (unsigned)lane * 16;

  const rsrc_t wo = make_rsrc(p.wo, (unsigned)(DIM * INNER * 2));
  const rsrc_t w1 = make_rsrc(p.w1, (unsigned)(hidden * DIM * 2));
  const rsrc_t w2 = make_rsrc(p.w2, (unsigned)(DIM * hidden * 2));
  const rsrc_t b1r = make_rsrc(p.b1, (unsigned)(hidden * 4));
  const rsrc_t b2r = make_rsrc(p.b2, (unsigned)(DIM * 4));
  const rsrc_t scr = make_rsrc(p.out_scale ? p.out_scale : p.b2, (unsigned)(DIM * 4));

  for (int blk = blockIdx.x; blk * kRows < p.rows; blk += gridDim.x) {
    const int row0 = blk * kRows;
    const int nrows = min(kRows, p.rows - row0);
    const rsrc_t att = make_rsrc(p.attended + (long)row0 * INNER, (unsigned)(nrows * INNER * 2));
    const rsrc_t xr = make_rsrc(p.x + (long)row0 * DIM, (unsigned)(nrows * DIM * 4));
    const rsrc_t outr = make_rsrc(p.out + (long)row0 * DIM, (unsigned)(nrows * DIM * 4));
    const rsrc_t xhr = make_rsrc(p.xh ? p.xh + (long)row0 * DIM : p.attended,
                                 p.xh ? (unsigned)(nrows * DIM * 2) : 0u);

    // ---- the attended tile, straight into LDS as B fragments: fragment f = (jb, s) holds
    // rows 32 jb + (l % 32), k 16 s + 8 (l / 32) .. + 7 in lane order.
    for (int f = wave; f < 2 * S0; f += kWaves) {
      const int jb = f / S0, s = f % S0;
      const unsigned off = ((unsigned)(32 * jb + col) * INNER + 16 * s + 8 * half) * 2;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          att, (__attribute__((address_space(3))) void*)(lds + f * kFrag), 16, off, 0, 0, 0);
    }
    // ---- out accumulator = the residual x: lane holds row 32 (2 rh + j) + col, features
    // fb + 8 q + 4 h .. + 3 (fb = 32 (fq NI + i)).
    f32x16 acc[NI][2];
#pragma unroll
    for (int i = 0; i < NI; i++)
#pragma unroll
      for (int j = 0; j < 2; j++)
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const float4 v = __builtin_bit_cast(
              float4, __builtin_amdgcn_raw_buffer_load_b128(
                          xr, ((unsigned)(32 * (2 * rh + j) + col) * DIM + 4 * half) * 4,
                          (unsigned)(32 * (fq * NI + i) + 8 * q) * 4, 0));
          acc[i][j][4 * q] = v.x;
          acc[i][j][4 * q + 1] = v.y;
          acc[i][j][4 * q + 2] = v.z;
          acc[i][j][4 * q + 3] = v.w;
        }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    // ---- out projection: acc += W_out^T . attended^T over INNER (S0 steps of 16).
    {
      constexpr int PD = NI > 3 ? 2 : 4;  // weight fragments prefetched this many steps ahead
      u32x4 a[PD][NI];
      auto load_a = [&](int s, u32x4 (&dst)[NI]) {
#pragma unroll
        for (int i = 0; i < NI; i++)
          dst[i] = __builtin_amdgcn_raw_buffer_load_b128(
              wo, lane16, (unsigned)(((fq * NI + i) * S0 + s) * kFrag), 0);
      };
#pragma unroll
      for (int s = 0; s < PD; s++) load_a(s, a[s]);
      u32x4 b[kBD + 1][2];
      auto load_b = [&](int s, u32x4 (&dst)[2]) {
#pragma unroll
        for (int j = 0; j < 2; j++)
          dst[j] = *reinterpret_cast<const u32x4*>(lds + ((2 * rh + j) * S0 + s) * kFrag + lane16);
      };
#pragma unroll
      for (int s = 0; s < kBD; s++) load_b(s, b[s]);
#pragma unroll
      for (int s = 0; s < S0; s++) {
        u32x4 cur[NI];
#pragma unroll
        for (int i = 0; i < NI; i++) cur[i] = a[s % PD][i];
        if (s + PD < S0) load_a(s + PD, a[s % PD]);
        if (s + kBD < S0) load_b(s + kBD, b[(s + kBD) % (kBD + 1)]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < NI; i++)
#pragma unroll
          for (int j = 0; j < 2; j++) acc[i][j] = mfma32(cur[i], b[s % (kBD + 1)][j], acc[i][j]);
      }
    }
    __syncthreads();  // the attended tile is dead: X / H may be written

    // ---- xh1 = fp16(x1 / max(||x1||, 1e-12)) into X as FF-in B fragments.
    {
      float part[2], tot[2];
#pragma unroll
      for (int j = 0; j < 2; j++) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < NI; i++)
#pragma unroll
          for (int r = 0; r < 16; r++) s += acc[i][j][r] * acc[i][j][r];
        part[j] = s + __shfl_xor(s, 32);
      }
      row_totals<2>(red, part, tot, fq, rh, lane);
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const float inv = 1.0f / fmaxf(sqrtf(tot[j]), 1e-12f);
#pragma unroll
        for (int i = 0; i < NI; i++)
#pragma unroll
          for (int sub = 0; sub < 2; sub++) {
            const int s = 2 * (fq * NI + i) + sub;
            *reinterpret_cast<u32x4*>(X + ((2 * rh + j) * SD + s) * kFrag + lane16) =
                pack_frag(acc[i][j], sub, inv);
          }
      }
    }
    __syncthreads();

    // ---- feed-forward, NB x 128 hidden units per chunk (NB 32-unit hidden blocks per wave).
    for (int c = 0; c < hidden / kCH; c++) {
      // FF in: this wave's hidden blocks NB fq + x (x < NB) of the chunk, units kCH c +
      // 32 (NB fq + x) + (8 q + 4 h + e), the accumulators starting at b1 (issued ahead of the
      // chunk's first weight fragments, which the first MFMA waits for anyway).
      f32x16 hacc[NB][2];
#pragma unroll
      for (int x = 0; x < NB; x++)
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const float4 b = __builtin_bit_cast(
              float4, __builtin_amdgcn_raw_buffer_load_b128(
                          b1r, 16 * half, (unsigned)(kCH * c + 32 * (NB * fq + x) + 8 * q) * 4, 0));
#pragma unroll
          for (int j = 0; j < 2; j++) {
            hacc[x][j][4 * q] = b.x;
            hacc[x][j][4 * q + 1] = b.y;
            hacc[x][j][4 * q + 2] = b.z;
            hacc[x][j][4 * q + 3] = b.w;
          }
        }
      {
        constexpr int PD = NB > 1 ? 4 : 8;
        const int blk0 = (kCH / 32) * c + NB * fq;
        u32x4 a[PD][NB];
        auto load_a = [&](int s, u32x4 (&dst)[NB]) {
#pragma unroll
          for (int x = 0; x < NB; x++)
            dst[x] = __builtin_amdgcn_raw_buffer_load_b128(
                w1, lane16, (unsigned)(((blk0 + x) * SD + s) * kFrag), 0);
        };
#pragma unroll
        for (int s = 0; s < PD && s < SD; s++) load_a(s, a[s]);
        u32x4 b[kBD + 1][2];
        auto load_b = [&](int s, u32x4 (&dst)[2]) {
#pragma unroll
          for (int j = 0; j < 2; j++)
            dst[j] = *reinterpret_cast<const u32x4*>(X + ((2 * rh + j) * SD + s) * kFrag + lane16);
        };
#pragma unroll
        for (int s = 0; s < kBD; s++) load_b(s, b[s]);
#pragma unroll
        for (int s = 0; s < SD; s++) {
          u32x4 cur[NB];
#pragma unroll
          for (int x = 0; x < NB; x++) cur[x] = a[s % PD][x];
          if (s + PD < SD) load_a(s + PD, a[s % PD]);
          if (s + kBD < SD) load_b(s + kBD, b[(s + kBD) % (kBD + 1)]);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int x = 0; x < NB; x++)
#pragma unroll
            for (int j = 0; j < 2; j++)
              hacc[x][j] = mfma32(cur[x], b[s % (kBD + 1)][j], hacc[x][j]);
        }
      }
      // GELU(h + b1), fp16, into H as FF-out B fragments (hidden steps 2 (NB fq + x) + sub).
      __syncthreads();  // the previous chunk's FF-out has read H
#pragma unroll
      for (int x = 0; x < NB; x++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
          f32x16 g;
#pragma unroll
          for (int r = 0; r < 16; r++) g[r] = gemm::gelu_fast(hacc[x][j][r]);
#pragma unroll
          for (int sub = 0; sub < 2; sub++)
            *reinterpret_cast<u32x4*>(H + ((2 * rh + j) * kSC + 2 * (NB * fq + x) + sub) * kFrag +
                                      lane16) = pack_frag(g, sub, 1.0f);
        }
      __syncthreads();
      // FF out: acc += W2^T . h^T over the chunk's kCH hidden units (kSC steps of 16).
      {
        constexpr int PD = NI > 3 ? 2 : 4;
        const int sh = hidden / 16;
        u32x4 a[PD][NI];
        auto load_a = [&](int s, u32x4 (&dst)[NI]) {
#pragma unroll
          for (int i = 0; i < NI; i++)
            dst[i] = __builtin_amdgcn_raw_buffer_load_b128(
                w2, lane16, (unsigned)(((fq * NI + i) * sh + kSC * c + s) * kFrag), 0);
        };
#pragma unroll
        for (int s = 0; s < PD; s++) load_a(s, a[s]);
        u32x4 b[kBD + 1][2];
        auto load_b = [&](int s, u32x4 (&dst)[2]) {
#pragma unroll
          for (int j = 0; j < 2; j++)
            dst[j] = *reinterpret_cast<const u32x4*>(H + ((2 * rh + j) * kSC + s) * kFrag + lane16);
        };
#pragma unroll
        for (int s = 0; s < kBD; s++) load_b(s, b[s]);
#pragma unroll
        for (int s = 0; s < kSC; s++) {
          u32x4 cur[NI];
#pragma unroll
          for (int i = 0; i < NI; i++) cur[i] = a[s % PD][i];
          if (s + PD < kSC) load_a(s + PD, a[s % PD]);
          if (s + kBD < kSC) load_b(s + kBD, b[(s + kBD) % (kBD + 1)]);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int i = 0; i < NI; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) acc[i][j] = mfma32(cur[i], b[s % (kBD + 1)][j], acc[i][j]);
        }
      }
    }
    __syncthreads();  // H (the reduction buffer) is free again

    // ---- epilogue: + b2, optional output norm (and the next block's fp16 operand), stores.
#pragma unroll
    for (int i = 0; i < NI; i++)
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const float4 b = __builtin_bit_cast(
            float4, __builtin_amdgcn_raw_buffer_load_b128(
                        b2r, 16 * half, (unsigned)(32 * (fq * NI + i) + 8 * q) * 4, 0));
#pragma unroll
        for (int j = 0; j < 2; j++) {
          acc[i][j][4 * q] += b.x;
          acc[i][j][4 * q + 1] += b.y;
          acc[i][j][4 * q + 2] += b.z;
          acc[i][j][4 * q + 3] += b.w;
        }
      }
    if (p.out_scale) {
      float part[2], tot[2];
#pragma unroll
      for (int j = 0; j < 2; j++) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < NI; i++)
#pragma unroll
          for (int r = 0; r < 16; r++) s += acc[i][j][r] * acc[i][j][r];
        part[j] = s + __shfl_xor(s, 32);
      }
      row_totals<2>(red, part, tot, fq, rh, lane);
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const float inv = 1.0f / fmaxf(sqrtf(tot[j]), 1e-12f);
#pragma unroll
        for (int i = 0; i < NI; i++)
#pragma unroll
          for (int q = 0; q < 4; q++) {
            const float4 sc = __builtin_bit_cast(
                float4, __builtin_amdgcn_raw_buffer_load_b128(
                            scr, 16 * half, (unsigned)(32 * (fq * NI + i) + 8 * q) * 4, 0));
            acc[i][j][4 * q] = acc[i][j][4 * q] * inv * sc.x;
            acc[i][j][4 * q + 1] = acc[i][j][4 * q + 1] * inv * sc.y;
            acc[i][j][4 * q + 2] = acc[i][j][4 * q + 2] * inv * sc.z;
            acc[i][j][4 * q + 3] = acc[i][j][4 * q + 3] * inv * sc.w;
          }
      }
    }
    if (p.xh) {
      // The next block's fp16 operand, fp16(unit_norm(y)) (y after the output norm, if any).
      float part[2], tot[2];
#pragma unroll
      for (int j = 0; j < 2; j++) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < NI; i++)
#pragma unroll
          for (int r = 0; r < 16; r++) s += acc[i][j][r] * acc[i][j][r];
        part[j] = s + __shfl_xor(s, 32);
      }
      row_totals<2>(red, part, tot, fq, rh, lane);
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const float inv = 1.0f / fmaxf(sqrtf(tot[j]), 1e-12f);
#pragma unroll
        for (int i = 0; i < NI; i++)
#pragma unroll
          for (int q = 0; q < 4; q++) {
            const u32x2 h = {pack_h2(acc[i][j][4 * q] * inv, acc[i][j][4 * q + 1] * inv),
                             pack_h2(acc[i][j][4 * q + 2] * inv, acc[i][j][4 * q + 3] * inv)};
            __builtin_amdgcn_raw_buffer_store_b64(
                h, xhr, ((unsigned)(32 * (2 * rh + j) + col) * DIM + 4 * half) * 2,
                (unsigned)(32 * (fq * NI + i) + 8 * q) * 2, 0);
          }
      }
    }
#pragma unroll
    for (int i = 0; i < NI; i++)
#pragma unroll
      for (int j = 0; j < 2; j++)
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const float4 v = make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1],
                                       acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
          __builtin_amdgcn_raw_buffer_store_b128(
              __builtin_bit_cast(u32x4, v), outr,
              ((unsigned)(32 * (2 * rh + j) + col) * DIM + 4 * half) * 4,
              (unsigned)(32 * (fq * NI + i) + 8 * q) * 4, 0);
        }
    __syncthreads();  // LDS is rewritten by the next row block's attended tile
  }
}

template <int NI, int INNER>
hipError_t launch_t(const TailParams& p, int grid, hipStream_t stream) {
  hipLaunchKernelGGL((block_tail_kernel<NI, INNER>), dim3(grid), dim3(kWaves * 64), 0, stream, p);
  return hipGetLastError();
}

}  // namespace

bool block_tail_supported(int dim, int inner, int hidden) {
  // Chunks of 256 hidden units up to dim 384, of 128 at dim 512.
  const int chunk = dim <= 384 ? 2 * kChunk : kChunk;
  return (dim == 128 || dim == 256 || dim == 384 || dim == 512) && (inner == 128 || inner == 512) &&
         hidden > 0 && hidden % chunk == 0;
}

hipError_t launch_block_tail(const TailParams& p, hipStream_t stream) {
  if (!block_tail_supported(p.dim, p.inner, p.hidden)) return hipErrorInvalidValue;
  if (p.rows <= 0) return hipSuccess;
  const int cus = device_cus();
  const int blocks = (p.rows + kRows - 1) / kRows;
  const int grid = blocks < 2 * cus ? blocks : 2 * cus;  // two workgroups per CU
  const int ni = p.dim / 128;
  if (p.inner == 512) {
    switch (ni) {
      case 1: return launch_t<1, 512>(p, grid, stream);
      case 2: return launch_t<2, 512>(p, grid, stream);
      case 3: return launch_t<3, 512>(p, grid, stream);
      default: return launch_t<4, 512>(p, grid, stream);
    }
  }
  switch (ni) {
    case 1: return launch_t<1, 128>(p, grid, stream);
    case 2: return launch_t<2, 128>(p, grid, stream);
    case 3: return launch_t<3, 128>(p, grid, stream);
    default: return launch_t<4, 128>(p, grid, stream);
  }
}

}  // namespace ancha
