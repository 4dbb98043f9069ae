// Fused attention over long sequences (the time axis, T > 64: 801 frames for Mel-RoFormer,
// 1101 for BS-RoFormer) on v_mfma_f32_32x32x16_f16. Same operation and boundary as
// attention.hip (crates/ancha-models/src/fused/attention.rs:26-227): softmax(q.k^T).v per
// (group, head), optional interleaved RoPE on load, optional per-head sigmoid gate.
//
// One workgroup = 16 waves x 32 queries of one (group, head); each 64-key tile is staged once
// into LDS as fp16 (K rotated on the way) and read by all 16 waves. The kernel is bound by the
// VALU work of the softmax (exp2, max, fp16 packing: about as many cycles as the MFMAs), so it
// is built for overlap: at most 128 VGPRs, which puts four waves on every SIMD, one wave's
// softmax running beside another's MFMAs.
//
// Per 32-key block a wave computes S^T = K.Q^T (4 MFMAs over head_dim 64) with the accumulator
// seeded with -m, so the scores come out already shifted by the running maximum; each lane then
// holds one query (l % 32) and 16 keys (8i + 4(l/32) + e), exactly the lane's B operand of
// O^T = V^T.P^T once packed to fp16, when V^T's keys are taken in kPerm16 order within each
// 16-key step. The row maximum is a per-lane max3 chain plus one permlane32 swap, taken only
// when some score of the block exceeds the running maximum by kTau (a lazy rescale); row sums
// are v_dot2 of the packed probabilities against (1, 1), so numerator and denominator see the
// same fp16 values.
#include <type_traits>

#include "attention.hpp"

namespace ancha {
namespace {

constexpr int kWaves = 16;
constexpr int kQueries = kWaves * 32;

// Byte offset of 16-byte chunk c (0..7) of row r in a tile of 128-byte rows (K: row = key;
// V^T: row = channel; a wave's queries: row = query). Chunks are XOR-swizzled by (r >> 1) & 7,
// so the 16 lanes that one LDS cycle serves (rows r .. r + 15 of a fragment read, two rows per
// 256-byte bank line) land on 16 different bank groups.
__device__ __forceinline__ int row_offset(int r, int c) { return r * 128 + ((c ^ ((r >> 1) & 7)) << 4); }

// Position of key k (0..63) in a V^T row: bits 2 and 3 swapped, so each 16-key step holds keys
// 0-3, 8-11, 4-7, 12-15 (kPerm16 order) and a lane's 8 keys are one contiguous 16-byte chunk.
__device__ __forceinline__ int v_position(int k) {
  return (k & 0x33) | ((k & 4) << 1) | ((k & 8) >> 1);
}

// Byte offset of the dword holding positions pos, pos + 1 (pos even) of V^T row ch.
__device__ __forceinline__ int v_offset(int ch, int pos) {
  return row_offset(ch, pos >> 3) + (pos & 7) * 2;
}

// The value of lane l ^ 16 (the partner in the other row of the same 32-lane half).
__device__ __forceinline__ unsigned row_partner(unsigned x, bool odd_row) {
  const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
  const unsigned a = r[0], b = r[1];
  return odd_row ? a : b;
}

// Maximum / sum of x over lanes l and l ^ 32 (the two lanes holding one query).
__device__ __forceinline__ float pair_max(float x) {
  const unsigned xb = __builtin_bit_cast(unsigned, x);
  const auto r = __builtin_amdgcn_permlane32_swap(xb, xb, false, false);
  const unsigned a = r[0], b = r[1];
  return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}

__device__ __forceinline__ float pair_sum(float x) {
  const unsigned xb = __builtin_bit_cast(unsigned, x);
  const auto r = __builtin_amdgcn_permlane32_swap(xb, xb, false, false);
  const unsigned a = r[0], b = r[1];
  return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}

// acc + the two fp16 halves of h.
__device__ __forceinline__ float add_halves(unsigned h, float acc) {
  const h16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(h16x2, h), one, acc, false);
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4v __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));

// A 16-register accumulator holding x everywhere: eight 64-bit moves, each an asm result, so
// the tuple is a value of its own on every call (never a copy kept from an earlier block). The
// MFMA it seeds is then tied to these registers, and its destination cannot overlap its A / B
// operands.
__device__ __forceinline__ f32x16 seed16(float x) {
  const f32x2 pair = {x, x};
  f32x2 a[8];
#pragma unroll
  for (int i = 0; i < 8; i++) asm volatile("v_mov_b64 %0, %1" : "=v"(a[i]) : "v"(pair));
  const f32x4v b[4] = {__builtin_shufflevector(a[0], a[1], 0, 1, 2, 3),
                       __builtin_shufflevector(a[2], a[3], 0, 1, 2, 3),
                       __builtin_shufflevector(a[4], a[5], 0, 1, 2, 3),
                       __builtin_shufflevector(a[6], a[7], 0, 1, 2, 3)};
  const f32x8 c0 = __builtin_shufflevector(b[0], b[1], 0, 1, 2, 3, 4, 5, 6, 7);
  const f32x8 c1 = __builtin_shufflevector(b[2], b[3], 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_shufflevector(c0, c1, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15);
}

__device__ __forceinline__ u32x4 lds16(const unsigned char* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

template <bool GATED, bool ROPE, bool XH>
__global__ __launch_bounds__(kWaves * 64, 1) void attention_long_kernel(AttnParams p,
                                                                        int qblocks, int total) {
  // K tile: row = key (128 bytes of fp16 channels); V^T tile: row = channel (64 keys in
  // v_position order). Double buffered.
  __shared__ __attribute__((aligned(16))) unsigned char lds_k[2][64 * 128];
  __shared__ __attribute__((aligned(16))) unsigned char lds_v[2][64 * 128];
  // Each wave's 32 queries (fp16 rows), staged once.
  __shared__ __attribute__((aligned(16))) unsigned char lds_q[kWaves][32 * 128];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, col = lane & 31;
  const int logical = xcd_remap(blockIdx.x, total);
  const int qblk = logical % qblocks, gh = logical / qblocks;
  const int h = gh % p.heads, g = gh / p.heads;
  const int T = p.tokens;
  const long row0 = group_row(p, g), ts = p.tstep;
  constexpr unsigned kEsz = XH ? 2 : 4, kRowBytes = 64 * kEsz;
  const unsigned ldq4 = (unsigned)(ts * p.ldq * kEsz), ldk4 = (unsigned)(ts * p.ldk * kEsz),
                 ldv4 = (unsigned)(ts * p.ldv * kEsz);
  const unsigned char* kbase =
      reinterpret_cast<const unsigned char*>(p.k) + (row0 * p.ldk + h * 64) * kEsz;
  const unsigned char* vbase =
      reinterpret_cast<const unsigned char*>(p.v) + (row0 * p.ldv + h * 64) * kEsz;
  const int q0 = qblk * kQueries + wave * 32;
  const bool active = q0 < T;

  // Staging: thread -> key skey of the tile, channels 4 sc .. 4 sc + 3 of K and V (16 threads
  // read one 256-byte fp32 row). Lanes l and l ^ 16 hold keys 2i and 2i + 1: V^T dwords pair
  // them, so each lane writes two channels of its key pair (even key: 4 sc, 4 sc + 1; odd key:
  // 4 sc + 2, 4 sc + 3) after trading halves with its partner.
  const int skey = tid >> 4, sc = tid & 15;
  const bool odd = (skey & 1) != 0;
  const int vch = 4 * sc + 2 * (int)odd, vpos = v_position(skey & ~1);
  float4 kx = {}, kc = {}, ks = {}, vx = {};
  u32x2 kh = {}, vh = {};
  auto load_tile = [&](int key0) {
    const unsigned rows = (unsigned)(T - key0);
    const rsrc_t kr = make_rsrc(kbase + (long)key0 * ldk4, (rows - 1) * ldk4 + kRowBytes);
    const rsrc_t vr = make_rsrc(vbase + (long)key0 * ldv4, (rows - 1) * ldv4 + kRowBytes);
    if constexpr (XH) {
      kh = __builtin_amdgcn_raw_buffer_load_b64(kr, (unsigned)skey * ldk4 + sc * 8, 0, 0);
      vh = __builtin_amdgcn_raw_buffer_load_b64(vr, (unsigned)skey * ldv4 + sc * 8, 0, 0);
    } else {
      kx = bload4<true>(kr, (unsigned)skey * ldk4 + sc * 16);
      vx = bload4<true>(vr, (unsigned)skey * ldv4 + sc * 16);
      if constexpr (ROPE) {
        // Key cos rows (table 2) and sign-folded sin rows (table 3) of this tile.
        const rsrc_t cr = make_rsrc(p.rope + (long)(2 * T + key0) * 64, rows * 256);
        const rsrc_t sr = make_rsrc(p.rope + (long)(3 * T + key0) * 64, rows * 256);
        kc = bload4<true>(cr, (unsigned)skey * 256 + sc * 16);
        ks = bload4<true>(sr, (unsigned)skey * 256 + sc * 16);
      }
    }
  };
  auto store_tile = [&](int buf) {
    u32x2 kw = kh, vw = vh;
    if constexpr (!XH) {
      float4 x = kx;
      if constexpr (ROPE) x = rotate4(x, kc, ks);
      kw = u32x2{pack_h2(x.x, x.y), pack_h2(x.z, x.w)};
      vw = u32x2{pack_h2(vx.x, vx.y), pack_h2(vx.z, vx.w)};
    }
    *reinterpret_cast<u32x2*>(lds_k[buf] + row_offset(skey, sc >> 1) + ((sc & 1) << 3)) = kw;
    // Even key: (mine, partner's) of channels 4 sc, 4 sc + 1 (the partner sends its first
    // dword); odd key: (partner's, mine) of 4 sc + 2, 4 sc + 3 (the partner sends its second).
    const unsigned other = row_partner(odd ? vw[0] : vw[1], odd);
    const unsigned lo = odd ? other : vw[0], hi = odd ? vw[1] : other;
    unsigned char* V = lds_v[buf];
    *reinterpret_cast<unsigned*>(V + v_offset(vch, vpos)) =
        __builtin_amdgcn_perm(hi, lo, 0x05040100u);
    *reinterpret_cast<unsigned*>(V + v_offset(vch + 1, vpos)) =
        __builtin_amdgcn_perm(hi, lo, 0x07060302u);
  };

  // This wave's queries as B fragments of S^T = K.Q^T: fragment ds = query q0 + (l % 32),
  // channels 16 ds + 8 (l / 32) .. + 7, rotated, times log2(e) (fp32 inputs), fp16. Rows are
  // read whole (16 lanes per 256-byte fp32 row, 8 per 128-byte fp16 row) into the wave's LDS
  // rows and read back in fragment order.
  u32x4 qf[4];
  if (active) {
    unsigned char* Q = lds_q[wave];
    const unsigned rows = (unsigned)(T - q0);
    const rsrc_t qr = make_rsrc(reinterpret_cast<const unsigned char*>(p.q) +
                                    ((row0 + (long)q0 * ts) * p.ldq + h * 64) * kEsz,
                                (rows - 1) * ldq4 + kRowBytes);
    if constexpr (XH) {
#pragma unroll
      for (int it = 0; it < 4; it++) {
        const int r = (lane >> 3) + 8 * it, c = lane & 7;
        *reinterpret_cast<u32x4*>(Q + row_offset(r, c)) =
            __builtin_amdgcn_raw_buffer_load_b128(qr, (unsigned)r * ldq4 + c * 16, 0, 0);
      }
    } else {
      const rsrc_t cr = make_rsrc(ROPE ? p.rope + (long)q0 * 64 : p.q, ROPE ? rows * 256 : 0);
      const rsrc_t sr =
          make_rsrc(ROPE ? p.rope + (long)(T + q0) * 64 : p.q, ROPE ? rows * 256 : 0);
#pragma unroll
      for (int it = 0; it < 8; it++) {
        const int r = (lane >> 4) + 4 * it, c = lane & 15;
        float4 x = bload4<true>(qr, (unsigned)r * ldq4 + c * 16);
        if constexpr (ROPE)
          x = rotate4(x, bload4<true>(cr, (unsigned)r * 256 + c * 16),
                      bload4<true>(sr, (unsigned)r * 256 + c * 16));
        x = scale4(x, kLog2e);
        *reinterpret_cast<u32x2*>(Q + row_offset(r, c >> 1) + ((c & 1) << 3)) =
            u32x2{pack_h2(x.x, x.y), pack_h2(x.z, x.w)};
      }
    }
    // LDS operations of one wave complete in order: the reads see the rows just written.
#pragma unroll
    for (int ds = 0; ds < 4; ds++) qf[ds] = lds16(Q + row_offset(col, 2 * ds + half));
  }

  const int ntiles = (T + 63) / 64;
  load_tile(0);
  store_tile(0);
  __builtin_amdgcn_s_waitcnt(kWaitVmem);
  __syncthreads();

  // Per-lane LDS offsets: K fragment (kb, ds) = keys 32 kb + (l % 32), chunk 2 ds + l / 32;
  // V^T fragment (db, kb, k2) = channel 32 db + (l % 32), chunk 4 kb + 2 k2 + l / 32.
  // Both are chunk 2 i + l / 32 of row l % 32 (i = ds, or 2 kb + k2), plus 4096 per 32 rows.
  int fq[4];
#pragma unroll
  for (int i = 0; i < 4; i++) fq[i] = row_offset(col, 2 * i + half);

  f32x16 o[2];  // O^T: channel 32 db + 8 i + 4 (l / 32) + e of query l % 32 in o[db][4 i + e]
  o[0] = mfma32_zero();
  o[1] = mfma32_zero();
  float negm = 0.f, lsum = 0.f;  // -(running maximum), this lane's share of the row sum
  if (active) {
    // The running maximum starts at the exact maximum over the first 32 keys (T > 64).
    f32x16 s = mfma32_zero();
#pragma unroll
    for (int ds = 0; ds < 4; ds++) s = mfma32(lds16(lds_k[0] + fq[ds]), qf[ds], s);
    float mx = fmaxf(fmaxf(s[0], s[1]), s[2]);
#pragma unroll
    for (int r = 3; r < 15; r += 2) mx = fmaxf(fmaxf(mx, s[r]), s[r + 1]);
    negm = -pair_max(fmaxf(mx, s[15]));
  }

  // One 32-key block kb of the tile in buffer buf. MASK: keys at or past T may be present.
  auto block = [&](auto mask_tag, int buf, int kb, int key0) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const unsigned char* K = lds_k[buf] + kb * 4096;
    u32x4 kf[4];
#pragma unroll
    for (int ds = 0; ds < 4; ds++) kf[ds] = lds16(K + fq[ds]);
    f32x16 s = seed16(negm);
#pragma unroll
    for (int ds = 0; ds < 4; ds++) s = mfma32(kf[ds], qf[ds], s);
    // All four K reads in flight before the first MFMA waits on one.
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    if constexpr (MASK) {
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int e = 0; e < 4; e++)
          if (key0 + 32 * kb + 8 * i + 4 * half + e >= T) s[4 * i + e] = kMasked;
    }
    float lm = fmaxf(fmaxf(s[0], s[1]), s[2]);
#pragma unroll
    for (int r = 3; r < 15; r += 2) lm = fmaxf(fmaxf(lm, s[r]), s[r + 1]);
    lm = fmaxf(lm, s[15]);
    if (__builtin_amdgcn_uicmp(lm > kTau, 0, 33)) {
      const float cm = pair_max(lm);
      if (cm > kTau) {
        const float alpha = fast_exp2(-cm);
        negm -= cm;
        s -= cm;
        o[0] *= alpha;
        o[1] *= alpha;
        lsum *= alpha;
      }
    }
#pragma unroll
    for (int r = 0; r < 16; r++) s[r] = fast_exp2(s[r]);
    u32x4 pf[2];
#pragma unroll
    for (int k2 = 0; k2 < 2; k2++) {
      pf[k2] = u32x4{pack_h2(s[8 * k2], s[8 * k2 + 1]), pack_h2(s[8 * k2 + 2], s[8 * k2 + 3]),
                     pack_h2(s[8 * k2 + 4], s[8 * k2 + 5]), pack_h2(s[8 * k2 + 6], s[8 * k2 + 7])};
#pragma unroll
      for (int d = 0; d < 4; d++) lsum = add_halves(pf[k2][d], lsum);
    }
    const unsigned char* V = lds_v[buf];
#pragma unroll
    for (int k2 = 0; k2 < 2; k2++)
#pragma unroll
      for (int db = 0; db < 2; db++)
        o[db] = mfma32(lds16(V + db * 4096 + fq[2 * kb + k2]), pf[k2], o[db]);
  };

  for (int j = 0; j + 1 < ntiles; j++) {
    load_tile((j + 1) * 64);
    if (active) {
      block(std::false_type{}, j & 1, 0, j * 64);
      block(std::false_type{}, j & 1, 1, j * 64);
    }
    store_tile((j + 1) & 1);
    __builtin_amdgcn_s_waitcnt(kWaitVmem);
    __syncthreads();
  }
  if (!active) return;
  {
    const int j = ntiles - 1;
    if (T % 64) {
      block(std::true_type{}, j & 1, 0, j * 64);
      if (T - j * 64 > 32) block(std::true_type{}, j & 1, 1, j * 64);
    } else {
      block(std::false_type{}, j & 1, 0, j * 64);
      block(std::false_type{}, j & 1, 1, j * 64);
    }
  }

  // Epilogue: 1/l (and the gate), then this lane's channels 32 db + 8 i + 4 (l / 32) .. + 3 of
  // query q0 + (l % 32). Rows at or past T are dropped by the range check.
  const OutRows out = out_rows(p, g, h);
  const int t = q0 + col;
  float scale = 1.0f / pair_sum(lsum);
  if constexpr (GATED) {
    const float gl =
        out.gate_half
            ? (float)__builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(
                                                      out.gate, (unsigned)t * out.ldg4, 0, 0))
            : bload1(out.gate, (unsigned)t * out.ldg4);
    scale = scale / (1.0f + expf(-gl));
  }
#pragma unroll
  for (int db = 0; db < 2; db++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const unsigned c = (unsigned)(32 * db + 8 * i + 4 * half);
      const float4 v = make_float4(o[db][4 * i] * scale, o[db][4 * i + 1] * scale,
                                   o[db][4 * i + 2] * scale, o[db][4 * i + 3] * scale);
      if (out.half)
        __builtin_amdgcn_raw_buffer_store_b64(u32x2{pack_h2(v.x, v.y), pack_h2(v.z, v.w)},
                                              out.out, (unsigned)t * out.ld4 + c * 2, 0, 0);
      else
        bstore4<true>(out.out, (unsigned)t * out.ld4 + c * 4, v);
    }
}

template <bool GATED, bool ROPE, bool XH>
hipError_t launch_t(const AttnParams& p, hipStream_t stream) {
  const int qblocks = (p.tokens + kQueries - 1) / kQueries;
  const int total = p.groups * p.heads * qblocks;
  hipLaunchKernelGGL((attention_long_kernel<GATED, ROPE, XH>), dim3(total), dim3(kWaves * 64), 0,
                     stream, p, qblocks, total);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_attention_long(const AttnParams& p, bool gated, bool rope, hipStream_t stream) {
  if (p.tokens <= 64) return hipErrorInvalidValue;
  if (p.in_half) {
    if (!gated || rope) return hipErrorInvalidValue;
    return launch_t<true, false, true>(p, stream);
  }
  if (gated) return rope ? launch_t<true, true, false>(p, stream) : launch_t<true, false, false>(p, stream);
  return rope ? launch_t<false, true, false>(p, stream) : launch_t<false, false, false>(p, stream);
}

}  // namespace ancha
