// Fused RoFormer attention for CDNA4 (gfx950): softmax(q.k^T).v per (group, head) with the
// optional interleaved RoPE applied while q/k are loaded and the optional per-head sigmoid gate
// in the epilogue. Replaces the CubeCL `flash_attention` of
// crates/ancha-models/src/fused/attention.rs:26-227 (launch :250-298).
//
// Both kernels compute S^T = K.Q^T and O^T = V^T.P^T with v_mfma_f32_16x16x32_f16, so that the
// score tile produced by the first product is already, lane for lane, the B operand of the
// second: each lane owns one query column and 4+4 keys of every 32-key step. The softmax runs
// in fp32 in the log2 domain (q carries log2(e)); row maxima are two cross-lane shuffles, row
// sums come from the MFMA (a ones matrix times P^T, so numerator and denominator see the same
// fp16-rounded probabilities), and 1/l and the gate are applied once in the epilogue.
//
// All global traffic goes through raw buffer loads/stores whose hardware range check returns 0
// for rows at or past `tokens` (and drops stores there), so ragged tails need no branches.
//
//  * attention_time_kernel: long sequences whose rows are not 16-byte aligned (aligned ones,
//    every call the library itself makes, go to attention_long.hip's 32x32x16 kernel). One
//    workgroup = 8 waves x 64 queries of one (group, head); 64-key K / V^T tiles are staged in
//    LDS as fp16 (K rotated
//    on the way), double buffered, the next tile's loads in flight while the current one is
//    multiplied. The online softmax rescales lazily: the running maximum only moves when a
//    tile exceeds it by more than kTau, so most tiles skip the O / l rescale.
//  * attention_band_kernel: T <= 64 (the band axis, 60-62 bands, huge batch). One 4-wave
//    workgroup per (group, head) problem stages q, k (rotated) and v^T through LDS with
//    coalesced row loads, then each wave takes 16 queries; softmax is exact (one key tile).
#include <type_traits>

#include "attention.hpp"

namespace ancha {

// fp16 1.0 in both halves of a dword: the A operand of the row-sum MFMA.
constexpr unsigned kOnesH2 = 0x3C003C00u;

// Chunked V^T tile (time kernel): row d holds the 64 keys of channel d, and the 16-byte chunk
// ks*4 + grp holds keys ks*32 + {grp*4 + i, 16 + grp*4 + i} (i = 0..3) in that order, so one
// chunk is exactly one lane's A operand of O^T = V^T.P^T. Chunks are XOR-swizzled by
// (d ^ d >> 2) & 7, which differs across 8 consecutive rows (the operand reads) and across rows
// 4 apart (the transposing writes of the staging threads).
__device__ __forceinline__ int vtc_offset(int d, int key) {
  const int chunk = (key >> 5) * 4 + ((key & 15) >> 2);
  const int elem = (key & 3) + ((key & 16) >> 2);
  return d * 128 + ((chunk ^ ((d ^ (d >> 2)) & 7)) << 4) + elem * 2;
}

// B operand of O^T = V^T.P^T from the score tiles of key blocks 2ks and 2ks+1.
__device__ __forceinline__ u32x4 p_fragment(f32x4 a, f32x4 b) {
  return u32x4{pack_h2(a[0], a[1]), pack_h2(a[2], a[3]), pack_h2(b[0], b[1]),
               pack_h2(b[2], b[3])};
}

// Dword j (keys a, b of channel j) of a V^T chunk from the fp16 channels 4c .. 4c+3 of two keys.
__device__ __forceinline__ unsigned v_pair(u32x2 a, u32x2 b, int j) {
  return __builtin_amdgcn_perm(b[j >> 1], a[j >> 1], (j & 1) ? 0x07060302u : 0x05040100u);
}

// 1/l and sigmoid(gate) scaling and store of one lane's 16 channels (grp*4 + 16*db) of query t.
// HALF: 1 = fp16 gate and output, 0 = fp32 gate and output, -1 = as o.gate_half / o.half say
// (a branch the compiler's wait counting cannot see through).
template <bool GATED, bool ALIGNED, int CP = 0, int HALF = -1>
__device__ __forceinline__ void store_output(const OutRows& o, const f32x4 (&acc)[4], float l,
                                             int t, int grp) {
  float scale = 1.0f / l;
  const bool gate_half = HALF < 0 ? o.gate_half : HALF > 0;
  const bool out_half = HALF < 0 ? o.half : HALF > 0;
  if constexpr (GATED) {
    const float gl =
        gate_half ? (float)__builtin_bit_cast(
                          _Float16, __builtin_amdgcn_raw_buffer_load_b16(o.gate, (unsigned)t * o.ldg4, 0, 0))
                    : bload1(o.gate, (unsigned)t * o.ldg4);
    scale = scale / (1.0f + expf(-gl));
  }
  if (out_half) {
    const unsigned base = (unsigned)t * o.ld4 + grp * 8;
#pragma unroll
    for (int db = 0; db < 4; db++) {
      const u32x2 h = {pack_h2(acc[db][0] * scale, acc[db][1] * scale),
                       pack_h2(acc[db][2] * scale, acc[db][3] * scale)};
      __builtin_amdgcn_raw_buffer_store_b64(h, o.out, base + db * 32, 0, CP);
    }
    return;
  }
  const unsigned base = (unsigned)t * o.ld4 + grp * 16;
#pragma unroll
  for (int db = 0; db < 4; db++)
    bstore4<ALIGNED, CP>(o.out, base + db * 64,
                     make_float4(acc[db][0] * scale, acc[db][1] * scale, acc[db][2] * scale,
                                 acc[db][3] * scale));
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// Maximum over the four lanes {l, l^16, l^32, l^48} holding one column of an MFMA tile, with
// the gfx950 row-swap permutes (each returns the lane's own value and its partner's).
// (The swap results are copied to scalars before reinterpreting: bit-casting a vector element
// lvalue directly would read element 0.)
__device__ __forceinline__ float column_max(float x) {
  const unsigned xb = __builtin_bit_cast(unsigned, x);
  const auto a = __builtin_amdgcn_permlane32_swap(xb, xb, false, false);
  const unsigned a0 = a[0], a1 = a[1];
  const float y = fmaxf(__builtin_bit_cast(float, a0), __builtin_bit_cast(float, a1));
  const unsigned yb = __builtin_bit_cast(unsigned, y);
  const auto b = __builtin_amdgcn_permlane16_swap(yb, yb, false, false);
  const unsigned b0 = b[0], b1 = b[1];
  return fmaxf(__builtin_bit_cast(float, b0), __builtin_bit_cast(float, b1));
}

// acc *= s, written so the result stays in acc's registers: a conditional rescale then costs
// nothing on the path that skips it (no register copies where the two paths join).
__device__ __forceinline__ void scale_in_place(f32x4& acc, float s) {
#pragma unroll
  for (int i = 0; i < 4; i++) asm volatile("v_mul_f32 %0, %0, %1" : "+v"(acc[i]) : "v"(s));
}

// ------------------------------------------------------------------------------------------
// Long sequences: 8 waves x 64 queries of one (group, head) per workgroup (one per CU).
// ------------------------------------------------------------------------------------------
constexpr int kTimeWaves = 8;
constexpr int kTimeQueries = kTimeWaves * 64;

template <bool GATED, bool ROPE, bool ALIGNED, bool XH>
__global__ __launch_bounds__(kTimeWaves * 64) void attention_time_kernel(AttnParams p, int qblocks,
                                                                         int total) {
  __shared__ __attribute__((aligned(16))) unsigned char lds_k[2][64 * 128];
  __shared__ __attribute__((aligned(16))) unsigned char lds_v[2][64 * 128];
  // Each wave's 64 rotated, log2(e)-scaled fp16 queries, laid out like a K tile.
  __shared__ __attribute__((aligned(16))) unsigned char lds_q[kTimeWaves][64 * 128];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int logical = xcd_remap(blockIdx.x, total);
  const int qblk = logical % qblocks, gh = logical / qblocks;
  const int h = gh % p.heads, g = gh / p.heads;
  const int T = p.tokens;
  const long row0 = group_row(p, g), ts = p.tstep;
  // XH: fp16 q / k / v rows (64 * 2 bytes per head), else fp32.
  constexpr unsigned kEsz = XH ? 2 : 4, kRowBytes = 64 * kEsz;
  const unsigned ldq4 = (unsigned)(ts * p.ldq * kEsz), ldk4 = (unsigned)(ts * p.ldk * kEsz),
                 ldv4 = (unsigned)(ts * p.ldv * kEsz);
  const unsigned char* kbase =
      reinterpret_cast<const unsigned char*>(p.k) + (row0 * p.ldk + h * 64) * kEsz;
  const unsigned char* vbase =
      reinterpret_cast<const unsigned char*>(p.v) + (row0 * p.ldv + h * 64) * kEsz;
  const int q0 = qblk * kTimeQueries + wave * 64;
  const bool active = q0 < T;

  // B operand of S^T = K.Q^T (query q0 + qb*16 + col, channels ds*32 + grp*8 .. +7) is read
  // per work unit from this wave's LDS rows, staged once below.
  unsigned char* Q = lds_q[wave];

  // Tile staging (512 threads): thread owns K rows lrow and lrow + 32 at channels 4*lchunk,
  // and the 2-key x 4-channel V block (keys 2*lrow, 2*lrow + 1). Offsets are relative to
  // per-tile buffer descriptors, so they stay fixed across tiles.
  const int lrow = tid >> 4, lchunk = tid & 15;
  const unsigned koff = (unsigned)lrow * ldk4 + lchunk * 16;
  const unsigned voff = (unsigned)(2 * lrow) * ldv4 + lchunk * 16;
  const unsigned toff = (unsigned)lrow * 256 + lchunk * 16;
  float4 kreg[2], vreg[2];
  float4 kcos[2], ksin[2];
  int tile_key0 = 0;
  // fp16 staging: thread owns the 16-byte chunk tid & 7 of K row tid >> 3, and the same V
  // block as above as two 8-byte rows.
  u32x4 kh;
  u32x2 vh[2];
  auto load_tile = [&](int key0) {
    const unsigned rows = (unsigned)(T - key0);
    const rsrc_t kr = make_rsrc(kbase + (long)key0 * ldk4, (rows - 1) * ldk4 + kRowBytes);
    const rsrc_t vr = make_rsrc(vbase + (long)key0 * ldv4, (rows - 1) * ldv4 + kRowBytes);
    if constexpr (XH) {
      kh = __builtin_amdgcn_raw_buffer_load_b128(kr, (unsigned)(tid >> 3) * ldk4 + (tid & 7) * 16,
                                                 0, 0);
#pragma unroll
      for (int r = 0; r < 2; r++)
        vh[r] = __builtin_amdgcn_raw_buffer_load_b64(vr, (unsigned)(2 * lrow + r) * ldv4 + lchunk * 8,
                                                     0, 0);
      return;
    }
#pragma unroll
    for (int it = 0; it < 2; it++) kreg[it] = bload4<ALIGNED>(kr, koff + it * 32 * ldk4);
#pragma unroll
    for (int r = 0; r < 2; r++) vreg[r] = bload4<ALIGNED>(vr, voff + r * ldv4);
    tile_key0 = key0;
  };
  // Key cos rows (table 2) and +sin values (odd channels of table 3) of the staged tile, read
  // when the tile is stored (not a tile ahead: this kernel serves rows that are not 16-byte
  // aligned, and the table registers held across the tile's compute would spill).
  auto load_table = [&]() {
    const unsigned rows = (unsigned)(T - tile_key0);
    const rsrc_t cr = make_rsrc(p.rope + (long)(2 * T + tile_key0) * 64, rows * 256);
    const rsrc_t sr = make_rsrc(p.rope + (long)(3 * T + tile_key0) * 64, rows * 256);
#pragma unroll
    for (int it = 0; it < 2; it++) {
      const unsigned o = toff + it * 32 * 256;
      kcos[it] = bload4<ALIGNED>(cr, o);
      ksin[it] = bload4<ALIGNED>(sr, o);
    }
  };
  auto store_tile = [&](int buf) {
    if constexpr (XH) {
      *reinterpret_cast<u32x4*>(lds_k[buf] + k_offset(tid >> 3, tid & 7)) = kh;
#pragma unroll
      for (int j = 0; j < 4; j++)
        *reinterpret_cast<unsigned*>(lds_v[buf] + vtc_offset(lchunk * 4 + j, 2 * lrow)) =
            v_pair(vh[0], vh[1], j);
      return;
    }
    if constexpr (ROPE) load_table();
#pragma unroll
    for (int it = 0; it < 2; it++) {
      const int r = lrow + 32 * it;
      float4 x = kreg[it];
      if constexpr (ROPE) x = rotate4(x, kcos[it], ksin[it]);
      const u32x2 w = {pack_h2(x.x, x.y), pack_h2(x.z, x.w)};
      *reinterpret_cast<u32x2*>(lds_k[buf] + k_offset(r, lchunk >> 1) + ((lchunk & 1) << 3)) = w;
    }
    // V^T rows 4*lchunk + j get the key pair (2*lrow, 2*lrow + 1) as one dword.
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const unsigned w = pack_h2(comp(vreg[0], j), comp(vreg[1], j));
      *reinterpret_cast<unsigned*>(lds_v[buf] + vtc_offset(lchunk * 4 + j, 2 * lrow)) = w;
    }
  };

  f32x4 o[4][4];
  f32x4 lsum[4];
  const u32x4 ones = {kOnesH2, kOnesH2, kOnesH2, kOnesH2};
  // Running maximum per query block (log2 units). Scores come out of the MFMA as s - m
  // because the S accumulators are seeded with -m.
  float m[4];
#pragma unroll
  for (int qb = 0; qb < 4; qb++) {
#pragma unroll
    for (int db = 0; db < 4; db++) o[db][qb] = zero4();
    lsum[qb] = zero4();
  }

  const int ntiles = (T + 63) / 64;
  load_tile(0);
  if (active) {
    // Stage this wave's 64 query rows: coalesced row loads (16 lanes per 256-byte row), RoPE
    // with the query table rows (carrying 1/sqrt(64)), log2(e), fp16, into the K-tile layout.
    const unsigned rows = (unsigned)(T - q0);
    const rsrc_t qr = make_rsrc(reinterpret_cast<const unsigned char*>(p.q) +
                                    ((row0 + q0 * ts) * p.ldq + h * 64) * kEsz,
                                (rows - 1) * ldq4 + kRowBytes);
    const rsrc_t cr = make_rsrc(ROPE ? p.rope + (long)q0 * 64 : p.q, ROPE ? rows * 256 : 0);
    const rsrc_t sr = make_rsrc(ROPE ? p.rope + (long)(T + q0) * 64 : p.q, ROPE ? rows * 256 : 0);
    const int chunk = lane & 15;
    if constexpr (XH) {
      // Already scaled fp16 rows: 8 rows of eight 16-byte chunks per pass.
#pragma unroll
      for (int it = 0; it < 8; it++) {
        const int r = it * 8 + (lane >> 3);
        *reinterpret_cast<u32x4*>(Q + k_offset(r, lane & 7)) =
            __builtin_amdgcn_raw_buffer_load_b128(qr, (unsigned)r * ldq4 + (lane & 7) * 16, 0, 0);
      }
    }
#pragma unroll
    for (int it = 0; it < (XH ? 0 : 16); it++) {
      const int r = it * 4 + (lane >> 4);
      float4 x = bload4<ALIGNED>(qr, (unsigned)r * ldq4 + chunk * 16);
      if constexpr (ROPE) {
        const unsigned t = (unsigned)r * 256 + chunk * 16;
        x = rotate4(x, bload4<ALIGNED>(cr, t), bload4<ALIGNED>(sr, t));
      }
      x = scale4(x, kLog2e);
      *reinterpret_cast<u32x2*>(Q + k_offset(r, chunk >> 1) + ((chunk & 1) << 3)) =
          u32x2{pack_h2(x.x, x.y), pack_h2(x.z, x.w)};
    }
  }
  store_tile(0);
  // Nothing global is in flight when the tile loop starts, so no load issued above can hold
  // a wait inside it.
  __builtin_amdgcn_s_waitcnt(kWaitVmem);
  __syncthreads();

  // Fragment rows are 16*x + col, so the chunk swizzle depends on col only: one per-lane base
  // per channel step ds (K and Q) or key step ks (V^T), plus compile-time row offsets.
  const int kq_base[2] = {k_offset(col, grp), k_offset(col, 4 + grp)};
  const int vsw = (col ^ (col >> 2)) & 7;
  const int v_base[2][2] = {{col * 128 + ((grp ^ vsw) << 4), col * 128 + ((grp ^ vsw ^ 4) << 4)},
                            {col * 128 + (((4 + grp) ^ vsw) << 4),
                             col * 128 + (((4 + grp) ^ vsw ^ 4) << 4)}};
  auto q_frag = [&](int qb, int ds) {
    return *reinterpret_cast<const u32x4*>(Q + kq_base[ds] + qb * 2048);
  };
  auto k_frag = [&](const unsigned char* K, int half, int kb2, int ds) {
    return *reinterpret_cast<const u32x4*>(K + kq_base[ds] + (half * 2 + kb2) * 2048);
  };
  auto v_frag = [&](const unsigned char* V, int ks, int db) {
    return *reinterpret_cast<const u32x4*>(V + v_base[ks][db & 1] + db * 2048);
  };
  // S^T block of 32 keys (half) x 16 queries (qb): acc[kb2][r] = S[key (half*2+kb2)*16 +
  // grp*4 + r][query qb*16 + col] + init.
  auto score = [&](const u32x4 (&kf)[2][2], const u32x4 (&qf)[2], float init, f32x4 (&acc)[2]) {
    const f32x4 c = {init, init, init, init};
#pragma unroll
    for (int kb2 = 0; kb2 < 2; kb2++) acc[kb2] = mfma16x16x32(kf[kb2][0], qf[0], c);
#pragma unroll
    for (int kb2 = 0; kb2 < 2; kb2++) acc[kb2] = mfma16x16x32(kf[kb2][1], qf[1], acc[kb2]);
  };
  auto lane_max = [](const f32x4 (&acc)[2]) {
    return fmaxf(fmaxf(fmaxf(acc[0][0], acc[0][1]), fmaxf(acc[0][2], acc[0][3])),
                 fmaxf(fmaxf(acc[1][0], acc[1][1]), fmaxf(acc[1][2], acc[1][3])));
  };

  if (active) {
    // The running maximum starts at the exact maximum of the first 32 keys.
    const unsigned char* K = lds_k[0];
    u32x4 kf[2][2];
#pragma unroll
    for (int kb2 = 0; kb2 < 2; kb2++)
#pragma unroll
      for (int ds = 0; ds < 2; ds++) kf[kb2][ds] = k_frag(K, 0, kb2, ds);
#pragma unroll
    for (int qb = 0; qb < 4; qb++) {
      const u32x4 qf[2] = {q_frag(qb, 0), q_frag(qb, 1)};
      f32x4 acc[2];
      score(kf, qf, 0.f, acc);
      if (T < 32) {
#pragma unroll
        for (int kb2 = 0; kb2 < 2; kb2++)
#pragma unroll
          for (int r = 0; r < 4; r++)
            if (kb2 * 16 + grp * 4 + r >= T) acc[kb2][r] = kMasked;
      }
      m[qb] = column_max(lane_max(acc));
    }
  }

  // One 64-key tile: 4 work units u = query block u, each over all 64 keys. Unit u
  // exponentiates its scores while the MFMAs of unit u+1's scores run, then issues its PV
  // MFMAs while the VALU takes unit u+1's maxima. MASK: keys at or past T exist in this tile.
  auto tile = [&](auto mask_tag, int j) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const int buf = j & 1, key0 = j * 64;
    const unsigned char* K = lds_k[buf];
    const unsigned char* V = lds_v[buf];
    u32x4 kf[2][2][2], vf[2][4];  // [half][kb2][ds], [half][db]
    u32x4 qf[2][2];               // Q fragments of the next unit, double buffered
    f32x4 sa[4], sb[4];           // [kb]: keys kb*16 + grp*4 + r
    auto score4 = [&](const u32x4 (&qq)[2], float init, f32x4 (&acc)[4]) {
      const f32x4 c = {init, init, init, init};
#pragma unroll
      for (int kb = 0; kb < 4; kb++) acc[kb] = mfma16x16x32(kf[kb >> 1][kb & 1][0], qq[0], c);
#pragma unroll
      for (int kb = 0; kb < 4; kb++) acc[kb] = mfma16x16x32(kf[kb >> 1][kb & 1][1], qq[1], acc[kb]);
    };
    auto mask_scores = [&](f32x4 (&acc)[4]) {
      if constexpr (MASK) {
#pragma unroll
        for (int kb = 0; kb < 4; kb++)
#pragma unroll
          for (int r = 0; r < 4; r++)
            if (key0 + kb * 16 + grp * 4 + r >= T) acc[kb][r] = kMasked;
      }
    };
    auto settle = [&](int qb, f32x4 (&acc)[4]) {
      const float lm = fmaxf(fmaxf(fmaxf(acc[0][0], acc[0][1]), fmaxf(acc[0][2], acc[0][3])),
                             fmaxf(fmaxf(acc[1][0], acc[1][1]), fmaxf(acc[1][2], acc[1][3])));
      const float lm2 = fmaxf(fmaxf(fmaxf(acc[2][0], acc[2][1]), fmaxf(acc[2][2], acc[2][3])),
                              fmaxf(fmaxf(acc[3][0], acc[3][1]), fmaxf(acc[3][2], acc[3][3])));
      const float l = fmaxf(lm, lm2);
      if (!__builtin_amdgcn_uicmp(l > kTau, 0, 33)) return;
      const float cm = column_max(l);
      if (cm > kTau) {
        const float alpha = fast_exp2(-cm);
        m[qb] += cm;
#pragma unroll
        for (int kb = 0; kb < 4; kb++) acc[kb] -= cm;
        scale_in_place(lsum[qb], alpha);
#pragma unroll
        for (int db = 0; db < 4; db++) scale_in_place(o[db][qb], alpha);
      }
    };
#pragma unroll
    for (int h2 = 0; h2 < 2; h2++)
#pragma unroll
      for (int kb2 = 0; kb2 < 2; kb2++)
#pragma unroll
        for (int ds = 0; ds < 2; ds++) kf[h2][kb2][ds] = k_frag(K, h2, kb2, ds);
    qf[0][0] = q_frag(0, 0);
    qf[0][1] = q_frag(0, 1);
    qf[1][0] = q_frag(1, 0);
    qf[1][1] = q_frag(1, 1);
#pragma unroll
    for (int h2 = 0; h2 < 2; h2++)
#pragma unroll
      for (int db = 0; db < 4; db++) vf[h2][db] = v_frag(V, h2, db);
    score4(qf[0], -m[0], sa);
    mask_scores(sa);
    settle(0, sa);
#pragma unroll
    for (int u = 0; u < 4; u++) {
      __builtin_amdgcn_sched_barrier(0);
      if (u + 2 < 4) {
        qf[u & 1][0] = q_frag(u + 2, 0);
        qf[u & 1][1] = q_frag(u + 2, 1);
      }
      if (u + 1 < 4) score4(qf[(u + 1) & 1], -m[u + 1], sb);
#pragma unroll
      for (int kb = 0; kb < 4; kb++)
#pragma unroll
        for (int r = 0; r < 4; r++) sa[kb][r] = fast_exp2(sa[kb][r]);
      const u32x4 pf0 = p_fragment(sa[0], sa[1]), pf1 = p_fragment(sa[2], sa[3]);
      lsum[u] = mfma16x16x32(ones, pf0, lsum[u]);
      lsum[u] = mfma16x16x32(ones, pf1, lsum[u]);
      if (u + 1 < 4) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          __builtin_amdgcn_sched_group_barrier(0x400, 2, 0);  // transcendental
        }
      }
#pragma unroll
      for (int db = 0; db < 4; db++) o[db][u] = mfma16x16x32(vf[0][db], pf0, o[db][u]);
#pragma unroll
      for (int db = 0; db < 4; db++) o[db][u] = mfma16x16x32(vf[1][db], pf1, o[db][u]);
      if (u + 1 < 4) {
        mask_scores(sb);
        settle(u + 1, sb);
#pragma unroll
        for (int kb = 0; kb < 4; kb++) sa[kb] = sb[kb];
      }
    }
  };

  for (int j = 0; j + 1 < ntiles; j++) {
    load_tile((j + 1) * 64);
    if (active) tile(std::false_type{}, j);
    store_tile((j + 1) & 1);
    __syncthreads();
  }
  if (active) {
    if (T % 64)
      tile(std::true_type{}, ntiles - 1);
    else
      tile(std::false_type{}, ntiles - 1);
  }

  if (active) {
    const OutRows out = out_rows(p, g, h);
#pragma unroll
    for (int qb = 0; qb < 4; qb++) {
      const f32x4 oq[4] = {o[0][qb], o[1][qb], o[2][qb], o[3][qb]};
      store_output<GATED, ALIGNED>(out, oq, lsum[qb][0], q0 + qb * 16 + col, grp);
    }
  }
}

// ------------------------------------------------------------------------------------------
// Short sequences (T <= 64): 4-wave workgroups on (group, head) problems. Per problem the whole
// workgroup stages q, k (rotated, fp16) and v^T (fp16) through LDS from coalesced 16-byte row
// loads, all issued at once; then wave w computes queries 16w .. 16w+15 against all keys with
// an exact softmax. The shape is HBM-bound: q / k / v and the output are streamed
// (non-temporal), each byte being touched once. Two ways to keep loads in flight:
//
//  * fp32 input (the op boundary): persistent workgroups, as many as the CUs hold, each walking
//    problems b, b + grid, ... in two alternating register sets: once a problem is staged, the
//    next one's loads are issued and stay in flight through the current compute and its
//    stores. A thread stages the same rows and channels of every problem, so its rotary table
//    values are loaded once, into registers, for the whole walk.
//  * fp16 input (the network's packed projection): one problem per workgroup; with half the
//    bytes and registers per problem, six workgroups per CU keep enough loads in flight.
//    Workgroups are dealt to the eight XCDs round-robin (workgroup b to XCD b % 8), each with
//    its own L2, and the heads of one group are pieces of the same token rows, so the order
//    gives one XCD all heads of a group on consecutive workgroups: with chunks of 8 * heads
//    workgroups, workgroup b (chunk c = b / (8 * heads), r = b % (8 * heads)) takes group
//    8c + r % 8, head r / 8; groups past the last whole chunk of eight keep the plain order.
// ------------------------------------------------------------------------------------------
__device__ __forceinline__ void band_problem(int b, int groups, int heads, int& g, int& h) {
  const int chunk = kXcds * heads;
  if (b < (groups / kXcds) * chunk) {
    const int c = b / chunk, r = b - c * chunk;
    g = c * kXcds + r % kXcds;
    h = r / kXcds;
  } else {
    g = b / heads;
    h = b - g * heads;
  }
}

// One problem's raw rows in the staging roles (below) of one thread.
template <bool XH>
struct BandRaw;
template <>
struct BandRaw<false> {
  float4 q[4], k[4], v[4];
};
template <>
struct BandRaw<true> {
  u32x4 q[2], k[2];
  u32x2 v[4];
};

template <bool GATED, bool ROPE, bool ALIGNED, bool XH>
__global__ __launch_bounds__(256) void attention_band_kernel(AttnParams p, int problems) {
  static_assert(!(XH && ROPE), "fp16 input arrives rotated");
  constexpr bool kWalk = !XH;
  __shared__ __attribute__((aligned(16))) unsigned char lds_q[64 * 128];
  __shared__ __attribute__((aligned(16))) unsigned char lds_k[64 * 128];
  __shared__ __attribute__((aligned(16))) unsigned char lds_v[64 * 128];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, grp = lane >> 4;
  const int T = p.tokens;
  const long ts = p.tstep;
  constexpr unsigned kEsz = XH ? 2 : 4, kRowBytes = 64 * kEsz;
  const unsigned ldq4 = (unsigned)(ts * p.ldq * kEsz), ldk4 = (unsigned)(ts * p.ldk * kEsz),
                 ldv4 = (unsigned)(ts * p.ldv * kEsz);

  // Staging roles: q / k rows srow + 16*it at channels 4*sc; v key pairs (2*(srow + 16*it),
  // +1), it < 2. fp16 input: q / k rows (tid >> 3) + 32*it as 16-byte chunks tid & 7, v key
  // pairs at 8-byte channel groups sc. Rows at or past T read as 0.
  const int srow = tid >> 4, sc = tid & 15;
  // This thread's rotary table values (query cos / sin, key cos / sin of its four rows).
  float4 tab[4][4];
  if constexpr (ROPE) {
    const rsrc_t tr = make_rsrc(p.rope, (unsigned)T * 1024);
#pragma unroll
    for (int it = 0; it < 4; it++)
#pragma unroll
      for (int t = 0; t < 4; t++)
        tab[it][t] = bload4<ALIGNED>(tr, (unsigned)(t * T + srow + 16 * it) * 256 + sc * 16);
  }
  auto load = [&](int g, int h, BandRaw<XH>& r) {
    const long row0 = group_row(p, g);
    auto rows_of = [&](const float* base, long ld, unsigned ld4) {
      return make_rsrc(reinterpret_cast<const unsigned char*>(base) + (row0 * ld + h * 64) * kEsz,
                       (unsigned)(T - 1) * ld4 + kRowBytes);
    };
    const rsrc_t qr = rows_of(p.q, p.ldq, ldq4);
    const rsrc_t kr = rows_of(p.k, p.ldk, ldk4);
    const rsrc_t vr = rows_of(p.v, p.ldv, ldv4);
    if constexpr (XH) {
#pragma unroll
      for (int it = 0; it < 2; it++) {
        const unsigned rr = (unsigned)((tid >> 3) + 32 * it);
        r.q[it] = __builtin_amdgcn_raw_buffer_load_b128(qr, rr * ldq4 + (tid & 7) * 16, 0, kStream);
        r.k[it] = __builtin_amdgcn_raw_buffer_load_b128(kr, rr * ldk4 + (tid & 7) * 16, 0, kStream);
      }
#pragma unroll
      for (int it = 0; it < 2; it++)
#pragma unroll
        for (int j = 0; j < 2; j++)
          r.v[it * 2 + j] = __builtin_amdgcn_raw_buffer_load_b64(
              vr, (unsigned)(2 * (srow + 16 * it) + j) * ldv4 + sc * 8, 0, kStream);
    } else {
#pragma unroll
      for (int it = 0; it < 4; it++) {
        const unsigned rr = (unsigned)(srow + 16 * it);
        r.q[it] = bload4<ALIGNED, kStream>(qr, rr * ldq4 + sc * 16);
        r.k[it] = bload4<ALIGNED, kStream>(kr, rr * ldk4 + sc * 16);
      }
#pragma unroll
      for (int it = 0; it < 2; it++)
#pragma unroll
        for (int j = 0; j < 2; j++)
          r.v[it * 2 + j] =
              bload4<ALIGNED, kStream>(vr, (unsigned)(2 * (srow + 16 * it) + j) * ldv4 + sc * 16);
    }
  };
  auto stage = [&](const BandRaw<XH>& r) {
    if constexpr (XH) {
#pragma unroll
      for (int it = 0; it < 2; it++) {
        const int off = k_offset((tid >> 3) + 32 * it, tid & 7);
        *reinterpret_cast<u32x4*>(lds_q + off) = r.q[it];
        *reinterpret_cast<u32x4*>(lds_k + off) = r.k[it];
      }
#pragma unroll
      for (int it = 0; it < 2; it++)
#pragma unroll
        for (int j = 0; j < 4; j++)
          *reinterpret_cast<unsigned*>(lds_v + vtc_offset(sc * 4 + j, 2 * (srow + 16 * it))) =
              v_pair(r.v[it * 2], r.v[it * 2 + 1], j);
    } else {
#pragma unroll
      for (int it = 0; it < 4; it++) {
        const int rr = srow + 16 * it;
        float4 q = r.q[it], k = r.k[it];
        if constexpr (ROPE) {
          q = rotate4(q, tab[it][0], tab[it][1]);
          k = rotate4(k, tab[it][2], tab[it][3]);
        }
        q = scale4(q, kLog2e);
        const int off = k_offset(rr, sc >> 1) + ((sc & 1) << 3);
        *reinterpret_cast<u32x2*>(lds_q + off) = u32x2{pack_h2(q.x, q.y), pack_h2(q.z, q.w)};
        *reinterpret_cast<u32x2*>(lds_k + off) = u32x2{pack_h2(k.x, k.y), pack_h2(k.z, k.w)};
      }
#pragma unroll
      for (int it = 0; it < 2; it++)
#pragma unroll
        for (int j = 0; j < 4; j++)
          *reinterpret_cast<unsigned*>(lds_v + vtc_offset(sc * 4 + j, 2 * (srow + 16 * it))) =
              pack_h2(comp(r.v[it * 2], j), comp(r.v[it * 2 + 1], j));
    }
  };

  const int q0 = wave * 16;
  const int kq_base[2] = {k_offset(col, grp), k_offset(col, 4 + grp)};
  const int vsw = (col ^ (col >> 2)) & 7;
  const int v_base[2][2] = {{col * 128 + ((grp ^ vsw) << 4), col * 128 + ((grp ^ vsw ^ 4) << 4)},
                            {col * 128 + (((4 + grp) ^ vsw) << 4),
                             col * 128 + (((4 + grp) ^ vsw ^ 4) << 4)}};
  auto compute = [&](int g, int h) {
    const u32x4 qf[2] = {*reinterpret_cast<const u32x4*>(lds_q + kq_base[0] + wave * 2048),
                         *reinterpret_cast<const u32x4*>(lds_q + kq_base[1] + wave * 2048)};
    f32x4 s[4];
#pragma unroll
    for (int kb = 0; kb < 4; kb++) {
      s[kb] = zero4();
#pragma unroll
      for (int ds = 0; ds < 2; ds++)
        s[kb] = mfma16x16x32(*reinterpret_cast<const u32x4*>(lds_k + kq_base[ds] + kb * 2048),
                             qf[ds], s[kb]);
    }
    if (T < 64) {
#pragma unroll
      for (int kb = 0; kb < 4; kb++)
#pragma unroll
        for (int r = 0; r < 4; r++)
          if (kb * 16 + grp * 4 + r >= T) s[kb][r] = kMasked;
    }
    float mx = kMasked;
#pragma unroll
    for (int kb = 0; kb < 4; kb++)
#pragma unroll
      for (int r = 0; r < 4; r++) mx = fmaxf(mx, s[kb][r]);
    mx = max_over_rows(mx);
#pragma unroll
    for (int kb = 0; kb < 4; kb++)
#pragma unroll
      for (int r = 0; r < 4; r++) s[kb][r] = fast_exp2(s[kb][r] - mx);
    const u32x4 pf[2] = {p_fragment(s[0], s[1]), p_fragment(s[2], s[3])};
    const u32x4 ones = {kOnesH2, kOnesH2, kOnesH2, kOnesH2};
    f32x4 o[4] = {zero4(), zero4(), zero4(), zero4()}, lsum = zero4();
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
#pragma unroll
      for (int db = 0; db < 4; db++)
        o[db] = mfma16x16x32(
            *reinterpret_cast<const u32x4*>(lds_v + v_base[ks][db & 1] + db * 2048), pf[ks], o[db]);
      lsum = mfma16x16x32(ones, pf[ks], lsum);
    }
    // fp16 input stores fp16 (fixed at compile time: no branch between the loads and the
    // waits, 1.5 % off the layer). The fp32 walk keeps the run-time form: with the branch
    // removed the compiler's wait placement changes and the walk measured 5 % slower.
    store_output<GATED, ALIGNED, kStream, XH ? 1 : -1>(out_rows(p, g, h), o, lsum[0], q0 + col,
                                                       grp);
  };

  if constexpr (kWalk) {
    // Workgroup-uniform: every wave runs every step and reaches both barriers. The next loads
    // go out after the staging barrier and ahead of this problem's stores, so the wait before
    // the next staging leaves those stores outstanding. Past the end they reload the last
    // problem (unused), and a wave whose 16 queries all lie at or past T (T <= 48) computes
    // anyway (its q rows are zero; rows at or past T lie outside the output's buffer range, so
    // their stores are dropped): no branch around the loads and stores keeps the wait counts
    // fixed.
    auto step = [&](int prob, const BandRaw<XH>& cur, BandRaw<XH>& nxt) {
      stage(cur);
      __syncthreads();
      const int next = min(prob + (int)gridDim.x, problems - 1);
      load(next / p.heads, next % p.heads, nxt);
      compute(prob / p.heads, prob % p.heads);
      __syncthreads();  // the next step restages LDS
    };
    // The first step is peeled so the loop is entered with the same loads and stores
    // outstanding as each turn ends with (else the wait counts at the loop head are merged down
    // to a full drain).
    BandRaw<XH> a, b;
    int prob = blockIdx.x;
    load(prob / p.heads, prob % p.heads, a);
    step(prob, a, b);
    while (true) {
      prob += gridDim.x;
      if (prob >= problems) break;
      step(prob, b, a);
      prob += gridDim.x;
      if (prob >= problems) break;
      step(prob, a, b);
    }
  } else {
    int g, h;
    band_problem(blockIdx.x, p.groups, p.heads, g, h);
    BandRaw<XH> r;
    load(g, h, r);
    stage(r);
    __syncthreads();
    if (q0 < T) compute(g, h);
  }
}

template <bool GATED, bool ROPE, bool ALIGNED, bool XH = false>
static hipError_t launch_attention_t(const AttnParams& p, hipStream_t stream) {
  const int T = p.tokens;
  if (T <= 64) {
    auto kernel = attention_band_kernel<GATED, ROPE, ALIGNED, XH>;
    const int problems = p.groups * p.heads;
    int grid = problems;
    if constexpr (!XH) {
      // The walk: as many workgroups as the CUs hold at once.
      static int per_cu = 0;
      if (per_cu <= 0 &&
          (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 256, 0) != hipSuccess ||
           per_cu <= 0))
        per_cu = 2;
      const long cap = (long)per_cu * device_cus();
      if (cap < problems) grid = (int)cap;
    }
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(256), 0, stream, p, problems);
  } else {
    if constexpr (ALIGNED) {
      return launch_attention_long(p, GATED, ROPE, stream);
    } else {
      const int qblocks = (T + kTimeQueries - 1) / kTimeQueries;
      const int total = p.groups * p.heads * qblocks;
      hipLaunchKernelGGL((attention_time_kernel<GATED, ROPE, ALIGNED, XH>), dim3(total),
                         dim3(kTimeWaves * 64), 0, stream, p, qblocks, total);
    }
  }
  return hipGetLastError();
}

bool attention_grid_fits(size_t groups, size_t tokens, size_t heads) {
  const size_t problems = groups * heads;
  if (groups != 0 && problems / groups != heads) return false;
  const size_t blocks =
      tokens <= 64 ? problems : problems * ((tokens + kTimeQueries - 1) / kTimeQueries);
  const size_t threads = tokens <= 64 ? 256 : kTimeWaves * 64;
  return blocks < (size_t(1) << 31) && blocks * threads < (size_t(1) << 32);
}

hipError_t launch_attention(const AttnParams& params, bool aligned, hipStream_t stream) {
  AttnParams p = params;
  if (p.gsplit == 0) {
    p.gsplit = 1;
    p.gouter = p.tokens;
    p.gstep = 0;
    p.tstep = 1;
  }
  const bool gated = p.gate != nullptr, rope = p.rope != nullptr;
  if ((p.in_half != 0) != (p.out_half != 0)) return hipErrorInvalidValue;
  if (p.in_half) {
    // The block's packed fp16 projection only.
    if (!gated || rope || !aligned) return hipErrorInvalidValue;
    return launch_attention_t<true, false, true, true>(p, stream);
  }
  if (aligned) {
    if (gated) return rope ? launch_attention_t<true, true, true>(p, stream)
                           : launch_attention_t<true, false, true>(p, stream);
    return rope ? launch_attention_t<false, true, true>(p, stream)
                : launch_attention_t<false, false, true>(p, stream);
  }
  if (gated) return rope ? launch_attention_t<true, true, false>(p, stream)
                         : launch_attention_t<true, false, false>(p, stream);
  return rope ? launch_attention_t<false, true, false>(p, stream)
              : launch_attention_t<false, false, false>(p, stream);
}

}  // namespace ancha
