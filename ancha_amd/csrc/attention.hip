// Fused RoFormer attention for CDNA4 (gfx950): softmax(q.k^T).v per (group, head) with the
// optional interleaved RoPE applied while q/k are loaded and the optional per-head sigmoid gate
// in the epilogue. Replaces the CubeCL `flash_attention` of
// crates/ancha-models/src/fused/attention.rs:26-227 (launch :250-298).
//
// Both kernels compute S^T = K.Q^T and O^T = V^T.P^T with v_mfma_f32_16x16x32_f16, so that the
// score tile produced by the first product is already, lane for lane, the B operand of the
// second: each lane owns one query column and 4+4 keys of every 32-key step. The online softmax
// runs in fp32 in the log2 domain (q carries log2(e)), the row max/sum reductions are two
// cross-lane shuffles, and the 1/l normalisation and the gate are applied once at the end.
//
//  * attention_time_kernel: long sequences (the time axis, T ~ 801). One workgroup = 4 waves =
//    128 queries of one (group, head); 64-key K / V^T tiles are staged in LDS as fp16, double
//    buffered, the next tile's global loads in flight while the current one is multiplied.
//  * attention_band_kernel: T <= 64 (the band axis, 60-62 bands, huge batch). One wave owns one
//    whole (group, head) problem: K and Q fragments come straight from global memory into
//    registers, V goes through a wave-private LDS transpose, softmax is exact (one key tile).
#include "common.hpp"
#include "kernels.hpp"

namespace ancha {

template <bool ALIGNED>
__device__ __forceinline__ float4 load4(const float* p) {
  if constexpr (ALIGNED) {
    return *reinterpret_cast<const float4*>(p);
  } else {
    return make_float4(p[0], p[1], p[2], p[3]);
  }
}

template <bool ALIGNED>
__device__ __forceinline__ void store4(float* p, float4 v) {
  if constexpr (ALIGNED) {
    *reinterpret_cast<float4*>(p) = v;
  } else {
    p[0] = v.x;
    p[1] = v.y;
    p[2] = v.z;
    p[3] = v.w;
  }
}

__device__ __forceinline__ float comp(float4 v, int j) {
  return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w;
}

// 8-byte chunk swizzle of a transposed V^T row `d` (64 keys = 16 chunks of 4 fp16): keeps both
// the 4x4-block transposing writes and the MFMA operand reads free of LDS bank conflicts.
__device__ __forceinline__ int vt_swizzle(int d) { return ((d >> 2) ^ (d << 2)) & 15; }

// Loads 8 consecutive channels [d, d+8) of row t (zero when t >= T), applies the rotary table
// rows (cos at table `ct`, signed sin at `ct + 1`) when ROPE, scales, and packs to fp16.
template <bool ROPE, bool ALIGNED>
__device__ __forceinline__ u32x4 load_fragment(const float* base, long ld, int t, int T, int d,
                                               const float* rope, int ct, float scale) {
  float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
  if (t < T) {
    const float* src = base + (long)t * ld + d;
    a = load4<ALIGNED>(src);
    b = load4<ALIGNED>(src + 4);
    if constexpr (ROPE) {
      const float* c = rope + ((long)ct * T + t) * 64 + d;
      const float* s = c + (long)T * 64;
      a = rotate4(a, load4<ALIGNED>(c), load4<ALIGNED>(s));
      b = rotate4(b, load4<ALIGNED>(c + 4), load4<ALIGNED>(s + 4));
    }
    a = scale4(a, scale);
    b = scale4(b, scale);
  }
  return u32x4{pack_h2(a.x, a.y), pack_h2(a.z, a.w), pack_h2(b.x, b.y),
               pack_h2(b.z, b.w)};
}

// Writes a 4-key x 4-channel block (rows r = 0..3 of `vr` are keys 4*kq+r, channels 4*dq..+3)
// transposed into the V^T tile: row 4*dq+j gets keys 4*kq..4*kq+3 as one 8-byte chunk.
__device__ __forceinline__ void store_vt_block(unsigned char* vt, const float4 (&vr)[4], int kq,
                                               int dq) {
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int d = dq * 4 + j;
    const u32x2 w = {pack_h2(comp(vr[0], j), comp(vr[1], j)),
                     pack_h2(comp(vr[2], j), comp(vr[3], j))};
    *reinterpret_cast<u32x2*>(vt + d * 128 + ((kq ^ vt_swizzle(d)) << 3)) = w;
  }
}

// A operand of O^T = V^T.P^T for channel block db and 32-key step ks: lane holds channel
// db*16 + col and keys ks*32 + {grp*4 + i, 16 + grp*4 + i}, i = 0..3.
__device__ __forceinline__ u32x4 vt_fragment(const unsigned char* vt, int db, int ks, int col,
                                             int grp) {
  const int d = db * 16 + col, sw = vt_swizzle(d);
  const u32x2 lo = *reinterpret_cast<const u32x2*>(vt + d * 128 + (((ks * 8 + grp) ^ sw) << 3));
  const u32x2 hi =
      *reinterpret_cast<const u32x2*>(vt + d * 128 + (((ks * 8 + 4 + grp) ^ sw) << 3));
  return u32x4{lo.x, lo.y, hi.x, hi.y};
}

// B operand of O^T = V^T.P^T from the score tiles of key blocks 2ks and 2ks+1.
__device__ __forceinline__ u32x4 p_fragment(f32x4 a, f32x4 b) {
  return u32x4{pack_h2(a[0], a[1]), pack_h2(a[2], a[3]), pack_h2(b[0], b[1]),
               pack_h2(b[2], b[3])};
}

// Final 1/l and sigmoid(gate) scaling and store of one lane's 16 channels of query t.
template <bool GATED, bool ALIGNED>
__device__ __forceinline__ void store_output(const AttnParams& p, const f32x4 (&o)[4], float l,
                                             int g, int h, int t, int grp) {
  float scale = 1.0f / l;
  if constexpr (GATED) {
    const float gate = p.gate[((long)g * p.tokens + t) * p.ldg + h];
    scale = scale / (1.0f + expf(-gate));
  }
  float* dst = p.out + (((long)g * p.tokens + t) * p.heads + h) * 64 + grp * 4;
#pragma unroll
  for (int db = 0; db < 4; db++)
    store4<ALIGNED>(dst + db * 16, make_float4(o[db][0] * scale, o[db][1] * scale,
                                               o[db][2] * scale, o[db][3] * scale));
}

// ------------------------------------------------------------------------------------------
// Long sequences: 4 waves x 32 queries of one (group, head) per workgroup.
// ------------------------------------------------------------------------------------------
template <bool GATED, bool ROPE, bool ALIGNED>
__global__ __launch_bounds__(256) void attention_time_kernel(AttnParams p, int qblocks,
                                                             int total) {
  __shared__ __attribute__((aligned(16))) unsigned char lds_k[2][64 * 128];
  __shared__ __attribute__((aligned(16))) unsigned char lds_v[2][64 * 128];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int logical = xcd_remap(blockIdx.x, total);
  const int qblk = logical % qblocks, gh = logical / qblocks;
  const int h = gh % p.heads, g = gh / p.heads;
  const int T = p.tokens;
  const float* qg = p.q + (long)g * T * p.ldq + h * 64;
  const float* kg = p.k + (long)g * T * p.ldk + h * 64;
  const float* vg = p.v + (long)g * T * p.ldv + h * 64;
  const int q0 = qblk * 128 + wave * 32;
  const bool active = q0 < T;

  // B operand of S^T = K.Q^T: query qb*16 + col, channels ds*32 + grp*8 .. +7, log2(e) folded.
  u32x4 qf[2][2];
#pragma unroll
  for (int qb = 0; qb < 2; qb++)
#pragma unroll
    for (int ds = 0; ds < 2; ds++)
      qf[qb][ds] = load_fragment<ROPE, ALIGNED>(qg, p.ldq, q0 + qb * 16 + col, T,
                                                ds * 32 + grp * 8, p.rope, 0, kLog2e);

  // Tile staging: thread owns key rows (tid>>4) + 16*it of K at channels 4*(tid&15), and the
  // 4x4 V block (keys 4*(tid>>4)..+3, channels 4*(tid&15)..+3).
  const int lrow = tid >> 4, lchunk = tid & 15;
  float4 kreg[4], kcos[4], ksin[4], vreg[4];
  auto load_tile = [&](int key0) {
#pragma unroll
    for (int it = 0; it < 4; it++) {
      const int t = key0 + lrow + 16 * it;
      const bool ok = t < T;
      kreg[it] = ok ? load4<ALIGNED>(kg + (long)t * p.ldk + lchunk * 4)
                    : make_float4(0.f, 0.f, 0.f, 0.f);
      if constexpr (ROPE) {
        const float* c = p.rope + ((long)2 * T + (ok ? t : 0)) * 64 + lchunk * 4;
        kcos[it] = load4<ALIGNED>(c);
        ksin[it] = load4<ALIGNED>(c + (long)T * 64);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int t = key0 + lrow * 4 + r;
      vreg[r] = t < T ? load4<ALIGNED>(vg + (long)t * p.ldv + lchunk * 4)
                      : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int it = 0; it < 4; it++) {
      const int r = lrow + 16 * it;
      float4 x = kreg[it];
      if constexpr (ROPE) x = rotate4(x, kcos[it], ksin[it]);
      const u32x2 w = {pack_h2(x.x, x.y), pack_h2(x.z, x.w)};
      *reinterpret_cast<u32x2*>(lds_k[buf] + r * 128 + ((((lchunk >> 1) ^ (r & 7))) << 4) +
                                ((lchunk & 1) << 3)) = w;
    }
    store_vt_block(lds_v[buf], vreg, lrow, lchunk);
  };

  f32x4 o[4][2];
#pragma unroll
  for (int db = 0; db < 4; db++)
#pragma unroll
    for (int qb = 0; qb < 2; qb++) o[db][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m[2] = {kMasked, kMasked}, l[2] = {0.f, 0.f};

  const int ntiles = (T + 63) / 64;
  load_tile(0);
  store_tile(0);
  __syncthreads();
  for (int j = 0; j < ntiles; j++) {
    const int buf = j & 1;
    if (j + 1 < ntiles) load_tile((j + 1) * 64);
    if (active) {
      const unsigned char* K = lds_k[buf];
      const unsigned char* V = lds_v[buf];
      // S^T[key kb*16 + grp*4 + r][query qb*16 + col] in s[kb][qb][r].
      f32x4 s[4][2];
#pragma unroll
      for (int kb = 0; kb < 4; kb++) {
        s[kb][0] = f32x4{0.f, 0.f, 0.f, 0.f};
        s[kb][1] = s[kb][0];
        const int r = kb * 16 + col;
#pragma unroll
        for (int ds = 0; ds < 2; ds++) {
          const int c16 = ds * 4 + grp;
          const u32x4 kf = *reinterpret_cast<const u32x4*>(K + r * 128 + ((c16 ^ (r & 7)) << 4));
          s[kb][0] = mfma16x16x32(kf, qf[0][ds], s[kb][0]);
          s[kb][1] = mfma16x16x32(kf, qf[1][ds], s[kb][1]);
        }
      }
      const int key0 = j * 64;
      if (key0 + 64 > T) {
#pragma unroll
        for (int kb = 0; kb < 4; kb++)
#pragma unroll
          for (int r = 0; r < 4; r++)
            if (key0 + kb * 16 + grp * 4 + r >= T) {
              s[kb][0][r] = kMasked;
              s[kb][1][r] = kMasked;
            }
      }
#pragma unroll
      for (int qb = 0; qb < 2; qb++) {
        float mx = kMasked;
#pragma unroll
        for (int kb = 0; kb < 4; kb++)
#pragma unroll
          for (int r = 0; r < 4; r++) mx = fmaxf(mx, s[kb][qb][r]);
        mx = max_over_rows(mx);
        const float mn = fmaxf(m[qb], mx);
        const float alpha = fast_exp2(m[qb] - mn);
        m[qb] = mn;
        float sum = 0.f;
#pragma unroll
        for (int kb = 0; kb < 4; kb++)
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const float e = fast_exp2(s[kb][qb][r] - mn);
            s[kb][qb][r] = e;
            sum += e;
          }
        l[qb] = l[qb] * alpha + sum;
#pragma unroll
        for (int db = 0; db < 4; db++) o[db][qb] *= alpha;
      }
#pragma unroll
      for (int ks = 0; ks < 2; ks++) {
        const u32x4 pf0 = p_fragment(s[2 * ks][0], s[2 * ks + 1][0]);
        const u32x4 pf1 = p_fragment(s[2 * ks][1], s[2 * ks + 1][1]);
#pragma unroll
        for (int db = 0; db < 4; db++) {
          const u32x4 vf = vt_fragment(V, db, ks, col, grp);
          o[db][0] = mfma16x16x32(vf, pf0, o[db][0]);
          o[db][1] = mfma16x16x32(vf, pf1, o[db][1]);
        }
      }
    }
    if (j + 1 < ntiles) store_tile(buf ^ 1);
    __syncthreads();
  }

  if (active) {
#pragma unroll
    for (int qb = 0; qb < 2; qb++) {
      const float lt = sum_over_rows(l[qb]);
      const int t = q0 + qb * 16 + col;
      f32x4 oq[4] = {o[0][qb], o[1][qb], o[2][qb], o[3][qb]};
      if (t < T) store_output<GATED, ALIGNED>(p, oq, lt, g, h, t, grp);
    }
  }
}

// ------------------------------------------------------------------------------------------
// Short sequences (T <= 64): one wave per (group, head), 4 problems per workgroup.
// ------------------------------------------------------------------------------------------
template <bool GATED, bool ROPE, bool ALIGNED>
__global__ __launch_bounds__(256) void attention_band_kernel(AttnParams p, int problems) {
  __shared__ __attribute__((aligned(16))) unsigned char lds_v[4][64 * 128];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int prob = blockIdx.x * 4 + wave;
  const bool active = prob < problems;
  const int pr = active ? prob : 0;
  const int h = pr % p.heads, g = pr / p.heads;
  const int T = p.tokens;
  const float* qg = p.q + (long)g * T * p.ldq + h * 64;
  const float* kg = p.k + (long)g * T * p.ldk + h * 64;
  const float* vg = p.v + (long)g * T * p.ldv + h * 64;
  unsigned char* vt = lds_v[wave];

  if (active) {
    // V^T through LDS: lane owns the 4x4 blocks (keys 4*kq..+3, channels 4*col..+3),
    // kq = grp + 4*it.
#pragma unroll
    for (int it = 0; it < 4; it++) {
      const int kq = grp + 4 * it;
      float4 vr[4];
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int t = kq * 4 + r;
        vr[r] = t < T ? load4<ALIGNED>(vg + (long)t * p.ldv + col * 4)
                      : make_float4(0.f, 0.f, 0.f, 0.f);
      }
      store_vt_block(vt, vr, kq, col);
    }
  }
  __syncthreads();
  if (!active) return;

  // A operand of S^T = K.Q^T: key kb*16 + col, channels ds*32 + grp*8 .. +7 (rotated).
  u32x4 kf[4][2];
#pragma unroll
  for (int kb = 0; kb < 4; kb++)
#pragma unroll
    for (int ds = 0; ds < 2; ds++)
      kf[kb][ds] = load_fragment<ROPE, ALIGNED>(kg, p.ldk, kb * 16 + col, T, ds * 32 + grp * 8,
                                                p.rope, 2, 1.0f);

#pragma unroll
  for (int qp = 0; qp < 2; qp++) {
    u32x4 qf[2][2];
#pragma unroll
    for (int qb = 0; qb < 2; qb++)
#pragma unroll
      for (int ds = 0; ds < 2; ds++)
        qf[qb][ds] = load_fragment<ROPE, ALIGNED>(qg, p.ldq, (qp * 2 + qb) * 16 + col, T,
                                                  ds * 32 + grp * 8, p.rope, 0, kLog2e);
    f32x4 s[4][2];
#pragma unroll
    for (int kb = 0; kb < 4; kb++) {
      s[kb][0] = f32x4{0.f, 0.f, 0.f, 0.f};
      s[kb][1] = s[kb][0];
#pragma unroll
      for (int ds = 0; ds < 2; ds++) {
        s[kb][0] = mfma16x16x32(kf[kb][ds], qf[0][ds], s[kb][0]);
        s[kb][1] = mfma16x16x32(kf[kb][ds], qf[1][ds], s[kb][1]);
      }
    }
    if (T < 64) {
#pragma unroll
      for (int kb = 0; kb < 4; kb++)
#pragma unroll
        for (int r = 0; r < 4; r++)
          if (kb * 16 + grp * 4 + r >= T) {
            s[kb][0][r] = kMasked;
            s[kb][1][r] = kMasked;
          }
    }
    float l[2];
#pragma unroll
    for (int qb = 0; qb < 2; qb++) {
      float mx = kMasked;
#pragma unroll
      for (int kb = 0; kb < 4; kb++)
#pragma unroll
        for (int r = 0; r < 4; r++) mx = fmaxf(mx, s[kb][qb][r]);
      mx = max_over_rows(mx);
      float sum = 0.f;
#pragma unroll
      for (int kb = 0; kb < 4; kb++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const float e = fast_exp2(s[kb][qb][r] - mx);
          s[kb][qb][r] = e;
          sum += e;
        }
      l[qb] = sum_over_rows(sum);
    }
    f32x4 o[4][2];
#pragma unroll
    for (int db = 0; db < 4; db++) {
      o[db][0] = f32x4{0.f, 0.f, 0.f, 0.f};
      o[db][1] = o[db][0];
    }
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
      const u32x4 pf0 = p_fragment(s[2 * ks][0], s[2 * ks + 1][0]);
      const u32x4 pf1 = p_fragment(s[2 * ks][1], s[2 * ks + 1][1]);
#pragma unroll
      for (int db = 0; db < 4; db++) {
        const u32x4 vf = vt_fragment(vt, db, ks, col, grp);
        o[db][0] = mfma16x16x32(vf, pf0, o[db][0]);
        o[db][1] = mfma16x16x32(vf, pf1, o[db][1]);
      }
    }
#pragma unroll
    for (int qb = 0; qb < 2; qb++) {
      const int t = (qp * 2 + qb) * 16 + col;
      f32x4 oq[4] = {o[0][qb], o[1][qb], o[2][qb], o[3][qb]};
      if (t < T) store_output<GATED, ALIGNED>(p, oq, l[qb], g, h, t, grp);
    }
  }
}

template <bool GATED, bool ROPE, bool ALIGNED>
static hipError_t launch_attention_t(const AttnParams& p, hipStream_t stream) {
  const int T = p.tokens;
  if (T <= 64) {
    const int problems = p.groups * p.heads;
    hipLaunchKernelGGL((attention_band_kernel<GATED, ROPE, ALIGNED>), dim3((problems + 3) / 4),
                       dim3(256), 0, stream, p, problems);
  } else {
    const int qblocks = (T + 127) / 128;
    const int total = p.groups * p.heads * qblocks;
    hipLaunchKernelGGL((attention_time_kernel<GATED, ROPE, ALIGNED>), dim3(total), dim3(256), 0,
                       stream, p, qblocks, total);
  }
  return hipGetLastError();
}

hipError_t launch_attention(const AttnParams& p, bool aligned, hipStream_t stream) {
  const bool gated = p.gate != nullptr, rope = p.rope != nullptr;
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
