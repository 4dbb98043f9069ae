// Fused RoFormer attention for CDNA4 (gfx950): softmax(q.k^T).v per (group, head) with the
// optional interleaved RoPE applied while q/k are loaded and the optional per-head sigmoid gate
// in the epilogue. Replaces the CubeCL `flash_attention` of
// crates/ancha-models/src/fused/attention.rs:26-227 (launch :250-298).
//
// The kernel here computes S^T = K.Q^T and O^T = V^T.P^T with v_mfma_f32_16x16x32_f16, so that
// the score tile produced by the first product is already, lane for lane, the B operand of the
// second: each lane owns one query column and 4+4 keys of every 32-key step. The softmax runs
// in fp32 in the log2 domain (q carries log2(e)); row sums come from the MFMA (a ones matrix
// times P^T, so numerator and denominator see the same fp16-rounded probabilities), and 1/l and
// the gate are applied once in the epilogue.
//
// All global traffic goes through raw buffer loads/stores whose hardware range check returns 0
// for rows at or past `tokens` (and drops stores there), so ragged tails need no branches.
//
//  * attention_band_kernel: T <= 64 (the band axis, 60-62 bands, huge batch). One 4-wave
//    workgroup per (group, head) problem stages q, k (rotated) and v^T through LDS with
//    coalesced row loads, then each wave takes 16 queries; softmax is exact (one key tile).
//  * T > 64 (the time axis), aligned rows or not: attention_long.hip's 32x32x16 kernel.
#include <type_traits>

#include "attention.hpp"

namespace ancha {

// fp16 1.0 in both halves of a dword: the A operand of the row-sum MFMA.
constexpr unsigned kOnesH2 = 0x3C003C00u;

// Chunked V^T tile: row d holds the 64 keys of channel d, and the 16-byte chunk
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

// fp32 output of one wave's 16 queries q0 .. q0 + 15 as whole 256-byte rows: the lanes' values
// (1/l and the gate applied) go through the wave's 4 KB LDS area W (row r = query, 16-byte chunk
// c of row r at position c ^ r, conflict-free for the 16-lane cycles of both passes), then 16
// lanes store one row per instruction, i.e. whole 128-byte lines (non-temporal stores of
// 64-byte pieces reach HBM partly as partial lines).
template <bool GATED, bool ALIGNED, int CP>
__device__ __forceinline__ void store_output_rows(const OutRows& o, const f32x4 (&acc)[4], float l,
                                                  int q0, int col, int grp, int lane,
                                                  unsigned char* W) {
  float scale = 1.0f / l;
  if constexpr (GATED) {
    const unsigned t = (unsigned)(q0 + col);
    const float gl =
        o.gate_half ? (float)__builtin_bit_cast(
                          _Float16, __builtin_amdgcn_raw_buffer_load_b16(o.gate, t * o.ldg4, 0, 0))
                    : bload1(o.gate, t * o.ldg4);
    scale = scale / (1.0f + expf(-gl));
  }
#pragma unroll
  for (int db = 0; db < 4; db++)
    *reinterpret_cast<f32x4*>(W + col * 256 + (((grp + 4 * db) ^ col) << 4)) = acc[db] * scale;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int r = 4 * k + (lane >> 4), c = lane & 15;
    const f32x4 v = *reinterpret_cast<const f32x4*>(W + r * 256 + ((c ^ r) << 4));
    bstore4<ALIGNED, CP>(o.out, (unsigned)(q0 + r) * o.ld4 + c * 16,
                         make_float4(v[0], v[1], v[2], v[3]));
  }
}

// The same for fp16 output (the block's packed projection): 128-byte rows, 8 lanes a row, staged
// in the wave's own 2 KB of query rows (read into registers before; chunk c of row r at position
// c ^ ((r >> 1) & 7), conflict-free for the 8-byte writes and the 16-byte reads).
template <bool GATED, int CP>
__device__ __forceinline__ void store_output_rows_h(const OutRows& o, const f32x4 (&acc)[4], float l,
                                                    int q0, int col, int grp, int lane,
                                                    unsigned char* W) {
  float scale = 1.0f / l;
  if constexpr (GATED) {
    const unsigned t = (unsigned)(q0 + col);
    const float gl =
        o.gate_half ? (float)__builtin_bit_cast(
                          _Float16, __builtin_amdgcn_raw_buffer_load_b16(o.gate, t * o.ldg4, 0, 0))
                    : bload1(o.gate, t * o.ldg4);
    scale = scale / (1.0f + expf(-gl));
  }
#pragma unroll
  for (int db = 0; db < 4; db++) {
    const int chunk = 2 * db + (grp >> 1);
    *reinterpret_cast<u32x2*>(W + col * 128 + ((chunk ^ ((col >> 1) & 7)) << 4) + 8 * (grp & 1)) =
        u32x2{pack_h2(acc[db][0] * scale, acc[db][1] * scale),
              pack_h2(acc[db][2] * scale, acc[db][3] * scale)};
  }
#pragma unroll
  for (int k = 0; k < 2; k++) {
    const int r = 8 * k + (lane >> 3), c = lane & 7;
    const u32x4 v = *reinterpret_cast<const u32x4*>(W + r * 128 + ((c ^ ((r >> 1) & 7)) << 4));
    __builtin_amdgcn_raw_buffer_store_b128(v, o.out, (unsigned)(q0 + r) * o.ld4 + c * 16, 0, CP);
  }
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

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

// PK: problems side by side in one workgroup (PK x 4 waves): the heads h0 .. h0 + PK - 1 of one
// group, whose rows are one contiguous PK x 256-byte piece of each token row (fp32 walk).
template <bool GATED, bool ROPE, bool ALIGNED, bool XH, int PK = 1>
__global__ __launch_bounds__(256 * PK) void attention_band_kernel(AttnParams p, int items) {
  static_assert(!(XH && ROPE), "fp16 input arrives rotated");
  static_assert(PK == 1 || PK == 2, "one or two heads side by side");
  constexpr bool kWalk = !XH;
  __shared__ __attribute__((aligned(16))) unsigned char lds_q[PK][64 * 128];
  __shared__ __attribute__((aligned(16))) unsigned char lds_k[PK][64 * 128];
  __shared__ __attribute__((aligned(16))) unsigned char lds_v[PK][64 * 128];
  // The walk (fp32 output): each wave's output rows on their way to whole-row stores.
  __shared__ __attribute__((aligned(16)))
  unsigned char lds_o[kWalk ? 4 * PK : 1][kWalk ? 4096 : 16];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Problem slot of this wave (its head h0 + ps) and its wave index within the slot.
  const int ps = PK > 1 ? wave >> 2 : 0, w4 = wave & 3;
  const int col = lane & 15, grp = lane >> 4;
  const int T = p.tokens;
  const long ts = p.tstep;
  constexpr unsigned kEsz = XH ? 2 : 4, kRowBytes = 64 * kEsz;
  const unsigned ldq4 = (unsigned)(ts * p.ldq * kEsz), ldk4 = (unsigned)(ts * p.ldk * kEsz),
                 ldv4 = (unsigned)(ts * p.ldv * kEsz);

  // Staging roles: q / k rows srow + 16*it at channels 4*sc of head slot hs; v key pairs
  // (2*(srow + 16*it), +1), it < 2 (32 threads a row of PK = 2 heads). fp16 input: q / k rows
  // xrow + 32*it as 16-byte chunks xc of head slot xhs (16 threads a row of 2 heads), v key pairs
  // at 8-byte channel groups sc of head slot hs. Rows at or past T read as 0.
  const int srow = PK > 1 ? tid >> 5 : tid >> 4, sc = tid & 15;
  const int hs = PK > 1 ? (tid >> 4) & 1 : 0;
  const int xrow = PK > 1 ? tid >> 4 : tid >> 3, xc = tid & 7;
  const int xhs = PK > 1 ? (tid >> 3) & 1 : 0;
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
    // The descriptor's base is wave-uniform (head h); a thread's head slot hs is a 256-byte
    // offset in its vector offset, which the range check covers (rows at or past T read 0: the
    // row stride is at least PK heads).
    auto rows_of = [&](const float* base, long ld, unsigned ld4) {
      return make_rsrc(reinterpret_cast<const unsigned char*>(base) + (row0 * ld + h * 64) * kEsz,
                       (unsigned)(T - 1) * ld4 + PK * kRowBytes);
    };
    const unsigned hoff = (unsigned)hs * kRowBytes, xhoff = (unsigned)xhs * kRowBytes;
    const rsrc_t qr = rows_of(p.q, p.ldq, ldq4);
    const rsrc_t kr = rows_of(p.k, p.ldk, ldk4);
    const rsrc_t vr = rows_of(p.v, p.ldv, ldv4);
    if constexpr (XH) {
#pragma unroll
      for (int it = 0; it < 2; it++) {
        const unsigned rr = (unsigned)(xrow + 32 * it);
        r.q[it] =
            __builtin_amdgcn_raw_buffer_load_b128(qr, rr * ldq4 + xhoff + xc * 16, 0, kStream);
        r.k[it] =
            __builtin_amdgcn_raw_buffer_load_b128(kr, rr * ldk4 + xhoff + xc * 16, 0, kStream);
      }
#pragma unroll
      for (int it = 0; it < 2; it++)
#pragma unroll
        for (int j = 0; j < 2; j++)
          r.v[it * 2 + j] = __builtin_amdgcn_raw_buffer_load_b64(
              vr, (unsigned)(2 * (srow + 16 * it) + j) * ldv4 + hoff + sc * 8, 0, kStream);
    } else {
#pragma unroll
      for (int it = 0; it < 4; it++) {
        const unsigned rr = (unsigned)(srow + 16 * it);
        r.q[it] = bload4<ALIGNED, kStream>(qr, rr * ldq4 + hoff + sc * 16);
        r.k[it] = bload4<ALIGNED, kStream>(kr, rr * ldk4 + hoff + sc * 16);
      }
#pragma unroll
      for (int it = 0; it < 2; it++)
#pragma unroll
        for (int j = 0; j < 2; j++)
          r.v[it * 2 + j] = bload4<ALIGNED, kStream>(
              vr, (unsigned)(2 * (srow + 16 * it) + j) * ldv4 + hoff + sc * 16);
    }
  };
  auto stage = [&](const BandRaw<XH>& r) {
    if constexpr (XH) {
#pragma unroll
      for (int it = 0; it < 2; it++) {
        const int off = k_offset(xrow + 32 * it, xc);
        *reinterpret_cast<u32x4*>(lds_q[xhs] + off) = r.q[it];
        *reinterpret_cast<u32x4*>(lds_k[xhs] + off) = r.k[it];
      }
#pragma unroll
      for (int it = 0; it < 2; it++)
#pragma unroll
        for (int j = 0; j < 4; j++)
          *reinterpret_cast<unsigned*>(lds_v[hs] + vtc_offset(sc * 4 + j, 2 * (srow + 16 * it))) =
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
        *reinterpret_cast<u32x2*>(lds_q[hs] + off) = u32x2{pack_h2(q.x, q.y), pack_h2(q.z, q.w)};
        *reinterpret_cast<u32x2*>(lds_k[hs] + off) = u32x2{pack_h2(k.x, k.y), pack_h2(k.z, k.w)};
      }
#pragma unroll
      for (int it = 0; it < 2; it++)
#pragma unroll
        for (int j = 0; j < 4; j++)
          *reinterpret_cast<unsigned*>(lds_v[hs] + vtc_offset(sc * 4 + j, 2 * (srow + 16 * it))) =
              pack_h2(comp(r.v[it * 2], j), comp(r.v[it * 2 + 1], j));
    }
  };

  const int q0 = w4 * 16;
  const int kq_base[2] = {k_offset(col, grp), k_offset(col, 4 + grp)};
  const int vsw = (col ^ (col >> 2)) & 7;
  const int v_base[2][2] = {{col * 128 + ((grp ^ vsw) << 4), col * 128 + ((grp ^ vsw ^ 4) << 4)},
                            {col * 128 + (((4 + grp) ^ vsw) << 4),
                             col * 128 + (((4 + grp) ^ vsw ^ 4) << 4)}};
  auto compute = [&](int g, int h) {
    const u32x4 qf[2] = {*reinterpret_cast<const u32x4*>(lds_q[ps] + kq_base[0] + w4 * 2048),
                         *reinterpret_cast<const u32x4*>(lds_q[ps] + kq_base[1] + w4 * 2048)};
    f32x4 s[4];
#pragma unroll
    for (int kb = 0; kb < 4; kb++) {
      s[kb] = zero4();
#pragma unroll
      for (int ds = 0; ds < 2; ds++)
        s[kb] = mfma16x16x32(*reinterpret_cast<const u32x4*>(lds_k[ps] + kq_base[ds] + kb * 2048),
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
            *reinterpret_cast<const u32x4*>(lds_v[ps] + v_base[ks][db & 1] + db * 2048), pf[ks],
            o[db]);
      lsum = mfma16x16x32(ones, pf[ks], lsum);
    }
    // Whole output rows per store: the fp32 walk (fp32 in and out) through the wave's LDS
    // area, fp16 input (fp16 out) through the wave's own query rows.
    if constexpr (kWalk)
      store_output_rows<GATED, ALIGNED, kStream>(out_rows(p, g, h + ps), o, lsum[0], q0, col, grp,
                                                 lane, lds_o[wave]);
    else
      store_output_rows_h<GATED, kStream>(out_rows(p, g, h + ps), o, lsum[0], q0, col, grp, lane,
                                          lds_q[ps] + w4 * 2048);
  };

  if constexpr (kWalk) {
    // Workgroup-uniform: every wave runs every step and reaches both barriers. The next loads
    // go out after the staging barrier and ahead of this problem's stores, so the wait before
    // the next staging leaves those stores outstanding. Past the end they reload the last
    // problem (unused), and a wave whose 16 queries all lie at or past T (T <= 48) computes
    // anyway (its q rows are zero; rows at or past T lie outside the output's buffer range, so
    // their stores are dropped): no branch around the loads and stores keeps the wait counts
    // fixed.
    // Item b: group b / (heads / PK), heads PK * (b % (heads / PK)) + 0 .. PK - 1.
    const int hpg = p.heads / PK;
    auto step = [&](int item, const BandRaw<XH>& cur, BandRaw<XH>& nxt) {
      stage(cur);
      __syncthreads();
      const int next = min(item + (int)gridDim.x, items - 1);
      load(next / hpg, PK * (next % hpg), nxt);
      compute(item / hpg, PK * (item % hpg));
      __syncthreads();  // the next step restages LDS
    };
    // The first step is peeled so the loop is entered with the same loads and stores
    // outstanding as each turn ends with (else the wait counts at the loop head are merged down
    // to a full drain).
    BandRaw<XH> a, b;
    int item = blockIdx.x;
    load(item / hpg, PK * (item % hpg), a);
    step(item, a, b);
    while (true) {
      item += gridDim.x;
      if (item >= items) break;
      step(item, b, a);
      item += gridDim.x;
      if (item >= items) break;
      step(item, a, b);
    }
  } else {
    // One item per workgroup: group g, heads h .. h + PK - 1 (pairs of heads as units).
    int g, h;
    band_problem(blockIdx.x, p.groups, p.heads / PK, g, h);
    h *= PK;
    BandRaw<XH> r;
    load(g, h, r);
    stage(r);
    __syncthreads();
    if (q0 < T) compute(g, h);
  }
}

// The fp32 walk: as many workgroups of 256 * PK threads as the CUs hold at once.
template <bool GATED, bool ROPE, bool ALIGNED, int PK>
static hipError_t launch_band_walk(const AttnParams& p, hipStream_t stream) {
  auto kernel = attention_band_kernel<GATED, ROPE, ALIGNED, false, PK>;
  const int items = p.groups * (p.heads / PK);
  static int per_cu = 0;
  if (per_cu <= 0 &&
      (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 256 * PK, 0) != hipSuccess ||
       per_cu <= 0))
    per_cu = 2 / PK;
  const long cap = (long)per_cu * device_cus();
  const int grid = cap < items ? (int)cap : items;
  hipLaunchKernelGGL(kernel, dim3(grid), dim3(256 * PK), 0, stream, p, items);
  return hipGetLastError();
}

template <bool GATED, bool ROPE, bool ALIGNED, bool XH = false>
static hipError_t launch_attention_t(const AttnParams& p, hipStream_t stream) {
  const int T = p.tokens;
  if (T > 64) return launch_attention_long(p, GATED, ROPE, ALIGNED, stream);
  if constexpr (!XH) {
    // Two heads side by side where the head count is even (each token row's two head slices
    // are one contiguous 512-byte piece), one problem per slot otherwise.
    if (p.heads % 2 == 0) return launch_band_walk<GATED, ROPE, ALIGNED, 2>(p, stream);
    return launch_band_walk<GATED, ROPE, ALIGNED, 1>(p, stream);
  } else {
    // One item (one or two heads of a group) per workgroup.
    if (p.heads % 2 == 0) {
      const int items = p.groups * (p.heads / 2);
      hipLaunchKernelGGL((attention_band_kernel<GATED, ROPE, ALIGNED, XH, 2>), dim3(items),
                         dim3(512), 0, stream, p, items);
    } else {
      const int items = p.groups * p.heads;
      hipLaunchKernelGGL((attention_band_kernel<GATED, ROPE, ALIGNED, XH>), dim3(items), dim3(256),
                         0, stream, p, items);
    }
    return hipGetLastError();
  }
}

bool attention_grid_fits(size_t groups, size_t tokens, size_t heads) {
  const size_t problems = groups * heads;
  if (groups != 0 && problems / groups != heads) return false;
  // T <= 64: one 256-thread workgroup per problem at most. T > 64: the long-sequence kernel's
  // 512-query passes are counted in an int (its grid is at most twice the CU count).
  const size_t blocks = tokens <= 64 ? problems : problems * ((tokens + 511) / 512);
  const size_t threads = tokens <= 64 ? 256 : 1024;
  return blocks < (size_t(1) << 31) && (tokens > 64 || blocks * threads < (size_t(1) << 32));
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
