// Fused attention over long sequences (the time axis, T > 64: 801 frames for Mel-RoFormer,
// 1101 for BS-RoFormer) on v_mfma_f32_32x32x16_f16. Same operation and boundary as
// attention.hip (crates/ancha-models/src/fused/attention.rs:26-227): softmax(q.k^T).v per
// (group, head), optional interleaved RoPE on load, optional per-head sigmoid gate.
//
// Work unit ("pass") = 512 queries of one (group, head): 16 waves x 32 queries; each 64-key tile
// is staged once into LDS as fp16 (K rotated on the way) and read by all 16 waves. Workgroups
// are persistent, one per CU, and walk the passes in rounds; the walk is pipelined so that a
// pass starts with its inputs already on chip: while a pass runs its K/V tiles, each wave
// prefetches the next pass's 32 query rows (fp32 inputs: rows plus their rotary table rows, in
// 4-row chunks landing in LDS by direct buffer loads, rotated and packed to fp16 at the end of
// the step), and the next pass's first K/V tile loads beside this pass's epilogue. Output rows
// are stored after the step's loads have landed, so they drain behind the next pass. Within a
// step the next tile's K / V rows are requested first and its table rows (and the query chunk)
// after the first 32-key block, so the 16 waves' requests do not all queue at once.
//
// The softmax VALU work (exp2, max, fp16 packing) costs about as many cycles as the MFMAs, so
// the kernel is built for overlap: at most 128 VGPRs, which puts four waves on every SIMD, one
// wave's softmax running beside another's MFMAs.
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
// Prefetch of the next pass's query rows, one chunk per K/V step: fp32 inputs in 8 chunks of 4
// rows (each with its cos and sin table rows: 3 x 1 KB per wave), fp16 inputs in 4 chunks of 8
// rows (1 KB per wave, loaded straight into place).
template <bool XH>
constexpr int kChunks = XH ? 4 : 8;

// Byte offset of 16-byte chunk c (0..7) of row r in a tile of 128-byte rows (K: row = key; a
// wave's queries: row = query; V^T has its own layout below). Chunks are XOR-swizzled by
// (r >> 1) & 7,
// so the 16 lanes that one LDS cycle serves (rows r .. r + 15 of a fragment read, two rows per
// 256-byte bank line) land on 16 different bank groups.
__device__ __forceinline__ int row_offset(int r, int c) { return r * 128 + ((c ^ ((r >> 1) & 7)) << 4); }

// Position of key k (0..63) in a V^T row: bits 2 and 3 swapped, so each 16-key step holds keys
// 0-3, 8-11, 4-7, 12-15 (kPerm16 order) and a lane's 8 keys are one contiguous 16-byte chunk.
__device__ __forceinline__ int v_position(int k) {
  return (k & 0x33) | ((k & 4) << 1) | ((k & 8) >> 1);
}

// Byte offset of 16-byte chunk c of V^T row r (a channel): rows r and r ^ 1 trade places when
// bit 2 of r is set, and the chunk is XOR-swizzled by (r3, r1 ^ r4, r2 ^ r5). Two rows share a
// 256-byte line of the 64 banks, so a 16-byte access's bank group is (physical row & 1, chunk):
// the 16 lanes that one LDS cycle of the fragment reads serves (rows 16m .. 16m + 15, one
// chunk) and the 32 lanes that one cycle of the staging writes serves (rows 4i + w, i < 16, one
// dword of one of two chunks per row) both land on distinct bank groups. Rows 32 + r sit 4 KB
// after row r with chunk bit 2 flipped.
__device__ __forceinline__ int vt_row_offset(int r, int c) {
  const int sw = ((r >> 3) & 1) | ((((r >> 1) ^ (r >> 4)) & 1) << 1) | ((((r >> 2) ^ (r >> 5)) & 1) << 2);
  return (r ^ ((r >> 2) & 1)) * 128 + ((c ^ sw) << 4);
}

// Byte offset of the dword holding positions pos, pos + 1 (pos even) of V^T row ch.
__device__ __forceinline__ int v_offset(int ch, int pos) {
  return vt_row_offset(ch, pos >> 3) + (pos & 7) * 2;
}

// The value of lane l ^ 32 (the partner in the other half of the wave).
__device__ __forceinline__ unsigned half_partner(unsigned x, bool upper) {
  const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  const unsigned a = r[0], b = r[1];
  return upper ? a : b;
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

// Zero accumulator built in place by asm moves: a value of its own in every pass (the compiler
// cannot hoist it out of the pass loop and hold it in registers across the walk), and a
// register C operand, so the MFMA it starts is tied to it (see mfma32_zero).
__device__ __forceinline__ f32x16 zero16() {
  f32x2 a[8];
#pragma unroll
  for (int i = 0; i < 8; i++) asm volatile("v_mov_b64 %0, 0" : "=v"(a[i]));
  const f32x4v b[4] = {__builtin_shufflevector(a[0], a[1], 0, 1, 2, 3),
                       __builtin_shufflevector(a[2], a[3], 0, 1, 2, 3),
                       __builtin_shufflevector(a[4], a[5], 0, 1, 2, 3),
                       __builtin_shufflevector(a[6], a[7], 0, 1, 2, 3)};
  const f32x8 c0 = __builtin_shufflevector(b[0], b[1], 0, 1, 2, 3, 4, 5, 6, 7);
  const f32x8 c1 = __builtin_shufflevector(b[2], b[3], 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_shufflevector(c0, c1, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15);
}

// LDS-direct buffer load: each lane's 16 bytes at `off` land at dst + 16 * lane.
template <int CP = 0>
__device__ __forceinline__ void load_lds16(rsrc_t r, unsigned char* dst, unsigned off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16,
                                           off, 0, 0, CP);
}

// The same with 4 bytes per lane: lane l's dword at `off` lands at dst + 4 * l.
__device__ __forceinline__ void load_lds4(rsrc_t r, unsigned char* dst, unsigned off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 4,
                                           off, 0, 0, 0);
}

// ALIGNED: q / k / v rows and the output are 16-byte aligned (every call the library itself
// makes); otherwise their accesses are 4-byte ones (rows of an odd column count, e.g. a packed
// projection with 1549 columns), with the same tiles and walk. TALIGNED: the same for the
// rotary table.
template <bool GATED, bool ROPE, bool XH, bool ALIGNED, bool TALIGNED = ALIGNED>
__global__ __launch_bounds__(kWaves * 64, 1) void attention_long_kernel(AttnParams p, int qblocks,
                                                                        int passes) {
  // K tile: row = key (128 bytes of fp16 channels); V^T tile: row = channel (64 keys in
  // v_position order). Double buffered, the buffer index running on across passes.
  __shared__ __attribute__((aligned(16))) unsigned char lds_k[2][64 * 128];
  __shared__ __attribute__((aligned(16))) unsigned char lds_v[2][64 * 128];
  // Each wave's 32 queries of the next pass (fp16 rows), read into registers when it starts.
  __shared__ __attribute__((aligned(16))) unsigned char lds_q[kWaves][32 * 128];
  // fp32 inputs: one prefetched chunk per wave (4 query rows, their cos rows, their sin rows).
  __shared__ __attribute__((aligned(16))) unsigned char lds_raw[XH ? 1 : kWaves][XH ? 16 : 3072];
  constexpr int kCh = kChunks<XH>;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grid = gridDim.x;
  const int lb = xcd_remap(blockIdx.x, grid);
  const long ts = p.tstep;
  constexpr unsigned kEsz = XH ? 2 : 4, kRowBytes = 64 * kEsz;
  const int ntiles = (p.tokens + 63) / 64;
  // Passes run in rounds of `grid`; odd rounds walk backwards, so a workgroup alternates between
  // the full and the partial query blocks of a (group, head) and both halves of one (group,
  // head) run side by side on neighbouring workgroups of one XCD (shared K / V in its L2).
  //
  // Two query blocks per (group, head) (T = 513 .. 1024) when the rounds do not come out even:
  // the workgroups with one pass more than the others should get the cheap partial blocks. Each
  // XCD's workgroups split into halves B and A; in every full round, B workgroup jj runs the full
  // block and A workgroup jj the partial block of one (group, head) of the same XCD; the
  // leftover (group, head) problems then run on A workgroups only, two neighbours per problem.
  // B ends with full rounds only, A with one pass more, most of them partial (at T = 801 and 960
  // problems on 256 CUs: A 7 partial + 1 against 4 full + 4 partial for the alternating walk).
  // The partial side gains ~7 % of a pass per round on its partner, so after the first rounds
  // the two reads of a K / V stream no longer meet in L2: the balance is worth more here.
  // When the rounds come out even the alternating walk is the balanced one and stays.
  const int xcd_wgs = grid / kXcds, pair_half = xcd_wgs / 2, pairs = grid / 2;
  const int problems = passes / 2, full_rounds = qblocks == 2 ? problems / pairs : 0;
  const int leftover = problems - full_rounds * pairs;
  const bool paired = qblocks == 2 && grid % (2 * kXcds) == 0 && passes > 2 * grid &&
                      leftover > 0 && 2 * leftover <= pairs;
  const int px = lb / (xcd_wgs > 0 ? xcd_wgs : 1), pj = lb % (xcd_wgs > 0 ? xcd_wgs : 1);
  const bool pa = pj >= pair_half;
  const int pjj = pa ? pj - pair_half : pj;
  auto pass_of = [&](int rnd) -> long {
    if (paired) {
      if (rnd < full_rounds) {
        const long problem = ((long)rnd * kXcds + px) * pair_half + pjj;
        return 2 * problem + (pa ? 1 : 0);
      }
      const int idx = px * pair_half + pjj;
      if (rnd > full_rounds || !pa || idx >= 2 * leftover) return passes;
      return 2 * ((long)full_rounds * pairs + idx / 2) + (idx & 1);
    }
    return (long)rnd * grid + ((rnd & 1) ? grid - 1 - lb : lb);
  };
  // Per-pass opaque copies (set at the top of every pass): the compiler cannot hoist values
  // derived from them out of the pass loop and hold them in registers across the whole walk.
  int T = p.tokens, lane = tid & 63, tid_o = tid;
  unsigned ldq4 = (unsigned)(ts * p.ldq * kEsz), ldk4 = (unsigned)(ts * p.ldk * kEsz),
           ldv4 = (unsigned)(ts * p.ldv * kEsz);

  // K / V staging: thread -> channels 4 sc .. 4 sc + 3 of K row skey and of V row vkey (16
  // threads read one 256-byte fp32 row). A wave's four K rows are tid / 16 in order; its four V
  // rows the same with bits 0 and 1 of tid / 16 swapped, so that lanes l and l ^ 32 hold keys 2i
  // and 2i + 1: V^T dwords pair them, and each lane writes two channels of its key pair (even
  // key: 4 sc, 4 sc + 1; odd key: 4 sc + 2, 4 sc + 3) after trading halves with its partner.
  // A write instruction's 32 lanes then cover both key pairs of the wave.
  float4 kx = {}, kc = {}, ks = {}, vx = {};
  u32x2 kh = {}, vh = {};
  // parts: 0 = K / V and the key table rows, 1 = K / V only, 2 = the table rows only.
  auto load_tile = [&](const unsigned char* kbase, const unsigned char* vbase, int key0,
                       int parts) {
    const int skey = tid_o >> 4, sc = tid_o & 15;
    const int vkey = (skey & ~3) | ((skey & 1) << 1) | ((skey >> 1) & 1);
    const unsigned rows = (unsigned)(T - key0);
    if (parts != 2) {
      const rsrc_t kr = make_rsrc(kbase + (long)key0 * ldk4, (rows - 1) * ldk4 + kRowBytes);
      const rsrc_t vr = make_rsrc(vbase + (long)key0 * ldv4, (rows - 1) * ldv4 + kRowBytes);
      if constexpr (XH) {
        kh = __builtin_amdgcn_raw_buffer_load_b64(kr, (unsigned)skey * ldk4 + sc * 8, 0, 0);
        vh = __builtin_amdgcn_raw_buffer_load_b64(vr, (unsigned)vkey * ldv4 + sc * 8, 0, 0);
      } else {
        kx = bload4<ALIGNED>(kr, (unsigned)skey * ldk4 + sc * 16);
        vx = bload4<ALIGNED>(vr, (unsigned)vkey * ldv4 + sc * 16);
      }
    }
    if constexpr (ROPE && !XH) {
      if (parts != 1) {
        // Key cos rows (table 2) and sign-folded sin rows (table 3) of this tile.
        const rsrc_t cr = make_rsrc(p.rope + (long)(2 * T + key0) * 64, rows * 256);
        const rsrc_t sr = make_rsrc(p.rope + (long)(3 * T + key0) * 64, rows * 256);
        kc = bload4<TALIGNED>(cr, (unsigned)skey * 256 + sc * 16);
        ks = bload4<TALIGNED>(sr, (unsigned)skey * 256 + sc * 16);
      }
    }
  };
  auto store_tile = [&](int buf) {
    const int skey = tid_o >> 4, sc = tid_o & 15;
    const int vkey = (skey & ~3) | ((skey & 1) << 1) | ((skey >> 1) & 1);
    const bool odd = (vkey & 1) != 0;
    const int vch = 4 * sc + 2 * (int)odd, vpos = v_position(vkey & ~1);
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
    const unsigned other = half_partner(odd ? vw[0] : vw[1], odd);
    const unsigned lo = odd ? other : vw[0], hi = odd ? vw[1] : other;
    unsigned char* V = lds_v[buf];
    *reinterpret_cast<unsigned*>(V + v_offset(vch, vpos)) =
        __builtin_amdgcn_perm(hi, lo, 0x05040100u);
    *reinterpret_cast<unsigned*>(V + v_offset(vch + 1, vpos)) =
        __builtin_amdgcn_perm(hi, lo, 0x07060302u);
  };

  // Query rows q0 .. q0 + 31 of (row0, head h); the buffer range ends at row T - 1, so rows
  // past the sequence read as zeros.
  auto query_rsrc = [&](long row0, int h, int q0) {
    const unsigned rows = (unsigned)(T - q0);
    return make_rsrc(reinterpret_cast<const unsigned char*>(p.q) +
                         ((row0 + (long)q0 * ts) * p.ldq + h * 64) * kEsz,
                     (rows - 1) * ldq4 + kRowBytes);
  };
  // This wave's 32 query rows, rotated, times log2(e) (fp32 inputs), fp16, into its LDS rows;
  // all at once (the first pass of the walk, and sequences too short to prefetch).
  auto stage_queries = [&](long row0, int h, int q0) {
    unsigned char* Q = lds_q[wave];
    const rsrc_t qr = query_rsrc(row0, h, q0);
    const unsigned rows = (unsigned)(T - q0);
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
        float4 x = bload4<ALIGNED>(qr, (unsigned)r * ldq4 + c * 16);
        if constexpr (ROPE)
          x = rotate4(x, bload4<TALIGNED>(cr, (unsigned)r * 256 + c * 16),
                      bload4<TALIGNED>(sr, (unsigned)r * 256 + c * 16));
        x = scale4(x, kLog2e);
        *reinterpret_cast<u32x2*>(Q + row_offset(r, c >> 1) + ((c & 1) << 3)) =
            u32x2{pack_h2(x.x, x.y), pack_h2(x.z, x.w)};
      }
    }
  };
  // Chunk c of the prefetch: direct-to-LDS loads, completed by the step's vmcnt wait.
  auto issue_chunk = [&](long row0, int h, int q0, int c) {
    int lane = tid & 63;
    asm volatile("" : "+v"(lane));
    const rsrc_t qr = query_rsrc(row0, h, q0);
    if constexpr (XH) {
      // Rows 8 c .. 8 c + 7 straight into their swizzled place: LDS slot l of the chunk holds
      // row 8 c + l / 8, stored chunk l % 8 = logical chunk (l % 8) ^ ((row >> 1) & 7).
      const int r = 8 * c + (lane >> 3);
      const int cc = (lane & 7) ^ ((r >> 1) & 7);
      load_lds16<kStream>(qr, lds_q[wave] + 1024 * c, (unsigned)r * ldq4 + cc * 16);
    } else if constexpr (ALIGNED) {
      // Rows 4 c + l / 16, 16-byte piece l % 16: query row, then cos and sin table rows.
      const int r = 4 * c + (lane >> 4), cc = lane & 15;
      unsigned char* R = lds_raw[wave];
      load_lds16<kStream>(qr, R, (unsigned)r * ldq4 + cc * 16);
      if constexpr (ROPE) {
        const unsigned rows = (unsigned)(T - q0);
        const rsrc_t cr = make_rsrc(p.rope + (long)q0 * 64, rows * 256);
        const rsrc_t sr = make_rsrc(p.rope + (long)(T + q0) * 64, rows * 256);
        load_lds16(cr, R + 1024, (unsigned)r * 256 + cc * 16);
        load_lds16(sr, R + 2048, (unsigned)r * 256 + cc * 16);
      }
    } else {
      // Query rows as four dword loads, row 4 c + i each (lane l: float l): the same LDS layout;
      // the table rows as above when the table is aligned.
      unsigned char* R = lds_raw[wave];
      const unsigned rows = (unsigned)(T - q0);
      const rsrc_t cr = make_rsrc(ROPE ? p.rope + (long)q0 * 64 : p.q, ROPE ? rows * 256 : 0);
      const rsrc_t sr = make_rsrc(ROPE ? p.rope + (long)(T + q0) * 64 : p.q, ROPE ? rows * 256 : 0);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const unsigned r = (unsigned)(4 * c + i);
        load_lds4(qr, R + 256 * i, r * ldq4 + lane * 4);
        if constexpr (ROPE && !TALIGNED) {
          load_lds4(cr, R + 1024 + 256 * i, r * 256 + lane * 4);
          load_lds4(sr, R + 2048 + 256 * i, r * 256 + lane * 4);
        }
      }
      if constexpr (ROPE && TALIGNED) {
        const int r = 4 * c + (lane >> 4), cc = lane & 15;
        load_lds16(cr, R + 1024, (unsigned)r * 256 + cc * 16);
        load_lds16(sr, R + 2048, (unsigned)r * 256 + cc * 16);
      }
    }
  };
  // fp32: rotate, scale and pack the landed chunk into the wave's fp16 query rows.
  auto convert_chunk = [&](int c) {
    if constexpr (!XH) {
      int lane = tid & 63;
      asm volatile("" : "+v"(lane));
      const int r = 4 * c + (lane >> 4), cc = lane & 15;
      const unsigned char* R = lds_raw[wave];
      float4 x = __builtin_bit_cast(float4, lds16(R + 16 * lane));
      if constexpr (ROPE)
        x = rotate4(x, __builtin_bit_cast(float4, lds16(R + 1024 + 16 * lane)),
                    __builtin_bit_cast(float4, lds16(R + 2048 + 16 * lane)));
      x = scale4(x, kLog2e);
      *reinterpret_cast<u32x2*>(lds_q[wave] + row_offset(r, cc >> 1) + ((cc & 1) << 3)) =
          u32x2{pack_h2(x.x, x.y), pack_h2(x.z, x.w)};
    }
  };

  // Prologue of the walk: the first pass's queries and first K / V tile.
  {
    const int pi = (int)pass_of(0);
    const int qblk = pi % qblocks, gh = pi / qblocks;
    const int h = gh % p.heads, g = gh / p.heads;
    const long row0 = group_row(p, g);
    const int q0 = qblk * kQueries + wave * 32;
    if (q0 < T) stage_queries(row0, h, q0);
    load_tile(reinterpret_cast<const unsigned char*>(p.k) + (row0 * p.ldk + h * 64) * kEsz,
              reinterpret_cast<const unsigned char*>(p.v) + (row0 * p.ldv + h * 64) * kEsz, 0, 0);
    store_tile(0);
    __builtin_amdgcn_s_waitcnt(kWaitVmem);
    __syncthreads();
  }

  int buf = 0;  // LDS buffer holding the current tile
  for (int rnd = 0;; rnd++) {
    const long pl = pass_of(rnd);
    if (pl >= passes) break;
    const int pi = (int)pl;
    const long pnl = pass_of(rnd + 1);
    const bool has_next = pnl < passes;
    const int pn = has_next ? (int)pnl : pi;
    T = p.tokens;
    lane = tid & 63;
    tid_o = tid;
    asm volatile("" : "+s"(T), "+s"(ldq4), "+s"(ldk4), "+s"(ldv4), "+v"(lane), "+v"(tid_o));
    const int half = lane >> 5, col = lane & 31;

    const int qblk = pi % qblocks, gh = pi / qblocks;
    const int h = gh % p.heads, g = gh / p.heads;
    const long row0 = group_row(p, g);
    const unsigned char* kbase =
        reinterpret_cast<const unsigned char*>(p.k) + (row0 * p.ldk + h * 64) * kEsz;
    const unsigned char* vbase =
        reinterpret_cast<const unsigned char*>(p.v) + (row0 * p.ldv + h * 64) * kEsz;
    const int q0 = qblk * kQueries + wave * 32;
    const bool active = q0 < T;
    // The next pass (this workgroup's next round).
    const int qblkn = pn % qblocks, ghn = pn / qblocks;
    const int hn = ghn % p.heads, gn = ghn / p.heads;
    const long row0n = group_row(p, gn);
    const int q0n = qblkn * kQueries + wave * 32;
    const bool active_n = has_next && q0n < T;
    // The prefetch takes the last kCh K / V steps of the pass.
    const bool prefetch = active_n && ntiles - 1 >= kCh;
    const int cstart = ntiles - 1 - kCh;

    // This wave's queries as B fragments of S^T = K.Q^T: fragment ds = query q0 + (l % 32),
    // channels 16 ds + 8 (l / 32) .. + 7. LDS operations of one wave complete in order: these
    // reads see the rows staged before, and precede this pass's prefetch into the same rows.
    // Per-lane LDS offsets: K fragment (kb, ds) = keys 32 kb + (l % 32), chunk 2 ds + l / 32;
    // V^T fragment (db, kb, k2) = channel 32 db + (l % 32), chunk 4 kb + 2 k2 + l / 32. Both are
    // chunk 2 i + l / 32 of row l % 32 (i = ds, or 2 kb + k2), plus 4096 per 32 rows (in the V^T
    // layout, chunk 2 (i ^ 2) + l / 32 of the row 32 below).
    int fq[4], fv[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      fq[i] = row_offset(col, 2 * i + half);
      fv[i] = vt_row_offset(col, 2 * i + half);
    }
    u32x4 qf[4];
    if (active) {
#pragma unroll
      for (int ds = 0; ds < 4; ds++) qf[ds] = lds16(lds_q[wave] + fq[ds]);
    }

    f32x16 o[2];  // O^T: channel 32 db + 8 i + 4 (l / 32) + e of query l % 32 in o[db][4 i + e]
    o[0] = zero16();
    o[1] = zero16();
    float negm = 0.f, lsum = 0.f;  // -(running maximum), this lane's share of the row sum
    // fp16 input (109 registers otherwise): -m held in a register tuple, the C operand of every
    // block's first score MFMA, rebuilt only when the running maximum moves; fp32 input (119)
    // builds it per block.
    constexpr bool kSeedReg = XH;
    f32x16 sd = {};
    // The running maximum starts at the exact maximum over the first 32 keys (T > 64); their
    // scores are kept for the first block, which then needs no score MFMAs of its own.
    f32x16 s0 = zero16();
    if (active) {
#pragma unroll
      for (int ds = 0; ds < 4; ds++) s0 = mfma32(lds16(lds_k[buf] + fq[ds]), qf[ds], s0);
      float mx = fmaxf(fmaxf(s0[0], s0[1]), s0[2]);
#pragma unroll
      for (int r = 3; r < 15; r += 2) mx = fmaxf(fmaxf(mx, s0[r]), s0[r + 1]);
      negm = -pair_max(fmaxf(mx, s0[15]));
      if constexpr (kSeedReg) sd = seed16(negm);
    }

    // One 32-key block kb of the tile in buffer b. MASK: keys at or past T may be present.
    // FIRST: the pass's first block, whose scores s0 are already computed (shifted here).
    auto block = [&](auto mask_tag, int b, int kb, int key0, auto first_tag) {
      constexpr bool MASK = decltype(mask_tag)::value;
      constexpr bool FIRST = decltype(first_tag)::value;
      const unsigned char* K = lds_k[b] + kb * 4096;
      f32x16 s;
      if constexpr (FIRST) {
        s = s0 + negm;
      } else {
        if constexpr (kSeedReg) {
          s = mfma32(lds16(K + fq[0]), qf[0], sd);
#pragma unroll
          for (int ds = 1; ds < 4; ds++) s = mfma32(lds16(K + fq[ds]), qf[ds], s);
        } else {
          s = seed16(negm);
#pragma unroll
          for (int ds = 0; ds < 4; ds++) s = mfma32(lds16(K + fq[ds]), qf[ds], s);
        }
      }
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
          if constexpr (kSeedReg) sd = seed16(negm);
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
      const unsigned char* V = lds_v[b];
#pragma unroll
      for (int k2 = 0; k2 < 2; k2++)
#pragma unroll
        for (int db = 0; db < 2; db++)
          o[db] = mfma32(lds16(V + db * 4096 + fv[(2 * kb + k2) ^ (2 * db)]), pf[k2], o[db]);
    };

    for (int j = 0; j + 1 < ntiles; j++) {
      // The next tile's K / V rows first; its table rows and the query chunk after the first
      // block, so that the 16 waves' loads do not all queue at the start of the step.
      load_tile(kbase, vbase, (j + 1) * 64, 1);
      const int c = j - cstart;
      if (active) {
        if (j == 0)
          block(std::false_type{}, buf, 0, 0, std::true_type{});
        else
          block(std::false_type{}, buf, 0, j * 64, std::false_type{});
      }
      load_tile(kbase, vbase, (j + 1) * 64, 2);
      if (prefetch && c >= 0) issue_chunk(row0n, hn, q0n, c);
      if (active) block(std::false_type{}, buf, 1, j * 64, std::false_type{});
      __builtin_amdgcn_s_waitcnt(kWaitVmem);
      if (prefetch && c >= 0) convert_chunk(c);
      store_tile(buf ^ 1);
      __syncthreads();
      buf ^= 1;
    }

    // Last tile of this pass (keys at or past T masked; a fully masked block adds zeros). The
    // next pass's first tile loads after its blocks, beside this pass's epilogue.
    if (active) {
      const int j = ntiles - 1;
      block(std::true_type{}, buf, 0, j * 64, std::false_type{});
      block(std::true_type{}, buf, 1, j * 64, std::false_type{});
    }
    if (has_next)
      load_tile(reinterpret_cast<const unsigned char*>(p.k) + (row0n * p.ldk + hn * 64) * kEsz,
                reinterpret_cast<const unsigned char*>(p.v) + (row0n * p.ldv + hn * 64) * kEsz,
                0, 0);
    float scale = 0.f, gl = 0.f;
    const OutRows out = out_rows(p, g, h);
    if (active) {
      scale = 1.0f / pair_sum(lsum);
      if constexpr (GATED) {
        const int t = q0 + col;
        gl = out.gate_half ? (float)__builtin_bit_cast(
                                 _Float16, __builtin_amdgcn_raw_buffer_load_b16(
                                               out.gate, (unsigned)t * out.ldg4, 0, 0))
                           : bload1(out.gate, (unsigned)t * out.ldg4);
      }
    }
    __builtin_amdgcn_s_waitcnt(kWaitVmem);
    if (has_next) store_tile(buf ^ 1);
    if (active_n && !prefetch) stage_queries(row0n, hn, q0n);
    if (active) {
      // Epilogue: 1/l (and the gate), then this lane's channels 32 db + 8 i + 4 (l / 32) .. + 3
      // of query q0 + (l % 32). Rows at or past T are dropped by the range check. Issued after
      // the wait above, so the stores drain while the next pass runs.
      if constexpr (GATED) scale = scale / (1.0f + expf(-gl));
      const int t = q0 + col;
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
            bstore4<ALIGNED>(out.out, (unsigned)t * out.ld4 + c * 4, v);
        }
    }
    // The next pass's first tile and query rows are in place; this pass's tiles are free.
    __syncthreads();
    buf ^= 1;
  }
}

template <bool GATED, bool ROPE, bool XH, bool ALIGNED = true, bool TALIGNED = ALIGNED>
hipError_t launch_t(const AttnParams& p, hipStream_t stream) {
  const int qblocks = (p.tokens + kQueries - 1) / kQueries;
  const int passes = p.groups * p.heads * qblocks;
  // One workgroup per CU walks the passes when there are more than two rounds of them; fewer
  // passes run one per workgroup (the walk would only lengthen the critical path).
  const int cus = device_cus();
  const int grid = passes <= 2 * cus ? passes : cus;
  hipLaunchKernelGGL((attention_long_kernel<GATED, ROPE, XH, ALIGNED, TALIGNED>), dim3(grid),
                     dim3(kWaves * 64), 0, stream, p, qblocks, passes);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_attention_long(const AttnParams& p, bool gated, bool rope, bool aligned,
                                 hipStream_t stream) {
  if (p.tokens <= 64) return hipErrorInvalidValue;
  if (p.in_half) {
    if (!gated || rope || !aligned) return hipErrorInvalidValue;
    return launch_t<true, false, true>(p, stream);
  }
  if (!aligned) {
    // Rows not 16-byte aligned; the table (256-byte rows) is aligned when its base is.
    const bool table_aligned = (reinterpret_cast<uintptr_t>(p.rope) & 15) == 0;
    if (rope)
      return gated ? (table_aligned ? launch_t<true, true, false, false, true>(p, stream)
                                    : launch_t<true, true, false, false, false>(p, stream))
                   : (table_aligned ? launch_t<false, true, false, false, true>(p, stream)
                                    : launch_t<false, true, false, false, false>(p, stream));
    return gated ? launch_t<true, false, false, false>(p, stream)
                 : launch_t<false, false, false, false>(p, stream);
  }
  if (gated) return rope ? launch_t<true, true, false>(p, stream) : launch_t<true, false, false>(p, stream);
  return rope ? launch_t<false, true, false>(p, stream) : launch_t<false, false, false>(p, stream);
}

}  // namespace ancha
