// Quantized matrix-vector product, one row (decode, M = 1):
// out[N] = x[K] . deq(W[N, K])^T.  The reference's M = 1 path is
// mx.quantized_matmul -> MLX qmv (mlxturbo/kernels/dispatch.py:317-327,
// fast_qmm.py:360-362); config 2's M = 1 is the north-star shape.
//
// The layout follows how the MI355X memory system streams a one-pass read,
// measured with read-only kernels over config 2's 44.6 MB of weights:
//
//  * A wave owns a quad of 4 weight rows over its K range.  Load instruction
//    s of the quad reads 256 contiguous bytes of each of the 4 rows (lane
//    4b + j: row j, bytes 256 s + 16 b): whole 128-byte lines, non-temporal.
//    That pattern read in 8.0 us, as fast as a contiguous read (7.8); 16
//    rows x 64 bytes per instruction (half lines, the 16-row skinny tile's
//    B operand) took 9.0, and 11.9 with the non-temporal bit.
//  * Waves deal evenly over the SIMDs.  With too few quads, K is split over
//    KS waves of a workgroup whose partial sums meet in LDS.  With many, one
//    wave per quad leaves a partial last round: K=5120 N=17408 is 4352 quads
//    on 1024 SIMDs, 4 waves each and a fifth on a quarter of them, and the
//    kernel is VALU-bound per SIMD (about 950 VALU per wave), so those SIMDs
//    set the time.  The leftover quads (quads mod 4 x CUs) are then split W
//    ways (W = 2 or 4 waves per workgroup, the full quads W to a workgroup,
//    one wave each): every SIMD gets 4 whole quads and a quarter of one
//    (11.5-12.0 against 12.6-13.1 us).
//  * The scales and biases of the wave's groups are copied into the wave's
//    LDS once, with 16-byte loads (per-instruction 4-byte scale loads cost
//    2.1 us of a 10 us read, the copy 0.9).
//  * x is read as one coalesced slab per instruction (lane l: the 8 codes
//    at 8 l for 4-bit, 4 codes at 4 l for 8-bit), not staged: lane 4b + p
//    then holds the x codes of word p of every lane of its 4-lane block.  In
//    v_mfma_f32_4x4x4_16b, output row i of block b pairs lane 4b + i's A with
//    lane 4b + j's B, so with each lane's own x piece as A, row p of the
//    product of word p is the right pairing: word p goes to accumulator p,
//    whose row p is kept (the other rows pair mismatched codes and are
//    discarded).
//  * Exact per-weight dequantization (mq_common.h), rounded to T as MLX's
//    dequantize does; a wave whose scales hold |s| >= 2^100 (or inf / NaN)
//    runs the plain float route instead, found once in the scale copy (a
//    per-instruction check costs a branch per instruction).
//  * The kept rows are summed in class order, then over the 16 lanes of a
//    row in a fixed tree (DPP rotations within each 16-lane row, then xor 16
//    and 32), then over the K split in wave order; one rounding.  The K split depends on (N, K, bits, group_size) and the
//    device's CU count only.
//
// Calls of 2+ rows run the 16-row skinny family (qmv.cuh): a 4 x 4 block
// product over x rows read per lane (64 bytes per lane per instruction)
// measured 20-28 us at K=5120 N=17408 M=2-4 against 14-15 there, and one
// class-form product per x row 15-20 us (M x the MFMAs and x slabs), so
// rows of one call are bit-identical across M = 2..32 but M = 1 rounds its
// own sums (the same values within the output tolerance).
//
// The accumulators must live in VGPRs: with AGPR accumulators the compiler
// moved all four through one AGPR block with v_accvgpr copies (8 extra VALU
// per word, 13.6 against 11.6 us), so this file's translation unit is built
// with -mllvm -amdgpu-mfma-vgpr-form.
#pragma once
#include <type_traits>

#include "launch.h"

namespace mq {

typedef short qq_s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 qq_f16x4 __attribute__((ext_vector_type(4)));

template <int DT>
__device__ __forceinline__ f32x4 quad_mfma(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1,
                                           f32x4 c) {
  const u32x2 a = {a0, a1}, b = {b0, b1};
  if constexpr (DT == kBF16)
    return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(qq_s16x4, a),
                                                   __builtin_bit_cast(qq_s16x4, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(qq_f16x4, a),
                                              __builtin_bit_cast(qq_f16x4, b), c, 0, 0, 0);
}

// Geometry of one load instruction of a quad.
template <int BITS, int GS>
struct QuadGeom {
  static constexpr int RB = 256;                    // bytes of each row per instruction
  static constexpr int CPI = RB * 8 / BITS;         // codes per instruction (per row)
  static constexpr int GPI = CPI / GS;              // groups per instruction
  static constexpr int XB = 2 * CPI / 64;           // x bytes per lane per slab: 16 / 8
  static_assert(GS * BITS / 8 >= 16, "a 16-byte lane piece lies in one group");
};

// Largest K split (waves per quad).
constexpr int kQuadMaxKS = 8;
// 16-byte chunks of the scale copy per lane (the kernel's SB: 1 or 2): a
// row's chunks <= 16 x SB.
constexpr int kQuadMaxSb = 2;
// Load instructions in flight ahead of the one computed.  Two keep the
// kernel at 72 VGPRs (7 waves per SIMD); three and four needed 91-99 (4-5
// waves per SIMD) and ran 0-20% slower (K=5120 N=17408, one process).
constexpr int kQuadDepth = 2;

// 16-byte chunks of one row's scale copy for ninst instructions.  The copy
// starts at the 16-byte boundary at or below the wave's first group; it
// needs one chunk more than the bytes unless that start is the group itself
// for every row (tight: rows of G % 8 == 0 groups, and a wave start at a
// 16-byte multiple of groups).
template <int BITS, int GS>
__host__ __device__ inline int quad_sb_chunks(int ninst, bool tight) {
  return (ninst * QuadGeom<BITS, GS>::GPI * 2 + 15) / 16 + (tight ? 0 : 1);
}

// Whether waves of a K split over 1 << lks waves start their copies tight.
template <int BITS, int GS>
__host__ __device__ inline bool quad_tight(int G, int lks) {
  return G % 8 == 0 && (lks == 0 || (QuadGeom<BITS, GS>::GPI * 2) % 16 == 0);
}

// Per-wave LDS chunk stride of a launch: nI instructions, workgroups of
// 1 << lw waves, full_wgs > 0 when some waves run whole quads.
template <int BITS, int GS>
__host__ __device__ inline int quad_lds_chunks(int nI, int G, int lw, bool full) {
  const int split = quad_sb_chunks<BITS, GS>((nI + (1 << lw) - 1) >> lw, quad_tight<BITS, GS>(G, lw));
  if (!full) return split;
  const int whole = quad_sb_chunks<BITS, GS>(nI, quad_tight<BITS, GS>(G, 0));
  return whole > split ? whole : split;
}

// Workgroups of W waves (a power of two).  The first full_wgs run W whole
// quads each (wave w: quad W g + w, all of K); the rest run one quad each
// (quad W full_wgs + g - full_wgs), K split over its W waves.  Dynamic LDS
// W * 2 KB * SB (scales and biases of 4 rows x 16 SB chunks per wave; every
// lane stores its chunks, zeros past the copy); the copy of a wave at most
// 16 SB chunks per row; x, scales and biases 16-byte aligned.
template <int DT, int BITS, int GS, int SB, bool LATE>
__global__ __launch_bounds__(64 * kQuadMaxKS) void qmv_quad_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ w,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    uint16_t* __restrict__ out, int N, int K, int full_wgs) {
  using Q = QuadGeom<BITS, GS>;
  using T = T16<DT>;
  constexpr int D = kQuadDepth;
  typedef __attribute__((address_space(3))) unsigned char lds8;
  typedef __attribute__((address_space(3))) uint16_t lds16;
  typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
  extern __shared__ __align__(16) unsigned char qq_smem[];
  __shared__ float red[kQuadMaxKS][4];

  // (the K split is a power of two, so its divisions are scalar shifts)
  const int lane = threadIdx.x & 63;
  const int lw = __builtin_ctz(blockDim.x >> 6);
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool split = (int)blockIdx.x >= full_wgs;
  const int lks = split ? lw : 0;
  const int KS = 1 << lks;
  const int kp = split ? wid : 0;
  const int j = lane & 3, bb = lane >> 2;
  const int quad = split ? (full_wgs << lw) + ((int)blockIdx.x - full_wgs)
                         : ((int)blockIdx.x << lw) + wid;
  const int row0 = 4 * quad;
  const int nrows = min(4, N - row0);
  const uint32_t rowB = (uint32_t)K * BITS / 8;
  const int G = K / GS;
  const int nI = (int)((rowB + Q::RB - 1) / Q::RB);
  const int s0 = (nI * kp) >> lks, s1 = (nI * (kp + 1)) >> lks;
  const int n = s1 - s0;
  const int nmax = (nI + KS - 1) >> lks;

  // ---- scale / bias copy of the wave's groups: the loads -----------------
  // Row r's groups [s0 GPI, s1 GPI) start at byte a_r of the arrays; chunk c
  // of row r is bytes [(a_r & ~15) + 16 c, +16), at LDS row r.  Lane
  // (r = lane & 3, c = lane >> 2) loads chunks c + 16 u of row r (zeros
  // past the CH chunks of the copy) and stores them unconditionally: a
  // store under a branch let the compiler sink that lane's load into the
  // branch, behind the weight loads.
  const int CH = quad_sb_chunks<BITS, GS>(nmax, quad_tight<BITS, GS>(G, lks));
  constexpr int CS = 16 * SB;                      // LDS chunks per row (every lane stores)
  lds8* ls = (lds8*)qq_smem + wid * (2 * 4 * 16 * CS);
  u32x4 sq[SB], bq[SB];
  const int cr = lane & 3, cc0 = lane >> 2;
  // (32-bit offsets: the launch keeps the arrays below 2^31 bytes)
  const uint32_t crow = (uint32_t)(row0 + cr) * (uint32_t)G * 2u;
  const uint32_t ca0 = ((crow + (uint32_t)s0 * (Q::GPI * 2)) & ~15u) + 16u * cc0;
  const uint32_t sbytes = (uint32_t)N * (uint32_t)G * 2u;
  const auto rs = make_rsrc(scales, sbytes);
  const auto rb = make_rsrc(biases, sbytes);
  uint32_t go[SB];
#pragma unroll
  for (int u = 0; u < SB; ++u) {
    go[u] = cc0 + 16 * u < CH && cr < nrows ? ca0 + 256u * u : 0x80000000u;
    sq[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, go[u], 0, 0);
    bq[u] = __builtin_amdgcn_raw_buffer_load_b128(rb, go[u], 0, 0);
  }
  // this lane's scale at instruction s0: row j, group s0 GPI + gb
  const int gb = 16 * bb * (8 / BITS) / GS;
  const uint32_t aj = ((uint32_t)(row0 + j) * (uint32_t)G + (uint32_t)s0 * Q::GPI) * 2u;
  const lds8* lsj = ls + j * 16 * CS + (int)(aj & 15u) + 2 * gb;

  // ---- loads: weights (4 rows x 256 B) and the x slab per instruction -----
  // A ring of R = D + 1 slots: instruction t + D is issued into the slot
  // freed by instruction t - 1 before instruction t is computed.  A lane's
  // offsets are fixed; the instruction's step goes in the scalar offset, and
  // slots past the wave's range set its bit 31 (past every buffer range:
  // zeros, no memory access), so an issue costs no VALU and no branch (a
  // branch around the loads made the compiler drain every load at the join).
  // A weight piece past the end of its row (the ragged last instruction)
  // reads the next row's codes or zeros, times scales and biases the copy
  // zeroed and x past K (zeros): it adds nothing.
  constexpr int R = D + 1;
  constexpr int XW = Q::XB / 4;                      // x dwords per lane per slot
  const auto rw = make_rsrc(reinterpret_cast<const char*>(w) + (int64_t)row0 * rowB,
                            nrows > 0 ? (uint32_t)nrows * rowB : 0u);
  const auto rx = make_rsrc(x, (uint32_t)K * 2);
  const uint32_t wlane = (uint32_t)j * rowB + 16u * bb;
  const uint32_t xlane = (uint32_t)Q::XB * lane;
  u32x4 wv[R];
  uint32_t xv[R][XW];
  auto issue = [&](int slot, int t) {
    const uint32_t s = (uint32_t)(s0 + t);
    const uint32_t dead = (uint32_t)(n - 1 - t) & 0x80000000u;
    wv[slot] = __builtin_amdgcn_raw_buffer_load_b128(rw, wlane, (int)((s * Q::RB) | dead), 2);
    const int xs = (int)((s * (2 * Q::CPI)) | dead);
    if constexpr (XW == 4) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rx, xlane, xs, 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) xv[slot][e] = v[e];
    } else {
      const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rx, xlane, xs, 0);
      xv[slot][0] = v[0];
      xv[slot][1] = v[1];
    }
  };
  // LATE: the first weight loads wait for the scale copy (launches of long
  // waves: K=17408 N=5120, 9 instructions a wave, 12.8 against 13.2 us);
  // else they go out with it (2-3 instructions a wave: 4.9 against 5.1 us
  // at K=4096 N=4096)
  if constexpr (!LATE) {
#pragma unroll
    for (int i = 0; i < D; ++i) issue(i, i);
  }

  // ---- the scale copy lands in LDS --------------------------------------
  // Entries past the row (groups >= G: the ragged last instruction) are
  // stored as zeros, so a lane whose piece lies past K dequantizes zeros;
  // only a row's last chunk holds any.  The big-scale check is a packed
  // 16-bit max over every stored chunk; a big scale of a neighbouring row
  // only costs the wave the plain route.
  typedef unsigned short qq_u16x2 __attribute__((ext_vector_type(2)));
  qq_u16x2 hmax = {0, 0};
  // Chunk u's entries past the row zeroed, into LDS, into the big check.
  // Only a wave whose copy reaches past G (a ragged last instruction, or an
  // untight copy's extra chunk) has such entries in a live chunk (dead
  // chunks read zeros): a uniform flag keeps the others off the masking
  // (else the compiler selects every entry, ~30 VALU per wave).
  const bool ragged = s1 * Q::GPI > G || !quad_tight<BITS, GS>(G, lks);
  auto put = [&](int u, u32x4 sv, u32x4 bv, auto masked) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      hmax = __builtin_elementwise_max(hmax, __builtin_bit_cast(qq_u16x2, sv[e] & 0x7fff7fffu));
    if constexpr (decltype(masked)::value) {
      // group of the chunk's entry 0 (negative: the chunk starts before the row)
      const int g0c = (int)(ca0 + 256u * u - crow) >> 1;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t keep = (g0c + 2 * e < G ? 0x0000ffffu : 0u) |
                              (g0c + 2 * e + 1 < G ? 0xffff0000u : 0u);
        sv[e] &= keep;
        bv[e] &= keep;
      }
    }
    const int cc = cc0 + 16 * u;
    *(lds_u32x4*)(ls + cr * 16 * CS + 16 * cc) = sv;
    *(lds_u32x4*)(ls + 4 * 16 * CS + cr * 16 * CS + 16 * cc) = bv;
  };
  if (ragged) {
#pragma unroll
    for (int u = 0; u < SB; ++u) put(u, sq[u], bq[u], std::true_type{});
  } else {
#pragma unroll
    for (int u = 0; u < SB; ++u) put(u, sq[u], bq[u], std::false_type{});
  }
  // the one chunk across the end of the arrays (their size not a multiple
  // of 16 bytes) read zeros where it crosses the range: its lane reads the
  // entries one by one and stores the chunk again (after the plain stores,
  // so no copy load waits behind this branch)
#pragma unroll
  for (int u = 0; u < SB; ++u) {
    if (go[u] < sbytes && go[u] + 16 > sbytes) {
      u32x4 sv, bv;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t o = go[u] + 4 * e;
        sv[e] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, o, 0, 0) |
                ((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, o + 2, 0, 0) << 16);
        bv[e] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rb, o, 0, 0) |
                ((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rb, o + 2, 0, 0) << 16);
      }
      put(u, sv, bv, std::true_type{});
    }
  }
  if constexpr (LATE) {
#pragma unroll
    for (int i = 0; i < D; ++i) issue(i, i);
  }
  const uint32_t hm = hmax[0] > hmax[1] ? hmax[0] : hmax[1];
  const bool big = DT == kBF16 ? hm >= 0x7180u : hm >= 0x7c00u;   // bf16 2^100 / f16 inf
  const bool plain = __builtin_amdgcn_ballot_w64(big) != 0;
  // the scale copy is this wave's own: order its LDS stores before the reads
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  f32x4 acc[4];

  // word p's MFMAs: its 8 (4-bit) or 4 (8-bit) codes against the lane's own
  // x piece, into accumulator p
  auto mma = [&](const uint32_t (&xq)[XW], int p, const uint32_t* o) {
    acc[p] = quad_mfma<DT>(xq[0], xq[1], o[0], o[1], acc[p]);
    if constexpr (BITS == 4) acc[p] = quad_mfma<DT>(xq[2], xq[3], o[2], o[3], acc[p]);
  };
  auto compute = [&](const u32x4& wq, const uint32_t (&xq)[XW], int t, auto plain_route,
                     auto first) {
    const float sf = T::to_f32(*(const lds16*)(lsj + t * Q::GPI * 2));
    const float bf = T::to_f32(*(const lds16*)(lsj + 4 * 16 * CS + t * Q::GPI * 2));
    const GroupScale g = make_group(sf, bf);
    if constexpr (decltype(plain_route)::value) {
      // one word at a time, so the route's float codes add no registers
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        uint32_t o[4];
        deq_word_plain<DT, BITS>(wq[p], g, o);
        mma(xq, p, o);
      }
    } else {
      // all four words dequantized first, then the MFMAs, so no MFMA waits
      // on the one before it (accumulator p takes word p's halves in order)
      uint32_t o[4][4];
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        if constexpr (BITS == 4) deq4_word<DT>(wq[p], g, o[p]);
        else deq8_word<DT>(wq[p], g, o[p]);
      }
#pragma unroll
      for (int p = 0; p < 4; ++p)
        acc[p] = quad_mfma<DT>(xq[0], xq[1], o[p][0], o[p][1],
                               decltype(first)::value ? (f32x4){0.f, 0.f, 0.f, 0.f} : acc[p]);
      if constexpr (BITS == 4) {
#pragma unroll
        for (int p = 0; p < 4; ++p)
          acc[p] = quad_mfma<DT>(xq[2], xq[3], o[p][2], o[p][3], acc[p]);
      }
    }
  };

  if (!plain) {
    // instruction 0 (every wave has one) starts the accumulators from its
    // products; then the steady state in straight-line blocks of R
    // instructions (a branch per instruction kept the scheduler from
    // overlapping one instruction's MFMAs with the next one's dequant), then
    // the last ones, whose further loads are all past the range
    issue(D % R, D);
    compute(wv[0], xv[0], 0, std::false_type{}, std::true_type{});
    int t = 1;
    for (; t + R <= n; t += R) {
#pragma unroll
      for (int i = 0; i < R; ++i) {
        issue((1 + i + D) % R, t + i + D);
        compute(wv[(1 + i) % R], xv[(1 + i) % R], t + i, std::false_type{}, std::false_type{});
      }
    }
#pragma unroll
    for (int i = 0; i < R - 1; ++i)
      if (t + i < n)
        compute(wv[(1 + i) % R], xv[(1 + i) % R], t + i, std::false_type{}, std::false_type{});
  } else {
    // the plain route (|s| >= 2^100 in this wave's scales, never in real
    // checkpoints): one instruction at a time, the ring's loads discarded,
    // so it adds no registers to the kernel
#pragma unroll
    for (int p = 0; p < 4; ++p) acc[p] = (f32x4){0.f, 0.f, 0.f, 0.f};
    for (int t = 0; t < n; ++t) {
      issue(0, t);
      compute(wv[0], xv[0], t, std::true_type{}, std::false_type{});
    }
  }

  // ---- kept rows in class order, xor tree over the row's 16 lanes ---------
  float v = acc[0][0] + acc[1][1] + acc[2][2] + acc[3][3];
  // lanes 16 r + 4 b + j, b = 0..3: rotate by one and by two b within the
  // row of 16 (DPP row_ror 4, 8), then across the rows
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                             0x124, 0xf, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                             0x128, 0xf, 0xf, false));
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  if (KS == 1) {
    if (bb == 0 && j < nrows) out[row0 + j] = T::round1(v);
    return;
  }
  if (bb == 0) red[kp][j] = v;
  __syncthreads();
  if (kp == 0 && lane < nrows) {
    float t = red[0][lane];
    for (int u = 1; u < KS; ++u) t += red[u][lane];
    out[row0 + lane] = T::round1(t);
  }
}

// K split of a quad launch: the fewest waves per quad (1, 2, 4, 8) giving at
// least 4 waves per SIMD, with at least two instructions per wave.
inline int quad_ks(int64_t N, int64_t K, int bits, int cus) {
  const int64_t quads = (N + 3) / 4;
  const int64_t nI = (K * bits / 8 + 255) / 256;
  int ks = 1;
  while (ks < kQuadMaxKS && quads * ks < 16 * (int64_t)cus && nI / (2 * ks) >= 2) ks *= 2;
  return ks;
}

// Split of the leftover quads when one wave per quad leaves a partial round
// (quads >= 4 cus, L = quads mod 4 cus > 0): the largest W in {2, 4} with
// L W <= 4 cus (one split wave per SIMD at most) and at least one
// instruction per wave; 1 when none applies.
inline int quad_tail_split(int64_t N, int64_t K, int bits, int cus) {
  const int64_t quads = (N + 3) / 4, S = 4 * (int64_t)cus, L = quads % S;
  const int64_t nI = (K * bits / 8 + 255) / 256;
  if (quads < S || L == 0) return 1;
  int W = 1;
  while (W < 4 && L * 2 * W <= S && nI >= 2 * W) W *= 2;
  return W;
}

template <int DT, int BITS, int GS>
int QuadLaunch<DT, BITS, GS>::run(const void* x, const uint32_t* w, const void* s, const void* b,
                                  void* out, int64_t M, int64_t N, int64_t K, hipStream_t st,
                                  int* nlaunch) {
  auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (M != 1 || !a16(x) || !a16(s) || !a16(b)) return kStatusUnsupported;
  // the scale copy addresses the whole scale array through one buffer range
  if (N * (K / GS) * 2 >= ((int64_t)1 << 31)) return kStatusUnsupported;
  const int cus = device_cu_count();
  const int G = (int)(K / GS);
  const int nI = (int)((K * BITS / 8 + 255) / 256);
  const int64_t quads = (N + 3) / 4;
  int W = quad_ks(N, K, BITS, cus);
  int64_t full_wgs = 0, wgs = quads;
  if (W == 1 && quad_lds_chunks<BITS, GS>(nI, G, 0, false) <= 16 * kQuadMaxSb) {
    const int Wt = quad_tail_split(N, K, BITS, cus);
    if (Wt > 1) {
      const int64_t L = quads % (4 * (int64_t)cus);
      W = Wt;
      full_wgs = (quads - L) / W;
      wgs = full_wgs + L;
    }
  }
  const int lw = __builtin_ctz(W);
  int CHW = quad_lds_chunks<BITS, GS>(nI, G, lw, full_wgs > 0);
  if (full_wgs == 0) {
    while (W < kQuadMaxKS && CHW > 16 * kQuadMaxSb) {
      W *= 2;
      CHW = quad_lds_chunks<BITS, GS>(nI, G, __builtin_ctz(W), false);
    }
  }
  if (CHW > 16 * kQuadMaxSb) return kStatusUnsupported;
  const int SBn = CHW <= 16 ? 1 : 2;
  const size_t lds = (size_t)W * 2 * 4 * 16 * 16 * SBn;
  const bool late = (full_wgs > 0 ? nI : (nI + W - 1) / W) >= 4;
  auto kern = SBn == 1 ? (late ? qmv_quad_kernel<DT, BITS, GS, 1, true>
                               : qmv_quad_kernel<DT, BITS, GS, 1, false>)
                       : (late ? qmv_quad_kernel<DT, BITS, GS, 2, true>
                               : qmv_quad_kernel<DT, BITS, GS, 2, false>);
  hipLaunchKernelGGL(kern, dim3((unsigned)wgs), dim3(64 * W), lds, st, (const uint16_t*)x, w,
                     (const uint16_t*)s, (const uint16_t*)b, (uint16_t*)out, (int)N, (int)K,
                     (int)full_wgs);
  ++*nlaunch;
  return 0;
}

}  // namespace mq
