// Skinny quantized matmul, M <= 16 rows: out[M,N] = x[M,K] . deq(W[N,K])^T.
//
// One kernel family covers the reference's M=1 decode path (mx.quantized_matmul
// -> MLX qmv_fast, mlxturbo/kernels/dispatch.py:317-327) and its M=2..16
// verify window (kernels/qmv_small_m.py:289-335, fast_qmm.py:334-374,
// kernels/qmv_wide_nocap.py:240-288).
//
// The packed weights stream from HBM once; everything is laid out for that
// stream, for the number of memory requests and for the VALU cost of exact
// dequantization, which measurement showed to be the limiters:
//
//  * A workgroup owns a tile of 16 weight rows; its NW waves split the tile's
//    K range into contiguous slices of whole steps.  Lane (r = lane & 15,
//    c = lane >> 4) reads row r.  A step covers 4*GPL quantization groups
//    (STEPB bytes) of each row, read with STEPB/64 16-byte loads per lane:
//    load L of lane c covers bytes [64 L + 16 c, +16) of the step's row, so
//    one load instruction reads 64 contiguous bytes of each of the 16 rows
//    (whole 64-byte sectors; an interleaved layout that touched every sector
//    twice cost ~10% at the headline shape).
//  * Weights are read with buffer loads whose descriptor is rebuilt per step
//    in scalar registers.  A step beyond the wave's slice gets num_records =
//    0, so its loads return zeros without touching memory; that keeps the
//    PF-stage prefetch pipeline free of conditional loads (vmcnt waits stay
//    exact).  Rows past N are past num_records as well.
//  * Scales and biases of the whole tile (16 rows x K/GS groups, contiguous
//    in memory) are copied into LDS once per tile with 16-byte loads issued
//    ahead of the weight prologue (SBL).  Reading them per step straight
//    from memory (16 scattered 16-byte pieces per instruction) took ~2 us of
//    a 15 us launch at the headline shape.  Shapes whose scale rows are not
//    16-byte multiples, or too long for the copy, read them per step.
//  * x (M <= 16 rows) streams with the weights: each step's x slice is
//    loaded in the same batch as the step's weights and staged through a
//    per-wave LDS region from which the MFMA A fragments are read
//    (ds_read_b128).  An up-front copy of all of x stalled every wave for
//    microseconds behind the weight prologue in the memory queues.  Lanes
//    whose A row is >= M read row M-1: it only fills output rows that are
//    never stored, since the rows of an MFMA product are independent.
//    Rows beyond the streamed capacity read A fragments from global memory
//    in the same order.
//  * From 8 rows on, a workgroup runs two 16-row tiles (TJ = 2) over each x
//    slice, halving the x traffic per weight byte; each tile keeps its own
//    accumulator, so results do not depend on TJ.
//  * With 48 or more weight rows per CU, 5-16 rows run one workgroup per CU
//    of three 4-wave groups (two tiles each) that read x once for all three:
//    5-8 rows copy all of x into LDS before the first step, and no step loads
//    x; 9-16 rows (x too large for LDS) stage each step's x slice once for
//    the groups, in two buffers per K slice with a workgroup barrier per
//    step; 17-32 rows run in one such launch, each group multiplying every
//    weight fragment with two 16-row A tiles (x staged in one buffer per
//    slice, a barrier before and after).  Each group's arithmetic is that of
//    the one-group launch.
//  * Given a workspace, 5-64 rows on matrices of fewer than 640 tiles (K=17408
//    N=5120) run each tile's K slices on separate workgroups, one slice per
//    workgroup over ten whole tiles (17-64 rows as 2 or 4 16-row A tiles), and
//    a second kernel adds the float slices in order: the same arithmetic as
//    the one-workgroup launch of each 16 rows.
//  * Dequantization is the exact fma_mix trick of mq_common.h, rounded to T
//    per weight (bit-exact MLX dequantization); the packed T pairs are the
//    B operand of v_mfma_f32_16x16x32 (32 k x 16 rows).  A and B use the same
//    lane -> k mapping, so the permuted k order inside each MFMA is harmless.
//    Scales with |s| >= 2^100 (never seen in real checkpoints) switch the
//    whole step, wave-uniformly, to a plain float route.
//  * The NW partial 16x16 tiles are summed in LDS in wave order and rounded
//    once.  The K decomposition depends on (N, K, bits, group_size) only, so
//    each output row is bit-identical for every M (the property the
//    reference tests for its small-M kernel: bench/test_qmm_smallm.py:70-85).
#pragma once
#include <type_traits>
#include "launch.h"

namespace mq {

typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) u32x2 lds_u32x2;
typedef __attribute__((address_space(3))) unsigned char lds_u8;

// v_perm selector moving 16-bit half h (0..3 of the 64-bit pair {hi:lo}) to
// where a float conversion wants it: bf16 -> bits 16..31 (the float's bits),
// f16 -> bits 0..15.  Selector byte 0x0c yields 0x00.
template <int DT>
__device__ __forceinline__ uint32_t half_selector(int h) {
  const uint32_t b0 = 2u * (uint32_t)h, b1 = b0 + 1u;
  if constexpr (DT == kBF16) return 0x0c0cu | (b0 << 16) | (b1 << 24);
  else return b0 | (b1 << 8) | 0x0c0c0000u;
}

template <int DT>
__device__ __forceinline__ float selected_to_f32(uint32_t v) {
  if constexpr (DT == kBF16) return __uint_as_float(v);
  else return (float)bitcast<_Float16>((uint16_t)v);
}

template <int BITS, int GS, int GPL>
struct QmvGeom {
  static constexpr int GB = GS * BITS / 8;         // bytes of one group of one row
  static constexpr int STEPG = 4 * GPL;            // groups per row per step
  static constexpr int STEPB = STEPG * GB;         // weight bytes per row per step
  static constexpr int STEPK = STEPG * GS;         // codes per step
  static constexpr int NSV = STEPG / 2;            // scale dwords per row per step
  static constexpr int NL = STEPB / 64;            // 16-byte weight loads per lane per step
  static constexpr int CPL = 128 / BITS;           // codes per 16-byte load
  static constexpr int MPL = (BITS == 4) ? 4 : 2;  // MFMAs per 16-byte load (8 codes each)
  // group of lane c's load L within the step: (4 L + c) >> SH
  static constexpr int SH = (GB == 16) ? 0 : (GB == 32) ? 1 : (GB == 64) ? 2 : 3;
  static_assert(GB >= 16 && GB <= 128, "a group spans 16..128 bytes");
  static_assert(NL >= 1 && STEPB % 64 == 0, "a step is whole 64-byte row pieces");
  static_assert(NSV == 2 || NSV % 4 == 0, "scale vector must be 8 bytes or whole 16-byte loads");
};

// Launch geometry of the skinny kernel for one (bits, group_size): groups per
// lane per step (steps of 128 bytes per row where the format allows: shorter
// steps measured 8% faster than 256-byte ones at the headline shape), waves
// per workgroup, pipeline stages.  Fixed per format and (N, K), never per M,
// so every output row is computed in the same order for every M.
template <int BITS, int GS>
struct QmvConf {
  static constexpr int GPL = (BITS == 4 && GS == 32) ? 2 : 1;
  static constexpr int NW = 4;
  static constexpr int PF = 2;
};

// Waves per workgroup: 8 when the matrix has few 16-row tiles (the K split
// then keeps more waves in flight; K=17408 N=5120: 15.5 us against 16.3 with
// 4), 4 otherwise.
inline int qmv_nw_for(int64_t N) { return (N + 15) / 16 < 640 ? 8 : 4; }

// Streamed-x capacities: 1, 2, 4 and 8 rows everywhere, 16 rows in the
// skinny kernel for steps of at most 256 codes (longer steps would hold 64
// x registers per stage).  Rows beyond the capacity read A fragments straight
// from global memory (same arithmetic order).
constexpr int kQmvMaxXM = 8;

// Smallest streamed-x capacity (1, 2, 4, 8) holding M rows, or 0.
inline int qmv_xm_for(int64_t M) {
  return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : M <= kQmvMaxXM ? 8 : 0;
}

template <int BITS, int GS, int GPL>
inline int qmv_skinny_xm_for(int64_t M) {
  if (M > kQmvMaxXM && M <= 16 && QmvGeom<BITS, GS, GPL>::STEPK <= 256) return 16;
  return qmv_xm_for(M);
}

// Tiles per workgroup of the skinny kernel: two 16-row tiles share each x
// slice once x outweighs the tile's weights per step (8+ streamed rows:
// M=8 18.4 against 18.7 us, M=16 21.9 against 24.8 at K=5120 N=17408; 19.4
// against 22.4 and 23.3 against 31.9 at K=17408 N=5120); fewer rows run one
// tile per workgroup (M=1..4 lose 1.5-2.5 us with two: fewer, longer
// workgroups).
inline int qmv_tj_for(int xm) { return xm >= 8 ? 2 : 1; }

// Dynamic LDS of a workgroup streaming x for up to XM rows: one region of
// XM rows x one step (rows padded by 16 bytes) per wave.
template <int BITS, int GS, int GPL>
__host__ __device__ inline size_t qmv_x_lds(int NW, int XM) {
  return (size_t)NW * (XM ? XM : 1) * (2 * QmvGeom<BITS, GS, GPL>::STEPK + 16);
}

// Scale/bias copy of one tile: 16-byte chunks of each array per thread, LDS
// row stride and LDS bytes (16 rows of scales, then 16 rows of biases).
constexpr int kQmvSbChunks = 3;
__host__ __device__ inline int qmv_sb_stride(int G) { return 2 * G + 16; }
__host__ __device__ inline size_t qmv_sb_lds(int G) { return 2 * 16 * (size_t)qmv_sb_stride(G); }

// Upper bound of the dynamic LDS of one skinny launch over every K the
// scale copy accepts (TJ * 16 * G / 8 <= kQmvSbChunks * 64 * NW).
template <int BITS, int GS, int GPL>
__host__ __device__ inline size_t qmv_lds_bound(int NW, int XM, bool sbl, int TJ) {
  const int gmax = 8 * (kQmvSbChunks * 64 * NW / (16 * TJ));
  return qmv_x_lds<BITS, GS, GPL>(NW, XM) + (sbl ? TJ * qmv_sb_lds(gmax) : 0);
}

// Whether the scales/biases of TJ tiles can be copied to LDS: rows of whole
// 16-byte chunks (so the copy never splits a chunk across rows), 16-byte
// aligned bases, and at most kQmvSbChunks chunks of each array per thread.
inline bool qmv_sb_fits(int64_t G, int NW, int TJ, const void* scales, const void* biases) {
  return G % 8 == 0 && TJ * 16 * (G / 8) <= (int64_t)kQmvSbChunks * 64 * NW &&
         (reinterpret_cast<uintptr_t>(scales) & 15) == 0 &&
         (reinterpret_cast<uintptr_t>(biases) & 15) == 0;
}

// Row sources of a tile: where the A rows (x) come from and where outputs go.
// Every Rows type gives x (base of all A rows), x_nrec (bytes of x readable
// from x, < 2^31 when x streams through LDS), xoff(m) (element offset of A
// row m from x) and either store(m, nn, v) of a rounded 16-bit output
// (kCombine false) or store_combined(m, nn, v[TJ]) of the float sums of all
// tiles of the call (kCombine true).
// A Rows type may also give kXAux, the cache-policy bits of its x loads
// (0 when absent).
template <class R, class = void>
struct RowsXAux {
  static constexpr int value = 0;
};
template <class R>
struct RowsXAux<R, std::void_t<decltype(R::kXAux)>> {
  static constexpr int value = R::kXAux;
};

// Dense: A row m is x row m; output (m, column n0 + nn).
struct DenseRows {
  static constexpr bool kCombine = false;
  const uint16_t* x;
  uint32_t x_nrec;
  uint16_t* out;
  int64_t ldx, ldo;
  int n0;
  __device__ __forceinline__ int64_t xoff(int m) const { return (int64_t)m * ldx; }
  __device__ __forceinline__ void store(int m, int nn, uint16_t v) const {
    out[(int64_t)m * ldo + n0 + nn] = v;
  }
};

// The tiles of one qmv_tile call: tile j is rows[j] (<= 16; <= 0 is an empty
// tile) rows of a [*, K] quantized matrix whose first row starts at w[j] /
// s[j] / b[j].  rows[] must be wave-uniform.
template <int TJ>
struct QmvTiles {
  const char* w[TJ];
  const char* s[TJ];
  const char* b[TJ];
  int rows[TJ];
};

template <class T, class Rows>
__device__ __forceinline__ void rows_put(const Rows& src, int m, int nn, float v) {
  src.store(m, nn, T::round1(v));
}

// Output (m, nn) of every tile: tile j's value goes to column 16 j + nn, or
// a combining Rows (kCombine) turns the TJ values into one output.
template <class T, int TJ, class Rows>
__device__ __forceinline__ void rows_put_tiles(const Rows& src, int m, int nn,
                                               const float (&v)[TJ], const int (&rows)[TJ]) {
  if constexpr (Rows::kCombine) {
    if (nn < rows[0]) src.store_combined(m, nn, v);
  } else {
#pragma unroll
    for (int j = 0; j < TJ; ++j)
      if (nn < rows[j]) rows_put<T>(src, m, 16 * j + nn, v[j]);
  }
}

// Shared x slices of SHX wave groups (qmv_tile with SHX > 1): the groups
// that run the same K slice (wave kw of each group) stage each step's x slice
// once, into one of two buffers per slice, each group loading every SHX-th
// piece; every step then ends its staging with a workgroup barrier.
template <int BITS, int GS, int GPL>
__host__ __device__ inline size_t qmv_shx_lds(int NW, int XM) {
  return 2 * qmv_x_lds<BITS, GS, GPL>(NW, XM);
}

// TJ 16-row weight tiles times M <= 16 A rows, computed by a group of NW
// waves: kw is the (wave-uniform) wave index in the group, gt = 64 kw + lane.
// The TJ tiles share every x slice (x is read once per call, not per tile)
// and each has its own accumulator, so a tile's sum does not depend on TJ.
// The group owns qmv_x_lds(NW, XM) (+ TJ qmv_sb_lds(G) when SBL) bytes of
// LDS at qmv_smem and red[0 .. NW*TJ-1].  Every wave of the workgroup calls
// it the same number of times (it holds workgroup barriers); requires M <=
// XM when XM > 0, and qmv_sb_fits(G, NW, TJ) when SBL.
// SHX > 1 (XM > 0): the workgroup is SHX groups of NW waves over the same x
// rows (group grp of them); the x slices live in the qmv_shx_lds(NW, XM)
// bytes at xsh, shared by the groups, and qmv_smem then only holds the
// group's scale copy.  Each group's arithmetic is the SHX = 1 arithmetic.
// SPLIT (NW = 1): the wave runs K slice ksl of nsl (the slice wave ksl of
// an nsl-wave group runs) and hands its float tiles to a combining Rows.
template <int DT, int BITS, int GS, int GPL, int NW, int PF, int XM, bool SBL, int TJ, int SHX = 1,
          bool XRES = false, int MT = 1, bool SPLIT = false, class Rows>
__device__ __forceinline__ void qmv_tile(const QmvTiles<TJ>& tl, int M, int K, const Rows& src,
                                         unsigned char* qmv_smem, f32x4 (*red)[64], int kw,
                                         int gt, unsigned char* xsh = nullptr, int grp = 0,
                                         int ksl = 0, int nsl = 1) {
  using Gm = QmvGeom<BITS, GS, GPL>;
  constexpr int STEPG = Gm::STEPG, STEPB = Gm::STEPB, STEPK = Gm::STEPK, NSV = Gm::NSV;
  constexpr int NL = Gm::NL, CPL = Gm::CPL, MPL = Gm::MPL, SH = Gm::SH;
  // x pieces (16 bytes = 8 codes) of one step: piece i = lane + 64*q covers
  // row i / XPR, codes 8*(i % XPR) of the step.
  constexpr int XPR = STEPK / 8;                          // pieces per x row per step
  constexpr int XPL = XM ? (XM * XPR + 63) / 64 : 1;      // pieces per lane per step
  constexpr int XSR = 2 * STEPK + 16;                     // LDS bytes per x row (padded)
  static_assert(SHX == 1 || XM > 0, "shared x slices stream through LDS");
  constexpr int XAUX = RowsXAux<Rows>::value;
  static_assert(XAUX == 0 || XM > 0, "x loads with cache-policy bits are buffer loads");
  // pieces this wave loads: q-th of them is piece q * SHX + grp
  constexpr int XPW = XRES ? 1 : (XPL + SHX - 1) / SHX;
  static_assert(!XRES || (XM > 0 && SBL), "resident x is filled with the scale copy");
  static_assert(MT == 1 || (SHX > 1 && !XRES && XM == 16 * MT && (NW > 1 || SPLIT)),
                "16-row A tiles beyond the first share staged x slices");
  static_assert(!SPLIT || (NW == 1 && Rows::kCombine), "a split slice hands floats on");
  using T = T16<DT>;
  struct Stage {
    u32x4 w[TJ][NL];
    uint32_t s[TJ][SBL ? 1 : NSV], b[TJ][SBL ? 1 : NSV];
    u32x4 xq[XPW];
  };
  const int lane = threadIdx.x & 63;
  const int wave = kw;
  const int r = lane & 15, c = lane >> 4;
  const uint32_t rowB = (uint32_t)K * BITS / 8;
  const int G = K / GS;
  const uint32_t sRowB = (uint32_t)G * 2;
  uint32_t w_nrec[TJ], s_nrec[TJ];
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int rj = tl.rows[j];
    w_nrec[j] = rj > 0 ? (uint32_t)(rj - 1) * rowB + STEPB : 0u;
    s_nrec[j] = rj > 0 ? (uint32_t)(rj - 1) * sRowB + STEPG * 2 : 0u;
  }
  const uint32_t wofs = (uint32_t)r * rowB + (uint32_t)c * 16;
  const uint32_t sofs = (uint32_t)r * sRowB;
  // scale of load L: half ((4 L + c) >> SH) & 3 of dword pair ((4 L) >> SH) >> 2
  uint32_t selL[NL];
#pragma unroll
  for (int L = 0; L < NL; ++L) selL[L] = half_selector<DT>(((4 * L + c) >> SH) & 3);

  const int nsteps = (G + STEPG - 1) / STEPG;
  const int full = G / STEPG;                 // steps with every group inside K
  const int sw = SPLIT ? ksl : wave, swn = SPLIT ? nsl : NW;   // K slice of this wave
  const int sb = (int)((int64_t)nsteps * sw / swn);
  const int se = (int)((int64_t)nsteps * (sw + 1) / swn);
  const int fe = se < full ? se : full;      // pipelined (unchecked) steps: [sb, fe)

  const int xr = min(r, M - 1);              // A row of this lane (rows >= M repeat row M-1)
  int xrm[MT];                               // same, in each 16-row A tile
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) xrm[mt] = min(16 * mt + r, M - 1);
  // SHX > 1: buffer b (0, 1) of slice kw at xsh + (2 kw + b) XM XSR; with
  // MT > 1 one buffer per slice, at xsh + kw XM XSR
  lds_u8* xreg = SHX > 1 ? (lds_u8*)xsh + (MT > 1 ? 1 : 2) * wave * XM * XSR
                         : (lds_u8*)qmv_smem + wave * (XM ? XM : 1) * XSR;
  // XRES: row m of x at xsh + m XRS, codes [0, nsteps STEPK), zero past K
  const int XRS = 2 * nsteps * STEPK + 16;
  const lds_u8* xl = XRES ? (const lds_u8*)xsh + xr * XRS : xreg + xr * XSR;
  const lds_u8* xlm[MT];                     // A rows of the 16-row tiles (MT > 1)
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) xlm[mt] = xreg + xrm[mt] * XSR;
  const uint16_t* xg = src.x + src.xoff(xr);
  const int SBS = qmv_sb_stride(G);
  // tile j's scale rows at sbl + j * 32 SBS, its bias rows 16 SBS further
  lds_u8* sbl = (lds_u8*)qmv_smem + (SHX > 1 ? 0 : NW * (XM ? XM : 1) * XSR);
  // XM > 0: byte offset of this lane's x pieces from the step's x slice;
  // pieces of rows >= M are out of the buffer range (no memory access, zeros)
  uint32_t xvo[XPW];
  int xpk[XPW], xpi[XPW];
#pragma unroll
  for (int q = 0; q < XPW; ++q) {
    const int qq = SHX > 1 ? q * SHX + grp : q;
    const int i = lane + 64 * qq;
    const int m = i / XPR;
    xpi[q] = qq < XPL && i < (XM ? XM : 1) * XPR ? i : -1;   // -1: no piece of this wave
    xpk[q] = 8 * (i - m * XPR);
    xvo[q] = (m < M && xpi[q] >= 0) ? (uint32_t)(src.xoff(m) + xpk[q]) * 2u : 0x80000000u;
  }

  auto load = [&](Stage& s, int t, bool live) {
    if constexpr (XM > 0 && !XRES) {
      const uint32_t xstep = (uint32_t)t * STEPK * 2;
      const auto rx = make_rsrc(reinterpret_cast<const char*>(src.x) + xstep,
                                live ? src.x_nrec - xstep : 0u);
#pragma unroll
      for (int q = 0; q < XPW; ++q)
        s.xq[q] = __builtin_amdgcn_raw_buffer_load_b128(rx, xvo[q], 0, XAUX);
    }
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const auto rw = make_rsrc(tl.w[j] + (int64_t)t * STEPB, live ? w_nrec[j] : 0u);
#pragma unroll
      for (int L = 0; L < NL; ++L)
        s.w[j][L] = __builtin_amdgcn_raw_buffer_load_b128(rw, wofs + L * 64, 0, 0);
    }
    if constexpr (!SBL) {
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        const auto rs = make_rsrc(tl.s[j] + (int64_t)t * STEPG * 2, live ? s_nrec[j] : 0u);
        const auto rb = make_rsrc(tl.b[j] + (int64_t)t * STEPG * 2, live ? s_nrec[j] : 0u);
        if constexpr (NSV == 2) {
          const u32x2 a = __builtin_amdgcn_raw_buffer_load_b64(rs, sofs, 0, 0);
          const u32x2 q = __builtin_amdgcn_raw_buffer_load_b64(rb, sofs, 0, 0);
          s.s[j][0] = a[0]; s.s[j][1] = a[1]; s.b[j][0] = q[0]; s.b[j][1] = q[1];
        } else {
#pragma unroll
          for (int v = 0; v < NSV / 4; ++v) {
            const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(rs, sofs + 16 * v, 0, 0);
            const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(rb, sofs + 16 * v, 0, 0);
#pragma unroll
            for (int e = 0; e < 4; ++e) { s.s[j][4 * v + e] = a[e]; s.b[j][4 * v + e] = q[e]; }
          }
        }
      }
    }
  };

  f32x4 acc[TJ][MT];
#pragma unroll
  for (int j = 0; j < TJ; ++j)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[j][mt] = (f32x4){0.f, 0.f, 0.f, 0.f};

  // A fragment covering codes [k, k+8): k relative to the step (LDS slice) or
  // absolute (global).  Codes past K read zeros (LDS slices are zeroed there).
  auto afrag = [&](int krel, int kabs, bool checked, int mt = 0) -> u32x4 {
    if constexpr (MT > 1) {
      (void)kabs; (void)checked;
      return *(const lds_u32x4*)(xlm[mt] + 2 * krel);
    } else if constexpr (XRES) {
      (void)krel; (void)checked;
      return *(const lds_u32x4*)(xl + 2 * kabs);
    } else if constexpr (XM > 0) {
      (void)kabs; (void)checked;
      return *(const lds_u32x4*)(xl + 2 * krel);
    } else {
      (void)krel;
      if (checked && kabs >= K) return (u32x4){0u, 0u, 0u, 0u};
      return *reinterpret_cast<const u32x4*>(xg + kabs);
    }
  };

  // par: buffer of the step's x slice (SHX > 1); dead: the step is past this
  // wave's slice and only stages (zeros) and joins the barrier (SHX > 1).
  // MT > 1: one buffer per K slice, so the staging first waits for every
  // wave to have read the previous step's slice.
  auto compute = [&](const Stage& s, int t, bool checked, int par = 0, bool dead = false) {
    if constexpr (XM > 0 && !XRES) {
      lds_u8* xb = xreg + (SHX > 1 && MT == 1 ? par * XM * XSR : 0);
      if constexpr (MT > 1) __syncthreads();
#pragma unroll
      for (int q = 0; q < XPW; ++q) {
        const int i = xpi[q];
        if ((SHX == 1 && XPL * 64 == XM * XPR) || i >= 0) {
          u32x4 v = s.xq[q];
          if (checked && t * STEPK + xpk[q] >= K) v = (u32x4){0u, 0u, 0u, 0u};
          *(lds_u32x4*)(xb + (i / XPR) * XSR + 2 * xpk[q]) = v;
        }
      }
      if constexpr (SHX > 1) {
        __syncthreads();
        if (dead) return;
        xl = xb + xr * XSR;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) xlm[mt] = xb + xrm[mt] * XSR;
      } else {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
    }
    float sf[TJ][NL], bf[TJ][NL];
    bool big = false;
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      uint32_t sv[NSV], bv[NSV];
      if constexpr (SBL) {
        const lds_u8* ps = sbl + j * 32 * SBS + r * SBS + t * STEPG * 2;
        const lds_u8* pb = ps + 16 * SBS;
        if constexpr (NSV == 2) {
          const u32x2 a = *(const lds_u32x2*)ps, q = *(const lds_u32x2*)pb;
          sv[0] = a[0]; sv[1] = a[1]; bv[0] = q[0]; bv[1] = q[1];
        } else {
#pragma unroll
          for (int v = 0; v < NSV / 4; ++v) {
            const u32x4 a = *(const lds_u32x4*)(ps + 16 * v);
            const u32x4 q = *(const lds_u32x4*)(pb + 16 * v);
#pragma unroll
            for (int e = 0; e < 4; ++e) { sv[4 * v + e] = a[e]; bv[4 * v + e] = q[e]; }
          }
        }
      } else {
#pragma unroll
        for (int v = 0; v < NSV; ++v) { sv[v] = s.s[j][v]; bv[v] = s.b[j][v]; }
      }
#pragma unroll
      for (int L = 0; L < NL; ++L) {
        const int q = ((4 * L) >> SH) >> 2;     // same for the 4 lanes of a row
        sf[j][L] = selected_to_f32<DT>(__builtin_amdgcn_perm(sv[2 * q + 1], sv[2 * q], selL[L]));
        bf[j][L] = selected_to_f32<DT>(__builtin_amdgcn_perm(bv[2 * q + 1], bv[2 * q], selL[L]));
        if (checked && t * STEPG + ((4 * L + c) >> SH) >= G) { sf[j][L] = 0.f; bf[j][L] = 0.f; }
        big |= needs_plain(sf[j][L]);
      }
    }
    const int kr = c * CPL;                   // lane's first code, relative to the step
    const int kt = t * STEPK + kr;            // same, absolute
    // shared-x groups of whole tiles (qmv_shx_kernel, MT = 1): a group
    // without tiles only stages x, and a tile past the group's rows is
    // skipped (uniform branches)
    constexpr bool SKIP = SHX > 1 && MT == 1;
    if (SKIP && tl.rows[0] <= 0) return;
    if (__builtin_amdgcn_ballot_w64(big) == 0) {
#pragma unroll
      for (int L = 0; L < NL; ++L) {
        GroupScale g[TJ];
#pragma unroll
        for (int j = 0; j < TJ; ++j) g[j] = make_group(sf[j][L], bf[j][L]);
#pragma unroll
        for (int p = 0; p < MPL; ++p) {
          const int ko = 4 * L * CPL + 8 * p;
          u32x4 a[MT];
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) a[mt] = afrag(kr + ko, kt + ko, checked, mt);
#pragma unroll
          for (int j = 0; j < TJ; ++j) {
            if (SKIP && j > 0 && tl.rows[j] <= 0) continue;
            uint32_t bo[4];
            if constexpr (BITS == 4) {
              deq4_word<DT>(s.w[j][L][p], g[j], bo);
            } else {
              deq8_word<DT>(s.w[j][L][2 * p], g[j], bo);
              deq8_word<DT>(s.w[j][L][2 * p + 1], g[j], bo + 2);
            }
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
              acc[j][mt] = T::mfma(a[mt], (u32x4){bo[0], bo[1], bo[2], bo[3]}, acc[j][mt]);
          }
        }
      }
    } else {
#pragma unroll
      for (int L = 0; L < NL; ++L) {
        GroupScale g[TJ];
#pragma unroll
        for (int j = 0; j < TJ; ++j) g[j] = make_group(sf[j][L], bf[j][L]);
#pragma unroll
        for (int p = 0; p < MPL; ++p) {
          const int ko = 4 * L * CPL + 8 * p;
          u32x4 a[MT];
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) a[mt] = afrag(kr + ko, kt + ko, checked, mt);
#pragma unroll
          for (int j = 0; j < TJ; ++j) {
            uint32_t bo[4];
            if constexpr (BITS == 4) {
              deq_word_plain<DT, 4>(s.w[j][L][p], g[j], bo);
            } else {
              deq_word_plain<DT, 8>(s.w[j][L][2 * p], g[j], bo);
              deq_word_plain<DT, 8>(s.w[j][L][2 * p + 1], g[j], bo + 2);
            }
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
              acc[j][mt] = T::mfma(a[mt], (u32x4){bo[0], bo[1], bo[2], bo[3]}, acc[j][mt]);
          }
        }
      }
    }
  };

  // ---- scale/bias copy: loads issued ahead of the weight prologue ---------
  // Chunk i (16 bytes of scales and of biases) of the TJ tiles: tile
  // i / (16 cpr), 16-byte chunk i % (16 cpr) of that tile's contiguous rows.
  // Each tile's buffer range ends at its last row, so a lane's chunk loads
  // from exactly one tile and reads zeros from the others.
  Stage S[PF];
  u32x4 sbq[2][SBL ? kQmvSbChunks : 1];
  const int cpr = G / 8;                      // 16-byte chunks per scale row (SBL)
  const int tch = 16 * cpr;                   // chunks per tile
  if constexpr (SBL) {
#pragma unroll
    for (int u = 0; u < kQmvSbChunks; ++u) {
      const uint32_t i = gt + u * 64 * NW;
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        const uint32_t nb = (uint32_t)(max(tl.rows[j], 0) * cpr) * 16u;
        const auto rs0 = make_rsrc(tl.s[j], nb);
        const auto rb0 = make_rsrc(tl.b[j], nb);
        const uint32_t o = (i - (uint32_t)(j * tch)) * 16u;   // wraps past the range below
        const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(rs0, o, 0, 0);
        const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(rb0, o, 0, 0);
        sbq[0][u] = j ? (sbq[0][u] | a) : a;
        sbq[1][u] = j ? (sbq[1][u] | q) : q;
      }
    }
  }
  // ---- resident x (XRES): the workgroup's threads copy rows [0, M) of x,
  // the first XRU pieces of each thread loaded ahead of the weight prologue
  constexpr int XRU = 8;
  u32x4 xrq[XRES ? XRU : 1];
  const int xnt = 64 * NW * SHX;               // threads of the workgroup
  const int xtid = grp * 64 * NW + gt;
  const int xrp = nsteps * STEPK / 8;          // pieces per resident row
  const int xtot = M * xrp;
  auto xres_piece = [&](int i, uint32_t& lofs) -> uint32_t {
    const int m = i / xrp, k = 8 * (i - m * xrp);
    lofs = (uint32_t)(m * XRS + 2 * k);
    return (i < xtot && k < K) ? (uint32_t)(src.xoff(m) + k) * 2u : 0x80000000u;
  };
  if constexpr (XRES) {
    const auto rx = make_rsrc(src.x, src.x_nrec);
#pragma unroll
    for (int u = 0; u < XRU; ++u) {
      uint32_t lo;
      xrq[u] = __builtin_amdgcn_raw_buffer_load_b128(rx, xres_piece(xtid + u * xnt, lo), 0, XAUX);
    }
  }
  // ---- main loop: PF-stage pipeline over the unchecked steps --------------
#pragma unroll
  for (int i = 0; i < PF - 1; ++i) load(S[i], sb + i, sb + i < fe);
  if constexpr (XRES) {
#pragma unroll
    for (int u = 0; u < XRU; ++u) {
      const int i = xtid + u * xnt;
      uint32_t lo;
      xres_piece(i, lo);
      if (i < xtot) *(lds_u32x4*)((lds_u8*)xsh + lo) = xrq[u];
    }
    const auto rx = make_rsrc(src.x, src.x_nrec);
    for (int i = xtid + XRU * xnt; i < xtot; i += xnt) {
      uint32_t lo;
      const uint32_t go = xres_piece(i, lo);
      *(lds_u32x4*)((lds_u8*)xsh + lo) = __builtin_amdgcn_raw_buffer_load_b128(rx, go, 0, XAUX);
    }
  }
  if constexpr (SBL) {
#pragma unroll
    for (int u = 0; u < kQmvSbChunks; ++u) {
      const int i = gt + u * 64 * NW;
      if (i < TJ * tch) {
        const int j = TJ == 1 ? 0 : i / tch;
        const int ii = i - j * tch;
        const int rr = ii / cpr, cc = ii - rr * cpr;
        lds_u8* d = sbl + j * 32 * SBS + rr * SBS + cc * 16;
        *(lds_u32x4*)d = sbq[0][u];
        *(lds_u32x4*)(d + 16 * SBS) = sbq[1][u];
      }
    }
    __syncthreads();
  }
  if constexpr (SHX > 1 && !XRES) {
    // every wave takes as many steps as the longest slice (each step's
    // staging ends with a workgroup barrier); steps past its own are dead
    int nmax = SPLIT ? fe - sb : 0;          // SPLIT: every group runs the one slice
    for (int w2 = 0; w2 < (SPLIT ? 0 : NW); ++w2) {
      const int b2 = (int)((int64_t)nsteps * w2 / NW);
      const int e2 = min((int)((int64_t)nsteps * (w2 + 1) / NW), full);
      nmax = max(nmax, e2 - b2);
    }
    for (int u = 0; u < nmax; u += PF) {
#pragma unroll
      for (int i = 0; i < PF; ++i) {
        const int tl2 = sb + u + i + PF - 1;
        load(S[(i + PF - 1) % PF], tl2, tl2 < fe);
        if (u + i < nmax) compute(S[i], sb + u + i, false, (u + i) & 1, sb + u + i >= fe);
      }
    }
    // No ragged step here: these launches need the scale copy, which takes
    // G % 8 == 0 groups (qmv_sb_fits), and the steps' 2, 4 or 8 groups
    // divide 8, so every step lies inside K (full == nsteps).
  } else {
    for (int t = sb; t < fe; t += PF) {
#pragma unroll
      for (int i = 0; i < PF; ++i) {
        const int tl2 = t + i + PF - 1;
        load(S[(i + PF - 1) % PF], tl2, tl2 < fe);
        if (t + i < fe) compute(S[i], t + i, false);
      }
    }
    // ---- ragged tail: at most one step; groups past K are zeroed ----------
    if (fe < se) {
      Stage s;
      load(s, fe, true);
#pragma unroll
      for (int j = 0; j < TJ; ++j)
#pragma unroll
        for (int L = 0; L < NL; ++L)
          if (fe * STEPG + ((4 * L + c) >> SH) >= G) s.w[j][L] = (u32x4){0u, 0u, 0u, 0u};
      compute(s, fe, true);
    }
  }

  // ---- sum the waves' partial tiles in wave order, round once -------------
  // lane l holds D[4*(l>>4)+v][l&15]: output row 4c+v, column r of the tile
  if constexpr (NW == 1) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = 16 * mt + 4 * c + v;
        float val[TJ];
#pragma unroll
        for (int j = 0; j < TJ; ++j) val[j] = acc[j][mt][v];
        if (m < M) rows_put_tiles<T, TJ>(src, m, r, val, tl.rows);
      }
  } else {
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) red[(wave * TJ + j) * MT + mt][lane] = acc[j][mt];
    __syncthreads();
    for (int tu = gt; tu < 256 * MT; tu += 64 * NW) {
      const int mt = tu >> 8, tt = tu & 255;
      const int mm = tt >> 4, nn = tt & 15;
      const int sl = ((mm >> 2) << 4) | nn, v = mm & 3;
      float sum[TJ];
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        sum[j] = red[j * MT + mt][sl][v];
#pragma unroll
        for (int q = 1; q < NW; ++q) sum[j] += red[(q * TJ + j) * MT + mt][sl][v];
      }
      if (16 * mt + mm < M) rows_put_tiles<T, TJ>(src, 16 * mt + mm, nn, sum, tl.rows);
    }
    // the next tile of this workgroup reuses red and the LDS copies
    __syncthreads();
  }
}

// Workgroup barriers one qmv_tile call executes without shared x slices,
// resident x or stacked A tiles (SHX = 1, XRES off, MT = 1): the scale
// copy's, and the two of the cross-wave sum when NW > 1.  Waves of a
// workgroup that sit a call out execute as many.
template <int NW, bool SBL>
constexpr int qmv_tile_barriers() {
  return (SBL ? 1 : 0) + (NW > 1 ? 2 : 0);
}

// Workgroups of the skinny kernel.  By default one per 16 TJ rows.  When the
// workgroups do not divide evenly over the CUs, some CUs run one more than
// others and finish last (K=5120 N=17408: 1088 tiles on 256 CUs, the CUs
// holding 5 workgroups ended 1.3 us after those holding 4), or some CUs get
// none (K=17408 N=5120 with two tiles per workgroup: 160 workgroups).  The
// launch then spreads the rows evenly over R workgroups per CU, as long as R
// workgroups stay resident together and the idle lanes of the partial tiles
// cost less than the balance gains, which measurement put at: one streamed
// row with at least 13 of 16 rows per workgroup (1280 x 13.6 rows: 14.0
// against 14.5 us; 10 rows lost), and two tiles per workgroup with more than
// one full tile (M=16, two boxes: 768 x 22.7 rows 21.5-21.7 against 22.7 us
// at K=5120, 256 x 20 rows 23.2-23.3 against 24.7 us at K=17408; M=8 0-6%).
// 2..4-row calls keep the default (balanced lost 0.3-0.6 us).  The grouping
// of rows never changes a row's arithmetic.
inline unsigned qmv_grid(int64_t N, int TJ, int NW, int xm, int cus) {
  const int64_t tiles = (N + 16 * TJ - 1) / (16 * TJ);
  if (cus > 0 && tiles % cus != 0 && (xm == 1 || TJ == 2)) {
    const int64_t R = (tiles + cus - 1) / cus;
    const bool enough = TJ == 1 ? N >= 13 * cus * R : N > 16 * cus * R;
    if (R * NW <= 24 && enough) return (unsigned)(cus * R);
  }
  return (unsigned)tiles;
}

// grid.x >= ceil(N / (16 TJ)) workgroups (qmv_grid), block = 64 * NW threads;
// workgroup i owns rows [i N / grid, (i + 1) N / grid) as TJ tiles of <= 16.
// Dynamic LDS qmv_x_lds<BITS, GS, GPL>(NW, XM) (+ TJ qmv_sb_lds(K / GS) when
// SBL) bytes; M <= XM unless XM == 0, and then ((M - 1) * ldx + K) * 2 < 2^31.
template <int DT, int BITS, int GS, int GPL, int NW, int PF, int XM, bool SBL, int TJ>
__global__ __launch_bounds__(64 * NW) void qmv_kernel(const uint16_t* __restrict__ x,
                                                      const uint32_t* __restrict__ w,
                                                      const uint16_t* __restrict__ scales,
                                                      const uint16_t* __restrict__ biases,
                                                      uint16_t* __restrict__ out, int M, int N,
                                                      int K, int64_t ldx, int64_t ldo) {
  extern __shared__ __align__(16) unsigned char qmv_smem[];
  __shared__ f32x4 red[NW * TJ][64];
  const int n0 = (int)((int64_t)blockIdx.x * N / gridDim.x);
  const int n1 = (int)((int64_t)(blockIdx.x + 1) * N / gridDim.x);
  const uint32_t rowB = (uint32_t)K * BITS / 8;
  const uint32_t sRowB = (uint32_t)(K / GS) * 2;
  QmvTiles<TJ> tl;
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int nj = n0 + 16 * j;
    const int rj = min(16, n1 - nj);
    const int64_t base = rj > 0 ? nj : 0;
    tl.w[j] = reinterpret_cast<const char*>(w) + base * rowB;
    tl.s[j] = reinterpret_cast<const char*>(scales) + base * sRowB;
    tl.b[j] = reinterpret_cast<const char*>(biases) + base * sRowB;
    tl.rows[j] = rj;
  }
  const DenseRows src{x, (uint32_t)(((int64_t)(M - 1) * ldx + K) * 2), out, ldx, ldo, n0};
  qmv_tile<DT, BITS, GS, GPL, NW, PF, XM, SBL, TJ>(
      tl, M, K, src, qmv_smem, red, __builtin_amdgcn_readfirstlane(threadIdx.x >> 6),
      threadIdx.x);
}

// Bytes of a resident copy of M rows of x (rows padded to whole steps).
template <int BITS, int GS, int GPL>
__host__ __device__ inline size_t qmv_xres_lds(int M, int K) {
  using Gm = QmvGeom<BITS, GS, GPL>;
  const int nsteps = (K / GS + Gm::STEPG - 1) / Gm::STEPG;
  return (size_t)M * (2 * nsteps * Gm::STEPK + 16);
}

// The skinny kernel with NG wave groups per workgroup over the same x rows
// (qmv_tile with SHX = NG): the groups stage each x slice once, so x is read
// once per 16 NG TJ weight rows instead of once per 16 TJ; with XRES the
// workgroup copies rows [0, M) of x into LDS once, before its first step,
// and no step loads or stages x.  With one A tile (MT = 1) workgroup i owns
// the 16-row tiles [i T / grid, (i + 1) T / grid) of the T = ceil(N / 16),
// group g TJ of them from the g TJ-th on; with two, rows [i N / grid, (i +
// 1) N / grid), group g the g-th NG-th of them as TJ tiles of <= 16 rows;
// rows per workgroup <= 16 NG TJ either way.  Block 64 NW NG, dynamic
// LDS qmv_shx_lds(NW, XM) (XRES: qmv_xres_lds(M, K)) + NG TJ
// qmv_sb_lds(K / GS) (SBL).
template <int DT, int BITS, int GS, int GPL, int NW, int PF, int XM, bool SBL, int TJ, int NG,
          bool XRES, int MT = 1>
__global__ __launch_bounds__(64 * NW * NG) void qmv_shx_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ w,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    uint16_t* __restrict__ out, int M, int N, int K, int64_t ldx, int64_t ldo) {
  extern __shared__ __align__(16) unsigned char qmv_smem[];
  __shared__ f32x4 red[NG * NW * TJ * MT][64];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = wave / NW, kw = wave - g * NW;
  int n0, n1;
  if constexpr (MT == 1) {
    // whole 16-row tiles: workgroup i owns tiles [i T / grid, (i + 1) T /
    // grid) of the T = ceil(N / 16), group g the TJ from the g TJ-th on
    // (fewer or none for the last groups), so no wave dequantizes a partly
    // empty tile: 68 rows per workgroup at K=5120 N=17408 ran as 3 x 2
    // tiles of 11-12 rows, now as 2 + 2 + 0 or 2 + 2 + 1 whole ones (two
    // boxes, one process each: M=5 17.2-17.9 -> 16.3-16.6 us, M=8 17.6-17.9
    // -> 16.8-17.0, M=12 / 16 0-5% faster; two A tiles (17-32 rows) lost
    // 2-3% that way)
    const int64_t nt = (N + 15) / 16;
    const int64_t t0 = (int64_t)blockIdx.x * nt / gridDim.x;
    const int64_t t1 = (int64_t)(blockIdx.x + 1) * nt / gridDim.x;
    const int64_t g0 = t0 + TJ * g < t1 ? t0 + TJ * g : t1;
    const int64_t g1 = g0 + TJ < t1 ? g0 + TJ : t1;
    n0 = (int)(16 * g0 < N ? 16 * g0 : N);
    n1 = (int)(16 * g1 < N ? 16 * g1 : N);
  } else {
    const int64_t wn0 = (int64_t)blockIdx.x * N / gridDim.x;
    const int64_t wn1 = (int64_t)(blockIdx.x + 1) * N / gridDim.x;
    n0 = (int)(wn0 + (wn1 - wn0) * g / NG);
    n1 = (int)(wn0 + (wn1 - wn0) * (g + 1) / NG);
  }
  const uint32_t rowB = (uint32_t)K * BITS / 8;
  const uint32_t sRowB = (uint32_t)(K / GS) * 2;
  QmvTiles<TJ> tl;
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int nj = n0 + 16 * j;
    const int rj = min(16, n1 - nj);
    const int64_t base = rj > 0 ? nj : 0;
    tl.w[j] = reinterpret_cast<const char*>(w) + base * rowB;
    tl.s[j] = reinterpret_cast<const char*>(scales) + base * sRowB;
    tl.b[j] = reinterpret_cast<const char*>(biases) + base * sRowB;
    tl.rows[j] = rj;
  }
  const DenseRows src{x, (uint32_t)(((int64_t)(M - 1) * ldx + K) * 2), out, ldx, ldo, n0};
  const size_t xb = XRES ? qmv_xres_lds<BITS, GS, GPL>(M, K)
                    : MT > 1 ? qmv_x_lds<BITS, GS, GPL>(NW, XM)
                             : qmv_shx_lds<BITS, GS, GPL>(NW, XM);
  unsigned char* gsm = qmv_smem + xb + (SBL ? (size_t)g * TJ * qmv_sb_lds(K / GS) : 0);
  qmv_tile<DT, BITS, GS, GPL, NW, PF, XM, SBL, TJ, NG, XRES, MT>(
      tl, M, K, src, gsm, red + g * NW * TJ * MT, kw, threadIdx.x - 64 * NW * g, qmv_smem, g);
}

// Float tiles of one K slice: A row m, column n of [n0, n1) to part[m N + n].
struct SplitRows {
  static constexpr bool kCombine = true;
  const uint16_t* x;
  uint32_t x_nrec;
  float* part;
  int64_t ldx;
  int N, n0, n1;
  __device__ __forceinline__ int64_t xoff(int m) const { return (int64_t)m * ldx; }
  template <int TJ>
  __device__ __forceinline__ void store_combined(int m, int nn, const float (&v)[TJ]) const {
#pragma unroll
    for (int j = 0; j < TJ; ++j)
      if (n0 + 16 * j + nn < n1) part[(int64_t)m * N + n0 + 16 * j + nn] = v[j];
  }
};

// The K slices of a skinny launch over separate workgroups (5-64 rows on
// matrices of few tiles).  The one-workgroup launch runs a tile's nsl K
// slices on the nsl waves of one workgroup, so every workgroup streams all
// of x (16 x 17408 x 2 B = 557 KB per workgroup at K=17408, three times the
// weight bytes of the call) and 20 rows per CU run as a 16- and a 4-row
// tile.  Here workgroup i runs K slice i % nsl (launch order deals
// consecutive workgroups to the 8 XCDs, so each XCD's L2 serves one slice of
// x) over the whole 16-row tiles [b T / B, (b + 1) T / B) of the T =
// ceil(N / 16), b = i / nsl, B = grid / nsl, on NG one-wave groups of TJ
// tiles that stage each step's x slice once for the workgroup.  Each wave's
// arithmetic is that of wave i % nsl of the one-workgroup launch (same
// steps, same accumulator); its float tile goes to part[i % nsl], and
// qmv_split_sum_kernel adds the nsl planes in slice order and rounds once,
// as that launch's cross-wave sum does, so the bits are the same.  K must be
// whole steps.  With MT = 2 or 4 (17-32 or 33-64 rows) every dequantized
// weight fragment meets MT 16-row A tiles, each with its own accumulator
// (the arithmetic of a 16-row launch for each), x slices of 16 MT rows
// staged in one buffer.  Block 64 NG, dynamic LDS qmv_shx_lds(1, 16) (MT =
// 1) or qmv_x_lds(1, 16 MT).
template <int DT, int BITS, int GS, int GPL, int PF, int TJ, int NG, int MT = 1>
__global__ __launch_bounds__(64 * NG) void qmv_split_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ w,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    float* __restrict__ part, int M, int N, int K, int64_t ldx, int nsl) {
  extern __shared__ __align__(16) unsigned char qmv_smem[];
  const int g = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ks = (int)(blockIdx.x % (unsigned)nsl);
  const int64_t blk = blockIdx.x / (unsigned)nsl, nblk = gridDim.x / (unsigned)nsl;
  const int64_t nt = (N + 15) / 16;
  const int64_t t0 = blk * nt / nblk, t1 = (blk + 1) * nt / nblk;
  const int64_t g0 = t0 + TJ * g < t1 ? t0 + TJ * g : t1;
  const int64_t g1 = g0 + TJ < t1 ? g0 + TJ : t1;
  const int n0 = (int)(16 * g0 < N ? 16 * g0 : N);
  const int n1 = (int)(16 * g1 < N ? 16 * g1 : N);
  const uint32_t rowB = (uint32_t)K * BITS / 8;
  const uint32_t sRowB = (uint32_t)(K / GS) * 2;
  QmvTiles<TJ> tl;
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int nj = n0 + 16 * j;
    const int rj = min(16, n1 - nj);
    const int64_t base = rj > 0 ? nj : 0;
    tl.w[j] = reinterpret_cast<const char*>(w) + base * rowB;
    tl.s[j] = reinterpret_cast<const char*>(scales) + base * sRowB;
    tl.b[j] = reinterpret_cast<const char*>(biases) + base * sRowB;
    tl.rows[j] = rj;
  }
  const SplitRows src{x,  (uint32_t)(((int64_t)(M - 1) * ldx + K) * 2),
                      part + (int64_t)ks * M * N, ldx, N, n0, n1};
  qmv_tile<DT, BITS, GS, GPL, 1, PF, 16 * MT, false, TJ, NG, false, MT, true>(
      tl, M, K, src, qmv_smem, nullptr, 0, threadIdx.x & 63, qmv_smem, g, ks, nsl);
}

// out[i] = round(part[0][i] + part[1][i] + ... + part[NSL - 1][i]), the
// planes added in slice order (the order of the one-workgroup launch's
// cross-wave sum); mn = M N outputs, rows of N contiguous.  The NSL loads
// are issued together (a loop over a run-time count waited for each in
// turn: 4.6 us per call at M=16 N=5120).
template <int DT, int NSL>
__global__ __launch_bounds__(256) void qmv_split_sum_kernel(const float* __restrict__ part,
                                                            uint16_t* __restrict__ out,
                                                            int64_t mn) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= mn) return;
  float p[NSL];
#pragma unroll
  for (int q = 0; q < NSL; ++q) p[q] = part[q * mn + i];
  float v = p[0];
#pragma unroll
  for (int q = 1; q < NSL; ++q) v += p[q];
  out[i] = T16<DT>::round1(v);
}

// One-wave groups per split workgroup and tiles per group.  K=17408 N=5120
// (320 tiles x 8 slices, one box, graph-timed): 10 x 1 on 256 workgroups
// M=16 22.9-23.1 us, M=9 22.2-22.3, against 24.1-24.5 / 23.0-23.2 for the
// one-workgroup launch; 5 x 1 on 512 23.95-24.0, 5 x 2 26.4-26.5, 2 x 1 on
// 1280 26.9.  Deeper prefetch lost (10 x 1, M=16: 3 / 4 / 6 / 8 stages
// 24.5 / 25.6 / 27.8 / 29.8 us against 23.1 with 2).
constexpr int kQmvSplitNG = 10;
constexpr int kQmvSplitTJ = 1;

// Wave groups per shared-x workgroup and tiles per group (K=5120 N=17408
// M=16, one process: 3 x 2 19.4 us, 2 x 3 20.5, 4 x 2 21.6, against 21.4
// for one group of two tiles on three workgroups per CU).
constexpr int kQmvShxNG = 3;
constexpr int kQmvShxTJ = 2;

// Grid of a shared-x launch: a multiple of the CU count (one workgroup per
// CU, the rows spread evenly) holding at most 16 NG TJ rows per workgroup,
// or 0 when the rows are too few for every group to fill a tile.
inline unsigned qmv_shx_grid(int64_t N, int cus) {
  const int64_t cap = 16 * kQmvShxNG * kQmvShxTJ;
  if (cus <= 0 || N < (int64_t)cus * 16 * kQmvShxNG) return 0;
  int64_t grid = cus;
  while (grid * cap < N) grid += cus;
  return (unsigned)grid;
}

// Dynamic LDS the shared-x kernel (4 waves per group, MT 16-row A tiles) may
// use: all of the CU's LDS but its static reduction buffer.
constexpr size_t qmv_shx_lds_max(int MT) {
  return 160 * 1024 - (size_t)kQmvShxNG * 4 * kQmvShxTJ * MT * 64 * sizeof(f32x4);
}
constexpr size_t kQmvShxLdsMax = qmv_shx_lds_max(1);

// One skinny launch of M <= 16 rows.  Launches above 64 KiB of dynamic LDS
// (16 streamed rows with 8 waves) need the kernel's limit raised once per
// device.
template <int DT, int BITS, int GS, int NW, int XM, bool SBL, int TJ>
inline int skinny_launch_one(const uint16_t* x, const uint32_t* w, const void* s, const void* b,
                             uint16_t* out, int M, int64_t N, int64_t K, size_t lds,
                             hipStream_t st) {
  using C = QmvConf<BITS, GS>;
  auto kern = &qmv_kernel<DT, BITS, GS, C::GPL, NW, C::PF, XM, SBL, TJ>;
  if (lds > 65536) {
    static std::atomic<uint64_t> lds_set{0};
    if (hipError_t e = ensure_lds_limit(reinterpret_cast<const void*>(kern),
                                        (int)qmv_lds_bound<BITS, GS, C::GPL>(NW, XM, SBL, TJ),
                                        lds_set))
      return (int)e;
  }
  hipLaunchKernelGGL(kern, dim3(qmv_grid(N, TJ, NW, XM, device_cu_count())), dim3(64 * NW), lds,
                     st, x, w, (const uint16_t*)s, (const uint16_t*)b, out, M, (int)N, (int)K,
                     (int64_t)K, (int64_t)N);
  return 0;
}

// One shared-x launch (4 waves per group, scale copy) streaming XM x rows.
template <int DT, int BITS, int GS, int XM, bool XRES = false, int MT = 1>
inline int skinny_launch_shx_xm(const uint16_t* x, const uint32_t* w, const void* s,
                                const void* b, uint16_t* out, int M, int64_t N, int64_t K,
                                size_t lds, unsigned grid, hipStream_t st) {
  using C = QmvConf<BITS, GS>;
  // the streamed-x launches have no ragged-step code: K must be whole steps
  if (!XRES && (K / GS) % QmvGeom<BITS, GS, C::GPL>::STEPG != 0) return kStatusUnsupported;
  auto kern =
      &qmv_shx_kernel<DT, BITS, GS, C::GPL, 4, C::PF, XM, true, kQmvShxTJ, kQmvShxNG, XRES, MT>;
  static std::atomic<uint64_t> lds_set{0};
  if (hipError_t e = ensure_lds_limit(reinterpret_cast<const void*>(kern),
                                      (int)qmv_shx_lds_max(MT), lds_set))
    return (int)e;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * 4 * kQmvShxNG), lds, st, x, w,
                     (const uint16_t*)s, (const uint16_t*)b, out, M, (int)N, (int)K, (int64_t)K,
                     (int64_t)N);
  return 0;
}

template <int DT, int BITS, int GS>
inline int skinny_launch_shx(int xm, const uint16_t* x, const uint32_t* w, const void* s,
                             const void* b, uint16_t* out, int M, int64_t N, int64_t K,
                             size_t lds, unsigned grid, hipStream_t st) {
  using C = QmvConf<BITS, GS>;
  if (xm == 8) return skinny_launch_shx_xm<DT, BITS, GS, 8>(x, w, s, b, out, M, N, K, lds, grid, st);
  if constexpr (QmvGeom<BITS, GS, C::GPL>::STEPK <= 256) {
    if (xm == 16)
      return skinny_launch_shx_xm<DT, BITS, GS, 16>(x, w, s, b, out, M, N, K, lds, grid, st);
  }
  return kStatusUnsupported;
}

// One split launch (qmv_split_kernel then qmv_split_sum_kernel) of M <= 64
// rows: nsl float planes of M x N in part.
template <int DT, int BITS, int GS>
inline int skinny_launch_split(const uint16_t* x, const uint32_t* w, const void* s, const void* b,
                               uint16_t* out, int M, int64_t N, int64_t K, float* part, int nsl,
                               hipStream_t st) {
  using C = QmvConf<BITS, GS>;
  if (nsl != 8) return kStatusUnsupported;            // the sum kernel adds 8 planes
  constexpr int per = kQmvSplitNG * kQmvSplitTJ;
  const int64_t nblk = ((N + 15) / 16 + per - 1) / per;
  if (M > 32) {
    const size_t lds = qmv_x_lds<BITS, GS, C::GPL>(1, 64);
    hipLaunchKernelGGL((qmv_split_kernel<DT, BITS, GS, C::GPL, C::PF, kQmvSplitTJ, kQmvSplitNG, 4>),
                       dim3((unsigned)(nblk * nsl)), dim3(64 * kQmvSplitNG), lds, st, x, w,
                       (const uint16_t*)s, (const uint16_t*)b, part, M, (int)N, (int)K,
                       (int64_t)K, nsl);
  } else if (M > 16) {
    const size_t lds = qmv_x_lds<BITS, GS, C::GPL>(1, 32);
    hipLaunchKernelGGL((qmv_split_kernel<DT, BITS, GS, C::GPL, C::PF, kQmvSplitTJ, kQmvSplitNG, 2>),
                       dim3((unsigned)(nblk * nsl)), dim3(64 * kQmvSplitNG), lds, st, x, w,
                       (const uint16_t*)s, (const uint16_t*)b, part, M, (int)N, (int)K,
                       (int64_t)K, nsl);
  } else {
    const size_t lds = qmv_shx_lds<BITS, GS, C::GPL>(1, 16);
    hipLaunchKernelGGL((qmv_split_kernel<DT, BITS, GS, C::GPL, C::PF, kQmvSplitTJ, kQmvSplitNG>),
                       dim3((unsigned)(nblk * nsl)), dim3(64 * kQmvSplitNG), lds, st, x, w,
                       (const uint16_t*)s, (const uint16_t*)b, part, M, (int)N, (int)K,
                       (int64_t)K, nsl);
  }
  const int64_t mn = (int64_t)M * N;
  hipLaunchKernelGGL((qmv_split_sum_kernel<DT, 8>), dim3((unsigned)((mn + 255) / 256)), dim3(256),
                     0, st, part, out, mn);
  return 0;
}

template <int DT, int BITS, int GS, int NW>
inline int skinny_launch_nw(const void* x, const uint32_t* w, const void* s, const void* b,
                            void* out, int64_t M, int64_t N, int64_t K, void* ws, size_t ws_bytes,
                            hipStream_t st, int* nlaunch) {
  using C = QmvConf<BITS, GS>;
  const int G = (int)(K / GS);
  for (int64_t m0 = 0, step = 16; m0 < M; m0 += step, ++*nlaunch) {
    step = 16;
    const int mt = (int)((M - m0) < 16 ? (M - m0) : 16);
    const uint16_t* xp = (const uint16_t*)x + m0 * K;
    uint16_t* op = (uint16_t*)out + m0 * N;
    // 5-64 rows on matrices of few tiles, with the caller's workspace: the
    // K slices on separate workgroups, up to 64 rows per launch (same bits)
    const int ms = (int)((M - m0) < 64 ? (M - m0) : 64);
    if (ws && skinny_split_slices(ms, N, K, BITS, GS) == NW &&
        ws_bytes >= (size_t)ms * N * NW * sizeof(float) && (int64_t)ms * K * 2 < ((int64_t)1 << 31)) {
      if constexpr (QmvGeom<BITS, GS, C::GPL>::STEPK <= 256) {
        if (int rc = skinny_launch_split<DT, BITS, GS>(xp, w, s, b, op, ms, N, K, (float*)ws, NW,
                                                       st))
          return rc;
        ++*nlaunch;
        step = ms;
        continue;
      }
    }
    if constexpr (NW == 4 && QmvGeom<BITS, GS, C::GPL>::STEPK <= 256) {
      // 17-32 rows: one shared-x launch whose groups multiply every weight
      // fragment with two 16-row A tiles (x staged once per step, in one
      // buffer per K slice)
      const int m2 = (int)((M - m0) < 32 ? (M - m0) : 32);
      if (m2 > 16 && (int64_t)m2 * K * 2 < ((int64_t)1 << 31)) {
        const unsigned sg = qmv_shx_grid(N, device_cu_count());
        const size_t lds2 = qmv_x_lds<BITS, GS, C::GPL>(NW, 32) +
                            (size_t)kQmvShxNG * kQmvShxTJ * qmv_sb_lds(G);
        if (sg > 0 && qmv_sb_fits(G, NW, kQmvShxTJ, s, b) && lds2 <= qmv_shx_lds_max(2)) {
          if (int rc = skinny_launch_shx_xm<DT, BITS, GS, 32, false, 2>(xp, w, s, b, op, m2, N, K,
                                                                       lds2, sg, st))
            return rc;
          step = m2;
          continue;
        }
      }
    }
    // x streams through LDS when a buffer range covers its bytes
    int xm = ((int64_t)mt * K * 2 < ((int64_t)1 << 31)) ? qmv_skinny_xm_for<BITS, GS, C::GPL>(mt)
                                                        : 0;
    int tj = qmv_tj_for(xm);
    // 3-4 rows on tall matrices (256+ rows per CU, so still many workgroups
    // per CU): two tiles per x slice (8-bit lm_head N=248320 M=4 258.8 ->
    // 247.3 us; 1-2 rows 0-2% slower that way)
    if (xm == 4 && N >= (int64_t)device_cu_count() * 256) tj = 2;
    if (tj == 2 && !qmv_sb_fits(G, NW, 2, s, b)) tj = 1;
    // two tiles need more than one tile's rows per CU, or half the CUs idle
    // (K=N=4096 M=8: 128 workgroups on 256 CUs, 7.5 us against 5.6 with one)
    if (tj == 2 && N <= 16 * (int64_t)device_cu_count()) tj = 1;
    const bool sbl = qmv_sb_fits(G, NW, tj, s, b);
    // without the scale copy: one tile per workgroup, 8 or 16 streamed rows
    if (!sbl && xm) xm = xm > kQmvMaxXM ? 16 : kQmvMaxXM;
    const size_t lds = qmv_x_lds<BITS, GS, C::GPL>(NW, xm) + (sbl ? tj * qmv_sb_lds(G) : 0);
    int rc = kStatusUnsupported;
    if constexpr (NW == 4) {
      // 5-16 rows with the scale copy on matrices of >= 48 rows per CU: one
      // workgroup of three wave groups per CU, x resident in LDS for 5-8
      // rows, staged once per step for all groups for 9-16 (K=5120 N=17408,
      // one process: M=8 16.7 against 17.5 us, M=16 19.4 against 21.4).
      // Fewer rows keep more, smaller workgroups: there, this geometry lost
      // 1-3 us (M=1 16.3 against 13.2), the x it saves being small.
      const unsigned sg = qmv_shx_grid(N, device_cu_count());
      const size_t lds_sh = qmv_shx_lds<BITS, GS, C::GPL>(NW, xm) +
                            (size_t)kQmvShxNG * kQmvShxTJ * qmv_sb_lds(G);
      const size_t lds_xr = qmv_xres_lds<BITS, GS, C::GPL>(mt, (int)K) +
                            (size_t)kQmvShxNG * kQmvShxTJ * qmv_sb_lds(G);
      if (xm == 8 && qmv_sb_fits(G, NW, kQmvShxTJ, s, b) && sg > 0 && lds_xr <= kQmvShxLdsMax) {
        rc = skinny_launch_shx_xm<DT, BITS, GS, 8, true>(xp, w, s, b, op, mt, N, K, lds_xr, sg, st);
        if (rc) return rc;
        continue;
      }
      if (xm == 16 && qmv_sb_fits(G, NW, kQmvShxTJ, s, b) && sg > 0 && lds_sh <= kQmvShxLdsMax) {
        rc = skinny_launch_shx<DT, BITS, GS>(xm, xp, w, s, b, op, mt, N, K, lds_sh, sg, st);
        if (rc) return rc;
        continue;
      }
    }
#define MQ_SX(X, SB, J)                                                                   \
    if (xm == X && sbl == SB && tj == J)                                                  \
      rc = skinny_launch_one<DT, BITS, GS, NW, X, SB, J>(xp, w, s, b, op, mt, N, K, lds, st);
    MQ_SX(0, true, 1) MQ_SX(1, true, 1) MQ_SX(2, true, 1) MQ_SX(4, true, 1) MQ_SX(4, true, 2)
    MQ_SX(8, true, 1) MQ_SX(8, true, 2) MQ_SX(0, false, 1) MQ_SX(8, false, 1)
    if constexpr (QmvGeom<BITS, GS, C::GPL>::STEPK <= 256) {
      MQ_SX(16, true, 1) MQ_SX(16, true, 2) MQ_SX(16, false, 1)
    }
#undef MQ_SX
    if (rc) return rc;
  }
  return 0;
}

template <int DT, int BITS, int GS>
int SkinnyLaunch<DT, BITS, GS>::run(const void* x, const uint32_t* w, const void* s,
                                    const void* b, void* out, int64_t M, int64_t N, int64_t K,
                                    void* ws, size_t ws_bytes, hipStream_t st, int* nlaunch) {
  if (qmv_nw_for(N) == 8)
    return skinny_launch_nw<DT, BITS, GS, 8>(x, w, s, b, out, M, N, K, ws, ws_bytes, st, nlaunch);
  return skinny_launch_nw<DT, BITS, GS, 4>(x, w, s, b, out, M, N, K, ws, ws_bytes, st, nlaunch);
}

}  // namespace mq
