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
//  * x (M <= 8 rows) streams with the weights: each step's x slice is loaded
//    in the same batch as the step's weights and staged through a per-wave
//    LDS region from which the MFMA A fragments are read (ds_read_b128).  An
//    up-front copy of all of x stalled every wave for microseconds behind the
//    weight prologue in the memory queues.  Lanes whose A row is >= M read
//    row M-1: it only fills output rows that are never stored, since the
//    rows of an MFMA product are independent.  For M > 8 A fragments come
//    from global memory in the same order.
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
#include "launch.h"

namespace mq {

typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) u32x2 lds_u32x2;
typedef __attribute__((address_space(3))) unsigned char lds_u8;

// Buffer resource for a raw (unstructured) byte range.  Word 3 is the gfx9
// default for 32-bit data; out-of-range loads return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

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

// Most A rows whose x slices stream through LDS; more rows read A fragments
// straight from global memory (same arithmetic order).
constexpr int kQmvMaxXM = 8;

// Smallest streamed-x capacity (1, 2, 4, 8) holding M rows, or 0.
inline int qmv_xm_for(int64_t M) {
  return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : M <= kQmvMaxXM ? 8 : 0;
}

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

// Whether a tile's scales/biases can be copied to LDS: rows of whole 16-byte
// chunks (so the copy never splits a chunk across rows), 16-byte aligned
// bases, and at most kQmvSbChunks chunks of each array per thread.
inline bool qmv_sb_fits(int64_t G, int NW, const void* scales, const void* biases) {
  return G % 8 == 0 && 16 * (G / 8) <= (int64_t)kQmvSbChunks * 64 * NW &&
         (reinterpret_cast<uintptr_t>(scales) & 15) == 0 &&
         (reinterpret_cast<uintptr_t>(biases) & 15) == 0;
}

// Row sources of a tile: where the A rows (x) come from and where outputs go.
// Every Rows type gives x (base of all A rows), x_nrec (bytes of x readable
// from x, < 2^31 when x streams through LDS), xoff(m) (element offset of A
// row m from x) and store(m, nn, v).
// Dense: A row m is x row m; output (m, column n0 + nn).
struct DenseRows {
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

// One 16-row weight tile (rows n0 .. n0+rows-1 of a [*, K] quantized matrix
// whose row n0 starts at wt / st / bt; rows <= 0 is an empty tile that only
// joins the barriers) times M <= 16 A rows, computed by a group of NW waves:
// kw is the (wave-uniform) wave index in the group, gt = 64 kw + lane.  The
// group owns qmv_x_lds(NW, XM) (+ qmv_sb_lds(G) when SBL) bytes of LDS at
// qmv_smem and red[0 .. NW-1].  Every wave of the workgroup calls it the same
// number of times (it holds workgroup barriers); requires M <= XM when XM >
// 0, and qmv_sb_fits when SBL.
template <int DT, int BITS, int GS, int GPL, int NW, int PF, int XM, bool SBL, class Rows>
__device__ __forceinline__ void qmv_tile(const char* __restrict__ wt, const char* __restrict__ st,
                                         const char* __restrict__ bt, int rows, int M, int K,
                                         const Rows& src, unsigned char* qmv_smem,
                                         f32x4 (*red)[64], int kw, int gt) {
  using Gm = QmvGeom<BITS, GS, GPL>;
  constexpr int STEPG = Gm::STEPG, STEPB = Gm::STEPB, STEPK = Gm::STEPK, NSV = Gm::NSV;
  constexpr int NL = Gm::NL, CPL = Gm::CPL, MPL = Gm::MPL, SH = Gm::SH;
  // x pieces (16 bytes = 8 codes) of one step: piece i = lane + 64*q covers
  // row i / XPR, codes 8*(i % XPR) of the step.
  constexpr int XPR = STEPK / 8;                          // pieces per x row per step
  constexpr int XPL = XM ? (XM * XPR + 63) / 64 : 1;      // pieces per lane per step
  constexpr int XSR = 2 * STEPK + 16;                     // LDS bytes per x row (padded)
  using T = T16<DT>;
  struct Stage {
    u32x4 w[NL];
    uint32_t s[SBL ? 1 : NSV], b[SBL ? 1 : NSV];
    u32x4 xq[XPL];
  };
  const int lane = threadIdx.x & 63;
  const int wave = kw;
  const int r = lane & 15, c = lane >> 4;
  const uint32_t rowB = (uint32_t)K * BITS / 8;
  const int G = K / GS;
  const uint32_t sRowB = (uint32_t)G * 2;
  const uint32_t w_nrec = rows > 0 ? (uint32_t)(rows - 1) * rowB + STEPB : 0u;
  const uint32_t s_nrec = rows > 0 ? (uint32_t)(rows - 1) * sRowB + STEPG * 2 : 0u;
  const uint32_t wofs = (uint32_t)r * rowB + (uint32_t)c * 16;
  const uint32_t sofs = (uint32_t)r * sRowB;
  // scale of load L: half ((4 L + c) >> SH) & 3 of dword pair ((4 L) >> SH) >> 2
  uint32_t selL[NL];
#pragma unroll
  for (int L = 0; L < NL; ++L) selL[L] = half_selector<DT>(((4 * L + c) >> SH) & 3);

  const int nsteps = (G + STEPG - 1) / STEPG;
  const int full = G / STEPG;                 // steps with every group inside K
  const int sb = (int)((int64_t)nsteps * wave / NW);
  const int se = (int)((int64_t)nsteps * (wave + 1) / NW);
  const int fe = se < full ? se : full;      // pipelined (unchecked) steps: [sb, fe)

  const int xr = min(r, M - 1);              // A row of this lane (rows >= M repeat row M-1)
  lds_u8* xreg = (lds_u8*)qmv_smem + wave * (XM ? XM : 1) * XSR;
  const lds_u8* xl = xreg + xr * XSR;
  const uint16_t* xg = src.x + src.xoff(xr);
  const int SBS = qmv_sb_stride(G);
  lds_u8* sbl_s = (lds_u8*)qmv_smem + NW * (XM ? XM : 1) * XSR;
  lds_u8* sbl_b = sbl_s + 16 * SBS;
  // XM > 0: byte offset of this lane's x pieces from the step's x slice;
  // pieces of rows >= M are out of the buffer range (no memory access, zeros)
  uint32_t xvo[XPL];
  int xpk[XPL];
#pragma unroll
  for (int q = 0; q < XPL; ++q) {
    const int i = lane + 64 * q;
    const int m = i / XPR;
    xpk[q] = 8 * (i - m * XPR);
    xvo[q] = (m < M) ? (uint32_t)(src.xoff(m) + xpk[q]) * 2u : 0x80000000u;
  }

  auto load = [&](Stage& s, int t, bool live) {
    if constexpr (XM > 0) {
      const uint32_t xstep = (uint32_t)t * STEPK * 2;
      const auto rx = make_rsrc(reinterpret_cast<const char*>(src.x) + xstep,
                                live ? src.x_nrec - xstep : 0u);
#pragma unroll
      for (int q = 0; q < XPL; ++q)
        s.xq[q] = __builtin_amdgcn_raw_buffer_load_b128(rx, xvo[q], 0, 0);
    }
    const auto rw = make_rsrc(wt + (int64_t)t * STEPB, live ? w_nrec : 0u);
#pragma unroll
    for (int L = 0; L < NL; ++L)
      s.w[L] = __builtin_amdgcn_raw_buffer_load_b128(rw, wofs + L * 64, 0, 0);
    if constexpr (!SBL) {
      const auto rs = make_rsrc(st + (int64_t)t * STEPG * 2, live ? s_nrec : 0u);
      const auto rb = make_rsrc(bt + (int64_t)t * STEPG * 2, live ? s_nrec : 0u);
      if constexpr (NSV == 2) {
        const u32x2 a = __builtin_amdgcn_raw_buffer_load_b64(rs, sofs, 0, 0);
        const u32x2 q = __builtin_amdgcn_raw_buffer_load_b64(rb, sofs, 0, 0);
        s.s[0] = a[0]; s.s[1] = a[1]; s.b[0] = q[0]; s.b[1] = q[1];
      } else {
#pragma unroll
        for (int v = 0; v < NSV / 4; ++v) {
          const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(rs, sofs + 16 * v, 0, 0);
          const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(rb, sofs + 16 * v, 0, 0);
#pragma unroll
          for (int e = 0; e < 4; ++e) { s.s[4 * v + e] = a[e]; s.b[4 * v + e] = q[e]; }
        }
      }
    }
  };

  f32x4 acc = {0.f, 0.f, 0.f, 0.f};

  // A fragment covering codes [k, k+8): k relative to the step (LDS slice) or
  // absolute (global).  Codes past K read zeros (LDS slices are zeroed there).
  auto afrag = [&](int krel, int kabs, bool checked) -> u32x4 {
    if constexpr (XM > 0) {
      (void)kabs; (void)checked;
      return *(const lds_u32x4*)(xl + 2 * krel);
    } else {
      (void)krel;
      if (checked && kabs >= K) return (u32x4){0u, 0u, 0u, 0u};
      return *reinterpret_cast<const u32x4*>(xg + kabs);
    }
  };

  auto compute = [&](const Stage& s, int t, bool checked) {
    if constexpr (XM > 0) {
#pragma unroll
      for (int q = 0; q < XPL; ++q) {
        const int i = lane + 64 * q;
        if (XPL * 64 == XM * XPR || i < XM * XPR) {
          u32x4 v = s.xq[q];
          if (checked && t * STEPK + xpk[q] >= K) v = (u32x4){0u, 0u, 0u, 0u};
          *(lds_u32x4*)(xreg + (i / XPR) * XSR + 2 * xpk[q]) = v;
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    uint32_t sv[NSV], bv[NSV];
    if constexpr (SBL) {
      const lds_u8* ps = sbl_s + r * SBS + t * STEPG * 2;
      const lds_u8* pb = sbl_b + r * SBS + t * STEPG * 2;
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
      for (int v = 0; v < NSV; ++v) { sv[v] = s.s[v]; bv[v] = s.b[v]; }
    }
    float sf[NL], bf[NL];
    bool big = false;
#pragma unroll
    for (int L = 0; L < NL; ++L) {
      const int q = ((4 * L) >> SH) >> 2;     // same for the 4 lanes of a row
      sf[L] = selected_to_f32<DT>(__builtin_amdgcn_perm(sv[2 * q + 1], sv[2 * q], selL[L]));
      bf[L] = selected_to_f32<DT>(__builtin_amdgcn_perm(bv[2 * q + 1], bv[2 * q], selL[L]));
      if (checked && t * STEPG + ((4 * L + c) >> SH) >= G) { sf[L] = 0.f; bf[L] = 0.f; }
      big |= needs_plain(sf[L]);
    }
    const int kr = c * CPL;                   // lane's first code, relative to the step
    const int kt = t * STEPK + kr;            // same, absolute
    if (__builtin_amdgcn_ballot_w64(big) == 0) {
#pragma unroll
      for (int L = 0; L < NL; ++L) {
        const GroupScale g = make_group(sf[L], bf[L]);
#pragma unroll
        for (int p = 0; p < MPL; ++p) {
          uint32_t bo[4];
          if constexpr (BITS == 4) {
            deq4_word<DT>(s.w[L][p], g, bo);
          } else {
            deq8_word<DT>(s.w[L][2 * p], g, bo);
            deq8_word<DT>(s.w[L][2 * p + 1], g, bo + 2);
          }
          const int ko = 4 * L * CPL + 8 * p;
          const u32x4 a = afrag(kr + ko, kt + ko, checked);
          acc = T::mfma(a, (u32x4){bo[0], bo[1], bo[2], bo[3]}, acc);
        }
      }
    } else {
#pragma unroll
      for (int L = 0; L < NL; ++L) {
        const GroupScale g = make_group(sf[L], bf[L]);
#pragma unroll
        for (int p = 0; p < MPL; ++p) {
          uint32_t bo[4];
          if constexpr (BITS == 4) {
            deq_word_plain<DT, 4>(s.w[L][p], g, bo);
          } else {
            deq_word_plain<DT, 8>(s.w[L][2 * p], g, bo);
            deq_word_plain<DT, 8>(s.w[L][2 * p + 1], g, bo + 2);
          }
          const int ko = 4 * L * CPL + 8 * p;
          const u32x4 a = afrag(kr + ko, kt + ko, checked);
          acc = T::mfma(a, (u32x4){bo[0], bo[1], bo[2], bo[3]}, acc);
        }
      }
    }
  };

  // ---- scale/bias copy: loads issued ahead of the weight prologue ---------
  Stage S[PF];
  u32x4 sbq[2][SBL ? kQmvSbChunks : 1];
  const int cpr = G / 8;                      // 16-byte chunks per scale row (SBL)
  const int nch = max(rows, 0) * cpr;         // chunks of each of s and b
  if constexpr (SBL) {
    const auto rs0 = make_rsrc(st, (uint32_t)nch * 16u);
    const auto rb0 = make_rsrc(bt, (uint32_t)nch * 16u);
#pragma unroll
    for (int u = 0; u < kQmvSbChunks; ++u) {
      const uint32_t i = gt + u * 64 * NW;
      sbq[0][u] = __builtin_amdgcn_raw_buffer_load_b128(rs0, i * 16u, 0, 0);
      sbq[1][u] = __builtin_amdgcn_raw_buffer_load_b128(rb0, i * 16u, 0, 0);
    }
  }
  // ---- main loop: PF-stage pipeline over the unchecked steps --------------
#pragma unroll
  for (int i = 0; i < PF - 1; ++i) load(S[i], sb + i, sb + i < fe);
  if constexpr (SBL) {
#pragma unroll
    for (int u = 0; u < kQmvSbChunks; ++u) {
      const int i = gt + u * 64 * NW;
      if (i < nch) {
        const int rr = i / cpr, cc = i - rr * cpr;
        *(lds_u32x4*)(sbl_s + rr * SBS + cc * 16) = sbq[0][u];
        *(lds_u32x4*)(sbl_b + rr * SBS + cc * 16) = sbq[1][u];
      }
    }
    __syncthreads();
  }
  for (int t = sb; t < fe; t += PF) {
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int tl = t + i + PF - 1;
      load(S[(i + PF - 1) % PF], tl, tl < fe);
      if (t + i < fe) compute(S[i], t + i, false);
    }
  }
  // ---- ragged tail: at most one step; groups past K are zeroed ------------
  if (fe < se) {
    Stage s;
    load(s, fe, true);
#pragma unroll
    for (int L = 0; L < NL; ++L)
      if (fe * STEPG + ((4 * L + c) >> SH) >= G) s.w[L] = (u32x4){0u, 0u, 0u, 0u};
    compute(s, fe, true);
  }

  // ---- sum the waves' partial tiles in wave order, round once -------------
  // lane l holds D[4*(l>>4)+v][l&15]: output row 4c+v, column r of the tile
  if constexpr (NW == 1) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = 4 * c + v;
      if (m < M && r < rows) src.store(m, r, T::round1(acc[v]));
    }
  } else {
    red[wave][lane] = acc;
    __syncthreads();
    for (int tt = gt; tt < 256; tt += 64 * NW) {
      const int mm = tt >> 4, nn = tt & 15;
      const int sl = ((mm >> 2) << 4) | nn, v = mm & 3;
      float sum = red[0][sl][v];
#pragma unroll
      for (int q = 1; q < NW; ++q) sum += red[q][sl][v];
      if (mm < M && nn < rows) src.store(mm, nn, T::round1(sum));
    }
    // the next tile of this workgroup reuses red and the LDS copies
    __syncthreads();
  }
}

// grid.x = ceil(N / 16) tiles, block = 64 * NW threads, dynamic LDS
// qmv_x_lds<BITS, GS, GPL>(NW, XM) (+ qmv_sb_lds(K / GS) when SBL) bytes;
// M <= XM unless XM == 0, and then ((M - 1) * ldx + K) * 2 < 2^31.
template <int DT, int BITS, int GS, int GPL, int NW, int PF, int XM, bool SBL>
__global__ __launch_bounds__(64 * NW) void qmv_kernel(const uint16_t* __restrict__ x,
                                                      const uint32_t* __restrict__ w,
                                                      const uint16_t* __restrict__ scales,
                                                      const uint16_t* __restrict__ biases,
                                                      uint16_t* __restrict__ out, int M, int N,
                                                      int K, int64_t ldx, int64_t ldo) {
  extern __shared__ __align__(16) unsigned char qmv_smem[];
  __shared__ f32x4 red[NW][64];
  const int n0 = blockIdx.x * 16;
  const uint32_t rowB = (uint32_t)K * BITS / 8;
  const uint32_t sRowB = (uint32_t)(K / GS) * 2;
  const DenseRows src{x, (uint32_t)(((int64_t)(M - 1) * ldx + K) * 2), out, ldx, ldo, n0};
  qmv_tile<DT, BITS, GS, GPL, NW, PF, XM, SBL>(
      reinterpret_cast<const char*>(w) + (int64_t)n0 * rowB,
      reinterpret_cast<const char*>(scales) + (int64_t)n0 * sRowB,
      reinterpret_cast<const char*>(biases) + (int64_t)n0 * sRowB, min(16, N - n0), M, K, src,
      qmv_smem, red, __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), threadIdx.x);
}

template <int DT, int BITS, int GS, int NW>
inline void skinny_launch_nw(const void* x, const uint32_t* w, const void* s, const void* b,
                             void* out, int64_t M, int64_t N, int64_t K, hipStream_t st) {
  using C = QmvConf<BITS, GS>;
  const unsigned grid = (unsigned)((N + 15) / 16);
  const bool sbl = qmv_sb_fits(K / GS, NW, s, b);
  const size_t sb_lds = qmv_sb_lds((int)(K / GS));
  auto lds_for = [&](int xmax, bool with_sb) {
    return qmv_x_lds<BITS, GS, C::GPL>(NW, xmax) + (with_sb ? sb_lds : 0);
  };
  for (int64_t m0 = 0; m0 < M; m0 += 16) {
    const int mt = (int)((M - m0) < 16 ? (M - m0) : 16);
    const uint16_t* xp = (const uint16_t*)x + m0 * K;
    uint16_t* op = (uint16_t*)out + m0 * N;
    // x streams through LDS for up to 8 rows whose bytes a buffer range covers;
    // without the scale copy only the 8-row streamed-x variant is built
    int xm = ((int64_t)mt * K * 2 < ((int64_t)1 << 31)) ? qmv_xm_for(mt) : 0;
    if (!sbl && xm) xm = kQmvMaxXM;
#define MQ_SX(X, SB)                                                                        \
    if (xm == X && sbl == SB)                                                               \
      hipLaunchKernelGGL((qmv_kernel<DT, BITS, GS, C::GPL, NW, C::PF, X, SB>), dim3(grid),    \
                         dim3(64 * NW), lds_for(X, SB), st, xp, w, (const uint16_t*)s,      \
                         (const uint16_t*)b, op, mt, (int)N, (int)K, (int64_t)K, (int64_t)N);
    MQ_SX(0, true) MQ_SX(1, true) MQ_SX(2, true) MQ_SX(4, true) MQ_SX(8, true)
    MQ_SX(0, false) MQ_SX(8, false)
#undef MQ_SX
  }
}

template <int DT, int BITS, int GS>
int SkinnyLaunch<DT, BITS, GS>::run(const void* x, const uint32_t* w, const void* s,
                                    const void* b, void* out, int64_t M, int64_t N, int64_t K,
                                    hipStream_t st) {
  if (qmv_nw_for(N) == 8) skinny_launch_nw<DT, BITS, GS, 8>(x, w, s, b, out, M, N, K, st);
  else skinny_launch_nw<DT, BITS, GS, 4>(x, w, s, b, out, M, N, K, st);
  return 0;
}

}  // namespace mq
