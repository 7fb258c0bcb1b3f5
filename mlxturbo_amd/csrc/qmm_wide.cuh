// Wide (prefill) quantized matmul: out[M,N] = x[M,K] . deq(W[N,K])^T for M > 16,
// and the same tile over expert-grouped rows for prefill gather_qmm.
//
// Reference behaviour: mlxturbo/kernels/qmm_wide.py:456-502 (MLX steel
// qmm_t with a 64-row tile), reached from fused._qmm_wide_dispatch
// (fused.py:3477-3499) for prefill chunks; the MLX loader dequantizes each W
// tile to T in threadgroup memory (_steel_flat.py:1324-1335).  The grouped
// form follows moe_grouped_gemm.qmm_segmented (moe_grouped_gemm.py:913-1066):
// rows sorted by expert, each tile belongs to one expert.
//
// CDNA4 design (compute-bound: arithmetic intensity 1247-3483 FLOP/B at
// M = 512..8192, above the ~312 FLOP/B ridge):
//  * Block tile BM x 256, BK = 64 codes, 512 threads = 8 waves, two per SIMD
//    (one wave per SIMD left the LDS reads latency-bound: measured 213 B/ns
//    per CU with one wave per SIMD against 430 with four).  BM = 256: waves
//    in a 4 x 2 grid of 64 x 128 outputs (2 x 4 tiles of v_mfma_f32_32x32x16);
//    BM = 128 / 64 for shorter row counts.
//  * Per k-step the workgroup stages x[BM x 64] and the dequantized W[256 x
//    64] (T, exact MLX dequant) in LDS, rows padded to 144 bytes so the
//    16-lane phases of ds_read_b128 hit distinct banks (no bank conflicts in
//    SQ_LDS_BANK_CONFLICT).  Two LDS buffers and two register stages: the
//    global loads of step k+2 are issued while step k runs its MFMAs and the
//    data of step k+1, loaded a whole step earlier, is dequantized into the
//    other buffer; the loop body is straight-line so the compiler can
//    interleave the stores with the MFMAs.  With one register stage, 44% of
//    wave cycles waited on global loads (SQ_WAIT_INST_ANY).
//  * x, W, scales and biases are read with buffer loads; rows past M (or past
//    N) are past the buffer range and read zeros, so no row clamping.
//  * Each weight is dequantized once per BM output rows; a whole tile whose
//    scales include |s| >= 2^100 (never in real checkpoints) is recomputed on
//    the plain float dequantization route: the fast route checks each scale
//    as it uses it, so no tile waits for a scan of its scales before its
//    first weight load.
#pragma once
#include <type_traits>

#include "launch.h"

namespace mq {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kWideBN = 256, kWideBK = 64, kWideNT = 512;
constexpr int kWideLD = kWideBK + 8;  // LDS row stride in 16-bit elements (144 bytes)

template <int BM>
constexpr size_t wide_lds_bytes() { return 2 * (size_t)(BM + kWideBN) * kWideLD * 2; }

template <int DT>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (DT == kBF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(bitcast<bf16x8>(a), bitcast<bf16x8>(b), c, 0,
                                                   0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(bitcast<f16x8>(a), bitcast<f16x8>(b), c, 0, 0,
                                                  0);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t wide_rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0,
                                           (int)(bytes < 0x7fffffff ? bytes : 0x7fffffff),
                                           0x00020000);
}

// f(integral_constant<int, 0>) ... f(integral_constant<int, N - 1>), in order
template <int I, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// One BM x 256 output tile over k-steps kt0 .. kt0 + nkl - 1 (64 codes each).
// x rows come from xrsrc at per-row byte offsets xrow_off(r) (past the range
// for rows that do not exist); w / scales / biases point at the tile's first
// weight row, of which nrows (<= 256) exist; store(r, c, v) receives the
// float sum of row r, tile column c (< nrows).
// FRESH: the caller's tiles do not share weight tiles through L2 (grouped
// segments), which enables per-block scale loads below.
template <int DT, int BITS, int GS, int BM, class XRowOff, class Store, bool FRESH = false>
__device__ __forceinline__ void wide_tile(__amdgpu_buffer_rsrc_t xrsrc, XRowOff xrow_off,
                                          const uint32_t* __restrict__ w,
                                          const uint16_t* __restrict__ scales,
                                          const uint16_t* __restrict__ biases, int nrows, int K,
                                          int kt0, int nkl, Store store, uint16_t* wide_smem) {
  constexpr int BN = kWideBN, BK = kWideBK, LD = kWideLD, NT = kWideNT;
  constexpr int WGM = BM == 256 ? 4 : 2;        // waves along M
  constexpr int WGN = 8 / WGM;                  // waves along N
  constexpr int TM = BM / WGM / 32, TN = BN / WGN / 32;
  constexpr int WCH = BK * BITS / 128;          // 16-byte weight chunks per row per step
  constexpr int WCT = BN * WCH;                 // weight chunks per step
  static_assert(WCT % NT == 0, "whole weight chunks per thread");
  constexpr int WPT = WCT / NT;                 // weight chunks per thread
  constexpr int XPT = BM * 8 / NT;              // x chunks per thread
  constexpr int XROWS = NT / 8;                 // tile rows between a thread's x chunks
  constexpr int CPC = 128 / BITS;               // codes per chunk
  constexpr int KS = BK / 16;                   // MFMA k-substeps per step
  static_assert(XPT >= 1 && (XPT % KS == 0 || XPT < KS), "x chunks spread over substeps");
  using T = T16<DT>;
  uint16_t* As = wide_smem;                     // [2][BM*LD]
  uint16_t* Bs = wide_smem + 2 * BM * LD;       // [2][BN*LD]

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = wave / WGN, wn = wave % WGN;
  const int64_t Kw = (int64_t)K * BITS / 32;
  const int G = K / GS;
  const int nk = nkl;

  // rows past nrows are past the weight range and read zeros
  const auto rwd = wide_rsrc(w, (int64_t)nrows * Kw * 4);
  const auto rsd = wide_rsrc(scales, (int64_t)nrows * G * 2);
  const auto rbd = wide_rsrc(biases, (int64_t)nrows * G * 2);
  uint32_t xo[XPT];
#pragma unroll
  for (int i = 0; i < XPT; ++i) {
    const uint32_t ro = xrow_off((t >> 3) + XROWS * i);
    xo[i] = ro == 0xffffffffu ? 0xffffffffu : ro + 16u * (t & 7);
  }
  const int xl0 = (t >> 3) * LD + 8 * (t & 7);
  uint32_t wo[WPT], so[WPT];
  int wl[WPT], wch[WPT];
#pragma unroll
  for (int i = 0; i < WPT; ++i) {
    const int id = t + NT * i;
    const int row = id / WCH, ch = id % WCH;
    wo[i] = (uint32_t)(((int64_t)row * Kw + ch * CPC * BITS / 32) * 4);
    so[i] = (uint32_t)((int64_t)min(row, nrows - 1) * G * 2);
    wl[i] = row * LD + ch * CPC;
    wch[i] = ch;
  }

  struct Set {
    u32x4 xa[XPT];
    u32x4 wv[WPT];
    uint16_t s[WPT], b[WPT];
  };
  Set S0, S1;
  bool big = false;   // a scale with |s| >= 2^100 met on the fast route
  // Scales and biases, 64- and 128-row tiles of weights that no other tile
  // reads through L2 (on dense tiles it cost 1.5-4%), K / GS a multiple of 8,
  // both arrays 16-byte aligned and whose k range is whole blocks of SPB
  // steps: each thread loads the 16-byte block (8 groups) of its rows'
  // scales and biases with the block's first step (ns / nb) and takes it
  // over (cs / cb) when that step is stored, instead of two 2-byte loads
  // per step; the loop is unrolled over a block so every block load and
  // every group index is fixed at compile time.  A tile streaming fresh
  // weights (a thin expert) spends ~15% of its time on the per-step
  // requests at K = 2048.
  constexpr int SPB = GS / 8;                   // 64-code steps per block
  constexpr bool SBLK = FRESH && BM <= 128 && SPB >= 4 && SPB <= 8;
  const bool sblk = SBLK && G % 8 == 0 && kt0 % SPB == 0 && nk % SPB == 0 &&
                    ((uintptr_t)scales | (uintptr_t)biases) % 16 == 0;
  u32x4 ns[WPT], nb[WPT], cs[WPT], cb[WPT];
  auto bload = [&](int kt) {
    const uint32_t bo = 16u * (uint32_t)((kt0 + kt) * BK / GS / 8);
#pragma unroll
    for (int i = 0; i < WPT; ++i) {
      ns[i] = __builtin_amdgcn_raw_buffer_load_b128(rsd, so[i] + bo, 0, 0);
      nb[i] = __builtin_amdgcn_raw_buffer_load_b128(rbd, so[i] + bo, 0, 0);
    }
  };
  auto gload_w = [&](Set& st, int kt) {
    const int k0 = (kt0 + kt) * BK;
#pragma unroll
    for (int i = 0; i < XPT; ++i)
      st.xa[i] = __builtin_amdgcn_raw_buffer_load_b128(xrsrc, xo[i], k0 * 2, 0);
#pragma unroll
    for (int i = 0; i < WPT; ++i)
      st.wv[i] = __builtin_amdgcn_raw_buffer_load_b128(rwd, wo[i], k0 * BITS / 8, 0);
  };
  auto gload = [&](Set& st, int kt) {
    const int k0 = (kt0 + kt) * BK;
#pragma unroll
    for (int i = 0; i < XPT; ++i)
      st.xa[i] = __builtin_amdgcn_raw_buffer_load_b128(xrsrc, xo[i], k0 * 2, 0);
#pragma unroll
    for (int i = 0; i < WPT; ++i) {
      st.wv[i] = __builtin_amdgcn_raw_buffer_load_b128(rwd, wo[i], k0 * BITS / 8, 0);
      const uint32_t go = so[i] + 2u * (uint32_t)((k0 + wch[i] * CPC) / GS);
      st.s[i] = __builtin_amdgcn_raw_buffer_load_b16(rsd, go, 0, 0);
      st.b[i] = __builtin_amdgcn_raw_buffer_load_b16(rbd, go, 0, 0);
    }
  };
  // part ks of storing register stage st into LDS buffer buf
  // LB >= 0: step LB of an aligned block, scales from cs / cb
  auto spart = [&](const Set& st, int buf, int ks, auto plainc, auto lbc) {
    constexpr int LB = decltype(lbc)::value;
    constexpr bool PLAIN = decltype(plainc)::value;
    uint16_t* A = As + buf * BM * LD;
    uint16_t* B = Bs + buf * BN * LD;
    if constexpr (XPT >= KS) {
#pragma unroll
      for (int i = ks * (XPT / KS); i < (ks + 1) * (XPT / KS); ++i)
        *reinterpret_cast<u32x4*>(A + xl0 + i * XROWS * LD) = st.xa[i];
    } else {
      if (ks < XPT) *reinterpret_cast<u32x4*>(A + xl0 + ks * XROWS * LD) = st.xa[ks];
    }
    constexpr int WW = 4 * WPT;                 // weight words per thread
#pragma unroll
    for (int q = ks * WW / KS; q < (ks + 1) * WW / KS; ++q) {
      const int i = q / 4, j = q % 4;
      uint16_t s16, b16;
      if constexpr (LB >= 0) {
        // group of this chunk within the block (a constant for GS >= 64)
        const int e = GS >= BK ? LB * BK / GS % 8 : (LB * BK + wch[i] * CPC) / GS % 8;
        const uint32_t ws = (e & 4) ? ((e & 2) ? cs[i][3] : cs[i][2]) : ((e & 2) ? cs[i][1] : cs[i][0]);
        const uint32_t wb = (e & 4) ? ((e & 2) ? cb[i][3] : cb[i][2]) : ((e & 2) ? cb[i][1] : cb[i][0]);
        s16 = (uint16_t)((e & 1) ? ws >> 16 : ws);
        b16 = (uint16_t)((e & 1) ? wb >> 16 : wb);
      } else {
        s16 = st.s[i];
        b16 = st.b[i];
      }
      const GroupScale g = make_group(T::to_f32(s16), T::to_f32(b16));
      if constexpr (!PLAIN) big |= needs_plain(g.s);
      uint32_t o[CPC / 8];
      if constexpr (PLAIN) deq_word_plain<DT, BITS>(st.wv[i][j], g, o);
      else deq_word<DT, BITS>(st.wv[i][j], g, o);
      uint32_t* dst = reinterpret_cast<uint32_t*>(B + wl[i] + j * (CPC / 4));
      if constexpr (CPC / 8 == 4) *reinterpret_cast<u32x4*>(dst) = (u32x4){o[0], o[1], o[2], o[3]};
      else *reinterpret_cast<u32x2*>(dst) = (u32x2){o[0], o[1]};
    }
  };

  f32x16 acc[TM][TN];
  auto clear = [&]() {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
  };

  const int lr = lane & 31, lk = 8 * (lane >> 5);
  auto mma = [&](int buf) {
    const uint16_t* A = As + buf * BM * LD + (32 * TM * wm + lr) * LD + lk;
    const uint16_t* B = Bs + buf * BN * LD + (32 * TN * wn + lr) * LD + lk;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4 a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) a[i] = *reinterpret_cast<const u32x4*>(A + 32 * i * LD + 16 * ks);
#pragma unroll
      for (int j = 0; j < TN; ++j) b[j] = *reinterpret_cast<const u32x4*>(B + 32 * j * LD + 16 * ks);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma32<DT>(a[i], b[j], acc[i][j]);
    }
  };

  auto run = [&](auto plainc) {
    clear();
    auto stage_store = [&](const Set& st, int buf) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) spart(st, buf, ks, plainc, std::integral_constant<int, -1>{});
    };
    // step LB of an aligned block; its first step takes over the block loaded
    auto stage_store_b = [&](const Set& st, int buf, auto lbc) {
      if constexpr (decltype(lbc)::value == 0) {
#pragma unroll
        for (int i = 0; i < WPT; ++i) {
          cs[i] = ns[i];
          cb[i] = nb[i];
        }
      }
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) spart(st, buf, ks, plainc, lbc);
    };
    if constexpr (SBLK) {
      if (sblk) {
        gload_w(S0, 0);
        bload(0);
        gload_w(S1, 1);
        stage_store_b(S0, 0, std::integral_constant<int, 0>{});
        __syncthreads();
        // Each pass runs one block (SPB steps, an even number); the loads
        // for steps past the end reload step nk - 1 (valid memory, unused).
        for (int kb = 0; kb < nk; kb += SPB) {
          static_for<0, SPB / 2>([&](auto hc) {
            constexpr int h = decltype(hc)::value;
            constexpr bool next = 2 * h + 2 == SPB;   // step kb + 2h + 2 opens a block
            // buffer 0 holds step kb + 2h, S1 step kb + 2h + 1, S0 is free
            gload_w(S0, min(kb + 2 * h + 2, nk - 1));
            if constexpr (next) bload(min(kb + SPB, nk - SPB));
            mma(0);
            stage_store_b(S1, 1, std::integral_constant<int, 2 * h + 1>{});
            __syncthreads();
            // buffer 1 holds step kb + 2h + 1, S0 step kb + 2h + 2, S1 is free
            gload_w(S1, min(kb + 2 * h + 3, nk - 1));
            mma(1);
            stage_store_b(S0, 0, std::integral_constant<int, (2 * h + 2) % SPB>{});
            __syncthreads();
          });
        }
        return;
      }
    }
    gload(S0, 0);
    gload(S1, min(1, nk - 1));
    stage_store(S0, 0);
    __syncthreads();
    // The last iterations reload step nk - 1 (valid memory, unused) so the
    // body stays free of load conditions.
    for (int kt = 0; kt < nk; kt += 2) {
      // buffer 0 holds step kt, S1 step kt + 1, S0 is free
      gload(S0, min(kt + 2, nk - 1));
      mma(0);
      stage_store(S1, 1);
      __syncthreads();
      if (kt + 1 < nk) {
        // buffer 1 holds step kt + 1, S0 step kt + 2, S1 is free
        gload(S1, min(kt + 3, nk - 1));
        mma(1);
        stage_store(S0, 0);
        __syncthreads();
      }
    }
  };
  // Optimistic fast dequantization: every scale a thread uses on the fast
  // path is checked as it is used; a tile that met |s| >= 2^100 (never in
  // real checkpoints) is recomputed from scratch on the plain float route
  // before anything is stored.
  run(std::integral_constant<bool, false>{});
  if (__syncthreads_or(big)) run(std::integral_constant<bool, true>{});

  // D[row][col] of a 32x32 tile: col = lane & 31, row = 8*(e/4) + 4*(lane>>5) + e%4
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int c = 32 * TN * wn + 32 * j + lr;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int r = 32 * TM * wm + 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        if (c < nrows) store(r, c, acc[i][j][e]);
      }
    }
}

// Dense rows: grid (ceil(N / 256), ceil(M / BM), splits), 512 threads,
// dynamic LDS wide_lds_bytes<BM>(); 256 * K * 2 < 2^31 and 256 * K * BITS / 8
// < 2^31.  With part == nullptr (splits == 1) the tile rounds its sums into
// out; otherwise split z sums k-steps [z nk / splits, (z + 1) nk / splits)
// into the float plane part[z] ([M, N]) and wide_reduce_kernel adds the
// planes in split order.
template <int DT, int BITS, int GS, int BM>
__global__ __launch_bounds__(kWideNT) void qmm_wide_kernel(const uint16_t* __restrict__ x,
                                                           const uint32_t* __restrict__ w,
                                                           const uint16_t* __restrict__ scales,
                                                           const uint16_t* __restrict__ biases,
                                                           uint16_t* __restrict__ out,
                                                           float* __restrict__ part, int M,
                                                           int N, int K) {
  extern __shared__ __align__(16) uint16_t wide_smem[];
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * kWideBN;
  const int mrows = min(BM, M - m0);
  const int64_t G = K / GS;
  const int nk = K / kWideBK, z = blockIdx.z, splits = gridDim.z;
  const int kt0 = (int)((int64_t)nk * z / splits), kt1 = (int)((int64_t)nk * (z + 1) / splits);
  // descriptors cover this tile's rows only: rows past M read zeros, no
  // 64-bit offsets inside the tile
  const auto xr = wide_rsrc(x + (int64_t)m0 * K, (int64_t)mrows * K * 2);
  auto xrow_off = [&](int r) { return (uint32_t)r * (uint32_t)K * 2u; };
  if (part) {
    float* pt = part + ((int64_t)z * M + m0) * N + n0;
    auto store = [&](int r, int c, float v) {
      if (r < mrows) pt[(int64_t)r * N + c] = v;
    };
    wide_tile<DT, BITS, GS, BM>(xr, xrow_off, w + (int64_t)n0 * K * BITS / 32, scales + n0 * G,
                                biases + n0 * G, min(kWideBN, N - n0), K, kt0, kt1 - kt0, store,
                                wide_smem);
  } else {
    uint16_t* ot = out + (int64_t)m0 * N + n0;
    auto store = [&](int r, int c, float v) {
      if (r < mrows) ot[(int64_t)r * N + c] = T16<DT>::round1(v);
    };
    wide_tile<DT, BITS, GS, BM>(xr, xrow_off, w + (int64_t)n0 * K * BITS / 32, scales + n0 * G,
                                biases + n0 * G, min(kWideBN, N - n0), K, kt0, kt1 - kt0, store,
                                wide_smem);
  }
}

// out = round(sum over splits of part[s]) in split order, 4 elements per
// thread; grid ceil(M * N / 1024), 256 threads.
template <int DT>
__global__ __launch_bounds__(256) void wide_reduce_kernel(const float* __restrict__ part,
                                                          uint16_t* __restrict__ out,
                                                          int64_t MN, int splits) {
  const int64_t i0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int64_t i = i0 + e;
    if (i < MN) {
      float v = part[i];
      for (int z = 1; z < splits; ++z) v += part[(int64_t)z * MN + i];
      out[i] = T16<DT>::round1(v);
    }
  }
}

// One expert-grouped tile (prefill gather_qmm, reference moe_grouped_gemm.py:
// 913-1066): segment seg of the prep tables in ws (up to BM / Mi pairs of one
// expert, pairs sorted by expert) times the 256 columns from n0.  Pair p
// contributes rows p*Mi .. p*Mi+Mi-1 of the output and reads x batch
// x_batch(lhs, p, P, B).  Segments of out-of-range experts write zeros.  s_xoff / s_orow
// hold BM entries of LDS; B * Mi * K * 2 < 2^31.
template <int DT, int BITS, int GS, int BM>
__device__ __forceinline__ void grouped_body(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ w,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    const int32_t* __restrict__ lhs, uint16_t* __restrict__ out, const int32_t* __restrict__ ws,
    int P, int B, int Mi, int N, int K, int E, int seg, int n0, uint16_t* wide_smem,
    uint32_t* s_xoff, int* s_orow) {
  const int32_t* perm = ws + 1;
  const int st0 = perm[P + seg], len = perm[2 * P + seg], e = perm[3 * P + seg];
  const int rows = len * Mi;                      // <= BM
  const int t = threadIdx.x;
  for (int r = t; r < BM; r += kWideNT) {
    if (r < rows) {
      const int p = perm[st0 + r / Mi], mi = r % Mi;
      const int xb = x_batch(lhs, p, P, B);
      s_xoff[r] = (uint32_t)(((int64_t)xb * Mi + mi) * K * 2);
      s_orow[r] = p * Mi + mi;
    } else {
      s_xoff[r] = 0xffffffffu;
      s_orow[r] = -1;
    }
  }
  __syncthreads();
  const int ncols = min(kWideBN, N - n0);
  if (e >= E) {
    for (int i = t; i < rows * ncols; i += kWideNT) {
      const int r = i / ncols, c = i - r * ncols;
      out[(int64_t)s_orow[r] * N + n0 + c] = 0;
    }
    return;
  }
  const int64_t G = K / GS;
  const int64_t wrow = (int64_t)e * N + n0;
  const auto xr = wide_rsrc(x, (int64_t)B * Mi * K * 2);
  auto xrow_off = [&](int r) { return s_xoff[r]; };
  uint16_t* ot = out + n0;
  auto store = [&](int r, int c, float v) {
    const int o = s_orow[r];
    if (o >= 0) ot[(int64_t)o * N + c] = T16<DT>::round1(v);
  };
  wide_tile<DT, BITS, GS, BM, decltype(xrow_off), decltype(store), true>(
      xr, xrow_off, w + wrow * K * BITS / 32, scales + wrow * G, biases + wrow * G, ncols, K, 0,
      K / kWideBK, store, wide_smem);
}

// Expert-grouped tiles of one height over the prep tables' size class cls:
// 1-D grid of ceil(N / 256) x the class's segment bound workgroups (tiles
// placed by grouped_tile), 512 threads, dynamic LDS wide_lds_bytes<BM>().
template <int DT, int BITS, int GS, int BM>
__global__ __launch_bounds__(kWideNT) void qmm_grouped_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ w,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    const int32_t* __restrict__ lhs, uint16_t* __restrict__ out, const int32_t* __restrict__ ws,
    int P, int B, int Mi, int N, int K, int E, int cls) {
  extern __shared__ __align__(16) uint16_t wide_smem[];
  __shared__ uint32_t s_xoff[BM];
  __shared__ int s_orow[BM];
  const int32_t* hdr = ws + gather_ws_header(P);
  const int s0 = hdr[2 - cls];
  int seg, col;
  if (!grouped_tile(blockIdx.x, hdr[3 - cls] - s0, (N + kWideBN - 1) / kWideBN, seg, col)) return;
  grouped_body<DT, BITS, GS, BM>(x, w, scales, biases, lhs, out, ws, P, B, Mi, N, K, E, seg + s0,
                                 col * kWideBN, wide_smem, s_xoff, s_orow);
}

// Expert-grouped tiles of all three size classes in one launch, so the tall
// tiles of hot experts and the short ones of thin experts share the GPU
// (three launches in a row left most CUs idle during the first two: config 4
// gate/up zipf 446 us against 416 with 64-row tiles for all).  Workgroups
// [0, 8 q2) run class 2 (256-row tiles), the next 8 q1 class 1 (128 rows),
// the rest class 0 (64 rows); each class's tiles are placed by grouped_tile
// (q = its tiles / 8, rounded up).  Grid: the sum of 8 q over the classes'
// segment bounds; dynamic LDS wide_lds_bytes<256>() (one workgroup per CU,
// as for every height).
template <int DT, int BITS, int GS>
__global__ __launch_bounds__(kWideNT) void qmm_grouped_classes_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ w,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    const int32_t* __restrict__ lhs, uint16_t* __restrict__ out, const int32_t* __restrict__ ws,
    int P, int B, int Mi, int N, int K, int E) {
  extern __shared__ __align__(16) uint16_t wide_smem[];
  __shared__ uint32_t s_xoff[256];
  __shared__ int s_orow[256];
  const int32_t* hdr = ws + gather_ws_header(P);
  const int ncol = (N + kWideBN - 1) / kWideBN;
  int i = blockIdx.x, cls = 2;
  for (; cls > 0; --cls) {
    const int q = ((hdr[3 - cls] - hdr[2 - cls]) * ncol + 7) / 8;
    if (i < 8 * q) break;
    i -= 8 * q;
  }
  const int s0 = hdr[2 - cls];
  int seg, col;
  if (!grouped_tile(i, hdr[3 - cls] - s0, ncol, seg, col)) return;
  seg += s0;
  if (cls == 2)
    grouped_body<DT, BITS, GS, 256>(x, w, scales, biases, lhs, out, ws, P, B, Mi, N, K, E, seg,
                                    col * kWideBN, wide_smem, s_xoff, s_orow);
  else if (cls == 1)
    grouped_body<DT, BITS, GS, 128>(x, w, scales, biases, lhs, out, ws, P, B, Mi, N, K, E, seg,
                                    col * kWideBN, wide_smem, s_xoff, s_orow);
  else
    grouped_body<DT, BITS, GS, 64>(x, w, scales, biases, lhs, out, ws, P, B, Mi, N, K, E, seg,
                                   col * kWideBN, wide_smem, s_xoff, s_orow);
}

template <int DT, int BITS, int GS, int BM>
inline int wide_launch_bm(const void* x, const uint32_t* w, const void* s, const void* b,
                          void* out, int64_t M, int64_t N, int64_t K, int splits, void* ws,
                          hipStream_t st) {
  static std::atomic<uint64_t> lds_set{0};
  if (hipError_t e = ensure_lds_limit(
          reinterpret_cast<const void*>(&qmm_wide_kernel<DT, BITS, GS, BM>),
          (int)wide_lds_bytes<BM>(), lds_set))
    return (int)e;
  float* part = splits > 1 ? static_cast<float*>(ws) : nullptr;
  const dim3 grid((unsigned)((N + kWideBN - 1) / kWideBN), (unsigned)((M + BM - 1) / BM),
                  (unsigned)splits);
  hipLaunchKernelGGL((qmm_wide_kernel<DT, BITS, GS, BM>), grid, dim3(kWideNT),
                     wide_lds_bytes<BM>(), st, (const uint16_t*)x, w, (const uint16_t*)s,
                     (const uint16_t*)b, (uint16_t*)out, part, (int)M, (int)N, (int)K);
  if (splits > 1) {
    const int64_t MN = M * N;
    hipLaunchKernelGGL((wide_reduce_kernel<DT>), dim3((unsigned)((MN + 1023) / 1024)), dim3(256),
                       0, st, (const float*)part, (uint16_t*)out, MN, splits);
  }
  return 0;
}

template <int DT, int BITS, int GS>
int WideLaunch<DT, BITS, GS>::run(const void* x, const uint32_t* w, const void* s, const void* b,
                                  void* out, int64_t M, int64_t N, int64_t K, void* ws,
                                  size_t ws_bytes, hipStream_t st, int* nlaunch) {
  // one tile's x rows and weight rows must fit a 31-bit buffer range
  if (K * 2 * 256 >= ((int64_t)1 << 31) || M > ((int64_t)1 << 31) / 256 * 256)
    return kStatusUnsupported;
  const int cus = device_cu_count();
  WidePlan plan = wide_plan(M, N, K, cus);
  if (plan.splits > 1 && (!ws || ws_bytes < wide_workspace_bytes(plan, M, N)))
    plan = wide_plan(M, N, K, cus, 1);
  const int splits = plan.splits;
  *nlaunch += splits > 1 ? 2 : 1;
  switch (plan.bm) {
    case 64: return wide_launch_bm<DT, BITS, GS, 64>(x, w, s, b, out, M, N, K, splits, ws, st);
    case 128: return wide_launch_bm<DT, BITS, GS, 128>(x, w, s, b, out, M, N, K, splits, ws, st);
    case 192: return wide_launch_bm<DT, BITS, GS, 192>(x, w, s, b, out, M, N, K, splits, ws, st);
    default: return wide_launch_bm<DT, BITS, GS, 256>(x, w, s, b, out, M, N, K, splits, ws, st);
  }
}

}  // namespace mq
