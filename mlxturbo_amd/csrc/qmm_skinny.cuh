// Skinny quantized matmul, M <= 16 rows: out[M,N] = x[M,K] . deq(W[N,K])^T.
//
// Covers the reference's M=1 decode path (mx.quantized_matmul -> qmv_fast,
// dispatch.py:317-327) and the M=2..16 verify window (qmv_small_m.py:289-335,
// fast_qmm.py:334-374, qmv_wide_nocap.py:240-288) with one CDNA4 design:
//
//  * The work is HBM-bound (K=5120 N=17408 streams 50 MB), so the layout is
//    chosen for the weight stream: a workgroup owns 16 consecutive rows of W
//    (one contiguous 16*K*bits/8-byte block); its waves split K into
//    k-blocks (256 codes per row at 4 bits) taken round-robin.
//  * Each lane loads two 16-byte chunks of one row per k-block (lane&15 is
//    the row, lane>>4 picks the chunk), dequantizes in registers with the
//    exact fma_mix trick (mq_common.h) and feeds the packed T pairs straight
//    into v_mfma_f32_16x16x32 as the B operand (32 k x 16 n).  The A operand
//    is x (16 m x 32 k, rows >= M zero), loaded with the same lane->k
//    mapping, so the permuted k order inside each MFMA is the same for A and
//    B.  The multiply-adds leave the VALU for every M <= 16; the VALU only
//    unpacks and rounds (17 ops per 8 codes at 4 bits).
//  * Partial 16x16 tiles of the waves are summed in LDS in a fixed order
//    (deterministic) and rounded once to T.
#pragma once
#include "mq_common.h"

namespace mq {

constexpr int kSkinnyMaxWaves = 4;

template <int BITS>
struct SkinnyGeom {
  static constexpr int CPC = 128 / BITS;          // codes per 16-byte chunk
  static constexpr int KBLK = 8 * CPC;            // codes per row per k-block
  static constexpr int WPM = (BITS == 4) ? 1 : 2; // words per MFMA (8 codes)
  static constexpr int MPC = 4 / WPM;             // MFMAs per chunk
};

// One wave's share of a 16(n) x 16(m) output tile: k-blocks kb_begin,
// kb_begin + kb_step, ...  xrow is this lane's A row (used when mval).
template <int DT, int BITS, int GS>
__device__ __forceinline__ f32x4 skinny_accumulate(const uint16_t* __restrict__ xrow, bool mval,
                                                   const uint32_t* __restrict__ wrow,
                                                   const uint16_t* __restrict__ srow,
                                                   const uint16_t* __restrict__ brow, bool nval,
                                                   int K, int kb_begin, int kb_step, int c) {
  using T = T16<DT>;
  using Gm = SkinnyGeom<BITS>;
  constexpr int CPC = Gm::CPC, KBLK = Gm::KBLK, MPC = Gm::MPC;
  static_assert(GS % CPC == 0, "a chunk must sit inside one group");
  const int nkb = (K + KBLK - 1) / KBLK;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int kb = kb_begin; kb < nkb; kb += kb_step) {
    const int kbase = kb * KBLK;
    u32x4 wv[2];
    uint16_t sr[2], br[2];
    u32x4 xv[2][MPC];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int k0 = kbase + (h * 4 + c) * CPC;
      const bool kval = k0 < K;
      if (nval && kval) {
        wv[h] = *reinterpret_cast<const u32x4*>(wrow + (int64_t)k0 * BITS / 32);
        sr[h] = srow[k0 / GS];
        br[h] = brow[k0 / GS];
      } else {
        wv[h] = (u32x4){0u, 0u, 0u, 0u};
        sr[h] = 0;
        br[h] = 0;
      }
#pragma unroll
      for (int j = 0; j < MPC; ++j) {
        if (mval && kval)
          xv[h][j] = *reinterpret_cast<const u32x4*>(xrow + k0 + 8 * j);
        else
          xv[h][j] = (u32x4){0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float sf = T::to_f32(sr[h]);
      const GroupScale g = make_group(sf, T::to_f32(br[h]));
      const bool plain = __builtin_amdgcn_ballot_w64(needs_plain(sf)) != 0;
#pragma unroll
      for (int j = 0; j < MPC; ++j) {
        uint32_t bo[4];
        if (plain) {
          if constexpr (BITS == 4) {
            deq_word_plain<DT, 4>(wv[h][j], g, bo);
          } else {
            deq_word_plain<DT, 8>(wv[h][2 * j], g, bo);
            deq_word_plain<DT, 8>(wv[h][2 * j + 1], g, bo + 2);
          }
        } else {
          if constexpr (BITS == 4) {
            deq4_word<DT>(wv[h][j], g, bo);
          } else {
            deq8_word<DT>(wv[h][2 * j], g, bo);
            deq8_word<DT>(wv[h][2 * j + 1], g, bo + 2);
          }
        }
        acc = T::mfma(xv[h][j], (u32x4){bo[0], bo[1], bo[2], bo[3]}, acc);
      }
    }
  }
  return acc;
}

// Sum the waves' partial tiles in a fixed order and hand element (mm, nn)
// (mm = A row, nn = column within the 16-column tile) to store(mm, nn, v).
// Lane l of a wave holds D[4*(l>>4)+v][l&15] for v = 0..3.
template <typename Store>
__device__ __forceinline__ void skinny_reduce(f32x4 acc, int nwaves, Store store) {
  __shared__ f32x4 red[kSkinnyMaxWaves][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  red[wave][lane] = acc;
  __syncthreads();
  for (int t = threadIdx.x; t < 256; t += blockDim.x) {
    const int mm = t >> 4;
    const int nn = t & 15;
    const int src = ((mm >> 2) << 4) | nn;
    const int v = mm & 3;
    float sum = red[0][src][v];
    for (int q = 1; q < nwaves; ++q) sum += red[q][src][v];
    store(mm, nn, sum);
  }
}

template <int DT, int BITS, int GS>
__global__ __launch_bounds__(256) void qmm_skinny_kernel(const uint16_t* __restrict__ x,
                                                         const uint32_t* __restrict__ w,
                                                         const uint16_t* __restrict__ scales,
                                                         const uint16_t* __restrict__ biases,
                                                         uint16_t* __restrict__ out, int M, int N,
                                                         int K, int64_t ldx, int64_t ldo) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  const int r = lane & 15;
  const int c = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int n = n0 + r;
  const bool nval = n < N;
  const int64_t Kw = (int64_t)K * BITS / 32;
  const int G = K / GS;
  const int64_t nrow = nval ? n : 0;
  const bool mval = r < M;
  const f32x4 acc = skinny_accumulate<DT, BITS, GS>(
      x + (int64_t)(mval ? r : 0) * ldx, mval, w + nrow * Kw, scales + nrow * G,
      biases + nrow * G, nval, K, wave, nwaves, c);
  skinny_reduce(acc, nwaves, [&](int mm, int nn, float v) {
    if (mm < M && n0 + nn < N) out[(int64_t)mm * ldo + n0 + nn] = T16<DT>::round1(v);
  });
}

}  // namespace mq
