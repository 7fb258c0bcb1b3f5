// Wide (prefill) quantized matmul: out[M,N] = x[M,K] . deq(W[N,K])^T for M > 16.
//
// Reference behaviour: mlxturbo/kernels/qmm_wide.py:456-502 (MLX steel
// qmm_t with a 64-row tile), reached from fused._qmm_wide_dispatch
// (fused.py:3477-3499) for prefill chunks; the MLX loader dequantizes each W
// tile to T in threadgroup memory (_steel_flat.py:1324-1335).
//
// CDNA4 design (compute-bound: arithmetic intensity 1247-3483 FLOP/B at
// M = 512..8192, above the ~312 FLOP/B ridge):
//  * Block tile BM x BN = 256 x 128, BK = 64 codes, 256 threads (4 waves in a
//    2 x 2 grid, 128 x 64 outputs each = 4 x 2 tiles of v_mfma_f32_32x32x16).
//  * Per k-step the workgroup stages x[256 x 64] and the dequantized W[128 x
//    64] (T, exact MLX dequant, one group per row per step at gs = 64) in LDS,
//    rows padded to 144 bytes so the 8-lane groups of ds_read_b128 hit
//    distinct banks.  Two LDS buffers: the global loads of step k+1 are in
//    flight (registers) while step k runs its MFMAs, then are dequantized
//    into the other buffer.
//  * Each weight is dequantized once per 256 output rows, so the VALU work is
//    ~1/8 of the MFMA time; x tiles are re-read from L2 once per 128 columns.
#pragma once
#include "launch.h"

namespace mq {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kWideBM = 256, kWideBN = 128, kWideBK = 64;
constexpr int kWideLD = kWideBK + 8;  // LDS row stride in 16-bit elements (144 bytes)
constexpr size_t kWideLds = 2 * (size_t)(kWideBM + kWideBN) * kWideLD * 2;

template <int DT>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (DT == kBF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(bitcast<bf16x8>(a), bitcast<bf16x8>(b), c, 0,
                                                   0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(bitcast<f16x8>(a), bitcast<f16x8>(b), c, 0, 0,
                                                  0);
}

template <int DT, int BITS, int GS>
__global__ __launch_bounds__(256) void qmm_wide_kernel(const uint16_t* __restrict__ x,
                                                       const uint32_t* __restrict__ w,
                                                       const uint16_t* __restrict__ scales,
                                                       const uint16_t* __restrict__ biases,
                                                       uint16_t* __restrict__ out, int M, int N,
                                                       int K) {
  constexpr int BM = kWideBM, BN = kWideBN, BK = kWideBK, LD = kWideLD;
  constexpr int WCH = BK * BITS / 128;          // 16-byte weight chunks per row per step (2 or 4)
  constexpr int WPT = BN * WCH / 256;           // weight chunks per thread (1 or 2)
  constexpr int CPC = 128 / BITS;               // codes per chunk
  extern __shared__ __align__(16) uint16_t wide_smem[];
  uint16_t* As = wide_smem;                     // [2][BM*LD]
  uint16_t* Bs = wide_smem + 2 * BM * LD;       // [2][BN*LD]

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int64_t Kw = (int64_t)K * BITS / 32;
  const int G = K / GS;
  const int nk = K / BK;

  // global -> register staging of one k-step
  u32x4 ra[8];
  u32x4 rw[WPT];
  uint16_t rs[WPT], rb[WPT];
  auto gload = [&](int kt) {
    const int k0 = kt * BK;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int id = t + 256 * i;
      const int row = id >> 3, kc = id & 7;
      const int gm = min(m0 + row, M - 1);
      ra[i] = *reinterpret_cast<const u32x4*>(x + (int64_t)gm * K + k0 + 8 * kc);
    }
#pragma unroll
    for (int i = 0; i < WPT; ++i) {
      const int id = t + 256 * i;
      const int row = id / WCH, ch = id % WCH;
      const int gn = min(n0 + row, N - 1);
      const int kc = k0 + ch * CPC;
      rw[i] = *reinterpret_cast<const u32x4*>(w + (int64_t)gn * Kw + (int64_t)kc * BITS / 32);
      rs[i] = scales[(int64_t)gn * G + kc / GS];
      rb[i] = biases[(int64_t)gn * G + kc / GS];
    }
  };
  auto sstore = [&](int buf) {
    uint16_t* A = As + buf * BM * LD;
    uint16_t* B = Bs + buf * BN * LD;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int id = t + 256 * i;
      const int row = id >> 3, kc = id & 7;
      *reinterpret_cast<u32x4*>(A + row * LD + 8 * kc) = ra[i];
    }
    using T = T16<DT>;
#pragma unroll
    for (int i = 0; i < WPT; ++i) {
      const int id = t + 256 * i;
      const int row = id / WCH, ch = id % WCH;
      const float sf = T::to_f32(rs[i]);
      const GroupScale g = make_group(sf, T::to_f32(rb[i]));
      uint32_t o[CPC / 2];
      if (needs_plain(sf)) {
#pragma unroll
        for (int j = 0; j < 4; ++j) deq_word_plain<DT, BITS>(rw[i][j], g, o + j * (CPC / 8));
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) deq_word<DT, BITS>(rw[i][j], g, o + j * (CPC / 8));
      }
      u32x4* dst = reinterpret_cast<u32x4*>(B + row * LD + ch * CPC);
#pragma unroll
      for (int j = 0; j < CPC / 8; ++j) dst[j] = (u32x4){o[4 * j], o[4 * j + 1], o[4 * j + 2], o[4 * j + 3]};
    }
  };

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  gload(0);
  sstore(0);
  __syncthreads();
  const int lr = lane & 31, lk = 8 * (lane >> 5);
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload(kt + 1);
    const uint16_t* A = As + buf * BM * LD + (128 * wm + lr) * LD + lk;
    const uint16_t* B = Bs + buf * BN * LD + (64 * wn + lr) * LD + lk;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      u32x4 a[4], b[2];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const u32x4*>(A + 32 * i * LD + 16 * ks);
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = *reinterpret_cast<const u32x4*>(B + 32 * j * LD + 16 * ks);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma32<DT>(a[i], b[j], acc[i][j]);
    }
    if (kt + 1 < nk) sstore(buf ^ 1);
    __syncthreads();
  }

  // D[row][col] of a 32x32 tile: col = lane & 31, row = 8*(e/4) + 4*(lane>>5) + e%4
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = n0 + 64 * wn + 32 * j + lr;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = m0 + 128 * wm + 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        if (row < M && col < N) out[(int64_t)row * N + col] = T16<DT>::round1(acc[i][j][e]);
      }
    }
}

template <int DT, int BITS, int GS>
int WideLaunch<DT, BITS, GS>::run(const void* x, const uint32_t* w, const void* s, const void* b,
                                  void* out, int64_t M, int64_t N, int64_t K, hipStream_t st) {
  const dim3 grid((unsigned)((N + kWideBN - 1) / kWideBN), (unsigned)((M + kWideBM - 1) / kWideBM));
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&qmm_wide_kernel<DT, BITS, GS>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)kWideLds);
  if (attr != hipSuccess) return (int)attr;
  hipLaunchKernelGGL((qmm_wide_kernel<DT, BITS, GS>), grid, dim3(256), kWideLds, st,
                     (const uint16_t*)x, w, (const uint16_t*)s, (const uint16_t*)b,
                     (uint16_t*)out, (int)M, (int)N, (int)K);
  return 0;
}

}  // namespace mq
