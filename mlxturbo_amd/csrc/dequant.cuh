// Bit-exact MLX affine dequantization: out[n,k] = T(float(s)*q + float(b)).
// Reference: mx.dequantize / _steel_flat.py:1169-1256 (MLX's dequantize()).
//
// Memory-bound elementwise kernel: one thread turns one 16-byte chunk of
// packed codes (32 codes at 4 bits, 16 at 8 bits; always inside one group
// because group_size >= 32) into 2-4 16-byte stores.
#pragma once
#include "launch.h"

namespace mq {

template <int DT, int BITS, int GS>
__global__ __launch_bounds__(256) void dequantize16_kernel(const uint32_t* __restrict__ w,
                                                           const uint16_t* __restrict__ s,
                                                           const uint16_t* __restrict__ b,
                                                           uint16_t* __restrict__ out, int64_t N,
                                                           int64_t K) {
  constexpr int CPC = 128 / BITS;        // codes per 16-byte chunk
  constexpr int OW = CPC / 2;            // output dwords per chunk (two T per dword)
  const int64_t Kw = K * BITS / 32;
  const int64_t cpr = Kw / 4;            // chunks per row
  const int64_t total = N * cpr;
  const int64_t G = K / GS;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = i / cpr;
    const int64_t ci = i - n * cpr;
    const int64_t k0 = ci * CPC;
    const u32x4 wv = *reinterpret_cast<const u32x4*>(w + n * Kw + ci * 4);
    const float sf = T16<DT>::to_f32(s[n * G + k0 / GS]);
    const float bf = T16<DT>::to_f32(b[n * G + k0 / GS]);
    const GroupScale g = make_group(sf, bf);
    uint32_t o[OW];
    constexpr int WO = OW / 4;  // output dwords per input word
    if (needs_plain(sf)) {
#pragma unroll
      for (int j = 0; j < 4; ++j) deq_word_plain<DT, BITS>(wv[j], g, o + j * WO);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) deq_word<DT, BITS>(wv[j], g, o + j * WO);
    }
    u32x4* dst = reinterpret_cast<u32x4*>(out + n * K + k0);
#pragma unroll
    for (int j = 0; j < OW / 4; ++j) dst[j] = (u32x4){o[4 * j], o[4 * j + 1], o[4 * j + 2], o[4 * j + 3]};
  }
}

// float32 scales/biases/output: s*q and +b rounded separately, as MLX's
// float arithmetic does (no contraction into an fma).
template <int BITS, int GS>
__global__ __launch_bounds__(256) void dequantize32_kernel(const uint32_t* __restrict__ w,
                                                           const float* __restrict__ s,
                                                           const float* __restrict__ b,
                                                           float* __restrict__ out, int64_t N,
                                                           int64_t K) {
#pragma clang fp contract(off)
  constexpr int PER = 32 / BITS;
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  const int64_t Kw = K * BITS / 32;
  const int64_t total = N * Kw;
  const int64_t G = K / GS;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = i / Kw;
    const int64_t wi = i - n * Kw;
    const int64_t k0 = wi * PER;
    const uint32_t word = w[i];
    const float sf = s[n * G + k0 / GS];
    const float bf = b[n * G + k0 / GS];
#pragma unroll
    for (int j = 0; j < PER; ++j)
      out[n * K + k0 + j] = sf * (float)((word >> (BITS * j)) & MASK) + bf;
  }
}

inline int dequant_grid(int64_t work, int per_block) {
  int64_t g = (work + per_block - 1) / per_block;
  if (g > 65536) g = 65536;
  if (g < 1) g = 1;
  return (int)g;
}

template <int DT, int BITS, int GS>
int DequantLaunch<DT, BITS, GS>::run(const uint32_t* w, const void* s, const void* b, void* out,
                                     int64_t N, int64_t K, hipStream_t st) {
  const int64_t chunks = N * (K * BITS / 32) / 4;
  hipLaunchKernelGGL((dequantize16_kernel<DT, BITS, GS>), dim3(dequant_grid(chunks, 256)),
                     dim3(256), 0, st, w, (const uint16_t*)s, (const uint16_t*)b,
                     (uint16_t*)out, N, K);
  return 0;
}

}  // namespace mq
