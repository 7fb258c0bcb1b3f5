// Bit-exact MLX affine dequantization: out[n,k] = T(float(s)*q + float(b)).
// Reference: mx.dequantize / _steel_flat.py:1169-1256 (MLX's dequantize()).
//
// Memory-bound elementwise kernel: one packed word per lane and iteration
// (its codes always lie inside one group, group_size >= 32), so a wave's
// loads read 256 contiguous bytes and its stores write contiguous output.
// K=5120 N=17408 4-bit (228 MB moved): 58.7 -> 40.1 us against one 16-byte
// chunk of codes per lane, whose four 16-byte stores per lane each touched 64
// separate 64-byte pieces; non-temporal stores on that layout took 136 us.
#pragma once
#include "launch.h"

namespace mq {

template <int DT, int BITS, int GS>
__global__ __launch_bounds__(256) void dequantize16_kernel(const uint32_t* __restrict__ w,
                                                           const uint16_t* __restrict__ s,
                                                           const uint16_t* __restrict__ b,
                                                           uint16_t* __restrict__ out, int64_t N,
                                                           int64_t K) {
  constexpr int PER = 32 / BITS;         // codes per word
  const int64_t Kw = K * BITS / 32;      // words per row
  const int64_t total = N * Kw;
  const int64_t G = K / GS;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = i / Kw;
    const int64_t k0 = (i - n * Kw) * PER;
    const uint32_t wv = w[i];
    const float sf = T16<DT>::to_f32(s[n * G + k0 / GS]);
    const float bf = T16<DT>::to_f32(b[n * G + k0 / GS]);
    const GroupScale g = make_group(sf, bf);
    uint32_t o[PER / 2];
    if (needs_plain(sf)) deq_word_plain<DT, BITS>(wv, g, o);
    else deq_word<DT, BITS>(wv, g, o);
    if constexpr (BITS == 4)
      *reinterpret_cast<u32x4*>(out + n * K + k0) = (u32x4){o[0], o[1], o[2], o[3]};
    else
      *reinterpret_cast<u32x2*>(out + n * K + k0) = (u32x2){o[0], o[1]};
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
    float v[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) v[j] = sf * (float)((word >> (BITS * j)) & MASK) + bf;
    f32x4* dst = reinterpret_cast<f32x4*>(out + n * K + k0);
#pragma unroll
    for (int j = 0; j < PER / 4; ++j) dst[j] = (f32x4){v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]};
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
  const int64_t words = N * (K * BITS / 32);
  hipLaunchKernelGGL((dequantize16_kernel<DT, BITS, GS>), dim3(dequant_grid(words, 256 * 4)),
                     dim3(256), 0, st, w, (const uint16_t*)s, (const uint16_t*)b,
                     (uint16_t*)out, N, K);
  return 0;
}

}  // namespace mq
