// Shared device-side definitions for the mlxturbo_amd HIP kernels (gfx950).
//
// Weight format (MLX affine quantization):
//   w       uint32 [N, K*bits/32], code j of word i is element i*(32/bits)+j,
//           stored at bit bits*j (low bits first)
//   scales  T [N, K/group_size], biases T [N, K/group_size]
//   deq     T(float(s)*q + float(b)), rounded to nearest even
//
// Exact dequantization trick used by every kernel here:
//   A code masked in place inside the mantissa bits (0..9) of a 16-bit lane
//   of a register, e.g. (w & 0x00F000F0) keeps code 1 at bits 4..7 of the
//   low half, is the IEEE half subnormal (q << 4) * 2^-24 = q * 2^-20.  v_fma_mix_f32 converts the
//   half to float exactly (fp16 denormals are preserved in the kernel's mode
//   register) and computes fma(q*2^-20, s*2^20, b) with one rounding, which
//   equals float(s*q + b) because s*2^20 is exact whenever |s| < 2^100.
//   That replaces shift + convert + fma (3 VALU ops per code) by an AND
//   shared by two codes plus one fma_mix.  Scales with |s| >= 2^100 take a
//   plain float path selected per wave (never taken for real checkpoints).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mq {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

enum DTypeCode { kBF16 = 0, kF16 = 1, kF32 = 2 };

// Status returned by internal launchers for a configuration with no kernel.
constexpr int kStatusUnsupported = -2;

template <typename To, typename From>
__device__ __forceinline__ To bitcast(const From& v) {
  static_assert(sizeof(To) == sizeof(From), "bitcast size");
  return __builtin_bit_cast(To, v);
}

// Buffer resource for a raw (unstructured) byte range.  Word 3 is the gfx9
// default for 32-bit data; out-of-range loads return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// 16-bit storage types: bf16 (kBF16) and IEEE half (kF16).
template <int DT> struct T16;

template <> struct T16<kBF16> {
  static __device__ __forceinline__ float to_f32(uint16_t h) {
    return __uint_as_float((uint32_t)h << 16);
  }
  // two floats -> packed pair, round to nearest even (v_cvt_pk_bf16_f32)
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    return bitcast<uint32_t>(__builtin_convertvector((f32x2){a, b}, bf16x2));
  }
  static __device__ __forceinline__ uint16_t round1(float a) {
    return (uint16_t)(pack2(a, 0.0f) & 0xffffu);
  }
  static __device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(bitcast<bf16x8>(a), bitcast<bf16x8>(b), c,
                                                   0, 0, 0);
  }
};

template <> struct T16<kF16> {
  static __device__ __forceinline__ float to_f32(uint16_t h) {
    return (float)bitcast<_Float16>(h);
  }
  // v_cvt_pk_f16_f32: round to nearest even
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    return bitcast<uint32_t>(__builtin_convertvector((f32x2){a, b}, f16x2));
  }
  static __device__ __forceinline__ uint16_t round1(float a) {
    return (uint16_t)(pack2(a, 0.0f) & 0xffffu);
  }
  static __device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(bitcast<f16x8>(a), bitcast<f16x8>(b), c, 0,
                                                  0, 0);
  }
};

// SwiGLU of one gate / up pair of T values: T(T(silu(g)) * u), silu(g) =
// g / (1 + exp(-g)) in float (mlx-lm's SwitchGLU: nn.silu on the gate
// projection times the up projection, each step rounded to T).  The SwiGLU
// pass (swiglu.hip) and the fused prefill gate/up gather (grouped.cuh) both
// evaluate it here, so they give the same bits.
template <int DT>
__device__ __forceinline__ uint16_t swiglu_t(uint16_t g, uint16_t u) {
  const float gf = T16<DT>::to_f32(g);
  const float a = T16<DT>::to_f32(T16<DT>::round1(gf / (1.0f + expf(-gf))));
  return T16<DT>::round1(a * T16<DT>::to_f32(u));
}

__device__ __forceinline__ float half_lo(uint32_t v) { return (float)bitcast<f16x2>(v).x; }
__device__ __forceinline__ float half_hi(uint32_t v) { return (float)bitcast<f16x2>(v).y; }

// The x batch that gather pair p reads: lhs[p], or with no table p / (P / B)
// (B divides P: each x batch serves P / B consecutive pairs, as when tokens
// (T, 1) broadcast against their top-k expert indices (T, k); B == P is the
// identity).
__device__ __forceinline__ int x_batch(const int32_t* lhs, int p, int P, int B) {
  return lhs ? lhs[p] : (B == P ? p : p / (P / B));
}

// Per-group dequant parameters for the fast path.
struct GroupScale {
  float s24, s20;  // s * 2^24, s * 2^20
  float s, b;
};

__device__ __forceinline__ GroupScale make_group(float s, float b) {
  GroupScale g;
  g.s24 = s * 16777216.0f;
  g.s20 = s * 1048576.0f;
  g.s = s;
  g.b = b;
  return g;
}

// True when the fast (scaled) path would overflow: |s| >= 2^100 or inf.
__device__ __forceinline__ bool needs_plain(float s) { return __builtin_fabsf(s) >= 0x1p100f; }

// 4-bit: one word (codes k0..k7) -> four packed T pairs (k0,k1) (k2,k3) (k4,k5) (k6,k7).
// Only bits 0..9 of a half are mantissa, so a code may sit at bits 0..3 or
// 4..7 of each 16-bit lane; the upper byte of each lane is shifted down first.
template <int DT>
__device__ __forceinline__ void deq4_word(uint32_t w, const GroupScale& g, uint32_t o[4]) {
  const uint32_t t = w >> 8;
  const uint32_t h0 = w & 0x000F000Fu;          // k0, k4  (x 2^-24)
  const uint32_t h1 = w & 0x00F000F0u;          // k1, k5  (x 2^-20)
  const uint32_t h2 = t & 0x000F000Fu;          // k2, k6  (x 2^-24)
  const uint32_t h3 = t & 0x00F000F0u;          // k3, k7  (x 2^-20)
  const float v0 = __builtin_fmaf(half_lo(h0), g.s24, g.b);
  const float v4 = __builtin_fmaf(half_hi(h0), g.s24, g.b);
  const float v1 = __builtin_fmaf(half_lo(h1), g.s20, g.b);
  const float v5 = __builtin_fmaf(half_hi(h1), g.s20, g.b);
  const float v2 = __builtin_fmaf(half_lo(h2), g.s24, g.b);
  const float v6 = __builtin_fmaf(half_hi(h2), g.s24, g.b);
  const float v3 = __builtin_fmaf(half_lo(h3), g.s20, g.b);
  const float v7 = __builtin_fmaf(half_hi(h3), g.s20, g.b);
  o[0] = T16<DT>::pack2(v0, v1);
  o[1] = T16<DT>::pack2(v2, v3);
  o[2] = T16<DT>::pack2(v4, v5);
  o[3] = T16<DT>::pack2(v6, v7);
}

// 8-bit: one word (codes k0..k3) -> two packed T pairs (k0,k1) (k2,k3).
template <int DT>
__device__ __forceinline__ void deq8_word(uint32_t w, const GroupScale& g, uint32_t o[2]) {
  const uint32_t h0 = w & 0x00FF00FFu;          // k0, k2  (x 2^-24)
  const uint32_t h1 = (w >> 8) & 0x00FF00FFu;   // k1, k3  (x 2^-24)
  const float v0 = __builtin_fmaf(half_lo(h0), g.s24, g.b);
  const float v2 = __builtin_fmaf(half_hi(h0), g.s24, g.b);
  const float v1 = __builtin_fmaf(half_lo(h1), g.s24, g.b);
  const float v3 = __builtin_fmaf(half_hi(h1), g.s24, g.b);
  o[0] = T16<DT>::pack2(v0, v1);
  o[1] = T16<DT>::pack2(v2, v3);
}

// Plain float route: q -> float, fma(q, s, b).  Exact for any s (same value
// as MLX's float arithmetic including inf/NaN propagation).
template <int DT, int BITS>
__device__ __forceinline__ void deq_word_plain(uint32_t w, const GroupScale& g,
                                               uint32_t o[BITS == 4 ? 4 : 2]) {
  constexpr int PER = 32 / BITS;
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  float v[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) v[j] = __builtin_fmaf((float)((w >> (BITS * j)) & MASK), g.s, g.b);
#pragma unroll
  for (int j = 0; j < PER / 2; ++j) o[j] = T16<DT>::pack2(v[2 * j], v[2 * j + 1]);
}

template <int DT, int BITS>
__device__ __forceinline__ void deq_word(uint32_t w, const GroupScale& g,
                                         uint32_t o[BITS == 4 ? 4 : 2]) {
  if constexpr (BITS == 4) {
    deq4_word<DT>(w, g, o);
  } else {
    deq8_word<DT>(w, g, o);
  }
}

}  // namespace mq
