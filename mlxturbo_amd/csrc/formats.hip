// MLX affine format definers: quantize (float -> packed codes, scales,
// biases) and dequantize for the widths without a fast kernel (2, 3, 5, 6
// bits, any dtype; 4 and 8 bits into float32 go through dequant.cuh).
//
// Format: a row of K codes is a little-endian bitstream, code i at bits
// [bits*i, bits*i + bits) (MLX's pack factor / bytes per pack:
// kernels/_steel_flat.py:1158-1167; per-width decode 1184-1254), stored as
// uint32 words; scales and biases [N, K/group_size] in the dtype of the
// weights.  Every 8 consecutive codes fill exactly `bits` bytes, so one
// thread owns one octet of codes: 8 input values, `bits` output bytes.
//
// Quantize (mx.quantize, mode "affine", as called at mlxturbo/rebit.py:119
// and kernels/moe_verify_gather.py:887), per group in float32:
//   scale0 = max((max - min) / (2^bits - 1), 1e-7), negated unless
//   |min| > |max|; edge = min or max accordingly; q0 = rint(edge / scale0);
//   scale = q0 != 0 ? edge / q0 : scale0; bias = q0 == 0 ? 0 : edge;
//   code = clamp(rint((w - bias) / scale), 0, 2^bits - 1), NaN -> 0.
// Every operation is one correctly rounded IEEE float32 operation (the
// division is hipcc's correctly rounded sequence, rint is v_rndne), so the
// result is a deterministic function of the input bits.  NaN propagates
// through the group minimum and maximum.  The group's lanes (group_size / 8
// consecutive lanes of a wave) combine their minima and maxima with
// cross-lane exchanges.
#include "launch.h"

namespace mq {

namespace {

__device__ __forceinline__ float nan_max(float a, float b) { return (a > b || a != a) ? a : b; }
__device__ __forceinline__ float nan_min(float a, float b) { return (a < b || a != a) ? a : b; }

// float -> storage of dtype DT (16-bit types as their bits, NaN canonical)
template <int DT>
__device__ __forceinline__ void store_param(void* p, int64_t i, float v) {
  if constexpr (DT == kF32) {
    reinterpret_cast<float*>(p)[i] = v;
  } else {
    uint16_t h;
    const uint32_t sign = (__float_as_uint(v) >> 16) & 0x8000u;
    if (v != v) h = (uint16_t)(sign | (DT == kBF16 ? 0x7FC0u : 0x7E00u));
    else h = T16<DT>::round1(v);
    reinterpret_cast<uint16_t*>(p)[i] = h;
  }
}

template <int DT>
__device__ __forceinline__ void load_octet(const void* w, int64_t o, float v[8]) {
  if constexpr (DT == kF32) {
    const u32x4* p = reinterpret_cast<const u32x4*>(w) + 2 * o;
    const u32x4 a = p[0], b = p[1];
#pragma unroll
    for (int j = 0; j < 4; ++j) { v[j] = __uint_as_float(a[j]); v[4 + j] = __uint_as_float(b[j]); }
  } else {
    const u32x4 a = reinterpret_cast<const u32x4*>(w)[o];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[2 * j] = T16<DT>::to_f32((uint16_t)a[j]);
      v[2 * j + 1] = T16<DT>::to_f32((uint16_t)(a[j] >> 16));
    }
  }
}

// The `BITS` bytes of octet o (bitstream of 8 codes, lowest code lowest).
template <int BITS>
__device__ __forceinline__ void store_octet(uint8_t* wq, int64_t o, uint64_t bitsv) {
  uint8_t* p = wq + o * BITS;
  if constexpr (BITS == 2) {
    *reinterpret_cast<uint16_t*>(p) = (uint16_t)bitsv;
  } else if constexpr (BITS == 4) {
    *reinterpret_cast<uint32_t*>(p) = (uint32_t)bitsv;
  } else if constexpr (BITS == 8) {
    *reinterpret_cast<u32x2*>(p) = (u32x2){(uint32_t)bitsv, (uint32_t)(bitsv >> 32)};
  } else if constexpr (BITS == 6) {
    uint16_t* q = reinterpret_cast<uint16_t*>(p);
    q[0] = (uint16_t)bitsv; q[1] = (uint16_t)(bitsv >> 16); q[2] = (uint16_t)(bitsv >> 32);
  } else {
#pragma unroll
    for (int b = 0; b < BITS; ++b) p[b] = (uint8_t)(bitsv >> (8 * b));
  }
}

template <int BITS>
__device__ __forceinline__ uint64_t load_octet_codes(const uint8_t* wq, int64_t o) {
  const uint8_t* p = wq + o * BITS;
  if constexpr (BITS == 2) {
    return *reinterpret_cast<const uint16_t*>(p);
  } else if constexpr (BITS == 4) {
    return *reinterpret_cast<const uint32_t*>(p);
  } else if constexpr (BITS == 8) {
    const u32x2 v = *reinterpret_cast<const u32x2*>(p);
    return (uint64_t)v[0] | ((uint64_t)v[1] << 32);
  } else if constexpr (BITS == 6) {
    const uint16_t* q = reinterpret_cast<const uint16_t*>(p);
    return (uint64_t)q[0] | ((uint64_t)q[1] << 16) | ((uint64_t)q[2] << 32);
  } else {
    uint64_t v = 0;
#pragma unroll
    for (int b = 0; b < BITS; ++b) v |= (uint64_t)p[b] << (8 * b);
    return v;
  }
}

// One thread per octet of codes; group_size / 8 consecutive lanes form a
// group.  The loop bound is uniform per wave (octets is a multiple of the
// group's lane count and every wave starts on a multiple of 64), so every
// lane of a group takes part in the exchanges.
template <int DT, int BITS, int GS>
__global__ __launch_bounds__(256) void quantize_kernel(const void* __restrict__ w,
                                                       uint8_t* __restrict__ wq,
                                                       void* __restrict__ scales,
                                                       void* __restrict__ biases, int64_t octets) {
  constexpr int L = GS / 8;
  const float nb = (float)((1 << BITS) - 1);
  const int lane = threadIdx.x & 63;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t base = (int64_t)blockIdx.x * blockDim.x + (threadIdx.x & ~63); base < octets;
       base += stride) {
    const int64_t o = base + lane;
    const bool live = o < octets;
    float v[8];
    if (live) {
      load_octet<DT>(w, o, v);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = 0.f;
    }
    float hi = v[0], lo = v[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) { hi = nan_max(hi, v[j]); lo = nan_min(lo, v[j]); }
#pragma unroll
    for (int off = 1; off < L; off <<= 1) {
      hi = nan_max(hi, __shfl_xor(hi, off));
      lo = nan_min(lo, __shfl_xor(lo, off));
    }
    const float d = (hi - lo) / nb;
    float scale = (d != d) ? d : (d > 1e-7f ? d : 1e-7f);
    const bool neg_dom = __builtin_fabsf(lo) > __builtin_fabsf(hi);
    scale = neg_dom ? scale : -scale;
    const float edge = neg_dom ? lo : hi;
    const float q0 = __builtin_rintf(edge / scale);
    if (q0 != 0.0f) scale = edge / q0;
    const float bias = (q0 == 0.0f) ? 0.0f : edge;
    uint64_t packed = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float q = __builtin_rintf((v[j] - bias) / scale);
      q = (q != q) ? 0.f : __builtin_fminf(__builtin_fmaxf(q, 0.f), nb);
      packed |= (uint64_t)(uint32_t)q << (BITS * j);
    }
    if (live) {
      store_octet<BITS>(wq, o, packed);
      if ((lane & (L - 1)) == 0) {
        store_param<DT>(scales, o / L, scale);
        store_param<DT>(biases, o / L, bias);
      }
    }
  }
}

// Dequantize octets of codes of any width: T(float(s) * q + float(b)).
// For 16-bit scales s*q is exact in float32, so one fma rounds exactly as
// MLX's multiply-then-add does; float32 scales round the product and the
// sum separately, as MLX's float arithmetic does.
template <int DT, int BITS, int GS>
__global__ __launch_bounds__(256) void dequantize_bits_kernel(const uint8_t* __restrict__ wq,
                                                              const void* __restrict__ scales,
                                                              const void* __restrict__ biases,
                                                              void* __restrict__ out,
                                                              int64_t octets) {
#pragma clang fp contract(off)
  constexpr int L = GS / 8;
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < octets;
       o += (int64_t)gridDim.x * blockDim.x) {
    const uint64_t c = load_octet_codes<BITS>(wq, o);
    const int64_t g = o / L;
    if constexpr (DT == kF32) {
      const float s = reinterpret_cast<const float*>(scales)[g];
      const float b = reinterpret_cast<const float*>(biases)[g];
      float r[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float sq = s * (float)((uint32_t)(c >> (BITS * j)) & MASK);
        r[j] = sq + b;
      }
      u32x4* p = reinterpret_cast<u32x4*>(out) + 2 * o;
      p[0] = (u32x4){__float_as_uint(r[0]), __float_as_uint(r[1]), __float_as_uint(r[2]),
                     __float_as_uint(r[3])};
      p[1] = (u32x4){__float_as_uint(r[4]), __float_as_uint(r[5]), __float_as_uint(r[6]),
                     __float_as_uint(r[7])};
    } else {
      const float s = T16<DT>::to_f32(reinterpret_cast<const uint16_t*>(scales)[g]);
      const float b = T16<DT>::to_f32(reinterpret_cast<const uint16_t*>(biases)[g]);
      uint32_t r[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float q0 = (float)((uint32_t)(c >> (BITS * 2 * j)) & MASK);
        const float q1 = (float)((uint32_t)(c >> (BITS * (2 * j + 1))) & MASK);
        r[j] = T16<DT>::pack2(__builtin_fmaf(s, q0, b), __builtin_fmaf(s, q1, b));
      }
      reinterpret_cast<u32x4*>(out)[o] = (u32x4){r[0], r[1], r[2], r[3]};
    }
  }
}

inline unsigned octet_grid(int64_t octets) {
  int64_t g = (octets + 255) / 256;
  if (g > 65536) g = 65536;
  return (unsigned)(g < 1 ? 1 : g);
}

template <template <int, int, int> class F, typename... A>
int by_format(int dtype, int bits, int gs, A... args) {
#define MQ_F(DT, B)                                        \
  if (dtype == DT && bits == B) {                          \
    if (gs == 32) return F<DT, B, 32>::run(args...);       \
    if (gs == 64) return F<DT, B, 64>::run(args...);       \
    if (gs == 128) return F<DT, B, 128>::run(args...);     \
  }
#define MQ_FB(DT) MQ_F(DT, 2) MQ_F(DT, 3) MQ_F(DT, 4) MQ_F(DT, 5) MQ_F(DT, 6) MQ_F(DT, 8)
  MQ_FB(kBF16) MQ_FB(kF16) MQ_FB(kF32)
#undef MQ_FB
#undef MQ_F
  return kStatusUnsupported;
}

template <int DT, int BITS, int GS>
struct QuantizeRun {
  static int run(const void* w, uint32_t* wq, void* s, void* b, int64_t octets, hipStream_t st) {
    hipLaunchKernelGGL((quantize_kernel<DT, BITS, GS>), dim3(octet_grid(octets)), dim3(256), 0,
                       st, w, reinterpret_cast<uint8_t*>(wq), s, b, octets);
    return 0;
  }
};

template <int DT, int BITS, int GS>
struct DequantBitsRun {
  static int run(const uint32_t* wq, const void* s, const void* b, void* out, int64_t octets,
                 hipStream_t st) {
    hipLaunchKernelGGL((dequantize_bits_kernel<DT, BITS, GS>), dim3(octet_grid(octets)),
                       dim3(256), 0, st, reinterpret_cast<const uint8_t*>(wq), s, b, out, octets);
    return 0;
  }
};

}  // namespace

int launch_quantize(const void* w, uint32_t* wq, void* scales, void* biases, int64_t N,
                    int64_t K, int group_size, int bits, int dtype, hipStream_t st) {
  return by_format<QuantizeRun>(dtype, bits, group_size, w, wq, scales, biases, N * K / 8, st);
}

int launch_dequantize_bits(const uint32_t* wq, const void* scales, const void* biases, void* out,
                           int64_t N, int64_t K, int group_size, int bits, int dtype,
                           hipStream_t st) {
  return by_format<DequantBitsRun>(dtype, bits, group_size, wq, scales, biases, out, N * K / 8,
                                   st);
}

}  // namespace mq
