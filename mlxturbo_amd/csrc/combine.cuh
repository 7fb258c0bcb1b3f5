// MoE combine epilogue: out[t, n] = T( sum_k w[t*top_k + k] * y[inv[t*top_k + k], n] ).
//
// Reference: mlxturbo/kernels/moe_combine.py:160-195 (one pass over the down
// projection's expert-ordered output: unsort, router weight and top-k sum,
// fp32 accumulation in k order, one rounding).  inv may be NULL: then the
// rows of y are already in (token, k) order (decode widths, no sort).
//
// HBM-bound: bytes per call rows*top_k*N*2 (y) + rows*N*2 (out) + rows*top_k*8
// (inv, w).  One workgroup per token; each thread owns 8 columns (one 16-byte
// load per expert row, one 16-byte store), so every read of y is a
// contiguous 16-byte piece of a row and a wave reads 1 KiB per instruction.
// The token's row numbers and weights are read once into LDS; a row number
// outside [0, y_rows) is dropped there (its term is skipped), so a bad index
// never reads outside y.
#pragma once
#include "mq_common.h"

namespace mq {

constexpr int kCombineMaxTopK = 64;
constexpr int kCombineBatch = 8;

// SH: the shared expert merged in as the reference's decode combine does
// (kernels/moe_route_decode.py:392-398): out = T(float(T(sum)) +
// float(T(sgate[t] * shared[t, n]))), sgate the already-sigmoided gate.
template <int DT, bool SH = false>
__global__ __launch_bounds__(256) void moe_combine_kernel(const uint16_t* __restrict__ y,
                                                          const int32_t* __restrict__ inv,
                                                          const float* __restrict__ w,
                                                          uint16_t* __restrict__ out, int top_k,
                                                          int N, int y_rows,
                                                          const uint16_t* __restrict__ sgate = nullptr,
                                                          const uint16_t* __restrict__ shared = nullptr) {
  using T = T16<DT>;
  __shared__ int s_row[kCombineMaxTopK];
  __shared__ float s_w[kCombineMaxTopK];
  const int t = blockIdx.y;
  const int64_t base = (int64_t)t * top_k;
  for (int i = threadIdx.x; i < top_k; i += blockDim.x) {
    const int r = inv ? inv[base + i] : (int)(base + i);
    s_row[i] = (r >= 0 && r < y_rows) ? r : -1;
    s_w[i] = w[base + i];
  }
  __syncthreads();
  const int n = (blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (n >= N) return;
  float acc[8];
#pragma unroll
  for (int v = 0; v < 8; ++v) acc[v] = 0.f;
  // kCombineBatch rows in flight at once (a decode token's whole top-k): all
  // loads of a batch are issued before the first is used, then the terms
  // are added in k order
  for (int k0 = 0; k0 < top_k; k0 += kCombineBatch) {
    u32x4 p[kCombineBatch];
#pragma unroll
    for (int j = 0; j < kCombineBatch; ++j) {
      const int r = k0 + j < top_k ? s_row[k0 + j] : -1;
      p[j] = r >= 0 ? *reinterpret_cast<const u32x4*>(y + (int64_t)r * N + n)
                    : (u32x4){0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int j = 0; j < kCombineBatch; ++j) {
      if (k0 + j >= top_k || s_row[k0 + j] < 0) continue;
      const float wk = s_w[k0 + j];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        acc[2 * v] = __builtin_fmaf(wk, T::to_f32((uint16_t)p[j][v]), acc[2 * v]);
        acc[2 * v + 1] = __builtin_fmaf(wk, T::to_f32((uint16_t)(p[j][v] >> 16)),
                                        acc[2 * v + 1]);
      }
    }
  }
  u32x4 o;
#pragma unroll
  for (int v = 0; v < 4; ++v) o[v] = T::pack2(acc[2 * v], acc[2 * v + 1]);
  if constexpr (SH) {
    // no contraction of the product into the sum (each is rounded to T)
#pragma clang fp contract(off)
    const float sg = T::to_f32(sgate[t]);
    const u32x4 sh = *reinterpret_cast<const u32x4*>(shared + (int64_t)t * N + n);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const uint32_t m = T::pack2(sg * T::to_f32((uint16_t)sh[v]), sg * T::to_f32((uint16_t)(sh[v] >> 16)));
      o[v] = T::pack2(T::to_f32((uint16_t)o[v]) + T::to_f32((uint16_t)m),
                      T::to_f32((uint16_t)(o[v] >> 16)) + T::to_f32((uint16_t)(m >> 16)));
    }
  }
  *reinterpret_cast<u32x4*>(out + (int64_t)t * N + n) = o;
}

// sgate / shared: both null, or the shared expert's gate (T [rows]) and
// output (T [rows, N]) to merge in.
inline int launch_moe_combine(const void* y, int64_t y_rows, const int32_t* inv, const float* w,
                              void* out, int64_t rows, int64_t top_k, int64_t N, int dtype,
                              hipStream_t st, const void* sgate = nullptr,
                              const void* shared = nullptr) {
  const int64_t cols = N / 8;
  const int tb = cols >= 256 ? 256 : cols >= 128 ? 128 : 64;
  const dim3 grid((unsigned)((cols + tb - 1) / tb), (unsigned)rows);
  const auto* sg = static_cast<const uint16_t*>(sgate);
  const auto* sh = static_cast<const uint16_t*>(shared);
#define MQ_COMBINE(DT, SH)                                                                        \
  hipLaunchKernelGGL((moe_combine_kernel<DT, SH>), grid, dim3(tb), 0, st, (const uint16_t*)y, inv, \
                     w, (uint16_t*)out, (int)top_k, (int)N, (int)y_rows, sg, sh)
  if (dtype == kBF16) {
    if (sh) MQ_COMBINE(kBF16, true);
    else MQ_COMBINE(kBF16, false);
  } else if (dtype == kF16) {
    if (sh) MQ_COMBINE(kF16, true);
    else MQ_COMBINE(kF16, false);
  } else {
    return kStatusUnsupported;
  }
#undef MQ_COMBINE
  return 0;
}

}  // namespace mq
