// SwiGLU between a MoE layer's gate/up and down gathers at prefill widths:
// h = T(T(silu(g)) * u), silu(g) = g / (1 + exp(-g)) evaluated in float, as
// mlx-lm's SwitchGLU applies nn.silu to the gate projection and multiplies by
// the up projection (the reference's prefill path calls that activation on
// its grouped GEMM outputs, mlxturbo/fused.py:3302), each of the two steps
// rounded to T.
//
// The value itself is mq_common.h's swiglu_t.
//
// HBM-bound: 6 bytes per value (two reads, one write).  One pass, eight
// values per thread through 16-byte loads and stores where the three arrays
// are 16-byte aligned, a scalar tail for the last n % 8.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "launch.h"

namespace mq {

namespace {

constexpr int kSwigluThreads = 256;

template <int DT, bool VEC>
__global__ __launch_bounds__(kSwigluThreads) void swiglu_kernel(const uint16_t* __restrict__ g,
                                                                const uint16_t* __restrict__ u,
                                                                uint16_t* __restrict__ h,
                                                                int64_t n) {
  const int64_t i0 = ((int64_t)blockIdx.x * kSwigluThreads + threadIdx.x) * 8;
  if (i0 >= n) return;
  if (VEC && i0 + 8 <= n) {
    const u32x4 gv = *reinterpret_cast<const u32x4*>(g + i0);
    const u32x4 uv = *reinterpret_cast<const u32x4*>(u + i0);
    u32x4 hv;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t lo = swiglu_t<DT>((uint16_t)(gv[e] & 0xffffu), (uint16_t)(uv[e] & 0xffffu));
      const uint32_t hi = swiglu_t<DT>((uint16_t)(gv[e] >> 16), (uint16_t)(uv[e] >> 16));
      hv[e] = lo | (hi << 16);
    }
    *reinterpret_cast<u32x4*>(h + i0) = hv;
    return;
  }
  const int64_t i1 = i0 + 8 < n ? i0 + 8 : n;
  for (int64_t i = i0; i < i1; ++i) h[i] = swiglu_t<DT>(g[i], u[i]);
}

}  // namespace

int launch_swiglu(const void* g, const void* u, void* out, int64_t n, int dtype, hipStream_t st) {
  const int64_t blocks = (n + 8 * kSwigluThreads - 1) / (8 * kSwigluThreads);
  if (blocks > INT32_MAX) return kStatusUnsupported;
  const bool vec = ((reinterpret_cast<uintptr_t>(g) | reinterpret_cast<uintptr_t>(u) |
                     reinterpret_cast<uintptr_t>(out)) & 15u) == 0;
#define MQ_SWIGLU(DT, V)                                                                        \
  hipLaunchKernelGGL((swiglu_kernel<DT, V>), dim3((unsigned)blocks), dim3(kSwigluThreads), 0,  \
                     st, (const uint16_t*)g, (const uint16_t*)u, (uint16_t*)out, n)
  if (dtype == kBF16) {
    if (vec) MQ_SWIGLU(kBF16, true);
    else MQ_SWIGLU(kBF16, false);
  } else if (dtype == kF16) {
    if (vec) MQ_SWIGLU(kF16, true);
    else MQ_SWIGLU(kF16, false);
  } else {
    return kStatusUnsupported;
  }
#undef MQ_SWIGLU
  return 0;
}

}  // namespace mq
