// MoE routing at decode / verify widths: top-k experts of a row of router
// logits with their softmax weights, and optionally the shared expert's gate.
//
// Reference behaviour: mlxturbo/kernels/moe_route_decode.py:151-327 (`route`,
// kept off by default in the reference): per row, top_k rounds of "take the
// largest logit and drop it" (equal values: the smaller expert index wins, as
// torch.topk / HF decide), then a softmax over the selected logits with the
// largest subtracted, summed in float in selection order; with x and the
// shared expert's gate weight, sigmoid(T(x . sgw)) with the dot summed in
// float and the sigmoid evaluated in T one operation at a time (MLX's form:
// y = 1 / (1 + exp(|s|)), s < 0 ? y : 1 - y, each step rounded to T).
//
// CDNA4 design: one workgroup of 256 threads per row.  All four waves share
// the shared-gate dot product (16-byte loads, all of a thread's in flight at
// once, DPP wave sums, four partials in LDS); wave 0 then runs the top-k
// alone: lane l holds experts l, l + 64, ... (NK per lane, the power of two
// covering E / 64, up to 16 for E <= 1024) as order-preserving integer keys,
// sorts them once with a bitonic network (larger key first, equal keys by
// smaller expert), and each round is two DPP wave reductions over the lanes'
// heads (the largest key, then the smallest expert holding it) after which
// the winning lane drops its head, no barrier.  (A lane-local argmax per
// round made each round one long dependent chain: 3.2 us for eight rounds.)
// Latency-bound: bytes per row 4 E + 4 H (x and the gate weight, 16-bit)
// plus 8 top_k out.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "launch.h"

namespace mq {

namespace {

constexpr int kRouteThreads = 256;
constexpr int kRouteMaxPerLane = 16;   // E <= 1024

// Largest / smallest uint32 over the 64 lanes, returned to every lane:
// inclusive row scans (row_shr 1, 2, 4, 8), the row ends broadcast into the
// following rows (row_bcast 15 into rows 1 and 3, row_bcast 31 into rows 2
// and 3), the total read from lane 63.  Lanes without a source keep their
// own value (bound_ctrl off, old = x).
#define MQ_DPP_STEP(x, OP, CTRL, ROWS)                                                        \
  x = OP(x, (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, CTRL, ROWS, 0xf, false))
template <bool MAX>
__device__ __forceinline__ uint32_t wave_reduce_u32(uint32_t x) {
// (v_max_u32 / v_min_u32 directly: a compare-and-select lets the compiler
// re-run the DPP move under a partial exec mask, where disabled source
// lanes read as out of range)
#define MQ_OP(a, b) (MAX ? __builtin_elementwise_max(a, b) : __builtin_elementwise_min(a, b))
  MQ_DPP_STEP(x, MQ_OP, 0x111, 0xf);
  MQ_DPP_STEP(x, MQ_OP, 0x112, 0xf);
  MQ_DPP_STEP(x, MQ_OP, 0x114, 0xf);
  MQ_DPP_STEP(x, MQ_OP, 0x118, 0xf);
  MQ_DPP_STEP(x, MQ_OP, 0x142, 0xa);
  MQ_DPP_STEP(x, MQ_OP, 0x143, 0xc);
#undef MQ_OP
  return (uint32_t)__builtin_amdgcn_readlane((int)x, 63);
}
#undef MQ_DPP_STEP

// Sum over the 64 lanes (lanes without a source add 0), returned to every lane.
__device__ __forceinline__ float wave_sum_f32(float x) {
#define MQ_DPP_ADD(CTRL, ROWS)                                                                 \
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x),    \
                                                             CTRL, ROWS, 0xf, false))
  MQ_DPP_ADD(0x111, 0xf);
  MQ_DPP_ADD(0x112, 0xf);
  MQ_DPP_ADD(0x114, 0xf);
  MQ_DPP_ADD(0x118, 0xf);
  MQ_DPP_ADD(0x142, 0xa);
  MQ_DPP_ADD(0x143, 0xc);
#undef MQ_DPP_ADD
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 63));
}

// float -> uint32 with the same order (larger float, larger key; -0 and +0
// equal); 0 is below every float's key and marks a taken expert.
__device__ __forceinline__ uint32_t order_key(float v) {
  const uint32_t u = v == 0.0f ? 0u : __builtin_bit_cast(uint32_t, v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float from_key(uint32_t k) {
  return __builtin_bit_cast(float, (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// sigmoid in T, one rounding per operation (MLX's Sigmoid form)
template <int DT>
__device__ __forceinline__ uint16_t sigmoid_t(uint16_t s16) {
  using T = T16<DT>;
  const float s = T::to_f32(s16);
  const float e = T::to_f32(T::round1(expf(__builtin_fabsf(s))));
  const float d = T::to_f32(T::round1(1.0f + e));
  const float y = T::to_f32(T::round1(1.0f / d));
  return s < 0.0f ? T::round1(y) : T::round1(1.0f - y);
}

// x before y in the per-lane order: larger key, then smaller slot
__device__ __forceinline__ bool key_before(uint32_t kx, int ix, uint32_t ky, int iy) {
  return kx > ky || (kx == ky && ix < iy);
}

template <int DT, bool SG, int NK>
__global__ __launch_bounds__(kRouteThreads) void moe_route_kernel(
    const float* __restrict__ logits, int32_t* __restrict__ idx, float* __restrict__ wout,
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ sgw, uint16_t* __restrict__ sgate,
    int E, int H, int top_k) {
  const int row = blockIdx.x;
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  __shared__ float s_part[kRouteThreads / 64];
  // logits first: their loads are in flight during the shared-gate dot
  uint32_t key[NK];
  int slot[NK];                                 // expert = lane + 64 slot
  const float* lr = logits + (int64_t)row * E;
  if (wv == 0) {
#pragma unroll
    for (int j = 0; j < NK; ++j) {
      const int e = lane + 64 * j;
      key[j] = e < E ? order_key(lr[e]) : 0u;
      slot[j] = j;
    }
  }
  if constexpr (SG) {
    using T = T16<DT>;
    const uint16_t* xr = x + (int64_t)row * H;
    float acc = 0.0f;
    // 16-byte pieces of x and the gate weight (eight values each), four per
    // thread in flight; a ragged or unaligned row goes element by element
    const bool vec = H % 8 == 0 && (((uintptr_t)xr | (uintptr_t)sgw) & 15u) == 0;
    if (vec) {
      const u32x4* xv = reinterpret_cast<const u32x4*>(xr);
      const u32x4* gv = reinterpret_cast<const u32x4*>(sgw);
      for (int c0 = t; c0 < H / 8; c0 += 4 * kRouteThreads) {
        u32x4 a[4], b[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int c = c0 + i * kRouteThreads;
          a[i] = c < H / 8 ? xv[c] : (u32x4){0u, 0u, 0u, 0u};
          b[i] = c < H / 8 ? gv[c] : (u32x4){0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            acc += T::to_f32((uint16_t)a[i][v]) * T::to_f32((uint16_t)b[i][v]);
            acc += T::to_f32((uint16_t)(a[i][v] >> 16)) * T::to_f32((uint16_t)(b[i][v] >> 16));
          }
      }
    } else {
      for (int h0 = t; h0 < H; h0 += 8 * kRouteThreads) {
        float a[8], b[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int h = h0 + i * kRouteThreads;
          a[i] = h < H ? T::to_f32(xr[h]) : 0.0f;
          b[i] = h < H ? T::to_f32(sgw[h]) : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) acc += a[i] * b[i];
      }
    }
    acc = wave_sum_f32(acc);
    if (lane == 0) s_part[wv] = acc;
    __syncthreads();
    if (t == 0) {
      float s = 0.0f;
#pragma unroll
      for (int i = 0; i < kRouteThreads / 64; ++i) s += s_part[i];
      sgate[row] = sigmoid_t<DT>(T::round1(s));
    }
  }
  if (wv != 0) return;
  // bitonic sort of the lane's NK keys, descending in key_before order
#pragma unroll
  for (int k = 2; k <= NK; k <<= 1)
#pragma unroll
    for (int jj = k >> 1; jj > 0; jj >>= 1)
#pragma unroll
      for (int i = 0; i < NK; ++i) {
        const int l = i ^ jj;
        if (l > i) {
          const bool swap = (i & k) == 0 ? key_before(key[l], slot[l], key[i], slot[i])
                                         : key_before(key[i], slot[i], key[l], slot[l]);
          const uint32_t ka = key[i], kb = key[l];
          const int sa = slot[i], sb = slot[l];
          key[i] = swap ? kb : ka;
          key[l] = swap ? ka : kb;
          slot[i] = swap ? sb : sa;
          slot[l] = swap ? sa : sb;
        }
      }
  float sel_v = 0.0f;   // lane r keeps round r's value and expert
  int sel_e = 0;
  for (int r = 0; r < top_k; ++r) {
    // the lane's head is its best remaining expert (ties: smaller expert)
    const uint32_t mk = wave_reduce_u32<true>(key[0]);
    const uint32_t cand = (key[0] == mk && mk != 0u) ? (uint32_t)(lane + 64 * slot[0]) : 0xffffffffu;
    const uint32_t win = wave_reduce_u32<false>(cand);
    if ((int)win % 64 == lane) {
#pragma unroll
      for (int j = 0; j + 1 < NK; ++j) {
        key[j] = key[j + 1];
        slot[j] = slot[j + 1];
      }
      key[NK - 1] = 0u;
    }
    if (lane == r) {
      sel_v = from_key(mk);
      sel_e = (int)win;
    }
  }
  // softmax over the selected logits (round 0 holds the largest), summed in
  // float in selection order by lane 0
  const float m = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sel_v), 0));
  const float ex = lane < top_k ? expf(sel_v - m) : 0.0f;
  float s = 0.0f;
  for (int r = 0; r < top_k; ++r)
    s += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ex), r));
  if (lane < top_k) {
    idx[(int64_t)row * top_k + lane] = sel_e;
    wout[(int64_t)row * top_k + lane] = ex / s;
  }
}

}  // namespace

int launch_moe_route(const float* logits, int32_t* idx, float* w, int64_t rows, int64_t E,
                     int64_t top_k, const void* x, const void* sgw, void* sgate, int64_t H,
                     int dtype, hipStream_t st) {
  if (E < 1 || E > 64 * kRouteMaxPerLane || top_k < 1 || top_k > 64 || top_k > E)
    return kStatusUnsupported;
  const dim3 grid((unsigned)rows), block(kRouteThreads);
  const bool sg = x != nullptr;
  int nk = 1;
  while (64 * nk < E) nk *= 2;
#define MQ_ROUTE(DT, SG, NK)                                                                    \
  hipLaunchKernelGGL((moe_route_kernel<DT, SG, NK>), grid, block, 0, st, logits, idx, w,        \
                     (const uint16_t*)x, (const uint16_t*)sgw, (uint16_t*)sgate, (int)E, (int)H, \
                     (int)top_k)
#define MQ_ROUTE_NK(DT, SG)                                                                     \
  switch (nk) {                                                                                  \
    case 1: MQ_ROUTE(DT, SG, 1); break;                                                          \
    case 2: MQ_ROUTE(DT, SG, 2); break;                                                          \
    case 4: MQ_ROUTE(DT, SG, 4); break;                                                          \
    case 8: MQ_ROUTE(DT, SG, 8); break;                                                          \
    default: MQ_ROUTE(DT, SG, 16); break;                                                        \
  }
  if (dtype == kBF16) {
    if (sg) MQ_ROUTE_NK(kBF16, true)
    else MQ_ROUTE_NK(kBF16, false)
  } else if (dtype == kF16) {
    if (sg) MQ_ROUTE_NK(kF16, true)
    else MQ_ROUTE_NK(kF16, false)
  } else {
    return kStatusUnsupported;
  }
#undef MQ_ROUTE_NK
#undef MQ_ROUTE
  return 0;
}

}  // namespace mq
