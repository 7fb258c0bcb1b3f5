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
// CDNA4 design: one workgroup of two waves per row, each piece one whole
// wave (csrc/route.cuh, shared with the decode GLU gather that routes its
// own tokens, so both give the same bits).  Wave 0 runs the top-k: lane l
// holds the contiguous block of experts NK l .. NK l + NK - 1 (NK the power
// of two covering E / 64, up to 16 for E <= 1024) as order-preserving
// integer keys, sorts them once with a bitonic network, and each round is
// one DPP wave reduction over the lanes' heads (the largest key) and a
// ballot (the lowest lane holding it holds the smallest such expert), after
// which the winning lane drops its head, no barrier.  (A lane-local argmax
// per round made each round one long dependent chain: 3.2 us for eight
// rounds.)  Wave 1 computes the shared gate's dot product (16-byte loads,
// four per lane in flight, one DPP wave sum).  Latency-bound: bytes per row
// 4 E + 4 H (x and the gate weight, 16-bit) plus 8 top_k out.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "launch.h"
#include "route.cuh"

namespace mq {

namespace {

constexpr int kRouteThreads = 128;

template <int DT, bool SG, int NK>
__global__ __launch_bounds__(kRouteThreads) void moe_route_kernel(
    const float* __restrict__ logits, int32_t* __restrict__ idx, float* __restrict__ wout,
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ sgw, uint16_t* __restrict__ sgate,
    int E, int H, int top_k) {
  const int row = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (wv == 1) {
    if constexpr (SG) {
      const uint16_t g = route_wave_shared_gate<DT>(x + (int64_t)row * H, sgw, H, lane);
      if (lane == 0) sgate[row] = g;
    }
    return;
  }
  int sel_e;
  float sel_v;
  route_wave_topk<NK>(logits + (int64_t)row * E, E, top_k, lane, sel_e, sel_v);
  const float wgt = route_wave_softmax(sel_v, lane, top_k);
  if (lane < top_k) {
    idx[(int64_t)row * top_k + lane] = sel_e;
    wout[(int64_t)row * top_k + lane] = wgt;
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
