// MoE routing pieces shared by the routing kernel (route.hip) and the decode
// GLU gather that routes its own tokens (gather.cuh, ROUTE): each piece is
// computed by one whole wave, so both kernels give the same bits.
//
// Reference behaviour: mlxturbo/kernels/moe_route_decode.py:151-327
// (`route`): per row, top_k rounds of "take the largest logit and drop it"
// (equal values: the smaller expert index wins, as torch.topk / HF decide),
// then a softmax over the selected logits with the largest subtracted, summed
// in float in selection order; the shared expert's gate sigmoid(T(x . sgw))
// with the dot summed in float and the sigmoid evaluated in T one operation
// at a time (MLX's form: y = 1 / (1 + exp(|s|)), s < 0 ? y : 1 - y, each
// step rounded to T).
#pragma once
#include "mq_common.h"

namespace mq {

// experts per lane: E <= 64 kRouteMaxPerLane
constexpr int kRouteMaxPerLane = 16;

// Largest uint32 over the 64 lanes (all lanes active), returned to every
// lane: inclusive row scans (row_shr 1, 2, 4, 8), the row ends broadcast
// into the following rows (row_bcast 15 into rows 1 and 3, row_bcast 31 into
// rows 2 and 3), the total read from lane 63.  Each step is one v_max_u32
// with the DPP source in place: a lane without a source lane (bound_ctrl
// off) or outside the row mask is not written and keeps its own value.
// Two wait states before each DPP read of the previous step's result.  (As
// a DPP move and a separate max the compiler took four instructions per
// step; as a compare-and-select it re-ran a DPP move under a partial exec
// mask, where disabled source lanes read as out of range.)
__device__ __forceinline__ uint32_t route_wave_max_u32(uint32_t x) {
  asm volatile(
      "s_nop 1\n\t"
      "v_max_u32_dpp %0, %0, %0 row_shr:1 row_mask:0xf bank_mask:0xf\n\t"
      "s_nop 1\n\t"
      "v_max_u32_dpp %0, %0, %0 row_shr:2 row_mask:0xf bank_mask:0xf\n\t"
      "s_nop 1\n\t"
      "v_max_u32_dpp %0, %0, %0 row_shr:4 row_mask:0xf bank_mask:0xf\n\t"
      "s_nop 1\n\t"
      "v_max_u32_dpp %0, %0, %0 row_shr:8 row_mask:0xf bank_mask:0xf\n\t"
      "s_nop 1\n\t"
      "v_max_u32_dpp %0, %0, %0 row_bcast:15 row_mask:0xa bank_mask:0xf\n\t"
      "s_nop 1\n\t"
      "v_max_u32_dpp %0, %0, %0 row_bcast:31 row_mask:0xc bank_mask:0xf\n\t"
      "s_nop 1"
      : "+v"(x));
  return (uint32_t)__builtin_amdgcn_readlane((int)x, 63);
}

// Sum over the 64 lanes (lanes without a source add 0), returned to every lane.
__device__ __forceinline__ float route_wave_sum_f32(float x) {
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
__device__ __forceinline__ uint32_t route_order_key(float v) {
  const uint32_t u = v == 0.0f ? 0u : __builtin_bit_cast(uint32_t, v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float route_from_key(uint32_t k) {
  return __builtin_bit_cast(float, (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// sigmoid in T, one rounding per operation (MLX's Sigmoid form)
template <int DT>
__device__ __forceinline__ uint16_t route_sigmoid_t(uint16_t s16) {
  using T = T16<DT>;
  const float s = T::to_f32(s16);
  const float e = T::to_f32(T::round1(expf(__builtin_fabsf(s))));
  const float d = T::to_f32(T::round1(1.0f + e));
  const float y = T::to_f32(T::round1(1.0f / d));
  return s < 0.0f ? T::round1(y) : T::round1(1.0f - y);
}

// x before y in the per-lane order: larger key, then smaller slot
__device__ __forceinline__ bool route_key_before(uint32_t kx, int ix, uint32_t ky, int iy) {
  return kx > ky || (kx == ky && ix < iy);
}

// The top_k experts of one row of E float logits, by one whole wave: lane l
// holds experts NK l .. NK l + NK - 1 (NK the power of two covering E / 64;
// 16-byte loads where the lane's block is whole and aligned) as
// order-preserving keys, sorts them once with a bitonic network, and each
// round is one wave reduction over the lanes' heads (the largest key) and a
// ballot: a lane's experts are one contiguous block, so the lowest lane
// whose head holds that key holds the smallest such expert.  That lane drops
// its head.  Lane r < top_k gets round r's expert and logit (expert -1 for a
// round with no expert left: E < top_k, or logits whose key is 0).
template <int NK>
__device__ __forceinline__ void route_wave_topk(const float* __restrict__ lr, int E, int top_k,
                                                int lane, int& sel_e, float& sel_v) {
  uint32_t key[NK];
  int slot[NK];                                 // expert = NK lane + slot
  const int e0 = NK * lane;
  bool vec = false;
  if constexpr (NK % 4 == 0) vec = e0 + NK <= E && ((uintptr_t)lr & 15u) == 0;
  if (vec) {
#pragma unroll
    for (int q = 0; q < NK / 4; ++q) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(lr + e0 + 4 * q);
#pragma unroll
      for (int i = 0; i < 4; ++i) key[4 * q + i] = route_order_key(v[i]);
    }
  } else {
#pragma unroll
    for (int j = 0; j < NK; ++j) key[j] = e0 + j < E ? route_order_key(lr[e0 + j]) : 0u;
  }
#pragma unroll
  for (int j = 0; j < NK; ++j) slot[j] = j;
  // bitonic sort of the lane's NK keys, descending in route_key_before order
#pragma unroll
  for (int k = 2; k <= NK; k <<= 1)
#pragma unroll
    for (int jj = k >> 1; jj > 0; jj >>= 1)
#pragma unroll
      for (int i = 0; i < NK; ++i) {
        const int l = i ^ jj;
        if (l > i) {
          const bool swap = (i & k) == 0 ? route_key_before(key[l], slot[l], key[i], slot[i])
                                         : route_key_before(key[i], slot[i], key[l], slot[l]);
          const uint32_t ka = key[i], kb = key[l];
          const int sa = slot[i], sb = slot[l];
          key[i] = swap ? kb : ka;
          key[l] = swap ? ka : kb;
          slot[i] = swap ? sb : sa;
          slot[l] = swap ? sa : sb;
        }
      }
  sel_v = 0.0f;
  sel_e = 0;
  for (int r = 0; r < top_k; ++r) {
    // the lane's head is its best remaining expert (ties: smaller expert)
    const uint32_t mk = route_wave_max_u32(key[0]);
    const uint64_t held = __builtin_amdgcn_ballot_w64(key[0] == mk && mk != 0u);
    int win = -1;
    if (held != 0) {
      const int wl = __builtin_ctzll(held);
      win = NK * wl + __builtin_amdgcn_readlane(slot[0], wl);
      if (lane == wl) {
#pragma unroll
        for (int j = 0; j + 1 < NK; ++j) {
          key[j] = key[j + 1];
          slot[j] = slot[j + 1];
        }
        key[NK - 1] = 0u;
      }
    }
    if (lane == r) {
      sel_v = route_from_key(mk);
      sel_e = win;
    }
  }
}

// The same selection by NWV waves of a workgroup (E <= 64 NWV, top_k <= 8,
// NWV * top_k <= 64), as ranks instead of rounds: wave w keys experts
// 64 w + lane, one per lane, as c = key * 64 + (63 - lane) (unique; larger c
// first, so equal keys go by the smaller expert), and each lane's rank is
// the number of c in its wave above its own (LDS broadcast reads, 64
// independent compares: no dependent chain of wave reductions).  Ranks
// below top_k (with key != 0) are the wave's candidates in round order, at
// LDS slot top_k w + rank; after a workgroup barrier wave 0 ranks the
// NWV top_k candidates the same way by key and slot (slot order keeps
// equal keys in expert order: waves hold increasing experts, and a wave's
// candidates take equal keys by increasing expert).  Every wave of the
// workgroup calls it (one barrier); lane r < top_k of wave 0 gets round
// r's expert and logit, as route_wave_topk gives them (expert -1 and the
// logit of key 0 for a round with no expert).  LDS: s_c [64 NWV], s_ck /
// s_ce [64].
template <int NWV>
__device__ __forceinline__ void route_block_topk(const float* __restrict__ lr, int E, int top_k,
                                                 int wv, int lane, uint64_t* s_c, uint32_t* s_ck,
                                                 int* s_ce, int& sel_e, float& sel_v) {
  static_assert(NWV * 8 <= 64, "the candidates fit one wave");
  auto wave_sync = [] {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  // rank of c among the 64 values at base (c itself counts 0)
  auto rank_of = [](const uint64_t* base, uint64_t c) {
    int rk = 0;
#pragma unroll
    for (int d = 0; d < 64; ++d) rk += base[d] > c ? 1 : 0;
    return rk;
  };
  const int e = 64 * wv + lane;
  const uint32_t k = e < E ? route_order_key(lr[e]) : 0u;
  const uint64_t c = ((uint64_t)k << 6) | (uint64_t)(63 - lane);
  s_c[64 * wv + lane] = c;
  if (lane < top_k) {
    s_ck[top_k * wv + lane] = 0u;
    s_ce[top_k * wv + lane] = -1;
  }
  wave_sync();
  const int rk = rank_of(s_c + 64 * wv, c);
  if (k != 0u && rk < top_k) {
    s_ck[top_k * wv + rk] = k;
    s_ce[top_k * wv + rk] = e;
  }
  __syncthreads();
  sel_v = 0.0f;
  sel_e = 0;
  if (wv == 0) {
    const uint32_t k2 = lane < NWV * top_k ? s_ck[lane] : 0u;
    const int e2 = lane < NWV * top_k ? s_ce[lane] : -1;
    const uint64_t c2 = ((uint64_t)k2 << 6) | (uint64_t)(63 - lane);
    s_c[lane] = c2;                               // stage 1's values are read
    wave_sync();
    const int rk2 = rank_of(s_c, c2);
    wave_sync();
    // round r's key and expert, at s_c / s_ce slots 64 + r (key 0, -1: none)
    uint32_t* ok = reinterpret_cast<uint32_t*>(s_c + 64);
    int* oe = reinterpret_cast<int*>(s_c + 64) + 8;
    if (lane < top_k) {
      ok[lane] = 0u;
      oe[lane] = -1;
    }
    wave_sync();
    if (k2 != 0u && rk2 < top_k) {
      ok[rk2] = k2;
      oe[rk2] = e2;
    }
    wave_sync();
    if (lane < top_k) {
      sel_v = route_from_key(ok[lane]);
      sel_e = oe[lane];
    }
  }
}

// Softmax weight of lane r < top_k over the selected logits (round 0 holds
// the largest), summed in float in selection order; 0 on other lanes.
__device__ __forceinline__ float route_wave_softmax(float sel_v, int lane, int top_k) {
  const float m =
      __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sel_v), 0));
  const float ex = lane < top_k ? expf(sel_v - m) : 0.0f;
  float s = 0.0f;
  for (int r = 0; r < top_k; ++r)
    s += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ex), r));
  return lane < top_k ? ex / s : 0.0f;
}

// The shared expert's gate sigmoid(T(x . sgw)) of one row by one whole
// wave: lane l sums the 16-byte pieces l, l + 64, ... of x and the gate
// weight (eight values each, in piece order) in float, or the elements l,
// l + 64, ... of a ragged or unaligned row; then the wave sum, rounded to T.
template <int DT>
__device__ __forceinline__ uint16_t route_wave_shared_gate(const uint16_t* __restrict__ xr,
                                                           const uint16_t* __restrict__ sgw,
                                                           int H, int lane) {
  using T = T16<DT>;
  float acc = 0.0f;
  const bool vec = H % 8 == 0 && (((uintptr_t)xr | (uintptr_t)sgw) & 15u) == 0;
  if (vec) {
    const u32x4* xv = reinterpret_cast<const u32x4*>(xr);
    const u32x4* gv = reinterpret_cast<const u32x4*>(sgw);
    for (int c0 = lane; c0 < H / 8; c0 += 4 * 64) {
      u32x4 a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = c0 + i * 64;
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
    for (int h = lane; h < H; h += 64) acc += T::to_f32(xr[h]) * T::to_f32(sgw[h]);
  }
  acc = route_wave_sum_f32(acc);
  return route_sigmoid_t<DT>(T::round1(acc));
}

}  // namespace mq
