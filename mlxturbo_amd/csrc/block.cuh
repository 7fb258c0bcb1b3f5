// The decode MoE block of one token in one launch: routing, the fused
// gate+up+SiLU gather, and the down projection with the router-weighted
// combine and the shared-expert merge.
//
// Reference behaviour: moe_route_decode.py:151-327 (route) and 353-398
// (combine with the shared expert) around moe_decode_fused.py:331-397 (the
// decode gate/up and down kernels); the same bits as mq_moe_glu_route
// followed by mq_gather_qmm_combine, which run the same tile code
// (gather.cuh) as two dependent launches.
//
// CDNA4 design.  Phase 1 is the routed GLU gather at one token: every
// workgroup routes the token with all its waves (route.cuh route_block_topk,
// ranks instead of rounds: routed 3.3 us into the launch, against 3.8 with
// one wave's sorted rounds and 4.2 with rounds on 8 waves), and workgroup i
// computes the 16 h columns (i mod nsl) of the (i / nsl)-th selected
// expert.  The down projection needs every h value, so phase 2 starts
// behind a grid-wide arrival: the h tiles are stored with device-scope
// stores (sc1, written through to the point of coherence of all XCDs), each
// workgroup waits for its stores to complete and then sets its arrival flag
// to the call's epoch + 1, and the first ceil(N2 / 16) workgroups, which
// run phase 2, poll the flags with device-scope loads and read h the same
// way.  No L2 write-back
// or invalidate runs (a device-scope release per workgroup cost more than
// the launch it would save, since it writes back the XCD's whole L2).
//
// The epoch (a device word) is read by every workgroup at its start and
// advanced by workgroup 0 once every flag holds epoch + 1, that is once
// every workgroup of the call has read it, so no flag is ever cleared.
// The grid must be resident at once: the launcher checks the occupancy, and
// the poll is bounded, so a grid that is not resident ends the call with NaN
// outputs instead of a hang.  Calls that overlap on one GPU race on the
// flags; a stream's calls run one after another.
#pragma once
#include "gather.cuh"

namespace mq {

constexpr int kBlockMaxGrid = 256;             // arrival flags, four per polling lane
constexpr int kBlockSpin = 1 << 18;            // poll rounds before giving up
static __device__ uint32_t g_block_epoch;
static __device__ uint32_t g_block_flags[kBlockMaxGrid];

// Phase-1 rows: the token's x, h tile of pair p stored device-wide.
template <int DT>
struct BlockGluRows {
  static constexpr bool kCombine = true;
  const uint16_t* x;
  uint32_t x_nrec;
  uint16_t* out;
  int K, N, n0, p;
  __device__ __forceinline__ int64_t xoff(int m) const { return (int64_t)m * K; }
  __device__ __forceinline__ void store_combined(int m, int nn, const float (&v)[2]) const {
    (void)m;
    const float g = v[0], u = v[1];
    const uint16_t hv = T16<DT>::round1(g / (1.0f + __expf(-g)) * u);
    __hip_atomic_store(out + (int64_t)p * N + n0 + nn, hv, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
};

// Phase-2 rows: A row = h row of pair p, read with device-scope loads; the
// tile's y values go to the workgroup's LDS copy.
struct BlockFoldRows {
  static constexpr bool kCombine = false;
  static constexpr int kXAux = 16;             // sc1: coherent across the XCDs' L2s
  const uint16_t* x;
  uint32_t x_nrec;
  uint16_t (*ys)[16];
  int K, p;
  __device__ __forceinline__ int64_t xoff(int m) const { return (int64_t)(p + m) * K; }
  __device__ __forceinline__ void store(int m, int nn, uint16_t v) const { ys[p + m][nn] = v; }
};

// 1-D grid of top_k * ceil(N1 / 16) <= kBlockMaxGrid workgroups of NW waves: the
// phase-1 tile on waves 0 .. NWT-1 (the others take its barriers and
// wait), the phase-2 tiles one per wave and round; x [K1], logits [E]
// (E <= 512),
// gate / up banks [E, N1, K1], down bank [E, N2, K2 = N1], h [top_k, N1],
// out [N2].  ROUTE: logits [E] in ra.logits, and ra.idx / ra.w / ra.sgate
// get the routing as mq_moe_route writes it; else the pairs' experts and
// router weights are given in ra.idx / ra.w (an expert outside [0, E)
// gives a zero row, as in the gather).  SH (with ROUTE): shared [N2] merged
// with the gate sigmoid(T(x . ra.sgw)).
template <int DT, int BITS, int GS, int NW, int NWT, bool ROUTE, bool SH>
__global__ __launch_bounds__(64 * NW) void moe_block1_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ wg,
    const uint16_t* __restrict__ sg, const uint16_t* __restrict__ bg,
    const uint32_t* __restrict__ wu, const uint16_t* __restrict__ su,
    const uint16_t* __restrict__ bu, const uint32_t* __restrict__ wd,
    const uint16_t* __restrict__ sd, const uint16_t* __restrict__ bd,
    const uint16_t* __restrict__ shared, uint16_t* h, uint16_t* __restrict__ out, int N1, int K1,
    int N2, int E, int n2, RouteArgs ra) {
  extern __shared__ __align__(16) unsigned char qmv_smem[];
  using C = QmvConf<BITS, GS>;
  using T = T16<DT>;
  constexpr int NPOLL = NW < 4 ? NW : 4;       // waves polling the arrival flags
  static_assert(NW == 8 && NWT < NW, "8 waves: routing over 512 experts, a free wave per tile");
  static_assert(ROUTE || !SH, "the shared expert's gate comes with the routing");
  __shared__ f32x4 red[NW * 2][64];
  __shared__ uint16_t s_y[8][16];
  __shared__ int s_sel[8];
  __shared__ float s_w[8];
  __shared__ int s_expert;
  __shared__ uint32_t s_ep;
  __shared__ int s_ok;
  const int t = threadIdx.x, lane = t & 63;
  const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
  const int top_k = ra.top_k;
  const int nsl = (N1 + 15) / 16;
  const int seg = blockIdx.x / nsl, slot = blockIdx.x - seg * nsl;
  const int ngrid = gridDim.x;
  if (t == 0) s_ep = __hip_atomic_load(&g_block_epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // routing by the workgroup's waves (route_block_topk, one barrier), then
  // the softmax on wave 0; or the given experts and weights
  if constexpr (ROUTE) {
    __shared__ uint64_t s_c[64 * NW];
    __shared__ uint32_t s_ck[64];
    __shared__ int s_ce[64];
    int sel_e;
    float sel_v;
    route_block_topk<NW>(ra.logits, E, top_k, wv, lane, s_c, s_ck, s_ce, sel_e, sel_v);
    if (wv == 0) {
      const float wgt = route_wave_softmax(sel_v, lane, top_k);
      if (blockIdx.x == 0 && lane < top_k) {
        ra.idx[lane] = sel_e;
        ra.w[lane] = wgt;
      }
      if (lane < top_k) {
        s_sel[lane] = sel_e >= 0 ? sel_e : E;    // a round with no expert: zeros
        s_w[lane] = wgt;
      }
      const int es = __builtin_amdgcn_readlane(sel_e, seg < top_k ? seg : 0);
      if (lane == 0) s_expert = es >= 0 ? es : E;
    }
  } else if (wv == 0) {
    const int ei = lane < top_k ? ra.idx[lane] : 0;
    const int ek = (unsigned)ei < (unsigned)E ? ei : E;
    if (lane < top_k) {
      s_sel[lane] = ek;
      s_w[lane] = ra.w[lane];
    }
    const int es = __builtin_amdgcn_readlane(ek, seg < top_k ? seg : 0);
    if (lane == 0) s_expert = es;
  }
  __syncthreads();
  // the shared gate in workgroup 0 on its last wave, which the phase-1 tile
  // leaves free (phase 2 reads the gate after the arrival)
  if (SH && blockIdx.x == 0 && wv == NW - 1) {
    const uint16_t gsh = route_wave_shared_gate<DT>(x, ra.sgw, K1, lane);
    if (lane == 0)
      __hip_atomic_store(ra.sgate, gsh, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // ---- phase 1: 16 columns of h for pair seg, on waves 0 .. NWT-1 ---------
  {
    const int e = s_expert;
    const int n0 = slot * 16;
    const int rows = min(16, N1 - n0);
    if (seg < top_k && e >= E) {
      if (t < rows)
        __hip_atomic_store(h + (int64_t)seg * N1 + n0 + t, (uint16_t)0, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    } else if (seg < top_k && wv >= NWT) {
#pragma unroll
      for (int b = 0; b < qmv_tile_barriers<NWT, false>(); ++b) __syncthreads();
    } else if (seg < top_k) {
      const uint32_t rowB = (uint32_t)K1 * BITS / 8;
      const uint32_t sRowB = (uint32_t)(K1 / GS) * 2;
      const int64_t row0 = (int64_t)e * N1 + (rows > 0 ? n0 : 0);
      QmvTiles<2> tl;
      tl.w[0] = reinterpret_cast<const char*>(wg) + row0 * rowB;
      tl.s[0] = reinterpret_cast<const char*>(sg) + row0 * sRowB;
      tl.b[0] = reinterpret_cast<const char*>(bg) + row0 * sRowB;
      tl.w[1] = reinterpret_cast<const char*>(wu) + row0 * rowB;
      tl.s[1] = reinterpret_cast<const char*>(su) + row0 * sRowB;
      tl.b[1] = reinterpret_cast<const char*>(bu) + row0 * sRowB;
      tl.rows[0] = tl.rows[1] = rows;
      const BlockGluRows<DT> src{x, (uint32_t)K1 * 2u, h, K1, N1, n0, seg};
      qmv_tile<DT, BITS, GS, C::GPL, NWT, C::PF, 1, false, 2>(tl, 1, K1, src, qmv_smem, red, wv,
                                                             t);
    }
  }
  // ---- arrival: every wave's h stores complete, then the flag --------------
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  const uint32_t want = s_ep + 1u;
  if (t == 0)
    __hip_atomic_store(&g_block_flags[blockIdx.x], want, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  if ((int)blockIdx.x >= n2) return;

  // ---- phase 2: wait for every workgroup's h ------------------------------
  // NPOLL waves poll, each starting ~0.2 us after the previous one so that
  // a poll is in flight more often than once per memory round trip; the
  // first to see every flag tells the others through LDS
  __shared__ int s_done;
  if (t == 0) s_done = 0;
  __syncthreads();
  if (wv < NPOLL) {
    for (int d = 0; d < wv; ++d) __builtin_amdgcn_s_sleep(8);
    int ok = 0;
    for (int it = 0; it < kBlockSpin; ++it) {
      if (*(volatile int*)&s_done) {
        ok = 1;
        break;
      }
      // every flag load issued before the first compare (one round trip);
      // unconditional, lanes past the grid re-read its last flag
      uint32_t fl[kBlockMaxGrid / 64];
#pragma unroll
      for (int q = 0; q < kBlockMaxGrid / 64; ++q)
        fl[q] = __hip_atomic_load(&g_block_flags[min(lane + 64 * q, ngrid - 1)], __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
      bool mine = true;
#pragma unroll
      for (int q = 0; q < kBlockMaxGrid / 64; ++q) mine &= fl[q] == want;
      if (__builtin_amdgcn_ballot_w64(!mine) == 0) {
        ok = 1;
        if (lane == 0) *(volatile int*)&s_done = 1;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    if (wv == 0 && lane == 0) {
      s_ok = ok;
      // every workgroup has read the epoch once every flag holds want
      if (blockIdx.x == 0)
        __hip_atomic_store(&g_block_epoch, want, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
  const int n0 = blockIdx.x * 16;
  const int rows = min(16, N2 - n0);
  if (!s_ok) {                                  // the grid was not resident: NaN, not a hang
    if (t < rows) out[n0 + t] = T::round1(__builtin_nanf(""));
    return;
  }

  // ---- phase 2: down tiles of the top_k pairs, one per wave and round -----
  const int K2 = N1;
  const uint32_t rowB = (uint32_t)K2 * BITS / 8;
  const uint32_t sRowB = (uint32_t)(K2 / GS) * 2;
  unsigned char* gsm2 = qmv_smem + wv * gather_group_lds<BITS, GS, C::GPL>(1, 1, false, K2 / GS, 1);
  const int rounds = (top_k + NW - 1) / NW;
  for (int rd = 0; rd < rounds; ++rd) {
    const int p = rd * NW + wv;                  // wave-uniform
    const int e = p < top_k ? s_sel[p] : E;
    const bool live = p < top_k && e < E && rows > 0;
    if (p < top_k && e >= E && lane < 16) s_y[p][lane] = 0;
    const int64_t row0 = (int64_t)(live ? e : 0) * N2 + (live ? n0 : 0);
    QmvTiles<1> tl;
    tl.w[0] = reinterpret_cast<const char*>(wd) + row0 * rowB;
    tl.s[0] = reinterpret_cast<const char*>(sd) + row0 * sRowB;
    tl.b[0] = reinterpret_cast<const char*>(bd) + row0 * sRowB;
    tl.rows[0] = live ? rows : 0;
    const BlockFoldRows src{h, (uint32_t)top_k * (uint32_t)K2 * 2u, s_y, K2, live ? p : 0};
    qmv_tile<DT, BITS, GS, C::GPL, 1, C::PF, 1, false, 1>(tl, 1, K2, src, gsm2, red + wv, 0, lane);
  }
  __syncthreads();
  // the combine, as mq_moe_combine(_shared) sums it: k order, fma, rounded once
  if (t < rows) {
    float acc = 0.f;
    for (int k = 0; k < top_k; ++k) acc = __builtin_fmaf(s_w[k], T::to_f32(s_y[k][t]), acc);
    uint16_t o = T::round1(acc);
    if constexpr (SH) {
#pragma clang fp contract(off)
      const uint16_t sgv =
          __hip_atomic_load(ra.sgate, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const uint16_t m = T::round1(T::to_f32(sgv) * T::to_f32(shared[n0 + t]));
      o = T::round1(T::to_f32(o) + T::to_f32(m));
    }
    out[n0 + t] = o;
  }
}

// The launch (one token): kStatusUnsupported where the block's tile
// configuration is not this kernel's (phase-1 tiles of 4 waves without the
// scale copy, phase-2 tiles of one wave), top_k > 8, E > 512, or the grid
// does not fit the device at once; the caller then runs the two launches.
// Workgroups of 8 waves: the phase-1 tile takes 4 of them on every CU (a
// grid of half as many workgroups, each with two tiles, left half the CUs
// idle and took 5.2 against 3.3 us for the tiles), and all top_k <= 8
// phase-2 tiles run in one round (two rounds on 4 waves: 3.5 against 2.6
// us; config-4 banks, per-workgroup timestamps).  Grids of at most 256
// workgroups: their arrival flags are polled four per lane (16 per lane for
// up to 1024 workgroups: 14.0 against 13.7 us per block).
template <int DT, int BITS, int GS>
int MoeBlockLaunch<DT, BITS, GS>::run(const void* x, const uint32_t* wg, const void* sg,
                                      const void* bg, const uint32_t* wu, const void* su,
                                      const void* bu, const uint32_t* wd, const void* sd,
                                      const void* bd, const void* shared, void* h, void* out,
                                      int64_t N1, int64_t K1, int64_t N2, int64_t E,
                                      const RouteArgs& ra, hipStream_t st, int* nlaunch) {
  using C = QmvConf<BITS, GS>;
  constexpr int NW = 8;
  const int64_t top_k = ra.top_k;
  if (top_k < 1 || top_k > 8 || E > 512 || top_k > E || (ra.sgw != nullptr) != (shared != nullptr))
    return kStatusUnsupported;
  // the gather launches' choices for these shapes (gather_tile_waves /
  // gather_tile_sb), which this kernel's tiles must repeat
  if (gather_tile_waves<BITS, GS>(top_k, N1, K1) != 4 || gather_tile_sb<BITS, GS>(K1, 4))
    return kStatusUnsupported;
  if (gather_tile_waves<BITS, GS>(top_k, N2, N1) != 1 || gather_tile_sb<BITS, GS>(N1, 1))
    return kStatusUnsupported;
  const int64_t grid = top_k * ((N1 + 15) / 16), n2 = (N2 + 15) / 16;
  if (grid > kBlockMaxGrid || n2 > grid) return kStatusUnsupported;
  const size_t lds1 = gather_group_lds<BITS, GS, C::GPL>(4, 1, false, (int)(K1 / GS), 2);
  const size_t lds2 = NW * gather_group_lds<BITS, GS, C::GPL>(1, 1, false, (int)(N1 / GS), 1);
  const size_t lds = lds1 > lds2 ? lds1 : lds2;
  const bool sh = shared != nullptr, route = ra.logits != nullptr;
  if (sh && !route) return kStatusUnsupported;
  const void* kern =
      !route ? reinterpret_cast<const void*>(&moe_block1_kernel<DT, BITS, GS, NW, 4, false, false>)
      : sh   ? reinterpret_cast<const void*>(&moe_block1_kernel<DT, BITS, GS, NW, 4, true, true>)
             : reinterpret_cast<const void*>(&moe_block1_kernel<DT, BITS, GS, NW, 4, true, false>);
  // every workgroup resident at once (the arrival waits for all of them);
  // the occupancy query is kept per kernel and LDS size
  static std::atomic<uint64_t> occ[3];
  const int ki = route ? 1 + sh : 0;
  const uint64_t key = (uint64_t)lds << 32;
  uint64_t got = occ[ki].load(std::memory_order_relaxed);
  if ((got & ~0xffffffffull) != key || got == 0) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, 64 * NW, lds) != hipSuccess)
      return kStatusUnsupported;
    got = key | (uint32_t)(per_cu + 1);
    occ[ki].store(got, std::memory_order_relaxed);
  }
  const int64_t per_cu = (int64_t)(got & 0xffffffffull) - 1;
  if (per_cu * device_cu_count() < grid) return kStatusUnsupported;
#define MQ_BLK(RT, SH)                                                                          \
  hipLaunchKernelGGL((moe_block1_kernel<DT, BITS, GS, NW, 4, RT, SH>), dim3((unsigned)grid),   \
                     dim3(64 * NW), lds, st, (const uint16_t*)x, wg, (const uint16_t*)sg,       \
                     (const uint16_t*)bg, wu, (const uint16_t*)su, (const uint16_t*)bu, wd,     \
                     (const uint16_t*)sd, (const uint16_t*)bd, (const uint16_t*)shared,         \
                     (uint16_t*)h, (uint16_t*)out, (int)N1, (int)K1, (int)N2, (int)E, (int)n2, \
                     ra)
  if (!route) MQ_BLK(false, false);
  else if (sh) MQ_BLK(true, true);
  else MQ_BLK(true, false);
#undef MQ_BLK
  *nlaunch += 1;
  return 0;
}

}  // namespace mq
