// The decode MoE block of 1-8 tokens in one launch: routing, the fused
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
// Two to eight tokens (moe_blockn_kernel) take the same two phases with
// the tile configurations the separate gather launches pick for those
// shapes: token t is routed on wave t, the pairs are grouped into segments
// of up to min(8, T) pairs sharing an expert (one dequantized tile serves
// them all), phase-1 units are (segment, 16 columns) per wave group, and
// phase 2 deals (16-column block, token group) units.
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
  int K, p, j;                                 // h row p, LDS row j
  __device__ __forceinline__ int64_t xoff(int m) const { return (int64_t)(p + m) * K; }
  __device__ __forceinline__ void store(int m, int nn, uint16_t v) const { ys[j + m][nn] = v; }
};

// Phase-1 rows of a segment (pairs sharing an expert, T > 1): A row m is
// the token of pair members[m] (pair p's token is p / top_k), its h row is
// stored device-wide.
template <int DT>
struct BlockSegRows {
  static constexpr bool kCombine = true;
  const uint16_t* x;
  uint32_t x_nrec;
  uint16_t* out;
  const int* members;                          // LDS
  int top_k, K, N, n0;
  __device__ __forceinline__ int64_t xoff(int m) const {
    return (int64_t)(members[m] / top_k) * K;
  }
  __device__ __forceinline__ void store_combined(int m, int nn, const float (&v)[2]) const {
    const float g = v[0], u = v[1];
    const uint16_t hv = T16<DT>::round1(g / (1.0f + __expf(-g)) * u);
    __hip_atomic_store(out + (int64_t)members[m] * N + n0 + nn, hv, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
};

// The arrival of a workgroup: its waves' device-scope stores complete, then
// its flag holds want.
__device__ __forceinline__ void block_arrive(uint32_t want) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0)
    __hip_atomic_store(&g_block_flags[blockIdx.x], want, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// The wait of a workgroup that reads every workgroup's stores: true once
// every flag of the grid holds want, false after kBlockSpin polls (a grid
// that is not resident).  NPOLL waves poll, each starting ~0.2 us after the
// previous one so that a poll is in flight more often than once per memory
// round trip; the first to see every flag tells the others through LDS.
// Workgroup 0 then advances the epoch: every workgroup read it before
// setting its flag.  s_done / s_ok: two LDS words of the workgroup.
template <int NPOLL>
__device__ __forceinline__ bool block_wait(uint32_t want, int* s_done, int* s_ok) {
  const int t = threadIdx.x, lane = t & 63;
  const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
  const int ngrid = gridDim.x;
  if (t == 0) *s_done = 0;
  __syncthreads();
  if (wv < NPOLL) {
    for (int d = 0; d < wv; ++d) __builtin_amdgcn_s_sleep(8);
    int ok = 0;
    for (int it = 0; it < kBlockSpin; ++it) {
      if (*(volatile int*)s_done) {
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
        if (lane == 0) *(volatile int*)s_done = 1;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    if (wv == 0 && lane == 0) {
      *s_ok = ok;
      if (blockIdx.x == 0)
        __hip_atomic_store(&g_block_epoch, want, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
  return *s_ok != 0;
}

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
  // ---- arrival, then phase 2 waits for every workgroup's h ----------------
  const uint32_t want = s_ep + 1u;
  block_arrive(want);
  if ((int)blockIdx.x >= n2) return;
  __shared__ int s_done;
  const bool ok = block_wait<NPOLL>(want, &s_done, &s_ok);
  const int n0 = blockIdx.x * 16;
  const int rows = min(16, N2 - n0);
  if (!ok) {                                    // the grid was not resident: NaN, not a hang
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
    const BlockFoldRows src{h, (uint32_t)top_k * (uint32_t)K2 * 2u, s_y, K2, live ? p : 0,
                            live ? p : 0};
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

// T = 2 .. 8 tokens (P = T top_k <= 64 pairs): the same two phases over
// the tile configuration the gather launches pick for these shapes.  Every
// workgroup routes the tokens (token t on wave t, route_wave_topk, as the
// routed gate+up launch does) or reads the given experts, then groups the
// pairs into segments as the gather kernel does (up to min(8, T) pairs of
// one expert, numbered by leader position), so each expert's weights are
// dequantized once per segment.  Phase 1: unit u = (segment, 16 columns),
// NG = 8 / NWT groups of NWT waves per workgroup, group g of workgroup b
// taking units (r G + b) NG + g in rounds r.  Phase 2 on the first n2 tg
// workgroups:
// column block (b mod n2) for the tokens of group b / n2, one pair's down
// tile per wave and round, then the combine per token.  Dynamic LDS: the
// larger of NG phase-1 groups (gather_group_lds(NWT, 8, SBL, K1 / GS, 2))
// and 8 one-wave down tiles.
template <int DT, int BITS, int GS, int NWT, bool SBL, bool ROUTE, bool SH>
__global__ __launch_bounds__(512) void moe_blockn_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ wg,
    const uint16_t* __restrict__ sg, const uint16_t* __restrict__ bg,
    const uint32_t* __restrict__ wu, const uint16_t* __restrict__ su,
    const uint16_t* __restrict__ bu, const uint32_t* __restrict__ wd,
    const uint16_t* __restrict__ sd, const uint16_t* __restrict__ bd,
    const uint16_t* __restrict__ shared, uint16_t* h, uint16_t* __restrict__ out, int T, int N1,
    int K1, int N2, int E, int n2, int tgn, RouteArgs ra) {
  extern __shared__ __align__(16) unsigned char qmv_smem[];
  using C = QmvConf<BITS, GS>;
  using TT = T16<DT>;
  constexpr int NW = 8, NG = NW / NWT;
  static_assert(ROUTE || !SH, "the shared expert's gate comes with the routing");
  __shared__ f32x4 red[NW * 2][64];
  __shared__ uint16_t s_y[64][16];
  __shared__ int s_key[64];
  __shared__ float s_w[64];
  __shared__ int s_segk[64], s_segn[64];
  __shared__ int s_mem[64][8];
  __shared__ int s_nseg;
  __shared__ uint32_t s_ep;
  __shared__ int s_done, s_ok;
  const int t = threadIdx.x, lane = t & 63;
  const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
  const int top_k = ra.top_k, P = T * top_k, R = T < 8 ? T : 8;
  if (t == 0) s_ep = __hip_atomic_load(&g_block_epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (t < 64) s_segn[t] = 0;
  if constexpr (ROUTE) {
    if (wv < T) {
      int sel_e;
      float sel_v;
      route_wave_topk<8>(ra.logits + (int64_t)wv * E, E, top_k, lane, sel_e, sel_v);
      const float wgt = route_wave_softmax(sel_v, lane, top_k);
      if (lane < top_k) {
        s_key[wv * top_k + lane] = sel_e >= 0 ? sel_e : E;
        s_w[wv * top_k + lane] = wgt;
        if (blockIdx.x == 0) {
          ra.idx[wv * top_k + lane] = sel_e;
          ra.w[wv * top_k + lane] = wgt;
        }
      }
      // the shared gate of token wv, in workgroup 0 (phase 2 reads it after
      // the arrival)
      if (SH && blockIdx.x == 0) {
        const uint16_t gsh = route_wave_shared_gate<DT>(x + (int64_t)wv * K1, ra.sgw, K1, lane);
        if (lane == 0)
          __hip_atomic_store(ra.sgate + wv, gsh, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  } else if (wv == 0 && lane < P) {
    const int ei = ra.idx[lane];
    s_key[lane] = (unsigned)ei < (unsigned)E ? ei : E;
    s_w[lane] = ra.w[lane];
  }
  __syncthreads();
  // segments: pair p leads one when the number of earlier pairs with its key
  // is a multiple of R, segments numbered by leader position; a pair joins
  // the segment of the earlier pair of its key whose count is its own
  // rounded down to a multiple of R, at slot count mod R
  if (wv == 0) {
    const int key = lane < P ? s_key[lane] : -1;
    int cb = 0;
    for (int q = 0; q < P; ++q) {
      const int kq = __builtin_amdgcn_readlane(key, q);
      cb += (q < lane && kq == key) ? 1 : 0;
    }
    const bool lead = lane < P && cb % R == 0;
    const uint64_t lmask = __builtin_amdgcn_ballot_w64(lead);
    const int cb0 = cb - cb % R;
    int ldr = lane;
    for (int q = 0; q < P; ++q) {
      const int kq = __builtin_amdgcn_readlane(key, q);
      const int cq = __builtin_amdgcn_readlane(cb, q);
      if (kq == key && cq == cb0 && q <= lane) ldr = q;
    }
    if (lane < P) {
      const int sgi = __builtin_popcountll(lmask & ((1ull << ldr) - 1ull));
      s_mem[sgi][cb % R] = lane;
      atomicAdd(&s_segn[sgi], 1);
      if (lead) s_segk[sgi] = key;
    }
    if (lane == 0) s_nseg = __builtin_popcountll(lmask);
  }
  __syncthreads();
  const uint32_t want = s_ep + 1u;

  // ---- phase 1: units (segment, 16 columns), one per group and round -------
  // consecutive groups take consecutive units (a workgroup's groups mostly
  // share a segment's x rows); every group runs the same number of tiles,
  // empty ones (rows <= 0) where it has no unit or the unit's expert is
  // out of range, to keep the tiles' workgroup barriers
  {
    const int nsl = (N1 + 15) / 16;
    const int units = s_nseg * nsl;
    const int g = wv / NWT, kw = wv - g * NWT, gt = t - 64 * NWT * g;
    const int slots = NG * gridDim.x;
    const int rounds = (units + slots - 1) / slots;
    unsigned char* gsm =
        qmv_smem + g * gather_group_lds<BITS, GS, C::GPL>(NWT, kQmvMaxXM, SBL, K1 / GS, 2);
    const uint32_t rowB = (uint32_t)K1 * BITS / 8;
    const uint32_t sRowB = (uint32_t)(K1 / GS) * 2;
    for (int rd = 0; rd < rounds; ++rd) {        // uniform in the workgroup
      const int u = (rd * gridDim.x + blockIdx.x) * NG + g;   // wave-uniform
      const bool has = u < units;
      const int sgi = has ? u / nsl : 0, n0 = has ? (u - sgi * nsl) * 16 : 0;
      const int e = has ? s_segk[sgi] : E, M = has ? s_segn[sgi] : 1;
      const int rows = min(16, N1 - n0);
      if (has && e >= E) {                       // invalid pairs: zero rows
        for (int i = gt; i < M * 16; i += 64 * NWT)
          if ((i & 15) < rows)
            __hip_atomic_store(h + (int64_t)s_mem[sgi][i >> 4] * N1 + n0 + (i & 15),
                               (uint16_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      const bool live = has && e < E;
      const int64_t row0 = live ? (int64_t)e * N1 + n0 : 0;
      QmvTiles<2> tl;
      tl.w[0] = reinterpret_cast<const char*>(wg) + row0 * rowB;
      tl.s[0] = reinterpret_cast<const char*>(sg) + row0 * sRowB;
      tl.b[0] = reinterpret_cast<const char*>(bg) + row0 * sRowB;
      tl.w[1] = reinterpret_cast<const char*>(wu) + row0 * rowB;
      tl.s[1] = reinterpret_cast<const char*>(su) + row0 * sRowB;
      tl.b[1] = reinterpret_cast<const char*>(bu) + row0 * sRowB;
      tl.rows[0] = tl.rows[1] = live ? rows : 0;
      const BlockSegRows<DT> src{x, (uint32_t)T * (uint32_t)K1 * 2u, h, s_mem[sgi], top_k, K1,
                                 N1, n0};
      if (!live || M == 1)
        qmv_tile<DT, BITS, GS, C::GPL, NWT, C::PF, 1, SBL, 2>(tl, 1, K1, src, gsm,
                                                              red + g * NWT * 2, kw, gt);
      else
        qmv_tile<DT, BITS, GS, C::GPL, NWT, C::PF, kQmvMaxXM, SBL, 2>(tl, M, K1, src, gsm,
                                                                      red + g * NWT * 2, kw, gt);
    }
  }
  // ---- arrival, then phase 2 waits for every workgroup's h ----------------
  block_arrive(want);
  if ((int)blockIdx.x >= n2 * tgn) return;
  const bool ok = block_wait<4>(want, &s_done, &s_ok);
  const int c = blockIdx.x % n2, tg = blockIdx.x / n2;
  const int tpg = (T + tgn - 1) / tgn;
  const int t0 = tg * tpg, t1 = min(T, t0 + tpg);
  const int np = (t1 - t0) * top_k;
  const int n0 = c * 16;
  const int rows = min(16, N2 - n0);
  if (!ok) {                                    // the grid was not resident: NaN, not a hang
    for (int i = t; i < (t1 - t0) * 16; i += 64 * NW)
      if ((i & 15) < rows) out[(int64_t)(t0 + (i >> 4)) * N2 + n0 + (i & 15)] =
          TT::round1(__builtin_nanf(""));
    return;
  }

  // ---- phase 2: the down tiles of the group's pairs, one per wave and round
  {
    const int K2 = N1;
    const uint32_t rowB = (uint32_t)K2 * BITS / 8;
    const uint32_t sRowB = (uint32_t)(K2 / GS) * 2;
    unsigned char* gsm2 =
        qmv_smem + wv * gather_group_lds<BITS, GS, C::GPL>(1, 1, false, K2 / GS, 1);
    const int rounds = (np + NW - 1) / NW;
    for (int rd = 0; rd < rounds; ++rd) {
      const int j = rd * NW + wv;                // wave-uniform
      const int p = t0 * top_k + j;
      const int e = j < np ? s_key[p] : E;
      const bool live = j < np && e < E && rows > 0;
      if (j < np && e >= E && lane < 16) s_y[j][lane] = 0;
      const int64_t row0 = (int64_t)(live ? e : 0) * N2 + (live ? n0 : 0);
      QmvTiles<1> tl;
      tl.w[0] = reinterpret_cast<const char*>(wd) + row0 * rowB;
      tl.s[0] = reinterpret_cast<const char*>(sd) + row0 * sRowB;
      tl.b[0] = reinterpret_cast<const char*>(bd) + row0 * sRowB;
      tl.rows[0] = live ? rows : 0;
      const BlockFoldRows src{h, (uint32_t)P * (uint32_t)K2 * 2u, s_y, K2, live ? p : 0,
                              live ? j : 0};
      qmv_tile<DT, BITS, GS, C::GPL, 1, C::PF, 1, false, 1>(tl, 1, K2, src, gsm2, red + wv, 0,
                                                           lane);
    }
  }
  __syncthreads();
  // the combine, as mq_moe_combine(_shared) sums it: k order, fma, rounded once
  for (int i = t; i < (t1 - t0) * 16; i += 64 * NW) {
    const int tl_ = i >> 4, nn = i & 15;
    if (nn >= rows) continue;
    const int tok = t0 + tl_;
    float acc = 0.f;
    for (int k = 0; k < top_k; ++k)
      acc = __builtin_fmaf(s_w[tok * top_k + k], TT::to_f32(s_y[tl_ * top_k + k][nn]), acc);
    uint16_t o = TT::round1(acc);
    if constexpr (SH) {
#pragma clang fp contract(off)
      const uint16_t sgv =
          __hip_atomic_load(ra.sgate + tok, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const uint16_t m = TT::round1(TT::to_f32(sgv) * TT::to_f32(shared[(int64_t)tok * N2 + n0 + nn]));
      o = TT::round1(TT::to_f32(o) + TT::to_f32(m));
    }
    out[(int64_t)tok * N2 + n0 + nn] = o;
  }
}

// The launch of T = 2 .. 8 tokens: kStatusUnsupported beyond 64 pairs, for
// tile configurations other than the gather launches' choices this kernel
// is built for (gate/up tiles over 4 waves without the scale copy, over 2
// or 1 with it; down tiles on one wave), or where the grid (one workgroup
// per CU, at most kBlockMaxGrid) is not resident at once.
template <int DT, int BITS, int GS>
inline int launch_blockn(const void* x, const uint32_t* wg, const void* sg, const void* bg,
                         const uint32_t* wu, const void* su, const void* bu, const uint32_t* wd,
                         const void* sd, const void* bd, const void* shared, void* h, void* out,
                         int64_t T, int64_t N1, int64_t K1, int64_t N2, int64_t E,
                         const RouteArgs& ra, hipStream_t st) {
  using C = QmvConf<BITS, GS>;
  const int64_t top_k = ra.top_k, P = T * top_k;
  if (T < 2 || T > 8 || P > 64 || top_k > E || E > 512) return kStatusUnsupported;
  const bool route = ra.logits != nullptr, sh = shared != nullptr;
  if (sh && !route) return kStatusUnsupported;
  // the gather launches' tile choices for these shapes
  const int nwt = gather_tile_waves<BITS, GS>(P, N1, K1);
  const int G1 = (int)(K1 / GS);
  const bool sbl = gather_tile_sb<BITS, GS>(K1, nwt) && qmv_sb_fits(G1, nwt, 2, sg, bg) &&
                   qmv_sb_fits(G1, nwt, 2, su, bu);
  if (!((nwt == 4 && !sbl) || (nwt == 2 && sbl) || (nwt == 1 && sbl))) return kStatusUnsupported;
  if (gather_tile_waves<BITS, GS>(P, N2, N1) != 1 || gather_tile_sb<BITS, GS>(N1, 1))
    return kStatusUnsupported;
  const int64_t G = device_cu_count() < kBlockMaxGrid ? device_cu_count() : kBlockMaxGrid;
  const int64_t n2 = (N2 + 15) / 16;
  if (n2 > G || N1 > INT32_MAX) return kStatusUnsupported;
  const int64_t tgn = T < G / n2 ? T : G / n2;
  const size_t lds1 = (size_t)(8 / nwt) *
                      gather_group_lds<BITS, GS, C::GPL>(nwt, kQmvMaxXM, sbl, G1, 2);
  const size_t lds2 = 8 * gather_group_lds<BITS, GS, C::GPL>(1, 1, false, (int)(N1 / GS), 1);
  const size_t lds = lds1 > lds2 ? lds1 : lds2;
  // kernel per (tile configuration, routing, shared expert): index 3 cfg + mode
  const int cfg = nwt == 4 ? 0 : nwt == 2 ? 1 : 2;
  const int mode = !route ? 0 : sh ? 1 : 2;
#define MQ_BN_KERN(NWT, SB, RT, SH) reinterpret_cast<const void*>(&moe_blockn_kernel<DT, BITS, GS, NWT, SB, RT, SH>)
  const void* kerns[3][3] = {
      {MQ_BN_KERN(4, false, false, false), MQ_BN_KERN(4, false, true, true),
       MQ_BN_KERN(4, false, true, false)},
      {MQ_BN_KERN(2, true, false, false), MQ_BN_KERN(2, true, true, true),
       MQ_BN_KERN(2, true, true, false)},
      {MQ_BN_KERN(1, true, false, false), MQ_BN_KERN(1, true, true, true),
       MQ_BN_KERN(1, true, true, false)}};
#undef MQ_BN_KERN
  const void* kern = kerns[cfg][mode];
  // every workgroup resident at once; the occupancy query kept per kernel
  // and LDS size
  static std::atomic<uint64_t> occ[3][3];
  const uint64_t key = (uint64_t)lds << 32;
  uint64_t got = occ[cfg][mode].load(std::memory_order_relaxed);
  if ((got & ~0xffffffffull) != key || got == 0) {
    static std::atomic<uint64_t> lds_set[3][3];
    if (lds > 64 * 1024)
      if (hipError_t e = ensure_lds_limit(kern, (int)lds, lds_set[cfg][mode]))
        return (int)e;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, 512, lds) != hipSuccess)
      return kStatusUnsupported;
    got = key | (uint32_t)(per_cu + 1);
    occ[cfg][mode].store(got, std::memory_order_relaxed);
  }
  if (((int64_t)(got & 0xffffffffull) - 1) * device_cu_count() < G) return kStatusUnsupported;
#define MQ_BN(NWT, SB, RT, SH)                                                                   \
  hipLaunchKernelGGL((moe_blockn_kernel<DT, BITS, GS, NWT, SB, RT, SH>), dim3((unsigned)G),      \
                     dim3(512), lds, st, (const uint16_t*)x, wg, (const uint16_t*)sg,            \
                     (const uint16_t*)bg, wu, (const uint16_t*)su, (const uint16_t*)bu, wd,      \
                     (const uint16_t*)sd, (const uint16_t*)bd, (const uint16_t*)shared,          \
                     (uint16_t*)h, (uint16_t*)out, (int)T, (int)N1, (int)K1, (int)N2, (int)E,    \
                     (int)n2, (int)tgn, ra)
#define MQ_BN_MODES(NWT, SB)                  \
  if (mode == 0) MQ_BN(NWT, SB, false, false); \
  else if (mode == 1) MQ_BN(NWT, SB, true, true); \
  else MQ_BN(NWT, SB, true, false);
  if (cfg == 0) {
    MQ_BN_MODES(4, false)
  } else if (cfg == 1) {
    MQ_BN_MODES(2, true)
  } else {
    MQ_BN_MODES(1, true)
  }
#undef MQ_BN_MODES
#undef MQ_BN
  return 0;
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
                                      int64_t T, int64_t N1, int64_t K1, int64_t N2, int64_t E,
                                      const RouteArgs& ra, hipStream_t st, int* nlaunch) {
  using C = QmvConf<BITS, GS>;
  constexpr int NW = 8;
  const int64_t top_k = ra.top_k;
  if (T != 1) {
    if (int rc = launch_blockn<DT, BITS, GS>(x, wg, sg, bg, wu, su, bu, wd, sd, bd, shared, h, out,
                                             T, N1, K1, N2, E, ra, st))
      return rc;
    *nlaunch += 1;
    return 0;
  }
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
