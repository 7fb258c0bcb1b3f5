// gather_qmm for MoE experts at decode / verify widths:
//   out[p, M, N] = x[lhs[p], M, K] . deq(W[rhs[p]])^T      (M <= 16 rows per pair)
//
// Reference behaviour: mx.gather_qmm as called by mlx-lm's
// QuantizedSwitchLinear (fused.py:2389-2394, 3105-3116) and the reference's
// decode kernels (moe_decode_fused.py:331-397: one threadgroup per
// (pair, column block), weights re-read per pair) and verify kernels
// (moe_verify_gather.py:213-322: one threadgroup per run of equal sorted
// experts).
//
// CDNA4 design: pairs that use the same expert become the rows of the MFMA
// A operand.  A "segment" is up to R pairs sharing one expert (R * M <= 16 A
// rows, fewer when their x rows would not fit in LDS); each workgroup owns
// (segment, 16-row weight tile) and runs the streaming tile of qmv.cuh over
// that expert's rows, so every expert's weights stream from HBM once per call
// no matter how many tokens routed to it, and dequantization work scales with
// distinct experts, not with pairs.
//
// Segment discovery needs no host sync and no extra launch for P <= 256:
// every workgroup ranks the pairs itself in LDS (pair p leads a segment when
// the number of earlier pairs with its expert is a multiple of R; segments
// are numbered by leader position).  Larger P (prefill-sized batches) runs a
// one-workgroup counting-sort prep kernel into the caller's workspace first.
// Pairs with an out-of-range expert or x index produce zero rows.
#pragma once
#include "launch.h"
#include "grouped.cuh"
#include "qmm_wide.cuh"
#include "qmv.cuh"
#include "route.cuh"

namespace mq {

// A rows of a gather segment: pair members[j] contributes rows j*Mi .. j*Mi+Mi-1.
struct GatherRows {
  static constexpr bool kCombine = false;
  const uint16_t* x;
  uint32_t x_nrec;
  uint16_t* out;
  const int* members;      // LDS
  const int* xbase;        // LDS: x batch index of each member
  int Mi, K, N, n0;
  __device__ __forceinline__ int64_t xoff(int m) const {
    const int j = m / Mi;
    return ((int64_t)xbase[j] * Mi + (m - j * Mi)) * K;
  }
  __device__ __forceinline__ void store(int m, int nn, uint16_t v) const {
    const int j = m / Mi;
    out[((int64_t)members[j] * Mi + (m - j * Mi)) * N + n0 + nn] = v;
  }
};

// Fused gate+up+SiLU (the reference's moe_glu.py:30-105 and
// moe_decode_fused.py:135-223): the call's two tiles are the same rows of
// the gate and the up bank; the epilogue stores silu(g) * u =
// g / (1 + exp(-g)) * u from the float sums, rounded once.
template <int DT>
struct GluRows : GatherRows {
  static constexpr bool kCombine = true;
  __device__ __forceinline__ void store_combined(int m, int nn, const float (&v)[2]) const {
    const float g = v[0], u = v[1];
    store(m, nn, T16<DT>::round1(g / (1.0f + __expf(-g)) * u));
  }
};

// Dynamic LDS of one wave group of the gather kernel (see below).
template <int BITS, int GS, int GPL>
__host__ __device__ inline size_t gather_group_lds(int NWT, int XM, bool sbl, int G, int TJ) {
  return qmv_x_lds<BITS, GS, GPL>(NWT, XM) + (sbl ? TJ * qmv_sb_lds(G) : 0);
}

// 1-D grid, block 64 * NW.  Column slot = 16 * NW / NWT rows of N; once the
// workgroup knows the number of segments it takes tpw = 1, 2, 4 or 8 slots
// (doubled while more than wg_target workgroups would be busy; tpw divides
// the slots of a segment) and workgroup i serves slots [i tpw, i tpw + tpw)
// of the concatenated segments' slots; workgroups past the end return.
// Consecutive workgroups are the slots of one segment, so idle workgroups
// form a contiguous tail instead of holes spread over the CUs: workgroups
// are placed on CUs in launch order, and with segments fastest the busy
// ones of every slot landed on the same CUs (config-4 banks, zipf, 64
// pairs: gate/up 22.4 -> 17.6 us, down 18.5 -> 13.8 us).
// Segment = up to R pairs that share an expert (R * Mi <= 16 A rows); pairs
// whose expert or x index is out of range form their own segments and get
// zero outputs.  The workgroup's NW waves form NW / NWT groups of NWT waves;
// in each of tpw rounds every group computes its own 16-row tile of the
// expert (NWT = 1 when K is a single step, so short-K experts do not leave
// three of four waves idle).  Dynamic LDS: NW / NWT x gather_group_lds.
// XM > 0: x streams through LDS, R * Mi <= XM and B * Mi * K * 2 < 2^31; a
// segment of one pair with Mi == 1 runs the one-row variant of the tile.
// SBL: tile scales/biases are copied to LDS (qmv_sb_fits holds).
// GLU: (w, scales, biases) is the gate bank and (w2, scales2, biases2) the up
// bank of the same shape; out = silu(gate) * up (GluRows: the gate and up
// tiles of a row block run as the two tiles of one qmv_tile call).
// ROUTE (P <= 64, no lhs, B = P / top_k tokens): the pairs' experts are not
// read from rhs but routed here from the tokens' float logits (ra.logits
// [B, E], E <= 512) with the routing kernel's wave pieces (route.cuh), every
// wave alike; workgroup 0 also writes the routing (ra.idx, ra.w) and, with
// ra.sgw, the shared expert's gate (ra.sgate) for the down projection.
template <int DT, int BITS, int GS, int GPL, int NW, int NWT, int PF, int XM, bool SBL, bool GLU,
          bool ROUTE = false>
__global__ __launch_bounds__(64 * NW) void gather_qmv_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ w,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    const uint32_t* __restrict__ w2, const uint16_t* __restrict__ scales2,
    const uint16_t* __restrict__ biases2, const int32_t* __restrict__ lhs,
    const int32_t* __restrict__ rhs, uint16_t* __restrict__ out, const int32_t* __restrict__ ws,
    int P, int B, int Mi, int N, int K, int E, int R, int wg_target, RouteArgs ra) {
  extern __shared__ __align__(16) unsigned char qmv_smem[];
  constexpr int TJ = GLU ? 2 : 1;
  __shared__ f32x4 red[NW * TJ][64];
  __shared__ int s_key[kGatherFusedMaxP];
  __shared__ int s_cb[kGatherFusedMaxP];
  __shared__ int s_members[16];
  __shared__ int s_xbase[16];
  __shared__ int s_expert;
  __shared__ int s_found;
  __shared__ int s_nseg;
  const int t = threadIdx.x;
  const int nt = blockDim.x;
  constexpr int NG = NW / NWT;                 // tile groups per workgroup
  const int nsl = (N + 16 * NG - 1) / (16 * NG);  // column slots of a segment
  // Once the number of segments is known: tile rounds per workgroup (tpw),
  // doubled while more than wg_target workgroups would be busy, and this
  // workgroup's segment and first column slot (false: nothing to do).
  int tpw = 1, seg = 0, slot = 0;
  auto place = [&](int nseg) {
    while (tpw < 8 && nsl % (2 * tpw) == 0 && nseg * (nsl / tpw) > wg_target) tpw *= 2;
    const int64_t item = (int64_t)blockIdx.x * tpw;
    if (item >= (int64_t)nseg * nsl) return false;
    seg = (int)(item / nsl);
    slot = (int)(item - (int64_t)seg * nsl);
    return true;
  };
  // key of a pair: its expert, or E when the expert or the x index is invalid
  auto key_of = [&](int p) {
    const int e = rhs[p];
    const int xb = x_batch(lhs, p, P, B);
    return (e >= 0 && e < E && xb >= 0 && xb < B) ? e : E;
  };

  if (ws == nullptr && P <= 64) {
    // Wave-level discovery (every wave computes the same answer; no barrier):
    // lane p holds pair p's key and cb = number of earlier pairs with that key.
    const int lane = t & 63;
    int key = -1;
    if constexpr (ROUTE) {
      // token tok routed by wave tok % NW (pair p = tok * top_k + rank r
      // takes lane r's expert), the pairs' experts met in LDS; in
      // workgroup 0 the routing wave also writes the token's routing, and
      // wave (tok + NW / 2) % NW the token's shared gate, so that with few
      // tokens the gate's loads and dot run beside the top-k instead of
      // after it (the rest of the grid waits for workgroup 0's last wave)
      const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
      const bool writer = blockIdx.x == 0;
      if (writer && ra.sgw != nullptr) {
        for (int tok = (wv + NW / 2) % NW; tok < B; tok += NW) {
          const uint16_t g = route_wave_shared_gate<DT>(x + (int64_t)tok * K, ra.sgw, K, lane);
          if (lane == 0) ra.sgate[tok] = g;
        }
      }
      if (B == 1) {
        // one token: its top_k experts are distinct, so pair r is segment r
        // (one member), and the routing wave places the workgroup's segment
        // itself: one barrier where the general path takes two (T=1,
        // config-4 banks: discovery 0.8 of a 10.3 us launch)
        if (!place(ra.top_k)) return;                // identical in every wave
        if (wv == 0) {
          int sel_e;
          float sel_v;
          route_wave_topk<8>(ra.logits, E, ra.top_k, lane, sel_e, sel_v);
          if (writer) {
            const float wgt = route_wave_softmax(sel_v, lane, ra.top_k);
            if (lane < ra.top_k) {
              ra.idx[lane] = sel_e;
              ra.w[lane] = wgt;
            }
          }
          const int es = __builtin_amdgcn_readlane(sel_e, seg);
          if (lane < 16) {
            s_members[lane] = lane == 0 ? seg : -1;
            s_xbase[lane] = 0;
          }
          if (lane == 0) s_expert = es >= 0 ? es : E;  // a round with no expert: zeros
        }
        __syncthreads();
      } else {
        for (int tok = wv; tok < B; tok += NW) {
          int sel_e;
          float sel_v;
          route_wave_topk<8>(ra.logits + (int64_t)tok * E, E, ra.top_k, lane, sel_e, sel_v);
          if (lane < ra.top_k) s_key[tok * ra.top_k + lane] = sel_e >= 0 ? sel_e : E;
          if (writer) {
            const float wgt = route_wave_softmax(sel_v, lane, ra.top_k);
            if (lane < ra.top_k) {
              ra.idx[tok * ra.top_k + lane] = sel_e;
              ra.w[tok * ra.top_k + lane] = wgt;
            }
          }
        }
        __syncthreads();
        key = lane < P ? s_key[lane] : -1;
      }
    } else {
      key = lane < P ? key_of(lane) : -1;
    }
    if (!ROUTE || B != 1) {
      int cb = 0;
      for (int q = 0; q < P; ++q) {
        const int kq = __builtin_amdgcn_readlane(key, q);
        cb += (q < lane && kq == key) ? 1 : 0;
      }
      const bool lead = lane < P && (cb % R) == 0;
      const uint64_t lmask = __builtin_amdgcn_ballot_w64(lead);
      if (!place(__builtin_popcountll(lmask))) return;  // identical in every wave
      const int rank = __builtin_popcountll(lmask & ((1ull << lane) - 1ull));
      const uint64_t mine = __builtin_amdgcn_ballot_w64(lead && rank == seg);
      const int leader = __builtin_ctzll(mine);
      const int e = __builtin_amdgcn_readlane(key, leader);
      const int cb0 = __builtin_amdgcn_readlane(cb, leader);
      const int d = cb - cb0;
      if (t < 16) s_members[t] = -1;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      if (lane < P && key == e && d >= 0 && d < R) {
        s_members[d] = lane;
        s_xbase[d] = ROUTE ? lane / ra.top_k : x_batch(lhs, lane, P, B);
      }
      if (t == 0) s_expert = e;
      __syncthreads();
    }
  } else if (ws == nullptr) {
    if (t < 16) s_members[t] = -1;
    if (t == 0) {
      s_found = 0;
      s_nseg = 0;
    }
    // In-workgroup segment discovery (P <= kGatherFusedMaxP): pair p leads a
    // segment when the number of earlier pairs with its key is a multiple of
    // R; segments are numbered by leader position.
    for (int p = t; p < P; p += nt) s_key[p] = key_of(p);
    __syncthreads();
    for (int p = t; p < P; p += nt) {
      const int e = s_key[p];
      int cb = 0;
      for (int q = 0; q < p; ++q) cb += (s_key[q] == e);
      s_cb[p] = cb;
      if (cb % R == 0) atomicAdd(&s_nseg, 1);
    }
    __syncthreads();
    if (!place(s_nseg)) return;                       // uniform in the workgroup
    for (int p = t; p < P; p += nt) {
      if (s_cb[p] % R) continue;
      int rank = 0;
      for (int q = 0; q < p; ++q) rank += (s_cb[q] % R == 0);
      if (rank == seg) {
        s_expert = s_key[p];
        s_found = 1;
        s_members[0] = p;
      }
    }
    __syncthreads();
    if (!s_found) return;
    const int lead = s_members[0];
    const int e = s_expert;
    const int cb0 = s_cb[lead];
    for (int q = lead + 1 + t; q < P; q += nt) {
      const int d = s_cb[q] - cb0;
      if (s_key[q] == e && d > 0 && d < R) s_members[d] = q;
    }
    __syncthreads();
  } else {
    if (!place(ws[0])) return;
    const int32_t* perm = ws + 1;
    const int32_t* seg_start = perm + P;
    const int32_t* seg_len = seg_start + P;
    const int32_t* seg_exp = seg_len + P;
    const int st0 = seg_start[seg];
    const int ln = seg_len[seg];
    if (t < 16) s_members[t] = t < ln ? perm[st0 + t] : -1;
    if (t == 0) s_expert = seg_exp[seg];
    __syncthreads();
  }
  int nmem = 0;
#pragma unroll 1
  for (int j = 0; j < 16; ++j) nmem += (s_members[j] >= 0);
  if (!(ws == nullptr && P <= 64)) {
    if (t < 16) {
      const int p = s_members[t];
      s_xbase[t] = p >= 0 ? x_batch(lhs, p, P, B) : 0;
    }
    __syncthreads();
  }
  const int e = __builtin_amdgcn_readfirstlane(s_expert);
  const int M = nmem * Mi;
  const int nb = slot * 16 * NG;
  if (e >= E) {
    // invalid pairs: zero rows
    const int cols = min(16 * NG * tpw, N - nb);
    for (int i = t; i < M * cols; i += nt) {
      const int m = i / cols, nn = i - m * cols;
      const int j = m / Mi;
      out[((int64_t)s_members[j] * Mi + (m - j * Mi)) * N + nb + nn] = 0;
    }
    return;
  }
  const uint32_t rowB = (uint32_t)K * BITS / 8;
  const uint32_t sRowB = (uint32_t)(K / GS) * 2;
  const uint32_t x_nrec = XM > 0 ? (uint32_t)((int64_t)B * Mi * K * 2) : 0u;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int g = wave / NWT, kw = wave - g * NWT;
  unsigned char* gsm = qmv_smem + g * gather_group_lds<BITS, GS, GPL>(NWT, XM, SBL, K / GS, TJ);
  for (int tt = 0; tt < tpw; ++tt) {
    const int n00 = nb + 16 * NG * tt;
    if (n00 >= N) break;                       // uniform in the workgroup
    // a group past N runs an empty tile (rows <= 0) to keep the barriers
    const int n0 = n00 + 16 * g;
    const int rows = min(16, N - n0);
    const int64_t row0 = (int64_t)e * N + (rows > 0 ? n0 : 0);
    const GatherRows src{x, x_nrec, out, s_members, s_xbase, Mi, K, N, n0};
    QmvTiles<TJ> tl;
    tl.w[0] = reinterpret_cast<const char*>(w) + row0 * rowB;
    tl.s[0] = reinterpret_cast<const char*>(scales) + row0 * sRowB;
    tl.b[0] = reinterpret_cast<const char*>(biases) + row0 * sRowB;
    tl.rows[0] = rows;
    if constexpr (GLU) {
      tl.w[1] = reinterpret_cast<const char*>(w2) + row0 * rowB;
      tl.s[1] = reinterpret_cast<const char*>(scales2) + row0 * sRowB;
      tl.b[1] = reinterpret_cast<const char*>(biases2) + row0 * sRowB;
      tl.rows[1] = rows;
    }
    // the one-row variant uses a prefix of the group's x region; its scale
    // copy lands inside the group's region too
    auto tile = [&](const auto& rs) {
      if (XM > 1 && M == 1)
        qmv_tile<DT, BITS, GS, GPL, NWT, PF, (XM > 1 ? 1 : XM), SBL, TJ>(
            tl, M, K, rs, gsm, red + g * NWT * TJ, kw, t - 64 * NWT * g);
      else
        qmv_tile<DT, BITS, GS, GPL, NWT, PF, XM, SBL, TJ>(tl, M, K, rs, gsm, red + g * NWT * TJ,
                                                          kw, t - 64 * NWT * g);
    };
    if constexpr (GLU) tile(GluRows<DT>{src});
    else tile(src);
  }
}

// ---- down projection with the MoE combine folded in (decode widths) -------
// out[t, n] = T( sum_k w[t*top_k + k] * y[t*top_k + k, n] ) with
// y[p] = T(x[p] . deq(W[rhs[p]])^T): mq_gather_qmm (one x row per pair)
// followed by mq_moe_combine (inv = NULL), in one launch and bit for bit the
// same, since every y is computed by the same tile code with the same K
// split (gather_tile_waves) and the same segments, rounded to T, and summed
// in k order with fma as the combine kernel does.  Optionally the shared
// expert is merged as mq_moe_combine_shared does.
//
// Each workgroup owns 16 output columns for every token, so no sum crosses
// workgroups (a cross-workgroup fold needs a device-scope release per
// workgroup, which on MI355X writes back the XCD's L2 and cost more than the
// launch it saves).  Its kFoldNW / NWT wave groups take the segments of the
// call (pairs sharing an expert, up to 8) in rounds; each tile's y values go
// to LDS, and after the last round the workgroup sums them per token.  With
// only N / 16 workgroups, each round is a serial memory round trip: the
// launcher takes calls of at most two rounds (config-4 down bank, zipf
// routing, whole decode layer: T=1 15.3 us folded against 18.0 with the two
// kernels; at T=4 / 8, three or more rounds, 31.4 / 48.4 against 28.5 /
// 39.1, so those run the two kernels).
constexpr int kFoldNW = 8;

// A rows of a folded segment (one x row per pair): outputs go to the
// workgroup's LDS copy of y, row = pair.
struct FoldRows {
  static constexpr bool kCombine = false;
  const uint16_t* x;
  uint32_t x_nrec;
  uint16_t (*ys)[16];
  const int* members;      // LDS
  int K;
  __device__ __forceinline__ int64_t xoff(int m) const { return (int64_t)members[m] * K; }
  __device__ __forceinline__ void store(int m, int nn, uint16_t v) const { ys[members[m]][nn] = v; }
};

template <int DT, int BITS, int GS, int GPL, int NWT, int PF, bool SBL, bool SH>
__global__ __launch_bounds__(64 * kFoldNW) void gather_fold_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ w,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    const int32_t* __restrict__ rhs, const float* __restrict__ cw,
    const uint16_t* __restrict__ sgate, const uint16_t* __restrict__ shared,
    uint16_t* __restrict__ out, int P, int top_k, int N, int K, int E, int R) {
  extern __shared__ __align__(16) unsigned char qmv_smem[];
  constexpr int NW = kFoldNW, NG = NW / NWT, XM = kQmvMaxXM;
  using T = T16<DT>;
  __shared__ f32x4 red[NW][64];
  __shared__ uint16_t s_y[kFoldMaxP][16];
  __shared__ uint16_t s_sh[SH ? kFoldMaxP : 1][16];
  __shared__ float s_w[kFoldMaxP];
  __shared__ uint16_t s_sg[SH ? kFoldMaxP : 1];
  __shared__ int s_members[NG][16];
  const int t = threadIdx.x, lane = t & 63;
  const int n0 = blockIdx.x * 16;
  const int rows = min(16, N - n0);
  const int ntok = P / top_k;
  // router weights and the shared expert's columns load with the indices
  if (t < P) s_w[t] = cw[t];
  if constexpr (SH) {
    for (int i = t; i < ntok * 16; i += 64 * NW) {
      const int tok = i >> 4, nn = i & 15;
      s_sh[tok][nn] = nn < rows ? shared[(int64_t)tok * N + n0 + nn] : (uint16_t)0;
    }
    if (t < ntok) s_sg[t] = sgate[t];
  }
  // every wave ranks the pairs itself (as the gather kernel does for P <= 64):
  // lane p holds pair p's key (its expert, E when out of range) and cb = the
  // number of earlier pairs with that key; pair p leads a segment when cb is
  // a multiple of R, and segments are numbered by leader position
  const int key = lane < P ? ((unsigned)rhs[lane] < (unsigned)E ? rhs[lane] : E) : -1;
  int cb = 0;
  for (int q = 0; q < P; ++q) {
    const int kq = __builtin_amdgcn_readlane(key, q);
    cb += (q < lane && kq == key) ? 1 : 0;
  }
  const bool lead = lane < P && (cb % R) == 0;
  const uint64_t lmask = __builtin_amdgcn_ballot_w64(lead);
  const int nseg = __builtin_popcountll(lmask);
  const int rank = __builtin_popcountll(lmask & ((1ull << lane) - 1ull));
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int g = wave / NWT, kw = wave - g * NWT;
  unsigned char* gsm = qmv_smem + g * gather_group_lds<BITS, GS, GPL>(NWT, XM, SBL, K / GS, 1);
  const uint32_t rowB = (uint32_t)K * BITS / 8;
  const uint32_t sRowB = (uint32_t)(K / GS) * 2;
  const uint32_t x_nrec = (uint32_t)((int64_t)P * K * 2);
  const int rounds = (nseg + NG - 1) / NG;
  for (int rd = 0; rd < rounds; ++rd) {
    const int seg = rd * NG + g;                 // wave-uniform
    int e = E, nmem = 1;
    if (seg < nseg) {
      const uint64_t mine = __builtin_amdgcn_ballot_w64(lead && rank == seg);
      const int leader = __builtin_ctzll(mine);
      e = __builtin_amdgcn_readlane(key, leader);
      const int d = cb - __builtin_amdgcn_readlane(cb, leader);
      const bool mem = lane < P && key == e && d >= 0 && d < R;
      nmem = __builtin_popcountll(__builtin_amdgcn_ballot_w64(mem));
      if (kw == 0 && mem) {
        s_members[g][d] = lane;
        if (e >= E) {                            // invalid pairs: y = 0
          *reinterpret_cast<u32x4*>(&s_y[lane][0]) = (u32x4){0u, 0u, 0u, 0u};
          *reinterpret_cast<u32x4*>(&s_y[lane][8]) = (u32x4){0u, 0u, 0u, 0u};
        }
      }
    } else if (kw == 0 && lane == 0) {
      s_members[g][0] = 0;                       // empty tile: a valid x row
    }
    __syncthreads();
    const bool live = seg < nseg && e < E && rows > 0;
    const int64_t row0 = (int64_t)(live ? e : 0) * N + (live ? n0 : 0);
    QmvTiles<1> tl;
    tl.w[0] = reinterpret_cast<const char*>(w) + row0 * rowB;
    tl.s[0] = reinterpret_cast<const char*>(scales) + row0 * sRowB;
    tl.b[0] = reinterpret_cast<const char*>(biases) + row0 * sRowB;
    tl.rows[0] = live ? rows : 0;
    const FoldRows src{x, x_nrec, s_y, s_members[g], K};
    const int M = live ? nmem : 1;
    if (M == 1)
      qmv_tile<DT, BITS, GS, GPL, NWT, PF, 1, SBL, 1>(tl, M, K, src, gsm, red + g * NWT, kw,
                                                     t - 64 * NWT * g);
    else
      qmv_tile<DT, BITS, GS, GPL, NWT, PF, XM, SBL, 1>(tl, M, K, src, gsm, red + g * NWT, kw,
                                                      t - 64 * NWT * g);
    __syncthreads();                             // s_members is rewritten next round
  }
  // the combine: per token, the router-weighted sum over its top_k pairs in
  // k order, rounded once (then the shared expert's term, rounded, added)
  for (int i = t; i < ntok * 16; i += 64 * NW) {
    const int tok = i >> 4, nn = i & 15;
    if (nn >= rows) continue;
    float acc = 0.f;
    for (int k = 0; k < top_k; ++k) {
      const int p = tok * top_k + k;
      acc = __builtin_fmaf(s_w[p], T::to_f32(s_y[p][nn]), acc);
    }
    uint16_t o = T::round1(acc);
    if constexpr (SH) {
      // no contraction: for fp16 the compiler narrows the product and the sum
      // to half operations (exact) and would then fuse them into one fma_f16,
      // skipping the product's rounding
#pragma clang fp contract(off)
      const uint16_t m = T::round1(T::to_f32(s_sg[tok]) * T::to_f32(s_sh[tok][nn]));
      o = T::round1(T::to_f32(o) + T::to_f32(m));
    }
    out[(int64_t)tok * N + n0 + nn] = o;
  }
}

// One launch of the expert-grouped wide tile (BM rows) over the prep
// tables' size class cls, whose segments number at most seg_bound.
template <int DT, int BITS, int GS, int BM>
inline int launch_grouped_class(const void* x, const uint32_t* w, const void* s, const void* b,
                                const int32_t* lhs, void* out, int64_t P, int64_t B, int64_t M,
                                int64_t N, int64_t K, int64_t E, void* ws, int cls,
                                int64_t seg_bound, hipStream_t st, int* nlaunch) {
  static std::atomic<uint64_t> lds_set{0};
  if (hipError_t e = ensure_lds_limit(
          reinterpret_cast<const void*>(&qmm_grouped_kernel<DT, BITS, GS, BM>),
          (int)wide_lds_bytes<BM>(), lds_set))
    return (int)e;
  const int64_t ntiles = (N + kWideBN - 1) / kWideBN * seg_bound;
  const dim3 grid((unsigned)((ntiles + 7) / 8 * 8));
  hipLaunchKernelGGL((qmm_grouped_kernel<DT, BITS, GS, BM>), grid, dim3(kWideNT),
                     wide_lds_bytes<BM>(), st, (const uint16_t*)x, w, (const uint16_t*)s,
                     (const uint16_t*)b, lhs, (uint16_t*)out, (const int32_t*)ws, (int)P, (int)B,
                     (int)M, (int)N, (int)K, (int)E, cls);
  *nlaunch += 1;
  return 0;
}

// Segments of the pairs of a size class when experts with at least C pairs
// are cut into segments of R pairs: at most P / R + P / C (one partial
// segment per expert of the class) and never more than P.
inline int64_t class_seg_bound(int64_t P, int64_t R, int64_t C, int64_t E) {
  int64_t b = (P + R - 1) / R + (C > 0 ? P / C : E + 1);
  if (b > E + 1 + (P + R - 1) / R) b = E + 1 + (P + R - 1) / R;
  return b < P ? b : P;
}

// Prefill gather_qmm: prep tables, then the expert-grouped MFMA tile kernel.
// One row-tile height for every expert (BM rows) when the expected rows per
// expert call for it, or size classes: experts with 192+ rows get 256-row
// tiles, 96+ rows 128-row tiles, the rest 64-row tiles, one launch per class
// (zipf routing puts half the rows of config 4 in 27 experts).
template <int DT, int BITS, int GS, int BM>
inline int launch_grouped_bm(const void* x, const uint32_t* w, const void* s, const void* b,
                             const int32_t* lhs, const int32_t* rhs, void* out, int64_t P,
                             int64_t B, int64_t M, int64_t N, int64_t K, int64_t E, void* ws,
                             hipStream_t st, int* nlaunch, bool classes) {
  const int R = (int)(BM / M);
  const int64_t ncol = (N + kWideBN - 1) / kWideBN;
  if (ncol * (P + E + 1) > INT32_MAX - 8) return kStatusUnsupported;
  if (!classes || M > 64) {
    if (int rc = launch_prep(rhs, lhs, P, E, B, R, ws, st)) return rc;
    *nlaunch += kPrepLaunches;
    return launch_grouped_class<DT, BITS, GS, BM>(x, w, s, b, lhs, out, P, B, M, N, K, E, ws, 0,
                                                  class_seg_bound(P, R, 0, E), st, nlaunch);
  }
  // classes (BM is the small tile, 64 rows): 128-row tiles from 96 rows per
  // expert, 256-row tiles from 192, all in one launch
  const int R1 = (int)(128 / M), C1 = (int)((96 + M - 1) / M);
  const int R2 = (int)(256 / M), C2 = (int)((192 + M - 1) / M);
  if (int rc = launch_prep(rhs, lhs, P, E, B, R, ws, st, R1, C1, R2, C2)) return rc;
  static std::atomic<uint64_t> lds_set{0};
  if (hipError_t e = ensure_lds_limit(
          reinterpret_cast<const void*>(&qmm_grouped_classes_kernel<DT, BITS, GS>),
          (int)wide_lds_bytes<256>(), lds_set))
    return (int)e;
  int64_t nwg = 0;
  for (const int64_t b : {class_seg_bound(P, R2, C2, E), class_seg_bound(P, R1, C1, E),
                          class_seg_bound(P, R, 0, E)})
    nwg += (b * ncol + 7) / 8 * 8;
  if (nwg > INT32_MAX) return kStatusUnsupported;
  hipLaunchKernelGGL((qmm_grouped_classes_kernel<DT, BITS, GS>), dim3((unsigned)nwg),
                     dim3(kWideNT), wide_lds_bytes<256>(), st, (const uint16_t*)x, w,
                     (const uint16_t*)s, (const uint16_t*)b, lhs, (uint16_t*)out,
                     (const int32_t*)ws, (int)P, (int)B, (int)M, (int)N, (int)K, (int)E);
  *nlaunch += kPrepLaunches + 1;
  return 0;
}

// The thin grouped kernel (grouped.cuh) over two-class tables already built
// in ws (launch_thin_tables: segments of R = 64 / M pairs, and of 2 R for
// experts with more than R pairs).  GLU: gate bank (w, s, b) and up bank
// (w2, s2, b2), out = SwiGLU of the two gathers (N columns).
template <int DT, int BITS, int GS, bool GLU>
inline int launch_thin_kernel(const void* x, const uint32_t* w, const void* s, const void* b,
                              const uint32_t* w2, const void* s2, const void* b2,
                              const int32_t* lhs, void* out, int64_t P, int64_t B, int64_t M,
                              int64_t N, int64_t K, int64_t E, const void* ws, hipStream_t st) {
  const int R = (int)(kThinBM / M);
  // 4 waves (256 columns) per workgroup for 4-bit weights and at short K, 8
  // (512 columns, so each x tile serves twice the columns) for 8-bit weights
  // above K = 1024.  Config-4 banks, 2048 tokens x top-8, one process: down
  // (K=512) 143 / 122 us zipf / uniform with 4 against 173 / 141 with 8.
  // Gate/up (K=2048): 4-bit 4-wave tiles stream their weights through LDS
  // (the DMA form in grouped.cuh) and take 275 / 241 us against 285 / 261
  // with 8 waves; the fused SwiGLU layer 425 against 447 us zipf.  Without
  // that stream (8-bit) 8 waves won: 279 / 222 against 302 / 253 for the
  // size-class wide tiles and 282 / 264 with 16 waves (whose 128-register
  // budget spills).
  const int nwv = (K <= 1024 || BITS == 4) ? 4 : 8;
  const int64_t bn = (GLU ? 32 : 64) * nwv;     // output columns per tile
  const int64_t ncol = (N + bn - 1) / bn;
  // 8 waves: experts with more than 64 rows take 128-row tiles, which read
  // their weights once per 128 rows (the workgroup's register budget
  // already holds one workgroup per CU, so the taller tile costs no
  // occupancy).  4 waves run those segments as two 64-row tiles (128-row
  // tiles with 4 waves: config-4 down 261 against 176 us zipf), the same
  // work as one-class tables, so one table build serves both widths.
  const int64_t h1 = nwv == 4 ? 2 : 1;
  int64_t nwg = 0;
  for (const int64_t sb : {h1 * class_seg_bound(P, 2 * R, R + 1, E), class_seg_bound(P, R, 0, E)})
    nwg += (sb * ncol + 7) / 8 * 8;
  if (nwg > INT32_MAX) return kStatusUnsupported;
  const dim3 grid((unsigned)nwg);
#define MQ_THIN(NWV, HALVES)                                                                    \
  hipLaunchKernelGGL((qmm_grouped_thin_kernel<DT, BITS, GS, 2, NWV, true, HALVES, GLU>), grid,  \
                     dim3(64 * NWV), 0, st, (const uint16_t*)x, w, (const uint16_t*)s,           \
                     (const uint16_t*)b, w2, (const uint16_t*)s2, (const uint16_t*)b2, lhs,      \
                     (uint16_t*)out, (const int32_t*)ws, (int)P, (int)B, (int)M, (int)N, (int)K, \
                     (int)E, 0)
  if (nwv == 4) MQ_THIN(4, true);
  else MQ_THIN(8, false);
#undef MQ_THIN
  return 0;
}

// Prefill gather_qmm with thin experts: the register-B grouped kernel over
// two-class tables, built here unless the caller built them for this
// routing already (prepped).
template <int DT, int BITS, int GS>
inline int launch_grouped_thin(const void* x, const uint32_t* w, const void* s, const void* b,
                               const int32_t* lhs, const int32_t* rhs, void* out, int64_t P,
                               int64_t B, int64_t M, int64_t N, int64_t K, int64_t E, void* ws,
                               hipStream_t st, int* nlaunch, bool prepped) {
  if (!prepped) {
    if (int rc = launch_thin_tables(rhs, lhs, P, E, B, M, ws, st)) return rc;
    *nlaunch += kPrepLaunches;
  }
  if (int rc = launch_thin_kernel<DT, BITS, GS, false>(x, w, s, b, nullptr, nullptr, nullptr, lhs,
                                                       out, P, B, M, N, K, E, ws, st))
    return rc;
  *nlaunch += 1;
  return 0;
}

template <int DT, int BITS, int GS>
inline int launch_grouped(const void* x, const uint32_t* w, const void* s, const void* b,
                          const int32_t* lhs, const int32_t* rhs, void* out, int64_t P, int64_t B,
                          int64_t M, int64_t N, int64_t K, int64_t E, void* ws, hipStream_t st,
                          int* nlaunch, bool prepped) {
  if (gather_thin_path(P, M, K, E))
    return launch_grouped_thin<DT, BITS, GS>(x, w, s, b, lhs, rhs, out, P, B, M, N, K, E, ws, st,
                                             nlaunch, prepped);
  if (prepped) return kStatusUnsupported;      // the tables are the thin kernel's
  const int64_t active = P < E ? P : E;
  const int64_t rows_per_expert = P * M / (active > 0 ? active : 1);
  if (rows_per_expert >= 192)
    return launch_grouped_bm<DT, BITS, GS, 256>(x, w, s, b, lhs, rhs, out, P, B, M, N, K, E, ws,
                                                st, nlaunch, false);
  if (rows_per_expert >= 96)
    return launch_grouped_bm<DT, BITS, GS, 128>(x, w, s, b, lhs, rhs, out, P, B, M, N, K, E, ws,
                                                st, nlaunch, false);
  return launch_grouped_bm<DT, BITS, GS, 64>(x, w, s, b, lhs, rhs, out, P, B, M, N, K, E, ws, st,
                                             nlaunch, true);
}

// Waves per 16-row tile of the streaming gather kernel (its K split): 4 or 2
// only while the tiles are few (about 2048 waves in all) and each wave gets
// a step, and none for one or two steps.  Config-4 banks, zipf routing:
// gate/up T=1 6.9 us split 4 ways against 8.8 unsplit, T=8 22 unsplit
// against 30 split 4 ways; down T=4 10.0 unsplit against 12.2, T=1 (two
// steps) the same either way.  A tile's float sum depends on it, so the
// folded down projection below takes the same count.
// Whether a gather tile copies its scales and biases to LDS: not when each
// of its nwt waves runs at most two k-steps (decode gathers at T=1 and the
// down bank), where two per-step loads beat the copy's workgroup barrier
// (config-4 banks, one process: gate/up T=1 7.03 -> 6.85 us, down 6.14 ->
// 5.89, GLU 7.76 -> 7.42; with eight steps per wave, gate/up T=4, they lost
// 13.1 -> 13.8).
template <int BITS, int GS>
inline bool gather_tile_sb(int64_t K, int nwt) {
  using Gm = QmvGeom<BITS, GS, QmvConf<BITS, GS>::GPL>;
  const int64_t nsteps = (K / GS + Gm::STEPG - 1) / Gm::STEPG;
  return (nsteps + nwt - 1) / nwt > 2;
}

template <int BITS, int GS>
inline int gather_tile_waves(int64_t max_seg, int64_t N, int64_t K) {
  using Gm = QmvGeom<BITS, GS, QmvConf<BITS, GS>::GPL>;
  const int64_t nsteps = (K / GS + Gm::STEPG - 1) / Gm::STEPG;
  const int64_t tiles = max_seg * ((N + 15) / 16);
  if (nsteps <= 2) return 1;
  int nwt = 4;
  while (nwt > 1 && (nwt > nsteps || tiles * nwt > 2048)) nwt /= 2;
  return nwt;
}

// The streaming gather kernel over segments (GLU: fused gate+up+SiLU with the
// up bank in w2 / s2 / b2).
template <int DT, int BITS, int GS, bool GLU, bool ROUTE = false>
inline int gather_qmv_launch(const void* x, const uint32_t* w, const void* s, const void* b,
                             const uint32_t* w2, const void* s2, const void* b2,
                             const int32_t* lhs, const int32_t* rhs, void* out, int64_t P,
                             int64_t B, int64_t M, int64_t N, int64_t K, int64_t E, void* ws,
                             hipStream_t st, int* nlaunch, RouteArgs ra = RouteArgs{}) {
  using C = QmvConf<BITS, GS>;
  // Segments of up to R pairs; R * M <= 8 A rows stream x through LDS, one
  // pair of more than 8 rows reads x fragments from global memory.  A segment
  // holds at most one pair per x batch in the usual MoE call (each token
  // picks distinct experts), so R <= B wastes nothing; more pairs of one
  // expert simply form more segments.
  int R = M <= kQmvMaxXM ? (int)(kQmvMaxXM / M) : 1;
  if (R > B) R = (int)(B > 0 ? B : 1);
  const int XM = (B * M * K * 2 < ((int64_t)1 << 31)) ? qmv_xm_for(R * M) : 0;
  int64_t max_seg = P;
  if (P > kGatherFusedMaxP) {
    const int64_t bound = (P + R - 1) / R + E + 1;
    if (bound < max_seg) max_seg = bound;
  }
  const int nwt = gather_tile_waves<BITS, GS>(max_seg, N, K);
  const int ng = C::NW / nwt;
  constexpr int TJ = GLU ? 2 : 1;
  const bool sbl = gather_tile_sb<BITS, GS>(K, nwt) && qmv_sb_fits(K / GS, nwt, TJ, s, b) &&
                   (!GLU || qmv_sb_fits(K / GS, nwt, TJ, s2, b2));
  // without the scale copy only the 8-row streamed-x variant is built
  const int xml = (sbl || XM == 0) ? XM : kQmvMaxXM;
  auto lds_for = [&](int xmax, int wpt, bool with_sb) {
    return (size_t)(C::NW / wpt) *
           gather_group_lds<BITS, GS, C::GPL>(wpt, xmax, with_sb, (int)(K / GS), TJ);
  };
  const int32_t* wsp = nullptr;
  if (P > kGatherFusedMaxP) {
    if (int rc = launch_prep(rhs, lhs, P, E, B, R, ws, st)) return rc;
    wsp = (const int32_t*)ws;
    *nlaunch += kPrepLaunches;
  }
  // One workgroup per (segment bound, column slot); the kernel gives each
  // busy workgroup 1, 2, 4 or 8 slots in turn so that at most ~3 per CU are
  // busy, as it learns the number of distinct experts (config-4 banks, 64
  // pairs: the best count was 490-670 busy workgroups for zipf and uniform
  // routing alike: gate/up zipf 18.4 us with one slot each, uniform 22.8
  // with two; down zipf 14.5 with two, uniform 17.9 with four).
  // The grid covers the most workgroups any segment count can keep busy:
  // wg_target, or the bound's slots at the largest round count.  Launching
  // one workgroup per (bound, slot) instead cost the down bank 4 us (2048
  // workgroups, most of them exiting after discovery).
  const int64_t slots = (N + 16 * ng - 1) / (16 * ng);
  const int wg_target = 25 * device_cu_count() / 8;
  int tpw_cap = 1;
  while (tpw_cap < 8 && slots % (2 * tpw_cap) == 0) tpw_cap *= 2;
  int64_t nwg = max_seg * slots / tpw_cap;
  if (nwg < wg_target) nwg = wg_target;
  if (nwg > max_seg * slots) nwg = max_seg * slots;
  if (nwg > INT32_MAX) return kStatusUnsupported;
  const dim3 grid((unsigned)nwg);
#define MQ_GX(WPT, X, SB)                                                                    \
  if (nwt == WPT && xml == X && sbl == SB) {                                                  \
    hipLaunchKernelGGL((gather_qmv_kernel<DT, BITS, GS, C::GPL, C::NW, WPT, C::PF, X, SB, GLU, \
                                          ROUTE>),                                           \
                       grid, dim3(64 * C::NW), lds_for(X, WPT, SB), st, (const uint16_t*)x, w, \
                       (const uint16_t*)s, (const uint16_t*)b, w2, (const uint16_t*)s2,       \
                       (const uint16_t*)b2, lhs, rhs, (uint16_t*)out, wsp, (int)P, (int)B,    \
                       (int)M, (int)N, (int)K, (int)E, R, wg_target, ra);                    \
  }
#define MQ_GXW(WPT)                                                                          \
  MQ_GX(WPT, 0, true) MQ_GX(WPT, 1, true) MQ_GX(WPT, 2, true) MQ_GX(WPT, 4, true)            \
  MQ_GX(WPT, 8, true) MQ_GX(WPT, 0, false) MQ_GX(WPT, 8, false)
  MQ_GXW(1) MQ_GXW(2) MQ_GXW(4)
#undef MQ_GXW
#undef MQ_GX
  *nlaunch += 1;
  return 0;
}

template <int DT, int BITS, int GS>
int GatherLaunch<DT, BITS, GS>::run(const void* x, const uint32_t* w, const void* s,
                                    const void* b, const int32_t* lhs, const int32_t* rhs,
                                    void* out, int64_t P, int64_t B, int64_t M, int64_t N,
                                    int64_t K, int64_t E, void* ws, bool prepped, hipStream_t st,
                                    int* nlaunch) {
  if (P > kGatherFusedMaxP && E > kGatherPrepMaxE) return kStatusUnsupported;
  if ((N + 15) / 16 > 65535) return kStatusUnsupported;
  if (P * M >= kGroupedMinRows && E <= kGatherPrepMaxE && K % kWideBK == 0 &&
      B * M * K * 2 < ((int64_t)1 << 31) && 256 * K * 2 < ((int64_t)1 << 31))
    return launch_grouped<DT, BITS, GS>(x, w, s, b, lhs, rhs, out, P, B, M, N, K, E, ws, st,
                                        nlaunch, prepped);
  if (prepped) return kStatusUnsupported;
  return gather_qmv_launch<DT, BITS, GS, false>(x, w, s, b, nullptr, nullptr, nullptr, lhs, rhs,
                                                out, P, B, M, N, K, E, ws, st, nlaunch);
}

template <int DT, int BITS, int GS>
int GluRouteLaunch<DT, BITS, GS>::run(const void* x, const uint32_t* wg, const void* sg,
                                      const void* bg, const uint32_t* wu, const void* su,
                                      const void* bu, void* out, int64_t T, int64_t N, int64_t K,
                                      int64_t E, const RouteArgs& ra, hipStream_t st,
                                      int* nlaunch) {
  const int64_t P = T * ra.top_k;
  if (T < 1 || ra.top_k < 1 || ra.top_k > E || P > 64 || E > 64 * 8 || (N + 15) / 16 > 65535)
    return kStatusUnsupported;
  return gather_qmv_launch<DT, BITS, GS, true, true>(x, wg, sg, bg, wu, su, bu, nullptr, nullptr,
                                                     out, P, T, 1, N, K, E, nullptr, st, nlaunch,
                                                     ra);
}

template <int DT, int BITS, int GS>
int GluLaunch<DT, BITS, GS>::run(const void* x, const uint32_t* wg, const void* sg,
                                 const void* bg, const uint32_t* wu, const void* su,
                                 const void* bu, const int32_t* lhs, const int32_t* rhs,
                                 void* out, int64_t P, int64_t B, int64_t M, int64_t N,
                                 int64_t K, int64_t E, void* ws, hipStream_t st, int* nlaunch) {
  if (P > kGatherFusedMaxP && E > kGatherPrepMaxE) return kStatusUnsupported;
  if ((N + 15) / 16 > 65535 || P * M >= kGroupedMinRows) return kStatusUnsupported;
  return gather_qmv_launch<DT, BITS, GS, true>(x, wg, sg, bg, wu, su, bu, lhs, rhs, out, P, B, M,
                                               N, K, E, ws, st, nlaunch);
}


template <int DT, int BITS, int GS>
int SwigluTablesLaunch<DT, BITS, GS>::run(const void* x, const uint32_t* wg, const void* sg,
                                          const void* bg, const uint32_t* wu, const void* su,
                                          const void* bu, const int32_t* lhs, void* out,
                                          int64_t P, int64_t B, int64_t M, int64_t N, int64_t K,
                                          int64_t E, const void* tables, hipStream_t st,
                                          int* nlaunch) {
  if (!gather_thin_path(P, M, K, E)) return kStatusUnsupported;
  if (int rc = launch_thin_kernel<DT, BITS, GS, true>(x, wg, sg, bg, wu, su, bu, lhs, out, P, B,
                                                      M, N, K, E, tables, st))
    return rc;
  *nlaunch += 1;
  return 0;
}

template <int DT, int BITS, int GS>
int GatherFoldLaunch<DT, BITS, GS>::run(const void* x, const uint32_t* w, const void* s,
                                        const void* b, const int32_t* rhs, const float* cw,
                                        const void* sgate, const void* shared, void* out,
                                        int64_t T, int64_t top_k, int64_t N, int64_t K, int64_t E,
                                        hipStream_t st, int* nlaunch) {
  using C = QmvConf<BITS, GS>;
  const int64_t P = T * top_k;
  if (P < 1 || P > kFoldMaxP || P * K * 2 >= ((int64_t)1 << 31) || N > INT32_MAX)
    return kStatusUnsupported;
  const int R = (int)(P < kQmvMaxXM ? P : kQmvMaxXM);
  const int nwt = gather_tile_waves<BITS, GS>(P, N, K);
  if (P > 2 * (kFoldNW / nwt)) return kStatusUnsupported;   // more than two rounds
  // scales copied to LDS where the gather kernel copies them (the same tile
  // code either way)
  const bool sbl = gather_tile_sb<BITS, GS>(K, nwt) && qmv_sb_fits(K / GS, nwt, 1, s, b);
  const size_t lds = (size_t)(kFoldNW / nwt) *
                     gather_group_lds<BITS, GS, C::GPL>(nwt, kQmvMaxXM, sbl, (int)(K / GS), 1);
  // group-size-128 steps are 512 codes: eight streamed x rows per wave take
  // 8 KiB, so the limit is raised past the default 64 KiB once per kernel
  constexpr size_t kFoldMaxLds = 128 * 1024;
  if (lds > kFoldMaxLds) return kStatusUnsupported;
  const dim3 grid((unsigned)((N + 15) / 16));
  const bool sh = shared != nullptr;
#define MQ_FOLD(WT, SB, SH)                                                                     \
  if (nwt == WT && sbl == SB && sh == SH) {                                                      \
    static std::atomic<uint64_t> lds_set{0};                                                     \
    if (hipError_t e = ensure_lds_limit(                                                         \
            reinterpret_cast<const void*>(                                                       \
                &gather_fold_kernel<DT, BITS, GS, C::GPL, WT, C::PF, SB, SH>),                   \
            (int)kFoldMaxLds, lds_set))                                                          \
      return (int)e;                                                                             \
    hipLaunchKernelGGL((gather_fold_kernel<DT, BITS, GS, C::GPL, WT, C::PF, SB, SH>), grid,      \
                       dim3(64 * kFoldNW), lds, st, (const uint16_t*)x, w, (const uint16_t*)s,   \
                       (const uint16_t*)b, rhs, cw, (const uint16_t*)sgate,                      \
                       (const uint16_t*)shared, (uint16_t*)out, (int)P, (int)top_k, (int)N,      \
                       (int)K, (int)E, R);                                                       \
    *nlaunch += 1;                                                                               \
    return 0;                                                                                    \
  }
  MQ_FOLD(1, true, false) MQ_FOLD(2, true, false) MQ_FOLD(4, true, false)
  MQ_FOLD(1, true, true) MQ_FOLD(2, true, true) MQ_FOLD(4, true, true)
  MQ_FOLD(1, false, false) MQ_FOLD(2, false, false) MQ_FOLD(4, false, false)
  MQ_FOLD(1, false, true) MQ_FOLD(2, false, true) MQ_FOLD(4, false, true)
#undef MQ_FOLD
  return kStatusUnsupported;
}

}  // namespace mq
