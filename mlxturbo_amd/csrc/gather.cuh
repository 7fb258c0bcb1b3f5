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
// A operand.  A "segment" is up to R = 16/M pairs sharing one expert; each
// workgroup owns (segment, 16-column tile) and runs the skinny MFMA loop of
// qmm_skinny.cuh over that expert's rows, so every expert's weights stream
// from HBM once per call no matter how many tokens routed to it, and the
// dequantization work scales with distinct experts, not with pairs.
//
// Segment discovery needs no host sync and no extra launch for P <= 256:
// every workgroup ranks the pairs itself in LDS (pair p leads a segment when
// the number of earlier pairs with its expert is a multiple of R; segments
// are numbered by leader position).  Larger P (prefill-sized batches) runs a
// one-workgroup counting-sort prep kernel into the caller's workspace first.
// Pairs with an out-of-range expert or x index produce zero rows.
#pragma once
#include "qmm_skinny.cuh"

namespace mq {

constexpr int kGatherFusedMaxP = 256;
constexpr int kGatherPrepMaxE = 2048;

// Workspace (int32): [0] nseg | perm[P] | seg_start[P] | seg_len[P] | seg_expert[P]
__host__ __device__ inline size_t gather_ws_words(int64_t P) { return 1 + 4 * (size_t)P; }

inline size_t gather_workspace_bytes(int64_t P, int64_t M) {
  (void)M;
  if (P <= kGatherFusedMaxP) return 0;
  return (gather_ws_words(P) * 4 + 255) & ~(size_t)255;
}

__global__ __launch_bounds__(1024) void gather_prep_kernel(const int32_t* __restrict__ rhs, int P,
                                                           int E, int R,
                                                           int32_t* __restrict__ ws) {
  extern __shared__ int sh[];
  const int NE = E + 1;  // bucket E collects out-of-range experts
  int* cnt = sh;
  int* base = sh + NE;
  int* segb = sh + 2 * NE;
  int* cur = sh + 3 * NE;
  __shared__ int part[1024][2];
  const int t = threadIdx.x;
  const int nt = blockDim.x;
  for (int e = t; e < NE; e += nt) {
    cnt[e] = 0;
    cur[e] = 0;
  }
  __syncthreads();
  for (int p = t; p < P; p += nt) {
    int e = rhs[p];
    e = (e >= 0 && e < E) ? e : E;
    atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  // exclusive scans of cnt and ceil(cnt/R): chunk per thread, then Hillis-Steele.
  const int per = (NE + nt - 1) / nt;
  const int e0 = t * per;
  const int e1 = min(NE, e0 + per);
  int sc = 0, ss = 0;
  for (int e = e0; e < e1; ++e) {
    sc += cnt[e];
    ss += (cnt[e] + R - 1) / R;
  }
  part[t][0] = sc;
  part[t][1] = ss;
  __syncthreads();
  for (int off = 1; off < nt; off <<= 1) {
    int a = 0, b = 0;
    if (t >= off) {
      a = part[t - off][0];
      b = part[t - off][1];
    }
    __syncthreads();
    part[t][0] += a;
    part[t][1] += b;
    __syncthreads();
  }
  int rc = part[t][0] - sc;
  int rs = part[t][1] - ss;
  for (int e = e0; e < e1; ++e) {
    base[e] = rc;
    segb[e] = rs;
    rc += cnt[e];
    rs += (cnt[e] + R - 1) / R;
  }
  if (t == nt - 1) ws[0] = part[t][1];
  __syncthreads();
  int32_t* perm = ws + 1;
  int32_t* seg_start = perm + P;
  int32_t* seg_len = seg_start + P;
  int32_t* seg_exp = seg_len + P;
  for (int p = t; p < P; p += nt) {
    int e = rhs[p];
    e = (e >= 0 && e < E) ? e : E;
    perm[base[e] + atomicAdd(&cur[e], 1)] = p;
  }
  for (int e = t; e < NE; e += nt) {
    const int c = cnt[e];
    for (int j = 0; j * R < c; ++j) {
      const int s = segb[e] + j;
      seg_start[s] = base[e] + j * R;
      seg_len[s] = min(R, c - j * R);
      seg_exp[s] = e;
    }
  }
}

template <int DT, int BITS, int GS>
__global__ __launch_bounds__(256) void gather_skinny_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ w,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    const int32_t* __restrict__ lhs, const int32_t* __restrict__ rhs, uint16_t* __restrict__ out,
    const int32_t* __restrict__ ws, int P, int B, int M, int N, int K, int E) {
  __shared__ int s_rhs[kGatherFusedMaxP];
  __shared__ int s_cb[kGatherFusedMaxP];
  __shared__ int s_members[16];
  __shared__ int s_expert;
  __shared__ int s_found;
  const int t = threadIdx.x;
  const int nt = blockDim.x;
  const int R = 16 / M;
  const int seg = blockIdx.x;

  if (t < 16) s_members[t] = -1;
  if (t == 0) s_found = 0;
  if (ws == nullptr) {
    // In-workgroup segment discovery (P <= kGatherFusedMaxP).
    for (int p = t; p < P; p += nt) {
      const int e = rhs[p];
      s_rhs[p] = (e >= 0 && e < E) ? e : E;
    }
    __syncthreads();
    for (int p = t; p < P; p += nt) {
      const int e = s_rhs[p];
      int cb = 0;
      for (int q = 0; q < p; ++q) cb += (s_rhs[q] == e);
      s_cb[p] = cb;
    }
    __syncthreads();
    // the leader whose rank (number of earlier leaders) equals seg
    for (int p = t; p < P; p += nt) {
      if (s_cb[p] % R) continue;
      int rank = 0;
      for (int q = 0; q < p; ++q) rank += (s_cb[q] % R == 0);
      if (rank == seg) {
        s_expert = s_rhs[p];
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
      if (s_rhs[q] == e && d > 0 && d < R) s_members[d] = q;
    }
    __syncthreads();
  } else {
    if (seg >= ws[0]) return;
    const int32_t* perm = ws + 1;
    const int32_t* seg_start = perm + P;
    const int32_t* seg_len = seg_start + P;
    const int32_t* seg_exp = seg_len + P;
    const int st = seg_start[seg];
    const int ln = seg_len[seg];
    if (t < ln) s_members[t] = perm[st + t];
    if (t == 0) s_expert = seg_exp[seg];
    __syncthreads();
  }

  const int e = s_expert;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int nwaves = nt >> 6;
  const int r = lane & 15;
  const int c = lane >> 4;
  const int n0 = blockIdx.y * 16;
  const int n = n0 + r;
  const bool nval = (n < N) && (e < E);
  const int64_t Kw = (int64_t)K * BITS / 32;
  const int G = K / GS;
  const int64_t wrow_idx = nval ? ((int64_t)e * N + n) : 0;

  // A row r: pair members[r / M], row r % M within the pair.
  const int pi = r / M;
  const int pr = r - pi * M;
  const int q = (pi < R) ? s_members[pi] : -1;
  int xb = -1;
  if (q >= 0) xb = lhs ? lhs[q] : q;
  const bool mval = (q >= 0) && (xb >= 0) && (xb < B);
  const uint16_t* xrow = x + (mval ? ((int64_t)xb * M + pr) * K : 0);

  const f32x4 acc = skinny_accumulate<DT, BITS, GS>(xrow, mval, w + wrow_idx * Kw,
                                                    scales + wrow_idx * G, biases + wrow_idx * G,
                                                    nval, K, wave, nwaves, c);
  skinny_reduce(acc, nwaves, [&](int mm, int nn, float v) {
    const int pj = mm / M;
    if (pj >= R || n0 + nn >= N) return;
    const int qq = s_members[pj];
    if (qq < 0) return;
    const int rr = mm - pj * M;
    out[((int64_t)qq * M + rr) * N + n0 + nn] = T16<DT>::round1(v);
  });
}

template <int DT, int BITS, int GS>
inline void launch_gather_t(const void* x, const uint32_t* w, const void* s, const void* b,
                            const int32_t* lhs, const int32_t* rhs, void* out, int64_t P,
                            int64_t B, int64_t M, int64_t N, int64_t K, int64_t E, void* ws,
                            hipStream_t st, int* nlaunch) {
  using Gm = SkinnyGeom<BITS>;
  const int R = (int)(16 / M);
  const int nkb = (int)((K + Gm::KBLK - 1) / Gm::KBLK);
  const int waves = nkb < kSkinnyMaxWaves ? nkb : kSkinnyMaxWaves;
  int64_t max_seg = P;
  const int32_t* wsp = nullptr;
  if (P > kGatherFusedMaxP) {
    const int64_t bound = (P + R - 1) / R + E + 1;
    if (bound < max_seg) max_seg = bound;
    const size_t shmem = 4 * sizeof(int) * (size_t)(E + 1);
    hipLaunchKernelGGL(gather_prep_kernel, dim3(1), dim3(1024), shmem, st, rhs, (int)P, (int)E, R,
                       (int32_t*)ws);
    wsp = (const int32_t*)ws;
    *nlaunch += 1;
  }
  hipLaunchKernelGGL((gather_skinny_kernel<DT, BITS, GS>),
                     dim3((unsigned)max_seg, (unsigned)((N + 15) / 16)), dim3(64 * waves), 0, st,
                     (const uint16_t*)x, w, (const uint16_t*)s, (const uint16_t*)b, lhs, rhs,
                     (uint16_t*)out, wsp, (int)P, (int)B, (int)M, (int)N, (int)K, (int)E);
  *nlaunch += 1;
}

inline int launch_gather(const void* x, const uint32_t* w, const void* s, const void* b,
                         const int32_t* lhs, const int32_t* rhs, void* out, int64_t P, int64_t B,
                         int64_t M, int64_t N, int64_t K, int64_t E, int gs, int bits, int dtype,
                         int sorted, void* ws, hipStream_t st, int* nlaunch) {
  (void)sorted;  // segments are discovered either way; sortedness only orders them
  if (P > kGatherFusedMaxP && E > kGatherPrepMaxE) return kStatusUnsupported;
  if ((N + 15) / 16 > 65535) return kStatusUnsupported;
#define MQ_G(DT, BB, G)                                                                  \
  if (dtype == DT && bits == BB && gs == G) {                                            \
    launch_gather_t<DT, BB, G>(x, w, s, b, lhs, rhs, out, P, B, M, N, K, E, ws, st, nlaunch); \
    return 0;                                                                            \
  }
  MQ_G(kBF16, 4, 64) MQ_G(kBF16, 4, 32) MQ_G(kBF16, 4, 128)
  MQ_G(kBF16, 8, 64) MQ_G(kBF16, 8, 32) MQ_G(kBF16, 8, 128)
  MQ_G(kF16, 4, 64) MQ_G(kF16, 4, 32) MQ_G(kF16, 4, 128)
  MQ_G(kF16, 8, 64) MQ_G(kF16, 8, 32) MQ_G(kF16, 8, 128)
#undef MQ_G
  return kStatusUnsupported;
}

}  // namespace mq
