// Segment-table prep kernel of gather_qmm (one definition for the library:
// the matmul translation units call launch_prep, declared in launch.h).
// Reference: the prefill path's tile -> expert tables of
// kernels/moe_grouped_gemm.py:818-910 (segment_tables / counts_from_sorted_ids),
// built on the device here so no host synchronisation is needed.
#include "launch.h"

namespace mq {

namespace {

// Pairs whose keys the counting sort stages in LDS (larger P reads them from
// memory on each pass).
constexpr int kPrepLdsKeys = 24576;
// Dynamic LDS limit of the table kernel: the CU's 160 KiB less room for its
// static arrays.
constexpr int kPrepLdsMax = 159 * 1024;
constexpr int kPrepThreads = 1024;
// Experts per thread of the table kernel (E + 1 keys over its threads).
constexpr int kPrepPer = (kGatherPrepMaxE + 1 + kPrepThreads - 1) / kPrepThreads;
// Threads of the run kernel; each takes kPrepChunk / kRunThreads pairs.  One
// pair per thread and small chunks keep it one memory round trip deep (lab,
// graph of launches, 16384 sorted pairs: chunks of 256 pairs 2.4 us, 1024
// pairs on 1024 threads 2.9, 1024 pairs four per thread 4.2).
constexpr int kRunThreads = 256;
constexpr int kRunPer = kPrepChunk / kRunThreads;

// Dynamic LDS of the table kernel: counting-sort tables (4 (E + 1) ints and
// a spare counter), the staged keys, and where the whole fits the CU's
// 160 KiB the sorted pair order (prep_lds_perm), written to memory in one
// coalesced pass instead of as scattered 4-byte stores.
__host__ __device__ inline bool prep_lds_perm(int64_t P, int64_t E) {
  return P <= kPrepLdsKeys && 4 * (4 * (E + 1) + 1 + 2 * P) <= kPrepLdsMax;
}
inline size_t gather_prep_lds(int64_t P, int64_t E) {
  return sizeof(int) * (size_t)(4 * (E + 1) + 1 + (P <= kPrepLdsKeys ? P : 0) +
                                (prep_lds_perm(P, E) ? P : 0));
}

// key of pair p: its expert, or E when the expert or the x index is invalid.
// Without lhs the x index p / (P / B) is in range exactly when p < (P / B) B
// (no division per pair).
__device__ __forceinline__ int prep_key(const int32_t* rhs, const int32_t* lhs, int p, int P,
                                        int E, int B) {
  const int e = rhs[p];
  bool xok;
  if (lhs) {
    const int xb = lhs[p];
    xok = xb >= 0 && xb < B;
  } else {
    xok = B > 0 && p < (P / B) * B;
  }
  return (e >= 0 && e < E && xok) ? e : E;
}

// Inclusive sum over the 64 lanes (all active): row scans by row_shr 1, 2,
// 4, 8, then the row ends broadcast into the following rows (row_bcast 15
// into rows 1 and 3, row_bcast 31 into rows 2 and 3); lanes without a
// source add 0.
__device__ __forceinline__ int wave_incl_scan(int x) {
#define MQ_SCAN_STEP(CTRL, ROWS) x += __builtin_amdgcn_update_dpp(0, x, CTRL, ROWS, 0xf, false)
  MQ_SCAN_STEP(0x111, 0xf);
  MQ_SCAN_STEP(0x112, 0xf);
  MQ_SCAN_STEP(0x114, 0xf);
  MQ_SCAN_STEP(0x118, 0xf);
  MQ_SCAN_STEP(0x142, 0xa);
  MQ_SCAN_STEP(0x143, 0xc);
#undef MQ_SCAN_STEP
  return x;
}

// First of the two prep kernels, one workgroup per chunk of kPrepChunk
// pairs: perm = identity, order[chunk] = whether the chunk's keys do not
// descend (its first key compared with the pair before the chunk), and, in a
// chunk that is in order, lower[e] for every key e its ascents cover: the
// thread of pair p with key k after key k' < k (k' = -1 before pair 0)
// writes lower[k' + 1 .. k] = p, and the last pair's thread lower[k + 1 ..
// E + 1] = P.  When every chunk is in order each lower entry is written
// exactly once, so the table needs no clearing; otherwise the table kernel
// ignores it.
__global__ __launch_bounds__(kRunThreads) void prep_runs_kernel(
    const int32_t* __restrict__ rhs, const int32_t* __restrict__ lhs, int P, int E, int B,
    int32_t* __restrict__ ws) {
  int32_t* perm = ws + 1;
  int32_t* lower = ws + gather_ws_lower(P);
  int32_t* order = ws + gather_ws_order(P);
  const int t = threadIdx.x;
  const int p0 = blockIdx.x * kPrepChunk;
  int k[kRunPer], kp[kRunPer];
#pragma unroll
  for (int u = 0; u < kRunPer; ++u) {
    const int p = p0 + u * kRunThreads + t;
    k[u] = p < P ? prep_key(rhs, lhs, p, P, E, B) : 0;
    kp[u] = (p < P && p > 0) ? prep_key(rhs, lhs, p - 1, P, E, B) : -1;
  }
  bool ok = true;
#pragma unroll
  for (int u = 0; u < kRunPer; ++u) {
    const int p = p0 + u * kRunThreads + t;
    if (p < P) {
      ok &= kp[u] <= k[u];
      perm[p] = p;
    }
  }
  const bool ordered = __syncthreads_and(ok);
  if (t == 0) order[blockIdx.x] = ordered ? 1 : 0;
  if (!ordered) return;
#pragma unroll
  for (int u = 0; u < kRunPer; ++u) {
    const int p = p0 + u * kRunThreads + t;
    if (p >= P) continue;
    for (int e = kp[u] + 1; e <= k[u]; ++e) lower[e] = p;
    if (p == P - 1)
      for (int e = k[u] + 1; e <= E + 1; ++e) lower[e] = P;
  }
}

// Second prep kernel, one workgroup of kPrepThreads: the segment tables.
// Pairs sorted by key (expert, or E for invalid pairs) into segments of up
// to R pairs of one key.  When every chunk was in order (mlx-lm's
// _gather_sort, the reference's prefill path) the pairs keep their order and
// expert e's run is [lower[e], lower[e + 1]); otherwise the pairs are
// counting-sorted by key, with keys staged in LDS by coalesced loads (16 per
// thread in flight) and consecutive threads on consecutive pairs in every
// pass.
//
// Segment sizes by class: an expert with c pairs is cut into segments of R2
// pairs when R2 > 0 and c >= C2 (class 2), of R1 when R1 > 0 and c >= C1
// (class 1), else of R0 (class 0).  The tables hold class 2's segments first,
// then class 1's, then class 0's (each in key order); the header after them
// (gather_ws_header) gives the class boundaries, ws[0] the total.
__global__ __launch_bounds__(kPrepThreads) void gather_prep_kernel(
    const int32_t* __restrict__ rhs, const int32_t* __restrict__ lhs, int P, int E, int B,
    int R0, int R1, int C1, int R2, int C2, int32_t* __restrict__ ws) {
  extern __shared__ int sh[];
  const int NE = E + 1;  // bucket E collects out-of-range experts
  __shared__ int wtot[4][16];
  __shared__ int ctot[3];
  auto cls_of = [&](int c) { return (R2 > 0 && c >= C2) ? 2 : (R1 > 0 && c >= C1) ? 1 : 0; };
  auto r_of = [&](int k) { return k == 2 ? R2 : k == 1 ? R1 : R0; };
  const int t = threadIdx.x;
  const int nt = kPrepThreads;
  const int lane = t & 63, wv = t >> 6, nw = nt >> 6;
  int32_t* perm = ws + 1;
  int32_t* seg_start = perm + P;
  int32_t* seg_len = seg_start + P;
  int32_t* seg_exp = seg_len + P;
  int32_t* hdr = ws + gather_ws_header(P);
  const int32_t* lower = ws + gather_ws_lower(P);
  const int32_t* order = ws + gather_ws_order(P);
  // exclusive workgroup scan of four ints per thread: DPP wave scans, then
  // one wave over the wave totals
  auto wg_scan4 = [&](const int (&v)[4], int (&excl)[4]) {
    int x[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[i] = wave_incl_scan(v[i]);
      if (lane == 63) wtot[i][wv] = x[i];
    }
    __syncthreads();
    if (wv == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int z = wave_incl_scan(lane < nw ? wtot[i][lane] : 0);
        if (lane < nw) wtot[i][lane] = z;
      }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) excl[i] = (wv ? wtot[i][wv - 1] : 0) + x[i] - v[i];
  };
  // Segment numbering by class: thread-chunk counts ss[k] and their
  // exclusive scans sid[k] -> first segment id of the chunk in each class,
  // in table order (class 2, 1, 0); the last thread writes the header and
  // the total.
  auto class_ids = [&](const int (&ss)[3], int (&sid)[3]) {
    if (t == nt - 1) {
#pragma unroll
      for (int k = 0; k < 3; ++k) ctot[k] = sid[k] + ss[k];
      hdr[0] = 0;
      hdr[1] = ctot[2];
      hdr[2] = ctot[2] + ctot[1];
      hdr[3] = ctot[2] + ctot[1] + ctot[0];
      ws[0] = hdr[3];
    }
    __syncthreads();
    const int start[3] = {ctot[2] + ctot[1], ctot[2], 0};
#pragma unroll
    for (int k = 0; k < 3; ++k) sid[k] += start[k];
  };
  // contiguous key range [e0, e1) of this thread
  const int per = (NE + nt - 1) / nt;
  const int e0 = min(NE, t * per), e1 = min(NE, e0 + per);

  // ---- keys in order: runs from the lower table ----------------------------
  {
    // the table loads go out with the order flags (one round trip)
    int lw[kPrepPer + 1];
#pragma unroll
    for (int i = 0; i <= kPrepPer; ++i) lw[i] = e0 + i <= e1 ? lower[e0 + i] : 0;
    const int nch = (P + kPrepChunk - 1) / kPrepChunk;
    bool ok = true;
    for (int i = t; i < nch; i += nt) ok &= order[i] != 0;
    if (__syncthreads_and(ok)) {
      int ss[3] = {0, 0, 0};
#pragma unroll
      for (int i = 0; i < kPrepPer; ++i) {
        if (e0 + i < e1) {
          const int c = lw[i + 1] - lw[i];
          const int k = cls_of(c), R = r_of(k);
          ss[k] += (c + R - 1) / R;
        }
      }
      const int v4[4] = {ss[0], ss[1], ss[2], 0};
      int ex[4];
      wg_scan4(v4, ex);
      int sid[3] = {ex[0], ex[1], ex[2]};
      class_ids(ss, sid);
#pragma unroll
      for (int i = 0; i < kPrepPer; ++i) {
        if (e0 + i >= e1) continue;
        const int c = lw[i + 1] - lw[i];
        const int k = cls_of(c), R = r_of(k);
        for (int j = 0; j * R < c; ++j) {
          const int q = sid[k]++;
          seg_start[q] = lw[i] + j * R;
          seg_len[q] = min(R, c - j * R);
          seg_exp[q] = e0 + i;
        }
      }
      return;
    }
  }

  // ---- any order: counting sort by key ------------------------------------
  // Keys staged with every load of a thread issued before the first store
  // (clamped indices, no branch around the loads); the histogram and the
  // scatter take 16 pairs per thread and round, their LDS atomics
  // independent (the scatter's 16 returns in flight at once, pairs past P
  // counting into the spare counter cur[NE]).
  int* cnt = sh;
  int* base = sh + NE;
  int* segb = sh + 2 * NE;
  int* cur = sh + 3 * NE;                        // NE + 1 counters
  int* skey = sh + 4 * NE + 1;
  const bool staged = P <= kPrepLdsKeys;
  if (staged) {
    for (int p0 = t; p0 < P; p0 += 16 * nt) {
      int k[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) k[i] = prep_key(rhs, lhs, min(p0 + i * nt, P - 1), P, E, B);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int q = p0 + i * nt;
        if (q < P) skey[q] = k[i];
      }
    }
  }
  auto key_at = [&](int p) { return staged ? skey[p] : prep_key(rhs, lhs, p, P, E, B); };
  for (int e = t; e <= NE; e += nt) {
    if (e < NE) cnt[e] = 0;
    cur[e] = 0;
  }
  __syncthreads();
  for (int p0 = t; p0 < P; p0 += 16 * nt) {
    int k[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) k[i] = key_at(min(p0 + i * nt, P - 1));
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (p0 + i * nt < P) atomicAdd(&cnt[k[i]], 1);
  }
  __syncthreads();
  // one scan: the keys' counts and each class's segments over contiguous
  // key chunks
  int sc = 0, ss[3] = {0, 0, 0};
  for (int e = e0; e < e1; ++e) {
    sc += cnt[e];
    const int k = cls_of(cnt[e]), R = r_of(k);
    ss[k] += (cnt[e] + R - 1) / R;
  }
  int ex[4];
  {
    const int v4[4] = {ss[0], ss[1], ss[2], sc};
    wg_scan4(v4, ex);
  }
  int rc = ex[3];
  int rs[3] = {ex[0], ex[1], ex[2]};
  class_ids(ss, rs);
  for (int e = e0; e < e1; ++e) {
    const int k = cls_of(cnt[e]), R = r_of(k);
    base[e] = rc;
    segb[e] = rs[k];
    rc += cnt[e];
    rs[k] += (cnt[e] + R - 1) / R;
  }
  __syncthreads();
  // the pair order: into LDS and then to memory in one coalesced pass
  // (scattered 4-byte stores from this one CU took 5-8 us at 16384 pairs)
  const bool lperm = prep_lds_perm(P, E);
  int* sperm = skey + P;
  for (int p0 = t; p0 < P; p0 += 16 * nt) {
    int k[16], pos[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) k[i] = p0 + i * nt < P ? key_at(p0 + i * nt) : NE;
#pragma unroll
    for (int i = 0; i < 16; ++i) pos[i] = atomicAdd(&cur[k[i]], 1);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int q = p0 + i * nt;
      if (q >= P) continue;
      if (lperm) sperm[base[k[i]] + pos[i]] = q;
      else perm[base[k[i]] + pos[i]] = q;
    }
  }
  if (lperm) {
    __syncthreads();
    for (int i = t; i < P; i += nt) perm[i] = sperm[i];
  }
  for (int e = t; e < NE; e += nt) {
    const int c = cnt[e];
    const int R = r_of(cls_of(c));
    for (int j = 0; j * R < c; ++j) {
      const int s = segb[e] + j;
      seg_start[s] = base[e] + j * R;
      seg_len[s] = min(R, c - j * R);
      seg_exp[s] = e;
    }
  }
}

}  // namespace

// The two prep launches; the table kernel's LDS can pass 64 KiB, so its
// limit is raised once per device.
int launch_prep(const int32_t* rhs, const int32_t* lhs, int64_t P, int64_t E, int64_t B, int R,
                void* ws, hipStream_t st, int R1, int C1, int R2, int C2) {
  if (E < 0 || E > kGatherPrepMaxE || P < 1 || P > INT32_MAX / 4) return kStatusUnsupported;
  static std::atomic<uint64_t> lds_set{0};
  if (hipError_t e = ensure_lds_limit(reinterpret_cast<const void*>(&gather_prep_kernel),
                                      kPrepLdsMax, lds_set))
    return (int)e;
  const int64_t nch = (P + kPrepChunk - 1) / kPrepChunk;
  hipLaunchKernelGGL(prep_runs_kernel, dim3((unsigned)nch), dim3(kRunThreads), 0, st, rhs, lhs,
                     (int)P, (int)E, (int)B, (int32_t*)ws);
  hipLaunchKernelGGL(gather_prep_kernel, dim3(1), dim3(kPrepThreads), gather_prep_lds(P, E), st,
                     rhs, lhs, (int)P, (int)E, (int)B, R, R1, C1, R2, C2, (int32_t*)ws);
  return 0;
}

}  // namespace mq
