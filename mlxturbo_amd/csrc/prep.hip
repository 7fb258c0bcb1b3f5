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
constexpr int kPrepThreads = 1024;
// Experts per thread of the table kernel (E + 1 keys over its threads).
constexpr int kPrepPer = (kGatherPrepMaxE + 1 + kPrepThreads - 1) / kPrepThreads;
// Threads of the run kernel; each takes kPrepChunk / kRunThreads pairs.  One
// pair per thread and small chunks keep it one memory round trip deep (lab,
// graph of launches, 16384 sorted pairs: chunks of 256 pairs 2.4 us, 1024
// pairs on 1024 threads 2.9, 1024 pairs four per thread 4.2).
constexpr int kRunThreads = 256;
constexpr int kRunPer = kPrepChunk / kRunThreads;

// Dynamic LDS of the table kernel: counting-sort tables (4 (E + 1) ints) and
// the staged keys.
inline size_t gather_prep_lds(int64_t P, int64_t E) {
  return sizeof(int) * (size_t)(4 * (E + 1) + (P <= kPrepLdsKeys ? P : 0));
}

// key of pair p: its expert, or E when the expert or the x index is invalid
__device__ __forceinline__ int prep_key(const int32_t* rhs, const int32_t* lhs, int p, int P,
                                        int E, int B) {
  const int e = rhs[p];
  const int xb = x_batch(lhs, p, P, B);
  return (e >= 0 && e < E && xb >= 0 && xb < B) ? e : E;
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
  __shared__ int wtot[3][16];
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
  // exclusive workgroup scan of three ints per thread: wave scans with
  // cross-lane reads, then one wave over the wave totals
  auto wg_scan3 = [&](const int (&v)[3], int (&excl)[3]) {
    int x[3], below[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      x[i] = v[i];
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(x[i], d, 64);
        if (lane >= d) x[i] += y;
      }
      below[i] = __shfl_up(x[i], 1, 64);
      if (lane == 63) wtot[i][wv] = x[i];
    }
    __syncthreads();
    if (wv == 0) {
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        int z = lane < nw ? wtot[i][lane] : 0;
#pragma unroll
        for (int d = 1; d < 16; d <<= 1) {
          const int y = __shfl_up(z, d, 64);
          if (lane >= d) z += y;
        }
        if (lane < nw) wtot[i][lane] = z;
      }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 3; ++i) excl[i] = (wv ? wtot[i][wv - 1] : 0) + (lane ? below[i] : 0);
  };
  // Segment numbering by class: thread-chunk counts ss[k] -> first segment
  // id of the chunk in each class, in table order (class 2, 1, 0); the last
  // thread writes the header and the total.
  auto class_ids = [&](const int (&ss)[3], int (&sid)[3]) {
    wg_scan3(ss, sid);
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
      int sid[3];
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
  int* cnt = sh;
  int* base = sh + NE;
  int* segb = sh + 2 * NE;
  int* cur = sh + 3 * NE;
  int* skey = sh + 4 * NE;
  const bool staged = P <= kPrepLdsKeys;
  if (staged) {
    for (int p0 = t; p0 < P; p0 += 16 * nt) {
      int k[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) k[i] = p0 + i * nt < P ? prep_key(rhs, lhs, p0 + i * nt, P, E, B) : 0;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int q = p0 + i * nt;
        if (q < P) skey[q] = k[i];
      }
    }
  }
  auto key_at = [&](int p) { return staged ? skey[p] : prep_key(rhs, lhs, p, P, E, B); };
  for (int e = t; e < NE; e += nt) {
    cnt[e] = 0;
    cur[e] = 0;
  }
  __syncthreads();
  for (int p = t; p < P; p += nt) atomicAdd(&cnt[key_at(p)], 1);
  __syncthreads();
  // exclusive scans of cnt and of each class's segments over contiguous key
  // chunks
  int sc = 0, ss[3] = {0, 0, 0};
  for (int e = e0; e < e1; ++e) {
    sc += cnt[e];
    const int k = cls_of(cnt[e]), R = r_of(k);
    ss[k] += (cnt[e] + R - 1) / R;
  }
  int rc3[3];
  {
    const int v[3] = {sc, 0, 0};
    wg_scan3(v, rc3);
    __syncthreads();                        // wtot is reused by the next scan
  }
  int rc = rc3[0];
  int rs[3];
  class_ids(ss, rs);
  for (int e = e0; e < e1; ++e) {
    const int k = cls_of(cnt[e]), R = r_of(k);
    base[e] = rc;
    segb[e] = rs[k];
    rc += cnt[e];
    rs[k] += (cnt[e] + R - 1) / R;
  }
  __syncthreads();
  for (int p = t; p < P; p += nt) {
    const int k = key_at(p);
    perm[base[k] + atomicAdd(&cur[k], 1)] = p;
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
                                      (int)gather_prep_lds(kPrepLdsKeys, kGatherPrepMaxE), lds_set))
    return (int)e;
  const int64_t nch = (P + kPrepChunk - 1) / kPrepChunk;
  hipLaunchKernelGGL(prep_runs_kernel, dim3((unsigned)nch), dim3(kRunThreads), 0, st, rhs, lhs,
                     (int)P, (int)E, (int)B, (int32_t*)ws);
  hipLaunchKernelGGL(gather_prep_kernel, dim3(1), dim3(kPrepThreads), gather_prep_lds(P, E), st,
                     rhs, lhs, (int)P, (int)E, (int)B, R, R1, C1, R2, C2, (int32_t*)ws);
  return 0;
}

}  // namespace mq
