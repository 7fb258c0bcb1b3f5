// Segment-table prep kernel of gather_qmm (one definition for the library:
// the matmul translation units call launch_prep, declared in launch.h).
// Reference: the prefill path's tile -> expert tables of
// kernels/moe_grouped_gemm.py:818-910 (segment_tables / counts_from_sorted_ids),
// built on the device here so no host synchronisation is needed.
#include "launch.h"

namespace mq {

namespace {

// Pairs whose keys the prep kernel stages in LDS (larger P reads them from
// memory on each pass).
constexpr int kPrepLdsKeys = 24576;

// Dynamic LDS of the prep kernel: counting-sort tables (4 (E + 1) ints) and
// the staged keys.
inline size_t gather_prep_lds(int64_t P, int64_t E) {
  return sizeof(int) * (size_t)(4 * (E + 1) + (P <= kPrepLdsKeys ? P : 0));
}

// Segment tables for the pairs: sorted by key (expert, or E for invalid
// pairs) into segments of up to R pairs of one key; one workgroup of 1024
// threads.  Keys are staged in LDS with coalesced loads, 16 per thread in
// flight.  Every pass walks the pairs with consecutive threads on consecutive
// pairs (no per-thread chains: a sequential walk over contiguous chunks of 16
// took ~2.5 us per pass).  Pairs already in
// key order (mlx-lm's _gather_sort, the reference's prefill path) keep their
// order (perm = identity): each key's run is read off its boundaries, with
// no atomics; other orders are counting-sorted.
//
// Segment sizes by class: an expert with c pairs is cut into segments of R2
// pairs when R2 > 0 and c >= C2 (class 2), of R1 when R1 > 0 and c >= C1
// (class 1), else of R0 (class 0).  The tables hold class 2's segments first,
// then class 1's, then class 0's (each in key order); the header after them
// (gather_ws_header) gives the class boundaries, ws[0] the total.
__global__ __launch_bounds__(1024) void gather_prep_kernel(
    const int32_t* __restrict__ rhs, const int32_t* __restrict__ lhs, int P, int E, int B,
    int R0, int R1, int C1, int R2, int C2, int32_t* __restrict__ ws) {
  extern __shared__ int sh[];
  const int NE = E + 1;  // bucket E collects out-of-range experts
  __shared__ int wtot[16];
  __shared__ int ctot[3];
  auto cls_of = [&](int c) { return (R2 > 0 && c >= C2) ? 2 : (R1 > 0 && c >= C1) ? 1 : 0; };
  auto r_of = [&](int k) { return k == 2 ? R2 : k == 1 ? R1 : R0; };
  const int t = threadIdx.x;
  const int nt = blockDim.x;
  const int lane = t & 63, wv = t >> 6, nw = nt >> 6;
  int* cnt = sh;
  int* base = sh + NE;
  int* segb = sh + 2 * NE;
  int* cur = sh + 3 * NE;
  int* skey = sh + 4 * NE;
  const bool staged = P <= kPrepLdsKeys;
  auto key_of = [&](int p) {
    const int e = rhs[p];
    const int xb = x_batch(lhs, p, P, B);
    return (e >= 0 && e < E && xb >= 0 && xb < B) ? e : E;
  };
  if (staged) {
    for (int p0 = t; p0 < P; p0 += 16 * nt) {
      int k[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) k[i] = p0 + i * nt < P ? key_of(p0 + i * nt) : 0;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int q = p0 + i * nt;
        if (q < P) skey[q] = k[i];
      }
    }
    __syncthreads();
  }
  auto key_at = [&](int p) { return staged ? skey[p] : key_of(p); };
  int32_t* perm = ws + 1;
  int32_t* seg_start = perm + P;
  int32_t* seg_len = seg_start + P;
  int32_t* seg_exp = seg_len + P;
  int32_t* hdr = ws + gather_ws_header(P);
  // exclusive workgroup scan (sum, or max with identity -1) of one int per
  // thread: wave scans with cross-lane reads, then one wave over the totals
  auto wg_scan = [&](int v, bool is_max) {
    const int id = is_max ? -1 : 0;
    auto op = [&](int a, int b) { return is_max ? max(a, b) : a + b; };
    int x = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int y = __shfl_up(x, d, 64);
      if (lane >= d) x = op(x, y);
    }
    const int below = __shfl_up(x, 1, 64);
    if (lane == 63) wtot[wv] = x;
    __syncthreads();
    if (wv == 0) {
      int z = lane < nw ? wtot[lane] : id;
#pragma unroll
      for (int d = 1; d < 16; d <<= 1) {
        const int y = __shfl_up(z, d, 64);
        if (lane >= d) z = op(z, y);
      }
      if (lane < nw) wtot[lane] = z;
    }
    __syncthreads();
    const int off = wv ? wtot[wv - 1] : id;
    const int excl = op(off, lane ? below : id);
    __syncthreads();                          // wtot is reused by the next scan
    return excl;
  };

  // Segment numbering by class: thread-chunk counts ss[k] -> first segment
  // id of the chunk in each class, in table order (class 2, 1, 0); thread 0
  // writes the header and the total.
  auto class_ids = [&](const int (&ss)[3], int (&sid)[3]) {
#pragma unroll
    for (int k = 0; k < 3; ++k) sid[k] = wg_scan(ss[k], false);
    if (t == nt - 1) {
#pragma unroll
      for (int k = 0; k < 3; ++k) ctot[k] = sid[k] + ss[k];
    }
    __syncthreads();
    const int start[3] = {ctot[2] + ctot[1], ctot[2], 0};
#pragma unroll
    for (int k = 0; k < 3; ++k) sid[k] += start[k];
    if (t == 0) {
      hdr[0] = 0;
      hdr[1] = ctot[2];
      hdr[2] = ctot[2] + ctot[1];
      hdr[3] = ctot[2] + ctot[1] + ctot[0];
      ws[0] = hdr[3];
    }
  };

  // ---- keys already in order: runs from their boundaries, no atomics --------
  bool ordered = true;
  for (int p = t + 1; p < P; p += nt) ordered &= key_at(p) >= key_at(p - 1);
  if (__syncthreads_and(ordered)) {
    // base[e] / cur[e]: first / last pair of key e's run (base -1: absent)
    for (int e = t; e < NE; e += nt) base[e] = -1;
    __syncthreads();
    for (int p = t; p < P; p += nt) {
      const int k = key_at(p);
      if (p == 0 || key_at(p - 1) != k) base[k] = p;
      if (p == P - 1 || key_at(p + 1) != k) cur[k] = p;
      perm[p] = p;
    }
    __syncthreads();
    const int per = (NE + nt - 1) / nt;
    const int e0 = min(NE, t * per), e1 = min(NE, e0 + per);
    int ss[3] = {0, 0, 0};
    for (int e = e0; e < e1; ++e) {
      const int c = base[e] >= 0 ? cur[e] - base[e] + 1 : 0;
      const int k = cls_of(c), R = r_of(k);
      ss[k] += (c + R - 1) / R;
    }
    int sid[3];
    class_ids(ss, sid);
    for (int e = e0; e < e1; ++e) {
      const int c = base[e] >= 0 ? cur[e] - base[e] + 1 : 0;
      const int k = cls_of(c), R = r_of(k);
      for (int j = 0; j * R < c; ++j) {
        const int q = sid[k]++;
        seg_start[q] = base[e] + j * R;
        seg_len[q] = min(R, c - j * R);
        seg_exp[q] = e;
      }
    }
    return;
  }

  // ---- any order: counting sort by key ------------------------------------
  for (int e = t; e < NE; e += nt) {
    cnt[e] = 0;
    cur[e] = 0;
  }
  __syncthreads();
  for (int p = t; p < P; p += nt) atomicAdd(&cnt[key_at(p)], 1);
  __syncthreads();
  // exclusive scans of cnt and of each class's segments over contiguous key
  // chunks
  const int per = (NE + nt - 1) / nt;
  const int e0 = min(NE, t * per);
  const int e1 = min(NE, e0 + per);
  int sc = 0, ss[3] = {0, 0, 0};
  for (int e = e0; e < e1; ++e) {
    sc += cnt[e];
    const int k = cls_of(cnt[e]), R = r_of(k);
    ss[k] += (cnt[e] + R - 1) / R;
  }
  int rc = wg_scan(sc, false);
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

// One prep launch; its LDS can pass 64 KiB, so the limit is raised once per
// device.
int launch_prep(const int32_t* rhs, const int32_t* lhs, int64_t P, int64_t E, int64_t B, int R,
                void* ws, hipStream_t st, int R1, int C1, int R2, int C2) {
  static std::atomic<uint64_t> lds_set{0};
  if (hipError_t e = ensure_lds_limit(reinterpret_cast<const void*>(&gather_prep_kernel),
                                      (int)gather_prep_lds(kPrepLdsKeys, kGatherPrepMaxE), lds_set))
    return (int)e;
  hipLaunchKernelGGL(gather_prep_kernel, dim3(1), dim3(1024), gather_prep_lds(P, E), st, rhs, lhs,
                     (int)P, (int)E, (int)B, R, R1, C1, R2, C2, (int32_t*)ws);
  return 0;
}


}  // namespace mq
