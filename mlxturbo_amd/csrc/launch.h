// Per-format launchers shared by the C ABI (abi.hip) and the kernel
// translation units (inst.hip, compiled once per (dtype, bits) so the
// library's kernels build in parallel).  Each launcher's run() is defined
// next to its kernels and explicitly instantiated in inst.hip; it enqueues on
// the given stream and returns 0 or a HIP error / kStatusUnsupported.
#pragma once
#include <atomic>

#include "mq_common.h"

namespace mq {

// mx.dequantize to a 16-bit T (dequant.cuh).
template <int DT, int BITS, int GS>
struct DequantLaunch {
  static int run(const uint32_t* w, const void* s, const void* b, void* out, int64_t N, int64_t K,
                 hipStream_t st);
};

// quantized_matmul for M rows, in launches of up to 16 rows, or 32 on the
// shared-x workgroups (qmv.cuh); with a workspace (ws, ws_bytes; may be
// NULL) of skinny_split_bytes(...) bytes, launches of 5-32 rows on
// matrices of few tiles run their K slices on separate workgroups (same
// bits).  *nlaunch counts the kernels enqueued.
template <int DT, int BITS, int GS>
struct SkinnyLaunch {
  static int run(const void* x, const uint32_t* w, const void* s, const void* b, void* out,
                 int64_t M, int64_t N, int64_t K, void* ws, size_t ws_bytes, hipStream_t st,
                 int* nlaunch);
};

// quantized_matmul of one row on the quad kernel (qmv_quad.cuh, its own
// translation unit quad.hip); kStatusUnsupported where it does not apply
// (M != 1, unaligned operands: then SkinnyLaunch runs).  *nlaunch counts the
// kernels enqueued.
template <int DT, int BITS, int GS>
struct QuadLaunch {
  static int run(const void* x, const uint32_t* w, const void* s, const void* b, void* out,
                 int64_t M, int64_t N, int64_t K, hipStream_t st, int* nlaunch);
};

// quantized_matmul for M > 16 rows on the MFMA tile kernel (qmm_wide.cuh);
// with a workspace of wide_workspace_bytes(wide_plan(...), M, N) bytes the
// K range may be split over workgroups (float partial planes plus a reduce
// kernel).  *nlaunch counts the kernels enqueued.
template <int DT, int BITS, int GS>
struct WideLaunch {
  static int run(const void* x, const uint32_t* w, const void* s, const void* b, void* out,
                 int64_t M, int64_t N, int64_t K, void* ws, size_t ws_bytes, hipStream_t st,
                 int* nlaunch);
};

// gather_qmm over P (x batch, expert) pairs (gather.cuh); *nlaunch counts the
// kernels enqueued.  prepped: ws already holds launch_thin_tables' tables for
// this routing; only the thin grouped kernel takes them (kStatusUnsupported
// for any other path).
template <int DT, int BITS, int GS>
struct GatherLaunch {
  static int run(const void* x, const uint32_t* w, const void* s, const void* b,
                 const int32_t* lhs, const int32_t* rhs, void* out, int64_t P, int64_t B,
                 int64_t M, int64_t N, int64_t K, int64_t E, void* ws, bool prepped,
                 hipStream_t st, int* nlaunch);
};

// Fused gate+up+SiLU over P pairs: out = silu(x . Wg^T) * (x . Wu^T) with
// float sums and one rounding (gather.cuh); decode / verify widths only
// (P * M < kGroupedMinRows, else kStatusUnsupported).
template <int DT, int BITS, int GS>
struct GluLaunch {
  static int run(const void* x, const uint32_t* wg, const void* sg, const void* bg,
                 const uint32_t* wu, const void* su, const void* bu, const int32_t* lhs,
                 const int32_t* rhs, void* out, int64_t P, int64_t B, int64_t M, int64_t N,
                 int64_t K, int64_t E, void* ws, hipStream_t st, int* nlaunch);
};

// Routing arguments of the decode GLU gather that routes its own tokens
// (gather.cuh, ROUTE): float logits [T, E], top_k, and where workgroup 0
// writes the routing (idx int32 / w float [T, top_k]) and, with sgw [H],
// the shared expert's gate (sgate [T]).
struct RouteArgs {
  const float* logits = nullptr;
  const uint16_t* sgw = nullptr;
  int32_t* idx = nullptr;
  float* w = nullptr;
  uint16_t* sgate = nullptr;
  int top_k = 0;
};

// The fused gate+up+SiLU gather of T decode tokens with the tokens' routing
// computed inside it from their logits (the routing kernel's pieces, so idx,
// w and sgate are mq_moe_route's bits and out is mq_gather_glu's over them);
// kStatusUnsupported beyond T * top_k = 64 pairs or E = 512 experts.
template <int DT, int BITS, int GS>
struct GluRouteLaunch {
  static int run(const void* x, const uint32_t* wg, const void* sg, const void* bg,
                 const uint32_t* wu, const void* su, const void* bu, void* out, int64_t T,
                 int64_t N, int64_t K, int64_t E, const RouteArgs& ra, hipStream_t st,
                 int* nlaunch);
};

// A prefill MoE layer's gate and up gathers and its SwiGLU pass in one launch
// (grouped.cuh, GLU thin tiles) over the tables launch_thin_tables built for
// this routing in `tables`: per pair row, out [P * M, N] = swiglu_t(T(x .
// Wg^T), T(x . Wu^T)), bit for bit the two gathers over the tables followed
// by launch_swiglu.  kStatusUnsupported where the thin kernel does not run
// (gather_thin_path).
template <int DT, int BITS, int GS>
struct SwigluTablesLaunch {
  static int run(const void* x, const uint32_t* wg, const void* sg, const void* bg,
                 const uint32_t* wu, const void* su, const void* bu, const int32_t* lhs,
                 void* out, int64_t P, int64_t B, int64_t M, int64_t N, int64_t K, int64_t E,
                 const void* tables, hipStream_t st, int* nlaunch);
};

// Down projection with the MoE combine folded in (gather.cuh), decode widths:
// x [T * top_k, K] (one row per pair), rhs and cw (float router weights)
// [T * top_k], out [T, N] = the combine of mq_moe_combine (inv = NULL) over
// mq_gather_qmm's output, bit for bit; sgate / shared (both or neither) merge
// the shared expert.  kStatusUnsupported beyond kFoldMaxP pairs, beyond two
// rounds of segments per workgroup (8 / 4 pairs where the tile splits K over
// 2 / 4 waves) or where the tile configuration does not fit: the caller then
// runs the two kernels, which are faster there.
constexpr int kFoldMaxP = 16;
template <int DT, int BITS, int GS>
struct GatherFoldLaunch {
  static int run(const void* x, const uint32_t* w, const void* s, const void* b,
                 const int32_t* rhs, const float* cw, const void* sgate, const void* shared,
                 void* out, int64_t T, int64_t top_k, int64_t N, int64_t K, int64_t E,
                 hipStream_t st, int* nlaunch);
};

// The decode MoE block of T <= 8 tokens in one launch (block.cuh): the
// routing of logits [T, E], the fused gate+up+SiLU gather into h
// [T * top_k, N1], the down projection [E, N2, N1] with the router-weighted
// combine and, with shared / ra.sgw, the shared-expert merge into out
// [T, N2]; the same bits as
// GluRouteLaunch followed by GatherFoldLaunch.  With ra.logits NULL the
// experts and router weights are given in ra.idx / ra.w (the decode layer:
// GluLaunch followed by GatherFoldLaunch).  kStatusUnsupported where its
// tile configuration does not apply or its grid does not fit the device at
// once (the caller then runs those two launches).
template <int DT, int BITS, int GS>
struct MoeBlockLaunch {
  static int run(const void* x, const uint32_t* wg, const void* sg, const void* bg,
                 const uint32_t* wu, const void* su, const void* bu, const uint32_t* wd,
                 const void* sd, const void* bd, const void* shared, void* h, void* out,
                 int64_t T, int64_t N1, int64_t K1, int64_t N2, int64_t E, const RouteArgs& ra,
                 hipStream_t st, int* nlaunch);
};

// MoE routing (route.hip): per row of float logits [rows, E] the top_k
// experts (descending, equal values by smaller index) into idx and their
// softmax weights into w; with x ([rows, H]) and sgw ([H]) non-null (dtype
// DT) also sgate[r] = sigmoid(T(x[r] . sgw)).  kStatusUnsupported outside
// E <= 1024, 1 <= top_k <= min(64, E), dtype bf16 / f16.
int launch_moe_route(const float* logits, int32_t* idx, float* w, int64_t rows, int64_t E,
                     int64_t top_k, const void* x, const void* sgw, void* sgate, int64_t H,
                     int dtype, hipStream_t st);

// SwiGLU of a MoE layer's gate and up outputs (swiglu.hip): out = T(T(silu(g))
// * u) elementwise over n values of dtype T (bf16 / f16), silu(g) = g / (1 +
// exp(-g)) in float.  kStatusUnsupported for other dtypes.
int launch_swiglu(const void* g, const void* u, void* out, int64_t n, int dtype, hipStream_t st);

// MLX affine quantize of N x K float values (dtype DT: weights, scales and
// biases share it) into the bitstream format, and dequantize of any width
// (formats.hip).  Both return 0 or kStatusUnsupported for a configuration
// outside bits {2,3,4,5,6,8} x group {32,64,128} x dtype {bf16,f16,f32}.
int launch_quantize(const void* w, uint32_t* wq, void* scales, void* biases, int64_t N,
                    int64_t K, int group_size, int bits, int dtype, hipStream_t st);
int launch_dequantize_bits(const uint32_t* wq, const void* scales, const void* biases, void* out,
                           int64_t N, int64_t K, int group_size, int bits, int dtype,
                           hipStream_t st);

// ---- host-side routing and sizing ------------------------------------------

// Raises a kernel's dynamic-LDS limit to `bytes` on the current device, once
// per device (the attribute is held per device; `done` is the call site's
// bit mask of devices already set).  Returns the HIP error of the first
// failing attempt, which is retried on the next call.
inline hipError_t ensure_lds_limit(const void* kern, int bytes, std::atomic<uint64_t>& done) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = dev >= 0 && dev < 64 ? (uint64_t)1 << dev : 0;
  if (bit && (done.load(std::memory_order_acquire) & bit)) return hipSuccess;
  e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess && bit) done.fetch_or(bit, std::memory_order_release);
  return e;
}

// Expert-grouped tile of workgroup i (1-D grid), or false for a workgroup
// with nothing to do.  Tiles are (segment, column tile) pairs, column tiles
// fastest; nseg of the bound's segments exist.  Workgroups are dealt to the
// eight XCDs (each with its own L2) in launch order, i on XCD i % 8, so XCD x
// gets the contiguous tile range [x * per, (x + 1) * per): the column tiles
// of a segment and the segments of one expert, which read the same x rows
// and the same weights, then share an L2 instead of fetching them on every
// XCD.  Busy workgroups are the first 8 * per of the grid.
__device__ __forceinline__ bool grouped_tile(int i, int nseg, int ncol, int& seg, int& col) {
  const int n = nseg * ncol;
  const int per = (n + 7) / 8;
  if (i >= 8 * per) return false;
  const int tile = (i % 8) * per + i / 8;
  if (tile >= n) return false;
  seg = tile / ncol;
  col = tile - seg * ncol;
  return true;
}

// Compute units of the current device, cached per device.
inline int device_cu_count() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Launch plan of the wide kernel: row-tile height and K splits, the pair
// with the fewest (rounds of one workgroup per CU; every height needs 92-147
// KB of LDS) x (time of one tile), plus the split reduction.  Tile times at
// K=5120, measured: 71 us (64 rows), 81 (128), 105 (192), 119 (256); a tile
// over a K slice costs ~3 us plus its share.  A last round that fills few CUs
// costs as much as a full one (K=5120 N=17408, 68 column tiles on 256 CUs:
// M=256 81 us with BM 128 against 112 with 256; M=512 113 with 192 against
// 126 with 256 and 173 with 128; M=2048 362 with 192 against 406 with 256;
// M=8192 1332 with 256 against 1515 with 192).  Splitting K serves narrow
// matrices, whose few column tiles leave most CUs idle (K=17408 N=5120 has
// 20), and one-round grids of wider ones: three splits put the 68 column
// tiles of K=5120 N=17408 on 204 of 256 CUs (M=96 / 160 / 192 / 256: 48.9 /
// 62.1 / 65.0 / 77.2 us against 59.4 / 74.9 / 79.3 / 86.5 with one, two or
// four; graph-timed, one box).  Partial planes are float [M, N] per split,
// written by the tile kernel and summed in split order by a reduce kernel:
// (8 S + 2) M N bytes at ~3.5 TB/s.
struct WidePlan {
  int bm = 256, splits = 1;
  double cost_us = 0.0;
};

inline WidePlan wide_plan(int64_t M, int64_t N, int64_t K, int cus, int max_splits = 8) {
  const int64_t cols = (N + 255) / 256;
  const int64_t nk = K / 64;
  const int bms[4] = {64, 128, 192, 256};
  const double tile_us[4] = {71.0, 81.0, 105.0, 119.0};   // one tile at K=5120, measured
  WidePlan best;
  bool first = true;
  for (int sp = 1; sp <= max_splits; sp = sp == 2 ? 3 : sp == 3 ? 4 : 2 * sp) {   // 1 2 3 4 8
    if (sp > 1 && nk / sp < 8) break;                 // at least 8 k-steps per split
    for (int i = 3; i >= 0; --i) {
      const int64_t wgs = cols * ((M + bms[i] - 1) / bms[i]) * sp;
      const double tile = (sp > 1 ? 3.0 : 0.0) + tile_us[i] * ((double)K / sp) / 5120.0;
      double cost = (double)((wgs + cus - 1) / cus) * tile;
      if (sp > 1) cost += (8.0 * sp + 2.0) * (double)M * (double)N / 3.5e6;
      if (first || cost < best.cost_us) {
        best.bm = bms[i];
        best.splits = sp;
        best.cost_us = cost;
        first = false;
      }
    }
  }
  return best;
}

inline size_t wide_workspace_bytes(const WidePlan& plan, int64_t M, int64_t N) {
  return plan.splits > 1 ? (size_t)plan.splits * (size_t)M * (size_t)N * sizeof(float) : 0;
}

// The wide kernel takes M > 16 rows, K in whole 64-code steps, 4/8-bit codes
// and groups of 32/64/128.
inline bool wide_eligible(int64_t M, int64_t N, int64_t K, int bits, int gs) {
  (void)N;
  return M > 16 && K % 64 == 0 && (bits == 4 || bits == 8) && gs >= 32 && gs % 32 == 0;
}

// Wide tile or 16-row skinny launches for M > 16 rows: the cheaper by a
// model fitted to measurements.  Few column tiles starve the wide grid
// (K=17408 N=5120: 20 tiles; M=17..64 took 229-249 us wide against 40-87
// in 16-row launches; K=4096 N=4096: 48 against 12-29), while at K=5120
// N=17408 the wide tile wins from M ~ 70.  Skinny launch time: about 3 us
// plus the weight bytes at 3.6 TB/s for one row, x1.15 for 2-4 rows, x1.4
// for 5-8, x1.65 for 9-16; on matrices of 640+ row tiles and 48+ rows per CU
// (the shared-x workgroups of 5-16 rows) x1.35 for 5-8 and x1.42 for 9-16
// (K=5120 N=17408: 20.7 and 21.8 us against 15.4 for the one-row model), and
// 17-32 rows there in one launch at x1.5 (two 16-row A tiles per weight
// fragment: M=17/24/32 22.0/21.6/21.1 us, one process).
// split_ok: a workspace is available for K splits.
// Rows per launch of the shared-x skinny workgroups on this matrix (the
// launch conditions of qmv.cuh restated for the route model): 32 when a
// launch of two 16-row A tiles fits, 16 when only the 5-16-row launch does,
// 0 when neither runs (fewer than 640 row tiles or 48 rows per CU, steps of
// more than 256 codes, or x slices and scale copies beyond the LDS).
inline int skinny_shared_x_rows(int64_t N, int64_t K, int bits, int gs, int cus) {
  const int64_t stepk = 4 * (int64_t)gs * ((bits == 4 && gs == 32) ? 2 : 1);
  const int64_t G = K / gs;
  if ((N + 15) / 16 < 640 || cus <= 0 || N < 48 * (int64_t)cus || stepk > 256) return 0;
  if (G % 8 != 0 || 2 * 16 * (G / 8) > 3 * 64 * 4) return 0;         // the scale copy
  const int64_t xsr = 2 * stepk + 16, sb = 6 * 2 * 16 * (2 * G + 16);   // 3 groups x 2 tiles
  const int64_t lds = 160 * 1024;
  if (2 * 4 * 16 * xsr + sb > lds - 3 * 4 * 2 * 1024) return 0;       // 16 rows, two buffers
  if (4 * 32 * xsr + sb <= lds - 3 * 4 * 2 * 2 * 1024) return 32;     // 32 rows, one buffer
  return 16;
}

// Whether 5-8 rows run the shared-x launch with x resident in LDS (the
// condition of qmv.cuh's launcher restated): m rows of x padded to whole
// steps plus the three groups' scale copies within the launch's dynamic LDS
// (kQmvShxLdsMax: the CU's 160 KiB less the static reduction buffers).
inline bool skinny_resident_x_fits(int64_t m, int64_t K, int bits, int gs) {
  const int64_t stepk = 4 * (int64_t)gs * ((bits == 4 && gs == 32) ? 2 : 1);
  const int64_t G = K / gs, stepg = stepk / gs;
  const int64_t nsteps = (G + stepg - 1) / stepg;
  const int64_t xres = m * (2 * nsteps * stepk + 16);
  const int64_t sb = 6 * 2 * 16 * (2 * G + 16);                      // 3 groups x 2 tiles
  return xres + sb <= 160 * 1024 - 3 * 4 * 2 * 64 * 16;
}

// K slices (the waves of the one-workgroup launch, 8 on matrices of fewer
// than 640 16-row tiles) that a skinny launch of m rows runs on separate
// workgroups (qmv.cuh qmv_split_kernel), or 0: 5-64 rows (16, 32 or 64
// streamed x rows: steps of at most 256 codes), 8 slices, K whole steps.  K=17408
// N=5120, one box: M=8 / 9 / 16 20.9-21.2 / 21.4 / 21.6 us against
// 21.6-21.8 / 23.0-23.2 / 24.1-24.5 on one workgroup per tile group, M=20 /
// 24 / 32 25.7 / 26.0 / 26.6 us against ~40-43 as a 16-row launch and a
// remainder (or ~49 on the wide tile at 32), M=40 / 48 / 64 32.2 / 32.8 /
// 35.2 us against 43.1 / 43.1 / 47-49; 2 and 4 rows lost (20.6-21.1
// against 17.9-19.4).
inline int skinny_split_slices(int64_t m, int64_t N, int64_t K, int bits, int gs) {
  const int64_t stepg = (bits == 4 && gs == 32) ? 8 : 4;   // groups per step
  if (m < 5 || m > 64 || (N + 15) / 16 >= 640 || stepg * gs > 256 || (K / gs) % stepg) return 0;
  return 8;
}

// Float partial planes of the split skinny launches of an M-row call (the
// launch loop of qmv.cuh: up to 64 rows per split launch, 16 otherwise).
inline size_t skinny_split_bytes(int64_t M, int64_t N, int64_t K, int bits, int gs) {
  int64_t most = 0;                                 // rows of the largest split launch
  for (int64_t r = M; r > 0;) {
    const int64_t ms = r < 64 ? r : 64;
    const int64_t step = skinny_split_slices(ms, N, K, bits, gs) ? ms : (r < 16 ? r : 16);
    if (skinny_split_slices(step, N, K, bits, gs)) most = step > most ? step : most;
    r -= step;
  }
  return (size_t)most * N * 8 * sizeof(float);
}

inline bool wide_route(int64_t M, int64_t N, int64_t K, int bits, int gs, int cus,
                       bool split_ok) {
  if (!wide_eligible(M, N, K, bits, gs)) return false;
  // The wide tile never streams its weights faster than ~0.9 TB/s at these
  // widths (few bytes in flight per CU: M=32 48.9 us, M=96 53.6 at K=5120
  // N=17408, M=64 49.8 at K=17408 N=5120), which the tile-time model, fitted
  // on full rounds, does not see.
  const double wbytes = (double)N * (double)K * bits / 8.0;
  double wide_us = wide_plan(M, N, K, cus, split_ok ? 8 : 1).cost_us;
  if (wide_us < wbytes / 0.9e6) wide_us = wbytes / 0.9e6;
  const double one = 3.0 + wbytes / 3.6e6;
  const int sx = skinny_shared_x_rows(N, K, bits, gs, cus);
  const bool shared_x = sx > 0;
  double skinny_us = 0.0;
  for (int64_t m0 = 0, step = 16; m0 < M; m0 += step) {
    // with the workspace, 5-64 rows on matrices of few tiles run as one
    // split launch (K=17408 N=5120: 16 / 32 / 64 rows 21.7 / 26.0-26.6 /
    // 35.2 us = 1.4 / 1.7 / 2.3 x one; from 96 rows the wide tile, 55.6 us)
    const int64_t ms = M - m0 < 64 ? M - m0 : 64;
    if (split_ok && skinny_split_slices(ms, N, K, bits, gs)) {
      step = ms;
      skinny_us += one * (ms > 32 ? 2.3 : ms > 16 ? 1.7 : 1.4);
      continue;
    }
    step = sx == 32 && M - m0 > 16 ? 32 : 16;
    const int64_t m = M - m0 < step ? M - m0 : step;
    skinny_us += one * (m > 16   ? 1.5
                        : m > 8  ? (shared_x ? 1.42 : 1.65)
                        : m > 4  ? (shared_x && skinny_resident_x_fits(m, K, bits, gs) ? 1.35
                                                                                       : 1.4)
                        : m > 1  ? 1.15
                                 : 1.0);
  }
  return wide_us < skinny_us;
}

// Workspace bytes of quantized_matmul (K splits of the wide kernel or of the
// split skinny launches), 0 when the chosen plan needs none.
inline size_t qmm_workspace_bytes(int64_t M, int64_t N, int64_t K, int bits, int gs, int cus) {
  if (!wide_route(M, N, K, bits, gs, cus, true)) return skinny_split_bytes(M, N, K, bits, gs);
  return wide_workspace_bytes(wide_plan(M, N, K, cus), M, N);
}

// gather_qmm: up to kGatherFusedMaxP pairs are grouped by expert inside the
// matmul kernel; more pairs go through a counting-sort prep kernel (experts
// up to kGatherPrepMaxE) that fills a caller-provided workspace.  Calls with
// at least kGroupedMinRows output rows (P * M, prefill) run the expert-grouped
// MFMA tile kernel on the same prep tables (the reference's prefill switch,
// fused.py:3122-3133, is at 1024 rows as well).
constexpr int kGatherFusedMaxP = 256;
constexpr int kGatherPrepMaxE = 2048;
constexpr int64_t kGroupedMinRows = 1024;

// Workspace (int32): [0] nseg | perm[P] | seg_start[P] | seg_len[P] | seg_expert[P] |
// header[4]: segments of size class 2 are [header[0], header[1]), class 1
// [header[1], header[2]), class 0 [header[2], header[3]) (header[3] = nseg) |
// lower[kGatherPrepMaxE + 2]: for keys in order, lower[e] = first pair whose
// key is >= e | order[ceil(P / kPrepChunk)]: 1 where chunk i of kPrepChunk
// pairs is in key order (its first pair compared with the pair before).
constexpr int kPrepChunk = 256;
__host__ __device__ inline size_t gather_ws_header(int64_t P) { return 1 + 4 * (size_t)P; }
__host__ __device__ inline size_t gather_ws_lower(int64_t P) { return gather_ws_header(P) + 4; }
__host__ __device__ inline size_t gather_ws_order(int64_t P) {
  return gather_ws_lower(P) + kGatherPrepMaxE + 2;
}
__host__ __device__ inline size_t gather_ws_words(int64_t P) {
  return gather_ws_order(P) + (size_t)((P + kPrepChunk - 1) / kPrepChunk);
}

// Builds gather_qmm's segment tables for P pairs into ws (prep.hip): pairs
// sorted by expert (E for invalid ones), cut into segments of up to R pairs,
// or by size class (R2 pairs from C2 pairs per expert, R1 from C1, R below).
// kPrepLaunches kernels; needs E <= kGatherPrepMaxE; returns 0 or a HIP error.
constexpr int kPrepLaunches = 2;
int launch_prep(const int32_t* rhs, const int32_t* lhs, int64_t P, int64_t E, int64_t B, int R,
                void* ws, hipStream_t st, int R1 = 0, int C1 = 0, int R2 = 0, int C2 = 0);

// Whether gather_qmm runs the thin grouped kernel (grouped.cuh): prefill
// widths (P M >= kGroupedMinRows output rows), banks within the prep
// tables, fewer than 96 rows per active expert, K <= 2048 in whole 64-code
// steps.  The same routing then serves calls of different K (a MoE layer's
// gate / up and down banks) from one table build.
inline bool gather_thin_path(int64_t P, int64_t M, int64_t K, int64_t E) {
  if (P * M < kGroupedMinRows || E > kGatherPrepMaxE || M > 64 || K > 2048 || K % 64) return false;
  const int64_t active = P < E ? P : E;
  return P * M / (active > 0 ? active : 1) < 96;
}

// The thin kernel's tables (launch_prep): segments of R = 64 / M pairs, and
// of 2 R pairs for experts with more than R pairs (class 1).
inline int launch_thin_tables(const int32_t* rhs, const int32_t* lhs, int64_t P, int64_t E,
                              int64_t B, int64_t M, void* ws, hipStream_t st) {
  const int R = (int)(64 / M);
  return launch_prep(rhs, lhs, P, E, B, R, ws, st, 2 * R, R + 1);
}

inline size_t gather_workspace_bytes(int64_t P, int64_t M) {
  if (P <= kGatherFusedMaxP && P * M < kGroupedMinRows) return 0;
  return (gather_ws_words(P) * 4 + 255) & ~(size_t)255;
}

}  // namespace mq
