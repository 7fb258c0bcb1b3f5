// Per-format launchers shared by the C ABI (abi.hip) and the kernel
// translation units (inst.hip, compiled once per (dtype, bits) so the
// library's kernels build in parallel).  Each launcher's run() is defined
// next to its kernels and explicitly instantiated in inst.hip; it enqueues on
// the given stream and returns 0 or a HIP error / kStatusUnsupported.
#pragma once
#include "mq_common.h"

namespace mq {

// mx.dequantize to a 16-bit T (dequant.cuh).
template <int DT, int BITS, int GS>
struct DequantLaunch {
  static int run(const uint32_t* w, const void* s, const void* b, void* out, int64_t N, int64_t K,
                 hipStream_t st);
};

// quantized_matmul for M rows, in launches of up to 16 rows (qmv.cuh).
template <int DT, int BITS, int GS>
struct SkinnyLaunch {
  static int run(const void* x, const uint32_t* w, const void* s, const void* b, void* out,
                 int64_t M, int64_t N, int64_t K, hipStream_t st);
};

// quantized_matmul for M > 16 rows on the MFMA tile kernel (qmm_wide.cuh).
template <int DT, int BITS, int GS>
struct WideLaunch {
  static int run(const void* x, const uint32_t* w, const void* s, const void* b, void* out,
                 int64_t M, int64_t N, int64_t K, hipStream_t st);
};

// gather_qmm over P (x batch, expert) pairs (gather.cuh); *nlaunch counts the
// kernels enqueued.
template <int DT, int BITS, int GS>
struct GatherLaunch {
  static int run(const void* x, const uint32_t* w, const void* s, const void* b,
                 const int32_t* lhs, const int32_t* rhs, void* out, int64_t P, int64_t B,
                 int64_t M, int64_t N, int64_t K, int64_t E, void* ws, hipStream_t st,
                 int* nlaunch);
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

// ---- host-side routing and sizing ------------------------------------------

// The wide kernel takes M > 16 rows, K in whole 64-code steps, 4/8-bit codes
// and groups of 32/64/128.
inline bool wide_eligible(int64_t M, int64_t N, int64_t K, int bits, int gs) {
  (void)N;
  return M > 16 && K % 64 == 0 && (bits == 4 || bits == 8) && gs >= 32 && gs % 32 == 0;
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

// Workspace (int32): [0] nseg | perm[P] | seg_start[P] | seg_len[P] | seg_expert[P]
__host__ __device__ inline size_t gather_ws_words(int64_t P) { return 1 + 4 * (size_t)P; }

inline size_t gather_workspace_bytes(int64_t P, int64_t M) {
  if (P <= kGatherFusedMaxP && P * M < kGroupedMinRows) return 0;
  return (gather_ws_words(P) * 4 + 255) & ~(size_t)255;
}

}  // namespace mq
