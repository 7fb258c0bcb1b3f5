// C ABI of mlxturbo_amd (declared in include/mlxturbo_amd.h): argument
// validation, route selection and kernel launches.  No allocation, no
// synchronisation; every error is a status code plus a thread-local message.
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>

#include "../../include/mlxturbo_amd.h"
#include "combine.cuh"
#include "dequant.cuh"
#include "launch.h"

namespace {

thread_local std::string g_last_error;
std::atomic<uint64_t> g_launches{0};
// one-row calls on the 2..32-row kernel family (mq_set_row_identity)
std::atomic<int> g_row_identity{0};

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail((int)e, "%s: launch failed: %s", what, hipGetErrorString(e));
  g_launches.fetch_add(1, std::memory_order_relaxed);
  return MQ_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Arguments every format shares: MLX's widths, group sizes and dtypes.
int check_format(const void* w, const void* scales, const void* biases, int64_t N, int64_t K,
                 int group_size, int bits, int dtype) {
  if (!w || !scales) return fail(MQ_EINVAL, "w and scales must be non-null");
  if (!biases) return fail(MQ_EINVAL, "affine mode requires biases");
  if (N < 0 || K <= 0) return fail(MQ_EINVAL, "invalid sizes N=%lld K=%lld", (long long)N, (long long)K);
  if (bits != 2 && bits != 3 && bits != 4 && bits != 5 && bits != 6 && bits != 8)
    return fail(MQ_EINVAL, "bits must be one of 2,3,4,5,6,8 (got %d)", bits);
  if (group_size != 32 && group_size != 64 && group_size != 128)
    return fail(MQ_EINVAL, "group_size must be 32, 64 or 128 (got %d)", group_size);
  if (K % group_size)
    return fail(MQ_EINVAL, "K=%lld is not a multiple of group_size=%d", (long long)K, group_size);
  if (dtype != MQ_BFLOAT16 && dtype != MQ_FLOAT16 && dtype != MQ_FLOAT32)
    return fail(MQ_EINVAL, "unknown dtype code %d", dtype);
  if (!aligned16(w)) return fail(MQ_EINVAL, "w must be 16-byte aligned");
  return MQ_OK;
}

// check_format plus the widths the matmul kernels take (4 and 8 bits).
int check_common(const void* w, const void* scales, const void* biases, int64_t N, int64_t K,
                 int group_size, int bits, int dtype) {
  const int rc = check_format(w, scales, biases, N, K, group_size, bits, dtype);
  if (rc) return rc;
  if (bits != 4 && bits != 8)
    return fail(MQ_EUNSUPPORTED, "bits=%d has no matmul kernel (4 and 8 do)", bits);
  return MQ_OK;
}

template <template <int, int, int> class Launcher, typename... Args>
int dispatch_16(int dtype, int bits, int gs, Args... args) {
#define MQ_CASE(DT, B, G)                                   \
  if (dtype == DT && bits == B && gs == G) return Launcher<DT, B, G>::run(args...);
  MQ_CASE(mq::kBF16, 4, 64) MQ_CASE(mq::kBF16, 4, 32) MQ_CASE(mq::kBF16, 4, 128)
  MQ_CASE(mq::kBF16, 8, 64) MQ_CASE(mq::kBF16, 8, 32) MQ_CASE(mq::kBF16, 8, 128)
  MQ_CASE(mq::kF16, 4, 64) MQ_CASE(mq::kF16, 4, 32) MQ_CASE(mq::kF16, 4, 128)
  MQ_CASE(mq::kF16, 8, 64) MQ_CASE(mq::kF16, 8, 32) MQ_CASE(mq::kF16, 8, 128)
#undef MQ_CASE
  return mq::kStatusUnsupported;
}

// ---- scratch of mq_gather_qmm_noalloc --------------------------------------
// A file-scope device array holds the gather workspace (the prep kernel's
// segment tables) for callers that cannot allocate.  Each GPU holds its own
// copy until the process ends.  In host code `scratch` is only a stand-in
// for the symbol: its device address on the current device comes from
// hipGetSymbolAddress, resolved once per device and kept in g_scratch.
constexpr size_t kScratchBytes = MQ_GATHER_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices];

// Device address of the current device's scratch, or a status.
int scratch_for_current_device(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail((int)e, "hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(MQ_EUNSUPPORTED, "device %d is beyond the %d devices with a scratch slot", dev,
                kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(e != hipSuccess ? (int)e : MQ_EINVAL,
                  "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                  hipGetErrorString(e));
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return MQ_OK;
}

}  // namespace

namespace {

int moe_combine_checked(const void* y, int64_t y_rows, const int32_t* inv, const float* w,
                        const void* sgate, const void* shared, void* out, int64_t rows,
                        int64_t top_k, int64_t N, int dtype, void* hip_stream, const char* what) {
  if (!y || !w || !out) return fail(MQ_EINVAL, "y, w and out must be non-null");
  if (rows < 0 || N <= 0 || y_rows < 0) return fail(MQ_EINVAL, "invalid sizes rows=%lld N=%lld y_rows=%lld",
                                      (long long)rows, (long long)N, (long long)y_rows);
  if (y_rows > INT32_MAX) return fail(MQ_EUNSUPPORTED, "%s supports y_rows < 2^31", what);
  if (top_k < 1 || top_k > mq::kCombineMaxTopK)
    return fail(MQ_EINVAL, "top_k must be in 1..%d (got %lld)", mq::kCombineMaxTopK,
                (long long)top_k);
  if (N % 8) return fail(MQ_EUNSUPPORTED, "%s needs N %% 8 == 0 (got %lld)", what, (long long)N);
  if (dtype != MQ_BFLOAT16 && dtype != MQ_FLOAT16)
    return fail(MQ_EUNSUPPORTED, "%s supports bf16 and fp16 (dtype %d)", what, dtype);
  if (!aligned16(y) || !aligned16(out)) return fail(MQ_EINVAL, "y and out must be 16-byte aligned");
  if (shared && !aligned16(shared)) return fail(MQ_EINVAL, "shared must be 16-byte aligned");
  if (rows > 65535) return fail(MQ_EUNSUPPORTED, "%s supports up to 65535 rows per call", what);
  if (!inv && y_rows < rows * top_k)
    return fail(MQ_EINVAL, "inv=NULL needs y_rows >= rows*top_k (%lld < %lld)", (long long)y_rows,
                (long long)(rows * top_k));
  if (rows == 0) return MQ_OK;
  int rc = mq::launch_moe_combine(y, y_rows, inv, w, out, rows, top_k, N, dtype,
                                  reinterpret_cast<hipStream_t>(hip_stream), sgate, shared);
  if (rc) return fail(rc, "%s: no kernel for this configuration", what);
  return check_launch(what);
}

}  // namespace

extern "C" {

int mq_version(void) { return 8; }

const char* mq_last_error(void) { return g_last_error.c_str(); }

uint64_t mq_launch_count(void) { return g_launches.load(std::memory_order_relaxed); }

int mq_set_row_identity(int on) { return g_row_identity.exchange(on != 0 ? 1 : 0); }

int mq_dequantize(const uint32_t* w, const void* scales, const void* biases, void* out,
                  int64_t N, int64_t K, int group_size, int bits, int dtype, void* hip_stream) {
  int rc = check_format(w, scales, biases, N, K, group_size, bits, dtype);
  if (rc) return rc;
  if (!out) return fail(MQ_EINVAL, "out must be non-null");
  if (!aligned16(out)) return fail(MQ_EINVAL, "out must be 16-byte aligned");
  if (N == 0) return MQ_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(hip_stream);
  if (bits != 4 && bits != 8) {
    rc = mq::launch_dequantize_bits(w, scales, biases, out, N, K, group_size, bits, dtype, st);
    if (rc) return fail(rc, "dequantize: no kernel for bits=%d group_size=%d", bits, group_size);
    return check_launch("dequantize");
  }
  if (dtype == MQ_FLOAT32) {
    const int64_t words = N * (K * bits / 32);
#define MQ_D32(B, G)                                                                         \
  if (bits == B && group_size == G) {                                                         \
    hipLaunchKernelGGL((mq::dequantize32_kernel<B, G>), dim3(mq::dequant_grid(words, 256)), dim3(256), \
                       0, st, w, (const float*)scales, (const float*)biases, (float*)out, N, K); \
    return check_launch("dequantize");                                                        \
  }
    MQ_D32(4, 32) MQ_D32(4, 64) MQ_D32(4, 128) MQ_D32(8, 32) MQ_D32(8, 64) MQ_D32(8, 128)
#undef MQ_D32
    return fail(MQ_EUNSUPPORTED, "dequantize: unsupported float32 configuration");
  }
  rc = dispatch_16<mq::DequantLaunch>(dtype, bits, group_size, w, scales, biases, out, N, K, st);
  if (rc) return fail(rc, "dequantize: no kernel for dtype=%d bits=%d group_size=%d", dtype, bits,
                      group_size);
  return check_launch("dequantize");
}

int mq_quantize(const void* w, uint32_t* wq, void* scales, void* biases, int64_t N, int64_t K,
                int group_size, int bits, int dtype, void* hip_stream) {
  int rc = check_format(w, scales, biases, N, K, group_size, bits, dtype);
  if (rc) return rc;
  if (!wq) return fail(MQ_EINVAL, "wq must be non-null");
  if (!aligned16(wq)) return fail(MQ_EINVAL, "wq must be 16-byte aligned");
  if (dtype != MQ_FLOAT32 && (!aligned16(scales) || !aligned16(biases)))
    return fail(MQ_EINVAL, "scales and biases must be 16-byte aligned");
  if (N == 0) return MQ_OK;
  rc = mq::launch_quantize(w, wq, scales, biases, N, K, group_size, bits, dtype,
                           reinterpret_cast<hipStream_t>(hip_stream));
  if (rc) return fail(rc, "quantize: no kernel for bits=%d group_size=%d", bits, group_size);
  return check_launch("quantize");
}

size_t mq_quantized_matmul_workspace_size(int64_t M, int64_t N, int64_t K, int group_size,
                                          int bits) {
  if (M <= 0 || N <= 0 || K <= 0 || group_size <= 0 || K % group_size) return 0;
  return mq::qmm_workspace_bytes(M, N, K, bits, group_size, mq::device_cu_count());
}

int mq_quantized_matmul_ws(const void* x, const uint32_t* w, const void* scales,
                           const void* biases, void* out, int64_t M, int64_t N, int64_t K,
                           int group_size, int bits, int dtype, int transpose, void* workspace,
                           size_t workspace_bytes, void* hip_stream) {
  int rc = check_common(w, scales, biases, N, K, group_size, bits, dtype);
  if (rc) return rc;
  if (!x || !out) return fail(MQ_EINVAL, "x and out must be non-null");
  if (M < 0) return fail(MQ_EINVAL, "invalid M=%lld", (long long)M);
  if (!transpose)
    return fail(MQ_EUNSUPPORTED, "transpose=False is not implemented on this path");
  if (dtype == MQ_FLOAT32)
    return fail(MQ_EUNSUPPORTED, "float32 activations are not implemented on this path");
  if (N > INT32_MAX || K > INT32_MAX || M > INT32_MAX)
    return fail(MQ_EINVAL, "dimension exceeds int32 range");
  if (!aligned16(x)) return fail(MQ_EINVAL, "x must be 16-byte aligned");
  if (workspace && !aligned16(workspace)) return fail(MQ_EINVAL, "workspace must be 16-byte aligned");
  if (M == 0 || N == 0) return MQ_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(hip_stream);
  const int cus = mq::device_cu_count();
  // K splits only when the caller's workspace holds the planned partials
  const size_t need = mq::qmm_workspace_bytes(M, N, K, bits, group_size, cus);
  const bool split_ok = workspace && need && workspace_bytes >= need;
  if (mq::wide_route(M, N, K, bits, group_size, cus, split_ok)) {
    int nl = 0;
    rc = dispatch_16<mq::WideLaunch>(dtype, bits, group_size, x, w, scales, biases, out, M, N, K,
                                     split_ok ? workspace : nullptr,
                                     split_ok ? workspace_bytes : (size_t)0, st, &nl);
    if (rc) return fail(rc, "quantized_matmul: no wide kernel for this configuration");
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
      return fail((int)e, "quantized_matmul(wide): launch failed: %s", hipGetErrorString(e));
    g_launches.fetch_add((uint64_t)nl, std::memory_order_relaxed);
    return MQ_OK;
  }
  int nl = 0;
  if (M == 1 && !g_row_identity.load(std::memory_order_relaxed)) {
    rc = dispatch_16<mq::QuadLaunch>(dtype, bits, group_size, x, w, scales, biases, out, M, N, K,
                                     st, &nl);
    if (rc == 0) {
      hipError_t e = hipGetLastError();
      if (e != hipSuccess)
        return fail((int)e, "quantized_matmul(quad): launch failed: %s", hipGetErrorString(e));
      g_launches.fetch_add((uint64_t)nl, std::memory_order_relaxed);
      return MQ_OK;
    }
    if (rc != mq::kStatusUnsupported)
      return fail(rc, "quantized_matmul(quad): launch failed: %s",
                  hipGetErrorString((hipError_t)rc));
  }
  rc = dispatch_16<mq::SkinnyLaunch>(dtype, bits, group_size, x, w, scales, biases, out, M, N, K,
                                     split_ok ? workspace : nullptr,
                                     split_ok ? workspace_bytes : (size_t)0, st, &nl);
  if (rc) return fail(rc, "quantized_matmul: no kernel for dtype=%d bits=%d group_size=%d", dtype,
                      bits, group_size);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail((int)e, "quantized_matmul(skinny): launch failed: %s", hipGetErrorString(e));
  g_launches.fetch_add((uint64_t)nl, std::memory_order_relaxed);
  return MQ_OK;
}

int mq_quantized_matmul(const void* x, const uint32_t* w, const void* scales,
                        const void* biases, void* out, int64_t M, int64_t N, int64_t K,
                        int group_size, int bits, int dtype, int transpose, void* hip_stream) {
  return mq_quantized_matmul_ws(x, w, scales, biases, out, M, N, K, group_size, bits, dtype,
                                transpose, nullptr, 0, hip_stream);
}

size_t mq_gather_qmm_workspace_size(int64_t P, int64_t M) {
  return mq::gather_workspace_bytes(P, M);
}

int mq_gather_qmm(const void* x, const uint32_t* w, const void* scales, const void* biases,
                  const int32_t* lhs_indices, const int32_t* rhs_indices, void* out, int64_t P,
                  int64_t B, int64_t M, int64_t N, int64_t K, int64_t E, int group_size, int bits,
                  int dtype, int sorted_indices, void* workspace, size_t workspace_bytes,
                  void* hip_stream) {
  int rc = check_common(w, scales, biases, N, K, group_size, bits, dtype);
  if (rc) return rc;
  if (!x || !out || !rhs_indices) return fail(MQ_EINVAL, "x, out and rhs_indices must be non-null");
  if (P < 0 || M < 0 || E <= 0 || B < 0)
    return fail(MQ_EINVAL, "invalid sizes P=%lld M=%lld E=%lld B=%lld", (long long)P,
                (long long)M, (long long)E, (long long)B);
  if (!lhs_indices && P > 0 && (B <= 0 || P % B))
    return fail(MQ_EINVAL,
                "lhs_indices=NULL requires B to divide P (pair p reads x batch p / (P / B); "
                "B=%lld P=%lld)",
                (long long)B, (long long)P);
  if (dtype == MQ_FLOAT32)
    return fail(MQ_EUNSUPPORTED, "float32 activations are not implemented on this path");
  if (N > INT32_MAX || K > INT32_MAX || P > INT32_MAX || E > INT32_MAX || M > 16)
    return fail(MQ_EUNSUPPORTED, "gather_qmm supports M <= 16 rows per pair");
  if (!aligned16(x)) return fail(MQ_EINVAL, "x must be 16-byte aligned");
  if (P == 0 || M == 0 || N == 0) return MQ_OK;
  const size_t ws_need = mq::gather_workspace_bytes(P, M);
  if (ws_need && (workspace_bytes < ws_need || !workspace))
    return fail(MQ_EINVAL, "workspace too small: need %zu bytes",
                mq::gather_workspace_bytes(P, M));
  hipStream_t st = reinterpret_cast<hipStream_t>(hip_stream);
  int nl = 0;
  (void)sorted_indices;  // segments are discovered either way; sortedness only orders them
  rc = dispatch_16<mq::GatherLaunch>(dtype, bits, group_size, x, w, scales, biases, lhs_indices,
                                     rhs_indices, out, P, B, M, N, K, E, workspace, false, st,
                                     &nl);
  if (rc) return fail(rc, "gather_qmm: no kernel for this configuration");
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail((int)e, "gather_qmm: launch failed: %s", hipGetErrorString(e));
  g_launches.fetch_add((uint64_t)nl, std::memory_order_relaxed);
  return MQ_OK;
}

int mq_gather_tables(const int32_t* lhs_indices, const int32_t* rhs_indices, int64_t P,
                     int64_t B, int64_t M, int64_t E, void* tables, size_t tables_bytes,
                     void* hip_stream) {
  if (!rhs_indices) return fail(MQ_EINVAL, "rhs_indices must be non-null");
  if (P < 1 || M < 1 || E < 1 || B < 1)
    return fail(MQ_EINVAL, "invalid sizes P=%lld M=%lld E=%lld B=%lld", (long long)P,
                (long long)M, (long long)E, (long long)B);
  if (!lhs_indices && P % B)
    return fail(MQ_EINVAL, "lhs_indices=NULL requires B to divide P (B=%lld P=%lld)",
                (long long)B, (long long)P);
  if (P > INT32_MAX || P * M < mq::kGroupedMinRows || E > mq::kGatherPrepMaxE || M > 16)
    return fail(MQ_EUNSUPPORTED,
                "gather tables are built for prefill widths (P * M >= %lld output rows, "
                "E <= %d, M <= 16; got P=%lld M=%lld E=%lld)",
                (long long)mq::kGroupedMinRows, mq::kGatherPrepMaxE, (long long)P, (long long)M,
                (long long)E);
  const size_t need = mq::gather_workspace_bytes(P, M);
  if (!tables || tables_bytes < need)
    return fail(MQ_EINVAL, "tables too small: need %zu bytes", need);
  const int rc = mq::launch_thin_tables(rhs_indices, lhs_indices, P, E, B, M, tables,
                                        reinterpret_cast<hipStream_t>(hip_stream));
  if (rc) return fail(rc, "gather_tables: launch failed: %s", hipGetErrorString((hipError_t)rc));
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail((int)e, "gather_tables: launch failed: %s", hipGetErrorString(e));
  g_launches.fetch_add((uint64_t)mq::kPrepLaunches, std::memory_order_relaxed);
  return MQ_OK;
}

int mq_gather_qmm_tables(const void* x, const uint32_t* w, const void* scales,
                         const void* biases, const int32_t* lhs_indices,
                         const int32_t* rhs_indices, void* out, int64_t P, int64_t B, int64_t M,
                         int64_t N, int64_t K, int64_t E, int group_size, int bits, int dtype,
                         const void* tables, size_t tables_bytes, void* hip_stream) {
  int rc = check_common(w, scales, biases, N, K, group_size, bits, dtype);
  if (rc) return rc;
  if (!x || !out || !rhs_indices || !tables)
    return fail(MQ_EINVAL, "x, out, rhs_indices and tables must be non-null");
  if (P < 1 || M < 1 || E < 1 || B < 1)
    return fail(MQ_EINVAL, "invalid sizes P=%lld M=%lld E=%lld B=%lld", (long long)P,
                (long long)M, (long long)E, (long long)B);
  if (!lhs_indices && P % B)
    return fail(MQ_EINVAL, "lhs_indices=NULL requires B to divide P (B=%lld P=%lld)",
                (long long)B, (long long)P);
  if (dtype == MQ_FLOAT32)
    return fail(MQ_EUNSUPPORTED, "float32 activations are not implemented on this path");
  if (N > INT32_MAX || K > INT32_MAX || P > INT32_MAX || M > 16 ||
      !mq::gather_thin_path(P, M, K, E))
    return fail(MQ_EUNSUPPORTED, "this gather does not run on the tables' kernel");
  if (tables_bytes < mq::gather_workspace_bytes(P, M))
    return fail(MQ_EINVAL, "tables too small: need %zu bytes", mq::gather_workspace_bytes(P, M));
  if (!aligned16(x)) return fail(MQ_EINVAL, "x must be 16-byte aligned");
  if (N == 0) return MQ_OK;
  int nl = 0;
  rc = dispatch_16<mq::GatherLaunch>(dtype, bits, group_size, x, w, scales, biases, lhs_indices,
                                     rhs_indices, out, P, B, M, N, K, E, const_cast<void*>(tables),
                                     true, reinterpret_cast<hipStream_t>(hip_stream), &nl);
  if (rc) return fail(rc, "gather_qmm_tables: no kernel for this configuration");
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail((int)e, "gather_qmm_tables: launch failed: %s", hipGetErrorString(e));
  g_launches.fetch_add((uint64_t)nl, std::memory_order_relaxed);
  return MQ_OK;
}

int mq_gather_swiglu_tables(const void* x, const uint32_t* w_gate, const void* scales_gate,
                            const void* biases_gate, const uint32_t* w_up, const void* scales_up,
                            const void* biases_up, const int32_t* lhs_indices,
                            const int32_t* rhs_indices, void* out, int64_t P, int64_t B,
                            int64_t M, int64_t N, int64_t K, int64_t E, int group_size, int bits,
                            int dtype, const void* tables, size_t tables_bytes,
                            void* hip_stream) {
  int rc = check_common(w_gate, scales_gate, biases_gate, N, K, group_size, bits, dtype);
  if (rc) return rc;
  rc = check_common(w_up, scales_up, biases_up, N, K, group_size, bits, dtype);
  if (rc) return rc;
  if (!x || !out || !rhs_indices || !tables)
    return fail(MQ_EINVAL, "x, out, rhs_indices and tables must be non-null");
  if (P < 1 || M < 1 || E < 1 || B < 1)
    return fail(MQ_EINVAL, "invalid sizes P=%lld M=%lld E=%lld B=%lld", (long long)P,
                (long long)M, (long long)E, (long long)B);
  if (!lhs_indices && P % B)
    return fail(MQ_EINVAL, "lhs_indices=NULL requires B to divide P (B=%lld P=%lld)",
                (long long)B, (long long)P);
  if (dtype == MQ_FLOAT32)
    return fail(MQ_EUNSUPPORTED, "float32 activations are not implemented on this path");
  if (N > INT32_MAX || K > INT32_MAX || P > INT32_MAX || M > 16 ||
      !mq::gather_thin_path(P, M, K, E))
    return fail(MQ_EUNSUPPORTED, "this gather does not run on the tables' kernel");
  if (tables_bytes < mq::gather_workspace_bytes(P, M))
    return fail(MQ_EINVAL, "tables too small: need %zu bytes", mq::gather_workspace_bytes(P, M));
  if (!aligned16(x)) return fail(MQ_EINVAL, "x must be 16-byte aligned");
  if (N == 0) return MQ_OK;
  int nl = 0;
  rc = dispatch_16<mq::SwigluTablesLaunch>(dtype, bits, group_size, x, w_gate, scales_gate,
                                           biases_gate, w_up, scales_up, biases_up, lhs_indices,
                                           out, P, B, M, N, K, E, tables,
                                           reinterpret_cast<hipStream_t>(hip_stream), &nl);
  if (rc) return fail(rc, "gather_swiglu_tables: no kernel for this configuration");
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail((int)e, "gather_swiglu_tables: launch failed: %s", hipGetErrorString(e));
  g_launches.fetch_add((uint64_t)nl, std::memory_order_relaxed);
  return MQ_OK;
}

int mq_moe_glu_route(const void* x, const float* logits, const uint32_t* w_gate,
                     const void* scales_gate, const void* biases_gate, const uint32_t* w_up,
                     const void* scales_up, const void* biases_up, const void* sgw, int32_t* idx,
                     float* weights, void* sgate, void* out, int64_t T, int64_t top_k, int64_t N,
                     int64_t K, int64_t E, int group_size, int bits, int dtype,
                     void* hip_stream) {
  int rc = check_common(w_gate, scales_gate, biases_gate, N, K, group_size, bits, dtype);
  if (rc) return rc;
  rc = check_common(w_up, scales_up, biases_up, N, K, group_size, bits, dtype);
  if (rc) return rc;
  if (!x || !logits || !idx || !weights || !out)
    return fail(MQ_EINVAL, "x, logits, idx, weights and out must be non-null");
  if ((sgw == nullptr) != (sgate == nullptr))
    return fail(MQ_EINVAL, "sgw and sgate are given together or not at all");
  if (T < 0 || E < 1 || top_k < 1 || top_k > E)
    return fail(MQ_EINVAL, "invalid sizes T=%lld E=%lld top_k=%lld", (long long)T, (long long)E,
                (long long)top_k);
  if (dtype == MQ_FLOAT32)
    return fail(MQ_EUNSUPPORTED, "float32 activations are not implemented on this path");
  if (!aligned16(x)) return fail(MQ_EINVAL, "x must be 16-byte aligned");
  if (T == 0 || N == 0) return MQ_OK;
  if (T * top_k > 64 || E > 512 || N > INT32_MAX || K > INT32_MAX)
    return fail(MQ_EUNSUPPORTED,
                "moe_glu_route routes up to 64 pairs over up to 512 experts (T=%lld top_k=%lld "
                "E=%lld)", (long long)T, (long long)top_k, (long long)E);
  mq::RouteArgs ra;
  ra.logits = logits;
  ra.sgw = static_cast<const uint16_t*>(sgw);
  ra.idx = idx;
  ra.w = weights;
  ra.sgate = static_cast<uint16_t*>(sgate);
  ra.top_k = (int)top_k;
  int nl = 0;
  rc = dispatch_16<mq::GluRouteLaunch>(dtype, bits, group_size, x, w_gate, scales_gate,
                                       biases_gate, w_up, scales_up, biases_up, out, T, N, K, E,
                                       ra, reinterpret_cast<hipStream_t>(hip_stream), &nl);
  if (rc) return fail(rc, "moe_glu_route: no kernel for this configuration");
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail((int)e, "moe_glu_route: launch failed: %s", hipGetErrorString(e));
  g_launches.fetch_add((uint64_t)nl, std::memory_order_relaxed);
  return MQ_OK;
}

int mq_moe_block(const void* x, const float* logits, const uint32_t* w_gate,
                 const void* scales_gate, const void* biases_gate, const uint32_t* w_up,
                 const void* scales_up, const void* biases_up, const uint32_t* w_down,
                 const void* scales_down, const void* biases_down, const void* sgw,
                 const void* shared, int32_t* idx, float* weights, void* sgate, void* h,
                 void* out, int64_t T, int64_t top_k, int64_t N1, int64_t K1, int64_t N2,
                 int64_t E, int group_size, int bits, int dtype, void* hip_stream) {
  int rc = check_common(w_gate, scales_gate, biases_gate, N1, K1, group_size, bits, dtype);
  if (rc) return rc;
  rc = check_common(w_up, scales_up, biases_up, N1, K1, group_size, bits, dtype);
  if (rc) return rc;
  rc = check_common(w_down, scales_down, biases_down, N2, N1, group_size, bits, dtype);
  if (rc) return rc;
  if (!x || !logits || !idx || !weights || !h || !out)
    return fail(MQ_EINVAL, "x, logits, idx, weights, h and out must be non-null");
  if ((sgw == nullptr) != (sgate == nullptr) || (sgw == nullptr) != (shared == nullptr))
    return fail(MQ_EINVAL, "sgw, sgate and shared are given together or not at all");
  if (T < 0 || E < 1 || top_k < 1 || top_k > E)
    return fail(MQ_EINVAL, "invalid sizes T=%lld E=%lld top_k=%lld", (long long)T, (long long)E,
                (long long)top_k);
  if (dtype == MQ_FLOAT32)
    return fail(MQ_EUNSUPPORTED, "float32 activations are not implemented on this path");
  if (!aligned16(x) || !aligned16(h)) return fail(MQ_EINVAL, "x and h must be 16-byte aligned");
  if (T < 1 || T > 8 || top_k > 8 || T * top_k > 64 || E > 512 || N1 > INT32_MAX ||
      K1 > INT32_MAX || N2 > INT32_MAX)
    return fail(MQ_EUNSUPPORTED,
                "moe_block runs 1-8 tokens, top_k <= 8, E <= 512 (T=%lld top_k=%lld E=%lld)",
                (long long)T, (long long)top_k, (long long)E);
  if (N1 == 0 || N2 == 0) return fail(MQ_EUNSUPPORTED, "moe_block: empty projection");
  mq::RouteArgs ra;
  ra.logits = logits;
  ra.sgw = static_cast<const uint16_t*>(sgw);
  ra.idx = idx;
  ra.w = weights;
  ra.sgate = static_cast<uint16_t*>(sgate);
  ra.top_k = (int)top_k;
  int nl = 0;
  rc = dispatch_16<mq::MoeBlockLaunch>(dtype, bits, group_size, x, w_gate, scales_gate,
                                       biases_gate, w_up, scales_up, biases_up, w_down,
                                       scales_down, biases_down, shared, h, out, T, N1, K1, N2,
                                       E, ra, reinterpret_cast<hipStream_t>(hip_stream), &nl);
  if (rc) return fail(rc, "moe_block: no one-launch kernel for this configuration");
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail((int)e, "moe_block: launch failed: %s", hipGetErrorString(e));
  g_launches.fetch_add((uint64_t)nl, std::memory_order_relaxed);
  return MQ_OK;
}

int mq_moe_layer(const void* x, const int32_t* idx, const float* weights, const uint32_t* w_gate,
                 const void* scales_gate, const void* biases_gate, const uint32_t* w_up,
                 const void* scales_up, const void* biases_up, const uint32_t* w_down,
                 const void* scales_down, const void* biases_down, void* h, void* out,
                 int64_t T, int64_t top_k, int64_t N1, int64_t K1, int64_t N2, int64_t E,
                 int group_size, int bits, int dtype, void* hip_stream) {
  int rc = check_common(w_gate, scales_gate, biases_gate, N1, K1, group_size, bits, dtype);
  if (rc) return rc;
  rc = check_common(w_up, scales_up, biases_up, N1, K1, group_size, bits, dtype);
  if (rc) return rc;
  rc = check_common(w_down, scales_down, biases_down, N2, N1, group_size, bits, dtype);
  if (rc) return rc;
  if (!x || !idx || !weights || !h || !out)
    return fail(MQ_EINVAL, "x, idx, weights, h and out must be non-null");
  if (T < 0 || E < 1 || top_k < 1)
    return fail(MQ_EINVAL, "invalid sizes T=%lld E=%lld top_k=%lld", (long long)T, (long long)E,
                (long long)top_k);
  if (dtype == MQ_FLOAT32)
    return fail(MQ_EUNSUPPORTED, "float32 activations are not implemented on this path");
  if (!aligned16(x) || !aligned16(h)) return fail(MQ_EINVAL, "x and h must be 16-byte aligned");
  if (T < 1 || T > 8 || top_k > 8 || T * top_k > 64 || top_k > E || E > 512 ||
      N1 > INT32_MAX || K1 > INT32_MAX || N2 > INT32_MAX || N1 == 0 || N2 == 0)
    return fail(MQ_EUNSUPPORTED,
                "moe_layer runs 1-8 tokens, top_k <= 8, E <= 512 (T=%lld top_k=%lld E=%lld)",
                (long long)T, (long long)top_k, (long long)E);
  mq::RouteArgs ra;
  ra.idx = const_cast<int32_t*>(idx);
  ra.w = const_cast<float*>(weights);
  ra.top_k = (int)top_k;
  int nl = 0;
  rc = dispatch_16<mq::MoeBlockLaunch>(dtype, bits, group_size, x, w_gate, scales_gate,
                                       biases_gate, w_up, scales_up, biases_up, w_down,
                                       scales_down, biases_down, nullptr, h, out, T, N1, K1, N2,
                                       E, ra, reinterpret_cast<hipStream_t>(hip_stream), &nl);
  if (rc) return fail(rc, "moe_layer: no one-launch kernel for this configuration");
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail((int)e, "moe_layer: launch failed: %s", hipGetErrorString(e));
  g_launches.fetch_add((uint64_t)nl, std::memory_order_relaxed);
  return MQ_OK;
}

int mq_swiglu(const void* gate, const void* up, void* out, int64_t n, int dtype,
              void* hip_stream) {
  if (n < 0) return fail(MQ_EINVAL, "invalid size n=%lld", (long long)n);
  if (n == 0) return MQ_OK;
  if (!gate || !up || !out) return fail(MQ_EINVAL, "gate, up and out must be non-null");
  if (dtype != MQ_BFLOAT16 && dtype != MQ_FLOAT16)
    return fail(MQ_EUNSUPPORTED, "swiglu supports bf16 and fp16 (dtype %d)", dtype);
  const int rc = mq::launch_swiglu(gate, up, out, n, dtype,
                                   reinterpret_cast<hipStream_t>(hip_stream));
  if (rc) return fail(rc, "swiglu: no kernel for this configuration");
  return check_launch("swiglu");
}

int mq_gather_qmm_noalloc(const void* x, const uint32_t* w, const void* scales,
                          const void* biases, const int32_t* lhs_indices,
                          const int32_t* rhs_indices, void* out, int64_t P, int64_t B, int64_t M,
                          int64_t N, int64_t K, int64_t E, int group_size, int bits, int dtype,
                          int sorted_indices, void* hip_stream) {
  if (P < 0 || M < 0)
    return fail(MQ_EINVAL, "invalid sizes P=%lld M=%lld", (long long)P, (long long)M);
  const size_t need = mq::gather_workspace_bytes(P, M);
  if (need > kScratchBytes)
    return fail(MQ_EINVAL,
                "gather_qmm_noalloc: %lld pairs need %zu bytes of workspace; the static scratch "
                "holds %zu (use mq_gather_qmm with a workspace)",
                (long long)P, need, kScratchBytes);
  void* ws = nullptr;
  if (need) {
    const int rc = scratch_for_current_device(&ws);
    if (rc) return rc;
  }
  return mq_gather_qmm(x, w, scales, biases, lhs_indices, rhs_indices, out, P, B, M, N, K, E,
                       group_size, bits, dtype, sorted_indices, ws, need ? kScratchBytes : 0,
                       hip_stream);
}

int mq_gather_glu(const void* x, const uint32_t* w_gate, const void* scales_gate,
                  const void* biases_gate, const uint32_t* w_up, const void* scales_up,
                  const void* biases_up, const int32_t* lhs_indices,
                  const int32_t* rhs_indices, void* out, int64_t P, int64_t B, int64_t M,
                  int64_t N, int64_t K, int64_t E, int group_size, int bits, int dtype,
                  void* workspace, size_t workspace_bytes, void* hip_stream) {
  int rc = check_common(w_gate, scales_gate, biases_gate, N, K, group_size, bits, dtype);
  if (rc) return rc;
  rc = check_common(w_up, scales_up, biases_up, N, K, group_size, bits, dtype);
  if (rc) return rc;
  if (!x || !out || !rhs_indices) return fail(MQ_EINVAL, "x, out and rhs_indices must be non-null");
  if (P < 0 || M < 0 || E <= 0 || B < 0)
    return fail(MQ_EINVAL, "invalid sizes P=%lld M=%lld E=%lld B=%lld", (long long)P,
                (long long)M, (long long)E, (long long)B);
  if (!lhs_indices && P > 0 && (B <= 0 || P % B))
    return fail(MQ_EINVAL,
                "lhs_indices=NULL requires B to divide P (pair p reads x batch p / (P / B); "
                "B=%lld P=%lld)",
                (long long)B, (long long)P);
  if (dtype == MQ_FLOAT32)
    return fail(MQ_EUNSUPPORTED, "float32 activations are not implemented on this path");
  if (N > INT32_MAX || K > INT32_MAX || P > INT32_MAX || E > INT32_MAX || M > 16)
    return fail(MQ_EUNSUPPORTED, "gather_glu supports M <= 16 rows per pair");
  if (P * M >= mq::kGroupedMinRows)
    return fail(MQ_EUNSUPPORTED, "gather_glu is fused below %lld output rows (got %lld)",
                (long long)mq::kGroupedMinRows, (long long)(P * M));
  if (!aligned16(x)) return fail(MQ_EINVAL, "x must be 16-byte aligned");
  if (P == 0 || M == 0 || N == 0) return MQ_OK;
  const size_t ws_need = mq::gather_workspace_bytes(P, M);
  if (ws_need && (workspace_bytes < ws_need || !workspace))
    return fail(MQ_EINVAL, "workspace too small: need %zu bytes", ws_need);
  hipStream_t st = reinterpret_cast<hipStream_t>(hip_stream);
  int nl = 0;
  rc = dispatch_16<mq::GluLaunch>(dtype, bits, group_size, x, w_gate, scales_gate, biases_gate,
                                  w_up, scales_up, biases_up, lhs_indices, rhs_indices, out, P, B,
                                  M, N, K, E, workspace, st, &nl);
  if (rc) return fail(rc, "gather_glu: no kernel for this configuration");
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail((int)e, "gather_glu: launch failed: %s", hipGetErrorString(e));
  g_launches.fetch_add((uint64_t)nl, std::memory_order_relaxed);
  return MQ_OK;
}

int mq_gather_qmm_combine(const void* x, const uint32_t* w, const void* scales,
                          const void* biases, const int32_t* rhs_indices, const float* weights,
                          const void* sgate, const void* shared, void* out, int64_t T,
                          int64_t top_k, int64_t N, int64_t K, int64_t E, int group_size,
                          int bits, int dtype, void* hip_stream) {
  int rc = check_common(w, scales, biases, N, K, group_size, bits, dtype);
  if (rc) return rc;
  if (!x || !out || !rhs_indices || !weights)
    return fail(MQ_EINVAL, "x, out, rhs_indices and weights must be non-null");
  if (T < 0 || top_k < 1 || E <= 0)
    return fail(MQ_EINVAL, "invalid sizes T=%lld top_k=%lld E=%lld", (long long)T,
                (long long)top_k, (long long)E);
  if ((sgate != nullptr) != (shared != nullptr))
    return fail(MQ_EINVAL, "sgate and shared are given together or not at all");
  if (dtype == MQ_FLOAT32)
    return fail(MQ_EUNSUPPORTED, "float32 activations are not implemented on this path");
  if (N > INT32_MAX || K > INT32_MAX || E > INT32_MAX || T * top_k > mq::kFoldMaxP)
    return fail(MQ_EUNSUPPORTED, "gather_qmm_combine folds up to %d pairs per call (got %lld)",
                mq::kFoldMaxP, (long long)(T * top_k));
  if (!aligned16(x)) return fail(MQ_EINVAL, "x must be 16-byte aligned");
  if (T == 0 || N == 0) return MQ_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(hip_stream);
  int nl = 0;
  rc = dispatch_16<mq::GatherFoldLaunch>(dtype, bits, group_size, x, w, scales, biases,
                                         rhs_indices, weights, sgate, shared, out, T, top_k, N, K,
                                         E, st, &nl);
  if (rc) return fail(rc, "gather_qmm_combine: no folded kernel for this configuration");
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail((int)e, "gather_qmm_combine: launch failed: %s", hipGetErrorString(e));
  g_launches.fetch_add((uint64_t)nl, std::memory_order_relaxed);
  return MQ_OK;
}

int mq_moe_combine(const void* y, int64_t y_rows, const int32_t* inv, const float* w, void* out,
                   int64_t rows, int64_t top_k, int64_t N, int dtype, void* hip_stream) {
  return moe_combine_checked(y, y_rows, inv, w, nullptr, nullptr, out, rows, top_k, N, dtype,
                             hip_stream, "moe_combine");
}

int mq_moe_combine_shared(const void* y, int64_t y_rows, const int32_t* inv, const float* w,
                          const void* sgate, const void* shared, void* out, int64_t rows,
                          int64_t top_k, int64_t N, int dtype, void* hip_stream) {
  if (!sgate || !shared) return fail(MQ_EINVAL, "sgate and shared must be non-null");
  return moe_combine_checked(y, y_rows, inv, w, sgate, shared, out, rows, top_k, N, dtype,
                             hip_stream, "moe_combine_shared");
}

int mq_moe_route(const float* logits, int32_t* idx, float* weights, int64_t rows, int64_t E,
                 int64_t top_k, const void* x, const void* sgw, void* sgate, int64_t H, int dtype,
                 void* hip_stream) {
  if (!logits || !idx || !weights) return fail(MQ_EINVAL, "logits, idx and weights must be non-null");
  if (rows < 0 || E < 1 || top_k < 1)
    return fail(MQ_EINVAL, "invalid sizes rows=%lld E=%lld top_k=%lld", (long long)rows,
                (long long)E, (long long)top_k);
  if (top_k > E) return fail(MQ_EINVAL, "top_k=%lld exceeds E=%lld", (long long)top_k, (long long)E);
  const bool sg = x || sgw || sgate;
  if (sg && (!x || !sgw || !sgate))
    return fail(MQ_EINVAL, "x, sgw and sgate are given together or not at all");
  if (sg && H < 1) return fail(MQ_EINVAL, "invalid hidden size H=%lld", (long long)H);
  if (sg && dtype != MQ_BFLOAT16 && dtype != MQ_FLOAT16)
    return fail(MQ_EUNSUPPORTED, "moe_route's shared gate supports bf16 and fp16 (dtype %d)", dtype);
  if (E > 1024 || top_k > 64 || rows > INT32_MAX || H > INT32_MAX)
    return fail(MQ_EUNSUPPORTED, "moe_route takes E <= 1024 and top_k <= 64 (E=%lld top_k=%lld)",
                (long long)E, (long long)top_k);
  if (rows == 0) return MQ_OK;
  int rc = mq::launch_moe_route(logits, idx, weights, rows, E, top_k, x, sgw, sgate, H,
                                sg ? dtype : MQ_BFLOAT16, reinterpret_cast<hipStream_t>(hip_stream));
  if (rc) return fail(rc, "moe_route: no kernel for this configuration");
  return check_launch("moe_route");
}

}  // extern "C"
