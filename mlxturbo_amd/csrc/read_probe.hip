// Measurement helpers, not part of the library's C ABI (built into their own
// libmq_read_probe.so), used by bench.py as the measured second denominators
// of the rooflines: a plain streaming read of a device buffer (what one
// MI355X reads per second when nothing but reading is asked of it, launch
// and ramp included, at the kernel's own byte count), and a loop of bf16
// MFMAs on changing operands (what its matrix cores sustain, with the shader
// clock they run at: power limits the clock under MFMA load, and the
// operands' bit activity changes how far).
//
// Layout: workgroup g reads the contiguous chunk [g * chunk, (g + 1) * chunk)
// with 16-byte non-temporal loads, each lane keeping U loads in flight; the
// data are folded into a register and written only if they equal a magic
// value, so the loads cannot be dropped.  Swept over 50 MB-4.3 GB (default,
// sc0, sc1 and nt cache policies; 4, 8 and 16 workgroups per CU; U = 2, 4):
// nt with 4 workgroups per CU and U = 2 read fastest at every size (50 MB in
// 8.85 us, 4.3 GB at 6.99 TB/s), 7-10% ahead of the default policy.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256, kUnroll = 2;
constexpr int kNonTemporal = 2;  // cache-policy bits of the buffer load: nt

__global__ __launch_bounds__(kThreads) void read_probe_kernel(const char* __restrict__ p,
                                                              uint64_t bytes, uint64_t chunk,
                                                              uint32_t* __restrict__ sink) {
  const uint64_t begin = (uint64_t)blockIdx.x * chunk;
  if (begin >= bytes) return;
  const uint64_t end = begin + chunk < bytes ? begin + chunk : bytes;
  const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(p + begin), (short)0,
                                                    (int)(end - begin), 0x00020000);
  uint32_t acc = 0;
  for (uint32_t o = threadIdx.x * 16u; o < (uint32_t)(end - begin);
       o += kThreads * 16u * kUnroll) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      v[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, o + u * kThreads * 16u, 0, kNonTemporal);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  if (acc == 0x9e3779b9u) sink[threadIdx.x] = acc;
}

// Every wave keeps 4 independent v_mfma_f32_32x32x16_bf16 chains busy for
// `iters` rounds, its operands rewritten each round so the multipliers see
// changing bits (constant operands ran ~20% faster: the clock stayed higher);
// thread 0 of each workgroup records its shader-cycle and 100 MHz real-time
// counters at start and end.
__global__ __launch_bounds__(512) void mfma_probe_kernel(int iters, uint32_t* __restrict__ sink,
                                                         uint64_t* __restrict__ clk) {
  typedef float f32x16 __attribute__((ext_vector_type(16)));
  typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
  const uint64_t c0 = __builtin_readcyclecounter(), r0 = __builtin_amdgcn_s_memrealtime();
  f32x16 acc[4] = {};
  u32x4 a = {threadIdx.x * 0x9e3779b9u, 0x3f1f3e2du ^ threadIdx.x, 0xbe5d3c7au, 0x3e2b3f6eu};
  const u32x4 b = {0xbf3a3e11u, threadIdx.x * 0x85ebca6bu, 0x3e7dbf02u, 0x3f11be33u};
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                        __builtin_bit_cast(bf16x8, b), acc[j], 0,
                                                        0, 0);
    a = __builtin_elementwise_bitreverse(a) ^ b;
  }
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int q = 0; q < 16; ++q) sum += acc[j][q];
  if (sum == 1.2345f) sink[threadIdx.x] = 1u;
  if (threadIdx.x == 0) {
    uint64_t* c = clk + 4 * (uint64_t)blockIdx.x;
    c[0] = c0;
    c[1] = __builtin_readcyclecounter();
    c[2] = r0;
    c[3] = __builtin_amdgcn_s_memrealtime();
  }
}

}  // namespace

// Runs `workgroups` workgroups of 8 waves, each wave 4 x `iters` MFMAs of
// 32x32x16 (32768 FLOP each); `clk` holds 4 uint64 per workgroup (shader
// cycles at start / end, 100 MHz real time at start / end), `sink` 2 KiB
// written only by chance.  0 on success, else the HIP error code.
extern "C" int mq_mfma_probe(int iters, int workgroups, void* sink, void* clk, void* stream) {
  if (iters <= 0 || workgroups <= 0 || !sink || !clk) return -1;
  hipLaunchKernelGGL(mfma_probe_kernel, dim3((unsigned)workgroups), dim3(512), 0,
                     reinterpret_cast<hipStream_t>(stream), iters,
                     static_cast<uint32_t*>(sink), static_cast<uint64_t*>(clk));
  return (int)hipGetLastError();
}

// Reads `bytes` (a multiple of 16, each chunk under 2 GiB) from `p`; `sink`
// is 1 KiB of device memory that is written only by chance.  0 on success,
// else the HIP error code.
extern "C" int mq_read_probe(const void* p, uint64_t bytes, void* sink, int workgroups,
                             void* stream) {
  if (!p || !sink || bytes % 16 || workgroups <= 0) return -1;
  uint64_t chunk = (bytes + (uint64_t)workgroups - 1) / (uint64_t)workgroups;
  chunk = (chunk + 15) & ~(uint64_t)15;
  if (chunk >= ((uint64_t)1 << 31)) return -1;
  hipLaunchKernelGGL(read_probe_kernel, dim3((unsigned)workgroups), dim3(kThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<const char*>(p), bytes,
                     chunk, static_cast<uint32_t*>(sink));
  return (int)hipGetLastError();
}
