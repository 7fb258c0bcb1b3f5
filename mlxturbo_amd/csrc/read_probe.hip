// Measurement helper, not part of the library's C ABI (built into its own
// libmq_read_probe.so): a plain streaming read of a device buffer, used by
// bench.py as the measured second denominator of the roofline (what one
// MI355X reads per second when nothing but reading is asked of it, launch
// and ramp included, at the kernel's own byte count).
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

}  // namespace

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
