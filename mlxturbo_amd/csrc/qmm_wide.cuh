// Wide (prefill) quantized matmul: placeholder until the MFMA tile kernel lands.
#pragma once
#include "mq_common.h"

namespace mq {

inline bool wide_eligible(int64_t M, int64_t N, int64_t K, int bits, int gs) {
  (void)M; (void)N; (void)K; (void)bits; (void)gs;
  return false;
}

inline int launch_wide(const void*, const uint32_t*, const void*, const void*, void*, int64_t,
                       int64_t, int64_t, int, int, int, hipStream_t) {
  return kStatusUnsupported;
}

}  // namespace mq
