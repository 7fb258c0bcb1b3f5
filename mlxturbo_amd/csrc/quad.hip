// Kernel instantiations of the quad kernel (qmv_quad.cuh) for one (dtype,
// bits) pair and every group size.  Built once per pair with
// -DMQ_INST_DT=<0|1> -DMQ_INST_BITS=<4|8>, and with -mllvm
// -amdgpu-mfma-vgpr-form so the MFMA accumulators stay in VGPRs.
#include "qmv_quad.cuh"

#if !defined(MQ_INST_DT) || !defined(MQ_INST_BITS)
#error "compile with -DMQ_INST_DT=<0|1> -DMQ_INST_BITS=<4|8>"
#endif

namespace mq {

template struct QuadLaunch<MQ_INST_DT, MQ_INST_BITS, 32>;
template struct QuadLaunch<MQ_INST_DT, MQ_INST_BITS, 64>;
template struct QuadLaunch<MQ_INST_DT, MQ_INST_BITS, 128>;

}  // namespace mq
