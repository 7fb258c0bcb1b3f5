// Kernel instantiations of one (dtype, bits) pair for every group size.  The
// build compiles this file once per pair with -DMQ_INST_DT=<0|1> and
// -DMQ_INST_BITS=<4|8>, and once more per pair with -DMQ_INST_GLU for the
// fused gate+up kernels (decode, and prefill with SwiGLU), the folded
// down + combine kernel and the one-launch decode block; abi.hip calls the
// launchers through launch.h.
#include "launch.h"
#include "block.cuh"
#include "dequant.cuh"
#include "gather.cuh"
#include "qmm_wide.cuh"
#include "qmv.cuh"

#if !defined(MQ_INST_DT) || !defined(MQ_INST_BITS)
#error "compile with -DMQ_INST_DT=<0|1> -DMQ_INST_BITS=<4|8>"
#endif

namespace mq {

#ifdef MQ_INST_GLU
#define MQ_INST(GS)                                                  \
  template struct GluLaunch<MQ_INST_DT, MQ_INST_BITS, GS>;           \
  template struct GluRouteLaunch<MQ_INST_DT, MQ_INST_BITS, GS>;      \
  template struct GatherFoldLaunch<MQ_INST_DT, MQ_INST_BITS, GS>;   \
  template struct SwigluTablesLaunch<MQ_INST_DT, MQ_INST_BITS, GS>; \
  template struct MoeBlockLaunch<MQ_INST_DT, MQ_INST_BITS, GS>;
#else
#define MQ_INST(GS)                                                  \
  template struct DequantLaunch<MQ_INST_DT, MQ_INST_BITS, GS>;       \
  template struct SkinnyLaunch<MQ_INST_DT, MQ_INST_BITS, GS>;        \
  template struct WideLaunch<MQ_INST_DT, MQ_INST_BITS, GS>;          \
  template struct GatherLaunch<MQ_INST_DT, MQ_INST_BITS, GS>;
#endif

MQ_INST(32)
MQ_INST(64)
MQ_INST(128)

#undef MQ_INST

}  // namespace mq
