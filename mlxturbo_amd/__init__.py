"""mlxturbo_amd: MI355X-native (gfx950) quantized-matmul hot path of mlxturbo.

Drop-in operators with MLX's signatures over PyTorch-ROCm tensors, backed by
hand-written HIP kernels behind a C ABI (``include/mlxturbo_amd.h``):

* :func:`quantized_matmul` - decode (M=1), verify (M=2..16) and prefill widths
* :func:`gather_qmm`       - MoE expert gather
* :func:`dequantize`       - bit-exact MLX affine dequantization (every width)
* :func:`quantize`         - MLX affine quantization (``mx.quantize``)
* :func:`gather_glu`       - fused MoE gate+up+SiLU at decode widths
* :func:`moe_combine`      - MoE unsort + router weight + top-k sum epilogue
  (optionally merging the shared expert)
* :func:`gather_qmm_combine` - MoE down projection with the combine folded in
  (one kernel at decode widths)
* :func:`moe_route`        - MoE top-k routing with softmax weights and the
  shared-expert gate

Module level (:mod:`mlxturbo_amd.nn`, :mod:`mlxturbo_amd.dispatch`): torch
``QuantizedLinear`` / ``QuantizedSwitchLinear`` / ``SwitchGLU`` on MLX-format
tensors, and the reference's shape-by-M route table with per-instance and
class-level enabling.  :mod:`mlxturbo_amd.checkpoint` builds those modules
from MLX safetensors checkpoints; :mod:`mlxturbo_amd.rebit` re-quantizes loaded
layers to another width (dequantize + quantize on the GPU).
"""

from . import checkpoint, dispatch, nn, rebit
from .ops import (dequantize, gather_glu, gather_qmm, gather_qmm_combine, launch_count,
                  moe_combine, moe_route, quantize, quantized_matmul, row_identity,
                  set_row_identity)

__version__ = "0.2.0"

__all__ = ["checkpoint", "rebit", "dequantize", "dispatch", "gather_glu", "gather_qmm",
           "gather_qmm_combine", "launch_count",
           "moe_combine", "moe_route",
           "nn", "quantize", "quantized_matmul", "row_identity", "set_row_identity",
           "__version__"]
