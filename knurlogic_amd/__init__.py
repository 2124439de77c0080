"""knurlogic_amd: the reference's quantized-weight hot path on MI355X.

Drop-in torch-tensor mirrors of mlx's quantized ops and of the module
classes that call them, backed by hand-written gfx950 HIP kernels behind a
C ABI (include/knurlogic_amd.h, libknurlogic_amd.so).
"""
from .ops import (ROUND_FUSED, ROUND_OP_BY_OP, add_bias, dequantize, gather_qmm, linear, moe_combine, moe_experts,
                  moe_route, moe_shared_add, quantize, quantized_matmul, swiglu, switch_glu, switch_glu_mx,
                  vq_experts, vq_gather_qmm, vq_glu, vq_packed_experts, vq_packed_switch_glu, vq_switch_glu)

__all__ = ["quantize", "dequantize", "quantized_matmul", "gather_qmm", "moe_route", "swiglu",
           "moe_combine", "moe_shared_add", "switch_glu", "switch_glu_mx", "vq_gather_qmm", "vq_glu", "vq_switch_glu",
           "vq_packed_switch_glu", "vq_experts", "vq_packed_experts",
           "linear", "add_bias", "moe_experts", "ROUND_OP_BY_OP", "ROUND_FUSED"]
