"""m5kernels_amd: the quantized projection hot path of m5-max-kernels on MI355X (gfx950).

Python op contracts mirror the reference package ``m5kernels`` (quantize, gemm, rotate,
...) on torch tensors; every computation runs in libm5k.so, hand-written HIP kernels
behind a C ABI (include/m5k.h).  There is no CPU fallback.
"""

from .hip import gemm, gemm_i8_accumulators, quantize
from .qk_rope import projection_qk_rope, projection_qkv_rope, qk_norm_rope
from .hadamard import SUPPORTED_BLOCK_SIZES, rotate, rotate_quantize
from .rms_quant import rms_quantize
from .chains import gate_chain, norm_shift_split_gemm, shift_split_condition
from .norm_hadamard import (
    fused_gated_residual_norm_hadamard_quantize,
    fused_norm_hadamard_quantize,
    gated_residual_add,
    unfused_norm,
)

__all__ = [
    "quantize",
    "gemm",
    "gemm_i8_accumulators",
    "rotate",
    "rotate_quantize",
    "SUPPORTED_BLOCK_SIZES",
    "fused_norm_hadamard_quantize",
    "fused_gated_residual_norm_hadamard_quantize",
    "gated_residual_add",
    "unfused_norm",
    "projection_qk_rope",
    "qk_norm_rope",
    "projection_qkv_rope",
    "rms_quantize",
    "gate_chain",
    "shift_split_condition",
    "norm_shift_split_gemm",
]
