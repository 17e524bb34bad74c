"""Compositions of the hot-path ops that the reference's workloads time as one unit.

``gate_chain`` follows ``gate_epilogue_chain.prepare`` (src/m5kernels/gate_epilogue_chain.py:95-150):
previous W8A8 projection -> gated residual update -> AdaLN + H + INT8 -> next W8A8 projection,
with the gated update either in the previous GEMM's epilogue ("gate-in-gemm", metal.py:114-128)
or in the fused preparation ("gate-in-norm", norm_hadamard.py:198-265).  Both placements keep the
same BF16 boundaries (branch rounded to BF16, FP32 gate product and add, one BF16 cast of
R_next), so R_next, the INT8 codes and scales, and the next projection are bit-identical.
"""

from __future__ import annotations

import torch

from .hip import gemm
from .norm_hadamard import fused_gated_residual_norm_hadamard_quantize, fused_norm_hadamard_quantize

PLACEMENTS = ("gate-in-gemm", "gate-in-norm")


def gate_chain(q, s, w0, s0, w1, s1, residual, gate, gamma, scale, shift, signs, *, placement="gate-in-gemm",
               block_size=256, norm="rms", epsilon=1e-5):
    """Return (next projection BF16 [M, N], updated residual BF16 [M, H]).

    q, s: the previous projection's INT8 activation and row scales [M, PK], [M]; w0, s0: previous
    INT8 weights [H, PK] and scales [H]; w1, s1: next weights [N, H] and scales [N]; residual
    BF16 [M, H]; gate BF16 [H]; gamma/scale/shift/signs: the AdaLN + Hadamard tables of
    fused_norm_hadamard_quantize."""
    if placement not in PLACEMENTS:
        raise NotImplementedError("gate chain uses gate-in-norm/gate-in-gemm with INT8")
    bf = torch.bfloat16
    if placement == "gate-in-gemm":
        r_next = gemm(q, w0, "int8", a_scales=s, b_scales=s0, output_dtype=bf, residual=residual, gate=gate)
        qn, sn = fused_norm_hadamard_quantize(r_next, gamma, scale, shift, signs, block_size, norm=norm,
                                              epsilon=epsilon)
    else:
        branch = gemm(q, w0, "int8", a_scales=s, b_scales=s0, output_dtype=bf)
        qn, sn, r_next = fused_gated_residual_norm_hadamard_quantize(residual, branch, gate, gamma, scale, shift,
                                                                     signs, block_size, norm=norm, epsilon=epsilon)
    return gemm(qn, w1, "int8", a_scales=sn, b_scales=s1, output_dtype=bf), r_next
