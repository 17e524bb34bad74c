"""Compositions of the hot-path ops that the reference's workloads time as one unit.

``shift_split_condition`` / ``norm_shift_split_gemm`` follow the norm-shift-split backend of
``norm_hadamard_gemm.prepare`` (src/m5kernels/norm_hadamard_gemm.py:20-45,233-258,430-484): the
AdaLN shift moves through the projection as a cached FP32 output bias, beta_p W^T of the original
weights, while (x * gamma (1 + alpha_p)) D H is quantized with the inverse RMS folded into the
row scale.  This is a different precision policy from the fused BF16-boundary prep (no
intermediate BF16 AdaLN round; the bias uses the original weights, the main GEMM the rotated
INT8 weights).

``gate_chain`` follows ``gate_epilogue_chain.prepare`` (src/m5kernels/gate_epilogue_chain.py:95-150):
previous W8A8 projection -> gated residual update -> AdaLN + H + INT8 -> next W8A8 projection,
with the gated update either in the previous GEMM's epilogue ("gate-in-gemm", metal.py:114-128)
or in the fused preparation ("gate-in-norm", norm_hadamard.py:198-265).  Both placements keep the
same BF16 boundaries (branch rounded to BF16, FP32 gate product and add, one BF16 cast of
R_next), so R_next, the INT8 codes and scales, and the next projection are bit-identical.
"""

from __future__ import annotations

import torch

from . import _lib
from .hip import gemm
from .norm_hadamard import fused_gated_residual_norm_hadamard_quantize, fused_norm_hadamard_quantize
from .rms_quant import rms_quantize

PLACEMENTS = ("gate-in-gemm", "gate-in-norm")
BIAS_BACKENDS = ("mlx-fp32-convert", "mpp-bf16-to-fp32")
_FLOATS = (torch.bfloat16, torch.float16, torch.float32)


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


def shift_split_condition(gamma, scale, shift, w, *, bias_backend="mlx-fp32-convert"):
    """Return the conditioning tables (combined, bias) of the shift-split projection
    (condition_prepare / bias_prepare, norm_hadamard_gemm.py:233-247,459-460).

    gamma [K]; scale and shift [K] (one conditioning row) or [P, K]; w the original [N, K]
    projection weights.  combined = float32(gamma) * (1 + float32(scale)) has scale's shape;
    bias = float32(shift) @ float32(w).T is [N] or [P, N], FP32-accumulated on the GPU.
    "mlx-fp32-convert" converts both operands to FP32 first; "mpp-bf16-to-fp32" reads the BF16
    operands directly.  BF16 x BF16 products are exact in FP32, so up to 8 conditioning rows
    (one wave-per-weight-row pass, same accumulation order) the two agree bit for bit; more rows
    run on the MFMA GEMM, whose FP32 and BF16 forms sum in different orders."""
    if bias_backend not in BIAS_BACKENDS:
        raise NotImplementedError("unsupported bias preparation backend")
    for name, t in (("gamma", gamma), ("scale", scale), ("shift", shift), ("w", w)):
        if not isinstance(t, torch.Tensor) or t.dtype not in _FLOATS:
            raise ValueError(f"{name} must be a floating-point tensor")
    if w.dim() != 2 or not all(w.shape):
        raise ValueError("w must have nonempty shape [N,K]")
    n, k = w.shape
    if tuple(gamma.shape) != (k,):
        raise ValueError("gamma must have shape [K]")
    if scale.shape != shift.shape or scale.dim() not in (1, 2) or scale.shape[-1] != k or not scale.numel():
        raise ValueError("scale and shift must both have shape [K] or [P,K]")
    if gamma.dtype != scale.dtype:
        raise ValueError("gamma and scale must share a dtype")
    rows = 1 if scale.dim() == 1 else scale.shape[0]
    if bias_backend == "mpp-bf16-to-fp32":
        if shift.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
            raise ValueError("mpp-bf16-to-fp32 needs bfloat16 shift and weights")
    else:
        shift, w = shift.float(), w.float()
    gamma = _lib.aligned_device_tensor(gamma, "gamma")
    scale = _lib.aligned_device_tensor(scale, "scale")
    shift = _lib.aligned_device_tensor(shift, "shift")
    w = _lib.aligned_device_tensor(w, "w")
    combined = torch.empty((rows, k), dtype=torch.float32, device=w.device)
    bias = torch.empty((rows, n), dtype=torch.float32, device=w.device)
    _lib.call(
        "m5k_shift_split_condition",
        _lib.ptr(gamma), _lib.ptr(scale), _lib.dtype_code(scale), _lib.ptr(shift), _lib.ptr(w), _lib.dtype_code(w),
        rows, k, n, _lib.ptr(combined), _lib.ptr(bias), _lib.stream_of(w),
    )
    if scale.dim() == 1:
        return combined[0], bias[0]
    return combined, bias


def norm_shift_split_gemm(x, w_q, w_scales, signs, combined, bias, block_size=256, *, norm="rms", epsilon=1e-5,
                          round_output="fp32", passes="one_read", threads=256):
    """BF16 [M, N] = W8A8(rms_quantize((x * combined) D H, folded inverse RMS), rotated INT8 weights)
    + bias in the GEMM epilogue, for one conditioning row (online stage of the norm-shift-split
    backend, norm_hadamard_gemm.py:238-247,430-442).  Requires RMS, round_output="fp32" and
    passes="one_read" as the reference does (:39-44)."""
    if norm != "rms" or round_output != "fp32":
        raise NotImplementedError("shift splitting requires RMS and round_output=fp32")
    if passes != "one_read":
        raise NotImplementedError("shift splitting supports only passes=one_read")
    q, s = rms_quantize(x, combined, signs, block_size, threads=threads, fold_scale=True, epsilon=epsilon)
    return gemm(q, w_q, "int8", a_scales=s, b_scales=w_scales, output_dtype=torch.bfloat16, bias=bias)
