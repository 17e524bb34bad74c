"""Head-aligned Q/K projection, per-head RMSNorm and split-half RoPE on MI355X.

Drop-in mirror of the reference's ``qk_rope`` module (src/m5kernels/qk_rope.py:24-203): same
function names, signatures, defaults and exception types.  Boundaries: BF16 projection, FP32
RMS / gamma / RoPE, BF16 head-major output [heads, M, 128]; no BF16 norm intermediate.

``tile=(TM, TN, groups, swizzle)`` and ``threads`` are validated as in the reference (they
named Apple threadgroup shapes); the gfx950 kernels always use a 256-row x 2-head MFMA tile
and 16-lane groups per (row, head).
"""

from __future__ import annotations

import math
import struct

import torch

from . import _lib
from .hip import gemm, splitk_plan

HEAD_DIM = 128


def _epsilon(epsilon):
    if not _lib.is_real(epsilon) or not math.isfinite(epsilon) or epsilon <= 0:
        raise ValueError("epsilon must be a positive finite real scalar")
    try:
        value = struct.unpack("=f", struct.pack("=f", float(epsilon)))[0]
    except OverflowError:
        raise ValueError("epsilon must remain finite and positive in float32") from None
    if not math.isfinite(value) or value <= 0:
        raise ValueError("epsilon must remain finite and positive in float32")
    return value


def _validate_norm(m, n, gamma, cos, sin, epsilon):
    if m <= 0 or n <= 0 or n % HEAD_DIM:
        raise ValueError("projection must have nonempty [M,N] shape with whole 128-wide heads")
    if tuple(gamma.shape) != (HEAD_DIM,) or gamma.dtype != torch.bfloat16:
        raise ValueError("gamma must be a shared bfloat16 vector of length 128")
    if cos.dim() != 2 or cos.shape[0] != m or not 1 <= cos.shape[1] <= HEAD_DIM // 2:
        raise ValueError("cos must have shape [M,rope_half] with rope_half in [1,64]")
    if sin.shape != cos.shape or cos.dtype != torch.bfloat16 or sin.dtype != torch.bfloat16:
        raise ValueError("cos and sin must have matching bfloat16 [M,rope_half] shapes")
    return cos.shape[1], _epsilon(epsilon)


def _validate_tile(tile):
    if not isinstance(tile, (tuple, list)) or len(tile) != 4:
        raise ValueError("tile must contain TM, TN, SIMD groups and M swizzle")
    if any(not _lib.is_int(v) for v in tile):
        raise ValueError("tile entries must be integers")
    tm, tn, groups, swizzle = map(int, tile)
    if tm not in (16, 32, 64, 128) or tn not in (64, 128) or groups not in (4, 8):
        raise NotImplementedError("supported tiles have TM16/32/64/128, TN64/128 and 4/8 SIMD groups")
    if swizzle <= 0:
        raise ValueError("M swizzle must be positive")
    return tm, tn, groups, swizzle


def _tables(gamma, cos, sin):
    return (_lib.aligned_device_tensor(gamma, "gamma"), _lib.device_tensor(cos, "cos"), _lib.device_tensor(sin, "sin"))


def projection_qk_rope(
    a,
    b,
    gamma,
    cos,
    sin,
    mode="int8",
    tile=(32, 128, 4, 1),
    *,
    a_scales=None,
    b_scales=None,
    epsilon=1e-5,
):
    """Return BF16 [heads, M, 128] Q or K after projection, RMSNorm and RoPE
    (qk_rope.py:120-182).  A[M,K], B[N,K] INT8 with FP32 scales a_scales[M], b_scales[N],
    or BF16 when mode="bf16"; gamma BF16[128]; cos/sin BF16[M,R] rotate (d, d+R) for d < R."""
    if mode not in ("int8", "bf16"):
        raise NotImplementedError("Q/K projection fusion supports INT8 or BF16 only")
    if a.dim() != 2 or b.dim() != 2 or not all(a.shape) or not all(b.shape):
        raise ValueError("A and B must be nonempty matrices")
    m, k = a.shape
    n, kb = b.shape
    if k != kb:
        raise ValueError("K mismatch")
    expected = torch.int8 if mode == "int8" else torch.bfloat16
    if a.dtype != expected or b.dtype != expected:
        raise ValueError(f"A and B must both have {mode} dtype")
    if mode == "int8":
        if k > 131071:
            raise NotImplementedError("INT32 worst-case overflow bound exceeded for signed INT8")
        if (
            a_scales is None
            or b_scales is None
            or tuple(a_scales.shape) != (m,)
            or tuple(b_scales.shape) != (n,)
            or a_scales.dtype != torch.float32
            or b_scales.dtype != torch.float32
        ):
            raise ValueError("INT8 requires float32 a_scales[M] and b_scales[N]")
    elif a_scales is not None or b_scales is not None:
        raise ValueError("BF16 projection does not accept quantization scales")
    rope_half, eps32 = _validate_norm(m, n, gamma, cos, sin, epsilon)
    _validate_tile(tile)
    if mode == "int8" and splitk_plan(m, n, k) > 1:
        # Few output tiles (short M): the split-K W8A8 projection to BF16, then the staged
        # postprocess.  Both are the fused kernel's arithmetic, so the bits are the same.
        projected = gemm(a, b, "int8", a_scales=a_scales, b_scales=b_scales, output_dtype=torch.bfloat16)
        return qk_norm_rope(projected, gamma, cos, sin, epsilon=epsilon)
    epsilon = eps32
    a = _lib.device_tensor(a, "a")
    b = _lib.device_tensor(b, "b")
    gamma, cos, sin = _tables(gamma, cos, sin)
    y = torch.empty((n // HEAD_DIM, m, HEAD_DIM), dtype=torch.bfloat16, device=a.device)
    if mode == "int8":
        a_scales = _lib.device_tensor(a_scales, "a_scales")
        b_scales = _lib.device_tensor(b_scales, "b_scales")
    _lib.call(
        "m5k_projection_qk_rope",
        _lib.ptr(a), _lib.ptr(b), _lib.dtype_code(a), m, n, k, _lib.ptr(a_scales), _lib.ptr(b_scales),
        _lib.ptr(gamma), _lib.ptr(cos), _lib.ptr(sin), int(rope_half), float(epsilon), _lib.ptr(y), _lib.stream_of(a),
    )
    return y


def qk_norm_rope(projected, gamma, cos, sin, *, epsilon=1e-5, threads=128):
    """Standalone postprocess BF16[M,N] -> BF16[heads, M, 128] (qk_rope.py:185-203)."""
    if projected.dim() != 2 or projected.dtype != torch.bfloat16:
        raise ValueError("projected must be a bfloat16 [M,N] matrix")
    m, n = projected.shape
    rope_half, epsilon = _validate_norm(m, n, gamma, cos, sin, epsilon)
    if not _lib.is_int(threads):
        raise ValueError("threads must be an integer")
    if threads not in (128, 256):
        raise NotImplementedError("standalone Q/K normalization supports 128 or 256 threads")
    projected = _lib.aligned_device_tensor(projected, "projected")
    gamma, cos, sin = _tables(gamma, cos, sin)
    y = torch.empty((n // HEAD_DIM, m, HEAD_DIM), dtype=torch.bfloat16, device=projected.device)
    _lib.call(
        "m5k_qk_norm_rope",
        _lib.ptr(projected), m, n, _lib.ptr(gamma), _lib.ptr(cos), _lib.ptr(sin), int(rope_half), float(epsilon),
        _lib.ptr(y), _lib.stream_of(projected),
    )
    return y


def projection_qkv_rope(a, w, q_gamma, k_gamma, cos, sin, mode="int8", *, a_scales=None, w_scales=None,
                        epsilon=1e-6):
    """Grouped Q/K/V projection in the H3 runtime's native layout (integrations/h3/
    qkv_candidate.metal, qkv_reference.h:15-35): W rows [heads, 3, 128] ordered Q, K, V per head.

    Returns BF16 (Q, K, V), each [heads, M, 128].  Q and K get the per-head RMSNorm (q_gamma /
    k_gamma) and split-half RoPE of projection_qk_rope; V is the BF16-rounded projection."""
    if mode not in ("int8", "bf16"):
        raise NotImplementedError("grouped Q/K/V projection supports INT8 or BF16 only")
    if a.dim() != 2 or w.dim() != 2 or not all(a.shape) or not all(w.shape):
        raise ValueError("A and W must be nonempty matrices")
    m, k = a.shape
    n, kw = w.shape
    if k != kw:
        raise ValueError("K mismatch")
    if n % (3 * HEAD_DIM):
        raise ValueError("W must have heads*3*128 rows ordered [head][Q,K,V][channel]")
    heads = n // (3 * HEAD_DIM)
    expected = torch.int8 if mode == "int8" else torch.bfloat16
    if a.dtype != expected or w.dtype != expected:
        raise ValueError(f"A and W must both have {mode} dtype")
    if mode == "int8":
        if k > 131071:
            raise NotImplementedError("INT32 worst-case overflow bound exceeded for signed INT8")
        if (a_scales is None or w_scales is None or tuple(a_scales.shape) != (m,) or tuple(w_scales.shape) != (n,)
                or a_scales.dtype != torch.float32 or w_scales.dtype != torch.float32):
            raise ValueError("INT8 requires float32 a_scales[M] and w_scales[heads*384]")
    elif a_scales is not None or w_scales is not None:
        raise ValueError("BF16 projection does not accept quantization scales")
    rope_half, epsilon = _validate_norm(m, n, q_gamma, cos, sin, epsilon)
    if tuple(k_gamma.shape) != (HEAD_DIM,) or k_gamma.dtype != torch.bfloat16:
        raise ValueError("k_gamma must be a shared bfloat16 vector of length 128")
    a = _lib.device_tensor(a, "a")
    w = _lib.device_tensor(w, "w")
    q_gamma, cos, sin = _tables(q_gamma, cos, sin)
    k_gamma = _lib.aligned_device_tensor(k_gamma, "k_gamma")
    q, kk, v = (torch.empty((heads, m, HEAD_DIM), dtype=torch.bfloat16, device=a.device) for _ in range(3))
    if mode == "int8":
        a_scales = _lib.device_tensor(a_scales, "a_scales")
        w_scales = _lib.device_tensor(w_scales, "w_scales")
    _lib.call(
        "m5k_projection_qkv_rope",
        _lib.ptr(a), _lib.ptr(w), _lib.dtype_code(a), m, heads, k, _lib.ptr(a_scales), _lib.ptr(w_scales),
        _lib.ptr(q_gamma), _lib.ptr(k_gamma), _lib.ptr(cos), _lib.ptr(sin), int(rope_half), float(epsilon),
        _lib.ptr(q), _lib.ptr(kk), _lib.ptr(v), _lib.stream_of(a),
    )
    return q, kk, v
