"""CPU oracle for the quantized projection hot path (NumPy float64 + the C restatement).

TEST INFRASTRUCTURE ONLY: this module is the checker, never the product.  It may be
imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.  The
product path (m5kernels_amd -> libm5k.so) never imports it and has no CPU fallback.

Two layers:

* NumPy restatements of the reference's independent references (float64 between
  explicit BF16 boundaries, FP32 where the reference computes in FP32).  Each function
  cites the reference definition it restates (paths relative to the reference repo).
* ``c_*`` wrappers of liboracle.so (oracle/m5k_oracle.c): the same arithmetic in FP32
  with a fixed evaluation order, used for bit-exact comparisons at scale.

Parity status of each function, and the check that pins it, is listed in
tests/test_oracle.py (every function here has at least one pinning test).
"""

from __future__ import annotations

import ctypes
import math
import numbers
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
C_LIB_PATH = HERE / "liboracle.so"

# ----------------------------------------------------------------------------------------
# BF16 helpers
# ----------------------------------------------------------------------------------------


def f32_to_bf16_bits(x) -> np.ndarray:
    """FP32 -> BF16 round-to-nearest-even bits of an FP32 producer
    (qk_rope_reference.py:37-42 formula: (bits + 0x7FFF + ((bits >> 16) & 1)) >> 16)."""
    bits = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rounded = bits + np.uint32(0x7FFF) + ((bits >> np.uint32(16)) & np.uint32(1))
    return (rounded >> np.uint32(16)).astype(np.uint16)


def bf16_bits_to_f32(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def bf16_round_f32(x) -> np.ndarray:
    """FP32 values after a BF16 round trip (the ``O(...)`` cast of the Metal kernels)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


def _finite(value, name):
    value = np.asarray(value)
    if np.iscomplexobj(value):
        raise ValueError(f"{name} must be real")
    value = np.asarray(value, dtype=np.float64)
    if not np.isfinite(value).all():
        raise ValueError(f"{name} must be finite")
    return value


def bf16_round_reference(value):
    """FP32 producer then BF16 nearest-even, decoded to float64 (qk_rope_reference.py:24-42).

    Rejects inputs that overflow FP32 or BF16; keeps signed zeros and subnormals."""
    value = _finite(value, "BF16 input")
    with np.errstate(over="ignore", invalid="ignore"):
        fp32 = np.array(value, dtype=np.float32, order="C", copy=True)
    if not np.isfinite(fp32).all():
        raise ValueError("BF16 input exceeds finite FP32 range")
    out = bf16_bits_to_f32(f32_to_bf16_bits(fp32)).astype(np.float64).reshape(fp32.shape)
    if not np.isfinite(out).all():
        raise ValueError("BF16 rounding exceeds finite BF16 range")
    return out


# ----------------------------------------------------------------------------------------
# FP8 E4M3 and the per-row quantizer (numerics.py:6-54)
# ----------------------------------------------------------------------------------------


def fp8_decode(q) -> np.ndarray:
    """OCP E4M3 decode, NaN only for exponent 15 / mantissa 7 (numerics.py:6-14)."""
    q = np.asarray(q, dtype=np.uint8)
    exponent = ((q >> 3) & 15).astype(np.int32)
    mantissa = (q & 7).astype(np.float64)
    magnitude = np.where(
        exponent == 0, mantissa * 2.0**-9, (1.0 + mantissa / 8.0) * np.exp2(exponent - 7)
    )
    value = np.where(q & 128, -magnitude, magnitude)
    value = np.where((exponent == 15) & (mantissa == 7), np.nan, value)
    return value.astype(np.float32)


_FP8_POSITIVE = None


def fp8_encode(x) -> np.ndarray:
    """Nearest positive finite E4M3 code (ties to the even code), |x| saturated at 448,
    sign bit from signbit(x) (numerics.py:17-26)."""
    global _FP8_POSITIVE
    if _FP8_POSITIVE is None:
        _FP8_POSITIVE = fp8_decode(np.arange(127, dtype=np.uint8))
    table = _FP8_POSITIVE
    x = np.asarray(x, dtype=np.float32)
    mag = np.minimum(np.abs(x), np.float32(448.0))
    upper = np.minimum(np.searchsorted(table, mag, side="left"), 126)
    lower = np.maximum(upper - 1, 0)
    below = mag - table[lower]
    above = table[upper] - mag
    pick_lower = (below < above) | ((below == above) & (lower % 2 == 0))
    code = np.where(pick_lower, lower, upper).astype(np.uint8)
    return code | np.where(np.signbit(x), np.uint8(128), np.uint8(0))


def mx_exponent(peak):
    """MXINT8 block exponent (numerics.py:36-38): floor of the FP32 log2 of the block peak, minus
    6, clamped to [-127, 127]; 0 for an all-zero block.  The FP32 log2 rounds to nearest, so a
    peak just below 2**k gives k (floor(log2) of the rounded value), as numpy's float32 log2 does."""
    peak = np.asarray(peak, dtype=np.float32)
    safe = np.maximum(peak, np.finfo(np.float32).tiny)
    e = np.clip(np.floor(np.log2(safe.astype(np.float64)).astype(np.float32)) - 6, -127, 127)
    return np.where(peak == 0, np.float32(0), e).astype(np.float32)


def quantize_reference(x, mode):
    """Quantizer in FP32 (numerics.py:29-46).

    int8 / fp8: per row, peak = max|x|; scale = 1 if peak == 0 else peak / 127 (or 448);
    z = x / scale; int8 -> clip(rint(z), -127, 127); fp8 -> fp8_encode(z).
    mxint8: per 32-element block, e = mx_exponent(peak); codes clip(rint(x / 2**e), -127, 127);
    scales uint8 e + 127 of shape [rows, K/32].  Rejects non-finite input."""
    x = np.asarray(x, dtype=np.float32)
    if not np.isfinite(x).all():
        raise ValueError("quantization input must be finite")
    if mode == "mxint8":
        if x.shape[-1] % 32:
            raise ValueError("K must be divisible by 32")
        z = x.reshape(*x.shape[:-1], -1, 32)
        e = mx_exponent(np.max(np.abs(z), axis=-1, keepdims=True))
        q = np.clip(np.rint(z / np.exp2(e)), -127, 127).astype(np.int8)
        return q.reshape(x.shape), (e[..., 0] + 127).astype(np.uint8)
    if mode not in ("int8", "fp8"):
        raise ValueError(f"unsupported mode {mode!r}")
    peak = np.max(np.abs(x), axis=-1, keepdims=True)
    divisor = np.float32(448.0 if mode == "fp8" else 127.0)
    scale = np.where(peak == 0, np.float32(1.0), peak / divisor).astype(np.float32)
    z = (x / scale).astype(np.float32)
    if mode == "fp8":
        q = fp8_encode(z)
    else:
        q = np.clip(np.rint(z), -127, 127).astype(np.int8)
    return q, scale[..., 0]


def dequantize(q, s, mode):
    """Decoded FP32 values (numerics.py:49-54): codes * row scale, or for mxint8 codes * 2**(s - 127)
    per 32-element block."""
    if mode == "mxint8":
        q = np.asarray(q)
        z = q.reshape(*q.shape[:-1], -1, 32).astype(np.float32)
        return (z * np.exp2(np.asarray(s).astype(np.int32) - 127).astype(np.float32)[..., None]).reshape(q.shape)
    z = fp8_decode(q) if mode == "fp8" else np.asarray(q).astype(np.float32)
    return z * np.asarray(s, dtype=np.float32)[..., None]


def metrics(actual, reference):
    """relative_l2 / max_abs / rmse / cosine in float64 (numerics.py:57-75)."""
    a = np.asarray(actual, dtype=np.float64)
    r = np.asarray(reference, dtype=np.float64)
    if a.shape != r.shape:
        raise ValueError("reference shape mismatch")
    if not (np.isfinite(a).all() and np.isfinite(r).all()):
        return {"finite": False, "relative_l2": None, "max_abs": None, "rmse": None, "cosine": None}
    diff = a - r
    rn, an = np.linalg.norm(r), np.linalg.norm(a)
    cosine = float(np.dot(a.ravel(), r.ravel()) / max(rn * an, 1e-30)) if rn else float(an == 0)
    return {
        "finite": True,
        "relative_l2": float(np.linalg.norm(diff) / max(rn, 1e-30)),
        "max_abs": float(np.max(np.abs(diff))) if diff.size else 0.0,
        "rmse": float(np.sqrt(np.mean(diff**2))) if diff.size else 0.0,
        "cosine": cosine,
    }


def sample_indices(length, count=32):
    """Evenly spaced unique sample rows/cols (numerics.py:78-79)."""
    return np.unique(np.linspace(0, length - 1, min(length, count), dtype=int))


# ----------------------------------------------------------------------------------------
# Block Hadamard (hadamard_reference.py:19-68)
# ----------------------------------------------------------------------------------------


def _positive_int(value, name):
    if isinstance(value, bool) or not isinstance(value, numbers.Integral) or value <= 0:
        raise ValueError(f"{name} must be a positive integer")
    return int(value)


def hadamard_signs(k, seed):
    """Shared +-1 int8 signs from PCG64(seed) bits (hadamard_reference.py:19-23)."""
    k = _positive_int(k, "K")
    bits = np.random.Generator(np.random.PCG64(seed)).integers(0, 2, size=k, dtype=np.int8)
    return (bits * 2 - 1).astype(np.int8)


def block_hadamard_reference(x, block_size, signs=None):
    """float64 X D H with normalized block-diagonal Sylvester H (hadamard_reference.py:26-68).

    The 1/sqrt(B) normalization is applied before the butterflies, as in the reference."""
    block_size = _positive_int(block_size, "block_size")
    if block_size & (block_size - 1):
        raise ValueError("block_size must be a power of two")
    x = np.asarray(x)
    if x.ndim != 2 or not all(x.shape):
        raise ValueError("input must have nonempty shape [rows, K]")
    if np.iscomplexobj(x):
        raise ValueError("input must be real")
    if x.shape[1] % block_size:
        raise ValueError("K must be divisible by block_size")
    out = np.array(x, dtype=np.float64, order="C", copy=True)
    if not np.isfinite(out).all():
        raise ValueError("input must be finite")
    if signs is not None:
        signs = np.asarray(signs)
        if signs.shape != (x.shape[1],) or np.iscomplexobj(signs):
            raise ValueError("signs must be a real vector of length K")
        if not np.isin(signs, [-1, 1]).all():
            raise ValueError("signs must contain only -1 and +1")
        out *= signs
    out /= math.sqrt(block_size)
    view = out.reshape(-1, block_size)
    half = 1
    with np.errstate(over="ignore", invalid="ignore"):
        while half < block_size:
            pairs = view.reshape(view.shape[0], -1, 2, half)
            lo = pairs[:, :, 0, :].copy()
            hi = pairs[:, :, 1, :].copy()
            pairs[:, :, 0, :] = lo + hi
            pairs[:, :, 1, :] = lo - hi
            half *= 2
    if not np.isfinite(out).all():
        raise ValueError("transform output exceeds finite float64 range")
    return out


# ----------------------------------------------------------------------------------------
# Norm / modulation / gated residual (norm_hadamard_reference.py:24-94,
# gated_residual_reference.py:21-60)
# ----------------------------------------------------------------------------------------


def norm_modulate_reference(x, gamma, scale, shift, *, norm="rms", eps=1e-5):
    """float64 norm(X) * gamma * (1 + scale) + shift (norm_hadamard_reference.py:24-64).

    RMS: x / sqrt(mean(x^2) + eps).  LayerNorm: centred, population variance."""
    if norm not in ("rms", "layer"):
        raise ValueError("norm must be 'rms' or 'layer'")
    if isinstance(eps, bool) or not isinstance(eps, numbers.Real) or not np.isfinite(eps) or eps <= 0:
        raise ValueError("eps must be a positive finite real scalar")
    x = _finite(x, "input")
    if x.ndim != 2 or not all(x.shape):
        raise ValueError("input must have nonempty shape [rows, K]")
    vecs = []
    for value, name in ((gamma, "gamma"), (scale, "scale"), (shift, "shift")):
        value = _finite(value, name)
        if value.shape != (x.shape[1],):
            raise ValueError(f"{name} must have shape [K]")
        vecs.append(value)
    gamma, scale, shift = vecs
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        if norm == "layer":
            # Subtract the first element before the mean so constant rows centre exactly.
            centred = x - x[:, :1]
            centred = centred - centred.mean(axis=1, keepdims=True)
        else:
            centred = x
        moment = np.mean(centred * centred, axis=1, keepdims=True)
        y = centred / np.sqrt(moment + float(eps)) * gamma * (1.0 + scale) + shift
    if not (np.isfinite(moment).all() and np.isfinite(y).all()):
        raise ValueError("normalization or modulation exceeds finite float64 range")
    return y


def norm_hadamard_quantize_reference(x, gamma, scale, shift, block_size, signs=None, *, norm="rms", eps=1e-5):
    """Ideal stages norm/modulate -> X D H -> per-row INT8 (norm_hadamard_reference.py:67-94)."""
    modulated = norm_modulate_reference(x, gamma, scale, shift, norm=norm, eps=eps)
    rotated = block_hadamard_reference(modulated, block_size, signs)
    peak = np.max(np.abs(rotated), axis=1)
    scales = np.where(peak == 0, 1.0, peak / 127.0)
    if not (np.isfinite(scales).all() and np.all(scales > 0)):
        raise ValueError("INT8 scale exceeds finite positive float64 range")
    quantized = np.clip(np.rint(rotated / scales[:, None]), -127, 127).astype(np.int8)
    return {
        "modulated": modulated,
        "rotated": rotated,
        "quantized": quantized,
        "scales": scales,
        "dequantized": quantized.astype(np.float64) * scales[:, None],
    }


def gated_residual_reference(residual, branch, gate, *, row_map=None):
    """float64 residual + gate * branch, gate [K] or table [P,K] with int32 row_map
    (gated_residual_reference.py:21-60)."""
    residual = _finite(residual, "residual")
    branch = _finite(branch, "branch")
    gate = _finite(gate, "gate")
    if residual.ndim != 2 or not all(residual.shape):
        raise ValueError("residual must have nonempty shape [M,K]")
    if branch.shape != residual.shape:
        raise ValueError("branch must have the same shape as residual")
    rows, width = residual.shape
    if gate.ndim == 1:
        if gate.shape != (width,):
            raise ValueError("shared gate must have shape [K]")
        if row_map is not None:
            raise ValueError("row_map is only supported with a gate table")
        selected = gate
    elif gate.ndim == 2:
        if gate.shape[0] == 0 or gate.shape[1] != width:
            raise ValueError("gate table must have nonempty shape [P,K]")
        if row_map is None:
            raise ValueError("gate table requires row_map")
        row_map = np.asarray(row_map)
        if row_map.shape != (rows,) or row_map.dtype != np.dtype(np.int32):
            raise ValueError("row_map must be an int32 vector of length M")
        if np.any(row_map < 0) or np.any(row_map >= gate.shape[0]):
            raise ValueError("row_map indices must be in [0,P)")
        selected = gate[row_map]
    else:
        raise ValueError("gate must have shape [K] or [P,K]")
    with np.errstate(over="ignore", invalid="ignore"):
        out = residual + selected * branch
    if not np.isfinite(out).all():
        raise ValueError("gated residual exceeds finite float64 range")
    return out


# ----------------------------------------------------------------------------------------
# Q/K RMSNorm + split-half RoPE (qk_rope_reference.py:45-134)
# ----------------------------------------------------------------------------------------


def qk_rope_reference(projected, gamma, cos, sin, *, epsilon=1e-5, projection_bf16=True, norm_bf16=False,
                      output_bf16=True):
    """Per-(row, head) RMSNorm over D, gamma, RoPE on pairs (j, j+R), head-major output.

    projected [M,H,D]; gamma [D]; cos/sin [M,R] with 2R <= D.  float64 between the
    optional BF16 boundaries (projection, norm, output).  Returns the intermediates and
    the [H,M,D] output (qk_rope_reference.py:45-134)."""
    if isinstance(epsilon, bool) or not isinstance(epsilon, numbers.Real) or not np.isfinite(epsilon) or epsilon <= 0:
        raise ValueError("epsilon must be a positive finite real scalar")
    for name, flag in (("projection_bf16", projection_bf16), ("norm_bf16", norm_bf16), ("output_bf16", output_bf16)):
        if not isinstance(flag, (bool, np.bool_)):
            raise ValueError(f"{name} must be boolean")
    projected = _finite(projected, "projected")
    gamma = _finite(gamma, "gamma")
    cos = _finite(cos, "cos")
    sin = _finite(sin, "sin")
    if projected.ndim != 3 or not all(projected.shape):
        raise ValueError("projected must have nonempty shape [M,H,D]")
    rows, _, width = projected.shape
    if gamma.shape != (width,):
        raise ValueError("gamma must have shape [D]")
    if cos.ndim != 2 or cos.shape[0] != rows or cos.shape[1] * 2 > width:
        raise ValueError("cos must have shape [M,R] with 0 <= 2R <= D")
    if sin.shape != cos.shape:
        raise ValueError("sin must have the same shape as cos")
    if projection_bf16:
        projected = bf16_round_reference(projected)
    else:
        projected = np.array(projected, dtype=np.float64, order="C", copy=True)
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        moment = np.mean(projected * projected, axis=-1)
        inverse_rms = 1.0 / np.sqrt(moment + float(epsilon))
        normalized = projected * inverse_rms[..., None] * gamma
    if not (
        np.isfinite(moment).all()
        and np.isfinite(inverse_rms).all()
        and np.all(inverse_rms > 0)
        and np.isfinite(normalized).all()
    ):
        raise ValueError("RMS normalization exceeds finite float64 range")
    if norm_bf16:
        normalized = bf16_round_reference(normalized)
    half = cos.shape[1]
    rotated = normalized.copy()
    first = normalized[..., :half]
    second = normalized[..., half : 2 * half]
    c = cos[:, None, :]
    s = sin[:, None, :]
    with np.errstate(over="ignore", invalid="ignore"):
        rotated[..., :half] = first * c - second * s
        rotated[..., half : 2 * half] = second * c + first * s
    if not np.isfinite(rotated).all():
        raise ValueError("RoPE exceeds finite float64 range")
    output = bf16_round_reference(rotated) if output_bf16 else rotated
    return {
        "projected": projected,
        "inverse_rms": inverse_rms,
        "normalized": normalized,
        "rotated": rotated,
        "output": np.ascontiguousarray(output.transpose(1, 0, 2)),
    }


# ----------------------------------------------------------------------------------------
# liboracle.so (FP32 fixed-order restatement)
# ----------------------------------------------------------------------------------------

_C = None


def build_c(force: bool = False) -> Path:
    if force or not C_LIB_PATH.exists():
        subprocess.run(["make", "-s", "-C", str(HERE)] + (["-B"] if force else []), check=True)
    return C_LIB_PATH


def c_lib() -> ctypes.CDLL:
    global _C
    if _C is None:
        if not C_LIB_PATH.exists():
            build_c()
        lib = ctypes.CDLL(str(C_LIB_PATH))
        p, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        lib.oracle_bf16_bits.argtypes = [ctypes.c_float]
        lib.oracle_bf16_bits.restype = ctypes.c_uint16
        lib.oracle_fp8_encode.argtypes = [ctypes.c_float]
        lib.oracle_fp8_encode.restype = ctypes.c_uint8
        lib.oracle_fp8_decode.argtypes = [ctypes.c_uint8]
        lib.oracle_fp8_decode.restype = ctypes.c_float
        lib.oracle_inv_sqrt_block.argtypes = [i32]
        lib.oracle_inv_sqrt_block.restype = ctypes.c_float
        for name, args in {
            "oracle_bf16_round_array": [p, i64, p],
            "oracle_fp8_encode_array": [p, i64, p],
            "oracle_fp8_decode_array": [p, i64, p],
            "oracle_quantize_rows": [p, i64, i64, i32, p, p],
            "oracle_quantize_rows_bf16": [p, i64, i64, i32, p, p],
            "oracle_gemm_i8_acc": [p, p, i64, i64, i64, p],
            "oracle_i8_epilogue": [p, p, p, i64, i64, p, p, p, p, p, i32, p],
            "oracle_w8a8_linear_bf16": [p, p, p, i64, i64, i64, p, p, p],
            "oracle_hadamard_f32": [p, i64, i64, i32, p, p],
            "oracle_f16_round_array": [p, i64, p],
            "oracle_prep_rows": [p, i32, p, p, p, p, p, p, p, p, i64, i64, i32, i32, i32, ctypes.c_float, i32, p, p,
                                 p, p],
            "oracle_qk_norm_rope": [p, i64, i64, p, p, p, i32, ctypes.c_float, p],
            "oracle_qkv_norm_rope": [p, i64, i64, p, p, p, p, i32, ctypes.c_float, p, p, p],
        }.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = None
        _C = lib
    return _C


def _ptr(a):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


def c_quantize_rows(x, mode):
    """liboracle quantizer on FP32 or BF16-bit (uint16) input; returns (codes, scales)."""
    x = np.ascontiguousarray(x)
    rows, k = x.shape
    q = np.empty((rows, k), dtype=np.uint8 if mode == "fp8" else np.int8)
    s = np.empty(rows, dtype=np.float32)
    code = 1 if mode == "fp8" else 0
    if x.dtype == np.uint16:
        c_lib().oracle_quantize_rows_bf16(_ptr(x), rows, k, code, _ptr(q), _ptr(s))
    else:
        x = np.ascontiguousarray(x, dtype=np.float32)
        c_lib().oracle_quantize_rows(_ptr(x), rows, k, code, _ptr(q), _ptr(s))
    return q, s


def c_fp8_encode(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint8)
    c_lib().oracle_fp8_encode_array(_ptr(x), x.size, _ptr(out))
    return out


def c_gemm_i8_acc(a, b):
    a = np.ascontiguousarray(a, dtype=np.int8)
    b = np.ascontiguousarray(b, dtype=np.int8)
    m, k = a.shape
    n = b.shape[0]
    acc = np.empty((m, n), dtype=np.int32)
    c_lib().oracle_gemm_i8_acc(_ptr(a), _ptr(b), m, n, k, _ptr(acc))
    return acc


def c_i8_epilogue(acc, sa, sb, *, out="bf16", bias=None, bias_row_map=None, residual_bits=None, gate_bits=None,
                  gate_row_map=None):
    """FP32 epilogue of the W8A8 GEMM; out='bf16' returns uint16 bits, 'fp32' float32."""
    acc = np.ascontiguousarray(acc, dtype=np.int32)
    m, n = acc.shape
    sa = np.ascontiguousarray(sa, dtype=np.float32)
    sb = np.ascontiguousarray(sb, dtype=np.float32)
    conv = {
        "bias": None if bias is None else np.ascontiguousarray(bias, dtype=np.float32),
        "bias_map": None if bias_row_map is None else np.ascontiguousarray(bias_row_map, dtype=np.int32),
        "res": None if residual_bits is None else np.ascontiguousarray(residual_bits, dtype=np.uint16),
        "gate": None if gate_bits is None else np.ascontiguousarray(gate_bits, dtype=np.uint16),
        "gate_map": None if gate_row_map is None else np.ascontiguousarray(gate_row_map, dtype=np.int32),
    }
    result = np.empty((m, n), dtype=np.uint16 if out == "bf16" else np.float32)
    c_lib().oracle_i8_epilogue(
        _ptr(acc), _ptr(sa), _ptr(sb), m, n, _ptr(conv["bias"]), _ptr(conv["bias_map"]), _ptr(conv["res"]),
        _ptr(conv["gate"]), _ptr(conv["gate_map"]), 2 if out == "bf16" else 0, _ptr(result),
    )
    return result


def c_w8a8_linear_bf16(a_bits, wq, wscale):
    """The online W8A8 linear on the CPU: bf16 bits A -> uint16 bf16 bits C."""
    a_bits = np.ascontiguousarray(a_bits, dtype=np.uint16)
    wq = np.ascontiguousarray(wq, dtype=np.int8)
    wscale = np.ascontiguousarray(wscale, dtype=np.float32)
    m, k = a_bits.shape
    n = wq.shape[0]
    aq = np.empty((m, k), dtype=np.int8)
    sa = np.empty(m, dtype=np.float32)
    out = np.empty((m, n), dtype=np.uint16)
    c_lib().oracle_w8a8_linear_bf16(_ptr(a_bits), _ptr(wq), _ptr(wscale), m, n, k, _ptr(aq), _ptr(sa), _ptr(out))
    return out


def c_hadamard_f32(x, block, signs):
    x = np.ascontiguousarray(x, dtype=np.float32)
    signs = np.ascontiguousarray(signs, dtype=np.int8)
    rows, k = x.shape
    y = np.empty_like(x)
    c_lib().oracle_hadamard_f32(_ptr(x), rows, k, int(block), _ptr(signs), _ptr(y))
    return y


def rms_quantize_reference(x, gamma, signs=None, block_size=1, eps=1e-5):
    """float64 RMS INT8 encoding with the inverse RMS folded into the row scales
    (rms_quant_reference.py:24-89).

    Z = (X * gamma) D H, r = 1 / sqrt(mean(X^2) + eps) over the original X; for a nonzero row
    Q = clip(rint(Z / (max|Z| / 127)), -127, 127) and S = max|Z| / 127 * r; a zero row of Z gives
    Q = 0 and S = 1.  Returns a dict with the same keys as the reference."""
    if isinstance(eps, bool) or not isinstance(eps, (int, float, np.floating)) or not np.isfinite(eps) or eps <= 0:
        raise ValueError("eps must be a positive finite real scalar")
    x = np.asarray(x, dtype=np.float64)
    gamma = np.asarray(gamma, dtype=np.float64)
    if x.ndim != 2 or not all(x.shape):
        raise ValueError("input must have nonempty shape [M,K]")
    if gamma.shape != (x.shape[1],):
        raise ValueError("gamma must have shape [K]")
    if not (np.isfinite(x).all() and np.isfinite(gamma).all()):
        raise ValueError("input and gamma must be finite")
    inverse_rms = 1.0 / np.sqrt(np.mean(x * x, axis=1) + float(eps))
    unscaled = block_hadamard_reference(x * gamma, block_size, signs)
    peak = np.max(np.abs(unscaled), axis=1)
    nonzero = peak != 0
    unscaled_scales = np.where(nonzero, peak / 127.0, 1.0)
    scales = np.where(nonzero, unscaled_scales * inverse_rms, 1.0)
    quantized = np.clip(np.rint(unscaled / unscaled_scales[:, None]), -127, 127).astype(np.int8)
    return {
        "normalized_rotated": unscaled * inverse_rms[:, None],
        "quantized": quantized,
        "scales": scales,
        "dequantized": quantized.astype(np.float64) * scales[:, None],
        "unscaled_rotated": unscaled,
        "inverse_rms": inverse_rms,
        "unscaled_scales": unscaled_scales,
    }


# ----------------------------------------------------------------------------------------
# Fixed-order FP32 prep and Q/K epilogue (liboracle.so; the order is stated in m5k_oracle.c)
# ----------------------------------------------------------------------------------------

_DT_CODES = {"fp32": 0, "fp16": 1, "bf16": 2}


def c_f16_round(x):
    """FP32 values rounded to binary16 (nearest even) and back, by the C oracle."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    c_lib().oracle_f16_round_array(_ptr(x), x.size, _ptr(out))
    return out


def c_prep_rows(x, gamma, scale, shift, signs, block, *, dtype="bf16", norm="rms", eps=1e-5, round_output="input",
                row_map=None, branch=None, gate=None, gate_row_map=None, with_modulated=False):
    """Fused (gated) AdaLN / RMS prep in the fixed FP32 order of the library (norm_hadamard.py:
    122-265): returns (codes, scales) or (codes, scales, r_next FP32 values) when `branch` is given,
    plus the FP32 modulation before the O cast last when `with_modulated`.
    x, branch, gate, gamma, scale, shift are FP32 values (exact decodes of their storage dtypes);
    `dtype` names x's storage dtype (the R and O casts)."""
    f32 = lambda t: None if t is None else np.ascontiguousarray(t, dtype=np.float32)  # noqa: E731
    i32 = lambda t: None if t is None else np.ascontiguousarray(t, dtype=np.int32)  # noqa: E731
    x, branch, gate, gamma, scale, shift = map(f32, (x, branch, gate, gamma, scale, shift))
    signs = np.ascontiguousarray(signs, dtype=np.int8)
    rows, k = x.shape
    q = np.empty((rows, k), dtype=np.int8)
    s = np.empty(rows, dtype=np.float32)
    r_next = np.empty((rows, k), dtype=np.float32) if branch is not None else None
    modulated = np.empty((rows, k), dtype=np.float32) if with_modulated else None
    c_lib().oracle_prep_rows(
        _ptr(x), _DT_CODES[dtype], _ptr(branch), _ptr(gate), _ptr(i32(gate_row_map)), _ptr(gamma), _ptr(scale),
        _ptr(shift), _ptr(i32(row_map)), _ptr(signs), rows, k, int(block), max(8, int(block) // 64),
        1 if norm in ("layer", "layernorm") else 0, float(eps), 1 if round_output == "input" else 0, _ptr(q), _ptr(s),
        _ptr(r_next), _ptr(modulated))
    out = (q, s) if branch is None else (q, s, r_next)
    return out + (modulated,) if with_modulated else out


def c_qk_norm_rope(z_bits, gamma_bits, cos_bits, sin_bits, *, epsilon=1e-6):
    """Q/K epilogue in the library's FP32 order on a BF16 projection z [M, N] (uint16 bits):
    head-major [N/128, M, 128] BF16 bits (qk_rope_reference.py:45-134 order-fixed)."""
    z = np.ascontiguousarray(z_bits, dtype=np.uint16)
    m, n = z.shape
    cos_bits = np.ascontiguousarray(cos_bits, dtype=np.uint16)
    sin_bits = np.ascontiguousarray(sin_bits, dtype=np.uint16)
    rope_half = cos_bits.shape[1] if cos_bits.ndim == 2 else 0
    y = np.empty((n // 128, m, 128), dtype=np.uint16)
    c_lib().oracle_qk_norm_rope(_ptr(z), m, n, _ptr(np.ascontiguousarray(gamma_bits, dtype=np.uint16)),
                                _ptr(cos_bits), _ptr(sin_bits), rope_half, float(epsilon), _ptr(y))
    return y


def c_qkv_norm_rope(z_bits, q_gamma_bits, k_gamma_bits, cos_bits, sin_bits, *, epsilon=1e-6):
    """Grouped Q/K/V epilogue (weight rows [head, stream, 128]) on z [M, heads * 384] BF16 bits:
    (q, k, v) head-major [heads, M, 128] BF16 bits."""
    z = np.ascontiguousarray(z_bits, dtype=np.uint16)
    m, n = z.shape
    heads = n // 384
    cos_bits = np.ascontiguousarray(cos_bits, dtype=np.uint16)
    sin_bits = np.ascontiguousarray(sin_bits, dtype=np.uint16)
    outs = [np.empty((heads, m, 128), dtype=np.uint16) for _ in range(3)]
    c_lib().oracle_qkv_norm_rope(_ptr(z), m, heads, _ptr(np.ascontiguousarray(q_gamma_bits, dtype=np.uint16)),
                                 _ptr(np.ascontiguousarray(k_gamma_bits, dtype=np.uint16)), _ptr(cos_bits),
                                 _ptr(sin_bits), cos_bits.shape[1], float(epsilon), *map(_ptr, outs))
    return tuple(outs)


# ----------------------------------------------------------------------------------------
# oracle/_ref: the reference's own float64 grouped Q/K/V header (integrations/h3/
# qkv_reference.h), compiled where it lies by `make -C oracle ref`
# ----------------------------------------------------------------------------------------

REF_QKV_PATH = HERE / "_ref" / "libqkv_ref.so"
_REF_QKV = None


def ref_qkv_lib():
    """The compiled reference header, or None when oracle/_ref was not built."""
    global _REF_QKV
    if _REF_QKV is None and REF_QKV_PATH.exists():
        lib = ctypes.CDLL(str(REF_QKV_PATH))
        p, i64 = ctypes.c_void_p, ctypes.c_int64
        lib.ref_qkv_postprocess.argtypes = [p, i64, ctypes.c_uint, p, p, p, ctypes.c_double, p]
        lib.ref_qkv_postprocess.restype = None
        lib.ref_qkv_h256.argtypes = [p, ctypes.c_uint]
        lib.ref_qkv_h256.restype = None
        _REF_QKV = lib
    return _REF_QKV


def ref_qkv_postprocess(projection, stream, gamma_bits, cos_bits, sin_bits, epsilon):
    """qvr_postprocess (qkv_reference.h:17-35) over rows of float64 head projections [rows, 128]
    with rope half 48: BF16-rounded projection, float64 RMSNorm, gamma, RoPE, BF16 output
    (returned as float64 values)."""
    lib = ref_qkv_lib()
    projection = np.ascontiguousarray(projection, dtype=np.float64)
    rows = projection.shape[0]
    out = np.empty_like(projection)
    lib.ref_qkv_postprocess(_ptr(projection), rows, int(stream), _ptr(np.ascontiguousarray(gamma_bits, np.uint16)),
                            _ptr(np.ascontiguousarray(cos_bits, np.uint16)),
                            _ptr(np.ascontiguousarray(sin_bits, np.uint16)), float(epsilon), _ptr(out))
    return out
