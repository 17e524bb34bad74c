"""float64 check arithmetic of the experiment harness (the reference's numerics.py:45-79,
hadamard_reference.py:19-68, norm_hadamard_reference.py:24-64, qk_rope_reference.py:24-134,
rms_quant_reference.py:24-89), restated for the harness's own correctness gates.

These run on sampled rows/columns on the host after the GPU results are read back; they never
produce a result the harness reports as computed.  Each is written independently of the test
oracle (dense Sylvester matrices here, butterflies there) so the two cross-check each other.
"""

from __future__ import annotations

import numpy as np


def metrics(actual, reference):
    """relative_l2 / max_abs / rmse / cosine in float64 (numerics.py:57-75)."""
    a = np.asarray(actual, dtype=np.float64)
    r = np.asarray(reference, dtype=np.float64)
    if a.shape != r.shape:
        raise ValueError("reference shape mismatch")
    if not (np.isfinite(a).all() and np.isfinite(r).all()):
        return {"finite": False, "relative_l2": None, "max_abs": None, "rmse": None, "cosine": None}
    diff = a - r
    rn, an = float(np.linalg.norm(r)), float(np.linalg.norm(a))
    return {
        "finite": True,
        "relative_l2": float(np.linalg.norm(diff) / max(rn, 1e-30)),
        "max_abs": float(np.max(np.abs(diff))) if diff.size else 0.0,
        "rmse": float(np.sqrt(np.mean(diff**2))) if diff.size else 0.0,
        "cosine": float(np.dot(a.ravel(), r.ravel()) / max(rn * an, 1e-30)) if rn else float(an == 0),
    }


def passes(error, limit):
    return bool(error["finite"] and error["relative_l2"] <= limit)


def sample_indices(length, count=32):
    """Up to `count` evenly spaced indices including both ends (numerics.py:78-79)."""
    return np.unique(np.linspace(0, length - 1, min(length, count), dtype=int))


def fp8_decode(codes):
    """OCP E4M3 values of uint8 codes (sign bit 7, exponent bias 7, subnormals m * 2^-9)."""
    q = np.asarray(codes, dtype=np.uint8).astype(np.int32)
    e, m = (q >> 3) & 15, (q & 7).astype(np.float64)
    mag = np.where(e == 0, m / 512.0, (8.0 + m) * np.exp2(e - 10.0))
    mag = np.where((e == 15) & (m == 7), np.nan, mag)
    return np.where(q & 128, -mag, mag)


def dequantize(q, s, mode):
    """Decoded float64 values of (codes, scales) for int8 / fp8 / mxint8 (numerics.py:49-54)."""
    q, s = np.asarray(q), np.asarray(s)
    if mode == "mxint8":
        z = q.reshape(*q.shape[:-1], -1, 32).astype(np.float64)
        return (z * np.exp2(s.astype(np.float64) - 127)[..., None]).reshape(q.shape)
    z = fp8_decode(q) if mode == "fp8" else q.astype(np.float64)
    return z * s.astype(np.float64)[..., None]


def bf16_round(values):
    """float64 -> FP32 (nearest) -> BF16 (nearest even) -> float64: the BF16 boundary of an FP32
    producer (qk_rope_reference.py:24-42)."""
    f32 = np.ascontiguousarray(values, dtype=np.float32)
    bits = f32.view(np.uint32).astype(np.uint64)
    bits = (bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000
    return bits.astype(np.uint32).view(np.float32).astype(np.float64).reshape(f32.shape)


def hadamard_signs(k, seed):
    """+-1 int8 signs from PCG64(seed) bits (hadamard_reference.py:19-23)."""
    bits = np.random.Generator(np.random.PCG64(seed)).integers(0, 2, size=k, dtype=np.int8)
    return (2 * bits - 1).astype(np.int8)


def _sylvester(block):
    i = np.arange(block)
    parity = np.zeros((block, block), dtype=np.int64)
    both = i[:, None] & i[None, :]
    while both.any():
        parity ^= both & 1
        both = both >> 1
    return np.where(parity, -1.0, 1.0) / np.sqrt(block)


def block_hadamard(x, block, signs=None):
    """float64 X D blockdiag(H_B) with H[i, j] = (-1)^popcount(i & j) / sqrt(B) (dense form)."""
    x = np.asarray(x, dtype=np.float64)
    if signs is not None:
        x = x * np.asarray(signs, dtype=np.float64)
    if block == 1:
        return x.copy()
    rows, k = x.shape
    return (x.reshape(rows, k // block, block) @ _sylvester(block)).reshape(rows, k)


def symmetric_int8(rotated):
    """float64 per-row symmetric INT8: (codes, scales, decoded), scale 1 for a zero row."""
    rotated = np.asarray(rotated, dtype=np.float64)
    peak = np.max(np.abs(rotated), axis=-1)
    scales = np.where(peak == 0, 1.0, peak / 127.0)
    codes = np.clip(np.rint(rotated / scales[..., None]), -127, 127)
    return codes, scales, codes * scales[..., None]


def norm_modulate(x, gamma, scale, shift, *, norm="rms", eps=1e-5):
    """float64 norm(X) * gamma * (1 + scale) + shift; LayerNorm centres with the population
    variance, RMS uses mean(x^2) (norm_hadamard_reference.py:24-64)."""
    x = np.asarray(x, dtype=np.float64)
    if norm == "layer":
        x = x - x.mean(axis=1, keepdims=True)
    inv = 1.0 / np.sqrt(np.mean(x * x, axis=1, keepdims=True) + eps)
    return x * inv * np.asarray(gamma, np.float64) * (1.0 + np.asarray(scale, np.float64)) + np.asarray(
        shift, np.float64
    )


def qk_rope(projected, gamma, cos, sin, *, epsilon=1e-5):
    """Head-major [H, M, D] BF16-rounded output of per-(row, head) RMSNorm over D, gamma, and
    split-half RoPE on pairs (j, j + R); projected [M, H, D] is BF16-rounded first
    (qk_rope_reference.py:45-134)."""
    z = bf16_round(projected)
    u = z / np.sqrt(np.mean(z * z, axis=-1, keepdims=True) + epsilon) * np.asarray(gamma, np.float64)
    half = np.asarray(cos).shape[1]
    c, s = np.asarray(cos, np.float64)[:, None, :], np.asarray(sin, np.float64)[:, None, :]
    v = u.copy()
    a, b = u[..., :half], u[..., half : 2 * half]
    v[..., :half] = a * c - b * s
    v[..., half : 2 * half] = b * c + a * s
    return bf16_round(v).transpose(1, 0, 2)


def rms_quantize(x, gamma, signs, block, eps=1e-5):
    """float64 RMS INT8 encoding with the inverse RMS folded into the scale
    (rms_quant_reference.py:24-89): dict of codes, scales, dequantized, normalized_rotated."""
    x = np.asarray(x, dtype=np.float64)
    inv = 1.0 / np.sqrt(np.mean(x * x, axis=1) + eps)
    unscaled = block_hadamard(x * np.asarray(gamma, np.float64), block, signs)
    codes, unit_scales, _ = symmetric_int8(unscaled)
    peak = np.max(np.abs(unscaled), axis=1)
    scales = np.where(peak == 0, 1.0, unit_scales * inv)
    return {
        "quantized": codes,
        "scales": scales,
        "dequantized": codes * scales[:, None],
        "normalized_rotated": unscaled * inv[:, None],
        "inverse_rms": inv,
    }
