"""Signed block-Hadamard rotation on torch tensors, backed by libm5k.so.

Drop-in mirror of the reference's ``hadamard.rotate`` (src/m5kernels/hadamard.py:33-77):
Y = (X * signs) blockdiag(H_B) in FP32 for X[rows, K] (bf16/fp16/fp32), shared int8 +-1
signs[K], B in {32, ..., 1024}, K % B == 0, no padding.  ``implementation`` keeps the
reference's switch and default: "metal" (the default; alias "hip") selects the gfx950 kernel;
"mlx" named Apple's built-in transform and raises NotImplementedError here.

``rotate_quantize`` is the fused rotation + per-row INT8 quantizer: it returns exactly
``quantize(rotate(x, B, signs), "int8")`` without materializing the FP32 rotation.
"""

from __future__ import annotations


import torch

from . import _lib

SUPPORTED_BLOCK_SIZES = (32, 64, 128, 256, 512, 1024)
_FLOAT_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def _validate(x, block_size, signs):
    if not _lib.is_int(block_size) or block_size <= 0 or block_size & (
        block_size - 1
    ):
        raise ValueError("block_size must be a positive integer power of two")
    block_size = int(block_size)
    if block_size not in SUPPORTED_BLOCK_SIZES:
        raise NotImplementedError("supported block sizes are powers of two from 32 through 1024")
    if x.dim() != 2 or not all(x.shape):
        raise ValueError("input must have nonempty shape [rows, K]")
    if x.dtype not in _FLOAT_DTYPES:
        raise ValueError("input dtype must be float16, bfloat16 or float32")
    if x.shape[1] % block_size:
        raise NotImplementedError("K must be divisible by block_size; padding is not implicit")
    if tuple(signs.shape) != (x.shape[1],) or signs.dtype != torch.int8:
        raise ValueError("signs must be an int8 vector of length K containing only +/-1")
    return block_size


def rotate(x, block_size, signs, implementation="metal"):
    """Return FP32 X D H for nonempty X[rows, K] (hadamard.py:33-77)."""
    block_size = _validate(x, block_size, signs)
    if implementation == "mlx":
        raise NotImplementedError("the MLX built-in Hadamard transform does not exist on ROCm")
    if implementation not in ("hip", "metal"):
        raise ValueError(f"unknown Hadamard implementation: {implementation}")
    x = _lib.aligned_device_tensor(x, "x")
    signs = _lib.aligned_device_tensor(signs, "signs")
    y = torch.empty(tuple(x.shape), dtype=torch.float32, device=x.device)
    _lib.call(
        "m5k_hadamard_rotate",
        _lib.ptr(x),
        _lib.dtype_code(x),
        x.shape[0],
        x.shape[1],
        block_size,
        _lib.ptr(signs),
        _lib.ptr(y),
        _lib.stream_of(x),
    )
    return y


def rotate_quantize(x, block_size, signs):
    """Return (int8 codes, float32 scales) of quantize(rotate(x, block_size, signs), "int8")."""
    block_size = _validate(x, block_size, signs)
    x = _lib.aligned_device_tensor(x, "x")
    signs = _lib.aligned_device_tensor(signs, "signs")
    rows, k = x.shape
    q = torch.empty((rows, k), dtype=torch.int8, device=x.device)
    s = torch.empty((rows,), dtype=torch.float32, device=x.device)
    _lib.call(
        "m5k_hadamard_quantize_rows",
        _lib.ptr(x),
        _lib.dtype_code(x),
        rows,
        k,
        block_size,
        _lib.ptr(signs),
        _lib.ptr(q),
        _lib.ptr(s),
        _lib.stream_of(x),
    )
    return q, s
