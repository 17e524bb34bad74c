"""RMS dynamic INT8 quantization with the inverse RMS folded into the row scales, on MI355X.

Drop-in mirror of the reference's ``rms_quant.rms_quantize`` (src/m5kernels/rms_quant.py:41-117):
same signature, defaults, validation and exception types.  There is no additive shift and no
reduced-precision intermediate after normalization; gamma is a shared FP32 vector (which may
already hold gamma * (1 + AdaLN scale)) and signs a shared +-1 int8 vector.  ``threads`` and
``tag`` are validated as in the reference (they named Metal threadgroup sizes and kernel
names); the gfx950 kernel always uses one 256-thread workgroup per row.
"""

from __future__ import annotations

import math
import struct

import torch

from . import _lib

BLOCK_SIZES = (1, 32, 64, 128, 256, 512, 1024)


def rms_quantize(x, gamma, signs, block_size=1, *, threads=256, fold_scale=True, epsilon=1e-5, tag="default"):
    """Return per-row INT8 codes and FP32 scales for signed RMS(X)*gamma*H (rms_quant.py:41-68).

    fold_scale=True: u = (X*gamma)*D*H, codes round(127*u/max|u|), scales max|u|*inv_rms/127.
    fold_scale=False: X is normalized by inv_rms first, then transformed; scales max|v|/127.
    Both give scale 1 and codes 0 for a row whose transform is zero."""
    if x.dim() != 2 or not all(x.shape):
        raise ValueError("input must have nonempty shape [M,K]")
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError("input dtype must be float16, bfloat16 or float32")
    if tuple(gamma.shape) != (x.shape[1],) or gamma.dtype != torch.float32:
        raise ValueError("gamma must be a float32 vector of length K")
    if tuple(signs.shape) != (x.shape[1],) or signs.dtype != torch.int8:
        raise ValueError("signs must be an int8 vector of length K containing only +/-1")
    if not _lib.is_int(block_size) or block_size <= 0 or block_size & (
        block_size - 1
    ):
        raise ValueError("block_size must be a positive integer power of two")
    if block_size not in BLOCK_SIZES:
        raise NotImplementedError("supported blocks are 1 and powers of two from 32 through 1024")
    if x.shape[1] % block_size:
        raise NotImplementedError("K must be divisible by block_size; padding is not implicit")
    if not _lib.is_int(threads):
        raise ValueError("threads must be an integer")
    if threads not in (128, 256, 512):
        raise NotImplementedError("supported threadgroup sizes are 128, 256 and 512")
    if not isinstance(fold_scale, bool):
        raise ValueError("fold_scale must be a boolean")
    if not _lib.is_real(epsilon) or not math.isfinite(epsilon) or epsilon <= 0:
        raise ValueError("epsilon must be a positive finite real scalar")
    try:
        epsilon = struct.unpack("=f", struct.pack("=f", float(epsilon)))[0]
    except OverflowError:
        raise ValueError("epsilon must remain finite and positive in float32") from None
    if not math.isfinite(epsilon) or epsilon <= 0:
        raise ValueError("epsilon must remain finite and positive in float32")
    if not _lib.is_identifier(tag):
        raise ValueError("tag must be a valid nonempty Metal identifier")
    m, k = x.shape
    x = _lib.aligned_device_tensor(x, "x")
    gamma = _lib.aligned_device_tensor(gamma, "gamma")
    signs = _lib.aligned_device_tensor(signs, "signs")
    q = torch.empty((m, k), dtype=torch.int8, device=x.device)
    s = torch.empty((m,), dtype=torch.float32, device=x.device)
    _lib.call(
        "m5k_rms_quantize",
        _lib.ptr(x), _lib.dtype_code(x), m, k, _lib.ptr(gamma), _lib.ptr(signs), int(block_size), int(fold_scale),
        float(epsilon), _lib.ptr(q), _lib.ptr(s), _lib.stream_of(x),
    )
    return q, s
