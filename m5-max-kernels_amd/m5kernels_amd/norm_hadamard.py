"""One-dispatch normalization, modulation, block rotation and INT8 packing on MI355X.

Drop-in mirror of the reference's ``norm_hadamard`` module
(src/m5kernels/norm_hadamard.py:22-348): same function names, signatures, defaults and
exception types.  The modulation contract is ``norm(X) * gamma * (1 + scale) + shift``
evaluated in FP32, optionally rounded to X's dtype after the complete expression
(``round_output="input"``); shared +-1 signs are applied after that rounding and before the
normalized Hadamard butterflies; rows are then quantized to symmetric INT8 with
``scale = max|row| / 127`` (1 for an all-zero row).

Platform notes (contract unchanged):

* ``threads`` (128/256), ``passes`` ("one_read"/"two_read") and ``tag`` are validated as in
  the reference; the gfx950 kernel always keeps the row in registers with 256 lanes.
* gamma/scale/shift/gate and ``branch`` are read in their own float dtypes by the one kernel
  (no host-side casts): every table may have its own dtype, and the branch's need not be the
  residual's.  Each value enters the FP32 arithmetic exactly, as ``float(...)`` does.
* K must be a multiple of 8 (always true with a Hadamard block; checked for unfused_norm
  and gated_residual_add).
"""

from __future__ import annotations

import math

import torch

from . import _lib
from .hadamard import SUPPORTED_BLOCK_SIZES

FLOAT_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def _validate_common(x, gamma, scale, shift, norm, epsilon, round_output, threads, row_map):
    if x.dim() != 2 or not all(x.shape):
        raise ValueError("input must have nonempty shape [rows, K]")
    if x.dtype not in FLOAT_DTYPES:
        raise ValueError("input dtype must be float16, bfloat16 or float32")
    if tuple(gamma.shape) != (x.shape[1],) or gamma.dtype not in FLOAT_DTYPES:
        raise ValueError("gamma must be a floating vector of length K")
    if row_map is None:
        if tuple(scale.shape) != (x.shape[1],) or tuple(shift.shape) != tuple(scale.shape):
            raise ValueError("scale and shift must be vectors of length K without row_map")
    else:
        if scale.dim() != 2 or not all(scale.shape) or scale.shape[1] != x.shape[1] or shift.shape != scale.shape:
            raise ValueError("mapped scale and shift must have matching nonempty shape [P,K]")
        if tuple(row_map.shape) != (x.shape[0],) or row_map.dtype != torch.int32:
            raise ValueError("row_map must be an int32 vector of length M")
    if scale.dtype not in FLOAT_DTYPES or shift.dtype not in FLOAT_DTYPES:
        raise ValueError("scale and shift must have floating dtype")
    if norm == "layernorm":
        norm = "layer"
    if norm not in ("rms", "layer"):
        raise ValueError("norm must be 'rms' or 'layer'")
    if not _lib.is_real(epsilon):
        raise ValueError("epsilon must be a positive finite real scalar")
    if not math.isfinite(epsilon) or epsilon <= 0:
        raise ValueError("epsilon must be a positive finite real scalar")
    if round_output not in ("input", "fp32"):
        raise ValueError("round_output must be 'input' or 'fp32'")
    if not _lib.is_int(threads):
        raise ValueError("threads must be an integer")
    if threads not in (128, 256):
        raise NotImplementedError("supported threadgroup sizes are 128 and 256")
    return norm


def _validate_rotation(x, signs, block_size, passes, tag):
    if not _lib.is_int(block_size) or block_size <= 0 or block_size & (
        block_size - 1
    ):
        raise ValueError("block_size must be a positive integer power of two")
    if block_size not in SUPPORTED_BLOCK_SIZES:
        raise NotImplementedError("supported block sizes are powers of two from 32 through 1024")
    if x.shape[1] % block_size:
        raise NotImplementedError("K must be divisible by block_size; padding is not implicit")
    if tuple(signs.shape) != (x.shape[1],) or signs.dtype != torch.int8:
        raise ValueError("signs must be an int8 vector of length K containing only +/-1")
    if passes not in ("one_read", "two_read"):
        raise ValueError("passes must be 'one_read' or 'two_read'")
    if not _lib.is_identifier(tag):
        raise ValueError("tag must be a valid nonempty Metal identifier")


def _validate_gate(residual, branch, gate, gate_row_map):
    if residual.dim() != 2 or not all(residual.shape):
        raise ValueError("residual must have nonempty shape [M,K]")
    if residual.dtype not in FLOAT_DTYPES:
        raise ValueError("residual must have floating dtype")
    if branch.shape != residual.shape or branch.dtype not in FLOAT_DTYPES:
        raise ValueError("branch must have the same shape as residual and floating dtype")
    if gate.dtype not in FLOAT_DTYPES:
        raise ValueError("gate must have floating dtype")
    if gate_row_map is None:
        if tuple(gate.shape) != (residual.shape[1],):
            raise ValueError("gate must be a vector of length K without gate_row_map")
    else:
        if gate.dim() != 2 or not all(gate.shape) or gate.shape[1] != residual.shape[1]:
            raise ValueError("mapped gate must have nonempty shape [P,K]")
        if tuple(gate_row_map.shape) != (residual.shape[0],) or gate_row_map.dtype != torch.int32:
            raise ValueError("gate_row_map must be an int32 vector of length M")


def _params(gamma, scale, shift, gate=None):
    """The device tables as given and their param_dtype code: BF16 when every table is BF16, else
    one dtype code per table (M5K_PARAM_TABLES; an absent gate's field is unused)."""
    tables = (gamma, scale, shift, gate)
    out = [None if t is None else _lib.aligned_device_tensor(t, "parameter") for t in tables]
    codes = [_lib.BF16 if t is None else _lib.dtype_code(t) for t in out]
    if all(c == _lib.BF16 for c in codes):
        return _lib.BF16, out
    return _lib.param_tables(*codes), out


def _map(t, name):
    return None if t is None else _lib.device_tensor(t, name)


def _branch(branch):
    """Device branch and its dtype code (any float dtype; the kernels read it as is)."""
    branch = _lib.aligned_device_tensor(branch, "branch")
    return branch, _lib.dtype_code(branch)


def _norm_code(norm):
    return _lib.NORM_LAYER if norm == "layer" else _lib.NORM_RMS


def _prep(x, gamma, scale, shift, signs, block_size, norm, epsilon, round_output, row_map, branch=None, gate=None,
          gate_row_map=None):
    x = _lib.aligned_device_tensor(x, "x")
    signs = _lib.aligned_device_tensor(signs, "signs")
    pdt, (gamma_d, scale_d, shift_d, gate_d) = _params(gamma, scale, shift, gate)
    rows, k = x.shape
    q = torch.empty((rows, k), dtype=torch.int8, device=x.device)
    s = torch.empty((rows,), dtype=torch.float32, device=x.device)
    r_next, branch_code = None, _lib.dtype_code(x)
    if branch is not None:
        branch, branch_code = _branch(branch)
        r_next = torch.empty_like(x)
    _lib.call(
        "m5k_norm_hadamard_quantize",
        _lib.ptr(x), _lib.dtype_code(x), rows, k,
        _lib.ptr(branch), branch_code, _lib.ptr(gate_d), _lib.ptr(_map(gate_row_map, "gate_row_map")),
        _lib.ptr(gamma_d), _lib.ptr(scale_d), _lib.ptr(shift_d), pdt, _lib.ptr(_map(row_map, "row_map")),
        _lib.ptr(signs), int(block_size), _norm_code(norm), float(epsilon), 1 if round_output == "input" else 0,
        _lib.ptr(q), _lib.ptr(s), _lib.ptr(r_next), _lib.stream_of(x),
    )
    return q, s, r_next


def fused_norm_hadamard_quantize(
    x,
    gamma,
    scale,
    shift,
    signs,
    block_size=256,
    *,
    norm="rms",
    epsilon=1e-5,
    round_output="input",
    threads=256,
    passes="one_read",
    tag="default",
    row_map=None,
):
    """Return symmetric per-row (INT8 codes, FP32 scales) of norm/modulate -> X D H
    (norm_hadamard.py:122-176).  Scale/shift are [K] vectors or [P,K] tables selected by
    int32 row_map[M]; map bounds, finite values and +-1 signs are caller preconditions."""
    norm = _validate_common(x, gamma, scale, shift, norm, epsilon, round_output, threads, row_map)
    _validate_rotation(x, signs, block_size, passes, tag)
    q, s, _ = _prep(x, gamma, scale, shift, signs, block_size, norm, epsilon, round_output, row_map)
    return q, s


def fused_gated_residual_norm_hadamard_quantize(
    residual,
    branch,
    gate,
    gamma,
    scale,
    shift,
    signs,
    block_size=256,
    *,
    norm="rms",
    epsilon=1e-5,
    round_output="input",
    threads=256,
    passes="one_read",
    tag="default",
    gate_row_map=None,
    row_map=None,
):
    """Return (INT8 codes, scales, updated residual) in one dispatch (norm_hadamard.py:198-265).

    The updated residual is cast_R(float(R) + float(branch) * float(gate)), written once and
    then normalized, modulated, rotated and quantized."""
    _validate_gate(residual, branch, gate, gate_row_map)
    norm = _validate_common(residual, gamma, scale, shift, norm, epsilon, round_output, threads, row_map)
    _validate_rotation(residual, signs, block_size, passes, tag)
    return _prep(residual, gamma, scale, shift, signs, block_size, norm, epsilon, round_output, row_map,
                 branch=branch, gate=gate, gate_row_map=gate_row_map)


def gated_residual_add(residual, branch, gate, *, gate_row_map=None, threads=256, tag="default"):
    """Staged FP32 gated addition with one residual-dtype cast (norm_hadamard.py:280-300)."""
    _validate_gate(residual, branch, gate, gate_row_map)
    if not _lib.is_int(threads):
        raise ValueError("threads must be an integer")
    if threads not in (128, 256):
        raise NotImplementedError("supported threadgroup sizes are 128 and 256")
    if not _lib.is_identifier(tag):
        raise ValueError("tag must be a valid nonempty Metal identifier")
    if residual.shape[1] % 8:
        raise NotImplementedError("K must be a multiple of 8 on MI355X")
    residual = _lib.aligned_device_tensor(residual, "residual")
    branch, branch_code = _branch(branch)
    gate_d = _lib.aligned_device_tensor(gate, "gate")
    out = torch.empty_like(residual)
    rows, k = residual.shape
    _lib.call(
        "m5k_gated_residual_add",
        _lib.ptr(residual), _lib.dtype_code(residual), rows, k, _lib.ptr(branch), branch_code, _lib.ptr(gate_d),
        _lib.dtype_code(gate_d),
        _lib.ptr(_map(gate_row_map, "gate_row_map")), _lib.ptr(out), _lib.stream_of(residual),
    )
    return out


def unfused_norm(
    x,
    gamma,
    scale,
    shift,
    *,
    norm="rms",
    epsilon=1e-5,
    round_output="input",
    threads=256,
    row_map=None,
):
    """Norm + modulation only, with the fused path's rounding contract (norm_hadamard.py:321-348)."""
    norm = _validate_common(x, gamma, scale, shift, norm, epsilon, round_output, threads, row_map)
    if x.shape[1] % 8:
        raise NotImplementedError("K must be a multiple of 8 on MI355X")
    x = _lib.aligned_device_tensor(x, "x")
    pdt, (gamma_d, scale_d, shift_d, _) = _params(gamma, scale, shift)
    out_dtype = x.dtype if round_output == "input" else torch.float32
    y = torch.empty(tuple(x.shape), dtype=out_dtype, device=x.device)
    rows, k = x.shape
    _lib.call(
        "m5k_norm_modulate",
        _lib.ptr(x), _lib.dtype_code(x), rows, k, _lib.ptr(gamma_d), _lib.ptr(scale_d), _lib.ptr(shift_d), pdt,
        _lib.ptr(_map(row_map, "row_map")), _norm_code(norm), float(epsilon), 1 if round_output == "input" else 0,
        _lib.ptr(y), _lib.stream_of(x),
    )
    return y
