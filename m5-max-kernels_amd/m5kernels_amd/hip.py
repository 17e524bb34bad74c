"""Quantizer and linear-layer op contracts on torch tensors, backed by libm5k.so.

Drop-in mirror of the reference's ``metal.quantize`` / ``metal.gemm``
(src/m5kernels/metal.py:27-44, 158-269): same names, positional/keyword
signatures, defaults, argument meaning and exception types.  Inputs are never
mutated; outputs are freshly allocated on the input's device and computed on
the current HIP stream.

Differences that follow from the platform, not the contract:

* ``tile=(TM, TN, groups, swizzle)`` names an Apple threadgroup tiling.  It is
  unpacked (so malformed tuples fail as in the reference) but the MI355X kernel
  always uses its own 256x256 MFMA tile with an XCD-aware raster.
* ``tag`` only specialized the Metal kernel name; it is accepted and ignored.
* ``mode="mxint8"`` GEMM expands both operands exactly to BF16 (codes times their block
  scale) and runs the BF16 MFMA GEMM with FP32 accumulation.
"""

from __future__ import annotations

import contextlib
import ctypes
import functools
import os
import threading

import torch

from . import _lib

_QUANT_MODES = {"int8": _lib.QUANT_INT8, "fp8": _lib.QUANT_FP8}
_FLOAT_DTYPES = (torch.float16, torch.bfloat16, torch.float32)
# metal.py:59-66 dtype table (the KeyError for unknown modes is preserved).
_MODE_DTYPES = {
    "fp16": torch.float16,
    "bf16": torch.bfloat16,
    "fp32": torch.float32,
    "int8": torch.int8,
    "mxint8": torch.int8,
    "fp8": torch.uint8,
}


def quantize(x, mode, tag="packed"):
    """Return (codes, scales) of symmetric per-row quantization of X[rows, K].

    INT8: int8 codes in [-127, 127], scale = max|row| / 127 (1 for an all-zero row),
    code = rint_even(x / scale).  FP8: uint8 OCP E4M3 codes of x / scale with
    scale = max|row| / 448.  MXINT8: int8 codes of 32-element blocks sharing a power-of-two
    scale, returned as uint8 exponent bytes [rows, K/32] (e + 127, numerics.py:33-41).
    Mirrors metal.quantize (metal.py:27-44).
    """
    rows, k = x.shape
    if mode == "mxint8":
        if k % 32:
            raise ValueError("MXINT8 requires K divisible by 32")
        if x.dtype not in _FLOAT_DTYPES:
            raise ValueError("quantization input must be float16, bfloat16 or float32")
        if rows == 0:
            raise ValueError("quantization input must be nonempty")
        x = _lib.aligned_device_tensor(x, "x")
        q = torch.empty((rows, k), dtype=torch.int8, device=x.device)
        e = torch.empty((rows, k // 32), dtype=torch.uint8, device=x.device)
        _lib.call("m5k_quantize_mxint8", _lib.ptr(x), _lib.dtype_code(x), rows, k, _lib.ptr(q), _lib.ptr(e),
                  _lib.stream_of(x))
        return q, e
    if mode not in _QUANT_MODES:
        raise ValueError(f"unknown quantization mode: {mode!r}")
    if x.dtype not in _FLOAT_DTYPES:
        raise ValueError("quantization input must be float16, bfloat16 or float32")
    if rows == 0 or k == 0:
        raise ValueError("quantization input must be nonempty")
    x = _lib.device_tensor(x, "x")
    q = torch.empty((rows, k), dtype=torch.uint8 if mode == "fp8" else torch.int8, device=x.device)
    s = torch.empty((rows,), dtype=torch.float32, device=x.device)
    _lib.call(
        "m5k_quantize_rows",
        _lib.ptr(x),
        _lib.dtype_code(x),
        rows,
        k,
        _QUANT_MODES[mode],
        _lib.ptr(q),
        _lib.ptr(s),
        _lib.stream_of(x),
    )
    return q, s


def _check_vector(t, n, dtype, message):
    if t is None or tuple(t.shape) != (n,) or t.dtype != dtype:
        raise ValueError(message)


def splitk_plan(m, n, k, cus=256, skinny=True):
    """Number of K ranges per output tile for the W8A8 linear (1 = one workgroup per tile).

    Shapes with few 256 x 256 tiles (short M) leave most of the 256 CUs idle; splitting K
    aims at ~224 workgroups, each over at least 4 slabs of 64 bytes.  The INT32 partial
    tiles cost 8 * splits * M * N bytes of extra traffic against the N * K bytes of weights,
    so splits also stay below K / (2 M).  (Measured on MI355X over M 16..512 and H3 widths:
    within ~10% of the best split count, 1.4-3.7x faster than one workgroup per tile.)

    It first tries the library's narrower split tiles, which m5k_gemm_i8_splitk uses whenever
    ceil(M / 256) * ceil(N / width) * splits fits in one round of `cus` workgroups: 256 x 64
    (K <= 8192), then 256 x 128.  Fewer K ranges then fill the chip (measured 1.4-1.6x faster
    at K 4096-5376 with 64-wide tiles, 1.15-1.23x at N 14336 or K 14336-16384 with 128-wide
    ones, 1.1-1.45x at M 384-1024).  Above M = 768, with at least 32 tiles of 256 x 256, the
    plain launch (the library's mixed or narrow tiles) measured faster than any split (M 1024:
    44.8 against 57.6 us at N = K = 5376, 35.5 against 37.2 us at N = K = 4096), so no split is
    planned there, unless K is long and the tiles fill under 3/8 of the CUs (then the chip takes
    cus // tiles K ranges); narrow outputs (N 32-96) keep the split, their few tiles leaving most
    CUs idle.
    skinny=False plans without the 256 x 64 tile (the FP8 split, m5k_gemm_f8_splitk)."""
    slabs = -(-k // 64)
    if m > 768 and -(-m // 256) * -(-n // 256) >= 32:
        # One partial round that even the mixed launch's half tiles fill to under 3/4, over a
        # long K: whole-tile K ranges fill the chip instead (M 1024: 84 tiles at N 5376, K 14336
        # ran 94.0 -> 84.3 us with 3 ranges; 64 at N 4096, K 16384 97.7 -> 77.5 us with 4; at
        # K 5376, or M 1536 and up, the plain and mixed launches stayed ahead).
        tiles = -(-m // 256) * -(-n // 256)
        if k >= 8192 and 2 * tiles <= 3 * cus // 4:
            return max(2, min(cus // tiles, slabs // 4, 64))
        return 1
    tiles_m = -(-m // 256)
    for width in ((64, 128) if k <= 8192 and skinny else (128,)):
        splits = min(cus // (tiles_m * -(-n // width)), slabs // 4, max(2, k // (2 * m)), 64)
        if splits >= 2:
            return splits
    tiles = tiles_m * -(-n // 256)
    splits = min(224 // tiles, slabs // 4, max(2, k // (2 * m)), 64)
    return splits if splits >= 2 else 1


def tail_split_plan(m, n, k, cus=256):
    """Row split of a W8A8 linear with a partial last round: (rows, splits) or None.

    With T tiles of 256 x 256 on `cus` CUs (one workgroup per CU, T >= cus), the last round
    runs at (T mod cus) / cus of the chip.  The first `rows` rows (whole tile rows filling
    at most the full rounds) then run as a plain launch and the remaining rows as a split-K
    launch with `splits` K ranges per tile, which refills the last round.  The split saves
    (1 - 1/splits) of a round and costs its INT32 partials, 8 * splits * (m - rows) * n
    bytes written and read, plus a second launch.  Cost model from MI355X measurements: a
    round of 256 x 256 tiles takes ~15.3 ns per unit of K (~2.2 POP/s), the partials move at
    ~5 TB/s and a launch costs ~4 us; the split is taken when it saves over 5% of the plain
    time.  (Measured: H3 widths N 5120-5376 at M 4096 7-18% faster; M 9914, N 4096, K 4096
    no faster, and the model declines it.)"""
    tiles_m, tiles_n = -(-m // 256), -(-n // 256)
    tiles = tiles_m * tiles_n
    if tiles < cus or tiles % cus == 0:
        return None
    rows_dp = (tiles // cus) * cus // tiles_n
    tail_tiles = (tiles_m - rows_dp) * tiles_n
    if rows_dp == 0:
        return None
    tail_m = m - rows_dp * 256
    round_s = 15.3e-9 * k
    best, best_gain = None, 0.05 * round_s * -(-tiles // cus)
    for splits in range(2, min(cus // tail_tiles, -(-k // 128) // 2, 16) + 1):
        gain = round_s * (1 - 1 / splits) - (tail_m * n * (8 * splits + 2) / 5e12 + 4e-6)
        if gain > best_gain:
            best, best_gain = splits, gain
    return None if best is None else (rows_dp * 256, best)


_PLAN_DTYPES = {"int8": _lib.I8, "fp8": _lib.U8, "bf16": _lib.BF16, "fp16": _lib.F16, "fp32": _lib.F32}
SCHEDULES = ("plain", "mixed", "narrow", "quad")

_override = threading.local()


_SCHEDULE_CODES = {name: i for i, name in enumerate(SCHEDULES)}


@contextlib.contextmanager
def launch_override(schedule=None, splits=None):
    """Fix the gfx950 GEMM launch for the calls this thread makes inside the block: `schedule`
    ("plain", "mixed", "narrow" or "quad"; set in the library for this host thread with
    m5k_gemm_set_schedule) and, for the W8A8 linear, the split-K count `splits` (1: no split;
    the INT32 partials are exact, so every choice gives the same bits).  A forced schedule with
    `splits` None runs unsplit: the launch timed is the one named.  None keeps the library's own
    plan.  These are the knobs the harness tuner searches; both settings are thread-local."""
    if schedule is not None and schedule not in SCHEDULES:
        raise ValueError(f"unknown GEMM schedule {schedule!r}")
    if splits is not None and (isinstance(splits, bool) or not isinstance(splits, int) or not 1 <= splits <= 64):
        raise ValueError("splits must be an integer in [1, 64]")
    saved_schedule = getattr(_override, "schedule", None)
    saved_splits = getattr(_override, "splits", None)
    previous = ctypes.c_int(-1)
    if schedule is not None:
        _lib.call("m5k_gemm_set_schedule", _SCHEDULE_CODES[schedule], ctypes.byref(previous))
        _override.schedule = schedule
    _override.splits = splits
    try:
        yield
    finally:
        _override.splits = saved_splits
        if schedule is not None:
            _lib.call("m5k_gemm_set_schedule", previous.value, None)
            _override.schedule = saved_schedule


def launch_plan(mode, m, n, cus=256):
    """The library's GEMM schedule for an [m, n] output on `cus` CUs (m5k_gemm_launch_plan;
    host only): ("plain" | "mixed" | "narrow" | "quad", full tiles of the mixed launch or -1)."""
    sched, full = ctypes.c_int(0), ctypes.c_int64(0)
    _lib.call("m5k_gemm_launch_plan", _PLAN_DTYPES[mode], m, n, cus, ctypes.byref(sched), ctypes.byref(full))
    return SCHEDULES[sched.value], full.value


@functools.lru_cache(maxsize=None)
def _cu_count_of(index):
    return torch.cuda.get_device_properties(index).multi_processor_count


def _cu_count(device):
    return _cu_count_of(device.index if device.index is not None else torch.cuda.current_device())


@functools.lru_cache(maxsize=4096)
def _i8_schedule(m, n, k, cus, env):
    """Host schedule of an aligned W8A8 linear, cached per shape, CU count and the library's
    schedule switches `env` (M5K_GEMM_MIXED_TILES, M5K_GEMM_NARROW_TILES, M5K_GEMM_SCHEDULE):
    (splits, tail), with
    tail = (rows of the plain launch, splits of the rest) or None."""
    if env[2]:
        return 1, None  # a schedule forced from the environment runs unsplit, as named
    splits = splitk_plan(m, n, k, cus)
    # The library's mixed and narrow launches refill a partial last round without INT32
    # partials and measured faster wherever both apply; the split-K tail takes the rest.
    tail = None
    if splits == 1 and launch_plan("int8", m, n, cus)[0] == "plain":
        tail = tail_split_plan(m, n, k, cus)
    return splits, tail


@functools.lru_cache(maxsize=4096)
def _f8_splits(m, n, k, cus, forced):
    """K ranges per tile of an aligned FP8 linear (1: the plain launch), cached per shape, CU
    count and M5K_GEMM_SCHEDULE (a schedule forced from the environment runs unsplit)."""
    return 1 if forced else splitk_plan(m, n, k, cus, skinny=False)


def gemm(
    a,
    b,
    mode="bf16",
    tile=(64, 64, 4, 1),
    a_scales=None,
    b_scales=None,
    output_dtype=None,
    bias=None,
    bias_row_map=None,
    residual=None,
    gate=None,
    gate_row_map=None,
):
    """A[M,K] @ B[N,K].T with INT32 (int8) or FP32 (fp8/bf16/fp16) accumulation.

    Quantized modes apply ``O(float(acc) * a_scales[m] * b_scales[n])`` in FP32, left to
    right.  INT8 optionally adds an FP32 bias [N] (or [P,N] selected by int32
    bias_row_map[M]) before the output cast.  INT8/BF16 optionally fuse a gated residual
    update ``bf16(float(residual) + float(bf16(branch)) * float(gate))`` (gate [N] or
    [P,N] with gate_row_map[M]); that requires BF16 output and cannot be combined with
    a bias.  output_dtype defaults to float32.  Mirrors metal.gemm (metal.py:158-269).
    """
    m, k = a.shape
    n, kb = b.shape
    if k != kb:
        raise ValueError("K mismatch")
    if mode == "fp8" and k % 128:
        raise NotImplementedError("FP8 requires K/row stride divisible by 128; padding is not implicit")
    if mode == "int8" and k > 133144:
        raise NotImplementedError("INT32 worst-case overflow bound exceeded")
    gated = residual is not None or gate is not None or gate_row_map is not None
    if gated:
        if residual is None or gate is None:
            raise ValueError("gated GEMM requires both residual and gate")
        if mode not in {"int8", "bf16"}:
            raise NotImplementedError("gated GEMM supports INT8 and BF16 only")
        if output_dtype is None or output_dtype != torch.bfloat16:
            raise NotImplementedError("gated GEMM requires explicit BF16 output_dtype")
        if bias is not None or bias_row_map is not None:
            raise NotImplementedError("combining GEMM bias and gated residual is unsupported")
        if tuple(residual.shape) != (m, n) or residual.dtype != torch.bfloat16:
            raise ValueError("residual must have BF16 dtype and shape [M,N]")
        if gate.dtype != torch.bfloat16:
            raise ValueError("gate must have BF16 dtype")
        if gate_row_map is None:
            if tuple(gate.shape) != (n,):
                raise ValueError("gate must have shape [N] without gate_row_map")
        else:
            if gate.dim() != 2 or not all(gate.shape) or gate.shape[1] != n:
                raise ValueError("mapped gate must have nonempty shape [P,N]")
            if tuple(gate_row_map.shape) != (m,) or gate_row_map.dtype != torch.int32:
                raise ValueError("gate_row_map must be an int32 vector of length M")
        expected_dtype = torch.int8 if mode == "int8" else torch.bfloat16
        if a.dtype != expected_dtype or b.dtype != expected_dtype:
            raise ValueError("gated GEMM operand dtypes must match the declared mode")
        if mode == "int8" and (
            a_scales is None
            or b_scales is None
            or tuple(a_scales.shape) != (m,)
            or tuple(b_scales.shape) != (n,)
            or a_scales.dtype != torch.float32
            or b_scales.dtype != torch.float32
        ):
            raise ValueError("gated INT8 GEMM requires float32 scales with shapes [M] and [N]")
    if bias is None:
        if bias_row_map is not None:
            raise ValueError("bias_row_map requires a bias table")
    else:
        if mode != "int8":
            raise NotImplementedError("optional GEMM bias currently supports INT8 only")
        if bias.dtype != torch.float32:
            raise ValueError("bias must have float32 dtype")
        if bias_row_map is None:
            if tuple(bias.shape) != (n,):
                raise ValueError("bias must have shape [N] without bias_row_map")
        else:
            if bias.dim() != 2 or not all(bias.shape) or bias.shape[1] != n:
                raise ValueError("mapped bias must have nonempty shape [P,N]")
            if tuple(bias_row_map.shape) != (m,) or bias_row_map.dtype != torch.int32:
                raise ValueError("bias_row_map must be an int32 vector of length M")
    tm, tn, groups, swizzle = tile
    operand_dtype = _MODE_DTYPES[mode]  # KeyError for an unknown mode, as in metal.py:59-66
    if mode in {"int8", "fp8", "mxint8"}:
        if a_scales is None or b_scales is None:
            raise ValueError("scales required")
    if mode == "mxint8":
        return _gemm_mxint8(a, b, a_scales, b_scales, output_dtype)
    if a.dtype != operand_dtype or b.dtype != operand_dtype:
        raise ValueError(f"{mode} GEMM requires {operand_dtype} operands")
    if m == 0 or n == 0 or k == 0:
        raise ValueError("GEMM operands must be nonempty")
    out_dtype = output_dtype or torch.float32
    if out_dtype not in _FLOAT_DTYPES:
        raise ValueError("output_dtype must be float16, bfloat16 or float32")

    a = _lib.device_tensor(a, "a")
    b = _lib.device_tensor(b, "b")
    c = torch.empty((m, n), dtype=out_dtype, device=a.device)
    out_code = _lib.dtype_code(c)
    stream = _lib.stream_of(a)
    if residual is not None:
        residual = _lib.device_tensor(residual, "residual")
        gate = _lib.device_tensor(gate, "gate")
        gate_row_map = None if gate_row_map is None else _lib.device_tensor(gate_row_map, "gate_row_map")
    if mode in {"int8", "fp8"}:
        _check_vector(a_scales, m, torch.float32, "a_scales must be a float32 vector of length M")
        _check_vector(b_scales, n, torch.float32, "b_scales must be a float32 vector of length N")
        a_scales = _lib.device_tensor(a_scales, "a_scales")
        b_scales = _lib.device_tensor(b_scales, "b_scales")
    if mode == "int8":
        if bias is not None:
            bias = _lib.device_tensor(bias, "bias")
            bias_row_map = None if bias_row_map is None else _lib.device_tensor(bias_row_map, "bias_row_map")
        # Split-K and the tail split run the direct-to-LDS main loop only (m5k_gemm_i8_splitk
        # rejects other operands): 16-byte aligned rows and bases.
        aligned = k % 16 == 0 and a.data_ptr() % 16 == 0 and b.data_ptr() % 16 == 0
        splits, tail = 1, None
        forced_splits = getattr(_override, "splits", None)
        if aligned and forced_splits is not None:
            splits = forced_splits
        elif aligned and getattr(_override, "schedule", None) is not None:
            splits = 1  # a forced schedule runs unsplit, without the tail split
        elif aligned:
            environ = os.environ
            env = (environ.get("M5K_GEMM_MIXED_TILES"), environ.get("M5K_GEMM_NARROW_TILES"),
                   environ.get("M5K_GEMM_SCHEDULE"))
            splits, tail = _i8_schedule(m, n, k, _cu_count(a.device), env)
        if tail is not None:
            # Whole tile rows in full rounds, then the remaining rows split along K.  Every
            # row-indexed operand is sliced at the same row; both launches are bit-exact.
            r0, tail_splits = tail

            def rows(t, lo, hi):
                return None if t is None else t[lo:hi]

            workspace = torch.empty((tail_splits, m - r0, n), dtype=torch.int32, device=a.device)
            for lo, hi, part in ((0, r0, 1), (r0, m, tail_splits)):
                args = [
                    _lib.ptr(a[lo:hi]), _lib.ptr(b), hi - lo, n, k, _lib.ptr(a_scales[lo:hi]), _lib.ptr(b_scales),
                    _lib.ptr(c[lo:hi]), out_code, _lib.ptr(bias), _lib.ptr(rows(bias_row_map, lo, hi)),
                    _lib.ptr(rows(residual, lo, hi)), _lib.ptr(gate), _lib.ptr(rows(gate_row_map, lo, hi)),
                ]
                if part == 1:
                    _lib.call("m5k_gemm_i8", *args, stream)
                else:
                    _lib.call("m5k_gemm_i8_splitk", *args, part, _lib.ptr(workspace), workspace.numel(), stream)
            return c
        if splits > 1:
            workspace = torch.empty((splits, m, n), dtype=torch.int32, device=a.device)
            _lib.call(
                "m5k_gemm_i8_splitk",
                _lib.ptr(a), _lib.ptr(b), m, n, k, _lib.ptr(a_scales), _lib.ptr(b_scales), _lib.ptr(c), out_code,
                _lib.ptr(bias), _lib.ptr(bias_row_map), _lib.ptr(residual), _lib.ptr(gate), _lib.ptr(gate_row_map),
                splits, _lib.ptr(workspace), workspace.numel(), stream,
            )
            return c
        _lib.call(
            "m5k_gemm_i8",
            _lib.ptr(a),
            _lib.ptr(b),
            m,
            n,
            k,
            _lib.ptr(a_scales),
            _lib.ptr(b_scales),
            _lib.ptr(c),
            out_code,
            _lib.ptr(bias),
            _lib.ptr(bias_row_map),
            _lib.ptr(residual),
            _lib.ptr(gate),
            _lib.ptr(gate_row_map),
            stream,
        )
    elif mode == "fp8":
        # Short M: split-K with FP32 partials (deterministic; the FP32 sums may differ from the
        # unsplit launch's in the last bits, FP8's accumulation order being unpinned).  A
        # schedule forced for the tuner runs unsplit, as named.
        splits = 1
        if a.data_ptr() % 16 == 0 and b.data_ptr() % 16 == 0 and getattr(_override, "schedule", None) is None:
            splits = _f8_splits(m, n, k, _cu_count(a.device), os.environ.get("M5K_GEMM_SCHEDULE"))
        if splits > 1:
            workspace = torch.empty((splits, m, n), dtype=torch.float32, device=a.device)
            _lib.call(
                "m5k_gemm_f8_splitk", _lib.ptr(a), _lib.ptr(b), m, n, k, _lib.ptr(a_scales), _lib.ptr(b_scales),
                _lib.ptr(c), out_code, splits, _lib.ptr(workspace), workspace.numel(), stream,
            )
            return c
        _lib.call(
            "m5k_gemm_f8",
            _lib.ptr(a),
            _lib.ptr(b),
            m,
            n,
            k,
            _lib.ptr(a_scales),
            _lib.ptr(b_scales),
            _lib.ptr(c),
            out_code,
            stream,
        )
    else:
        _lib.call(
            "m5k_gemm_float",
            _lib.ptr(a),
            _lib.ptr(b),
            _lib.dtype_code(a),
            m,
            n,
            k,
            _lib.ptr(c),
            out_code,
            _lib.ptr(residual),
            _lib.ptr(gate),
            _lib.ptr(gate_row_map),
            stream,
        )
    return c


def _mx_to_bf16(q, e, name):
    rows, k = q.shape
    if q.dtype != torch.int8 or e.dtype != torch.uint8 or tuple(e.shape) != (rows, k // 32):
        raise ValueError(f"MXINT8 {name} needs int8 codes [R,K] and uint8 exponents [R,K/32]")
    q = _lib.device_tensor(q, name)
    e = _lib.device_tensor(e, name + "_scales")
    y = torch.empty((rows, k), dtype=torch.bfloat16, device=q.device)
    _lib.call("m5k_mxint8_to_bf16", _lib.ptr(q), _lib.ptr(e), rows, k, _lib.ptr(y), _lib.stream_of(q))
    return y


def _gemm_mxint8(a, b, a_scales, b_scales, output_dtype):
    """MXINT8 linear (metal.py:81-86 plane scales): C = sum over 32-wide K blocks of
    2^(ea-127) 2^(eb-127) sum_k a b, FP32 accumulation.  Both operands expand exactly to BF16
    (|code| <= 127 times a power of two) and run on the BF16 MFMA GEMM."""
    m, k = a.shape
    if k % 32:
        raise ValueError("MXINT8 requires K divisible by 32")
    out_dtype = output_dtype or torch.float32
    if out_dtype not in _FLOAT_DTYPES:
        raise ValueError("output_dtype must be float16, bfloat16 or float32")
    ab = _mx_to_bf16(a, a_scales, "a")
    bb = _mx_to_bf16(b, b_scales, "b")
    c = torch.empty((m, b.shape[0]), dtype=out_dtype, device=ab.device)
    _lib.call("m5k_gemm_float", _lib.ptr(ab), _lib.ptr(bb), _lib.BF16, m, b.shape[0], k, _lib.ptr(c),
              _lib.dtype_code(c), None, None, None, _lib.stream_of(ab))
    return c


def gemm_i8_accumulators(a, b):
    """Raw INT32 accumulators sum_k a[m,k]*b[n,k] of the W8A8 main loop (parity hook)."""
    m, k = a.shape
    n, kb = b.shape
    if k != kb:
        raise ValueError("K mismatch")
    if a.dtype != torch.int8 or b.dtype != torch.int8:
        raise ValueError("accumulator hook requires int8 operands")
    if k > 133144:
        raise NotImplementedError("INT32 worst-case overflow bound exceeded")
    a = _lib.device_tensor(a, "a")
    b = _lib.device_tensor(b, "b")
    acc = torch.empty((m, n), dtype=torch.int32, device=a.device)
    _lib.call("m5k_gemm_i8_acc", _lib.ptr(a), _lib.ptr(b), m, n, k, _lib.ptr(acc), _lib.stream_of(a))
    return acc
