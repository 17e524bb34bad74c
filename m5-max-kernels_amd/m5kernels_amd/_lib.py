"""ctypes binding of libm5k.so and the torch-tensor plumbing around it.

PyTorch-ROCm supplies device memory and the current HIP stream; every compute call
goes through the C ABI declared in include/m5k.h.  There is no fallback: if the
library is missing or a tensor is not on a ROCm device, the call raises.
"""

from __future__ import annotations

import ctypes
import functools
import re
from numbers import Integral, Real
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent.parent / "lib" / "libm5k.so"

F32, F16, BF16, I8, U8, I32 = 0, 1, 2, 3, 4, 5
QUANT_INT8, QUANT_FP8 = 0, 1
NORM_RMS, NORM_LAYER = 0, 1
PARAM_PER_TABLE = 0x100  # include/m5k.h M5K_PARAM_PER_TABLE


def param_tables(gamma: int, scale: int, shift: int, gate: int = BF16) -> int:
    """M5K_PARAM_TABLES(gamma, scale, shift, gate): one float dtype code per prep table."""
    return PARAM_PER_TABLE | gamma | (scale << 2) | (shift << 4) | (gate << 6)

_DTYPE_CODES = {
    torch.float32: F32,
    torch.float16: F16,
    torch.bfloat16: BF16,
    torch.int8: I8,
    torch.uint8: U8,
    torch.int32: I32,
}

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float

# name -> argtypes (restype is int status unless noted)
SIGNATURES = {
    "m5k_quantize_rows": [_p, _i32, _i64, _i64, _i32, _p, _p, _p],
    "m5k_quantize_mxint8": [_p, _i32, _i64, _i64, _p, _p, _p],
    "m5k_rms_quantize": [_p, _i32, _i64, _i64, _p, _p, _i32, _i32, _f32, _p, _p, _p],
    "m5k_shift_split_condition": [_p, _p, _i32, _p, _p, _i32, _i64, _i64, _i64, _p, _p, _p],
    "m5k_projection_qkv_rope": [_p, _p, _i32, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p, _i32, _f32, _p, _p, _p, _p],
    "m5k_mxint8_to_bf16": [_p, _p, _i64, _i64, _p, _p],
    "m5k_gemm_i8": [_p, _p, _i64, _i64, _i64, _p, _p, _p, _i32, _p, _p, _p, _p, _p, _p],
    "m5k_gemm_i8_acc": [_p, _p, _i64, _i64, _i64, _p, _p],
    "m5k_gemm_launch_plan": [_i32, _i64, _i64, _i32, _p, _p],
    "m5k_gemm_set_schedule": [_i32, _p],
    "m5k_gemm_i8_splitk": [_p, _p, _i64, _i64, _i64, _p, _p, _p, _i32, _p, _p, _p, _p, _p, _i32, _p, _i64, _p],
    "m5k_gemm_i8_splitk_noalloc": [_p, _p, _i64, _i64, _i64, _p, _p, _p, _i32, _p, _p, _p, _p, _p, _i32, _p],
    "m5k_gemm_f8": [_p, _p, _i64, _i64, _i64, _p, _p, _p, _i32, _p],
    "m5k_gemm_f8_splitk": [_p, _p, _i64, _i64, _i64, _p, _p, _p, _i32, _i32, _p, _i64, _p],
    "m5k_gemm_float": [_p, _p, _i32, _i64, _i64, _i64, _p, _i32, _p, _p, _p, _p],
    "m5k_hadamard_rotate": [_p, _i32, _i64, _i64, _i32, _p, _p, _p],
    "m5k_hadamard_quantize_rows": [_p, _i32, _i64, _i64, _i32, _p, _p, _p, _p],
    "m5k_norm_hadamard_quantize": [
        _p, _i32, _i64, _i64, _p, _i32, _p, _p, _p, _p, _p, _i32, _p, _p, _i32, _i32, _f32, _i32, _p, _p, _p, _p,
    ],
    "m5k_norm_modulate": [_p, _i32, _i64, _i64, _p, _p, _p, _i32, _p, _i32, _f32, _i32, _p, _p],
    "m5k_gated_residual_add": [_p, _i32, _i64, _i64, _p, _i32, _p, _i32, _p, _p, _p],
    "m5k_projection_qk_rope": [_p, _p, _i32, _i64, _i64, _i64, _p, _p, _p, _p, _p, _i32, _f32, _p, _p],
    "m5k_qk_norm_rope": [_p, _i64, _i64, _p, _p, _p, _i32, _f32, _p, _p],
}

_LIB = None


def load(path: Path | str | None = None) -> ctypes.CDLL:
    """Load libm5k.so once; raise if it has not been built."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    target = Path(path) if path is not None else LIB_PATH
    if not target.exists():
        raise RuntimeError(
            f"{target} is missing: build it with `python -m m5kernels_amd.build` "
            "(or __graft_entry__.build()); there is no CPU fallback"
        )
    lib = ctypes.CDLL(str(target))
    lib.m5k_last_error.restype = ctypes.c_char_p
    lib.m5k_last_error.argtypes = []
    lib.m5k_abi_version.restype = ctypes.c_int
    lib.m5k_abi_version.argtypes = []
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_int
    if path is None:
        _LIB = lib
    return lib


def call(name: str, *args) -> None:
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        raise RuntimeError(f"{name} failed ({rc}): {lib.m5k_last_error().decode(errors='replace')}")


def is_int(v) -> bool:
    """An integer that is not a bool (numbers.Integral), with plain int checked first."""
    return type(v) is int or (not isinstance(v, bool) and isinstance(v, Integral))


def is_real(v) -> bool:
    """A real number that is not a bool (numbers.Real), with plain float and int checked first."""
    return type(v) is float or type(v) is int or (not isinstance(v, bool) and isinstance(v, Real))


@functools.lru_cache(maxsize=256)
def _identifier(tag: str) -> bool:
    return re.fullmatch(r"[A-Za-z_][A-Za-z_0-9]*", tag) is not None


def is_identifier(tag) -> bool:
    """A nonempty string of identifier characters (the reference's kernel-name tag rule)."""
    return isinstance(tag, str) and _identifier(tag)


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPE_CODES[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {t.dtype}") from None


def device_tensor(t: torch.Tensor, name: str) -> torch.Tensor:
    """Contiguous view of a ROCm device tensor (copies strided inputs, never mutates)."""
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a torch.Tensor")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a ROCm device tensor (got {t.device}); there is no CPU path")
    return t.contiguous()


def ptr(t: torch.Tensor | None):
    """Device address of t (None for an absent operand).  Every entry point's argument types
    are declared in SIGNATURES, so ctypes converts the integer to a pointer itself."""
    return None if t is None else t.data_ptr()


# The current stream's raw handle by device index: the call torch's own generated launchers
# use.  torch.cuda.current_stream(device) returns the same handle, at ~4 us of Python per call.
_current_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor) -> int:
    """The raw HIP stream handle current on t's device (the launch stream of every op; 0 is the
    null stream)."""
    if _current_raw_stream is not None:
        return _current_raw_stream(t.device.index)
    return torch.cuda.current_stream(t.device).cuda_stream


def aligned_device_tensor(t: torch.Tensor, name: str) -> torch.Tensor:
    """Like device_tensor, but also guarantees a 16-byte aligned base (vector kernels)."""
    t = device_tensor(t, name)
    if t.data_ptr() % 16:
        t = t.clone()
    return t
