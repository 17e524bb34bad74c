"""The C ABI boundary on the CPU: libm5k.so loads, exports every declared entry point, and
its argument checks fail cleanly (no device work is launched by any call here)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from m5kernels_amd import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "m5k.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(m5k_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_hot_path():
    names = declared_functions()
    for required in ("m5k_quantize_rows", "m5k_gemm_i8", "m5k_gemm_f8", "m5k_hadamard_rotate", "m5k_last_error"):
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert set(_lib.SIGNATURES) <= set(declared_functions())
    assert lib.m5k_abi_version() == 100


def test_argument_checks_return_einval_without_launching():
    lib = _lib.load()
    null = None
    assert lib.m5k_quantize_rows(null, _lib.BF16, 4, 8, 0, null, null, null) == 1
    assert b"null" in lib.m5k_last_error()
    fake = ctypes.c_void_p(16)  # never dereferenced: the shape check fails first
    assert lib.m5k_quantize_rows(fake, _lib.BF16, 0, 8, 0, fake, fake, null) == 1
    assert b"empty" in lib.m5k_last_error()
    assert lib.m5k_quantize_rows(fake, _lib.BF16, 4, 8, 7, fake, fake, null) == 1
    assert b"mode" in lib.m5k_last_error()
    assert lib.m5k_gemm_i8(fake, fake, 4, 4, 133145, fake, fake, fake, _lib.BF16, null, null, null, null, null,
                           null) == 1
    assert b"133144" in lib.m5k_last_error()
    assert lib.m5k_gemm_f8(fake, fake, 4, 4, 96, fake, fake, fake, _lib.BF16, null) == 1
    assert b"multiple of 128" in lib.m5k_last_error()
    assert lib.m5k_gemm_i8(fake, fake, 4, 4, 64, fake, fake, fake, _lib.BF16, fake, null, fake, fake, null,
                           null) == 1
    assert b"cannot be combined" in lib.m5k_last_error()
    assert lib.m5k_hadamard_rotate(fake, _lib.BF16, 2, 96, 64, fake, fake, null) == 1
    assert b"divisible" in lib.m5k_last_error()
    assert lib.m5k_hadamard_rotate(fake, _lib.BF16, 2, 96, 48, fake, fake, null) == 1
    assert b"block" in lib.m5k_last_error()


def test_product_path_never_imports_the_oracle():
    pkg = Path(_lib.__file__).resolve().parent
    for src in pkg.glob("*.py"):
        assert "oracle" not in src.read_text().replace("oracle/", ""), src


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        _lib.load(tmp_path / "libm5k.so")


def test_prep_param_dtype_codes():
    """M5K_PARAM_TABLES as the header defines it, and the prep entry points' checks of it (they
    fail before any launch: the pointers below are never dereferenced)."""
    text = HEADER.read_text()
    assert int(re.search(r"#define M5K_PARAM_PER_TABLE (0x[0-9a-fA-F]+)", text).group(1), 16) == _lib.PARAM_PER_TABLE
    assert "((gamma) | ((scale) << 2) | ((shift) << 4) | ((gate) << 6))" in text.replace("M5K_PARAM_PER_TABLE | ", "(")
    assert _lib.param_tables(_lib.F16, _lib.F32, _lib.BF16, _lib.F16) == 0x100 | 1 | (0 << 2) | (2 << 4) | (1 << 6)
    lib = _lib.load()
    fake = ctypes.c_void_p(64)
    args = lambda pdt: (fake, _lib.BF16, 2, 256, None, _lib.BF16, None, None, fake, fake, fake, pdt, None, fake,  # noqa: E731
                        128, _lib.NORM_RMS, ctypes.c_float(1e-5), 1, fake, fake, None, None)
    assert lib.m5k_norm_hadamard_quantize(*args(7)) == 1
    assert b"neither a float dtype code" in lib.m5k_last_error()
    assert lib.m5k_norm_hadamard_quantize(*args(_lib.PARAM_PER_TABLE | 3)) == 1
    assert b"M5K_PARAM_TABLES fields" in lib.m5k_last_error()
    assert lib.m5k_norm_modulate(fake, _lib.BF16, 2, 256, fake, fake, fake, 0x2FF, None, _lib.NORM_RMS,
                                 ctypes.c_float(1e-5), 1, fake, None) == 1
    assert b"neither a float dtype code" in lib.m5k_last_error()
