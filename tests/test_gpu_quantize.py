"""GPU parity of the per-row quantizer (m5k_quantize_rows) against the CPU oracle.

Bar: bit-exact codes and bit-exact FP32 scales (the reference itself demands exact codes,
tests/test_metal.py:70-82 of the reference, scale rtol 1e-6; we hold scales exactly).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bits_of, np_of
from m5kernels_amd import quantize
from oracle import reference as ref

pytestmark = pytest.mark.gpu

DTYPES = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}


def _input(kind, shape, seed=41):
    x = np.random.default_rng(seed).standard_normal(shape, dtype=np.float32)
    if kind == "zeros":
        x.fill(0)
    elif kind == "outliers":
        x[:, ::31] *= 30
    return x


def _check(xt, mode):
    q, s = quantize(xt, mode)
    torch.cuda.synchronize()
    x32 = xt.float().cpu().numpy()  # exact decode of the stored input
    rq, rs = ref.quantize_reference(x32, mode)
    assert q.dtype == (torch.uint8 if mode == "fp8" else torch.int8)
    np.testing.assert_array_equal(np_of(q), rq)
    np.testing.assert_array_equal(np_of(s), rs)
    return q, s


@pytest.mark.parametrize("mode", ["int8", "fp8"])
@pytest.mark.parametrize("kind", ["normal", "zeros", "outliers"])
@pytest.mark.parametrize("dtype", list(DTYPES))
@pytest.mark.parametrize("shape", [(7, 256), (3, 5376), (5, 100), (2, 33), (4, 40000), (3, 24576)])
def test_quantizer_bit_exact(mode, kind, dtype, shape, device):
    x = _input(kind, shape)
    _check(torch.from_numpy(x).to(device).to(DTYPES[dtype]), mode)


def test_config1_activation_bit_exact_vs_c_oracle(device):
    rng = np.random.default_rng(0)
    a = rng.standard_normal((256, 1024), dtype=np.float32)
    at = torch.from_numpy(a).to(device).to(torch.bfloat16)
    q, s = quantize(at, "int8")
    rq, rs = ref.c_quantize_rows(bits_of(at), "int8")
    np.testing.assert_array_equal(np_of(q), rq)
    np.testing.assert_array_equal(np_of(s), rs)


@pytest.mark.parametrize("mode", ["int8", "fp8"])
def test_ffn_down_activation_full_size_bit_exact(mode, device):
    """FFN-down activation [4096, 16384] bf16 with 0.1% x50 outlier channels."""
    g = torch.Generator(device="cpu").manual_seed(29)
    a = torch.randn((4096, 16384), generator=g, dtype=torch.float32)
    a[:, ::1024] *= 50
    at = a.to(device).to(torch.bfloat16)
    q, s = quantize(at, mode)
    rq, rs = ref.c_quantize_rows(bits_of(at), mode)
    np.testing.assert_array_equal(np_of(s), rs)
    np.testing.assert_array_equal(np_of(q), rq)


@pytest.mark.parametrize("mode", ["int8", "fp8"])
@pytest.mark.parametrize("dtype", list(DTYPES))
@pytest.mark.parametrize("rows,k", [(2048, 2048), (2051, 4096), (3001, 8192), (2049, 16384), (2500, 1000)])
def test_many_rows_bit_exact(mode, dtype, rows, k, device):
    """Long batches at each register-chunk width (K 1000..16384), odd row counts, outlier
    columns and one all-zero row."""
    g = torch.Generator(device="cpu").manual_seed(rows + k)
    x = torch.randn((rows, k), generator=g, dtype=torch.float32)
    x[:, ::97] *= 40
    x[rows // 3] = 0  # one all-zero row mid-stream
    xt = x.to(device).to(DTYPES[dtype])
    q, s = quantize(xt, mode)
    src = bits_of(xt) if dtype == "bf16" else xt.float().cpu().numpy()
    rq, rs = ref.c_quantize_rows(src, mode)
    np.testing.assert_array_equal(np_of(s), rs)
    np.testing.assert_array_equal(np_of(q), rq)


@pytest.mark.parametrize("dtype,m", [("fp16", 7), ("fp32", 7), ("fp32", 4095)])
def test_int8_dense_ties_bit_exact(dtype, m, device):
    """Rows with peak 127 m make the scale exactly m, so x = m (n + 1/2) is an exact tie of
    x / scale; x * fl(1/m) misses the tie for 78 (m = 7) or 126 (m = 4095) of the 254 values,
    so those elements must take the division path.  Neighbours one ulp either side of each tie
    check the rounding just off the boundary."""
    n = np.arange(-127, 127, dtype=np.float32)
    ties = np.float32(m) * (n + np.float32(0.5))
    row = np.concatenate([[127.0 * m], ties, np.nextafter(ties, np.float32(np.inf)), np.nextafter(ties, -np.float32(np.inf))])
    row = np.resize(row.astype(np.float32), 2048)
    x = np.stack([row, -row, np.roll(row, 5)])
    xt = torch.from_numpy(x).to(device).to(DTYPES[dtype])
    q, s = quantize(xt, "int8")
    x32 = xt.float().cpu().numpy()
    rq, rs = ref.c_quantize_rows(x32, "int8")
    assert np.all(rs == np.float32(m))
    fast = np.clip(np.rint(x32 * (np.float32(1) / np.float32(m))), -127, 127).astype(np.int8)
    assert np.count_nonzero(fast != rq) > 0  # the reciprocal alone would fail this row
    np.testing.assert_array_equal(np_of(s), rs)
    np.testing.assert_array_equal(np_of(q), rq)


@pytest.mark.parametrize("dtype", list(DTYPES))
def test_nan_ignored_by_row_peak(dtype, device):
    """The row peak ignores NaN like the reference's max (quantize.metal:7); the codes of the
    finite elements are unaffected.  (A NaN's own code has no defined value in the reference.)"""
    x = _input("outliers", (6, 4096), seed=5)
    x[0, 17] = np.nan
    x[1, :8] = np.nan
    x[2, 4095] = np.nan
    x[3, ::2] = np.nan
    xt = torch.from_numpy(x).to(device).to(DTYPES[dtype])
    q, s = quantize(xt, "int8")
    x32 = xt.float().cpu().numpy()
    rq, rs = ref.c_quantize_rows(x32, "int8")
    np.testing.assert_array_equal(np_of(s), rs)
    finite = np.isfinite(x32)
    np.testing.assert_array_equal(np_of(q)[finite], rq[finite])


@pytest.mark.parametrize("mode", ["int8", "fp8"])
@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
def test_extreme_row_scales_bit_exact(mode, dtype, device):
    """Rows whose reciprocal scale leaves the encoder's fast range (peak ~1e-33: scale below
    2^-100; peak ~1e37: reciprocal below 2^-100) take the exact chain for the whole row; a
    row holding +-inf has an infinite scale and codes 0 for its finite elements, as the IEEE
    division gives.  Finite elements' codes and every scale bit-exact against the oracle."""
    rng = np.random.default_rng(77)
    x = rng.standard_normal((6, 4096)).astype(np.float32)
    x[0] *= np.float32(1e-33)
    x[1] *= np.float32(1e-35)
    x[2] *= np.float32(1e37)
    x[3, 100] = np.inf
    x[4, 7] = -np.inf
    x[5] *= np.float32(2.5e-29)  # scale near 2^-100, the switch to the exact chain
    xt = torch.from_numpy(x).to(device).to(DTYPES[dtype])
    q, s = quantize(xt, mode)
    x32 = xt.float().cpu().numpy()
    rq, rs = ref.c_quantize_rows(x32, mode)
    np.testing.assert_array_equal(np_of(s), rs)
    finite = np.isfinite(x32)
    np.testing.assert_array_equal(np_of(q)[finite], rq[finite])


def test_round_half_even_kat(kats, device):
    kat = kats["int8_round_half_even"]
    x = torch.tensor([kat["row"]] * 3, dtype=torch.float32, device=device)
    q, s = quantize(x, "int8")
    np.testing.assert_array_equal(np_of(q), np.tile(kat["codes"], (3, 1)))
    np.testing.assert_array_equal(np_of(s), kat["scale"])


def test_fp8_encoder_kat_and_all_codes(kats, device):
    kat = kats["fp8_encode"]
    # With the row peak at 448 the scale is exactly 1, so codes are fp8_encode(x) itself.
    row = [v for v in kat["x"] if abs(v) <= 448]
    codes = [c for v, c in zip(kat["x"], kat["codes"]) if abs(v) <= 448]
    q, s = quantize(torch.tensor([row], dtype=torch.float32, device=device), "fp8")
    assert float(s[0]) == 1.0
    np.testing.assert_array_equal(np_of(q)[0], codes)
    every = np.concatenate([np.arange(127), np.arange(128, 255)]).astype(np.uint8)
    q, s = quantize(torch.from_numpy(ref.fp8_decode(every)[None, :]).to(device), "fp8")
    assert float(s[0]) == 1.0
    np.testing.assert_array_equal(np_of(q)[0], every)


def test_fp8_ties_and_saturation(device):
    table = ref.fp8_decode(np.arange(127, dtype=np.uint8)).astype(np.float64)
    mids = ((table[:-1] + table[1:]) / 2).astype(np.float32)
    row = np.concatenate([[448.0], mids, -mids, np.nextafter(mids, np.float32(0)), [447.99]]).astype(np.float32)
    q, s = quantize(torch.from_numpy(row[None, :]).to(device), "fp8")
    assert float(s[0]) == 1.0
    np.testing.assert_array_equal(np_of(q)[0], ref.fp8_encode(row))


@pytest.mark.parametrize("m", [7, 4095])
def test_fp8_dense_ties_bit_exact(m, device):
    """Rows with peak 448 m make the scale exactly m, so x = m * (midpoint of two adjacent E4M3
    values) is an exact tie of x / scale.  The reciprocal product misses some ties, so the
    encoder's bracket check must send those groups to the IEEE division; neighbours one ulp
    either side check the rounding just off each boundary, and -x the sign."""
    table = ref.fp8_decode(np.arange(127, dtype=np.uint8)).astype(np.float64)
    mids = ((table[:-1] + table[1:]) / 2) * m
    ties = mids.astype(np.float32)
    assert np.all(ties.astype(np.float64) == mids)  # exact in float32
    row = np.concatenate([[448.0 * m], ties, np.nextafter(ties, np.float32(np.inf)),
                          np.nextafter(ties, np.float32(0))]).astype(np.float32)
    row = np.resize(row, 2048)
    x = np.stack([row, -row, np.roll(row, 3)])
    q, s = quantize(torch.from_numpy(x).to(device), "fp8")
    rq, rs = ref.c_quantize_rows(x, "fp8")
    assert np.all(rs == np.float32(m))
    fast = ref.fp8_encode((x * (np.float32(1) / np.float32(m))).astype(np.float32))
    assert np.count_nonzero(fast != rq) > 0  # the reciprocal alone would fail these rows
    np.testing.assert_array_equal(np_of(s), rs)
    np.testing.assert_array_equal(np_of(q), rq)


def test_inputs_not_mutated_and_strided(device):
    base = torch.randn(64, 512, device=device, dtype=torch.bfloat16)
    view = base[:, ::2]
    before = base.clone()
    q, s = quantize(view, "int8")
    rq, rs = ref.quantize_reference(view.float().cpu().numpy(), "int8")
    np.testing.assert_array_equal(np_of(q), rq)
    assert torch.equal(base, before)


# ---- MXINT8 block quantizer (numerics.py:33-41) ----------------------------------------------


@pytest.mark.parametrize("dtype", list(DTYPES))
@pytest.mark.parametrize("shape", [(3, 32), (5, 4096), (129, 320), (2, 16384)])
def test_mxint8_bit_exact(dtype, shape, device):
    rng = np.random.default_rng(shape[0] * 7 + shape[1])
    lo, hi = (-10, 10) if dtype == "fp16" else (-30, 30)  # stay inside the fp16 range
    x = rng.standard_normal(shape).astype(np.float32) * np.exp2(rng.integers(lo, hi, (shape[0], 1)))
    x[:, 64:96] = 0  # an all-zero block where present
    xt = torch.from_numpy(x.astype(np.float32)).to(device).to(DTYPES[dtype])
    q, e = quantize(xt, "mxint8")
    assert q.dtype == torch.int8 and e.dtype == torch.uint8 and tuple(e.shape) == (shape[0], shape[1] // 32)
    rq, re_ = ref.quantize_reference(xt.float().cpu().numpy(), "mxint8")
    np.testing.assert_array_equal(np_of(e), re_)
    np.testing.assert_array_equal(np_of(q), rq)


def test_mxint8_kats_and_power_of_two_peaks(kats, device):
    kat = kats["mx_scale_boundaries"]
    q, e = quantize(torch.tensor(kat["x_rows"], dtype=torch.float32, device=device), "mxint8")
    np.testing.assert_array_equal(np_of(q), np.array(kat["codes"], np.int8))
    np.testing.assert_array_equal(np_of(e), np.array(kat["scales"], np.uint8))
    # Block peaks within 40 ulps either side of 2^k for k in [-120, 120]: the rounded FP32 log2
    # reaches k just below 2^k (exponent one higher than the peak's own), as in the reference.
    peaks = []
    for k in range(-120, 121, 3):
        p = np.float32(2.0**k)
        lo, hi = p, p
        for _ in range(40):
            lo, hi = np.nextafter(lo, np.float32(0)), np.nextafter(hi, np.float32(np.inf))
            peaks += [lo, hi]
    peaks = np.array(peaks, np.float32)
    rng = np.random.default_rng(11)
    x = (rng.uniform(-1, 1, (peaks.size, 32)) * peaks[:, None]).astype(np.float32)
    x[:, 7] = peaks * np.where(rng.random(peaks.size) < 0.5, -1, 1).astype(np.float32)
    q, e = quantize(torch.from_numpy(x).to(device), "mxint8")
    rq, re_ = ref.quantize_reference(x, "mxint8")
    np.testing.assert_array_equal(np_of(e), re_)
    np.testing.assert_array_equal(np_of(q), rq)
