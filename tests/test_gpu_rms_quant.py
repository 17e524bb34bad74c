"""GPU parity of the RMS scale-folded INT8 quantizer (m5k_rms_quantize).

Bar, as the reference's own GPU test sets it (tests/test_rms_quant_metal.py:17-50 of the
reference): against an independent float64 expression (normalize first, FP32 gamma, dense
signed H), codes within 1, scales within rtol 3e-6, decoded error bounded by the two scales,
and the quantization error bounded against the unquantized float64 signal.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import np_of
from m5kernels_amd import rms_quantize
from oracle import reference as ref

pytestmark = pytest.mark.gpu


def _check(xt, gamma, signs, block, *, epsilon=1e-5, **kw):
    device = xt.device
    q, s = rms_quantize(xt, torch.from_numpy(gamma).to(device), torch.from_numpy(signs).to(device), block,
                        epsilon=epsilon, **kw)
    q, s = np_of(q), np_of(s)
    x = xt.float().cpu().numpy().astype(np.float64)
    inv = 1 / np.sqrt(np.mean(x * x, axis=1, keepdims=True) + epsilon)
    rotated = ref.block_hadamard_reference((x * inv) * gamma.astype(np.float64), block, signs)
    peak = np.max(np.abs(rotated), axis=1)
    ref_s = np.where(peak == 0, 1.0, peak / 127.0)
    ref_q = np.clip(np.rint(rotated / ref_s[:, None]), -127, 127).astype(np.int8)
    assert q.dtype == np.int8 and s.dtype == np.float32
    assert np.isfinite(s).all() and np.all(s > 0)
    assert np.max(np.abs(q.astype(np.int16) - ref_q.astype(np.int16))) <= 1
    np.testing.assert_allclose(s, ref_s, rtol=3e-6, atol=1e-30)
    decoded = q.astype(np.float64) * s[:, None]
    expected = ref_q.astype(np.float64) * ref_s[:, None]
    bound = np.maximum(s, ref_s) + 127 * np.abs(s - ref_s)
    assert np.all(np.abs(decoded - expected) <= bound[:, None] * (1 + 1e-12))
    qbound = (0.5 * ref_s + 127 * np.abs(s - ref_s))[:, None]
    assert np.all(np.abs(decoded - rotated) <= qbound + 2e-6 * peak[:, None])
    # the oracle's folded form (statistics of X, peak after gamma/H) agrees with the codes too
    folded = ref.rms_quantize_reference(x, gamma, signs, block, eps=epsilon)
    assert np.max(np.abs(q.astype(np.int16) - folded["quantized"].astype(np.int16))) <= 1
    return q, s


DT = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}


@pytest.mark.parametrize("block", [1, 128, 256])
@pytest.mark.parametrize("fold", [False, True])
@pytest.mark.parametrize("kind", ["normal", "zeros", "outliers", "weighted_peak", "epsilon"])
def test_reference_widths_and_tails(block, fold, kind, device):
    """tests/test_rms_quant_metal.py:53-90: width 5376 with a transform, 769 (ragged) without."""
    rng = np.random.default_rng(2021)
    width = 5376 if block > 1 else 769
    x = rng.standard_normal((7, width), dtype=np.float32)
    gamma = rng.uniform(-1.7, 1.7, size=width).astype(np.float32)
    if kind == "zeros":
        x.fill(0)
    elif kind == "outliers":
        x[:, ::137] *= 100
    elif kind == "weighted_peak":
        x[:, 0] = 100
        gamma[0] = 1e-3
        gamma[1::31] *= 100
    elif kind == "epsilon":
        x *= 1e-9
    q, s = _check(torch.from_numpy(x).to(device), gamma, ref.hadamard_signs(width, 61), block, fold_scale=fold)
    if kind == "zeros":
        assert np.all(q == 0) and np.all(s == 1)


@pytest.mark.parametrize("dtype", list(DT))
@pytest.mark.parametrize("block", [1, 32, 512, 1024])
def test_dtypes_and_blocks(dtype, block, device):
    rng = np.random.default_rng(block)
    width = 4096 if block > 1 else 1000
    x = rng.standard_normal((33, width), dtype=np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(width)).astype(np.float32)
    xt = torch.from_numpy(x).to(device).to(DT[dtype])
    for fold in (False, True):
        _check(xt, gamma, ref.hadamard_signs(width, 5), block, fold_scale=fold)


def test_fold_changes_only_the_scale_path(device):
    """Folding moves the inverse RMS into the scale: codes of the two modes agree within one
    (FP32 operation order differs) and the scales agree closely."""
    rng = np.random.default_rng(3)
    x = torch.from_numpy(rng.standard_normal((16, 4096), dtype=np.float32)).to(device).to(torch.bfloat16)
    gamma = torch.from_numpy((1 + 0.2 * rng.standard_normal(4096)).astype(np.float32)).to(device)
    signs = torch.from_numpy(ref.hadamard_signs(4096, 7)).to(device)
    qf, sf = rms_quantize(x, gamma, signs, 256, fold_scale=True)
    qn, sn = rms_quantize(x, gamma, signs, 256, fold_scale=False)
    assert int((qf.to(torch.int16) - qn.to(torch.int16)).abs().max()) <= 1
    np.testing.assert_allclose(np_of(sf), np_of(sn), rtol=1e-5)


def test_inputs_not_mutated_and_repeatable(device):
    rng = np.random.default_rng(4)
    x = torch.from_numpy(rng.standard_normal((8, 1024), dtype=np.float32)).to(device)
    gamma = torch.ones(1024, device=device)
    signs = torch.ones(1024, dtype=torch.int8, device=device)
    before = x.clone()
    a = rms_quantize(x, gamma, signs, 128)
    b = rms_quantize(x, gamma, signs, 128)
    assert torch.equal(x, before) and torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def _folded_codes_fp32(x32, gamma, signs, block):
    """The folded quantizer's code chain in FP32, independent of its reduction order:
    z = H(fl(x * gamma) * sign) in the pinned sequential stage order (c_hadamard_f32),
    peak = max |z|, code = clamp(rint(fl(fl(z / peak) * 127)), -127, 127) (0 for a zero peak)."""
    z = ref.c_hadamard_f32((x32 * gamma).astype(np.float32), block, signs)
    peak = np.max(np.abs(z), axis=1, keepdims=True).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        v = ((z / np.where(peak == 0, np.float32(1), peak)).astype(np.float32) * np.float32(127)).astype(np.float32)
    q = np.clip(np.rint(v), -127, 127).astype(np.int8)
    return np.where(peak == 0, np.int8(0), q)


@pytest.mark.parametrize("block", [128, 256])
def test_folded_codes_bit_exact_fp32_chain(block, device):
    """Codes of the folded quantizer equal the FP32 chain rint(fl(fl(z/peak)*127)) bit for bit
    (they do not depend on the statistics' summation order), on ordinary rows, outlier rows, a
    zero row and rows whose 127/peak leaves the encoder's fast range."""
    rng = np.random.default_rng(block + 5)
    x = rng.standard_normal((8, 4096)).astype(np.float32)
    x[1, ::97] *= 80
    x[2] = 0.0
    x[3] *= np.float32(1e35)
    x[4] *= np.float32(1e-33)
    gamma = rng.uniform(0.5, 1.5, size=4096).astype(np.float32)
    signs = ref.hadamard_signs(4096, 11)
    xt = torch.from_numpy(x).to(device)
    q, _ = rms_quantize(xt, torch.from_numpy(gamma).to(device), torch.from_numpy(signs).to(device), block,
                        fold_scale=True)
    np.testing.assert_array_equal(np_of(q), _folded_codes_fp32(x, gamma, signs, block))
