"""The shift-split projection (norm-shift-split backend, norm_hadamard_gemm.py:20-45,233-258,
320-484 of the reference) and its conditioning tables, through the C ABI.

Gates follow the reference's transform_pass: projected bias rel-L2 <= 1e-5 against float64
shift @ W.T; activation scales rel-L2 <= 1e-5 and codes within 1 of the float64 FP32-policy
reference; decoded activation and end-to-end projection rel-L2 <= 0.008 (implementation) and
<= 0.05 against the unquantized float64 projection (quality).  The combined factor
gamma * (1 + scale) is an exact FP32 expression and is held bitwise."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import np_of
from m5kernels_amd import gemm, norm_shift_split_gemm, quantize, rms_quantize, rotate, shift_split_condition
from oracle import reference as ref

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def _bf(a, device):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device).to(BF)


def _f64(t):
    return t.float().cpu().numpy().astype(np.float64)


def _bias_bound(shift, w):
    """Rigorous FP32 dot-product error bound: K u sum |s_j w_j| (any order, FMA or not)."""
    k = shift.shape[-1]
    return k * 2.0**-24 * (np.abs(shift) @ np.abs(w).T) * 1.01


@pytest.mark.parametrize("backend", ["mlx-fp32-convert", "mpp-bf16-to-fp32"])
@pytest.mark.parametrize("p,k,n", [(None, 768, 33), (3, 768, 520), (9, 1024, 257), (17, 5376, 300), (2, 100, 65)])
def test_condition_tables(backend, p, k, n, device):
    rng = np.random.default_rng(k + n)
    rows = 1 if p is None else p
    gamma = _bf(1 + 0.1 * rng.standard_normal(k), device)
    scale = _bf(0.2 * rng.standard_normal((rows, k)), device)
    shift = _bf(0.1 * rng.standard_normal((rows, k)), device)
    w = _bf(rng.standard_normal((n, k)), device)
    w[:, ::131] *= 20
    if p is None:
        scale, shift = scale[0], shift[0]
    combined, bias = shift_split_condition(gamma, scale, shift, w, bias_backend=backend)
    assert combined.dtype == torch.float32 and bias.dtype == torch.float32
    assert tuple(combined.shape) == tuple(scale.shape) and tuple(bias.shape) == ((n,) if p is None else (p, n))
    g32, s32 = gamma.float().cpu().numpy(), scale.float().cpu().numpy()
    np.testing.assert_array_equal(np_of(combined), g32 * (np.float32(1) + s32))
    sh, wf = _f64(shift).reshape(rows, k), _f64(w)
    expected = sh @ wf.T
    actual = np_of(bias).astype(np.float64).reshape(rows, n)
    assert ref.metrics(actual, expected)["relative_l2"] <= 1e-5
    assert np.all(np.abs(actual - expected) <= _bias_bound(sh, wf))


def test_bias_backends_agree(device):
    """BF16 products are exact in FP32, so reading BF16 directly or converting to FP32 first
    gives the same accumulation, bit for bit."""
    rng = np.random.default_rng(3)
    k, n = 5376, 1000
    gamma, scale, shift = (_bf(rng.standard_normal(k), device) for _ in range(3))
    w = _bf(rng.standard_normal((n, k)), device)
    a = shift_split_condition(gamma, scale, shift, w, bias_backend="mlx-fp32-convert")
    b = shift_split_condition(gamma, scale, shift, w, bias_backend="mpp-bf16-to-fp32")
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def _case(m, n, k, distribution, seed, device):
    """Inputs laid out as the reference's prepare does (norm_hadamard_gemm.py:46-62)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k), dtype=np.float32)
    w = rng.standard_normal((n, k), dtype=np.float32)
    if distribution == "zeros":
        x[:], w[:] = 0, 0
    elif distribution == "outliers":
        x = x * np.where(np.arange(k) % 127 == 0, 20, 1).astype(np.float32)
        w = w * np.where(np.arange(k) % 131 == 0, 20, 1).astype(np.float32)
    gamma = 1 + 0.1 * rng.standard_normal(k).astype(np.float32)
    scale = 0.2 * rng.standard_normal(k).astype(np.float32)
    shift = 0.1 * rng.standard_normal(k).astype(np.float32)
    return [_bf(v, device) for v in (x, w, gamma, scale, shift)]


@pytest.mark.parametrize("distribution", ["normal", "outliers", "zeros"])
@pytest.mark.parametrize("backend", ["mlx-fp32-convert", "mpp-bf16-to-fp32"])
@pytest.mark.parametrize("m,n,k", [(7, 33, 768), (300, 520, 1024), (129, 7168, 5376)])
def test_shift_split_projection(distribution, backend, m, n, k, device):
    block = 256
    x, w, gamma, scale, shift = _case(m, n, k, distribution, 29, device)
    signs_np = ref.hadamard_signs(k, 0)
    signs = torch.from_numpy(signs_np).to(device)
    wq, ws = quantize(rotate(w, block, signs), "int8")
    combined, bias = shift_split_condition(gamma, scale, shift, w, bias_backend=backend)
    y = norm_shift_split_gemm(x, wq, ws, signs, combined, bias, block)
    q, s = rms_quantize(x, combined, signs, block, fold_scale=True)
    torch.cuda.synchronize()
    assert y.dtype == BF and tuple(y.shape) == (m, n)
    # The online stage is exactly the two ops it names.
    assert torch.equal(y, gemm(q, wq, "int8", a_scales=s, b_scales=ws, output_dtype=BF, bias=bias))

    xf, wf, shf = _f64(x), _f64(w), _f64(shift)
    ref_norm = ref.norm_modulate_reference(xf, _f64(gamma), _f64(scale), shf)
    ref_bias = shf @ wf.T
    bias_err = ref.metrics(np_of(bias).astype(np.float64), ref_bias)
    assert bias_err["finite"] and (bias_err["relative_l2"] or 0.0) <= 1e-5
    # Activation against the float64 FP32-policy reference of the dynamic part.
    rotated = ref.block_hadamard_reference(ref_norm - shf, block, signs_np)
    peak = np.max(np.abs(rotated), axis=1)
    ref_scale = np.where(peak == 0, 1.0, peak / 127)
    ref_q = np.clip(np.rint(rotated / ref_scale[:, None]), -127, 127)
    sa, qa = np_of(s).astype(np.float64), np_of(q).astype(np.float64)
    assert np.isfinite(sa).all() and np.all(sa > 0)
    assert ref.metrics(sa, ref_scale)["relative_l2"] <= 1e-5
    assert np.max(np.abs(qa - ref_q)) <= 1
    decoded_a = qa * sa[:, None]
    if distribution != "zeros":
        assert ref.metrics(decoded_a, ref_q * ref_scale[:, None])["relative_l2"] <= 0.008
    # End to end: implementation gate against the decoded operands plus the actual bias, and
    # quality against the unquantized float64 projection of the modulated activation.
    decoded_w = np_of(wq).astype(np.float64) * np_of(ws).astype(np.float64)[:, None]
    expected = decoded_a @ decoded_w.T + np_of(bias).astype(np.float64)
    original = ref_norm @ wf.T
    yf = _f64(y)
    assert np.isfinite(yf).all()
    if distribution == "zeros":
        assert np.all(yf == 0)
    else:
        assert ref.metrics(yf, expected)["relative_l2"] <= 0.008
        assert ref.metrics(yf, original)["relative_l2"] <= 0.05


def test_zero_rows_keep_unit_scale_and_output_the_bias(device):
    """A zero dynamic row keeps zero codes and unit scale; its output is the cached bias, rounded
    once to BF16 (affine-shift-splitting contract)."""
    m, n, k, block = 6, 130, 512, 256
    x, w, gamma, scale, shift = _case(m, n, k, "normal", 5, device)
    x[1] = 0
    x[4] = 0
    signs = torch.ones(k, dtype=torch.int8, device=device)
    wq, ws = quantize(rotate(w, block, signs), "int8")
    combined, bias = shift_split_condition(gamma, scale, shift, w, bias_backend="mpp-bf16-to-fp32")
    q, s = rms_quantize(x, combined, signs, block, fold_scale=True)
    y = norm_shift_split_gemm(x, wq, ws, signs, combined, bias, block)
    for r in (1, 4):
        assert torch.count_nonzero(q[r]) == 0 and float(s[r]) == 1.0
        assert torch.equal(y[r], bias.to(BF))


def test_inputs_not_mutated(device):
    x, w, gamma, scale, shift = _case(16, 64, 256, "normal", 9, device)
    before = [t.clone() for t in (x, w, gamma, scale, shift)]
    signs = torch.ones(256, dtype=torch.int8, device=device)
    wq, ws = quantize(rotate(w, 256, signs), "int8")
    combined, bias = shift_split_condition(gamma, scale, shift, w)
    norm_shift_split_gemm(x, wq, ws, signs, combined, bias)
    assert all(torch.equal(a, b) for a, b in zip((x, w, gamma, scale, shift), before))
