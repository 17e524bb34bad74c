"""GPU parity of the fused Q/K projection + RMSNorm + RoPE (m5k_projection_qk_rope) and the
staged postprocess (m5k_qk_norm_rope).

Bars: INT8 fused == staged (quantize -> gemm bf16 -> qk_norm_rope) bit for bit, as the reference
requires (tests/test_qk_rope_metal.py:78-81 of the reference), and here also for BF16 since both
paths share one main loop; both within rel-L2 1e-3 of the float64 reference fed the exact
projection (the north-star RoPE bar; the reference's own gate is 0.008).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from helpers import bits_of, np_of
from m5kernels_amd import gemm, projection_qk_rope, qk_norm_rope, quantize
from oracle import reference as ref

pytestmark = pytest.mark.gpu


def _f32(t):
    return t.float().cpu().numpy()


def _tables(rng, m, device, rope_half=48):
    gamma = torch.from_numpy(rng.uniform(-1.5, 1.5, 128).astype(np.float32)).to(device).to(torch.bfloat16)
    angles = rng.uniform(-4, 4, (m, rope_half)).astype(np.float32)
    cos = torch.from_numpy(np.cos(angles)).to(device).to(torch.bfloat16)
    sin = torch.from_numpy(np.sin(angles)).to(device).to(torch.bfloat16)
    return gamma, cos, sin


def _check(actual, expected, tol=1e-3):
    assert actual.dtype == torch.bfloat16
    got = _f32(actual)
    assert np.isfinite(got).all()
    assert ref.metrics(got, expected)["relative_l2"] < tol


def _projection(a, b, mode, sa=None, sb=None):
    """Exact projection: INT32 dot then the FP32 dequant order (float64 for BF16)."""
    if mode == "int8":
        dot = np_of(a).astype(np.int64) @ np_of(b).astype(np.int64).T
        return (dot.astype(np.float32) * np_of(sa)[:, None]) * np_of(sb)[None, :]
    return _f32(a).astype(np.float64) @ _f32(b).astype(np.float64).T


@pytest.mark.parametrize("mode", ["int8", "bf16"])
@pytest.mark.parametrize(
    "shape,tile",
    [
        ((1, 128, 33), (16, 128, 4, 1)),
        ((17, 384, 96), (32, 128, 4, 8)),
        ((65, 256, 257), (64, 128, 8, 1)),
        ((129, 128, 33), (128, 128, 4, 8)),
        ((1, 128, 5376), (128, 64, 8, 8)),
        ((300, 640, 1024), (64, 128, 4, 8)),
        ((7, 128, 16), (16, 128, 8, 1)),
    ],
)
@pytest.mark.parametrize("rope_half", [48, 64])
def test_fused_projection_tiles_tails_and_reference(mode, shape, tile, rope_half, device):
    """Fused and staged Q/K equal bitwise and match the reference; R = 64 takes the DPP
    partner exchange (lane lg ^ 8), R = 48 the general shuffle."""
    rng = np.random.default_rng(117)
    m, n, k = shape
    a = torch.from_numpy(rng.standard_normal((m, k), dtype=np.float32)).to(device).to(torch.bfloat16)
    b = torch.from_numpy(rng.standard_normal((n, k), dtype=np.float32)).to(device).to(torch.bfloat16)
    gamma, cos, sin = _tables(rng, m, device, rope_half)
    scales = {}
    if mode == "int8":
        a, sa = quantize(a, "int8")
        b, sb = quantize(b, "int8")
        scales = dict(a_scales=sa, b_scales=sb)
    projected = _projection(a, b, mode, scales.get("a_scales"), scales.get("b_scales"))
    expected = ref.qk_rope_reference(projected.reshape(m, n // 128, 128), _f32(gamma), _f32(cos), _f32(sin))["output"]
    fused = projection_qk_rope(a, b, gamma, cos, sin, mode, tile, **scales)
    staged = qk_norm_rope(gemm(a, b, mode, tile, output_dtype=torch.bfloat16, **scales), gamma, cos, sin)
    assert fused.shape == staged.shape == (n // 128, m, 128)
    _check(fused, expected)
    _check(staged, expected)
    np.testing.assert_array_equal(bits_of(fused), bits_of(staged))


@pytest.mark.parametrize("mode", ["int8", "bf16"])
@pytest.mark.parametrize("kind", ["zeros", "outliers"])
def test_zeros_outliers_and_input_immutability(mode, kind, device):
    rng = np.random.default_rng(33)
    a_np = rng.standard_normal((7, 257), dtype=np.float32)
    b_np = rng.standard_normal((384, 257), dtype=np.float32)
    if kind == "zeros":
        a_np.fill(0)
        b_np.fill(0)
    else:
        a_np[:, ::31] *= 100
        b_np[:, ::17] *= 100
    a = torch.from_numpy(a_np).to(device).to(torch.bfloat16)
    b = torch.from_numpy(b_np).to(device).to(torch.bfloat16)
    gamma, cos, sin = _tables(rng, 7, device)
    scales = {}
    if mode == "int8":
        a, sa = quantize(a, "int8")
        b, sb = quantize(b, "int8")
        scales = dict(a_scales=sa, b_scales=sb)
    inputs = [a, b, gamma, cos, sin, *scales.values()]
    saved = [t.clone() for t in inputs]
    y = projection_qk_rope(a, b, gamma, cos, sin, mode, (32, 64, 4, 8), **scales)
    projected = _projection(a, b, mode, scales.get("a_scales"), scales.get("b_scales"))
    expected = ref.qk_rope_reference(projected.reshape(7, 3, 128), _f32(gamma), _f32(cos), _f32(sin))["output"]
    _check(y, expected)
    if kind == "zeros":
        assert torch.all(y == 0)
    for t, s in zip(inputs, saved):
        assert torch.equal(t, s)


@pytest.mark.parametrize("rope_half", [1, 48, 64])
def test_standalone_norm_rope_reference(rope_half, device):
    rng = np.random.default_rng(713)
    p_np = rng.standard_normal((5, 3, 128), dtype=np.float32)
    p_np[0] = 0
    p_np[1, :, ::31] *= 100
    p = torch.from_numpy(p_np.reshape(5, 384)).to(device).to(torch.bfloat16)
    gamma, cos, sin = _tables(rng, 5, device, rope_half)
    for threads in (128, 256):
        y = qk_norm_rope(p, gamma, cos, sin, threads=threads)
        expected = ref.qk_rope_reference(_f32(p).reshape(5, 3, 128), _f32(gamma), _f32(cos), _f32(sin))["output"]
        _check(y, expected)
        assert torch.all(y[:, 0] == 0)


def test_split_half_pairs_unrotated_tail_and_head_major_layout(device):
    p_np = np.ones((3, 2, 128), dtype=np.float32)
    p_np[:, :, 48:96] = -1
    p_np[:, 1] *= -1
    p = torch.from_numpy(p_np.reshape(3, 256)).to(device).to(torch.bfloat16)
    gamma = torch.ones(128, dtype=torch.bfloat16, device=device)
    cos = torch.zeros((3, 48), dtype=torch.bfloat16, device=device)
    sin = torch.ones((3, 48), dtype=torch.bfloat16, device=device)
    y = qk_norm_rope(p, gamma, cos, sin)
    expected = p_np.copy()
    expected[:, :, :48] = -p_np[:, :, 48:96]
    expected[:, :, 48:96] = p_np[:, :, :48]
    np.testing.assert_array_equal(_f32(y), expected.transpose(1, 0, 2))


def test_no_bf16_norm_intermediate(device):
    values = np.ones((3, 2, 128), dtype=np.float32)
    values[:, :, 127] = 2
    gamma_np = np.ones(128, dtype=np.float32)
    gamma_np[0] = 1 + 1 / 128
    p = torch.from_numpy(values.reshape(3, 256)).to(device).to(torch.bfloat16)
    gamma = torch.from_numpy(gamma_np).to(device).to(torch.bfloat16)
    cos = torch.full((3, 48), 181 / 256, dtype=torch.bfloat16, device=device)
    sin = torch.full((3, 48), 181 / 256, dtype=torch.bfloat16, device=device)
    native = ref.qk_rope_reference(values, _f32(gamma), _f32(cos), _f32(sin))
    rounded = ref.qk_rope_reference(values, _f32(gamma), _f32(cos), _f32(sin), norm_bf16=True)
    actual = _f32(qk_norm_rope(p, gamma, cos, sin))
    np.testing.assert_array_equal(actual[:, :, 0], native["output"][:, :, 0])
    assert not np.array_equal(actual[:, :, 0], rounded["output"][:, :, 0])


@pytest.mark.parametrize("tile", [(16, 64, 4, 3), (32, 128, 4, 1)])
def test_tiny_projection_preserves_dequant_scales(tile, device):
    rng = np.random.default_rng(137)
    m, n, k = 3, 256, 257
    a_np = rng.integers(-7, 8, size=(m, k), dtype=np.int8)
    b_np = rng.integers(-7, 8, size=(n, k), dtype=np.int8)
    sa_np = np.array([1e-4, 1e-5, 5e-5], dtype=np.float32)
    sb_np = np.full(n, 1e-3, dtype=np.float32)
    gamma, cos, sin = _tables(rng, m, device)
    dot = a_np.astype(np.int64) @ b_np.astype(np.int64).T
    projected = ((dot.astype(np.float32) * sa_np[:, None]) * sb_np[None, :]).reshape(m, n // 128, 128)
    expected = ref.qk_rope_reference(projected, _f32(gamma), _f32(cos), _f32(sin))["output"]
    wrong = ref.qk_rope_reference(projected * 2, _f32(gamma), _f32(cos), _f32(sin))["output"]
    assert ref.metrics(wrong, expected)["relative_l2"] > 0.5
    y = projection_qk_rope(torch.from_numpy(a_np).to(device), torch.from_numpy(b_np).to(device), gamma, cos, sin,
                           "int8", tile, a_scales=torch.from_numpy(sa_np).to(device),
                           b_scales=torch.from_numpy(sb_np).to(device))
    _check(y, expected, tol=8e-3)
    assert ref.metrics(_f32(y), wrong)["relative_l2"] > 0.4


def test_qk_configuration_shape(device):
    """x bf16 [9914, 4096], Wq [4096, 4096] ~N(0, 0.02), 32 heads x 128, eps 1e-6, gamma ~1+N(0,.02),
    RoPE base 10000 over positions 0..9913 (R = 64); online INT8 and BF16 projections."""
    m, k, n = 9914, 4096, 4096
    g = torch.Generator(device=device).manual_seed(43)
    x = torch.randn((m, k), generator=g, device=device).to(torch.bfloat16)
    w = (0.02 * torch.randn((n, k), generator=g, device=device)).to(torch.bfloat16)
    gamma = (1 + 0.02 * torch.randn(128, generator=g, device=device)).to(torch.bfloat16)
    inv_freq = 10000.0 ** (-torch.arange(0, 64, dtype=torch.float64) * 2 / 128)
    angles = torch.arange(m, dtype=torch.float64)[:, None] * inv_freq[None, :]
    cos = torch.cos(angles).float().to(device).to(torch.bfloat16)
    sin = torch.sin(angles).float().to(device).to(torch.bfloat16)
    rows = ref.sample_indices(m)
    for mode in ("int8", "bf16"):
        if mode == "int8":
            aq, sa = quantize(x, "int8")
            wq, sw = quantize(w, "int8")
            y = projection_qk_rope(aq, wq, gamma, cos, sin, "int8", a_scales=sa, b_scales=sw, epsilon=1e-6)
            staged = qk_norm_rope(gemm(aq, wq, "int8", a_scales=sa, b_scales=sw, output_dtype=torch.bfloat16),
                                  gamma, cos, sin, epsilon=1e-6)
            dot = np_of(aq)[rows].astype(np.int64) @ np_of(wq).astype(np.int64).T
            proj = (dot.astype(np.float32) * np_of(sa)[rows][:, None]) * np_of(sw)[None, :]
        else:
            y = projection_qk_rope(x, w, gamma, cos, sin, "bf16", epsilon=1e-6)
            staged = qk_norm_rope(gemm(x, w, "bf16", output_dtype=torch.bfloat16), gamma, cos, sin, epsilon=1e-6)
            proj = _f32(x[rows]).astype(np.float64) @ _f32(w).astype(np.float64).T
        assert y.shape == (32, m, 128)
        assert torch.equal(y, staged)
        expected = ref.qk_rope_reference(proj.reshape(len(rows), 32, 128), _f32(gamma), _f32(cos)[rows],
                                         _f32(sin)[rows], epsilon=1e-6)["output"]
        _check(y[:, rows], expected)
        assert math.isfinite(float(y.float().abs().max()))


# ---- grouped Q/K/V layout (integrations/h3/qkv_candidate.metal, qkv_reference.h) ------------


@pytest.mark.parametrize("mode", ["int8", "bf16"])
@pytest.mark.parametrize("rope_half", [48, 5])
@pytest.mark.parametrize("m,heads", [(300, 3), (129, 2)])
def test_grouped_qkv_equals_staged(mode, rope_half, m, heads, device):
    """Q and K of the grouped layout equal the staged qk_norm_rope of their projection blocks
    bit for bit; V equals the BF16 projection itself, head-major.  Three heads give 1152
    columns, so 256-column tiles mix streams and heads; M = 300 / 129 leaves partial row tiles."""
    from m5kernels_amd import projection_qkv_rope

    rng = np.random.default_rng(31 + m + heads + rope_half)
    k = 512
    x = torch.from_numpy(rng.standard_normal((m, k), dtype=np.float32)).to(device).to(torch.bfloat16)
    w = torch.from_numpy((rng.standard_normal((heads * 384, k)) * 0.05).astype(np.float32)).to(device).to(torch.bfloat16)
    q_gamma, cos, sin = _tables(rng, m, device, rope_half)
    k_gamma = torch.from_numpy(rng.uniform(0.5, 1.5, 128).astype(np.float32)).to(device).to(torch.bfloat16)
    if mode == "int8":
        a, sa = quantize(x, "int8")
        b, sb = quantize(w, "int8")
        q, kk, v = projection_qkv_rope(a, b, q_gamma, k_gamma, cos, sin, "int8", a_scales=sa, w_scales=sb)
        proj = gemm(a, b, "int8", a_scales=sa, b_scales=sb, output_dtype=torch.bfloat16)
    else:
        q, kk, v = projection_qkv_rope(x, w, q_gamma, k_gamma, cos, sin, "bf16")
        proj = gemm(x, w, "bf16", output_dtype=torch.bfloat16)
    blocks = proj.view(m, heads, 3, 128)
    for stream, (out, gamma) in enumerate(((q, q_gamma), (kk, k_gamma))):
        staged = qk_norm_rope(blocks[:, :, stream, :].reshape(m, heads * 128), gamma, cos, sin, epsilon=1e-6)
        assert torch.equal(out, staged), f"stream {stream}"
    assert torch.equal(v, blocks[:, :, 2, :].permute(1, 0, 2).contiguous())
    assert q.shape == kk.shape == v.shape == (heads, m, 128)


@pytest.mark.parametrize("m", [1, 17, 128, 200])
def test_short_m_routing_matches_fused_kernel(m, device):
    """Short-M INT8 projections take the split-K GEMM plus the staged postprocess; the result
    equals the fused kernel's (called through the C ABI directly) bit for bit."""
    from m5kernels_amd import _lib
    from m5kernels_amd.hip import splitk_plan

    n, k = 768, 5376
    assert splitk_plan(m, n, k) > 1
    rng = np.random.default_rng(m)
    a, sa = quantize(torch.from_numpy(rng.standard_normal((m, k), dtype=np.float32)).to(device), "int8")
    b, sb = quantize(torch.from_numpy(rng.standard_normal((n, k), dtype=np.float32)).to(device), "int8")
    gamma, cos, sin = _tables(rng, m, device)
    routed = projection_qk_rope(a, b, gamma, cos, sin, "int8", a_scales=sa, b_scales=sb, epsilon=1e-6)
    fused = torch.empty((n // 128, m, 128), dtype=torch.bfloat16, device=device)
    _lib.call("m5k_projection_qk_rope", _lib.ptr(a), _lib.ptr(b), _lib.dtype_code(a), m, n, k, _lib.ptr(sa),
              _lib.ptr(sb), _lib.ptr(gamma.contiguous()), _lib.ptr(cos.contiguous()), _lib.ptr(sin.contiguous()),
              cos.shape[1], float(np.float32(1e-6)), _lib.ptr(fused), _lib.stream_of(a))
    np.testing.assert_array_equal(bits_of(routed), bits_of(fused))


# ---- bit-exact against the fixed-order FP32 oracle (oracle_qk_norm_rope / _qkv_) -------------


@pytest.mark.parametrize("rope_half", [1, 5, 48, 64])
@pytest.mark.parametrize("shape", [(17, 384, 96), (300, 640, 1024), (129, 256, 257)])
def test_int8_fused_bit_exact_vs_fixed_order_oracle(rope_half, shape, device):
    """INT8 fused projection: the oracle's exact INT32 projection through the FP32 dequant and
    BF16 cast, then the epilogue's FP32 order (16-lane sum tree, IEEE 1/sqrt, split-half RoPE)."""
    rng = np.random.default_rng(rope_half * 7 + shape[0])
    m, n, k = shape
    a, sa = quantize(torch.from_numpy(rng.standard_normal((m, k), dtype=np.float32)).to(device), "int8")
    b, sb = quantize(torch.from_numpy(rng.standard_normal((n, k), dtype=np.float32)).to(device), "int8")
    gamma, cos, sin = _tables(rng, m, device, rope_half)
    y = projection_qk_rope(a, b, gamma, cos, sin, "int8", a_scales=sa, b_scales=sb, epsilon=1e-6)
    z = ref.c_i8_epilogue(ref.c_gemm_i8_acc(np_of(a), np_of(b)), np_of(sa), np_of(sb))
    expected = ref.c_qk_norm_rope(z, bits_of(gamma), bits_of(cos), bits_of(sin), epsilon=float(np.float32(1e-6)))
    np.testing.assert_array_equal(bits_of(y), expected)


def test_staged_postprocess_bit_exact_vs_fixed_order_oracle(device):
    """The staged epilogue on a given BF16 projection (zeros, outliers, R = 48)."""
    rng = np.random.default_rng(9)
    p_np = rng.standard_normal((40, 4 * 128), dtype=np.float32) * 2
    p_np[0] = 0
    p_np[1, ::31] *= 100
    p = torch.from_numpy(p_np).to(device).to(torch.bfloat16)
    gamma, cos, sin = _tables(rng, 40, device, 48)
    y = qk_norm_rope(p, gamma, cos, sin, epsilon=1e-5)
    expected = ref.c_qk_norm_rope(bits_of(p), bits_of(gamma), bits_of(cos), bits_of(sin),
                                  epsilon=float(np.float32(1e-5)))
    np.testing.assert_array_equal(bits_of(y), expected)


@pytest.mark.parametrize("rope_half", [48, 5])
@pytest.mark.parametrize("m,heads", [(300, 3), (4096, 32)])
def test_grouped_qkv_bit_exact_vs_oracle(rope_half, m, heads, device):
    """Grouped Q/K/V (weight rows [head, stream, 128]): Q and K equal the fixed-order oracle of
    the INT8 projection bit for bit, V the BF16 projection (sampled rows at M 4096)."""
    from m5kernels_amd import projection_qkv_rope

    rng = np.random.default_rng(m + heads + rope_half)
    k = 1024
    x = torch.from_numpy(rng.standard_normal((m, k), dtype=np.float32)).to(device).to(torch.bfloat16)
    w = torch.from_numpy((rng.standard_normal((heads * 384, k)) * 0.05).astype(np.float32)).to(device)
    a, sa = quantize(x, "int8")
    b, sb = quantize(w.to(torch.bfloat16), "int8")
    q_gamma, cos, sin = _tables(rng, m, device, rope_half)
    k_gamma = torch.from_numpy(rng.uniform(0.5, 1.5, 128).astype(np.float32)).to(device).to(torch.bfloat16)
    q, kk, v = projection_qkv_rope(a, b, q_gamma, k_gamma, cos, sin, "int8", a_scales=sa, w_scales=sb)
    rows = ref.sample_indices(m) if m > 512 else np.arange(m)
    z = ref.c_i8_epilogue(ref.c_gemm_i8_acc(np_of(a[rows]), np_of(b)), np_of(sa[rows]), np_of(sb))
    oq, ok, ov = ref.c_qkv_norm_rope(z, bits_of(q_gamma), bits_of(k_gamma), bits_of(cos[rows]), bits_of(sin[rows]),
                                     epsilon=float(np.float32(1e-6)))
    np.testing.assert_array_equal(bits_of(q[:, rows]), oq)
    np.testing.assert_array_equal(bits_of(kk[:, rows]), ok)
    np.testing.assert_array_equal(bits_of(v[:, rows]), ov)
