"""Pins the fixed-order FP32 restatements of the fused prep and the Q/K epilogue
(oracle/m5k_oracle.c: oracle_prep_rows, oracle_qk_norm_rope, oracle_qkv_norm_rope,
oracle_f16_round) before the GPU tests hold the kernels to them bit for bit.

Oracle function            pinned by
-------------------------  -------------------------------------------------------------
c_f16_round                numpy's float16 cast (nearest even) on 2M spread values and the
                           binary16 edges (subnormals, ties, 65504 / 65520 overflow)
c_prep_rows                without the O cast, the float64 references (norm_hadamard_reference.py:
                           24-94, gated_residual_reference.py:21-60) within the reference's own
                           GPU bar (codes +-1, scales rtol 3e-5; tests/test_norm_hadamard_metal.py:
                           33-82) over norms, dtypes, every block, ragged chunk counts and row
                           maps; with it, the FP32 modulation within 2^-19 of float64 and the
                           codes exactly those of its O cast (hadamard and quantizer pinned in
                           test_oracle.py); the gated form: R_next bit-exact against numpy
                           float32 and equal to the ungated prep of R_next; KATs
                           layernorm_constant_row, the FP32-product cancellation and the BF16
                           tie boundary of the modulation
c_qk_norm_rope             the float64 qk_rope_reference within one BF16 ulp and rel-L2 1e-3;
                           KAT rope_split_half_pairing (cos 0, sin 1: exact partner swap)
c_qkv_norm_rope            the reference's own float64 header (integrations/h3/
                           qkv_reference.h:17-35, compiled into oracle/_ref) within one BF16
                           ulp; V equal to the rounded projection bit for bit
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import reference as ref


def _bf16(x):
    return ref.bf16_round_f32(np.asarray(x, dtype=np.float32))


def _round(x, dtype):
    if dtype == "bf16":
        return _bf16(x)
    if dtype == "fp16":
        return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)
    return np.asarray(x, dtype=np.float32)


# ------------------------------------------------------------------------------ binary16
def test_f16_round_matches_numpy():
    rng = np.random.default_rng(3)
    x = rng.standard_normal(2_000_000).astype(np.float32)
    x *= (np.float32(2.0) ** rng.integers(-30, 17, x.size)).astype(np.float32)
    edges = np.array([0.0, -0.0, 65504.0, 65519.996, 65520.0, -65520.0, 1e9, 2.0**-14, 2.0**-24, 2.0**-25,
                      1.5 * 2.0**-25, 3 * 2.0**-26, 1 + 2.0**-11, 1 + 3 * 2.0**-11, 2049.0, 2051.0], np.float32)
    x = np.concatenate([x, edges, -edges])
    with np.errstate(over="ignore"):
        expected = x.astype(np.float16).astype(np.float32)
    np.testing.assert_array_equal(ref.c_f16_round(x).view(np.uint32), expected.view(np.uint32))


# ------------------------------------------------------------------------------ fused prep
def _prep_case(rng, rows, width, dtype, mapped):
    x = _round(rng.standard_normal((rows, width), dtype=np.float32), dtype)
    gamma = _bf16(1 + 0.1 * rng.standard_normal(width))
    tables = (3, width) if mapped else (width,)
    scale = _bf16(0.2 * rng.standard_normal(tables))
    shift = _bf16(0.1 * rng.standard_normal(tables))
    row_map = (np.arange(rows, dtype=np.int32) * 2) % 3 if mapped else None
    return x, gamma, scale, shift, row_map


def _float64_codes(x, gamma, scale, shift, signs, block, norm, eps, out_dtype, row_map):
    if row_map is None:
        mod = ref.norm_modulate_reference(x, gamma, scale, shift, norm=norm, eps=eps)
    else:
        mod = np.concatenate([ref.norm_modulate_reference(x[r:r + 1], gamma, scale[i], shift[i], norm=norm, eps=eps)
                              for r, i in enumerate(row_map)])
    mod = _round(mod, out_dtype)
    return ref.quantize_reference(ref.block_hadamard_reference(mod, block, signs), "int8")


def _assert_within_one_code(q, s, rq, rs):
    assert np.max(np.abs(q.astype(np.int16) - rq.astype(np.int16))) <= 1
    np.testing.assert_allclose(s, rs, rtol=3e-5, atol=1e-7)


_BLOCK_WIDTHS = [(32, 768), (64, 1536), (128, 4096), (256, 5376), (512, 3072), (1024, 6144), (256, 16384)]


@pytest.mark.parametrize("norm", ["rms", "layer"])
@pytest.mark.parametrize("dtype", ["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("block,width", _BLOCK_WIDTHS)
def test_prep_within_one_code_of_float64(norm, dtype, block, width):
    """round_output="fp32" (no O cast): the reference's own GPU bar against float64."""
    rng = np.random.default_rng(block + width)
    x, gamma, scale, shift, row_map = _prep_case(rng, 5, width, dtype, mapped=width % 3 == 0)
    signs = ref.hadamard_signs(width, 9)
    q, s = ref.c_prep_rows(x, gamma, scale, shift, signs, block, dtype=dtype, norm=norm, round_output="fp32",
                           row_map=row_map)
    rq, rs = _float64_codes(x, gamma, scale, shift, signs, block, norm, 1e-5, "fp32", row_map)
    _assert_within_one_code(q, s, rq, rs)


@pytest.mark.parametrize("norm", ["rms", "layer"])
@pytest.mark.parametrize("dtype", ["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("block,width", _BLOCK_WIDTHS)
def test_prep_modulation_and_input_boundary(norm, dtype, block, width):
    """round_output="input": the FP32 modulation is within 2^-19 (relative to the row's peak) of
    float64, and the codes are exactly those of the O cast of that modulation, rotated and
    quantized (the O cast can flip one element by an ulp of the dtype where FP32 and float64
    straddle a rounding midpoint, so float64 alone cannot fix the codes)."""
    rng = np.random.default_rng(block * 7 + width)
    x, gamma, scale, shift, row_map = _prep_case(rng, 5, width, dtype, mapped=width % 3 == 0)
    signs = ref.hadamard_signs(width, 9)
    q, s, mod = ref.c_prep_rows(x, gamma, scale, shift, signs, block, dtype=dtype, norm=norm, row_map=row_map,
                                with_modulated=True)
    if row_map is None:
        exact = ref.norm_modulate_reference(x, gamma, scale, shift, norm=norm)
    else:
        exact = np.concatenate([ref.norm_modulate_reference(x[r:r + 1], gamma, scale[i], shift[i], norm=norm)
                                for r, i in enumerate(row_map)])
    peak = np.max(np.abs(exact), axis=1, keepdims=True)
    assert np.max(np.abs(mod - exact) / peak) < 2.0**-19
    rq, rs = ref.quantize_reference(ref.c_hadamard_f32(_round(mod, dtype), block, signs), "int8")
    np.testing.assert_array_equal(q, rq)
    np.testing.assert_array_equal(s, rs)


@pytest.mark.parametrize("norm", ["rms", "layer"])
@pytest.mark.parametrize("dtype,branch_dtype", [("bf16", "bf16"), ("bf16", "fp32"), ("fp16", "bf16"),
                                                ("fp32", "fp16")])
@pytest.mark.parametrize("mapped", [False, True])
def test_gated_prep_r_next_exact_and_codes(norm, dtype, branch_dtype, mapped):
    rng = np.random.default_rng(17)
    rows, width = 6, 5376
    x, gamma, scale, shift, row_map = _prep_case(rng, rows, width, dtype, mapped)
    branch = _round(rng.standard_normal((rows, width), dtype=np.float32) * np.float32(2), branch_dtype)
    gate = _bf16(rng.uniform(-0.7, 0.7, size=(3, width) if mapped else width))
    gmap = (np.arange(rows, dtype=np.int32) + 1) % 3 if mapped else None
    signs = ref.hadamard_signs(width, 4)
    q, s, r_next = ref.c_prep_rows(x, gamma, scale, shift, signs, 256, dtype=dtype, norm=norm, row_map=row_map,
                                   branch=branch, gate=gate, gate_row_map=gmap)
    g = gate if gmap is None else gate[gmap]
    expected = _round((x + branch * g).astype(np.float32), dtype)  # FP32 product, FP32 sum, one cast
    np.testing.assert_array_equal(r_next.view(np.uint32), expected.view(np.uint32))
    _, _, _, mod = ref.c_prep_rows(x, gamma, scale, shift, signs, 256, dtype=dtype, norm=norm, row_map=row_map,
                                   branch=branch, gate=gate, gate_row_map=gmap, with_modulated=True)
    rq, rs = ref.quantize_reference(ref.c_hadamard_f32(_round(mod, dtype), 256, signs), "int8")
    np.testing.assert_array_equal(q, rq)
    rq, rs = _float64_codes(r_next, gamma, scale, shift, signs, 256, norm, 1e-5, "fp32", row_map)
    q32, s32 = ref.c_prep_rows(r_next, gamma, scale, shift, signs, 256, dtype=dtype, norm=norm, row_map=row_map,
                               round_output="fp32")
    _assert_within_one_code(q32, s32, rq, rs)
    # The gated form equals the ungated prep of the materialized R_next, bit for bit.
    q2, s2 = ref.c_prep_rows(r_next, gamma, scale, shift, signs, 256, dtype=dtype, norm=norm, row_map=row_map)
    np.testing.assert_array_equal(q, q2)
    np.testing.assert_array_equal(s, s2)


def test_prep_kats(kats):
    # layernorm_constant_row (tests/test_norm_hadamard_reference.py:86-91): a constant row
    # centres to exact zeros, so every code is 0 and the scale is 1 whatever the tables.
    kat = kats["layernorm_constant_row"]
    width = 256
    x = np.full((3, width), kat["row_value"], np.float32)
    q, s = ref.c_prep_rows(x, np.ones(width), np.full(width, 0.5), np.zeros(width), np.ones(width, np.int8), 256,
                           dtype="fp32", norm="layer")
    assert np.all(q == 0) and np.all(s == 1.0)
    # gated_residual_cancellation in BF16: a product rounded before the add would cancel to
    # zero; the FP32 product keeps 2^-7 (1 + 2^-7)(1 - 2^-8) - 1 > 0 and R_next is its BF16 cast.
    res = np.full((1, 256), -1.0, np.float32)
    branch = np.full((1, 256), 1.0078125, np.float32)
    gate = np.full(256, 1.0 - 2.0**-8, np.float32)
    _, _, r_next = ref.c_prep_rows(res, np.ones(256), np.zeros(256), np.zeros(256), np.ones(256, np.int8), 256,
                                   branch=branch, gate=gate)
    exact = np.float32(-1.0) + np.float32(1.0078125) * np.float32(1.0 - 2.0**-8)
    assert r_next[0, 0] == _bf16([exact])[0] != 0.0
    # bf16_round_ties (tests/test_qk_rope_reference.py:79-101) at the modulation boundary: zero
    # input and gamma leave y = shift, rounded to BF16 with ties to even before the signs.
    ties = kats["bf16_round_ties"]
    shift = np.resize(np.array(ties["x"], np.float32), 256)
    zeros = np.zeros(256, np.float32)
    signs = np.ones(256, np.int8)
    q, s = ref.c_prep_rows(np.zeros((1, 256), np.float32), zeros, zeros, shift, signs, 256, dtype="bf16")
    rq, rs = ref.quantize_reference(ref.c_hadamard_f32(np.resize(np.array(ties["bf16"], np.float32), (1, 256)),
                                                       256, signs), "int8")
    np.testing.assert_array_equal(q, rq)
    np.testing.assert_array_equal(s, rs)


# ------------------------------------------------------------------------------ Q/K epilogue
def _qk_inputs(rng, m, heads, rope_half):
    z = _bf16(rng.standard_normal((m, heads * 128)) * 3)
    gamma = _bf16(1 + 0.02 * rng.standard_normal(128))
    ang = rng.uniform(-np.pi, np.pi, size=(m, rope_half))
    return z, gamma, _bf16(np.cos(ang)), _bf16(np.sin(ang))


@pytest.mark.parametrize("rope_half", [0, 16, 48, 64])
def test_qk_within_one_ulp_of_float64(rope_half):
    rng = np.random.default_rng(rope_half)
    m, heads = 33, 4
    z, gamma, cos, sin = _qk_inputs(rng, m, heads, rope_half)
    got = ref.c_qk_norm_rope(ref.f32_to_bf16_bits(z), ref.f32_to_bf16_bits(gamma), ref.f32_to_bf16_bits(cos),
                             ref.f32_to_bf16_bits(sin), epsilon=1e-6)
    exp = ref.qk_rope_reference(z.reshape(m, heads, 128), gamma, cos, sin, epsilon=1e-6)["output"]
    exp_bits = ref.f32_to_bf16_bits(exp.astype(np.float32))
    ulps = np.abs(got.astype(np.int32) - exp_bits.astype(np.int32))
    assert ulps.max() <= 1 and np.mean(ulps) < 0.05
    assert ref.metrics(ref.bf16_bits_to_f32(got), exp)["relative_l2"] < 1e-3


def test_qk_split_half_kat(kats):
    """rope_split_half_pairing (tests/test_qk_rope_reference.py:136-148): with cos 0 and sin 1,
    channel j < R becomes -u[j + R] and channel R + j becomes u[j], exactly."""
    kat = kats["rope_split_half_pairing"]
    r = len(kat["cos"])
    head = np.zeros(128, np.float32)
    head[: len(kat["projected"])] = kat["projected"]
    z = ref.f32_to_bf16_bits(head[None, :])
    ones = ref.f32_to_bf16_bits(np.ones(128, np.float32))
    cos = ref.f32_to_bf16_bits(np.array([kat["cos"]], np.float32))
    sin = ref.f32_to_bf16_bits(np.array([kat["sin"]], np.float32))
    y = ref.bf16_bits_to_f32(ref.c_qk_norm_rope(z, ones, cos, sin, epsilon=1e-6))[0, 0]
    plain = ref.bf16_bits_to_f32(ref.c_qk_norm_rope(z, ones, cos[:, :0], sin[:, :0], epsilon=1e-6))[0, 0]
    expected = np.array(kat["expected_over_inverse_rms"], np.float32)
    n = len(expected)
    # plain[d] = bf16(u[d]); the KAT's pattern is a signed permutation of u.
    perm = [int(abs(v)) - 1 for v in expected]
    np.testing.assert_array_equal(y[:n], np.sign(expected) * plain[perm])
    np.testing.assert_array_equal(y[n:], plain[n:])
    assert r * 2 <= n


@pytest.mark.skipif(ref.ref_qkv_lib() is None, reason="oracle/_ref not built (no reference checkout here)")
@pytest.mark.parametrize("seed", [0, 1])
def test_qkv_fixed_order_vs_reference_header(seed):
    """The grouped Q/K/V epilogue restatement against the reference's own float64 header
    (qkv_reference.h:17-35, rope half 48): V equals the BF16 projection bit for bit; Q and K
    within one BF16 ulp of the float64 result (its own bar is rel-L2 0.008)."""
    rng = np.random.default_rng(seed)
    m, heads = 17, 3
    proj = rng.standard_normal((m, heads * 384)) * 2.5
    proj[1] *= 1e-4  # an epsilon-dominated row
    z_bits = ref.f32_to_bf16_bits(proj.astype(np.float32))
    gq = ref.f32_to_bf16_bits((1 + 0.05 * rng.standard_normal(128)).astype(np.float32))
    gk = ref.f32_to_bf16_bits((1 + 0.05 * rng.standard_normal(128)).astype(np.float32))
    ang = rng.uniform(-3, 3, size=(m, 48))
    cos, sin = ref.f32_to_bf16_bits(np.cos(ang).astype(np.float32)), ref.f32_to_bf16_bits(np.sin(ang).astype(np.float32))
    eps = float(np.float32(1e-5))
    outs = ref.c_qkv_norm_rope(z_bits, gq, gk, cos, sin, epsilon=eps)
    for h in range(heads):
        for stream in range(3):
            block = proj[:, (3 * h + stream) * 128:(3 * h + stream + 1) * 128]
            want = ref.ref_qkv_postprocess(block, stream, gq if stream == 0 else gk, cos, sin, eps)
            got = outs[stream][h]
            want_bits = ref.f32_to_bf16_bits(want.astype(np.float32))
            if stream == 2:
                np.testing.assert_array_equal(got, want_bits)
            else:
                assert np.abs(got.astype(np.int32) - want_bits.astype(np.int32)).max() <= 1
