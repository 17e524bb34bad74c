"""Pins the CPU oracle (oracle/reference.py, oracle/m5k_oracle.c) before it is trusted.

Every oracle function is checked against the reference's own known-answer vectors
(tests/golden/reference_kats.json, transcribed from the reference's tests) and against
independent closed forms (dense Hadamard matrices, scalar math.fsum norms, brute-force
code searches, exact integer products), chosen so that a dropped term, wrong sign,
index or operand order fails at least one check.

Oracle function                        pinned by
-------------------------------------  ---------------------------------------------------
fp8_decode / fp8_encode (py + C)       KAT fp8_encode; all-254-code round trip; brute
                                       force over every FP32 midpoint/tie between codes
quantize_reference / c_quantize_rows   KAT int8_round_half_even; zero/outlier KAT;
                                       element-wise scalar restatement; C == NumPy
c_gemm_i8_acc                          exact int64 numpy matmul
c_i8_epilogue                          KAT gemm_bias_before_bf16_rounding; scalar FP32
                                       evaluation; gated form vs scalar
bf16 rounding (py + C)                 KAT bf16_round_ties (ties, FP32 producer);
                                       arithmetic frexp-based nearest-even oracle
block_hadamard_reference / c_hadamard  dense (-1)^popcount(i&j)/sqrt(B); signs-before-H;
                                       norm and dot preservation
norm_modulate_reference                scalar math.fsum restatement; constant-row KAT;
                                       epsilon inside the root
gated_residual_reference               scalar loop; cancellation KAT; row map selection
qk_rope_reference                      scalar RMS + dense rotation; split-half KAT;
                                       no-RoPE path; gamma/RoPE non-commutation
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import reference as ref


# ----------------------------------------------------------------------------- FP8 codes
def test_fp8_encode_kat(kats):
    kat = kats["fp8_encode"]
    x = np.array(kat["x"], dtype=np.float32)
    np.testing.assert_array_equal(ref.fp8_encode(x), kat["codes"])
    np.testing.assert_array_equal(ref.c_fp8_encode(x), kat["codes"])


def test_fp8_all_finite_codes_round_trip():
    codes = np.concatenate([np.arange(127), np.arange(128, 255)]).astype(np.uint8)
    decoded = ref.fp8_decode(codes)
    np.testing.assert_array_equal(ref.fp8_encode(decoded), codes)
    np.testing.assert_array_equal(ref.c_fp8_encode(decoded), codes)
    assert np.isnan(ref.fp8_decode(np.array([127, 255], np.uint8))).all()


def test_fp8_decode_closed_form():
    # value = (-1)^s * 2^(e-7) * (1 + m/8) for e > 0, m * 2^-9 for e == 0.
    for code in range(256):
        s, e, m = code >> 7, (code >> 3) & 15, code & 7
        if e == 15 and m == 7:
            continue
        expected = (-1) ** s * (m * 2.0**-9 if e == 0 else 2.0 ** (e - 7) * (1 + m / 8))
        assert ref.fp8_decode(np.array([code], np.uint8))[0] == np.float32(expected)


def test_fp8_encode_brute_force_midpoints_and_neighbours():
    table = ref.fp8_decode(np.arange(127, dtype=np.uint8)).astype(np.float64)
    mids = (table[:-1] + table[1:]) / 2
    probes = np.concatenate([table, mids, np.nextafter(mids, 0), np.nextafter(mids, 1e9), [449.0, 480.0, 1e30]])
    probes = probes.astype(np.float32)
    probes = np.concatenate([probes, -probes])
    got_py = ref.fp8_encode(probes)
    got_c = ref.c_fp8_encode(probes)
    for x, code_py, code_c in zip(probes, got_py, got_c):
        a = min(abs(float(x)), 448.0)
        dist = np.abs(table - a)
        best = np.flatnonzero(dist == dist.min())
        want = best[0] if len(best) == 1 else best[best % 2 == 0][0]  # tie -> even code
        want |= 128 if math.copysign(1.0, float(x)) < 0 else 0
        assert code_py == want and code_c == want, (x, code_py, code_c, want)


# ----------------------------------------------------------------------------- quantizer
def test_int8_round_half_even_kat(kats):
    kat = kats["int8_round_half_even"]
    x = np.array([kat["row"]] * 3, dtype=np.float32)
    for q, s in (ref.quantize_reference(x, "int8"), ref.c_quantize_rows(x, "int8")):
        np.testing.assert_array_equal(q, np.tile(kat["codes"], (3, 1)))
        np.testing.assert_array_equal(s, kat["scale"])


@pytest.mark.parametrize("mode", ["int8", "fp8"])
def test_quantize_zero_and_outlier_kat(kats, mode):
    kat = kats["quantize_zero_and_outlier"]
    x = np.zeros(kat["shape"], np.float32)
    x[kat["outlier"]["row"], kat["outlier"]["col"]] = kat["outlier"]["value"]
    for q, s in (ref.quantize_reference(x, mode), ref.c_quantize_rows(x, mode)):
        y = ref.dequantize(q, s, mode)
        assert s[0] == kat["zero_row_scale"]
        assert np.all(y[0] == 0)
        assert np.max(np.abs(y - x)) < kat["max_abs_dequant_error_below"]


@pytest.mark.parametrize("mode", ["int8", "fp8"])
def test_quantizer_scalar_restatement_and_c_agree(mode):
    rng = np.random.default_rng(41)
    x = rng.standard_normal((9, 96), dtype=np.float32)
    x[:, ::31] *= 30
    x[3] = 0
    q, s = ref.quantize_reference(x, mode)
    qc, sc = ref.c_quantize_rows(x, mode)
    np.testing.assert_array_equal(q, qc)
    np.testing.assert_array_equal(s, sc)
    # Scalar restatement with Python floats rounded to FP32 at every step.
    f32 = np.float32
    for r in range(x.shape[0]):
        peak = max(abs(float(v)) for v in x[r])
        scale = f32(1.0) if peak == 0 else f32(f32(peak) / f32(448.0 if mode == "fp8" else 127.0))
        assert s[r] == scale
        for j in range(x.shape[1]):
            z = f32(x[r, j] / scale)
            if mode == "int8":
                assert q[r, j] == max(-127, min(127, round(float(z))))  # round() is half-even
            else:
                assert q[r, j] == ref.fp8_encode(np.array([z]))[0]


def test_bf16_quantizer_matches_f32_path():
    rng = np.random.default_rng(5)
    bits = ref.f32_to_bf16_bits(rng.standard_normal((5, 64), dtype=np.float32))
    q1, s1 = ref.c_quantize_rows(bits, "int8")
    q2, s2 = ref.quantize_reference(ref.bf16_bits_to_f32(bits), "int8")
    np.testing.assert_array_equal(q1, q2)
    np.testing.assert_array_equal(s1, s2)


def test_quantizer_rejects_non_finite():
    with pytest.raises(ValueError, match="finite"):
        ref.quantize_reference(np.array([[1.0, np.nan]]), "int8")


# ----------------------------------------------------------------------------- GEMM
def test_integer_accumulators_exact():
    rng = np.random.default_rng(83)
    a = rng.integers(-127, 128, size=(7, 257), dtype=np.int8)
    b = rng.integers(-127, 128, size=(33, 257), dtype=np.int8)
    expected = a.astype(np.int64) @ b.astype(np.int64).T
    np.testing.assert_array_equal(ref.c_gemm_i8_acc(a, b), expected)
    # worst case magnitude still exact
    a[:] = -127
    b[:] = -127
    np.testing.assert_array_equal(ref.c_gemm_i8_acc(a, b), np.full((7, 33), 127 * 127 * 257))


def test_epilogue_bias_before_rounding_kat(kats):
    kat = kats["gemm_bias_before_bf16_rounding"]
    m, n = kat["a_shape"][0], kat["b_shape"][0]
    acc = np.ones((m, n), np.int32)  # a[:,0] = b[:,0] = 1, rest 0
    out = ref.c_i8_epilogue(
        acc, np.full(m, kat["a_scale"], np.float32), np.full(n, kat["b_scale"], np.float32),
        bias=np.full(n, kat["bias"], np.float32),
    )
    np.testing.assert_array_equal(ref.bf16_bits_to_f32(out), np.float32(kat["expected"]))


def test_epilogue_scalar_fp32_order_and_gate():
    rng = np.random.default_rng(97)
    acc = rng.integers(-(2**26), 2**26, size=(6, 10)).astype(np.int32)
    sa = rng.uniform(0.01, 0.13, 6).astype(np.float32)
    sb = rng.uniform(0.02, 0.17, 10).astype(np.float32)
    out = ref.c_i8_epilogue(acc, sa, sb, out="fp32")
    f32 = np.float32
    for i in range(6):
        for j in range(10):
            assert out[i, j] == f32(f32(f32(acc[i, j]) * sa[i]) * sb[j])
    # A different product order must be observable somewhere (pins the left-to-right order).
    other = (acc.astype(np.float32) * (sa[:, None] * sb[None, :])).astype(np.float32)
    assert np.any(other != out)
    res = ref.f32_to_bf16_bits(rng.standard_normal((6, 10)).astype(np.float32))
    gate = ref.f32_to_bf16_bits(rng.standard_normal(10).astype(np.float32))
    gated = ref.c_i8_epilogue(acc, sa, sb, residual_bits=res, gate_bits=gate)
    for i in range(6):
        for j in range(10):
            branch = ref.bf16_round_f32(np.array([out[i, j]]))[0]
            v = f32(ref.bf16_bits_to_f32(res[i, j]) + f32(branch * ref.bf16_bits_to_f32(gate[j])))
            assert gated[i, j] == ref.f32_to_bf16_bits(np.array([v]))[0]


def test_online_linear_composition():
    rng = np.random.default_rng(0)
    a_bits = ref.f32_to_bf16_bits(rng.standard_normal((16, 64), dtype=np.float32))
    w_bits = ref.f32_to_bf16_bits(rng.standard_normal((24, 64), dtype=np.float32) * np.float32(0.02))
    wq, ws = ref.c_quantize_rows(w_bits, "int8")
    out = ref.c_w8a8_linear_bf16(a_bits, wq, ws)
    aq, sa = ref.c_quantize_rows(a_bits, "int8")
    staged = ref.c_i8_epilogue(ref.c_gemm_i8_acc(aq, wq), sa, ws)
    np.testing.assert_array_equal(out, staged)


# ----------------------------------------------------------------------------- BF16
def _scalar_bf16(value):
    value = float(np.float32(value))
    if value == 0:
        return value
    _, exponent = math.frexp(abs(value))
    step = math.ldexp(1.0, max(exponent - 8, -133))
    return math.copysign(round(abs(value) / step) * step, value)


def test_bf16_rounding_kat_and_arithmetic_oracle(kats):
    kat = kats["bf16_round_ties"]
    np.testing.assert_array_equal(ref.bf16_round_reference(np.array(kat["x"])), kat["bf16"])
    assert ref.bf16_round_reference(kat["fp32_producer_case"]["x"]) == kat["fp32_producer_case"]["bf16"]
    rng = np.random.default_rng(107)
    vals = np.concatenate([rng.normal(size=200) * 10.0 ** rng.integers(-30, 30, 200), [0.0, -0.0, 2.0**-134]])
    got = ref.bf16_round_reference(vals)
    want = np.array([_scalar_bf16(v) for v in vals])
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(np.signbit(got), np.signbit(want))


# ----------------------------------------------------------------------------- Hadamard
def _dense_hadamard(block):
    return np.array(
        [[(-1) ** bin(i & j).count("1") for j in range(block)] for i in range(block)], dtype=np.float64
    ) / math.sqrt(block)


@pytest.mark.parametrize("block", [1, 4, 32, 128])
def test_hadamard_matches_dense_definition(block):
    rng = np.random.default_rng(19)
    x = rng.normal(size=(3, 3 * block)).astype(np.float32)
    x[:, ::block] *= 1000
    signs = ref.hadamard_signs(x.shape[1], 17)
    expected = ((x.astype(np.float64) * signs).reshape(-1, block) @ _dense_hadamard(block)).reshape(x.shape)
    np.testing.assert_allclose(ref.block_hadamard_reference(x, block, signs), expected, rtol=3e-14, atol=1e-11)
    if block >= 32:
        got = ref.c_hadamard_f32(x, block, signs)
        np.testing.assert_allclose(got, expected, rtol=2e-6, atol=1e-4)


def test_hadamard_signs_before_h_and_invariants():
    x = np.array([[1.0, 2.0, 4.0, 8.0]])
    signs = np.array([1, -1, 1, -1])
    got = ref.block_hadamard_reference(x, 4, signs)
    np.testing.assert_allclose(got, (x * signs) @ _dense_hadamard(4), atol=0)
    assert not np.allclose(got, (x @ _dense_hadamard(4)) * signs)
    rng = np.random.default_rng(21)
    a, w = rng.normal(size=(3, 256)), rng.normal(size=(5, 256))
    s = ref.hadamard_signs(256, 23)
    ra, rw = ref.block_hadamard_reference(a, 128, s), ref.block_hadamard_reference(w, 128, s)
    np.testing.assert_allclose(ra @ rw.T, a @ w.T, rtol=1e-12, atol=1e-9)
    np.testing.assert_allclose(np.linalg.norm(ra), np.linalg.norm(a), rtol=3e-15)
    first = ref.hadamard_signs(256, 17)
    np.testing.assert_array_equal(first, ref.hadamard_signs(256, 17))
    assert set(first.tolist()) == {-1, 1} and first.dtype == np.int8


def test_c_hadamard_fp32_stage_order_is_sequential_fp32():
    """The C oracle's FP32 values equal a direct Python FP32 evaluation of the stages."""
    rng = np.random.default_rng(7)
    x = rng.standard_normal((2, 64), dtype=np.float32)
    signs = ref.hadamard_signs(64, 3)
    got = ref.c_hadamard_f32(x, 32, signs)
    f32 = np.float32
    inv = f32(1.0 / math.sqrt(32))
    for r in range(2):
        v = [f32(x[r, j] * f32(signs[j])) for j in range(64)]
        for b0 in (0, 32):
            s = 1
            while s < 32:
                for base in range(b0, b0 + 32, 2 * s):
                    for t in range(s):
                        p, q = v[base + t], v[base + t + s]
                        v[base + t], v[base + t + s] = f32(p + q), f32(p - q)
                s *= 2
        np.testing.assert_array_equal(got[r], np.array([f32(t * inv) for t in v], np.float32))


# ----------------------------------------------------------------------------- norm / gate
def _scalar_modulation(x, gamma, scale, shift, norm, eps):
    out = np.empty(x.shape)
    for i, row in enumerate(x):
        mean = math.fsum(row) / len(row) if norm == "layer" else 0.0
        centred = [float(v) - mean for v in row]
        denom = math.sqrt(math.fsum(v * v for v in centred) / len(row) + eps)
        for j, v in enumerate(centred):
            out[i, j] = v / denom * gamma[j] * (1.0 + scale[j]) + shift[j]
    return out


@pytest.mark.parametrize("norm", ["rms", "layer"])
def test_norm_modulate_scalar(norm):
    rng = np.random.default_rng(41)
    x = rng.normal(size=(5, 24))
    x[:, 0] *= 1000
    g, s, b = rng.normal(size=24), rng.normal(size=24), rng.normal(size=24)
    np.testing.assert_allclose(
        ref.norm_modulate_reference(x, g, s, b, norm=norm), _scalar_modulation(x, g, s, b, norm, 1e-5),
        rtol=3e-14, atol=1e-11,
    )


def test_norm_kats(kats):
    kat = kats["layernorm_constant_row"]
    w = kat["width"]
    y = ref.norm_modulate_reference(np.full((3, w), kat["row_value"]), np.arange(w), np.arange(w), kat["shift"],
                                    norm="layer")
    np.testing.assert_array_equal(y, np.tile(kat["shift"], (3, 1)))
    x = np.array([[0.000137, 0.000211]])
    got = ref.norm_modulate_reference(x, np.ones(2), np.zeros(2), np.zeros(2), eps=0.125)
    np.testing.assert_array_equal(got, x / math.sqrt(math.fsum(v * v for v in x[0]) / 2 + 0.125))
    zero = ref.norm_hadamard_quantize_reference(np.zeros((3, 8)), np.ones(8), np.ones(8), np.zeros(8), 4)
    np.testing.assert_array_equal(zero["scales"], np.ones(3))
    np.testing.assert_array_equal(zero["quantized"], 0)


def test_gated_residual_scalar_and_kats(kats):
    rng = np.random.default_rng(47)
    res, br, gate = rng.normal(size=(5, 7)), rng.normal(size=(5, 7)), rng.normal(size=(4, 7))
    row_map = (np.arange(5, dtype=np.int32) * 3) % 4
    got = ref.gated_residual_reference(res, br, gate, row_map=row_map)
    for i in range(5):
        for j in range(7):
            assert got[i, j] == float(res[i, j]) + float(gate[row_map[i], j]) * float(br[i, j])
    kat = kats["gated_residual_cancellation"]
    out = ref.gated_residual_reference([kat["residual"]], [kat["branch"]], kat["gate"])
    np.testing.assert_array_equal(out[:, :2], 0)
    assert out[0, 2] == kat["branch"][2] - 1.0 and out[0, 2] != 0.0
    with pytest.raises(ValueError, match="indices"):
        ref.gated_residual_reference(np.ones((3, 7)), np.ones((3, 7)), np.ones((2, 7)),
                                     row_map=np.array([0, 2, 0], np.int32))


# ----------------------------------------------------------------------------- Q/K RoPE
def test_qk_rope_scalar_and_dense_rotation():
    rng = np.random.default_rng(103)
    shape, half = (5, 3, 128), 48
    projected = rng.normal(size=shape)
    gamma = rng.normal(size=128)
    angles = rng.uniform(-math.pi, math.pi, size=(5, half))
    cos, sin = np.cos(angles), np.sin(angles)
    got = ref.qk_rope_reference(projected, gamma, cos, sin, projection_bf16=False, output_bf16=False)
    for r in range(5):
        rot = np.eye(128)
        for j in range(half):
            rot[j, j] = rot[j + half, j + half] = cos[r, j]
            rot[j, j + half] = -sin[r, j]
            rot[j + half, j] = sin[r, j]
        for h in range(3):
            inv = 1 / math.sqrt(math.fsum(v * v for v in projected[r, h]) / 128 + 1e-5)
            np.testing.assert_allclose(got["output"][h, r], rot @ (projected[r, h] * inv * gamma), rtol=1e-13,
                                       atol=1e-13)


def test_qk_rope_kats(kats):
    kat = kats["rope_split_half_pairing"]
    p = np.array([[kat["projected"]]])
    out = ref.qk_rope_reference(p, np.ones(6), np.array([kat["cos"]]), np.array([kat["sin"]]),
                                projection_bf16=False, output_bf16=False)
    inv = out["inverse_rms"][0, 0]
    np.testing.assert_allclose(out["output"][0, 0], np.array(kat["expected_over_inverse_rms"]) * inv)
    x = np.arange(30).reshape(3, 2, 5)
    none = ref.qk_rope_reference(x, np.ones(5), np.empty((3, 0)), np.empty((3, 0)))
    np.testing.assert_array_equal(none["rotated"], none["normalized"])
    # gamma is applied before RoPE: rotating first gives a different answer.
    x4 = np.array([[[1.0, 2.0, 3.0, 4.0]]])
    gamma = np.array([2.0, 1.0, 1.0, 1.0])
    good = ref.qk_rope_reference(x4, gamma, np.zeros((1, 2)), np.ones((1, 2)), projection_bf16=False,
                                 output_bf16=False)["output"]
    rotated_first = np.array([[[-3.0, -4.0, 1.0, 2.0]]])
    bad = ref.qk_rope_reference(rotated_first, gamma, np.empty((1, 0)), np.empty((1, 0)), projection_bf16=False,
                                output_bf16=False)["output"]
    assert not np.allclose(good, bad)


# ---- MXINT8 (numerics.py:33-41, 49-52) -----------------------------------------------------


def test_mx_scale_boundaries_kat(kats):
    kat = kats["mx_scale_boundaries"]  # tests/test_numerics.py:28-34
    x = np.array(kat["x_rows"], dtype=np.float32)
    q, s = ref.quantize_reference(x, "mxint8")
    np.testing.assert_array_equal(q, np.array(kat["codes"], dtype=np.int8))
    np.testing.assert_array_equal(s, np.array(kat["scales"], dtype=np.uint8))
    np.testing.assert_array_equal(ref.dequantize(q, s, "mxint8"), x)


def test_mx_zero_and_outlier_kat(kats):
    kat = kats["mx_zero_and_outlier"]  # tests/test_numerics.py:17-25
    x = np.zeros(kat["shape"], np.float32)
    x[kat["outlier"]["row"], kat["outlier"]["col"]] = kat["outlier"]["value"]
    q, s = ref.quantize_reference(x, "mxint8")
    y = ref.dequantize(q, s, "mxint8")
    assert np.all(y[0] == 0) and np.max(np.abs(y - x)) < 1
    assert s.shape == (2, 2) and s.dtype == np.uint8


def test_mx_exponent_matches_float32_log2_at_power_of_two_boundaries():
    """The oracle takes log2 in float64 and rounds to float32 before the floor; the reference
    floors numpy's float32 log2.  Peaks within 64 ulps either side of every power of two (where
    the rounded log2 can reach the next integer) must give the same exponent."""
    peaks = []
    for k in range(-126, 128):
        p = np.float32(2.0**k)
        lo, hi = p, p
        for _ in range(64):
            lo = np.nextafter(lo, np.float32(0))
            hi = np.nextafter(hi, np.float32(np.inf))
            peaks += [lo, hi]
        peaks.append(p)
    peaks = np.array(peaks, dtype=np.float32)
    peaks = peaks[np.isfinite(peaks) & (peaks > 0)]
    literal = np.clip(np.floor(np.log2(np.maximum(peaks, np.finfo(np.float32).tiny))) - 6, -127, 127)
    np.testing.assert_array_equal(ref.mx_exponent(peaks), literal.astype(np.float32))
    # the rounded log2 really does reach the next power for some peaks below it
    assert np.any(ref.mx_exponent(peaks) > np.frexp(peaks)[1] - 1 - 6)


def test_mx_codes_bound_the_block_error():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((16, 256)) * np.exp2(rng.integers(-20, 20, (16, 1)))).astype(np.float32)
    q, s = ref.quantize_reference(x, "mxint8")
    step = np.repeat(np.exp2(s.astype(np.float64) - 127), 32, axis=1)
    err = np.abs(ref.dequantize(q, s, "mxint8").astype(np.float64) - x)
    clipped = np.abs(q) == 127  # a block peak in [127.5, 128) steps rounds past the clamp
    assert np.all(err <= np.where(clipped, step, step / 2) * (1 + 1e-6))
    assert np.all(np.abs(q.astype(np.int16)) <= 127)


# ---- RMS scale-folded quantizer (rms_quant_reference.py:24-89) --------------------------------


def _dense_h(block):
    return np.array([[(-1) ** bin(i & j).count("1") for j in range(block)] for i in range(block)], np.float64) / math.sqrt(block)


@pytest.mark.parametrize("block_size", [1, 4, 128])
@pytest.mark.parametrize("signed", [False, True])
def test_rms_quantize_matches_materialized_dense_definition(block_size, signed):
    """tests/test_rms_quant_reference.py:17-67: normalize with fsum statistics, multiply gamma,
    apply the dense Kronecker H; codes equal, scales to 3e-14."""
    rng = np.random.default_rng(59)
    width = 3 * block_size
    x = rng.normal(size=(5, width))
    gamma = rng.normal(size=width)
    gamma[0] = 0
    x[0, 0] *= 1000
    signs = ref.hadamard_signs(width, 61) if signed else None
    inv = np.array([1.0 / math.sqrt(math.fsum(float(v) ** 2 for v in row) / width + 1e-5) for row in x])
    normalized = x * inv[:, None] * gamma
    expected = (normalized * (signs if signed else 1)) @ np.kron(np.eye(3), _dense_h(block_size))
    peak = np.max(np.abs(expected), axis=1)
    exp_s = np.where(peak == 0, 1.0, peak / 127)
    exp_q = np.clip(np.rint(expected / exp_s[:, None]), -127, 127).astype(np.int8)
    got = ref.rms_quantize_reference(x, gamma, signs, block_size)
    np.testing.assert_allclose(got["inverse_rms"], inv, rtol=3e-14)
    np.testing.assert_allclose(got["scales"], exp_s, rtol=3e-14)
    np.testing.assert_array_equal(got["quantized"], exp_q)


def test_rms_statistics_use_original_input_kat():
    """tests/test_rms_quant_reference.py:91-101."""
    x = np.array([[1.0, 2.0, -4.0, 8.0]])
    gamma = np.array([-100.0, 0.0, 2.0, 0.01])
    got = ref.rms_quantize_reference(x, gamma, block_size=2)
    inv = 1 / math.sqrt((1 + 4 + 16 + 64) / 4 + 1e-5)
    np.testing.assert_allclose(got["inverse_rms"], [inv], rtol=0, atol=0)
    peak = np.max(np.abs((x * gamma) @ np.kron(np.eye(2), _dense_h(2))))
    np.testing.assert_allclose(got["scales"], [peak / 127 * inv], rtol=3e-15)


def test_rms_ties_zero_rows_and_epsilon():
    """tests/test_rms_quant_reference.py:104-123 and :70-88."""
    got = ref.rms_quantize_reference(np.array([[127.0, 2.5, 3.5, -2.5, -3.5, 0.0, -127.0, 1.5]]), np.ones(8))
    np.testing.assert_array_equal(got["quantized"], [[127, 2, 4, -2, -4, 0, -127, 2]])
    np.testing.assert_array_equal(got["scales"], got["inverse_rms"])
    zero = ref.rms_quantize_reference(np.ones((3, 8)), np.zeros(8), block_size=4)
    np.testing.assert_array_equal(zero["quantized"], 0)
    np.testing.assert_array_equal(zero["scales"], np.ones(3))
    rng = np.random.default_rng(67)
    x, g = rng.normal(size=(3, 24)) * 0.01, rng.normal(size=24)
    small, large = ref.rms_quantize_reference(x, g, block_size=8, eps=1e-8), ref.rms_quantize_reference(x, g, block_size=8, eps=1.0)
    np.testing.assert_array_equal(small["quantized"], large["quantized"])
    assert np.all(small["scales"] > large["scales"])


# ---- shift splitting (docs/affine-shift-splitting.md; tests/test_affine_rewrites.py) -----------


def test_shift_crosses_projection_before_rounding():
    """test_affine_rewrites.py:9-17 against the oracle's norm: (norm(x) c + beta) W^T equals
    r (x c) W^T + beta W^T, and the split RMS encoding's normalized rotation is exactly the
    rotation of the modulated activation without its shift (norm_hadamard_gemm.py:330-352)."""
    rng = np.random.default_rng(29)
    x, w = rng.normal(size=(7, 256)), rng.normal(size=(11, 256))
    gamma, scale, beta = rng.normal(size=(3, 256))
    y = ref.norm_modulate_reference(x, gamma, scale, beta)
    r = 1 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + 1e-5)
    c = gamma * (1 + scale)
    np.testing.assert_allclose(y @ w.T, r * ((x * c) @ w.T) + beta @ w.T, rtol=1e-12, atol=1e-12)
    signs = ref.hadamard_signs(256, 0)
    split = ref.rms_quantize_reference(x, c, signs, 128)
    dynamic = ref.block_hadamard_reference(y - beta, 128, signs)
    np.testing.assert_allclose(split["normalized_rotated"], dynamic, rtol=1e-12, atol=1e-12)
    rotated_w = ref.block_hadamard_reference(w, 128, signs)
    np.testing.assert_allclose(dynamic @ rotated_w.T + beta @ w.T, y @ w.T, rtol=1e-12, atol=1e-12)


def test_bf16_boundary_prevents_constant_shift_compensation():
    """test_affine_rewrites.py:20-25: the BF16 rounding correction depends on the activation."""
    a = np.array([1, 1 + 1 / 128], np.float32)
    correction = ref.bf16_round_f32(a + np.float32(1 / 256)) - a
    np.testing.assert_array_equal(correction, [0, 1 / 128])


def test_folding_gamma_into_weights_can_destroy_int8_quality():
    """test_affine_rewrites.py:28-39 through the oracle's quantize / dequantize."""
    x, gamma, w = np.array([[1, 1000]], np.float32), np.array([1000, 1], np.float32), np.ones((1, 2), np.float32)

    def qdq(z):
        return ref.dequantize(*ref.quantize_reference(z, "int8"), "int8")

    np.testing.assert_array_equal(qdq(x * gamma) @ qdq(w).T, [[2000]])
    np.testing.assert_array_equal(qdq(x) @ qdq(w * gamma).T, [[0]])


def test_shift_split_quantization_can_amplify_cancellation_error():
    """test_affine_rewrites.py:42-55."""
    u, beta = np.array([[1, 1000]], np.float32), np.array([[-0.99, -1000]], np.float32)

    def qdq(z):
        return ref.dequantize(*ref.quantize_reference(z, "int8"), "int8")

    target = u + beta
    assert np.linalg.norm(qdq(target) - target) < 1e-6
    assert np.linalg.norm(qdq(u) + beta - target) > 0.9
