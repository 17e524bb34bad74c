"""GPU parity of the MFMA GEMMs (m5k_gemm_i8 / _i8_acc / _f8 / _float).

Bars (north-star targets): INT32 accumulators bit-exact; W8A8 BF16/FP32 outputs
bit-exact against the oracle's FP32 epilogue (hence well within 1 bf16 ulp); FP8 and
float modes within the reference's rel-L2 gate 0.008 of float64 (tests/test_metal.py:85-112
of the reference) and rel-L2 1e-3 of the float64 product for FP32 output.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bits_of, np_of
from m5kernels_amd import gemm, gemm_i8_accumulators, quantize
from oracle import reference as ref

pytestmark = pytest.mark.gpu

SHAPES = [(1, 33, 64), (127, 65, 96), (65, 17, 257), (256, 1024, 1024), (300, 520, 1000), (513, 260, 4096)]


def _codes(m, n, k, seed=83, bound=127):
    rng = np.random.default_rng(seed)
    a = rng.integers(-bound, bound + 1, size=(m, k), dtype=np.int8)
    b = rng.integers(-bound, bound + 1, size=(n, k), dtype=np.int8)
    sa = rng.uniform(0.01, 0.13, size=m).astype(np.float32)
    sb = rng.uniform(0.02, 0.17, size=n).astype(np.float32)
    return a, b, sa, sb


@pytest.fixture(params=["auto", "plain", "quad"])
def schedule(request, monkeypatch):
    """Run a test under the library's launch choice ("auto": shapes with a partial last round
    take the mixed 256 x 256 / 256 x 128 launch or 256 x 224 tiles), with both switched off, and
    with the four-wave grid forced (W8A8; the other modes run plain under it)."""
    _set_schedule(monkeypatch, request.param)
    return request.param


def _set_schedule(monkeypatch, schedule):
    for var in ("M5K_GEMM_MIXED_TILES", "M5K_GEMM_NARROW_TILES"):
        if schedule == "plain":
            monkeypatch.setenv(var, "0")
        else:
            monkeypatch.delenv(var, raising=False)
    if schedule == "quad":
        monkeypatch.setenv("M5K_GEMM_SCHEDULE", "quad")
    else:
        monkeypatch.delenv("M5K_GEMM_SCHEDULE", raising=False)


@pytest.mark.parametrize("shape", SHAPES)
def test_int32_accumulators_bit_exact(shape, schedule, device):
    m, n, k = shape
    a, b, _, _ = _codes(m, n, k)
    acc = gemm_i8_accumulators(torch.from_numpy(a).to(device), torch.from_numpy(b).to(device))
    np.testing.assert_array_equal(np_of(acc), ref.c_gemm_i8_acc(a, b))


def test_int32_accumulators_worst_case_magnitude(device):
    m, n, k = 64, 96, 133144 // 8  # |acc| = 127^2 * K stays exact
    a = np.full((m, k), -127, np.int8)
    b = np.full((n, k), -127, np.int8)
    b[1::2] = 127
    acc = gemm_i8_accumulators(torch.from_numpy(a).to(device), torch.from_numpy(b).to(device))
    expected = np.where(np.arange(n) % 2 == 0, 127 * 127 * k, -127 * 127 * k)
    np.testing.assert_array_equal(np_of(acc), np.broadcast_to(expected, (m, n)))


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("out", ["bf16", "fp32"])
def test_w8a8_epilogue_bit_exact(shape, out, schedule, device):
    m, n, k = shape
    a, b, sa, sb = _codes(m, n, k)
    dt = torch.bfloat16 if out == "bf16" else torch.float32
    y = gemm(torch.from_numpy(a).to(device), torch.from_numpy(b).to(device), "int8",
             a_scales=torch.from_numpy(sa).to(device), b_scales=torch.from_numpy(sb).to(device), output_dtype=dt)
    expected = ref.c_i8_epilogue(ref.c_gemm_i8_acc(a, b), sa, sb, out=out)
    got = bits_of(y) if out == "bf16" else np_of(y)
    np.testing.assert_array_equal(got, expected)


def test_online_w8a8_config1_bit_exact(device):
    """CPU-reference configuration: A bf16 [256,1024] ~N(0,1), W bf16 [1024,1024] ~N(0,0.02), seed 0."""
    rng = np.random.default_rng(0)
    a = rng.standard_normal((256, 1024), dtype=np.float32)
    w = rng.standard_normal((1024, 1024), dtype=np.float32) * np.float32(0.02)
    at = torch.from_numpy(a).to(device).to(torch.bfloat16)
    wt = torch.from_numpy(w).to(device).to(torch.bfloat16)
    wq, ws = quantize(wt, "int8")
    aq, sa = quantize(at, "int8")
    y = gemm(aq, wq, "int8", a_scales=sa, b_scales=ws, output_dtype=torch.bfloat16)
    expected = ref.c_w8a8_linear_bf16(bits_of(at), np_of(wq), np_of(ws))
    np.testing.assert_array_equal(bits_of(y), expected)
    # quality vs the float64 product of the bf16 operands (reference gate 0.05)
    exact = at.double().cpu().numpy() @ wt.double().cpu().numpy().T
    assert ref.metrics(y.float().cpu().numpy(), exact)["relative_l2"] < 0.05


def test_ffn_down_full_size_sampled_rows_bit_exact(device):
    """FFN-down W8A8 (M4096 K16384 N4096) at full size: every output of 32 sampled rows bit-exact."""
    g = torch.Generator(device="cpu").manual_seed(29)
    a = torch.randn((4096, 16384), generator=g)
    a[:, ::1024] *= 50
    w = torch.randn((4096, 16384), generator=g) * 0.02
    at, wt = a.to(device).to(torch.bfloat16), w.to(device).to(torch.bfloat16)
    wq, ws = quantize(wt, "int8")
    aq, sa = quantize(at, "int8")
    y = gemm(aq, wq, "int8", a_scales=sa, b_scales=ws, output_dtype=torch.bfloat16)
    rows = ref.sample_indices(4096)
    aq_rows = np_of(aq)[rows]
    acc = ref.c_gemm_i8_acc(aq_rows, np_of(wq))
    expected = ref.c_i8_epilogue(acc, np_of(sa)[rows], np_of(ws))
    np.testing.assert_array_equal(bits_of(y)[rows], expected)
    # Size-independent property on the whole output: finite, and the row sums of the
    # INT32 accumulators equal A_q . (sum of W_q rows) (linearity, exact in int64).
    # Every partial sum is an integer below 2^53, so float64 is exact in any order.
    accs = gemm_i8_accumulators(aq, wq)
    lhs = accs.to(torch.float64).sum(dim=1)
    rhs = aq.to(torch.float64) @ wq.to(torch.float64).sum(dim=0)
    assert torch.equal(lhs, rhs)
    assert torch.isfinite(y.float()).all()


@pytest.mark.parametrize("mapped", [False, True])
@pytest.mark.parametrize("shape", [(1, 17, 128), (7, 33, 256), (65, 67, 257)])
def test_bias_epilogue_bit_exact(shape, mapped, device):
    m, n, k = shape
    a, b, sa, sb = _codes(m, n, k, bound=17)
    rng = np.random.default_rng(97)
    bias = rng.uniform(-1.5, 1.5, size=(4, n) if mapped else n).astype(np.float32)
    row_map = (np.arange(m, dtype=np.int32) * 3 + 1) % 4 if mapped else None
    y = gemm(torch.from_numpy(a).to(device), torch.from_numpy(b).to(device), "int8", (32, 64, 4, 8),
             a_scales=torch.from_numpy(sa).to(device), b_scales=torch.from_numpy(sb).to(device),
             output_dtype=torch.bfloat16, bias=torch.from_numpy(bias).to(device),
             bias_row_map=None if row_map is None else torch.from_numpy(row_map).to(device))
    expected = ref.c_i8_epilogue(ref.c_gemm_i8_acc(a, b), sa, sb, bias=bias, bias_row_map=row_map)
    np.testing.assert_array_equal(bits_of(y), expected)


def test_bias_before_bf16_rounding_kat(kats, device):
    kat = kats["gemm_bias_before_bf16_rounding"]
    a = torch.zeros(kat["a_shape"], dtype=torch.int8, device=device)
    b = torch.zeros(kat["b_shape"], dtype=torch.int8, device=device)
    a[:, 0] = 1
    b[:, 0] = 1
    y = gemm(a, b, "int8", a_scales=torch.full((a.shape[0],), kat["a_scale"], device=device),
             b_scales=torch.full((b.shape[0],), kat["b_scale"], device=device),
             bias=torch.full((b.shape[0],), kat["bias"], device=device), output_dtype=torch.bfloat16)
    np.testing.assert_array_equal(y.float().cpu().numpy(), np.float32(kat["expected"]))


@pytest.mark.parametrize("mapped", [False, True])
@pytest.mark.parametrize("mode", ["int8", "bf16"])
def test_gated_epilogue(mode, mapped, device):
    m, n, k = 65, 130, 257
    rng = np.random.default_rng(61)
    res = torch.from_numpy(rng.standard_normal((m, n), dtype=np.float32)).to(device).to(torch.bfloat16)
    gate = torch.from_numpy(rng.uniform(-0.7, 0.7, size=(3, n) if mapped else n).astype(np.float32))
    gate = gate.to(device).to(torch.bfloat16)
    gmap = torch.from_numpy((np.arange(m, dtype=np.int32) * 7) % 3).to(device) if mapped else None
    if mode == "int8":
        a, b, sa, sb = _codes(m, n, k)
        args = (torch.from_numpy(a).to(device), torch.from_numpy(b).to(device))
        kw = dict(a_scales=torch.from_numpy(sa).to(device), b_scales=torch.from_numpy(sb).to(device))
        y = gemm(*args, "int8", output_dtype=torch.bfloat16, residual=res, gate=gate, gate_row_map=gmap, **kw)
        expected = ref.c_i8_epilogue(ref.c_gemm_i8_acc(a, b), sa, sb, residual_bits=bits_of(res),
                                     gate_bits=bits_of(gate), gate_row_map=None if gmap is None else np_of(gmap))
        np.testing.assert_array_equal(bits_of(y), expected)
        staged = gemm(*args, "int8", output_dtype=torch.bfloat16, **kw)
    else:
        at = torch.randn(m, k, device=device).to(torch.bfloat16)
        bt = torch.randn(n, k, device=device).to(torch.bfloat16)
        y = gemm(at, bt, "bf16", output_dtype=torch.bfloat16, residual=res, gate=gate, gate_row_map=gmap)
        staged = gemm(at, bt, "bf16", output_dtype=torch.bfloat16)
    # Gated epilogue == staged bf16 branch followed by the FP32 gated add (bitwise).
    g = gate if gmap is None else gate[gmap.long()]
    manual = (res.float() + staged.float() * g.float()).to(torch.bfloat16)
    np.testing.assert_array_equal(bits_of(y), bits_of(manual))


@pytest.mark.parametrize("shape", [(1, 33, 128), (127, 65, 256), (300, 520, 1024), (256, 1024, 1024)])
def test_fp8_gemm(shape, schedule, device):
    m, n, k = shape
    rng = np.random.default_rng(5)
    a = torch.from_numpy(rng.standard_normal((m, k), dtype=np.float32)).to(device).to(torch.bfloat16)
    b = torch.from_numpy(rng.standard_normal((n, k), dtype=np.float32)).to(device).to(torch.bfloat16)
    aq, sa = quantize(a, "fp8")
    bq, sb = quantize(b, "fp8")
    decoded = (ref.dequantize(np_of(aq), np_of(sa), "fp8").astype(np.float64)
               @ ref.dequantize(np_of(bq), np_of(sb), "fp8").astype(np.float64).T)
    y32 = gemm(aq, bq, "fp8", a_scales=sa, b_scales=sb)
    assert y32.dtype == torch.float32
    # The FP8 MFMA sums its 128 products with less than FP32 precision before adding them
    # to the FP32 accumulator (measured rel-L2 ~1.6e-5 at K=128); the bar is 1e-3.
    assert ref.metrics(np_of(y32), decoded)["relative_l2"] < 1e-4
    y = gemm(aq, bq, "fp8", a_scales=sa, b_scales=sb, output_dtype=torch.bfloat16)
    assert ref.metrics(y.float().cpu().numpy(), decoded)["relative_l2"] < 0.008
    # bf16 output is the RNE cast of an FP32 value within 1e-5 of the fp32 output: at most one ulp apart
    diff = np.abs(bits_of(y).astype(np.int32) - ref.f32_to_bf16_bits(np_of(y32)).astype(np.int32))
    assert diff.max() <= 1


def test_fp8_ones_kat(kats, device):
    kat = kats["fp8_ones_gemm"]
    aq, sa = quantize(torch.ones(kat["a_shape"], device=device), "fp8")
    bq, sb = quantize(torch.ones(kat["b_shape"], device=device), "fp8")
    y = gemm(aq, bq, "fp8", a_scales=sa, b_scales=sb)
    np.testing.assert_allclose(np_of(y), kat["expected"], rtol=1e-5)


@pytest.mark.parametrize("mode", ["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("shape", [(1, 33, 64), (127, 65, 96), (65, 17, 257), (300, 520, 1024), (257, 129, 4099)])
def test_float_gemm(mode, shape, schedule, device):
    """Float GEMMs with FP32 accumulation against a float64 product of the same operands.
    Output gates: the reference's implementation rel-L2 (bf16 0.008, fp16 1e-3, fp32 1e-4,
    engine.py gates) on the declared output dtype; FP32 output held to 1e-5 (FP32 accumulation
    over K = 4099 alone is ~sqrt(K) * 2^-24 = 4e-6)."""
    m, n, k = shape
    rng = np.random.default_rng(5)
    dt = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}[mode]
    a = torch.from_numpy(rng.standard_normal((m, k), dtype=np.float32)).to(device).to(dt)
    b = torch.from_numpy(rng.standard_normal((n, k), dtype=np.float32)).to(device).to(dt)
    expected = a.double().cpu().numpy() @ b.double().cpu().numpy().T
    y = gemm(a, b, mode, output_dtype=dt)
    gate = {"bf16": 0.008, "fp16": 1e-3, "fp32": 1e-4}[mode]
    assert ref.metrics(y.float().cpu().numpy(), expected)["relative_l2"] < gate
    y32 = gemm(a, b, mode)
    assert y32.dtype == torch.float32
    assert ref.metrics(np_of(y32), expected)["relative_l2"] < 1e-5


def test_fp32_gemm_exact_small_integers(device):
    """Small-integer FP32 operands make every product and partial sum exact, so the FP32 MFMA
    result must equal the integer product exactly whatever its summation order."""
    rng = np.random.default_rng(9)
    a = rng.integers(-8, 9, (70, 300)).astype(np.float32)
    b = rng.integers(-8, 9, (45, 300)).astype(np.float32)
    y = gemm(torch.from_numpy(a).to(device), torch.from_numpy(b).to(device), "fp32")
    np.testing.assert_array_equal(np_of(y), (a.astype(np.int64) @ b.astype(np.int64).T).astype(np.float32))


def test_repeat_runs_identical(device):
    """Deterministic output across launches (no LDS races in the main loop)."""
    a, b, sa, sb = _codes(513, 777, 2048)
    args = [torch.from_numpy(t).to(device) for t in (a, b)]
    kw = dict(a_scales=torch.from_numpy(sa).to(device), b_scales=torch.from_numpy(sb).to(device),
              output_dtype=torch.bfloat16)
    first = gemm(*args, "int8", **kw)
    for _ in range(3):
        assert torch.equal(gemm(*args, "int8", **kw), first)


@pytest.mark.parametrize("shape", [(64, 96, 128), (257, 130, 4096)])
def test_mxint8_gemm(shape, device):
    """MXINT8 linear against the float64 product of the dequantized operands (reference
    dequantize, numerics.py:49-52): BF16 products are exact, so only FP32 accumulation order
    differs (gate rel-L2 1e-5; the reference's own int8-quality gate is 0.05)."""
    m, n, k = shape
    rng = np.random.default_rng(13)
    a = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(device)
    w = torch.from_numpy((rng.standard_normal((n, k)) * 0.02).astype(np.float32)).to(device)
    aq, ae = quantize(a, "mxint8")
    wq, we = quantize(w, "mxint8")
    y = gemm(aq, wq, "mxint8", a_scales=ae, b_scales=we)
    da = ref.dequantize(np_of(aq), np_of(ae), "mxint8").astype(np.float64)
    dw = ref.dequantize(np_of(wq), np_of(we), "mxint8").astype(np.float64)
    assert ref.metrics(np_of(y), da @ dw.T)["relative_l2"] < 1e-5
    assert ref.metrics(np_of(y), a.double().cpu().numpy() @ w.double().cpu().numpy().T)["relative_l2"] < 0.05
    yb = gemm(aq, wq, "mxint8", a_scales=ae, b_scales=we, output_dtype=torch.bfloat16)
    assert yb.dtype == torch.bfloat16


# ---- split-K W8A8 for short M (m5k_gemm_i8_splitk) -------------------------------------------


def _gemm_i8_call(entry, a, b, sa, sb, out, *, splits=None, bias=None, bias_map=None, residual=None, gate=None,
                  gate_map=None):
    from m5kernels_amd import _lib

    m, k = a.shape
    n = b.shape[0]
    c = torch.empty((m, n), dtype=out, device=a.device)
    args = [_lib.ptr(a), _lib.ptr(b), m, n, k, _lib.ptr(sa), _lib.ptr(sb), _lib.ptr(c), _lib.dtype_code(c),
            _lib.ptr(bias), _lib.ptr(bias_map), _lib.ptr(residual), _lib.ptr(gate), _lib.ptr(gate_map)]
    if entry == "m5k_gemm_i8_splitk":
        ws = torch.full((splits, m, n), 12345, dtype=torch.int32, device=a.device)  # stale contents must not leak
        args += [splits, _lib.ptr(ws), ws.numel()]
    _lib.call(entry, *args, _lib.stream_of(a))
    return c


@pytest.mark.parametrize("shape", [(1, 4096, 4096), (7, 33, 768), (128, 7168, 5376), (200, 1000, 2000),
                                   (300, 520, 1024)])
@pytest.mark.parametrize("splits", [2, 3, 7, 16])
@pytest.mark.parametrize("epilogue", ["bf16", "fp32", "fp16", "bias", "bias_table", "gate", "gate_table"])
def test_splitk_bit_identical_to_plain(shape, splits, epilogue, device):
    """Split-K sums exact INT32 partials and applies the plain epilogue, so every output bit
    matches m5k_gemm_i8 (K 2000 ends in a partial 64-byte slab; 16 splits of short K leave
    some ranges shorter than a stage)."""
    m, n, k = shape
    g = torch.Generator(device="cpu").manual_seed(m + n + k + splits)
    a = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8).to(device)
    b = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).to(device)
    sa = (torch.rand(m, generator=g) * 0.01 + 1e-3).to(device)
    sb = (torch.rand(n, generator=g) * 0.01 + 1e-3).to(device)
    kw, out = {}, {"fp32": torch.float32, "fp16": torch.float16}.get(epilogue, torch.bfloat16)
    rows = torch.tensor([i % 3 for i in range(m)], dtype=torch.int32, device=device)
    if epilogue.startswith("bias"):
        kw["bias"] = torch.randn((3, n) if epilogue == "bias_table" else (n,), generator=g).to(device)
        kw["bias_map"] = rows if epilogue == "bias_table" else None
    elif epilogue.startswith("gate"):
        kw["residual"] = torch.randn((m, n), generator=g).to(torch.bfloat16).to(device)
        kw["gate"] = torch.randn((3, n) if epilogue == "gate_table" else (n,), generator=g).to(torch.bfloat16).to(device)
        kw["gate_map"] = rows if epilogue == "gate_table" else None
    plain = _gemm_i8_call("m5k_gemm_i8", a, b, sa, sb, out, **kw)
    split = _gemm_i8_call("m5k_gemm_i8_splitk", a, b, sa, sb, out, splits=splits, **kw)
    assert torch.equal(plain.view(torch.int16 if out != torch.float32 else torch.int32),
                       split.view(torch.int16 if out != torch.float32 else torch.int32))


def test_splitk_plan_and_routing(device):
    """gemm() takes the split path for few-tile shapes and the plain one otherwise; both are
    bit-exact against the oracle's W8A8 epilogue."""
    from m5kernels_amd.hip import splitk_plan

    assert splitk_plan(4096, 4096, 16384) == 1
    assert splitk_plan(128, 7168, 5376) > 1 and splitk_plan(16, 4096, 4096) > 1
    g = torch.Generator(device="cpu").manual_seed(3)
    for m, n, k in ((128, 1536, 5376), (16, 4096, 4096)):
        assert splitk_plan(m, n, k) > 1
        a = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8).to(device)
        b = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).to(device)
        sa = (torch.rand(m, generator=g) + 0.5).to(device)
        sb = (torch.rand(n, generator=g) + 0.5).to(device)
        y = gemm(a, b, "int8", a_scales=sa, b_scales=sb, output_dtype=torch.bfloat16)
        acc = ref.c_gemm_i8_acc(np_of(a), np_of(b))
        expected = ref.c_i8_epilogue(acc, np_of(sa), np_of(sb), out="bf16")
        np.testing.assert_array_equal(bits_of(y), expected)



# Shapes of 8+ rounds with a partial last round that gemm() splits by rows (256 CUs; the
# library's mixed launch declines them, one shorter round saving under 5%): 2072 tiles (tail
# rows 256, 5 K ranges), 2064 tiles (tail rows 256, 6 ranges), 2080 tiles with a ragged last
# tile row (tail rows 332, 5 ranges).
_TAIL_CASES = [(18944, 7168, 4096), (33024, 4096, 4096), (33100, 4096, 4096)]


@pytest.mark.parametrize("shape", _TAIL_CASES)
@pytest.mark.parametrize("epilogue", ["bf16", "fp32", "fp16", "bias", "bias_table", "gate", "gate_table"])
def test_tail_split_bit_identical_to_plain(shape, epilogue, device):
    """gemm() runs whole tile rows as a plain launch and the rest as split-K, slicing every
    row-indexed operand (scales, row maps, residual, output) at the same row; the result
    matches one plain m5k_gemm_i8 launch bit for bit."""
    from m5kernels_amd.hip import launch_plan, tail_split_plan

    m, n, k = shape
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if cus != 256:
        pytest.skip("shapes chosen for 256 CUs")
    assert tail_split_plan(m, n, k, cus) is not None and launch_plan("int8", m, n, cus)[0] == "plain"
    g = torch.Generator(device="cpu").manual_seed(m + n + k)
    a = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8).to(device)
    b = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).to(device)
    sa = (torch.rand(m, generator=g) * 0.01 + 1e-3).to(device)
    sb = (torch.rand(n, generator=g) * 0.01 + 1e-3).to(device)
    out = {"fp32": torch.float32, "fp16": torch.float16}.get(epilogue, torch.bfloat16)
    rows = torch.tensor([(7 * i) % 3 for i in range(m)], dtype=torch.int32, device=device)
    kw, call_kw = {}, {}
    if epilogue.startswith("bias"):
        kw["bias"] = torch.randn((3, n) if epilogue == "bias_table" else (n,), generator=g).to(device)
        kw["bias_map"] = rows if epilogue == "bias_table" else None
        call_kw = {"bias": kw["bias"], "bias_row_map": kw["bias_map"]}
    elif epilogue.startswith("gate"):
        kw["residual"] = torch.randn((m, n), generator=g).to(torch.bfloat16).to(device)
        kw["gate"] = torch.randn((3, n) if epilogue == "gate_table" else (n,), generator=g).to(torch.bfloat16).to(device)
        kw["gate_map"] = rows if epilogue == "gate_table" else None
        call_kw = {"residual": kw["residual"], "gate": kw["gate"], "gate_row_map": kw["gate_map"]}
    plain = _gemm_i8_call("m5k_gemm_i8", a, b, sa, sb, out, **kw)
    y = gemm(a, b, "int8", a_scales=sa, b_scales=sb, output_dtype=out, **call_kw)
    view = torch.int16 if out != torch.float32 else torch.int32
    assert torch.equal(plain.view(view), y.view(view))


# Shapes the mixed launch takes on 256 CUs: 624 tiles (2 rounds + 224 halves), 128 tiles (all
# halved), a ragged 300 x 200 output (the second half of its one tile 72 wide), 1000 x 600
# (the right halves of the 88-wide last tile column exit at once) and 4096 x 5376 (a round of
# 256 tiles that ends inside a 4-row raster band, + 160 halves; K of 1.5 stages).  Then shapes
# that take 256 x 224 tiles (16 x 16 modes): 4096 x 7168 (512 narrow tiles) and 2048 x 5120
# (a 192-wide last narrow tile column).
_MIXED_CASES = [(9914, 4096, 256), (2048, 4096, 320), (300, 200, 64), (1000, 600, 352), (4096, 5376, 192),
                (4096, 7168, 128), (2048, 5120, 320)]


@pytest.mark.parametrize("shape", _MIXED_CASES)
@pytest.mark.parametrize("epilogue", ["bf16", "fp32", "fp16", "bias", "bias_table", "gate", "gate_table", "acc"])
def test_mixed_tiles_bit_identical_to_plain(shape, epilogue, monkeypatch, device):
    """Every output element of the mixed launch is one workgroup's dot product over all of K,
    like the plain launch's, so the two agree bit for bit in every epilogue."""
    m, n, k = shape
    g = torch.Generator(device="cpu").manual_seed(m + n + k)
    a = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8).to(device)
    b = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).to(device)
    sa = (torch.rand(m, generator=g) * 0.01 + 1e-3).to(device)
    sb = (torch.rand(n, generator=g) * 0.01 + 1e-3).to(device)
    out = {"fp32": torch.float32, "fp16": torch.float16}.get(epilogue, torch.bfloat16)
    rows = torch.tensor([(5 * i) % 3 for i in range(m)], dtype=torch.int32, device=device)
    kw = {}
    if epilogue.startswith("bias"):
        kw["bias"] = torch.randn((3, n) if epilogue == "bias_table" else (n,), generator=g).to(device)
        kw["bias_map"] = rows if epilogue == "bias_table" else None
    elif epilogue.startswith("gate"):
        kw["residual"] = torch.randn((m, n), generator=g).to(torch.bfloat16).to(device)
        kw["gate"] = torch.randn((3, n) if epilogue == "gate_table" else (n,), generator=g).to(torch.bfloat16).to(device)
        kw["gate_map"] = rows if epilogue == "gate_table" else None

    def run():
        if epilogue == "acc":
            return gemm_i8_accumulators(a, b)
        return _gemm_i8_call("m5k_gemm_i8", a, b, sa, sb, out, **kw)

    _set_schedule(monkeypatch, "auto")
    mixed = run()
    _set_schedule(monkeypatch, "plain")
    plain = run()
    view = torch.int16 if mixed.element_size() == 2 else torch.int32
    assert torch.equal(mixed.view(view), plain.view(view))


@pytest.mark.parametrize("shape", _MIXED_CASES)
@pytest.mark.parametrize("mode", ["bf16", "fp16", "fp32", "fp8"])
def test_mixed_tiles_float_modes_bit_identical(shape, mode, monkeypatch, device):
    m, n, k = shape
    if mode == "fp8":
        k = -(-k // 128) * 128  # FP8 rows are whole 128-byte stages
    rng = np.random.default_rng(m + k)
    a = torch.from_numpy(rng.standard_normal((m, k), dtype=np.float32)).to(device)
    b = torch.from_numpy(rng.standard_normal((n, k), dtype=np.float32)).to(device)
    if mode == "fp8":
        (a, sa), (b, sb) = quantize(a.to(torch.bfloat16), "fp8"), quantize(b.to(torch.bfloat16), "fp8")
        kw = dict(a_scales=sa, b_scales=sb, output_dtype=torch.bfloat16)
    else:
        dt = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}[mode]
        a, b = a.to(dt), b.to(dt)
        kw = dict(output_dtype=dt)
    _set_schedule(monkeypatch, "auto")
    mixed = gemm(a, b, mode, **kw)
    _set_schedule(monkeypatch, "plain")
    plain = gemm(a, b, mode, **kw)
    view = torch.int16 if mixed.element_size() == 2 else torch.int32
    assert torch.equal(mixed.view(view), plain.view(view))


@pytest.mark.parametrize("epilogue", ["scales", "bias_table", "gated"])
@pytest.mark.parametrize("shape", [(1000, 700, 528), (4096, 1280, 2048), (513, 4100, 1040)])
def test_quad_schedule_bit_identical_to_plain(shape, epilogue, monkeypatch, device):
    """The four-wave grid (forced quad schedule) against the eight-wave plain launch, with the
    scale, bias-table and gated epilogues, on ragged and multi-round shapes."""
    m, n, k = shape
    print(f"case m={m} n={n} k={k} {epilogue}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(m + n + k)
    a = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8).to(device)
    b = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).to(device)
    kw = dict(a_scales=(torch.rand(m, generator=g) + 0.5).to(device),
              b_scales=(torch.rand(n, generator=g) * 0.01 + 0.001).to(device), output_dtype=torch.bfloat16)
    if epilogue == "bias_table":
        kw.update(bias=torch.randn((3, n), generator=g).to(device),
                  bias_row_map=(torch.arange(m, dtype=torch.int32) % 3).to(device))
    elif epilogue == "gated":
        kw.update(residual=torch.randn((m, n), generator=g).to(torch.bfloat16).to(device),
                  gate=torch.randn((n,), generator=g).to(torch.bfloat16).to(device))
    _set_schedule(monkeypatch, "plain")
    plain = gemm(a, b, "int8", **kw)
    _set_schedule(monkeypatch, "quad")
    quad = gemm(a, b, "int8", **kw)
    assert torch.equal(quad.view(torch.int16), plain.view(torch.int16))


def _random_schedule_cases(count_per_schedule=20, seed=2024):
    """Seeded random [m, n, k, mode] cases, `count_per_schedule` for each of the plain, mixed and
    narrow schedules (as the library plans them on 256 CUs), with ragged m, n and K."""
    import random

    from m5kernels_amd.hip import launch_plan

    rng = random.Random(seed)
    counts = {"plain": 0, "mixed": 0, "narrow": 0}
    cases = []
    while len(cases) < 3 * count_per_schedule:
        m = rng.choice([rng.randint(1, 600), rng.randint(600, 5000), rng.randint(5000, 12000)])
        n = rng.choice([rng.randint(1, 700), rng.randint(700, 8000), rng.randint(8000, 16000)])
        sched = launch_plan("int8", m, n, 256)[0]
        if counts[sched] >= count_per_schedule:
            continue
        counts[sched] += 1
        mode = ("int8", "bf16", "fp16", "fp32", "fp8")[len(cases) % 5]
        k = 128 * rng.randint(1, 3) if mode == "fp8" else 16 * rng.randint(1, 24)
        cases.append((m, n, k, mode, sched))
    return cases


def test_schedules_random_shapes_bit_identical(monkeypatch, device):
    """60 seeded random shapes, 20 per INT8 schedule, spread over the five modes: the library's
    choice (plain, mixed, or narrow for the 16 x 16 modes) gives the same bits as the plain
    launch."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if cus != 256:
        pytest.skip("cases chosen for 256 CUs")
    g = torch.Generator(device="cpu").manual_seed(11)
    for m, n, k, mode, sched in _random_schedule_cases():
        print(f"case m={m} n={n} k={k} {mode} {sched}", flush=True)
        if mode == "int8":
            a = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8).to(device)
            b = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).to(device)
            kw = dict(a_scales=(torch.rand(m, generator=g) + 0.5).to(device),
                      b_scales=(torch.rand(n, generator=g) + 0.5).to(device), output_dtype=torch.bfloat16)
        elif mode == "fp8":
            a, sa = quantize(torch.randn((m, k), generator=g).to(torch.bfloat16).to(device), "fp8")
            b, sb = quantize(torch.randn((n, k), generator=g).to(torch.bfloat16).to(device), "fp8")
            kw = dict(a_scales=sa, b_scales=sb, output_dtype=torch.float32)
        else:
            dt = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[mode]
            a = torch.randn((m, k), generator=g).to(dt).to(device)
            b = torch.randn((n, k), generator=g).to(dt).to(device)
            kw = dict(output_dtype=dt)
        _set_schedule(monkeypatch, "auto")
        auto = gemm(a, b, mode, **kw)
        _set_schedule(monkeypatch, "plain")
        plain = gemm(a, b, mode, **kw)
        view = torch.int16 if auto.element_size() == 2 else torch.int32
        assert torch.equal(auto.view(view), plain.view(view)), (m, n, k, mode, sched)
        del a, b, auto, plain


def test_ops_launch_on_the_current_stream(device):
    """The wrappers launch on torch's current stream of the operand's device: on a side stream
    the handle passed to the library is that stream's, and the results equal the default
    stream's bit for bit."""
    from m5kernels_amd import _lib

    g = torch.Generator(device="cpu").manual_seed(7)
    x = torch.randn((300, 512), generator=g).to(torch.bfloat16).to(device)
    w = torch.randn((260, 512), generator=g).to(torch.bfloat16).to(device)
    assert _lib.stream_of(x) == torch.cuda.current_stream(device).cuda_stream
    wq, ws = quantize(w, "int8")
    q0, s0 = quantize(x, "int8")
    y0 = gemm(q0, wq, "int8", a_scales=s0, b_scales=ws, output_dtype=torch.bfloat16)
    side = torch.cuda.Stream(device=device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        assert _lib.stream_of(x) == side.cuda_stream
        q1, s1 = quantize(x, "int8")
        y1 = gemm(q1, wq, "int8", a_scales=s1, b_scales=ws, output_dtype=torch.bfloat16)
    torch.cuda.current_stream(device).wait_stream(side)
    torch.cuda.synchronize(device)
    assert torch.equal(q1, q0) and torch.equal(s1, s0)
    assert np.array_equal(bits_of(y1), bits_of(y0))


@pytest.mark.parametrize("shape", [(128, 5376, 14336), (16, 4096, 4096), (300, 1000, 1024), (1, 96, 5376)])
def test_fp8_split_k_against_float64_and_unsplit(shape, device):
    """Short-M FP8 GEMMs take the split-K launch (FP32 partials summed in split order): within the
    FP8 bar of the decoded float64 product, within FP32 rounding of the unsplit launch, and the
    same bits on a second call."""
    from m5kernels_amd import hip

    m, n, k = shape
    print(f"case m={m} n={n} k={k}", flush=True)
    assert hip.splitk_plan(m, n, k, 256, skinny=False) > 1
    g = torch.Generator(device="cpu").manual_seed(m + n + k)
    a = torch.randn((m, k), generator=g).to(torch.bfloat16).to(device)
    b = (torch.randn((n, k), generator=g) * 0.02).to(torch.bfloat16).to(device)
    aq, sa = quantize(a, "fp8")
    bq, sb = quantize(b, "fp8")
    decoded = (ref.dequantize(np_of(aq), np_of(sa), "fp8").astype(np.float64)
               @ ref.dequantize(np_of(bq), np_of(sb), "fp8").astype(np.float64).T)
    y_split = gemm(aq, bq, "fp8", a_scales=sa, b_scales=sb)
    with hip.launch_override("plain"):
        y_plain = gemm(aq, bq, "fp8", a_scales=sa, b_scales=sb)
    assert ref.metrics(np_of(y_split), decoded)["relative_l2"] < 1e-4
    assert ref.metrics(np_of(y_split), np_of(y_plain).astype(np.float64))["relative_l2"] < 1e-5
    assert torch.equal(gemm(aq, bq, "fp8", a_scales=sa, b_scales=sb), y_split)
    y16 = gemm(aq, bq, "fp8", a_scales=sa, b_scales=sb, output_dtype=torch.bfloat16)
    assert ref.metrics(y16.float().cpu().numpy(), decoded)["relative_l2"] < 0.008
