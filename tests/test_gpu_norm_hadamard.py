"""GPU parity of the fused AdaLN / gated-residual / Hadamard / INT8 prep and its staged
comparators (m5k_norm_hadamard_quantize, m5k_norm_modulate, m5k_gated_residual_add).

Bars, as the reference's own GPU tests set them (tests/test_norm_hadamard_metal.py:33-82 and
tests/test_gated_norm_hadamard_metal.py:42-103 of the reference): codes within 1 of the
float64 reference after the declared rounding boundary, scales within rtol 3e-5, decoded
error bounded by the two scales; R_next bit-exact (FP32 product then add, one cast); fused
R_next == standalone gated_residual_add bitwise.  Beyond the reference: the fused codes equal
the staged rotate(quantize(unfused_norm(x))) composition bit for bit (blocks <= 512).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bits_of, np_of
from m5kernels_amd import (
    fused_gated_residual_norm_hadamard_quantize,
    fused_norm_hadamard_quantize,
    gated_residual_add,
    quantize,
    rotate,
    rotate_quantize,
    unfused_norm,
)
from oracle import reference as ref

pytestmark = pytest.mark.gpu


def _round(y, dtype):
    y = np.asarray(y, dtype=np.float32)
    if dtype == torch.float16:
        return y.astype(np.float16).astype(np.float32)
    if dtype == torch.bfloat16:
        return ref.bf16_round_f32(y)
    return y


def _modulated_reference(x_cpu, gamma, scale, shift, row_map, norm, eps):
    if row_map is None:
        return ref.norm_modulate_reference(x_cpu, gamma, scale, shift, norm=norm, eps=eps)
    return np.concatenate([
        ref.norm_modulate_reference(x_cpu[r : r + 1], gamma, scale[i], shift[i], norm=norm, eps=eps)
        for r, i in enumerate(row_map)
    ])


def check_codes(q, s, x_f32, gamma, scale, shift, signs, block, *, norm, eps, out_dtype, row_map=None):
    q, s = np_of(q), np_of(s)
    modulated = _round(_modulated_reference(x_f32, gamma, scale, shift, row_map, norm, eps), out_dtype)
    rotated = ref.block_hadamard_reference(modulated, block, signs)
    rq, rs = ref.quantize_reference(rotated, "int8")
    assert q.dtype == np.int8 and s.dtype == np.float32
    assert np.isfinite(s).all() and np.all(s > 0)
    assert np.max(np.abs(q.astype(np.int16) - rq.astype(np.int16))) <= 1
    np.testing.assert_allclose(s, rs, rtol=3e-5, atol=1e-7)
    decoded = q.astype(np.float64) * s[:, None]
    expected = rq.astype(np.float64) * rs[:, None]
    bound = np.maximum(s, rs) + 127 * np.abs(s - rs)
    assert np.all(np.abs(decoded - expected) <= bound[:, None] + 1e-7)


def _f32(t):
    return t.float().cpu().numpy()


DT = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}


@pytest.mark.parametrize("norm", ["rms", "layer"])
@pytest.mark.parametrize("dtype", list(DT))
@pytest.mark.parametrize("kind", ["normal", "zeros", "outliers"])
@pytest.mark.parametrize("width", [5376, 6144])
def test_h3_width_full_output(norm, dtype, kind, width, device):
    rng = np.random.default_rng(621)
    x = rng.standard_normal((7, width), dtype=np.float32)
    if kind == "zeros":
        x.fill(0)
    elif kind == "outliers":
        x[:, ::137] *= 100
    gamma = rng.uniform(0.5, 1.5, size=width).astype(np.float32)
    scale = rng.uniform(-0.3, 0.3, size=width).astype(np.float32)
    shift = rng.uniform(-0.1, 0.1, size=width).astype(np.float32)
    signs = ref.hadamard_signs(width, 29)
    xt = torch.from_numpy(x).to(device).to(DT[dtype])
    args = [torch.from_numpy(t).to(device) for t in (gamma, scale, shift, signs)]
    q, s = fused_norm_hadamard_quantize(xt, *args, 256, norm=norm)
    check_codes(q, s, _f32(xt), gamma, scale, shift, signs, 256, norm=norm, eps=1e-5, out_dtype=DT[dtype])


@pytest.mark.parametrize("block", [32, 64, 128, 256, 512, 1024])
@pytest.mark.parametrize("norm", ["rms", "layer"])
def test_blocks(block, norm, device):
    rng = np.random.default_rng(31)
    width = block * 3
    x = torch.from_numpy(rng.standard_normal((3, width), dtype=np.float32)).to(device)
    gamma, scale, shift = np.ones(width, np.float32), np.full(width, 0.125, np.float32), np.full(width, 0.0625, np.float32)
    signs = ref.hadamard_signs(width, 13)
    q, s = fused_norm_hadamard_quantize(x, *[torch.from_numpy(t).to(device) for t in (gamma, scale, shift, signs)],
                                        block, norm=norm, threads=128)
    check_codes(q, s, _f32(x), gamma, scale, shift, signs, block, norm=norm, eps=1e-5, out_dtype=torch.float32)


@pytest.mark.parametrize("norm", ["rms", "layer"])
@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_fp32_post_modulation_boundary(norm, dtype, device):
    rng = np.random.default_rng(51)
    x = torch.from_numpy(rng.standard_normal((3, 768), dtype=np.float32)).to(device).to(DT[dtype])
    vals = [np.full(768, v, np.float32) for v in (1.1, -0.13, 0.037)]
    signs = ref.hadamard_signs(768, 41)
    q, s = fused_norm_hadamard_quantize(x, *[torch.from_numpy(t).to(device) for t in (*vals, signs)], 256, norm=norm,
                                        round_output="fp32", epsilon=1e-4, passes="two_read")
    check_codes(q, s, _f32(x), *vals, signs, 256, norm=norm, eps=1e-4, out_dtype=torch.float32)


def test_explicit_bf16_rounding_ties(device):
    width = 256
    shift = np.resize(np.array([1.00390625, 1.01171875, -1.00390625, -1.01171875], np.float32), width)
    x = torch.zeros((3, width), dtype=torch.bfloat16, device=device)
    zeros = torch.zeros(width, device=device)
    for round_output, dtype in (("input", torch.bfloat16), ("fp32", torch.float32)):
        y = unfused_norm(x, zeros, zeros, torch.from_numpy(shift).to(device), round_output=round_output)
        assert y.dtype == dtype
        np.testing.assert_array_equal(_f32(y), np.broadcast_to(_round(shift, dtype), (3, width)))
        signs = ref.hadamard_signs(width, 3)
        q, s = fused_norm_hadamard_quantize(x, zeros, zeros, torch.from_numpy(shift).to(device),
                                            torch.from_numpy(signs).to(device), width, round_output=round_output)
        check_codes(q, s, _f32(x), np.zeros(width), np.zeros(width), shift, signs, width, norm="rms", eps=1e-5,
                    out_dtype=dtype)


def test_layernorm_constant_rows_quantize_to_zero(device):
    x = torch.full((7, 5376), 17.0, device=device)
    q, s = fused_norm_hadamard_quantize(x, torch.ones(5376, device=device), torch.full((5376,), 0.5, device=device),
                                        torch.zeros(5376, device=device),
                                        torch.from_numpy(ref.hadamard_signs(5376, 43)).to(device), 256, norm="layer")
    assert torch.all(q == 0) and torch.all(s == 1.0)


@pytest.mark.parametrize("norm", ["rms", "layer"])
def test_row_map_tables(norm, device):
    rng = np.random.default_rng(61)
    x = torch.from_numpy(rng.standard_normal((7, 768), dtype=np.float32)).to(device).to(torch.bfloat16)
    gamma = rng.uniform(0.5, 1.5, size=768).astype(np.float32)
    scale = rng.uniform(-0.3, 0.3, size=(3, 768)).astype(np.float32)
    shift = rng.uniform(-0.1, 0.1, size=(3, 768)).astype(np.float32)
    row_map = np.array([2, 0, 1, 0, 2, 2, 1], dtype=np.int32)
    signs = ref.hadamard_signs(768, 11)
    d = [torch.from_numpy(t).to(device) for t in (gamma, scale, shift, signs, row_map)]
    q, s = fused_norm_hadamard_quantize(x, d[0], d[1], d[2], d[3], 256, norm=norm, row_map=d[4])
    check_codes(q, s, _f32(x), gamma, scale, shift, signs, 256, norm=norm, eps=1e-5, out_dtype=torch.bfloat16,
                row_map=row_map)
    mapped = unfused_norm(x, d[0], d[1], d[2], norm=norm, row_map=d[4])
    for r, i in enumerate(row_map):
        direct = unfused_norm(x[r : r + 1], d[0], d[1][i], d[2][i], norm=norm)
        assert torch.equal(mapped[r], direct[0])


@pytest.mark.parametrize("norm", ["rms", "layer"])
@pytest.mark.parametrize("round_output", ["input", "fp32"])
@pytest.mark.parametrize("block,width", [(128, 4096), (256, 4096), (512, 4096), (256, 5120), (128, 6144),
                                         (256, 3072), (512, 7168)])
def test_fused_equals_staged_bitwise(norm, round_output, block, width, device):
    """Widths cover every register-chunk count of a lane: 1.5, 2, 2.5, 3, 3.5 chunks of 8."""
    rng = np.random.default_rng(71)
    x = torch.from_numpy(rng.standard_normal((9, width), dtype=np.float32)).to(device).to(torch.bfloat16)
    gamma = (1 + 0.1 * torch.randn(width, device=device)).to(torch.bfloat16)
    scale = (0.1 * torch.randn(2, width, device=device)).to(torch.bfloat16)
    shift = (0.1 * torch.randn(2, width, device=device)).to(torch.bfloat16)
    row_map = torch.tensor([0, 1] * 4 + [1], dtype=torch.int32, device=device)
    signs = torch.from_numpy(ref.hadamard_signs(width, 5)).to(device)
    q, s = fused_norm_hadamard_quantize(x, gamma, scale, shift, signs, block, norm=norm, round_output=round_output,
                                        row_map=row_map)
    y = unfused_norm(x, gamma, scale, shift, norm=norm, round_output=round_output, row_map=row_map)
    sq, ss = quantize(rotate(y, block, signs), "int8")
    assert torch.equal(q, sq) and torch.equal(s, ss)
    q2, s2 = rotate_quantize(y, block, signs)
    assert torch.equal(q, q2) and torch.equal(s, s2)


@pytest.mark.parametrize("norm", ["rms", "layer"])
@pytest.mark.parametrize("distribution", ["normal", "outliers"])
@pytest.mark.parametrize("mapped", [False, True])
def test_gated_residual_prep(norm, distribution, mapped, device):
    rng = np.random.default_rng(323)
    shape = (7, 5376)
    residual = rng.standard_normal(shape, dtype=np.float32)
    branch = rng.standard_normal(shape, dtype=np.float32)
    if distribution == "outliers":
        branch[:, ::137] *= 100
        residual[:, ::251] *= 50
    rt = torch.from_numpy(residual).to(device).to(torch.bfloat16)
    bt = torch.from_numpy(branch).to(device).to(torch.bfloat16)
    gate = rng.uniform(-0.7, 0.7, size=(3, 5376) if mapped else 5376).astype(np.float32)
    gmap = np.array([1, 0, 2, 2, 1, 0, 1], np.int32) if mapped else None
    gamma = rng.uniform(0.7, 1.3, size=5376).astype(np.float32)
    scale = rng.uniform(-0.2, 0.2, size=5376).astype(np.float32)
    shift = rng.uniform(-0.1, 0.1, size=5376).astype(np.float32)
    signs = ref.hadamard_signs(5376, 29)
    before_r, before_b = rt.clone(), bt.clone()
    d = {k: torch.from_numpy(v).to(device) for k, v in dict(gate=gate, gamma=gamma, scale=scale, shift=shift,
                                                            signs=signs).items()}
    gm = None if gmap is None else torch.from_numpy(gmap).to(device)
    q, s, updated = fused_gated_residual_norm_hadamard_quantize(
        rt, bt, d["gate"], d["gamma"], d["scale"], d["shift"], d["signs"], 256, norm=norm, gate_row_map=gm)
    assert torch.equal(rt, before_r) and torch.equal(bt, before_b)
    assert updated.dtype == torch.bfloat16 and updated.shape == rt.shape
    # R_next: FP32 product, FP32 add, one BF16 cast -> bit-exact in numpy float32
    g_sel = gate if gmap is None else gate[gmap]
    expected = ref.f32_to_bf16_bits((_f32(rt) + _f32(bt) * g_sel).astype(np.float32))
    np.testing.assert_array_equal(bits_of(updated), expected)
    standalone = gated_residual_add(rt, bt, d["gate"], gate_row_map=gm)
    assert torch.equal(updated, standalone)
    check_codes(q, s, _f32(updated), gamma, scale, shift, signs, 256, norm=norm, eps=1e-5, out_dtype=torch.bfloat16)
    # The gated fused path equals ungated fused prep of the materialized R_next.
    q2, s2 = fused_norm_hadamard_quantize(updated, d["gamma"], d["scale"], d["shift"], d["signs"], 256, norm=norm)
    assert torch.equal(q, q2) and torch.equal(s, s2)


def test_gated_cancellation_needs_fp32_product(device):
    """A product rounded to BF16 before the add would cancel to 0; the FP32 product keeps it."""
    k = 256
    res = torch.full((1, k), -1.0, device=device, dtype=torch.bfloat16)
    branch = torch.full((1, k), 1.0078125, device=device, dtype=torch.bfloat16)  # 1 + 2^-7
    gate = torch.full((k,), 1.0 - 2**-8, device=device, dtype=torch.float32)
    out = gated_residual_add(res, branch, gate)
    exact = np.float32(-1.0) + np.float32(1.0078125) * np.float32(1.0 - 2**-8)
    assert float(out[0, 0]) == float(ref.bf16_round_f32(np.array([exact]))[0]) != 0.0


def test_prep_configuration_shapes(device):
    """Fused-prep configuration: M=4096 (and 9914 rows sampled), hidden 4096, LayerNorm, H128,
    per-batch tables (P=2), gated residual, then the W8A8 4096x4096 GEMM."""
    for m in (4096, 9914):
        g = torch.Generator(device=device).manual_seed(17)
        x = torch.randn((m, 4096), generator=g, device=device).to(torch.bfloat16)
        br = torch.randn((m, 4096), generator=g, device=device).to(torch.bfloat16)
        tab = lambda: (0.1 * torch.randn((2, 4096), generator=g, device=device)).to(torch.bfloat16)  # noqa: E731
        shift, scale, gate = tab(), tab(), tab()
        gamma = (1 + 0.1 * torch.randn(4096, generator=g, device=device)).to(torch.bfloat16)
        row_map = (torch.arange(m, device=device, dtype=torch.int32) >= m // 2).to(torch.int32)
        signs = torch.from_numpy(ref.hadamard_signs(4096, 7)).to(device)
        q, s, upd = fused_gated_residual_norm_hadamard_quantize(x, br, gate, gamma, scale, shift, signs, 128,
                                                                norm="layer", gate_row_map=row_map, row_map=row_map)
        rows = ref.sample_indices(m)
        rmap = np_of(row_map)[rows]
        check_codes(q[rows], s[rows], _f32(upd[rows]), _f32(gamma), _f32(scale), _f32(shift), np_of(signs), 128,
                    norm="layer", eps=1e-5, out_dtype=torch.bfloat16, row_map=rmap)
        staged = gated_residual_add(x, br, gate, gate_row_map=row_map)
        assert torch.equal(staged, upd)


# ---- bit-exact against the fixed-order FP32 oracle (oracle_prep_rows) ---------------------------


def _oracle_prep(x, gamma, scale, shift, signs, block, **kw):
    f32 = lambda t: None if t is None else (t.float().cpu().numpy() if isinstance(t, torch.Tensor) else t)  # noqa: E731
    dt = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}[x.dtype]
    for key in ("branch", "gate"):
        if key in kw:
            kw[key] = f32(kw[key])
    for key in ("row_map", "gate_row_map"):
        if kw.get(key) is not None:
            kw[key] = np_of(kw[key])
    return ref.c_prep_rows(f32(x), f32(gamma), f32(scale), f32(shift), np_of(signs), block, dtype=dt, **kw)


@pytest.mark.parametrize("norm", ["rms", "layer"])
@pytest.mark.parametrize("dtype", list(DT))
@pytest.mark.parametrize("round_output", ["input", "fp32"])
@pytest.mark.parametrize("block,width", [(32, 768), (128, 4096), (256, 5376), (512, 3072), (1024, 6144),
                                         (64, 5120), (256, 16384)])
def test_fused_prep_bit_exact_vs_fixed_order_oracle(norm, dtype, round_output, block, width, device):
    """Codes and scales equal the oracle's fixed FP32 order bit for bit: lane chunks of
    max(8, B/64) elements, the DPP row tree, fmaf squares and modulation, the O cast."""
    rng = np.random.default_rng(block + width + len(dtype))
    x = torch.from_numpy(rng.standard_normal((9, width), dtype=np.float32)).to(device).to(DT[dtype])
    x[3, ::97] *= 60
    gamma = (1 + 0.1 * torch.randn(width, device=device)).to(torch.bfloat16)
    scale = (0.1 * torch.randn(2, width, device=device)).to(torch.bfloat16)
    shift = (0.1 * torch.randn(2, width, device=device)).to(torch.bfloat16)
    row_map = torch.tensor([0, 1] * 4 + [1], dtype=torch.int32, device=device)
    signs = torch.from_numpy(ref.hadamard_signs(width, 5)).to(device)
    q, s = fused_norm_hadamard_quantize(x, gamma, scale, shift, signs, block, norm=norm, round_output=round_output,
                                        row_map=row_map)
    oq, os_ = _oracle_prep(x, gamma, scale, shift, signs, block, norm=norm, round_output=round_output, row_map=row_map)
    np.testing.assert_array_equal(np_of(q), oq)
    np.testing.assert_array_equal(np_of(s), os_)


@pytest.mark.parametrize("norm", ["rms", "layer"])
@pytest.mark.parametrize("dtype,branch_dtype", [("bf16", "bf16"), ("bf16", "fp32"), ("bf16", "fp16"),
                                                ("fp16", "bf16"), ("fp32", "bf16"), ("fp16", "fp16")])
@pytest.mark.parametrize("mapped", [False, True])
@pytest.mark.parametrize("width", [5376, 4096])
def test_gated_prep_mixed_branch_dtype_bit_exact(norm, dtype, branch_dtype, mapped, width, device):
    """A branch of another float dtype than the residual: float(branch) enters the FP32 product
    and add as is (norm_hadamard.py:184 accepts any float dtype); R_next, codes and scales equal
    the fixed-order oracle, and the staged gated_residual_add equals R_next.  Width 4096 fills
    every lane's chunks (the full-row instantiation), 5376 leaves lanes idle."""
    rng = np.random.default_rng(401)
    shape = (7, width)
    rt = torch.from_numpy(rng.standard_normal(shape, dtype=np.float32)).to(device).to(DT[dtype])
    bt = torch.from_numpy(rng.standard_normal(shape, dtype=np.float32) * 3).to(device).to(DT[branch_dtype])
    gate = torch.from_numpy(rng.uniform(-0.7, 0.7, size=(3, width) if mapped else width).astype(np.float32))
    gate = gate.to(device).to(torch.bfloat16)
    gmap = torch.tensor([1, 0, 2, 2, 1, 0, 1], dtype=torch.int32, device=device) if mapped else None
    gamma = (1 + 0.1 * torch.randn(width, device=device)).to(torch.bfloat16)
    scale = (0.1 * torch.randn(width, device=device)).to(torch.bfloat16)
    shift = (0.1 * torch.randn(width, device=device)).to(torch.bfloat16)
    signs = torch.from_numpy(ref.hadamard_signs(width, 29)).to(device)
    q, s, upd = fused_gated_residual_norm_hadamard_quantize(rt, bt, gate, gamma, scale, shift, signs, 256, norm=norm,
                                                            gate_row_map=gmap)
    assert upd.dtype == rt.dtype
    oq, os_, orn = _oracle_prep(rt, gamma, scale, shift, signs, 256, norm=norm, branch=bt, gate=gate,
                                gate_row_map=gmap)
    np.testing.assert_array_equal(upd.float().cpu().numpy(), orn)
    np.testing.assert_array_equal(np_of(q), oq)
    np.testing.assert_array_equal(np_of(s), os_)
    assert torch.equal(gated_residual_add(rt, bt, gate, gate_row_map=gmap), upd)


@pytest.mark.parametrize("norm", ["rms", "layer"])
@pytest.mark.parametrize("tables", [("fp16", "fp32", "bf16", "fp16"), ("fp32", "fp32", "fp32", "fp32"),
                                    ("fp16", "fp16", "fp16", "fp16"), ("bf16", "bf16", "fp32", "bf16"),
                                    ("bf16", "fp16", "bf16", "fp32")])
@pytest.mark.parametrize("dtype,branch_dtype,width", [("bf16", "fp16", 4096), ("fp16", "fp32", 5376),
                                                      ("fp32", "bf16", 4096), ("bf16", "bf16", 4096)])
def test_prep_mixed_table_dtypes_one_dispatch_bit_exact(norm, tables, dtype, branch_dtype, width, device,
                                                        monkeypatch):
    """gamma, scale, shift and gate each in their own float dtype, and a branch in any float dtype:
    the one prep dispatch reads every input as given (the reference's kernel reads float() of each
    input in its own dtype, norm_hadamard.py:67-70), so no host-side cast runs.  R_next, codes and
    scales equal the fixed-order oracle fed the same values, the ungated prep and the staged
    comparators agree, and the pointers handed to the C ABI are the caller's own tensors."""
    from m5kernels_amd import _lib

    rng = np.random.default_rng(733)
    shape = (6, width)
    rt = torch.from_numpy(rng.standard_normal(shape, dtype=np.float32)).to(device).to(DT[dtype])
    bt = torch.from_numpy(rng.standard_normal(shape, dtype=np.float32) * 2).to(device).to(DT[branch_dtype])
    g_dt, sc_dt, sh_dt, gt_dt = (DT[t] for t in tables)
    gamma = torch.from_numpy(1 + 0.1 * rng.standard_normal(width).astype(np.float32)).to(device).to(g_dt)
    scale = torch.from_numpy(0.1 * rng.standard_normal((2, width)).astype(np.float32)).to(device).to(sc_dt)
    shift = torch.from_numpy(0.1 * rng.standard_normal((2, width)).astype(np.float32)).to(device).to(sh_dt)
    gate = torch.from_numpy(rng.uniform(-0.8, 0.8, size=(3, width)).astype(np.float32)).to(device).to(gt_dt)
    row_map = torch.tensor([1, 0, 0, 1, 1, 0], dtype=torch.int32, device=device)
    gmap = torch.tensor([2, 0, 1, 1, 2, 0], dtype=torch.int32, device=device)
    signs = torch.from_numpy(ref.hadamard_signs(width, 31)).to(device)
    calls = []
    real_call = _lib.call

    def spy(name, *args):
        calls.append((name, args))
        return real_call(name, *args)

    monkeypatch.setattr(_lib, "call", spy)
    q, s, upd = fused_gated_residual_norm_hadamard_quantize(rt, bt, gate, gamma, scale, shift, signs, 256, norm=norm,
                                                            gate_row_map=gmap, row_map=row_map)
    name, args = calls[-1]
    assert name == "m5k_norm_hadamard_quantize"
    handed = {args[i] for i in (0, 4, 6, 8, 9, 10)}
    assert handed == {t.data_ptr() for t in (rt, bt, gate, gamma, scale, shift)}
    assert args[5] == _lib.dtype_code(bt)
    oq, os_, orn = _oracle_prep(rt, gamma, scale, shift, signs, 256, norm=norm, branch=bt, gate=gate,
                                gate_row_map=gmap, row_map=row_map)
    np.testing.assert_array_equal(upd.float().cpu().numpy(), orn)
    np.testing.assert_array_equal(np_of(q), oq)
    np.testing.assert_array_equal(np_of(s), os_)
    assert torch.equal(gated_residual_add(rt, bt, gate, gate_row_map=gmap), upd)
    q2, s2 = fused_norm_hadamard_quantize(upd, gamma, scale, shift, signs, 256, norm=norm, row_map=row_map)
    assert torch.equal(q2, q) and torch.equal(s2, s)
    f32 = lambda t: t.float()  # noqa: E731  (exact widening: the same values in FP32 tables)
    y = unfused_norm(upd, gamma, scale, shift, norm=norm, row_map=row_map)
    assert torch.equal(y, unfused_norm(upd, f32(gamma), f32(scale), f32(shift), norm=norm, row_map=row_map))


@pytest.mark.parametrize("norm", ["rms", "layer"])
@pytest.mark.parametrize("gated", [False, True])
@pytest.mark.parametrize("dtype,block,width,round_output", [("bf16", 128, 4096, "input"), ("fp32", 32, 768, "input"),
                                                            ("bf16", 1024, 4096, "fp32"), ("fp16", 64, 2048, "input"),
                                                            ("bf16", 256, 5376, "input")])
def test_irregular_table_maps_bit_exact(norm, gated, dtype, block, width, round_output, device):
    """Three scale/shift tables and two gate tables in irregular row orders, a row with a
    x40 outlier stripe and a constant row (LayerNorm centres it to zero); widths that fill
    the lanes and widths that leave lanes idle.  Codes, scales and R_next equal the
    fixed-order oracle bit for bit."""
    rows = 23
    rng = np.random.default_rng(width + block)
    x = torch.from_numpy(rng.standard_normal((rows, width), dtype=np.float32)).to(device).to(DT[dtype])
    x[5, ::61] *= 40
    x[11] = 0.5  # a constant row: LayerNorm centres it to zero
    gamma = (1 + 0.1 * torch.randn(width, device=device)).to(torch.bfloat16)
    scale = (0.1 * torch.randn(3, width, device=device)).to(torch.bfloat16)
    shift = (0.1 * torch.randn(3, width, device=device)).to(torch.bfloat16)
    row_map = torch.tensor([0, 0, 1, 2, 2, 2, 0, 1, 1, 0, 2, 2, 2, 2, 1, 0, 0, 0, 1, 2, 0, 1, 1], dtype=torch.int32,
                           device=device)
    signs = torch.from_numpy(ref.hadamard_signs(width, 3)).to(device)
    kw = {}
    if gated:
        kw = dict(branch=torch.from_numpy(rng.standard_normal((rows, width), dtype=np.float32)).to(device).to(DT[dtype]),
                  gate=(0.3 * torch.randn(2, width, device=device)).to(torch.bfloat16),
                  gate_row_map=torch.tensor([1, 0, 0, 0, 1, 1, 0, 1, 0, 0, 0, 1, 1, 1, 0, 0, 1, 1, 1, 0, 1, 0, 0],
                                            dtype=torch.int32, device=device))
        q, s, upd = fused_gated_residual_norm_hadamard_quantize(x, kw["branch"], kw["gate"], gamma, scale, shift, signs,
                                                                block, norm=norm, round_output=round_output,
                                                                gate_row_map=kw["gate_row_map"], row_map=row_map)
        oq, os_, orn = _oracle_prep(x, gamma, scale, shift, signs, block, norm=norm, round_output=round_output,
                                    row_map=row_map, **kw)
        np.testing.assert_array_equal(upd.float().cpu().numpy(), orn)
    else:
        q, s = fused_norm_hadamard_quantize(x, gamma, scale, shift, signs, block, norm=norm, round_output=round_output,
                                            row_map=row_map)
        oq, os_ = _oracle_prep(x, gamma, scale, shift, signs, block, norm=norm, round_output=round_output,
                               row_map=row_map)
    np.testing.assert_array_equal(np_of(q), oq)
    np.testing.assert_array_equal(np_of(s), os_)


def test_gated_residual_add_mixed_dtype_through_c_abi(device):
    """m5k_gated_residual_add with an F32 branch beside a BF16 residual, called directly."""
    from m5kernels_amd import _lib

    rng = np.random.default_rng(5)
    res = torch.from_numpy(rng.standard_normal((3, 256), dtype=np.float32)).to(device).to(torch.bfloat16)
    branch = torch.from_numpy(rng.standard_normal((3, 256), dtype=np.float32)).to(device)
    gate = torch.from_numpy(rng.uniform(-1, 1, 256).astype(np.float32)).to(device)
    out = torch.empty_like(res)
    _lib.call("m5k_gated_residual_add", _lib.ptr(res), _lib.BF16, 3, 256, _lib.ptr(branch), _lib.F32, _lib.ptr(gate),
              _lib.F32, None, _lib.ptr(out), _lib.stream_of(res))
    expected = ref.f32_to_bf16_bits((res.float().cpu().numpy() + branch.cpu().numpy() * gate.cpu().numpy())
                                    .astype(np.float32))
    np.testing.assert_array_equal(bits_of(out), expected)
    with pytest.raises(RuntimeError, match="branch dtype"):
        _lib.call("m5k_gated_residual_add", _lib.ptr(res), _lib.BF16, 3, 256, _lib.ptr(branch), _lib.I8,
                  _lib.ptr(gate), _lib.F32, None, _lib.ptr(out), _lib.stream_of(res))
    with pytest.raises(RuntimeError, match="gate dtype"):
        _lib.call("m5k_gated_residual_add", _lib.ptr(res), _lib.BF16, 3, 256, _lib.ptr(branch), _lib.F32,
                  _lib.ptr(gate), _lib.I32, None, _lib.ptr(out), _lib.stream_of(res))
