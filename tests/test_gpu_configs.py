"""GPU parity at the benchmark configurations, full size, against the oracle.

Every configuration the measurement names runs here at its real shape (rows sampled where the
oracle would take minutes), with the same data recipes as bench.py:

* Q projection 4096^3 online (quantize + W8A8): INT8 codes and BF16 outputs bit-exact on
  sampled rows, and the W8A8 and BF16 (torch F.linear) errors against the float64 product.
* FFN-up [4096,4096] x [16384,4096] and FFN-down [4096,16384] x [4096,16384] (0.1% outlier
  channels): INT8 bit-exact on sampled rows; FP8 within rel-L2 1e-3 of the float64 product of
  the decoded operands (the FP8 MFMA's internal sums are not IEEE FP32, so bits are not defined).
* FFN-down with the normalized block-128 Hadamard: rotate_quantize codes and scales and the
  GEMM rows bit-exact against the oracle's FP32 stage order.
* Fused gated prep (LayerNorm, H128, P = 2 tables) at M 4096 and 9914 -> W8A8 4096 x 4096:
  codes, scales and R_next bit-exact against the fixed-order FP32 oracle, then the GEMM rows.
* Q/K projection + RMSNorm + RoPE at [9914, 4096] x [4096, 4096], R = 64: head-major output
  bit-exact against the fixed-order oracle fed the oracle's own INT8 projection.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bits_of, np_of
from m5kernels_amd import (fused_gated_residual_norm_hadamard_quantize, gemm, projection_qk_rope, quantize, rotate,
                           rotate_quantize)
from oracle import reference as ref

pytestmark = pytest.mark.gpu


def _inputs(device, m, k, n, seed=29, outlier_every=None):
    g = torch.Generator(device=device).manual_seed(seed)
    a = torch.randn((m, k), generator=g, device=device)
    if outlier_every:
        a[:, ::outlier_every] *= 50.0
    w = torch.randn((n, k), generator=g, device=device) * 0.02
    return a.to(torch.bfloat16), w.to(torch.bfloat16)


def _int8_rows_bit_exact(aq, sa, wq, ws, y, rows):
    acc = ref.c_gemm_i8_acc(np_of(aq[rows]), np_of(wq))
    expected = ref.c_i8_epilogue(acc, np_of(sa[rows]), np_of(ws))
    np.testing.assert_array_equal(bits_of(y[rows]), expected)


def _codes_rows_bit_exact(a, aq, sa, rows):
    q, s = ref.quantize_reference(a[rows].float().cpu().numpy(), "int8")
    np.testing.assert_array_equal(np_of(aq[rows]), q)
    np.testing.assert_array_equal(np_of(sa[rows]), s)


def test_q_projection_4096_online(device):
    """C2: A bf16 [4096,4096] ~N(0,1), W ~N(0,0.02); online per-token INT8, offline per-channel W."""
    m = k = n = 4096
    a, w = _inputs(device, m, k, n)
    wq, ws = quantize(w, "int8")
    aq, sa = quantize(a, "int8")
    y = gemm(aq, wq, "int8", a_scales=sa, b_scales=ws, output_dtype=torch.bfloat16)
    rows = ref.sample_indices(m)
    _codes_rows_bit_exact(a, aq, sa, rows)
    _int8_rows_bit_exact(aq, sa, wq, ws, y, rows)
    exact = a[rows].double().cpu().numpy() @ w.double().cpu().numpy().T
    w8a8_err = ref.metrics(y[rows].float().cpu().numpy(), exact)["relative_l2"]
    bf16_err = ref.metrics(torch.nn.functional.linear(a, w)[rows].float().cpu().numpy(), exact)["relative_l2"]
    # The reference's quality gate for INT8 is 0.05 (engine.py); BF16 rounds only its output.
    assert w8a8_err < 0.05 and bf16_err < 0.008
    print(f"C2 rel-L2 vs float64: W8A8 {w8a8_err:.5f}, BF16 F.linear {bf16_err:.5f}")


@pytest.mark.parametrize("which", ["ffn_up", "ffn_down"])
def test_ffn_int8_online(which, device):
    """C3 INT8: FFN-up [4096,4096] x [16384,4096]; FFN-down [4096,16384] x [4096,16384] with
    every 1024th channel x50."""
    m, k, n = (4096, 4096, 16384) if which == "ffn_up" else (4096, 16384, 4096)
    a, w = _inputs(device, m, k, n, outlier_every=None if which == "ffn_up" else 1024)
    wq, ws = quantize(w, "int8")
    aq, sa = quantize(a, "int8")
    y = gemm(aq, wq, "int8", a_scales=sa, b_scales=ws, output_dtype=torch.bfloat16)
    rows = ref.sample_indices(m)
    _codes_rows_bit_exact(a, aq, sa, rows)
    _int8_rows_bit_exact(aq, sa, wq, ws, y, rows)


@pytest.mark.parametrize("which", ["ffn_up", "ffn_down"])
def test_ffn_fp8_online(which, device):
    """C3 FP8 E4M3 at full size (FFN-down: K = 16384): codes bit-exact; outputs within rel-L2
    1e-3 of the float64 product of the decoded codes (sampled rows)."""
    m, k, n = (4096, 4096, 16384) if which == "ffn_up" else (4096, 16384, 4096)
    a, w = _inputs(device, m, k, n, outlier_every=None if which == "ffn_up" else 1024)
    wq, ws = quantize(w, "fp8")
    aq, sa = quantize(a, "fp8")
    rows = ref.sample_indices(m)
    q, s = ref.quantize_reference(a[rows].float().cpu().numpy(), "fp8")
    np.testing.assert_array_equal(np_of(aq[rows]), q)
    np.testing.assert_array_equal(np_of(sa[rows]), s)
    decoded = (ref.dequantize(np_of(aq[rows]), np_of(sa[rows]), "fp8").astype(np.float64)
               @ ref.dequantize(np_of(wq), np_of(ws), "fp8").astype(np.float64).T)
    y32 = gemm(aq, wq, "fp8", a_scales=sa, b_scales=ws)
    err = ref.metrics(np_of(y32[rows]), decoded)["relative_l2"]
    assert err < 1e-3
    # BF16 output: the RNE cast of an FP32 value within 1e-3 of the float64 product, so within
    # rel-L2 1e-3 of that product's own BF16 rounding and at most one BF16 ulp from the cast of
    # the FP32 output.
    y = gemm(aq, wq, "fp8", a_scales=sa, b_scales=ws, output_dtype=torch.bfloat16)
    assert ref.metrics(y[rows].float().cpu().numpy(), ref.bf16_round_reference(decoded))["relative_l2"] < 1e-3
    ulps = np.abs(bits_of(y[rows]).astype(np.int32) - ref.f32_to_bf16_bits(np_of(y32[rows])).astype(np.int32))
    assert ulps.max() <= 1
    print(f"C3 {which} FP8 rel-L2 vs decoded float64: {err:.2e}")


def test_ffn_down_h128_rotate_quantize_gemm(device):
    """C3 Hadamard variant: W rotated (normalized block 128) offline and A online in FP32 before
    INT8; codes, scales and GEMM rows bit-exact."""
    m, k, n = 4096, 16384, 4096
    a, w = _inputs(device, m, k, n, outlier_every=1024)
    signs = torch.from_numpy(ref.hadamard_signs(k, 23)).to(device)
    wr = rotate(w, 128, signs)
    wrows = ref.sample_indices(n)
    np.testing.assert_array_equal(np_of(wr[wrows]), ref.c_hadamard_f32(np_of(w[wrows].float()), 128, np_of(signs)))
    wq, ws = quantize(wr, "int8")
    aq, sa = rotate_quantize(a, 128, signs)
    rows = ref.sample_indices(m)
    q, s = ref.quantize_reference(ref.c_hadamard_f32(np_of(a[rows].float()), 128, np_of(signs)), "int8")
    np.testing.assert_array_equal(np_of(aq[rows]), q)
    np.testing.assert_array_equal(np_of(sa[rows]), s)
    y = gemm(aq, wq, "int8", a_scales=sa, b_scales=ws, output_dtype=torch.bfloat16)
    _int8_rows_bit_exact(aq, sa, wq, ws, y, rows)


@pytest.mark.parametrize("m", [4096, 9914])
def test_gated_prep_then_w8a8_gemm(m, device):
    """C4: residual x bf16 ~N(0,1), branch ~N(0,1), per-batch shift/scale/gate bf16 ~N(0,0.1)
    (P = 2), gated residual update, LayerNorm + modulate, H128, dynamic INT8 in one kernel, then
    the W8A8 4096 x 4096 GEMM.  Bit-exact against the fixed-order oracle on sampled rows."""
    k = 4096
    g = torch.Generator(device=device).manual_seed(29)
    bf = torch.bfloat16
    res = torch.randn((m, k), generator=g, device=device).to(bf)
    branch = torch.randn((m, k), generator=g, device=device).to(bf)
    gate, scale, shift = ((torch.randn((2, k), generator=g, device=device) * 0.1).to(bf) for _ in range(3))
    gamma = (1 + 0.1 * torch.randn((k,), generator=g, device=device)).to(bf)
    row_map = (torch.arange(m, device=device, dtype=torch.int32) * 2 // m).to(torch.int32)
    signs = torch.from_numpy(ref.hadamard_signs(k, 7)).to(device)
    w = (torch.randn((k, k), generator=g, device=device) * 0.02).to(bf)
    wq, ws = quantize(w, "int8")
    q, s, r_next = fused_gated_residual_norm_hadamard_quantize(res, branch, gate, gamma, scale, shift, signs, 128,
                                                               norm="layer", gate_row_map=row_map, row_map=row_map)
    y = gemm(q, wq, "int8", a_scales=s, b_scales=ws, output_dtype=bf)
    rows = ref.sample_indices(m)
    f32 = lambda t: t.float().cpu().numpy()  # noqa: E731
    rmap = np_of(row_map[rows])
    oq, os_, orn = ref.c_prep_rows(f32(res[rows]), f32(gamma), f32(scale), f32(shift), np_of(signs), 128,
                                   dtype="bf16", norm="layer", row_map=rmap, branch=f32(branch[rows]), gate=f32(gate),
                                   gate_row_map=rmap)
    np.testing.assert_array_equal(f32(r_next[rows]), orn)
    np.testing.assert_array_equal(np_of(q[rows]), oq)
    np.testing.assert_array_equal(np_of(s[rows]), os_)
    _int8_rows_bit_exact(q, s, wq, ws, y, rows)


def test_qk_projection_rope_config(device):
    """C5: x bf16 [9914,4096] ~N(0,1), Wq ~N(0,0.02), 32 heads x 128, eps 1e-6, gamma ~1+N(0,0.02),
    RoPE base 10000 over positions 0..9913 (R = 64), INT8 online; head-major [32, 9914, 128]
    bit-exact against the fixed-order oracle on sampled rows."""
    m, k, n = 9914, 4096, 4096
    x, w = _inputs(device, m, k, n, seed=43)
    g = torch.Generator(device=device).manual_seed(44)
    gamma = (1 + 0.02 * torch.randn(128, generator=g, device=device)).to(torch.bfloat16)
    inv_freq = 10000.0 ** (-torch.arange(0, 64, dtype=torch.float64) * 2 / 128)
    angles = torch.arange(m, dtype=torch.float64)[:, None] * inv_freq[None, :]
    cos = torch.cos(angles).float().to(device).to(torch.bfloat16)
    sin = torch.sin(angles).float().to(device).to(torch.bfloat16)
    aq, sa = quantize(x, "int8")
    wq, sw = quantize(w, "int8")
    y = projection_qk_rope(aq, wq, gamma, cos, sin, "int8", a_scales=sa, b_scales=sw, epsilon=1e-6)
    rows = ref.sample_indices(m)
    z = ref.c_i8_epilogue(ref.c_gemm_i8_acc(np_of(aq[rows]), np_of(wq)), np_of(sa[rows]), np_of(sw))
    expected = ref.c_qk_norm_rope(z, bits_of(gamma), bits_of(cos[rows]), bits_of(sin[rows]),
                                  epsilon=float(np.float32(1e-6)))
    np.testing.assert_array_equal(bits_of(y[:, rows]), expected)
