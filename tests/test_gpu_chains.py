"""The gate-placement chain (gate_epilogue_chain.py:95-150 of the reference): moving the gated
residual update from the fused preparation into the previous GEMM's epilogue must keep every
BF16 boundary, so both placements give bitwise-equal R_next, INT8 codes/scales and next
projection (the reference's paired_path_parity, :134-143), and the chain's residual matches a
float64 reference of the decoded previous projection (branch rounded to BF16, FP32 gate product)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import np_of
from m5kernels_amd import gate_chain, gemm, quantize, rotate, fused_norm_hadamard_quantize
from oracle import reference as ref

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("distribution", ["normal", "outliers", "zeros"])
def test_gate_placements_bit_identical(distribution, device):
    rng = np.random.default_rng(61)
    m, pk, h, n, block = 192, 512, 768, 256, 256
    bf = torch.bfloat16

    def arr(shape, factor=1.0):
        return torch.from_numpy((rng.standard_normal(shape) * factor).astype(np.float32)).to(device).to(bf)

    x, w0, w1 = arr((m, pk)), arr((h, pk), pk**-0.5), arr((n, h), h**-0.5)
    residual, gate = arr((m, h)), arr((h,), 0.2)
    gamma, scale, shift = (1 + arr((h,), 0.1).float()).to(bf), arr((h,), 0.2), arr((h,), 0.1)
    if distribution == "outliers":
        x[:, ::127] *= 20
        residual[:, ::137] *= 20
    elif distribution == "zeros":
        x.zero_(); w0.zero_(); w1.zero_(); residual.zero_()
    s_in, s_h = torch.ones(pk, dtype=torch.int8, device=device), torch.ones(h, dtype=torch.int8, device=device)
    aq, sa = quantize(rotate(x, block, s_in), "int8")
    q0, sc0 = quantize(rotate(w0, block, s_in), "int8")
    q1, sc1 = quantize(rotate(w1, block, s_h), "int8")
    outs = {}
    for placement in ("gate-in-gemm", "gate-in-norm"):
        outs[placement] = gate_chain(aq, sa, q0, sc0, q1, sc1, residual, gate, gamma, scale, shift, s_h,
                                     placement=placement)
    (y_g, r_g), (y_n, r_n) = outs["gate-in-gemm"], outs["gate-in-norm"]
    assert torch.equal(r_g, r_n) and torch.equal(y_g, y_n)
    # Residual update against float64 of the decoded previous projection.
    branch = ref.bf16_round_f32((np_of(aq).astype(np.float64) * np_of(sa)[:, None]) @
                                (np_of(q0).astype(np.float64) * np_of(sc0)[:, None]).T)
    expected_r = ref.bf16_round_f32(residual.float().cpu().numpy().astype(np.float64) + branch * gate.float().cpu().numpy())
    assert ref.metrics(r_g.float().cpu().numpy(), expected_r)["relative_l2"] <= 0.008
    # The transition's codes also equal the ungated prep applied to the updated residual.
    qn, sn = fused_norm_hadamard_quantize(r_g, gamma, scale, shift, s_h, block)
    torch.testing.assert_close(gemm(qn, q1, "int8", a_scales=sn, b_scales=sc1, output_dtype=bf), y_g, rtol=0, atol=0)
