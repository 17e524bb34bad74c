"""The experiment harness end to end on the GPU: every op of the path through run_case with the
reference's gates (tests/test_engine.py, test_norm_hadamard_engine.py,
test_gated_norm_hadamard_engine.py, test_rms_quant_engine.py, test_gate_epilogue_chain.py,
test_shift_split_engine.py, test_qk_rope_experiment.py of the reference)."""

from __future__ import annotations

import json

import numpy as np
import pytest

from m5kernels_amd.harness import cli, experiments, workloads
from m5kernels_amd.harness.engine import run_case

pytestmark = pytest.mark.gpu


def _ok(r):
    assert r["status"] == "ok", {k: r.get(k) for k in ("status", "reason", "implementation_error", "transform_pass")}
    assert r["quality_pass"] and r["output_finite"]
    assert len(r["timing"]["samples_ms"]) == 3 and r["timing"]["device_median_ms"] > 0
    return r


@pytest.mark.parametrize("backend,precision", [("mlx", "bf16"), ("mpp", "bf16"), ("mpp", "fp16"), ("mpp", "fp32"),
                                               ("mpp", "int8"), ("mpp", "fp8"), ("mx-emulated", "mxint8"),
                                               ("mpp", "mxint8")])
def test_gemm_reference_and_timing(backend, precision):
    r = _ok(run_case(dict(id="test", op="gemm", m=32, n=64, k=128), backend, precision, warmup=1, repeat=3))
    if precision in ("int8", "fp8", "mxint8"):
        assert r["online_output_finite"] and r["online_implementation_error"]["relative_l2"] <= 0.008


@pytest.mark.parametrize("precision", ["int8", "fp8"])
@pytest.mark.parametrize("distribution", ["normal", "zeros", "outliers"])
def test_hadamard_gemm_harness(precision, distribution):
    case = dict(id="rotated", op="gemm", m=65, n=33, k=512,
                hadamard=dict(block_size=128, sign_seed=0, implementation="metal"))
    r = _ok(run_case(case, "mpp-hadamard", precision, distribution=distribution, warmup=1, repeat=3,
                     tile=(32, 64, 4, 8)))
    assert r["transform_pass"] and r["online_output_finite"]
    assert r["transform"]["float64_dot_preservation_error"]["relative_l2"] <= 1e-12
    assert "activation_hadamard_plus_quantization" in r["stages"]
    assert not r["weight_rotation_timed"] and not r["weight_quantization_timed"]


@pytest.mark.parametrize("norm", ["rms", "layer"])
@pytest.mark.parametrize("backend", ["norm-staged", "norm-fused"])
def test_norm_rotation_projection(norm, backend):
    case = dict(id="fused", op="norm_hadamard_gemm", m=9, n=33, k=768,
                fusion=dict(norm=norm, block_size=256, round_output="input", sign_seed=4))
    r = _ok(run_case(case, backend, "int8", distribution="outliers", warmup=1, repeat=3))
    assert r["transform_pass"] and r["online_output_finite"]
    assert r["activation_max_code_difference"] <= 1 and r["weight_max_code_difference"] <= 1
    assert r["weight_rotation_error"]["relative_l2"] < 1e-5
    assert r["stages"]["activation_prepare"]["median_ms"] > 0


@pytest.mark.parametrize("backend", ["residual-separate", "residual-fused", "mlx"])
def test_gated_projection_preserves_residual(backend):
    case = dict(id="gated", op="gated_norm_hadamard_gemm", m=7, n=33, k=768,
                fusion=dict(norm="rms", block_size=256, round_output="input"))
    r = _ok(run_case(case, backend, "bf16" if backend == "mlx" else "int8", warmup=1, repeat=3))
    assert r["online_output_finite"] and not r["residual_input_mutated"]
    if backend != "mlx":
        assert r["residual_update_exact_match"] and r["residual_update_error"]["max_abs"] == 0
        assert r["transform_pass"]


@pytest.mark.parametrize("distribution", ["normal", "outliers", "zeros"])
@pytest.mark.parametrize("backend", ["rms-direct", "rms-folded"])
@pytest.mark.parametrize("block_size", [1, 256])
def test_rms_quant_projection(backend, block_size, distribution):
    case = dict(id="rms", op="rms_quant_gemm", m=7, n=33, k=512,
                rms_quant=dict(block_size=block_size, gamma="random", sign_seed=3))
    r = _ok(run_case(case, backend, "int8", distribution=distribution, warmup=1, repeat=3))
    assert r["transform_pass"] and r["online_output_finite"]
    assert r["activation_scale_error"]["relative_l2"] <= 1e-5 and r["activation_max_code_difference"] <= 1
    assert r["stages"]["offline_weight_prepare"]["median_ms"] > 0
    if distribution == "zeros":
        assert r["quality_error"]["relative_l2"] == 0


@pytest.mark.parametrize("distribution", ["normal", "outliers", "zeros"])
@pytest.mark.parametrize("backend", ["gate-in-norm", "gate-in-gemm"])
def test_chain_rounding_and_both_outputs(distribution, backend):
    c = dict(id="chain.tail", op="gate_epilogue_chain", m=7, k=256, n=33, previous_k=768)
    r = _ok(run_case(c, backend, "int8", distribution=distribution, warmup=1, repeat=3))
    assert r["preparation_pass"] and all(chk["passed"] for chk in r["preparation_checks"].values())
    assert all(r["paired_path_parity"].values())
    assert r["online_output_finite"]


@pytest.mark.parametrize("distribution", ["normal", "outliers", "zeros"])
@pytest.mark.parametrize("bias_backend", ["mlx-fp32-convert", "mpp-bf16-to-fp32"])
def test_shift_split_projection_and_conditioning(distribution, bias_backend):
    c = dict(id="split.tail", op="norm_hadamard_gemm", m=7, n=33, k=768,
             fusion=dict(round_output="fp32", block_size=256, sign_seed=0, bias_backend=bias_backend))
    r = _ok(run_case(c, "norm-shift-split", "int8", distribution=distribution, warmup=1, repeat=3))
    assert r["shift_split"] and r["condition_prepare_timed"]
    assert r["conditioning_inclusive_implementation_error"]["relative_l2"] <= 0.008
    assert r["shift_projection_error"]["relative_l2"] <= 1e-5
    assert r["activation_scale_relative_l2_limit"] == 1e-5
    assert set(r["stages"]) == {"activation_prepare", "online_activation_plus_gemm", "condition_prepare",
                                "online_with_conditioning"}


@pytest.mark.parametrize("distribution", ["normal", "outliers", "zeros"])
@pytest.mark.parametrize("backend", ["qk-staged", "qk-fused"])
def test_qk_projection_paired_and_referenced(backend, distribution):
    c = dict(id="qk.tail", op="qk_rope", m=37, n=256, k=512, rope_half=48, epsilon=1e-6)
    r = _ok(run_case(c, backend, "int8", distribution=distribution, warmup=1, repeat=3, tile=(32, 128, 4, 1)))
    assert r["paired_path_exact"] and r["transform_pass"]
    assert r["projection_implementation_error"]["relative_l2"] <= 0.008


def test_direct_and_folded_use_identical_inputs():
    case = dict(id="rms", op="rms_quant_gemm", m=5, n=17, k=256, rms_quant=dict(block_size=256, gamma="random"))
    direct = experiments.prepare_rms_quant_gemm(case, "rms-direct", "int8", 17, "normal", (64, 64, 4, 1))
    folded = experiments.prepare_rms_quant_gemm(case, "rms-folded", "int8", 17, "normal", (64, 64, 4, 1))
    np.testing.assert_array_equal(direct[3], folded[3])
    assert direct[5]["gamma_sha256"] == folded[5]["gamma_sha256"]
    assert direct[5]["fold_scale"] is False and folded[5]["fold_scale"] is True


def test_cli_bench_smoke_suite(tmp_path, capsys):
    """The shipped smoke suite through the command line: every on-path case is ok, attention is
    recorded as unsupported, and the report renders every record."""
    out = tmp_path / "smoke.json"
    rc = cli.main(["bench", "--suite", "smoke", "--filter", "smoke.gemm", "--precisions", "bf16,int8",
                   "--backends", "mlx,mpp", "--warmup", "1", "--repeat", "3", "--output", str(out)])
    doc = json.loads(out.read_text())
    statuses = {(r["case"]["id"], r["backend"], r["precision"]): r["status"] for r in doc["results"]}
    assert rc == 0, statuses
    assert statuses[("smoke.gemm", "mpp", "int8")] == "ok" and statuses[("smoke.gemm", "mlx", "int8")] == "unsupported"
    assert doc["environment"]["device"]["arch"].startswith("gfx950")
    capsys.readouterr()
    assert cli.main(["report", str(out)]) == 0
    assert len(capsys.readouterr().out.splitlines()) == 2 + len(doc["results"])


def test_every_smoke_case_has_a_passing_backend():
    backends = {"gemm": ("mpp", "int8"), "norm_hadamard_gemm": ("norm-fused", "int8"),
                "gated_norm_hadamard_gemm": ("residual-fused", "int8"), "rms_quant_gemm": ("rms-folded", "int8"),
                "gate_epilogue_chain": ("gate-in-gemm", "int8"), "qk_rope": ("qk-fused", "int8")}
    for c in workloads.load("smoke")["cases"]:
        if c["op"] == "attention":
            assert run_case(c, "mlx", "bf16")["status"] == "unsupported"
            continue
        backend, precision = backends[c["op"]]
        if c.get("fusion", {}).get("round_output") == "fp32":
            backend = "norm-shift-split"
        tile = (32, 128, 4, 1) if c["op"] == "qk_rope" else (64, 64, 4, 1)
        _ok(run_case(c, backend, precision, warmup=1, repeat=3, tile=tile))


def test_generated_h3_fused_suite_at_128_tokens():
    """Every case of the generated h3-fused suite at M = 128 (the reference's fused workload
    files at their smallest token count) passes its gates on its fused backend."""
    backends = {"norm_hadamard_gemm": "norm-fused", "gated_norm_hadamard_gemm": "residual-fused",
                "gate_epilogue_chain": "gate-in-gemm", "qk_rope": "qk-fused"}
    cases = [c for c in workloads.load("h3-fused")["cases"] if c["m"] == 128]
    assert {c["op"] for c in cases} == set(backends)
    for c in cases:
        print(f"case {c['id']}", flush=True)
        tile = (32, 128, 4, 1) if c["op"] == "qk_rope" else (64, 64, 4, 1)
        _ok(run_case(c, backends[c["op"]], "int8", warmup=1, repeat=3, tile=tile))
