"""CPU tests of the experiment harness: workload schema, the harness's float64 check numerics
against the pinned oracle, config validation, record gating and the CLI's argument handling.
Nothing here touches a GPU (unsupported/invalid cases are rejected before device work)."""

from __future__ import annotations

import json

import numpy as np
import pytest

from m5kernels_amd.harness import cli, engine, experiments, workloads
from m5kernels_amd.harness import numerics as nx
from oracle import reference as ref


# ---- workloads (workloads.py:9-37) -------------------------------------------------------------


def test_validate_rejects_bad_cases():
    with pytest.raises(ValueError, match="nonempty id"):
        workloads.validate({"id": "", "op": "gemm", "m": 1, "n": 1, "k": 1})
    with pytest.raises(ValueError, match="k must be a positive integer"):
        workloads.validate({"id": "a", "op": "gemm", "m": 1, "n": 1, "k": 0})
    with pytest.raises(ValueError, match="previous_k"):
        workloads.validate({"id": "a", "op": "gate_epilogue_chain", "m": 1, "n": 1, "k": 1, "previous_k": 1.5})
    with pytest.raises(KeyError):
        workloads.validate({"id": "a", "op": "conv", "m": 1})


def test_load_suites_and_duplicates(tmp_path):
    smoke = workloads.load("smoke")
    assert {c["op"] for c in smoke["cases"]} >= {"gemm", "norm_hadamard_gemm", "gated_norm_hadamard_gemm",
                                                 "rms_quant_gemm", "gate_epilogue_chain", "qk_rope"}
    h3 = workloads.load("h3")["cases"]
    assert len(h3) == 55
    down = next(c for c in h3 if c["id"] == "h3.ffn_down.m4096")
    assert (down["m"], down["n"], down["k"]) == (4096, 5376, 14336)
    fused = {c["id"]: c for c in workloads.load("h3-fused")["cases"]}
    assert len(fused) == 29
    assert sum(c["op"] == "rms_quant_gemm" for c in fused.values()) == 6
    assert "h3.shift_q.m128" not in fused and "rms.plain.m128" not in fused
    chain = fused["h3.chain_attention_to_ffn.m4096"]
    assert (chain["k"], chain["n"], chain["previous_k"], chain["previous_tile"]) == (5376, 14336, 7168, [128, 64, 4, 8])
    assert fused["h3.shift_q.m9914"]["fusion"] == dict(norm="rms", block_size=256, round_output="fp32", threads=256)
    assert fused["rms.weighted_h256.m4096"]["rms_quant"]["block_size"] == 256
    assert (fused["h3.qk_rope.m9914"]["n"], fused["h3.qk_rope.m9914"]["rope_half"]) == (7168, 48)
    p = tmp_path / "dup.json"
    p.write_text(json.dumps({"cases": [{"id": "x", "op": "gemm", "m": 1, "n": 1, "k": 1}] * 2}))
    with pytest.raises(ValueError, match="duplicate"):
        workloads.load(str(p))


# ---- harness numerics against the pinned oracle -------------------------------------------------


def test_metrics_and_sampling_match_oracle():
    rng = np.random.default_rng(1)
    a, r = rng.normal(size=(5, 7)), rng.normal(size=(5, 7))
    assert nx.metrics(a, r) == ref.metrics(a, r)
    assert nx.metrics(np.zeros(3), np.zeros(3))["cosine"] == 1.0
    assert not nx.metrics([np.nan], [1.0])["finite"]
    for n in (1, 7, 32, 33, 4096, 9914):
        np.testing.assert_array_equal(nx.sample_indices(n), ref.sample_indices(n))


@pytest.mark.parametrize("block", [1, 32, 128, 256])
def test_block_hadamard_matches_oracle(block):
    rng = np.random.default_rng(block)
    x = rng.normal(size=(6, 1024))
    signs = ref.hadamard_signs(1024, 7)
    np.testing.assert_array_equal(nx.hadamard_signs(1024, 7), signs)
    expected = x * signs if block == 1 else ref.block_hadamard_reference(x, block, signs)
    np.testing.assert_allclose(nx.block_hadamard(x, block, signs), expected, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("norm", ["rms", "layer"])
def test_norm_modulate_matches_oracle(norm):
    rng = np.random.default_rng(3)
    x, g, s, b = rng.normal(size=(4, 64)), rng.normal(size=64), rng.normal(size=64), rng.normal(size=64)
    np.testing.assert_allclose(nx.norm_modulate(x, g, s, b, norm=norm), ref.norm_modulate_reference(x, g, s, b, norm=norm),
                               rtol=1e-12, atol=1e-12)


def test_bf16_round_and_dequantize_match_oracle():
    rng = np.random.default_rng(4)
    v = np.concatenate([rng.normal(size=1000) * 10.0 ** rng.integers(-30, 30, 1000), [0.0, -0.0, 1 + 2**-8]])
    np.testing.assert_array_equal(nx.bf16_round(v), ref.bf16_round_reference(v))
    codes = np.arange(256, dtype=np.uint8)
    finite = ~np.isnan(ref.fp8_decode(codes))
    np.testing.assert_array_equal(nx.fp8_decode(codes)[finite], ref.fp8_decode(codes)[finite].astype(np.float64))
    q = rng.integers(-127, 128, size=(3, 64)).astype(np.int8)
    e = rng.integers(100, 150, size=(3, 2)).astype(np.uint8)
    np.testing.assert_array_equal(nx.dequantize(q, e, "mxint8"), ref.dequantize(q, e, "mxint8"))
    s = rng.random(3).astype(np.float32)
    np.testing.assert_allclose(nx.dequantize(q, s, "int8"), ref.dequantize(q, s, "int8"), rtol=1e-7)


def test_qk_rope_and_rms_match_oracle():
    rng = np.random.default_rng(5)
    proj = rng.normal(size=(5, 3, 128))
    gamma, cos, sin = rng.normal(size=128), rng.normal(size=(5, 48)), rng.normal(size=(5, 48))
    np.testing.assert_allclose(nx.qk_rope(proj, gamma, cos, sin, epsilon=1e-6),
                               ref.qk_rope_reference(proj, gamma, cos, sin, epsilon=1e-6)["output"], rtol=0, atol=0)
    x, g = rng.normal(size=(4, 512)), rng.normal(size=512)
    signs = ref.hadamard_signs(512, 2)
    mine, theirs = nx.rms_quantize(x, g, signs, 256), ref.rms_quantize_reference(x, g, signs, 256)
    np.testing.assert_array_equal(mine["quantized"], theirs["quantized"])
    np.testing.assert_allclose(mine["scales"], theirs["scales"], rtol=1e-12)
    np.testing.assert_allclose(mine["normalized_rotated"], theirs["normalized_rotated"], rtol=1e-12, atol=1e-12)


# ---- validation before device work ---------------------------------------------------------------


def _rms_case(**extra):
    return dict(id="r", op="rms_quant_gemm", m=3, n=17, k=256, **extra)


def test_rms_config_validation():
    with pytest.raises(NotImplementedError, match="rms-direct/rms-folded"):
        experiments.validate_rms_config(_rms_case(), "mpp", "int8", "normal")
    with pytest.raises(NotImplementedError, match="block_size 1 or 256"):
        experiments.validate_rms_config(_rms_case(rms_quant={"block_size": 128}), "rms-direct", "int8", "normal")
    with pytest.raises(NotImplementedError, match="unsupported rms_quant options"):
        experiments.validate_rms_config(_rms_case(rms_quant={"norm": "layer"}), "rms-direct", "int8", "normal")
    with pytest.raises(NotImplementedError, match="semantics options"):
        experiments.validate_rms_config(_rms_case(shift=1), "rms-direct", "int8", "normal")
    with pytest.raises(ValueError, match="epsilon"):
        experiments.validate_rms_config(_rms_case(rms_quant={"epsilon": 1e-50}), "rms-folded", "int8", "normal")
    cfg = experiments.validate_rms_config(_rms_case(rms_quant={"block_size": 256, "gamma": "random"}), "rms-folded",
                                          "int8", "outliers")
    assert cfg["block_size"] == 256 and cfg["threads"] == 256 and cfg["sign_seed"] is None


def test_qk_config_validation():
    c = dict(id="q", op="qk_rope", m=4, n=256, k=512)
    assert experiments.validate_qk_config(c, "qk-fused", "int8", "normal", (32, 128, 4, 1))["rope_half"] == 48
    with pytest.raises(NotImplementedError, match="complete 128-wide heads"):
        experiments.validate_qk_config(dict(c, n=200), "qk-fused", "int8", "normal", (32, 128, 4, 1))
    with pytest.raises(NotImplementedError, match="H256"):
        experiments.validate_qk_config(dict(c, k=384), "qk-staged", "int8", "normal", (32, 128, 4, 1))
    with pytest.raises(ValueError, match="rope_half"):
        experiments.validate_qk_config(dict(c, rope_half=65), "qk-staged", "int8", "normal", (32, 128, 4, 1))
    with pytest.raises(NotImplementedError, match="Q/K tile"):
        experiments.validate_qk_config(c, "qk-staged", "int8", "normal", (64, 64, 2, 1))


@pytest.mark.parametrize("fusion,reason", [({}, "round_output=fp32"),
                                           ({"norm": "layer", "round_output": "fp32"}, "round_output=fp32"),
                                           ({"round_output": "fp32", "passes": "two_read"}, "passes=one_read"),
                                           ({"round_output": "fp32", "bias_backend": "numpy"}, "bias preparation")])
def test_shift_split_rejections_are_unsupported_records(fusion, reason):
    """test_shift_split_engine.py:40-61: incompatible contracts are rejected as unsupported."""
    c = dict(id="split.reject", op="norm_hadamard_gemm", m=3, n=17, k=256, fusion=fusion)
    r = engine.run_case(c, "norm-shift-split", "int8", warmup=1, repeat=3)
    assert r["status"] == "unsupported" and reason in r["reason"]


def test_out_of_scope_ops_are_unsupported():
    for c in workloads.load("h3")["cases"]:
        if c["op"] in ("attention", "rms_modulate", "swiglu"):
            r = engine.run_case(c, "mlx", "bf16")
            assert r["status"] == "unsupported" and "outside" in r["reason"]


def _fake_prepare(passing_transform, actual_offset):
    """A host-only experiment whose output misses `expected` by `actual_offset`."""
    import torch

    def prepare(c, backend, precision, seed, distribution, tile):
        expected = np.ones((2, 2))
        stages = {"online_activation_plus_gemm": lambda: torch.ones((2, 2), dtype=torch.float64)}
        meta = dict(transform_pass=passing_transform, mac_operations=8)
        return (lambda: torch.full((2, 2), 1.0 + actual_offset, dtype=torch.float64)), (lambda y: y.numpy()), \
            expected, expected, stages, meta

    return prepare


@pytest.mark.parametrize("transform,offset", [(False, 0.0), (True, 0.5)])
def test_incorrect_records_are_never_timed(monkeypatch, transform, offset):
    monkeypatch.setitem(experiments.PREPARE, "gemm", _fake_prepare(transform, offset))
    r = engine.run_case(dict(id="g", op="gemm", m=2, n=2, k=2), "mpp", "int8")
    assert r["status"] == "incorrect"
    assert "timing" not in r and "stages" not in r and "effective_tops" not in r


# ---- CLI and report -------------------------------------------------------------------------------


def test_cli_rejects_bad_arguments(capsys):
    assert cli.main(["bench", "--output", "x.json", "--warmup", "0"]) == 2
    assert cli.main(["bench", "--output", "x.json", "--tile", "64", "64", "40", "1"]) == 2
    assert "error:" in capsys.readouterr().err
    with pytest.raises(SystemExit):
        cli.main(["tune"])  # --output is required


def test_cli_shapes_prints_suite(capsys):
    assert cli.main(["shapes", "--suite", "smoke"]) == 0
    assert json.loads(capsys.readouterr().out)["cases"][0]["id"] == "smoke.gemm"


def test_report_table(tmp_path, capsys):
    doc = {"results": [
        {"case": {"id": "a"}, "backend": "mpp", "precision": "int8", "status": "ok", "quality_pass": True,
         "timing": {"median_ms": 1.5}, "stages": {"online_activation_plus_gemm": {"median_ms": 1.75}},
         "effective_tops": 12.345, "quality_error": {"relative_l2": 0.01234},
         "transform": {"block_size": 256, "implementation": "metal", "sign_seed": None}},
        {"case": {"id": "b"}, "backend": "mlx", "precision": "bf16", "status": "unsupported", "reason": "x"},
    ]}
    p = tmp_path / "r.json"
    p.write_text(json.dumps(doc))
    assert cli.main(["report", str(p)]) == 0
    out = capsys.readouterr().out.splitlines()
    assert out[2] == "| a | mpp | int8 | H256 / metal / signs=None | 1.5000 | 1.7500 | 12.35 | 0.01234 | pass | ok |"
    assert out[3] == "| b | mlx | bf16 | — | — | — | — | — | — | unsupported |"


def test_tune_launch_space():
    """The tuner's candidates are gfx950 launches: the library's plan, each forced schedule
    (narrow only for the 16 x 16 MFMA modes) and, for INT8, split-K counts."""
    case = {"id": "c", "op": "gemm", "m": 128, "n": 4096, "k": 16384}
    int8 = cli.launch_space(case, "int8")
    assert int8[0] == cli.Launch() and cli.Launch("narrow") in int8 and cli.Launch("quad") in int8
    splits = sorted(l.splits for l in int8 if l.splits)
    assert splits and all(2 <= s <= 64 for s in splits)
    fp8 = cli.launch_space(case, "fp8")
    assert cli.Launch("narrow") not in fp8 and cli.Launch("quad") not in fp8 and not any(l.splits for l in fp8)
    assert len(set(int8)) == len(int8)
    for launch in int8:
        assert cli.Launch.from_record(launch.record()) == launch


def test_launch_override_sets_and_restores():
    from m5kernels_amd import hip

    with hip.launch_override("narrow", 4):
        assert hip._override.schedule == "narrow" and hip._override.splits == 4
        with hip.launch_override(None, None):
            assert hip._override.schedule == "narrow" and hip._override.splits is None
        assert hip._override.splits == 4
    assert getattr(hip._override, "schedule", None) is None and hip._override.splits is None
    with pytest.raises(ValueError):
        with hip.launch_override("diagonal"):
            pass
    with pytest.raises(ValueError):
        with hip.launch_override(splits=0):
            pass


def _fake_run_case(times, calls):
    """A stand-in for engine.run_case: records the call and the launch in force, and times
    each launch by `times` (None: incorrect)."""
    from m5kernels_amd import hip

    def run_case(c, backend, precision, seed=17, distribution="normal", warmup=3, repeat=10, tile=(64, 64, 4, 1)):
        launch = cli.Launch(getattr(hip._override, "schedule", None), getattr(hip._override, "splits", None))
        calls.append((c["id"], backend, precision, seed, launch))
        ms = times.get(launch, 1.0) if backend != "mlx" else 2.0
        if ms is None:
            return dict(case=c, backend=backend, precision=precision, status="incorrect", tile=list(tile))
        return dict(case=c, backend=backend, precision=precision, status="ok", quality_pass=True, tile=list(tile),
                    timing={"median_ms": ms}, stages={"online_activation_plus_gemm": {"median_ms": ms + 0.1}})
    return run_case


def test_tune_selects_fastest_launch_then_holdout_on_fresh_seed(tmp_path, monkeypatch):
    times = {cli.Launch(): 1.0, cli.Launch("mixed"): 0.8, cli.Launch("plain"): None}
    calls = []
    monkeypatch.setattr(engine, "run_case", _fake_run_case(times, calls))
    monkeypatch.setattr(engine, "environment", lambda: {})
    out = tmp_path / "t.json"
    rc = cli.main(["tune", "--suite", "h3", "--filter", "attn_q.m128", "--precisions", "int8", "--seed", "5",
                   "--output", str(out)])
    assert rc == 0
    doc = json.loads(out.read_text())
    sel = doc["selections"]
    assert len(sel) == 1 and sel[0]["launch"] == {"schedule": "mixed", "splits": "auto"}
    assert sel[0]["holdout"]["launch"] == sel[0]["launch"]
    tuning = [c for c in calls if c[3] == 5]
    holdout = [c for c in calls if c[3] == 6]
    assert len(tuning) == len(cli.launch_space(doc["results"][0]["case"], "int8"))
    assert holdout == [(sel[0]["case_id"], "mpp", "int8", 6, cli.Launch("mixed"))]
    assert all("launch" in r for r in doc["results"])
    # validate-selections re-runs the selected launch beside the BF16 framework baseline.
    calls.clear()
    out2 = tmp_path / "v.json"
    assert cli.main(["validate-selections", str(out), "--seed", "29", "--output", str(out2)]) == 0
    assert [c[1:] for c in calls] == [("mlx", "bf16", 29, cli.Launch()), ("mpp", "int8", 29, cli.Launch("mixed"))]
    comparison = json.loads(out2.read_text())["comparisons"][0]
    assert comparison["speedup"] == pytest.approx(2.0 / 0.9)


def test_tune_fails_without_a_correct_launch(tmp_path, monkeypatch):
    calls = []
    monkeypatch.setattr(engine, "run_case", _fake_run_case({l: None for l in cli.launch_space(
        {"m": 128, "n": 7168, "k": 5376}, "int8")}, calls))
    monkeypatch.setattr(engine, "environment", lambda: {})
    out = tmp_path / "t.json"
    assert cli.main(["tune", "--suite", "h3", "--filter", "attn_q.m128", "--precisions", "int8",
                     "--output", str(out)]) == 1
    assert json.loads(out.read_text())["selections"] == []


def test_write_result_never_replaces(tmp_path):
    p = tmp_path / "out.json"
    engine.write_result(p, {"a": 1})
    with pytest.raises(FileExistsError):
        engine.write_result(p, {"a": 2})
    assert json.loads(p.read_text()) == {"a": 1}


# ---- profiling summary (profile_report.py:37-60) ------------------------------------------------


def _trace_rows(names_durations):
    rows, t = [], 1000
    for i, (name, dur) in enumerate(names_durations):
        rows.append(dict(Kernel_Name=name, Start_Timestamp=str(t), End_Timestamp=str(t + dur), VGPR_Count="128",
                         Accum_VGPR_Count="0", SGPR_Count="32", LDS_Block_Size="131072", Scratch_Size="0",
                         Workgroup_Size_X="512", Grid_Size_X="131072", Dispatch_Id=str(i)))
        t += dur + 10
    return rows


def test_profile_summary_counts_only_the_marked_calls():
    from m5kernels_amd.harness import profile

    spin = "void at::cuda::(anonymous namespace)::spin_kernel(long)"
    rows = _trace_rows([("warmup_kernel", 5000), (spin, 100)] + [("quant", 2000), ("gemm", 8000)] * 3
                       + [(spin, 100), ("after", 7)])
    s = profile.summarize_trace(list(reversed(rows)), expect_dispatches=2, iterations=3)
    assert s["dispatches"] == 6 and s["dispatches_per_iteration"] == 2
    names = [k["kernel"] for k in s["kernels"]]
    assert names == ["gemm", "quant"]
    gemm = s["kernels"][0]
    assert gemm["calls"] == 3 and gemm["mean_us"] == 8.0 and gemm["lds_bytes"] == 131072
    assert abs(gemm["share_of_kernel_time"] - 0.8) < 1e-12
    with pytest.raises(ValueError, match="expected 3 x 3"):
        profile.summarize_trace(rows, expect_dispatches=3, iterations=3)
    with pytest.raises(ValueError, match="boundary"):
        profile.summarize_trace(rows[2:-2])


def test_profile_cli_rejects_bad_arguments(capsys):
    from m5kernels_amd.harness import profile

    assert profile.main(["run", "--case", "x", "--iterations", "0", "--output", "o.json"]) == 2
    with pytest.raises(SystemExit):
        profile.main(["summarize"])
