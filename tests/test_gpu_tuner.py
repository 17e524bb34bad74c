"""The harness tuner on the GPU: every launch it times computes the same bits, and
tune -> validate-selections runs end to end with the holdout on the next seed
(reference: src/m5kernels/cli.py:66-151, scripts/validate_selections.py:10-60)."""

import json

import pytest
import torch

from m5kernels_amd import gemm, hip
from m5kernels_amd.harness import cli

pytestmark = pytest.mark.gpu


def _codes(shape, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randint(-127, 128, shape, generator=g, device="cuda", dtype=torch.int8)


@pytest.mark.parametrize("m,n,k", [(128, 7168, 5376), (4096, 5376, 5376), (9914, 4096, 4096), (300, 1000, 2064)])
def test_every_tuner_launch_is_bit_identical_to_the_plain_launch(m, n, k):
    a, b = _codes((m, k), 1), _codes((n, k), 2)
    sa = torch.rand(m, device="cuda") * 1e-3 + 1e-4
    sb = torch.rand(n, device="cuda") * 1e-3 + 1e-4
    with hip.launch_override("plain", 1):
        ref = gemm(a, b, "int8", a_scales=sa, b_scales=sb, output_dtype=torch.bfloat16)
    space = cli.launch_space({"m": m, "n": n, "k": k}, "int8")
    assert len(space) >= 4
    for launch in space:
        with launch.active():
            out = gemm(a, b, "int8", a_scales=sa, b_scales=sb, output_dtype=torch.bfloat16)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), launch


def test_tune_then_validate_selections(tmp_path, capsys):
    seed = 5
    tuned = tmp_path / "tune.json"
    rc = cli.main(["tune", "--suite", "h3", "--filter", "attn_q.m128", "--precisions", "int8", "--seed", str(seed),
                   "--warmup", "1", "--repeat", "3", "--output", str(tuned)])
    assert rc == cli.EXIT_OK
    doc = json.loads(tuned.read_text())
    results = doc["results"]
    case = results[0]["case"]
    space = cli.launch_space(case, "int8")
    assert len(results) == len(space)
    assert all(r["status"] == "ok" and r["seed"] == seed for r in results)
    assert [cli.Launch.from_record(r["launch"]) for r in results] == space
    (sel,) = doc["selections"]
    assert sel["case_id"] == "h3.attn_q.m128"
    holdout = sel["holdout"]
    assert holdout["seed"] == seed + 1 and holdout["status"] == "ok" and holdout["quality_pass"]
    assert holdout["launch"] == sel["launch"]
    assert cli.Launch.from_record(sel["launch"]) in space
    validated = tmp_path / "validate.json"
    rc = cli.main(["validate-selections", str(tuned), "--seed", "29", "--repeat", "3", "--output", str(validated)])
    assert rc == cli.EXIT_OK
    (comparison,) = json.loads(validated.read_text())["comparisons"]
    assert comparison["launch"] == sel["launch"] and comparison["speedup"] > 0
    capsys.readouterr()
