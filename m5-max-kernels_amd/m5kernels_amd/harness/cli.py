"""Command line of the MI355X experiment harness.

It keeps the reference's command names, flags, output documents and exit codes (the
``m5bench`` commands of src/m5kernels/cli.py:153-249 and scripts/validate_selections.py), so
scripts written against the reference run unchanged:

    python -m m5kernels_amd.harness.cli doctor
    python -m m5kernels_amd.harness.cli shapes --suite h3
    python -m m5kernels_amd.harness.cli bench --suite h3 --filter ffn_down --precisions int8,fp8 \\
        --backends mlx,mpp --seed 29 --output results/down.json
    python -m m5kernels_amd.harness.cli tune --suite h3 --filter attn_q --precisions int8 --output t.json
    python -m m5kernels_amd.harness.cli report results/*.json
    python -m m5kernels_amd.harness.cli validate-selections t.json --output v.json

Exit status: 0 when every record is "ok" or "unsupported", 1 when any is "incorrect" or
"error" (tune: when no selection was made or a selection's fresh-seed holdout fails), 2 for
invalid arguments.

What differs is what ``tune`` searches.  The reference sweeps Apple threadgroup tiles; the
gfx950 kernels have their own knobs, which a ``Launch`` names: the GEMM schedule (plain
256 x 256 tiles, mixed 256 x 256 + 256 x 128 tiles, or 256 x 224 tiles) and, for the W8A8
linear, the split-K count.  Every choice computes the same bits (the tests hold them equal), so
only time decides.  ``tune`` measures the library's own plan and every applicable alternative
on the tuning seed, keeps the fastest correct one, and re-measures it on a fresh seed (the
holdout); ``validate-selections`` re-runs each selected launch beside the framework's BF16
baseline.  ``--tile`` is still validated and recorded as the reference records it.
"""

from __future__ import annotations

import argparse
import json
import sys
from dataclasses import dataclass
from pathlib import Path

from .workloads import load

EXIT_OK, EXIT_FAILED, EXIT_USAGE = 0, 1, 2
_FAILED_STATUSES = ("error", "incorrect")
_DISTRIBUTIONS = ("normal", "outliers", "zeros")


# ---- gfx950 launch knobs -------------------------------------------------------------------


@dataclass(frozen=True)
class Launch:
    """One gfx950 GEMM launch choice; None fields keep the library's plan."""

    schedule: str | None = None  # "plain" | "mixed" | "narrow" | "quad"
    splits: int | None = None  # W8A8 split-K count (1 = no split)

    def record(self):
        return {"schedule": self.schedule or "auto", "splits": self.splits or "auto"}

    @classmethod
    def from_record(cls, rec):
        if not rec:
            return cls()
        schedule, splits = rec.get("schedule", "auto"), rec.get("splits", "auto")
        return cls(None if schedule == "auto" else schedule, None if splits == "auto" else int(splits))

    def active(self):
        from ..hip import launch_override

        return launch_override(self.schedule, self.splits)


def launch_space(case, precision, cus=256):
    """The library's plan first, then every forced alternative that applies to the case."""
    from ..hip import splitk_plan

    space = [Launch(), Launch("plain"), Launch("mixed")]
    if precision in ("int8", "bf16", "fp16", "mxint8"):
        space.append(Launch("narrow"))  # 256 x 224 tiles exist for the 16 x 16 MFMA modes
    if precision == "int8":
        space.append(Launch("quad"))  # four waves of 128 x 128, W8A8 only
    if precision == "int8" and case.get("k", 0) % 16 == 0:
        m, n, k = case["m"], case["n"], case["k"]
        planned = splitk_plan(m, n, k, cus)
        for splits in sorted({2, 4, 8, planned, 2 * planned} - {1}):
            if splits <= min(64, -(-k // 128)):
                space.append(Launch("plain", splits))
    unique = []
    for launch in space:
        if launch not in unique:
            unique.append(launch)
    return unique


# ---- result documents ------------------------------------------------------------------------


class _Document:
    """An output document that refuses to replace an existing file, collects records and
    prints one status line per record."""

    def __init__(self, output, **fields):
        if Path(output).exists():
            raise FileExistsError(output)
        from .engine import environment

        self.output = output
        self.body = dict(schema_version=1, environment=environment(), **fields)

    def record(self, result, *label):
        self.body.setdefault("results", []).append(result)
        timing = result.get("timing") or {}
        detail = f"{timing['median_ms']:.3f} ms" if "median_ms" in timing else result.get("reason", "")
        print(*label, result["status"], detail, flush=True)
        return result

    def failed(self):
        return any(r["status"] in _FAILED_STATUSES for r in self.body.get("results", []))

    def save(self):
        from .engine import write_result

        write_result(self.output, self.body)


def _accepted(result):
    return result["status"] == "ok" and result.get("quality_pass", False)


def online_ms(result):
    """The deployed time of a record: the online activation + GEMM stage where there is one."""
    stage = result.get("stages", {}).get("online_activation_plus_gemm")
    return (stage or result["timing"])["median_ms"]


def hadamard_overrides(case, args):
    """The case with the --hadamard-* options folded into its Hadamard configuration."""
    options = {"hadamard_block": "block_size", "hadamard_sign_seed": "sign_seed",
               "hadamard_implementation": "implementation"}
    config = dict(case.get("hadamard", {}))
    config.update({key: getattr(args, opt) for opt, key in options.items() if hasattr(args, opt)})
    return {**case, "hadamard": config}


def _selected_cases(args, gemm_only=False):
    cases = [c for c in load(args.suite)["cases"] if args.filter in c["id"] and (not gemm_only or c["op"] == "gemm")]
    if not cases:
        raise ValueError("no GEMM cases matched" if gemm_only else "no cases matched")
    return cases


def _measure(case, backend, precision, args, seed, tile, launch=Launch(), warmup=None):
    from .engine import run_case

    with launch.active():
        result = run_case(case, backend, precision, seed, args.distribution, args.warmup if warmup is None else warmup,
                          args.repeat, tile)
    result["launch"] = launch.record()
    return result


# ---- commands --------------------------------------------------------------------------------


def cmd_bench(args):
    cases = _selected_cases(args)
    doc = _Document(args.output, suite=args.suite, results=[])
    for case in cases:
        tile = (256, 1, 1, 1) if case["op"] == "rms_modulate" else tuple(args.tile)
        for precision in args.precisions.split(","):
            for backend in args.backends.split(","):
                job = hadamard_overrides(case, args) if backend == "mpp-hadamard" else case
                doc.record(_measure(job, backend, precision, args, args.seed, tile), case["id"], backend, precision)
    doc.save()
    return EXIT_FAILED if doc.failed() else EXIT_OK


def cmd_tune(args):
    cases = _selected_cases(args, gemm_only=True)
    doc = _Document(args.output, suite=args.suite, results=[], selections=[])
    backend, tile = args.tune_backend, tuple(args.tile)
    for case in cases:
        job = hadamard_overrides(case, args) if backend == "mpp-hadamard" else case
        for precision in args.precisions.split(","):
            trials = []
            for launch in launch_space(job, precision):
                result = doc.record(_measure(job, backend, precision, args, args.seed, tile, launch), case["id"],
                                    precision, launch.record())
                if _accepted(result):
                    trials.append((online_ms(result), launch))
            if not trials:
                continue
            _, best = min(trials, key=lambda t: t[0])
            # The choice was made on the tuning seed; the holdout re-measures it on the next seed.
            holdout = _measure(job, backend, precision, args, args.seed + 1, tile, best)
            doc.body["selections"].append(dict(case_id=case["id"], backend=backend, precision=precision,
                                               tile=list(tile), launch=best.record(), holdout=holdout))
            print(case["id"], precision, "selected", best.record(), "holdout", holdout["status"], flush=True)
    doc.save()
    selections = doc.body["selections"]
    return EXIT_OK if selections and all(_accepted(s["holdout"]) for s in selections) else EXIT_FAILED


def cmd_validate_selections(args):
    """Each selection against a fresh framework BF16 baseline, the pair run back to back."""
    if args.repeat < 3:
        raise ValueError("at least 3 repeats required")
    doc = _Document(args.output, results=[], comparisons=[])
    for path in args.inputs:
        for sel in json.loads(Path(path).read_text())["selections"]:
            case = sel["holdout"]["case"]
            launch = Launch.from_record(sel.get("launch"))
            baseline = doc.record(_measure(case, "mlx", "bf16", args, args.seed, (64, 64, 4, 1), warmup=5),
                                  case["id"], "mlx", "bf16")
            candidate = doc.record(_measure(case, sel.get("backend", "mpp"), sel["precision"], args, args.seed,
                                            tuple(sel["tile"]), launch, warmup=5),
                                   case["id"], sel.get("backend", "mpp"), sel["precision"])
            entry = dict(case_id=case["id"], precision=sel["precision"], tile=sel["tile"], launch=launch.record(),
                         selection_record=Path(path).name)
            if _accepted(baseline) and _accepted(candidate):
                base_ms, cand_ms = baseline["timing"]["median_ms"], online_ms(candidate)
                entry.update(baseline_ms=base_ms, candidate_ms=cand_ms, speedup=base_ms / cand_ms)
            doc.body["comparisons"].append(entry)
            print(json.dumps(entry), flush=True)
    doc.save()
    return EXIT_FAILED if doc.failed() else EXIT_OK


def _fmt(value, spec):
    return "—" if value is None else format(value, spec)


def _rotation(r):
    t = r.get("transform") or {}
    if "implementation" in t and "sign_seed" in t:
        return f"H{t['block_size']} / {t['implementation']} / signs={t['sign_seed']}"
    return "—"


# Report columns: (header, right-aligned, cell of a record).
REPORT_COLUMNS = [
    ("Case", False, lambda r: r["case"]["id"]),
    ("Backend", False, lambda r: r["backend"]),
    ("Precision", False, lambda r: r["precision"]),
    ("Rotation", False, _rotation),
    ("Compute ms", True, lambda r: _fmt((r.get("timing") or {}).get("median_ms"), ".4f")),
    ("Online ms", True,
     lambda r: _fmt(((r.get("stages") or {}).get("online_activation_plus_gemm") or {}).get("median_ms"), ".4f")),
    ("Compute TOPS", True, lambda r: _fmt(r.get("effective_tops"), ".2f")),
    ("Relative L2", True, lambda r: _fmt((r.get("quality_error") or {}).get("relative_l2"), ".5f")),
    ("Quality gate", False, lambda r: ("pass" if r["quality_pass"] else "reject") if "quality_pass" in r else "—"),
    ("Status", False, lambda r: r["status"]),
]


def report_lines(docs):
    """Markdown table of every record in the result documents."""
    lines = ["| " + " | ".join(h for h, _, _ in REPORT_COLUMNS) + " |",
             "|" + "|".join("---:" if right else "---" for _, right, _ in REPORT_COLUMNS) + "|"]
    lines += ["| " + " | ".join(cell(r) for _, _, cell in REPORT_COLUMNS) + " |"
              for doc in docs for r in doc["results"]]
    return lines


def cmd_report(args):
    print("\n".join(report_lines([json.loads(Path(p).read_text()) for p in args.inputs])))
    return EXIT_OK


def cmd_doctor(args):
    from .engine import environment

    print(json.dumps(environment(), indent=2))
    return EXIT_OK


def cmd_shapes(args):
    print(json.dumps(load(args.suite), indent=2))
    return EXIT_OK


# ---- arguments -------------------------------------------------------------------------------


def _sign_seed(value):
    return None if value == "none" else int(value)


def _experiment_options(sub, default_suite, tune):
    sub.add_argument("--suite", default=default_suite)
    sub.add_argument("--filter", default="")
    sub.add_argument("--precisions", default="bf16")
    sub.add_argument("--backends", default="mlx,mpp")
    sub.add_argument("--tile", type=int, nargs=4, default=[64, 64, 4, 1], metavar=("M", "N", "SIMDGROUPS", "M_GROUP"))
    sub.add_argument("--hadamard-block", type=int, default=argparse.SUPPRESS)
    sub.add_argument("--hadamard-sign-seed", type=_sign_seed, default=argparse.SUPPRESS)
    sub.add_argument("--hadamard-implementation", choices=["metal", "hip", "mlx"], default=argparse.SUPPRESS)
    if tune:
        sub.add_argument("--tune-backend", choices=["mpp", "mpp-hadamard"], default="mpp")
    sub.add_argument("--seed", type=int, default=17)
    sub.add_argument("--distribution", choices=_DISTRIBUTIONS, default="normal")
    sub.add_argument("--warmup", type=int, default=3)
    sub.add_argument("--repeat", type=int, default=10)
    sub.add_argument("--output", required=True)


def parser():
    p = argparse.ArgumentParser(description="MI355X quantized-projection accuracy and kernel benchmark harness")
    sub = p.add_subparsers(dest="command", required=True)
    sub.add_parser("doctor").set_defaults(run=cmd_doctor, locked=False)
    shapes = sub.add_parser("shapes")
    shapes.add_argument("--suite", default="h3")
    shapes.set_defaults(run=cmd_shapes, locked=False)
    bench = sub.add_parser("bench")
    _experiment_options(bench, "smoke", tune=False)
    bench.set_defaults(run=cmd_bench, locked=True, experiment=True)
    tune = sub.add_parser("tune")
    _experiment_options(tune, "h3", tune=True)
    tune.set_defaults(run=cmd_tune, locked=True, experiment=True)
    report = sub.add_parser("report")
    report.add_argument("inputs", nargs="+")
    report.set_defaults(run=cmd_report, locked=False)
    val = sub.add_parser("validate-selections")
    val.add_argument("inputs", nargs="+")
    val.add_argument("--seed", type=int, default=29)
    val.add_argument("--repeat", type=int, default=20)
    val.add_argument("--distribution", choices=_DISTRIBUTIONS, default="normal")
    val.add_argument("--output", required=True)
    val.set_defaults(run=cmd_validate_selections, locked=True)
    return p


def _check_experiment_args(args):
    if args.warmup < 1 or args.repeat < 3:
        raise ValueError("warmup >=1 and repeat >=3 required")
    if any(v <= 0 for v in args.tile) or args.tile[2] > 32:
        raise ValueError("invalid tile")


def main(argv=None):
    args = parser().parse_args(argv)
    try:
        if getattr(args, "experiment", False):
            _check_experiment_args(args)
        if not args.locked:
            return args.run(args)
        from .engine import gpu_lock

        with gpu_lock():
            return args.run(args)
    except (ValueError, KeyError, FileExistsError) as e:
        print(f"error: {e}", file=sys.stderr)
        return EXIT_USAGE


if __name__ == "__main__":
    sys.exit(main())
