"""Profiling entry: one numerically checked workload under rocprofv3, and a dispatch-gated
summary of the trace (the reference's profile.py:29-183 and scripts/profile_report.py:37-60,
with rocprofv3 in place of Xcode GPU capture and gpudebug replay).

    # capture: the parent starts rocprofv3 as a child process, before anything touches the GPU
    python -m m5kernels_amd.harness.profile run --suite h3 --case h3.ffn_down.m4096 \\
        --backend mpp --precision int8 --online --iterations 5 --trace-dir prof/down --output prof/down.json
    # summary: per-kernel calls, durations and register/LDS/scratch use between the markers
    python -m m5kernels_amd.harness.profile summarize --trace-dir prof/down --expect-dispatches 2 \\
        --output prof/down-summary.json

The worker warms the workload up, refuses an incorrect kernel (the same gates as run_case),
then runs ``--iterations`` calls between two boundary dispatches (a short device spin) so the
summary counts exactly the profiled calls.  Without ``--trace-dir`` it only writes the
sidecar, which suits running it under a profiler command of your own.  Sidecars are marked
``not_a_benchmark_result``: profiling adds overhead.
"""

from __future__ import annotations

import argparse
import csv
import json
import os
import statistics
import subprocess
import sys
from pathlib import Path

BOUNDARY = "spin_kernel"  # torch.cuda._sleep's kernel: the capture boundary marker


def _workload(args):
    import torch

    from . import experiments
    from .cli import hadamard_overrides
    from .engine import IMPLEMENTATION_LIMIT, all_finite
    from .numerics import metrics
    from .workloads import load

    cases = [c for c in load(args.suite)["cases"] if c["id"] == args.case]
    if len(cases) != 1:
        raise ValueError("select one exact case id")
    case = hadamard_overrides(cases[0], args) if args.backend == "mpp-hadamard" else cases[0]
    prepare = experiments.PREPARE.get(case["op"], experiments.prepare_unsupported)
    fn, check, expected, original, stages, meta = prepare(case, args.backend, args.precision, args.seed, "normal",
                                                          tuple(args.tile))
    if args.online:
        if "online_activation_plus_gemm" not in stages:
            raise ValueError("online stage requires a quantized GEMM backend")
        fn = stages["online_activation_plus_gemm"]
    for _ in range(5):
        fn()
    y = fn()
    torch.cuda.synchronize()
    error = metrics(check(y), expected)
    limit = IMPLEMENTATION_LIMIT.get(args.precision, 0.008)
    if not meta.get("transform_pass", True) or not error["finite"] or error["relative_l2"] > limit or not all_finite(y):
        raise ValueError("refusing to profile an incorrect kernel")
    return fn, dict(case=case, backend=args.backend, precision=args.precision, tile=list(args.tile),
                    online=args.online, implementation_error=error, quality_error=metrics(check(y), original),
                    **{k: v for k, v in meta.items() if k not in ("sample_rows", "sample_cols", "sample_heads")})


def _run(args):
    if args.trace_dir and not args.worker:
        # Start the profiler (which starts this program again as its worker) as a child process;
        # this process has not touched the GPU and only waits for the child's status.
        if Path(args.output).exists():
            raise FileExistsError(args.output)
        worker = [sys.executable, "-u", "-m", "m5kernels_amd.harness.profile", *args.argv, "--worker"]
        cmd = ["rocprofv3", "--kernel-trace", "--stats", "-d", str(Path(args.trace_dir).resolve()), "-o", "profile",
               "--output-format", "csv", "--", *worker]
        package_root = str(Path(__file__).resolve().parents[2])
        env = dict(os.environ, TMPDIR="/tmp")
        env["PYTHONPATH"] = os.pathsep.join(p for p in (package_root, env.get("PYTHONPATH")) if p)
        return subprocess.run(cmd, check=False, env=env).returncode
    import torch

    from .engine import environment, gpu_lock, write_result

    with gpu_lock():
        fn, capture = _workload(args)
        doc = dict(schema_version=1, environment=environment(), capture=capture, iterations=args.iterations,
                   boundary_kernel=BOUNDARY, profiling_overhead=True, not_a_benchmark_result=True)
        print("M5K_READY: warmed, numerically checked workload", flush=True)
        torch.cuda.synchronize()
        torch.cuda._sleep(1000)
        for _ in range(args.iterations):
            fn()
        torch.cuda._sleep(1000)
        torch.cuda.synchronize()
        write_result(args.output, doc)
        print(json.dumps(dict(output=Path(args.output).name, iterations=args.iterations)), flush=True)
    return 0


def summarize_trace(rows, expect_dispatches=None, iterations=1):
    """Per-kernel summary of the dispatches between the first and last boundary dispatch of a
    rocprofv3 kernel trace (rows of its CSV).  `expect_dispatches` gates the dispatch count per
    iteration, like the reference's capture gate (profile_report.py:37-43)."""
    rows = sorted(rows, key=lambda r: int(r["Start_Timestamp"]))
    marks = [i for i, r in enumerate(rows) if BOUNDARY in r["Kernel_Name"]]
    if len(marks) < 2:
        raise ValueError("trace has no pair of boundary dispatches")
    inside = rows[marks[0] + 1:marks[-1]]
    if expect_dispatches is not None and len(inside) != expect_dispatches * iterations:
        raise ValueError(f"trace has {len(inside)} dispatches, expected {expect_dispatches} x {iterations}")
    kernels = {}
    for r in inside:
        name = r["Kernel_Name"]
        k = kernels.setdefault(name, dict(kernel=name, calls=0, durations_us=[],
                                          vgpr=int(r.get("VGPR_Count") or 0),
                                          agpr=int(r.get("Accum_VGPR_Count") or 0),
                                          sgpr=int(r.get("SGPR_Count") or 0),
                                          lds_bytes=int(r.get("LDS_Block_Size") or 0),
                                          scratch_bytes=int(r.get("Scratch_Size") or 0),
                                          workgroup=int(r.get("Workgroup_Size_X") or 0),
                                          grid=int(r.get("Grid_Size_X") or 0)))
        k["calls"] += 1
        k["durations_us"].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0)
    total = sum(sum(k["durations_us"]) for k in kernels.values())
    out = []
    for k in kernels.values():
        d = k.pop("durations_us")
        k.update(mean_us=statistics.fmean(d), median_us=statistics.median(d), min_us=min(d),
                 share_of_kernel_time=sum(d) / total if total else 0.0)
        out.append(k)
    out.sort(key=lambda k: -k["share_of_kernel_time"])
    return dict(dispatches=len(inside), dispatches_per_iteration=len(inside) / iterations, kernels=out)


def _summarize(args):
    from .engine import write_result

    traces = sorted(Path(args.trace_dir).rglob("*kernel_trace.csv"))
    if len(traces) != 1:
        raise ValueError(f"expected one kernel trace under {args.trace_dir}, found {len(traces)}")
    with traces[0].open() as f:
        rows = list(csv.DictReader(f))
    iterations = args.iterations
    if args.sidecar:
        iterations = json.loads(Path(args.sidecar).read_text())["iterations"]
    summary = summarize_trace(rows, args.expect_dispatches, iterations)
    summary.update(schema_version=1, iterations=iterations, source="rocprofv3 kernel trace",
                   not_a_benchmark_result=True)
    write_result(args.output, summary)
    for k in summary["kernels"]:
        print(f"{k['calls']:5d} x {k['mean_us']:10.2f} us  {100 * k['share_of_kernel_time']:5.1f}%  "
              f"vgpr {k['vgpr']:3d} agpr {k['agpr']:3d} lds {k['lds_bytes']:6d} scratch {k['scratch_bytes']}  "
              f"{k['kernel'][:90]}", flush=True)
    return 0


def parser():
    from .cli import _sign_seed

    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    sub = p.add_subparsers(dest="command", required=True)
    r = sub.add_parser("run")
    r.add_argument("--suite", default="h3")
    r.add_argument("--case", required=True)
    r.add_argument("--backend", default="mpp")
    r.add_argument("--precision", default="int8")
    r.add_argument("--tile", nargs=4, type=int, default=[64, 64, 4, 1])
    r.add_argument("--hadamard-block", type=int, default=argparse.SUPPRESS)
    r.add_argument("--hadamard-sign-seed", type=_sign_seed, default=argparse.SUPPRESS)
    r.add_argument("--hadamard-implementation", choices=["metal", "hip", "mlx"], default=argparse.SUPPRESS)
    r.add_argument("--seed", type=int, default=17)
    r.add_argument("--iterations", type=int, default=1)
    r.add_argument("--online", action="store_true")
    r.add_argument("--trace-dir", default=None, help="run under rocprofv3 --kernel-trace --stats into this folder")
    r.add_argument("--output", required=True)
    r.add_argument("--worker", action="store_true", help=argparse.SUPPRESS)
    s = sub.add_parser("summarize")
    s.add_argument("--trace-dir", required=True)
    s.add_argument("--iterations", type=int, default=1)
    s.add_argument("--sidecar", default=None, help="take the iteration count from a run sidecar")
    s.add_argument("--expect-dispatches", type=int, default=None, help="dispatches per iteration")
    s.add_argument("--output", required=True)
    return p


def main(argv=None):
    argv = list(sys.argv[1:] if argv is None else argv)
    args = parser().parse_args(argv)
    args.argv = argv
    try:
        if args.command == "summarize":
            return _summarize(args)
        if args.iterations < 1:
            raise ValueError("iterations >= 1 required")
        return _run(args)
    except (ValueError, KeyError, FileExistsError) as e:
        print(f"error: {e}", file=sys.stderr)
        return 2


if __name__ == "__main__":
    sys.exit(main())
