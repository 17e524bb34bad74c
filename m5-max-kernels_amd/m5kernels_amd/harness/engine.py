"""Experiment engine: seeded cases, bounded float64 checks, timing only when correct, and the
reference's result-record format (engine.py:19-92,420-541 of the reference).

``run_case(case, backend, precision, ...)`` prepares one case through an experiment's
``prepare`` (which returns ``fn, check, expected, original, stages, meta``), checks the output
of ``fn`` against ``expected`` (implementation gate) and ``original`` (quality gate), checks the
deployed ``online_activation_plus_gemm`` stage separately, and only then times ``fn`` and every
stage.  Status is "ok", "incorrect", "unsupported" (NotImplementedError) or "error".

Timing (``timed``) keeps the reference's synchronized host-wall samples and adds device time
from HIP events on the launch stream; both come from the same calls.
"""

from __future__ import annotations

import fcntl
import hashlib
import json
import os
import platform
import statistics
import subprocess
import tempfile
import time
from contextlib import contextmanager
from datetime import datetime, timezone
from importlib.metadata import version
from pathlib import Path

import numpy as np
import torch

from .numerics import metrics

PACKAGE = Path(__file__).resolve().parents[1]  # m5kernels_amd/

IMPLEMENTATION_LIMIT = {"fp32": 1e-4, "fp16": 1e-3}  # everything else 0.008
QUALITY_LIMIT = {"fp16": 0.001, "bf16": 0.008, "fp32": 0.0001, "int8": 0.05, "mxint8": 0.05, "fp8": 0.10}


class NumericalMismatch(ValueError):
    """A checked output failed correctness, with serializable diagnostics."""

    def __init__(self, message, **diagnostics):
        super().__init__(message)
        self.diagnostics = diagnostics


def _command(args):
    try:
        return subprocess.check_output(args, text=True, stderr=subprocess.DEVNULL, cwd=PACKAGE).strip()
    except (OSError, subprocess.CalledProcessError):
        return None


def environment():
    """Host, toolchain, device and source provenance of a result document (engine.py:35-67)."""
    digest = hashlib.sha256()
    root = PACKAGE.parent
    for folder in ("m5kernels_amd", "csrc"):
        for p in sorted((root / folder).rglob("*")):
            if p.is_file() and "__pycache__" not in p.parts and p.suffix in (".py", ".hip", ".h", ".json"):
                digest.update(str(p.relative_to(root)).encode() + p.read_bytes())
    result = dict(
        timestamp_utc=datetime.now(timezone.utc).isoformat(),
        os=platform.platform(),
        machine=platform.machine(),
        python=platform.python_version(),
        numpy=version("numpy"),
        torch=torch.__version__,
        hip=torch.version.hip,
        git_commit=_command(["git", "rev-parse", "HEAD"]),
        git_dirty=bool(_command(["git", "status", "--porcelain"])),
        source_sha256=digest.hexdigest(),
        cpu_count=len(os.sched_getaffinity(0)),
        thread_settings={k: os.environ.get(k) for k in ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS", "MAX_JOBS")},
    )
    if torch.cuda.is_available():
        p = torch.cuda.get_device_properties(0)
        result["device"] = dict(name=p.name, arch=getattr(p, "gcnArchName", None), memory_bytes=p.total_memory,
                                compute_units=p.multi_processor_count)
    else:
        result["device"] = None
    return result


def _sync():
    if torch.cuda.is_available():
        torch.cuda.synchronize()


def timed(fn, warmup, repeat):
    """Synchronized host-wall samples (the reference's measure, engine.py:70-92) plus the
    device time of the same calls from HIP events on the current stream."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    samples, device = [], []
    for _ in range(repeat):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start = time.perf_counter_ns()
        e0.record()
        fn()
        e1.record()
        torch.cuda.synchronize()
        samples.append((time.perf_counter_ns() - start) / 1e6)
        device.append(e0.elapsed_time(e1))
    return dict(
        kind="synchronized_host_wall",
        samples_ms=samples,
        median_ms=statistics.median(samples),
        p10_ms=float(np.percentile(samples, 10)),
        p90_ms=float(np.percentile(samples, 90)),
        min_ms=min(samples),
        device_samples_ms=device,
        device_median_ms=statistics.median(device),
        warmup=warmup,
        repeat=repeat,
    )


def all_finite(outputs):
    """Every floating output is finite (tuples checked element by element)."""
    if isinstance(outputs, (tuple, list)):
        return all(all_finite(o) for o in outputs)
    if not outputs.is_floating_point():
        return True
    return bool(torch.isfinite(outputs).all().item())


def working_set_bytes(c):
    """Conservative working-set estimate of a case, references and temporaries included
    (engine.py:439-451)."""
    op = c["op"]
    if op in ("gemm", "norm_hadamard_gemm", "gated_norm_hadamard_gemm", "rms_quant_gemm", "gate_epilogue_chain",
              "qk_rope"):
        est = (c["m"] * c["k"] + c["n"] * c["k"] + c["m"] * c["n"]) * 24
        if op == "gated_norm_hadamard_gemm":
            est += c["m"] * c["k"] * 16
        if op == "gate_epilogue_chain":
            est += (c["m"] + c["k"]) * c["previous_k"] * 32
        return est
    if op == "attention":
        return c["batch"] * c["heads"] * c["seq"] * c["head_dim"] * 64
    return c["m"] * c["n"] * 48


def _budget():
    """Half of the device's memory (the reference allows 32 GiB of a unified-memory Mac)."""
    if torch.cuda.is_available():
        return torch.cuda.get_device_properties(0).total_memory // 2
    return 32 * 1024**3


def run_case(c, backend, precision, seed=17, distribution="normal", warmup=3, repeat=10, tile=(64, 64, 4, 1)):
    """One checked, timed experiment record (engine.py:420-532)."""
    from . import experiments

    result = dict(case=c, backend=backend, precision=precision, seed=seed, distribution=distribution,
                  tile=list(tile))
    meta = {}
    try:
        if working_set_bytes(c) > _budget():
            raise NotImplementedError("estimated experiment working set exceeds half the device memory; split workload")
        prepare = experiments.PREPARE.get(c["op"], experiments.prepare_unsupported)
        fn, check, expected, original, stages, meta = prepare(c, backend, precision, seed, distribution, tile)
        y = fn()
        _sync()
        output_finite = all_finite(y)
        actual = check(y)
        impl = metrics(actual, expected)
        quality = metrics(actual, original)
        tolerance = IMPLEMENTATION_LIMIT.get(precision, 0.008)
        passed = output_finite and impl["finite"] and impl["relative_l2"] <= tolerance and meta.get(
            "transform_pass", True)
        quality_limit = QUALITY_LIMIT[precision]
        result.update(
            meta,
            status="ok" if passed else "incorrect",
            output_finite=output_finite,
            implementation_error=impl,
            quality_error=quality,
            implementation_relative_l2_limit=tolerance,
            quality_relative_l2_limit=quality_limit,
            quality_pass=bool(quality["finite"] and quality["relative_l2"] <= quality_limit),
        )
        # The deployed path is validated on its own, not through its prequantized counterpart.
        if "online_activation_plus_gemm" in stages:
            online_y = stages["online_activation_plus_gemm"]()
            _sync()
            online_error = metrics(check(online_y), expected)
            online_finite = all_finite(online_y)
            result["online_implementation_error"] = online_error
            result["online_output_finite"] = online_finite
            passed = passed and online_finite and online_error["finite"] and online_error["relative_l2"] <= tolerance
            result["status"] = "ok" if passed else "incorrect"
            del online_y
        # An incorrect implementation is never timed.
        if passed:
            result["timing"] = timed(fn, warmup, repeat)
            result["stages"] = {name: timed(f, warmup, repeat) for name, f in stages.items()}
            if meta.get("mac_operations"):
                result["effective_tops"] = meta["mac_operations"] / (result["timing"]["median_ms"] * 1e9)
                result["effective_device_tops"] = meta["mac_operations"] / (result["timing"]["device_median_ms"] * 1e9)
        del y, fn, stages
    except NumericalMismatch as e:
        result.update(meta)
        result.update(status="incorrect", reason=str(e), **e.diagnostics)
    except NotImplementedError as e:
        result.update(status="unsupported", reason=str(e))
    except Exception as e:  # noqa: BLE001 - every failure becomes a record, as in the reference
        result.update(status="error", reason=str(e)[:5000])
    if torch.cuda.is_available():
        torch.cuda.empty_cache()
    return result


def write_result(path, document):
    """Write a result document; never replaces an existing file (engine.py:535-541)."""
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    with path.open("x") as f:
        json.dump(document, f, indent=2, allow_nan=False)
        f.write("\n")


@contextmanager
def gpu_lock():
    """Advisory per-user lock so two harness processes never benchmark at once (locking.py:11-21)."""
    path = Path(tempfile.gettempdir()) / f"m5k-mi355x-{os.getuid()}.lock"
    with path.open("a") as handle:
        try:
            fcntl.flock(handle, fcntl.LOCK_EX | fcntl.LOCK_NB)
        except BlockingIOError:
            raise ValueError("another harness process owns the GPU experiment lock") from None
        try:
            yield
        finally:
            fcntl.flock(handle, fcntl.LOCK_UN)
