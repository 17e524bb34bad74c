"""bench.py's command line on the CPU: it compiles, lists its options, and refuses more than one
GPU with the documented message and exit status (no GPU is touched on these paths)."""

from __future__ import annotations

import py_compile
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def test_bench_compiles():
    py_compile.compile(str(ROOT / "bench.py"), doraise=True)


def test_bench_help_lists_options():
    out = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--help"], capture_output=True, text=True,
                         timeout=120, check=True).stdout
    for opt in ("--gpus", "--steps", "--warmup", "--op-settle", "--vs-hipblaslt", "--counter-workload"):
        assert opt in out


def test_bench_refuses_several_gpus():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one MI355X" in r.stderr
