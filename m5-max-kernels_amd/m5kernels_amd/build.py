"""Build libm5k.so (gfx950 HIP kernels + C ABI) in-tree with hipcc.

Every translation unit under ``csrc/`` is compiled to an object under ``_build/``
(in parallel), then linked into ``lib/libm5k.so`` next to this package.  The measurement
kernels under ``diag/`` (bench.py's MFMA ceiling) go into ``lib/libm5k_diag.so``.  Flags:

* ``--offload-arch=gfx950`` only: MI355X is the single target.
* ``-ffp-contract=off``: no FMA contraction, so FP32 epilogues and normalization keep
  the rounding sequence the contract spells out.
* ``-fhip-fp32-correctly-rounded-divide-sqrt``: IEEE ``/`` and ``sqrt`` (the
  quantizer's ``x / scale`` must round exactly like the CPU reference).
* ``-Xclang -target-feature -Xclang -packed-fp32-ops``: no packed FP32 VALU ops.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent.parent  # m5-max-kernels_amd/
REPO_ROOT = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
INCLUDE = REPO_ROOT / "include"
BUILD_DIR = REPO_ROOT / "_build" / "libm5k"
LIB_PATH = PKG_ROOT / "lib" / "libm5k.so"
DIAG_DIR = PKG_ROOT / "diag"
DIAG_LIB_PATH = PKG_ROOT / "lib" / "libm5k_diag.so"

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build libm5k.so")
    return path


def sources() -> list[Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def _compile(src: Path, force: bool) -> Path:
    obj = BUILD_DIR / (src.name + ".o")
    headers = list(CSRC.glob("*.h")) + list(INCLUDE.glob("*.h"))
    newest_dep = max(p.stat().st_mtime for p in [src, *headers])
    if not force and obj.exists() and obj.stat().st_mtime >= newest_dep:
        return obj
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd = [hipcc(), "-O2", "-std=c++17", "-fPIC", f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr[-4000:]}")
    return obj


def build(force: bool = True, jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile every csrc/ translation unit for gfx950 and link lib/libm5k.so."""
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    LIB_PATH.parent.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(lambda s: _compile(s, force), srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link of libm5k.so failed:\n{proc.stderr[-4000:]}")
    os.replace(tmp, LIB_PATH)
    build_diag()
    if verbose:
        print(f"built {LIB_PATH} from {len(srcs)} sources, and {DIAG_LIB_PATH}", file=sys.stderr)
    return LIB_PATH


def build_diag() -> Path:
    """Link lib/libm5k_diag.so: measurement kernels used by bench.py (no op uses them)."""
    tmp = DIAG_LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, "-shared", "-o", str(tmp), *map(str, sorted(DIAG_DIR.glob("*.hip")))]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"build of libm5k_diag.so failed:\n{proc.stderr[-4000:]}")
    os.replace(tmp, DIAG_LIB_PATH)
    return DIAG_LIB_PATH


if __name__ == "__main__":
    build(force="--incremental" not in sys.argv, verbose=True)
