"""Accuracy and benchmark harness over the MI355X kernels, with the reference's workload schema,
result records and command line (``python -m m5kernels_amd.harness.cli``)."""

from .engine import NumericalMismatch, environment, run_case, timed, write_result
from .workloads import h3_cases, load, validate

__all__ = ["NumericalMismatch", "environment", "run_case", "timed", "write_result", "h3_cases", "load", "validate"]
