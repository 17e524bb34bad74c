#!/usr/bin/env python3
"""W8A8 FFN-down on one MI355X, online activation quantization included.

Workload (the headline metric: FFN-down of the FFN up/down configuration): A bf16 [4096, 16384] ~N(0,1)
with 0.1% of channels (every 1024th) scaled x50, W bf16 [4096, 16384] ~N(0, 0.02), seed 29,
synthetic.  Offline (untimed): W -> per-output-channel INT8 codes + FP32 scales.  One step
= quantize(A) (per-token INT8) + W8A8 MFMA GEMM with the FP32 scale epilogue -> BF16 C.

Prints ONE JSON line: value = TOPS = 2*M*N*K / (ms per online step), the roofline of the
dominant kernel (the GEMM, dense INT8 MFMA peak), per-kernel HIP-event timings and the CPU
baseline (the oracle's C/OpenMP W8A8 on a bounded row sample, rank 0 only).

Timing.  After the W warmup steps, further untimed steps run until at least --settle-seconds
(0.4 s) of device time has passed, whatever W is: on MI355X the first ~100 steps after idle run
10-15% slower while the clocks ramp (the count is reported as settle_steps).  The headline region has
only a start and an end event around the K steps (per-step timing events add ~3%).  The
per-kernel durations that the roofline uses come from passes with no event between two kernels
(an event there, even one without a system fence, slows both kernels it separates): K GEMM
launches back to back between one event pair, and K quantizer launches cycling over activation
sets beyond the Infinity Cache.

--schedules prints instead one JSON line comparing, on the shapes of SCHEDULE_SHAPES, the GEMM
schedule the library picks (mixed 256 x 256 + 256 x 128 tiles, or 256 x 224 tiles) with the
plain launch: bit equality and ABBA-ordered device times.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for _p in (REPO / "m5-max-kernels_amd", REPO):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

M, K, N = 4096, 16384, 4096
SEED = 29
PEAK_INT8_TOPS = 5000.0  # MI355X dense INT8 MFMA, 5.0 POP/s
PEAK_HBM_GBS = 8000.0  # MI355X HBM3E, 8 TB/s
TRAFFIC_FILE = REPO / "profiles" / "traffic.json"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class FenceFreeEvent:
    """A HIP timing event created with hipEventDisableSystemFence (through the HIP runtime torch
    has loaded).  torch.cuda.Event records with a system-scope release, which writes back and
    invalidates the caches between the kernels it separates: in the FFN-down step that moved
    ~15 us of the quantizer's and the GEMM's cache write-back into the wrong interval (the event
    pass summed to 231.6 us against a 214.5 us step; the rocprof kernel trace of an event-free
    step agreed with neither).  Without the fence the event only timestamps the stream."""

    _hip = None
    DISABLE_SYSTEM_FENCE = 0x20000000  # hipEventDisableSystemFence (hip_runtime_api.h)

    def __init__(self):
        import ctypes

        if FenceFreeEvent._hip is None:
            hip = ctypes.CDLL("libamdhip64.so.7")  # the runtime already loaded by torch (same SONAME)
            hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
            hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
            hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
            hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
            FenceFreeEvent._hip = hip
        self._ctypes = ctypes
        self.handle = ctypes.c_void_p()
        rc = FenceFreeEvent._hip.hipEventCreateWithFlags(ctypes.byref(self.handle), self.DISABLE_SYSTEM_FENCE)
        if rc != 0:
            raise RuntimeError(f"hipEventCreateWithFlags failed ({rc})")

    def record(self, stream):
        rc = FenceFreeEvent._hip.hipEventRecord(self.handle, self._ctypes.c_void_p(stream.cuda_stream))
        if rc != 0:
            raise RuntimeError(f"hipEventRecord failed ({rc})")

    def elapsed_time(self, end):
        ms = self._ctypes.c_float()
        rc = FenceFreeEvent._hip.hipEventElapsedTime(self._ctypes.byref(ms), self.handle, end.handle)
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return ms.value

    def __del__(self):
        hip = getattr(FenceFreeEvent, "_hip", None) if FenceFreeEvent is not None else None
        if hip is not None and self.handle:
            hip.hipEventDestroy(self.handle)


def make_inputs(torch, dev):
    g = torch.Generator(device=dev).manual_seed(SEED)
    a = torch.randn((M, K), generator=g, device=dev)
    a[:, ::1024] *= 50.0  # 16 of 16384 channels = 0.1% outliers
    w = torch.randn((N, K), generator=g, device=dev) * 0.02
    return a.to(torch.bfloat16), w.to(torch.bfloat16)


def cpu_baseline(torch, a, wq, ws, y, target_s):
    """Time the oracle's C W8A8 linear on a bounded row sample; check it against the GPU rows."""
    import numpy as np

    from oracle import reference as ref

    bits = lambda t: t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)  # noqa: E731
    wq_np, ws_np = wq.cpu().numpy(), ws.cpu().numpy()
    probe_rows = 8
    a_probe = bits(a[:probe_rows])
    ref.c_w8a8_linear_bf16(a_probe, wq_np, ws_np)  # warm (page in, thread pool)
    t0 = time.perf_counter()
    ref.c_w8a8_linear_bf16(a_probe, wq_np, ws_np)
    per_row = (time.perf_counter() - t0) / probe_rows
    rows = int(min(M, max(probe_rows, target_s / max(per_row, 1e-9))))
    a_rows = bits(a[:rows])
    t0 = time.perf_counter()
    out = ref.c_w8a8_linear_bf16(a_rows, wq_np, ws_np)
    elapsed = time.perf_counter() - t0
    equal = bool(np.array_equal(out, bits(y[:rows])))
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or len(os.sched_getaffinity(0))
    return {
        "value": 2.0 * rows * N * K / elapsed / 1e12,
        "unit": "TOPS",
        "cores": threads,
        "kind": "port",
        "sample": f"rows 0..{rows - 1} of the {M}-row FFN-down step (K={K}, N={N}): per-token INT8 quant + "
        f"exact INT32 GEMM + FP32 scale epilogue + BF16, oracle/m5k_oracle.c with OpenMP",
        "seconds": elapsed,
        "ms_per_full_step_extrapolated": elapsed / rows * M * 1e3,
        "bitwise_equal_to_gpu_rows": equal,
    }


def numpy_baseline(torch, a, wq, ws, y, target_s):
    """The reference's own validation idiom in NumPy on a bounded row sample: FP32 per-row
    quantize, then the float64 product of the decoded codes (engine.py:173-175 of the
    reference, there on sampled rows and columns).  W is decoded once, outside the timing, as
    it is quantized offline."""
    import numpy as np

    from oracle import reference as ref

    w_dec = ref.dequantize(wq.cpu().numpy(), ws.cpu().numpy(), "int8").astype(np.float64)

    def step(rows):
        q, s = ref.quantize_reference(a[:rows].float().cpu().numpy(), "int8")
        return ref.dequantize(q, s, "int8").astype(np.float64) @ w_dec.T

    probe_rows = 16
    step(probe_rows)  # warm (thread pool)
    t0 = time.perf_counter()
    step(probe_rows)
    per_row = (time.perf_counter() - t0) / probe_rows
    rows = int(min(M, max(probe_rows, target_s / max(per_row, 1e-9))))
    a_host = a[:rows].float().cpu()  # the device-to-host copy stays outside the timing
    t0 = time.perf_counter()
    q, s = ref.quantize_reference(a_host.numpy(), "int8")
    out = ref.dequantize(q, s, "int8").astype(np.float64) @ w_dec.T
    elapsed = time.perf_counter() - t0
    gpu = y[:rows].float().cpu().numpy().astype(np.float64)
    rel = float(np.linalg.norm(gpu - out) / np.linalg.norm(out))
    return {
        "value": 2.0 * rows * N * K / elapsed / 1e12,
        "unit": "TOPS",
        "cores": len(os.sched_getaffinity(0)),
        "threads_env": {k: os.environ.get(k) for k in ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS", "MKL_NUM_THREADS")},
        "sample": f"rows 0..{rows - 1} of the {M}-row FFN-down step: NumPy FP32 per-row INT8 quantize + float64 "
        f"matmul of the decoded codes against the decoded W [{N},{K}]",
        "seconds": elapsed,
        "ms_per_full_step_extrapolated": elapsed / rows * M * 1e3,
        "relative_l2_vs_gpu_bf16_rows": rel,
    }


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


OP_SETTLE_S = 0.15  # device seconds of back-to-back calls before each timed op (--op-settle)


def _set_op_settle(seconds):
    global OP_SETTLE_S
    OP_SETTLE_S = seconds


def time_op(torch, fn, reps=20, warm=10, settle_s=None):
    """Steady-state device time of fn on the current stream.

    fn first runs back to back for `settle_s` seconds of device time: MI355X ramps its clocks
    over the first ~100 ms of sustained load after idle and drops them again in an idle gap of
    tens of milliseconds.  A short GPU spin (~2 ms) is then queued ahead of the timed launches, so
    the host enqueues every one of them before the first runs: they execute back to back and the
    events measure device time only, not the Python wrapper's per-call overhead (which exceeds
    the run time of the smaller kernels).  With a 50M-cycle spin instead (tens of milliseconds
    near idle) the FFN-up GEMM measured 270.6 us against 227.3 us settled.  avg_ms comes from one
    event pair around `reps` back-to-back calls; an event pair around every call adds a few
    microseconds per call on this device, so the per-call pass only supplies the p10/p90 spread
    (and its own mean, per_call_avg_ms)."""
    settle_s = OP_SETTLE_S if settle_s is None else settle_s
    for _ in range(warm):
        fn()
    settle(torch, fn, settle_s)
    b0, b1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(5_000_000)
    b0.record()
    for _ in range(reps):
        fn()
    b1.record()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    settle(torch, fn, settle_s / 3)
    torch.cuda._sleep(10_000_000)
    for e0, e1 in evs:
        e0.record()
        fn()
        e1.record()
    torch.cuda.synchronize()
    ts = sorted(e0.elapsed_time(e1) for e0, e1 in evs)
    return {"avg_ms": b0.elapsed_time(b1) / reps, "p10_ms": ts[len(ts) // 10], "p90_ms": ts[(9 * len(ts)) // 10],
            "per_call_avg_ms": statistics.fmean(ts)}


INFINITY_CACHE_BYTES = 256 << 20  # MI355X's memory-side cache


def time_streaming(torch, fns, reps=24):
    """avg_ms like time_op's, but each call takes the next of `fns`, closures over independent
    input sets whose footprint together exceeds twice the 256 MB Infinity Cache, and every
    call's outputs stay referenced for a whole cycle (so the allocator hands out fresh output
    memory too).  On one repeated input set a kernel whose footprint fits that cache re-reads its
    inputs from it and overwrites its own dirty output lines; this is the HBM-streaming rate."""
    n = len(fns)
    keep = [None] * n
    state = [0]

    def step():
        i = state[0] % n
        keep[i] = None
        keep[i] = fns[i]()
        state[0] += 1

    for _ in range(2 * n):
        step()
    settle(torch, step, OP_SETTLE_S)
    b0, b1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(5_000_000)
    b0.record()
    for _ in range(reps):
        step()
    b1.record()
    torch.cuda.synchronize()
    return b0.elapsed_time(b1) / reps


def _sets_for(footprint_bytes):
    return max(2, -(-2 * INFINITY_CACHE_BYTES // footprint_bytes))


def _rel_l2(actual, reference):
    import numpy as np

    return float(np.linalg.norm(actual - reference) / np.linalg.norm(reference))


def _gemm_case(torch, dev, m, k, n, seed, mode="int8", outlier_every=None, bf16_compare=False):
    """Online W quantized offline; step = quantize(A) + GEMM -> BF16.  With bf16_compare, also
    the BF16 torch F.linear of the same A and W (timed the same way) and both outputs' rel-L2
    against the float64 product on 32 rows spread over M (the reference's sampled-row check)."""
    from m5kernels_amd import gemm, quantize

    g = torch.Generator(device=dev).manual_seed(seed)
    a = torch.randn((m, k), generator=g, device=dev)
    if outlier_every:
        a[:, ::outlier_every] *= 50.0
    a = a.to(torch.bfloat16)
    w = (torch.randn((n, k), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    wq, ws = quantize(w, mode)
    aq, sa = quantize(a, mode)
    ops = 2.0 * m * n * k

    def online():
        q, s = quantize(a, mode)
        return gemm(q, wq, mode, a_scales=s, b_scales=ws, output_dtype=torch.bfloat16)

    step = time_op(torch, online)
    only = time_op(torch, lambda: gemm(aq, wq, mode, a_scales=sa, b_scales=ws, output_dtype=torch.bfloat16))
    compare = {}
    if bf16_compare:
        import numpy as np

        bf = time_op(torch, lambda: torch.nn.functional.linear(a, w))
        rows = torch.linspace(0, m - 1, 32).round().long().to(dev)
        exact = a[rows].double().cpu().numpy() @ w.double().cpu().numpy().T
        y8 = online()[rows].float().cpu().numpy().astype(np.float64)
        y16 = torch.nn.functional.linear(a, w)[rows].float().cpu().numpy().astype(np.float64)
        compare = {"bf16_linear_ms": bf["avg_ms"], "bf16_linear_TFLOPs": ops / (bf["avg_ms"] * 1e-3) / 1e12,
                   "online_speedup_over_bf16": bf["avg_ms"] / step["avg_ms"],
                   "rel_l2_vs_float64_w8a8": _rel_l2(y8, exact), "rel_l2_vs_float64_bf16": _rel_l2(y16, exact),
                   "rel_l2_rows": "32 rows spread over M, full K, all N"}
    return {
        "shape": {"m": m, "k": k, "n": n},
        "mode": mode,
        "online_ms": step["avg_ms"],
        "online_TOPS": ops / (step["avg_ms"] * 1e-3) / 1e12,
        "gemm_ms": only["avg_ms"],
        "gemm_TOPS": ops / (only["avg_ms"] * 1e-3) / 1e12,
        "gemm_frac_of_peak": ops / (only["avg_ms"] * 1e-3) / 1e12 / PEAK_INT8_TOPS,
        "gemm_weight_GBps": n * k / (only["avg_ms"] * 1e-3) / 1e9,  # the bound that matters at short M
        "online_p10_p90_ms": [step["p10_ms"], step["p90_ms"]],
        **compare,
    }


def _hadamard_case(torch, dev):
    """FFN-down with a normalized block-128 Hadamard (signs +1): W rotated + quantized offline,
    A rotated in FP32 and quantized online in one kernel, then the W8A8 GEMM."""
    from m5kernels_amd import gemm, quantize, rotate, rotate_quantize

    g = torch.Generator(device=dev).manual_seed(SEED)
    a = torch.randn((M, K), generator=g, device=dev)
    a[:, ::1024] *= 50.0
    a = a.to(torch.bfloat16)
    w = (torch.randn((N, K), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    signs = torch.ones(K, dtype=torch.int8, device=dev)
    wq, ws = quantize(rotate(w, 128, signs), "int8")
    ops = 2.0 * M * N * K

    def online():
        q, s = rotate_quantize(a, 128, signs)
        return gemm(q, wq, "int8", a_scales=s, b_scales=ws, output_dtype=torch.bfloat16)

    step = time_op(torch, online)
    rq = time_op(torch, lambda: rotate_quantize(a, 128, signs))
    nbytes = 3 * M * K + 4 * M
    n = _sets_for(nbytes)
    As = [a] + [torch.randn((M, K), generator=g, device=dev).to(torch.bfloat16) for _ in range(n - 1)]
    rq_st = time_streaming(torch, [lambda i=i: rotate_quantize(As[i], 128, signs) for i in range(n)])
    return {
        "rotate_quantize_streaming_ms": rq_st,
        "rotate_quantize_streaming_frac_of_hbm_peak": nbytes / (rq_st * 1e-3) / 1e9 / PEAK_HBM_GBS,
        "online_ms": step["avg_ms"],
        "online_TOPS": ops / (step["avg_ms"] * 1e-3) / 1e12,
        "rotate_quantize_ms": rq["avg_ms"],
        "rotate_quantize_GBps": nbytes / (rq["avg_ms"] * 1e-3) / 1e9,
        "rotate_quantize_frac_of_hbm_peak": nbytes / (rq["avg_ms"] * 1e-3) / 1e9 / PEAK_HBM_GBS,
    }


def _prep_case(torch, dev, m, k=4096, tables=2):
    """Fused AdaLN prep (LayerNorm, H128, P per-batch tables, BF16 boundary) with and without
    the gated residual update, the staged comparators, and the W8A8 GEMM it feeds."""
    from m5kernels_amd import (fused_gated_residual_norm_hadamard_quantize, fused_norm_hadamard_quantize, gated_residual_add,
                               gemm, quantize, rotate_quantize, unfused_norm)

    g = torch.Generator(device=dev).manual_seed(SEED)
    bf = torch.bfloat16
    res = torch.randn((m, k), generator=g, device=dev).to(bf)
    branch = torch.randn((m, k), generator=g, device=dev).to(bf)
    gate = (torch.randn((tables, k), generator=g, device=dev) * 0.1).to(bf)
    scale = (torch.randn((tables, k), generator=g, device=dev) * 0.1).to(bf)
    shift = (torch.randn((tables, k), generator=g, device=dev) * 0.1).to(bf)
    gamma = (1 + 0.1 * torch.randn((k,), generator=g, device=dev)).to(bf)
    row_map = (torch.arange(m, device=dev, dtype=torch.int32) * tables // m).to(torch.int32)
    signs = torch.ones(k, dtype=torch.int8, device=dev)
    kw = dict(norm="layer", epsilon=1e-5, round_output="input", row_map=row_map)
    gated = time_op(torch, lambda: fused_gated_residual_norm_hadamard_quantize(
        res, branch, gate, gamma, scale, shift, signs, 128, gate_row_map=row_map, **kw))
    plain = time_op(torch, lambda: fused_norm_hadamard_quantize(res, gamma, scale, shift, signs, 128, **kw))

    def staged():
        r = gated_residual_add(res, branch, gate, gate_row_map=row_map)
        y = unfused_norm(r, gamma, scale, shift, **kw)
        return rotate_quantize(y, 128, signs)

    staged_t = time_op(torch, staged)
    w = (torch.randn((k, k), generator=g, device=dev) * 0.02).to(bf)
    wq, ws = quantize(w, "int8")
    q, s = fused_norm_hadamard_quantize(res, gamma, scale, shift, signs, 128, **kw)
    gemm_t = time_op(torch, lambda: gemm(q, wq, "int8", a_scales=s, b_scales=ws, output_dtype=bf))
    table_bytes = 2 * k + 3 * 2 * tables * k + 4 * m + k  # gamma, gate/scale/shift tables, row map, signs
    gated_bytes = 7 * m * k + 4 * m + table_bytes
    plain_bytes = 3 * m * k + 4 * m + table_bytes
    gbs = lambda b, t: b / (t * 1e-3) / 1e9  # noqa: E731
    streaming = {}
    if gated_bytes < INFINITY_CACHE_BYTES:
        n = _sets_for(gated_bytes)
        rs = [torch.randn((m, k), generator=g, device=dev).to(bf) for _ in range(n)]
        bs = [torch.randn((m, k), generator=g, device=dev).to(bf) for _ in range(n)]
        gs_ms = time_streaming(torch, [lambda i=i: fused_gated_residual_norm_hadamard_quantize(
            rs[i], bs[i], gate, gamma, scale, shift, signs, 128, gate_row_map=row_map, **kw) for i in range(n)])
        n2 = _sets_for(plain_bytes)
        xs = (rs + [torch.randn((m, k), generator=g, device=dev).to(bf) for _ in range(n2 - n)])[:n2]
        ps_ms = time_streaming(torch, [lambda i=i: fused_norm_hadamard_quantize(xs[i], gamma, scale, shift, signs, 128,
                                                                                **kw) for i in range(n2)])
        streaming = {
            "gated_fused_streaming_ms": gs_ms,
            "gated_fused_streaming_frac_of_hbm_peak": gbs(gated_bytes, gs_ms) / PEAK_HBM_GBS,
            "fused_streaming_ms": ps_ms,
            "fused_streaming_frac_of_hbm_peak": gbs(plain_bytes, ps_ms) / PEAK_HBM_GBS,
            "streaming_input_sets": [n, n2],
        }
    return {
        **streaming,
        "m": m,
        "k": k,
        "tables": tables,
        "gated_fused_ms": gated["avg_ms"],
        "gated_fused_GBps": gbs(gated_bytes, gated["avg_ms"]),
        "gated_fused_frac_of_hbm_peak": gbs(gated_bytes, gated["avg_ms"]) / PEAK_HBM_GBS,
        "gated_bytes_per_launch": gated_bytes,
        "fused_ms": plain["avg_ms"],
        "fused_GBps": gbs(plain_bytes, plain["avg_ms"]),
        "fused_frac_of_hbm_peak": gbs(plain_bytes, plain["avg_ms"]) / PEAK_HBM_GBS,
        "fused_bytes_per_launch": plain_bytes,
        "staged_gated_ms": staged_t["avg_ms"],
        "staged_over_fused": staged_t["avg_ms"] / gated["avg_ms"],
        "w8a8_gemm_4096_ms": gemm_t["avg_ms"],
        "w8a8_gemm_4096_TOPS": 2.0 * m * k * k / (gemm_t["avg_ms"] * 1e-3) / 1e12,
    }


def prep_mixed(torch, dev, reps):
    """--prep-mixed REPS: the C4 gated prep (M 4096, K 4096, LayerNorm, H128, two tables) with a BF16
    residual, an FP16 branch and the tables in three dtypes (gamma FP16, scale FP32, shift BF16,
    gate FP32), REPS calls after the inputs are made, then the same call on all-BF16 inputs
    (time_op each).  Under a rocprofv3 kernel trace the mixed calls are REPS dispatches of the one
    prep kernel and nothing else: no cast kernels."""
    from m5kernels_amd import fused_gated_residual_norm_hadamard_quantize

    m, k, tables = 4096, 4096, 2
    g = torch.Generator(device=dev).manual_seed(SEED)
    res = torch.randn((m, k), generator=g, device=dev).to(torch.bfloat16)
    branch = torch.randn((m, k), generator=g, device=dev).to(torch.float16)
    gate = (torch.randn((tables, k), generator=g, device=dev) * 0.1).to(torch.float32)
    scale = (torch.randn((tables, k), generator=g, device=dev) * 0.1).to(torch.float32)
    shift = (torch.randn((tables, k), generator=g, device=dev) * 0.1).to(torch.bfloat16)
    gamma = (1 + 0.1 * torch.randn((k,), generator=g, device=dev)).to(torch.float16)
    row_map = (torch.arange(m, device=dev, dtype=torch.int32) * tables // m).to(torch.int32)
    signs = torch.ones(k, dtype=torch.int8, device=dev)
    kw = dict(norm="layer", epsilon=1e-5, round_output="input", row_map=row_map, gate_row_map=row_map)
    bf = [t.to(torch.bfloat16) for t in (branch, gate, gamma, scale)]
    torch.cuda.synchronize()
    log(f"[bench] prep mixed dtypes: {reps} calls")
    for _ in range(reps):
        fused_gated_residual_norm_hadamard_quantize(res, branch, gate, gamma, scale, shift, signs, 128, **kw)
    torch.cuda.synchronize()
    mixed = time_op(torch, lambda: fused_gated_residual_norm_hadamard_quantize(
        res, branch, gate, gamma, scale, shift, signs, 128, **kw))
    same = time_op(torch, lambda: fused_gated_residual_norm_hadamard_quantize(
        res, bf[0], bf[1], bf[2], bf[3], shift, signs, 128, **kw))
    return {"m": m, "k": k, "calls": reps, "mixed_dtypes_ms": mixed["avg_ms"], "all_bf16_ms": same["avg_ms"],
            "dtypes": {"residual": "bf16", "branch": "fp16", "gamma": "fp16", "scale": "fp32", "shift": "bf16",
                       "gate": "fp32"}}


def _qk_case(torch, dev, m=9914, k=4096, n=4096):
    """Q projection + per-head RMSNorm + split-half RoPE (R = 64, base 10000, positions 0..m-1),
    head-major BF16 [32, m, 128]: INT8 online (quantize + fused projection) and BF16 modes, and
    the staged postprocess on a BF16 projection."""
    from m5kernels_amd import gemm, projection_qk_rope, qk_norm_rope, quantize

    g = torch.Generator(device=dev).manual_seed(SEED)
    bf = torch.bfloat16
    x = torch.randn((m, k), generator=g, device=dev).to(bf)
    w = (torch.randn((n, k), generator=g, device=dev) * 0.02).to(bf)
    gamma = (1 + 0.02 * torch.randn((128,), generator=g, device=dev)).to(bf)
    theta = 10000.0 ** (-torch.arange(64, device=dev, dtype=torch.float64) * 2 / 128)
    ang = torch.arange(m, device=dev, dtype=torch.float64)[:, None] * theta[None, :]
    cos, sin = ang.cos().float().to(bf), ang.sin().float().to(bf)
    wq, ws = quantize(w, "int8")
    ops = 2.0 * m * n * k

    def int8_online():
        q, s = quantize(x, "int8")
        return projection_qk_rope(q, wq, gamma, cos, sin, "int8", a_scales=s, b_scales=ws, epsilon=1e-6)

    t8 = time_op(torch, int8_online)
    xq, xs = quantize(x, "int8")
    fused = time_op(torch, lambda: projection_qk_rope(xq, wq, gamma, cos, sin, "int8", a_scales=xs, b_scales=ws,
                                                      epsilon=1e-6))
    staged = time_op(torch, lambda: qk_norm_rope(gemm(xq, wq, "int8", a_scales=xs, b_scales=ws,
                                                      output_dtype=torch.bfloat16), gamma, cos, sin, epsilon=1e-6))
    tb = time_op(torch, lambda: projection_qk_rope(x, w, gamma, cos, sin, "bf16", epsilon=1e-6))
    proj = gemm(x, w, "bf16", output_dtype=bf)
    tpost = time_op(torch, lambda: qk_norm_rope(proj, gamma, cos, sin, epsilon=1e-6))
    post_bytes = 2 * m * n * 2 + 2 * 2 * m * 64 + 2 * 128
    return {
        "m": m,
        "int8_online_ms": t8["avg_ms"],
        "int8_online_TOPS": ops / (t8["avg_ms"] * 1e-3) / 1e12,
        "int8_fused_ms": fused["avg_ms"],
        "int8_fused_TOPS": ops / (fused["avg_ms"] * 1e-3) / 1e12,
        "int8_staged_gemm_plus_postprocess_ms": staged["avg_ms"],
        "bf16_fused_ms": tb["avg_ms"],
        "bf16_fused_TFLOPs": ops / (tb["avg_ms"] * 1e-3) / 1e12,
        "staged_postprocess_ms": tpost["avg_ms"],
        "staged_postprocess_GBps": post_bytes / (tpost["avg_ms"] * 1e-3) / 1e9,
    }


def _qkv_case(torch, dev, m=4096, heads=32, k=4096):
    """Grouped Q/K/V projection (weights [heads, 3, 128, K]) with per-head RMSNorm + RoPE on Q/K
    and V passthrough, INT8 online (quantize + one fused kernel), R = 64, base 10000."""
    from m5kernels_amd import projection_qkv_rope, quantize

    g = torch.Generator(device=dev).manual_seed(SEED)
    bf = torch.bfloat16
    x = torch.randn((m, k), generator=g, device=dev).to(bf)
    w = (torch.randn((heads * 384, k), generator=g, device=dev) * 0.02).to(bf)
    qg = (1 + 0.02 * torch.randn((128,), generator=g, device=dev)).to(bf)
    kg = (1 + 0.02 * torch.randn((128,), generator=g, device=dev)).to(bf)
    theta = 10000.0 ** (-torch.arange(64, device=dev, dtype=torch.float64) * 2 / 128)
    ang = torch.arange(m, device=dev, dtype=torch.float64)[:, None] * theta[None, :]
    cos, sin = ang.cos().float().to(bf), ang.sin().float().to(bf)
    wq, ws = quantize(w, "int8")
    ops = 2.0 * m * heads * 384 * k

    def online():
        q, s = quantize(x, "int8")
        return projection_qkv_rope(q, wq, qg, kg, cos, sin, "int8", a_scales=s, w_scales=ws)

    t = time_op(torch, online)
    return {"m": m, "heads": heads, "k": k, "int8_online_ms": t["avg_ms"],
            "int8_online_TOPS": ops / (t["avg_ms"] * 1e-3) / 1e12}


def _chain_case(torch, dev, m=4096, h=5376, pk=7168, n=14336):
    """Gate-placement chain (gate_epilogue_chain.py:95-150): resident INT8 previous activation ->
    W8A8 projection [pk -> h] -> gated residual update + AdaLN + H256 + INT8 -> W8A8 projection
    [h -> n], with the gate in the previous GEMM's epilogue or in the fused preparation.  TOPS
    counts both projections' MACs x 2, the reference's effective_tops."""
    from m5kernels_amd import gate_chain, quantize

    g = torch.Generator(device=dev).manual_seed(SEED)
    bf = torch.bfloat16

    def arr(shape, factor=1.0):
        return (torch.randn(shape, generator=g, device=dev) * factor).to(bf)

    aq, sa = quantize(arr((m, pk)), "int8")
    q0, s0 = quantize(arr((h, pk), pk**-0.5), "int8")
    q1, s1 = quantize(arr((n, h), h**-0.5), "int8")
    residual, gate = arr((m, h)), arr((h,), 0.2)
    gamma, scale, shift = (1 + 0.1 * torch.randn((h,), generator=g, device=dev)).to(bf), arr((h,), 0.2), arr((h,), 0.1)
    signs = torch.ones(h, dtype=torch.int8, device=dev)
    ops = 2.0 * m * h * (pk + n)
    out = {"m": m, "k": h, "previous_k": pk, "n": n}
    for placement in ("gate-in-gemm", "gate-in-norm"):
        t = time_op(torch, lambda: gate_chain(aq, sa, q0, s0, q1, s1, residual, gate, gamma, scale, shift, signs,
                                              placement=placement))
        out[f"{placement}_ms"] = t["avg_ms"]
        out[f"{placement}_TOPS"] = ops / (t["avg_ms"] * 1e-3) / 1e12
    return out


def _shift_split_case(torch, dev, m=4096, k=5376, n=7168):
    """Shift-split Q projection (docs/affine-shift-splitting.md, P = 1): cached FP32 shift bias +
    RMS-folded H256 INT8 + W8A8 with bias epilogue, against the full FP32 AdaLN fused prep +
    W8A8; plus the conditioning-table build at P = 1, 3, 60, 117 rows (bias-cache study)."""
    from m5kernels_amd import (fused_norm_hadamard_quantize, gemm, norm_shift_split_gemm, quantize, rotate,
                               shift_split_condition)

    g = torch.Generator(device=dev).manual_seed(SEED)
    bf = torch.bfloat16

    def arr(shape, factor=1.0, offset=0.0):
        return (offset + torch.randn(shape, generator=g, device=dev) * factor).to(bf)

    x, w = arr((m, k)), arr((n, k))
    gamma, scale, shift = arr((k,), 0.1, 1.0), arr((k,), 0.2), arr((k,), 0.1)
    signs = torch.ones(k, dtype=torch.int8, device=dev)
    wq, ws = quantize(rotate(w, 256, signs), "int8")
    ops = 2.0 * m * n * k

    def condition():
        return shift_split_condition(gamma, scale, shift, w, bias_backend="mpp-bf16-to-fp32")

    combined, bias = condition()

    def split_online():
        return norm_shift_split_gemm(x, wq, ws, signs, combined, bias)

    def split_with_condition():
        c, b = condition()
        return norm_shift_split_gemm(x, wq, ws, signs, c, b)

    def full_fp32():
        q, s = fused_norm_hadamard_quantize(x, gamma, scale, shift, signs, 256, round_output="fp32")
        return gemm(q, wq, "int8", a_scales=s, b_scales=ws, output_dtype=bf)

    out = {"m": m, "k": k, "n": n}
    for key, fn in (("split_cached_online", split_online), ("split_with_condition", split_with_condition),
                    ("full_fp32_adaln_online", full_fp32), ("condition_prepare", condition)):
        t = time_op(torch, fn)
        out[f"{key}_ms"] = t["avg_ms"]
        if key != "condition_prepare":
            out[f"{key}_TOPS"] = ops / (t["avg_ms"] * 1e-3) / 1e12
    wbytes = 2 * n * k
    for p in (1, 3, 60, 117):
        sc, sh = arr((p, k), 0.2), arr((p, k), 0.1)
        t = time_op(torch, lambda: shift_split_condition(gamma, sc, sh, w, bias_backend="mpp-bf16-to-fp32"))
        out[f"bias_cache_p{p}_ms"] = t["avg_ms"]
        out[f"bias_cache_p{p}_weight_GBps"] = wbytes / (t["avg_ms"] * 1e-3) / 1e9
    return out


def _rms_case(torch, dev, m=4096, k=4096, block=256):
    """RMS scale-folded INT8 quantizer (rms_quantize) on a bf16 [m, k] activation, H256."""
    from m5kernels_amd import rms_quantize

    g = torch.Generator(device=dev).manual_seed(SEED)
    x = torch.randn((m, k), generator=g, device=dev).to(torch.bfloat16)
    gamma = (1 + 0.1 * torch.randn((k,), generator=g, device=dev)).float()
    signs = torch.ones(k, dtype=torch.int8, device=dev)
    nbytes = 3 * m * k + 4 * m + 5 * k
    out = {"m": m, "k": k, "block": block}
    for fold in (True, False):
        t = time_op(torch, lambda: rms_quantize(x, gamma, signs, block, fold_scale=fold))
        key = "fold" if fold else "no_fold"
        out[f"{key}_ms"] = t["avg_ms"]
        out[f"{key}_GBps"] = nbytes / (t["avg_ms"] * 1e-3) / 1e9
        out[f"{key}_frac_of_hbm_peak"] = out[f"{key}_GBps"] / PEAK_HBM_GBS
    n = _sets_for(nbytes)
    xs = [x] + [torch.randn((m, k), generator=g, device=dev).to(torch.bfloat16) for _ in range(n - 1)]
    st = time_streaming(torch, [lambda i=i: rms_quantize(xs[i], gamma, signs, block) for i in range(n)])
    out["fold_streaming_ms"] = st
    out["fold_streaming_frac_of_hbm_peak"] = nbytes / (st * 1e-3) / 1e9 / PEAK_HBM_GBS
    return out


def extras(torch, dev):
    """Every other configuration: parity-test shapes timed on the same GPU (not the headline)."""
    out = {}
    cases = [
        ("ffn_down_fp8_online", lambda: _gemm_case(torch, dev, M, K, N, SEED, "fp8", 1024)),
        ("ffn_down_h128_int8_online", lambda: _hadamard_case(torch, dev)),
        ("q_proj_4096_int8_online", lambda: _gemm_case(torch, dev, 4096, 4096, 4096, SEED, bf16_compare=True)),
        ("ffn_up_int8_online", lambda: _gemm_case(torch, dev, 4096, 4096, 16384, SEED)),
        ("ffn_down_m128_int8_online_splitk", lambda: _gemm_case(torch, dev, 128, K, N, SEED)),
        ("q_proj_m128_int8_online_splitk", lambda: _gemm_case(torch, dev, 128, 4096, 4096, SEED)),
        ("fused_prep_m4096", lambda: _prep_case(torch, dev, 4096)),
        ("fused_prep_m9914", lambda: _prep_case(torch, dev, 9914)),
        ("qk_rope_m9914", lambda: _qk_case(torch, dev)),
        ("rms_quantize_m4096_h256", lambda: _rms_case(torch, dev)),
        ("grouped_qkv_m4096_h32", lambda: _qkv_case(torch, dev)),
        ("gate_chain_attention_to_ffn_m4096", lambda: _chain_case(torch, dev)),
        ("gate_chain_ffn_to_q_m4096", lambda: _chain_case(torch, dev, pk=14336, n=7168)),
        ("shift_split_q_m4096", lambda: _shift_split_case(torch, dev)),
    ]
    for name, fn in cases:
        log(f"[bench] extra {name}")
        out[name] = fn()
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    return out


# Shapes (mode, M, N, K) of the GEMM schedule comparison (--schedules): partial last rounds
# that the library runs as mixed (256 x 256 + 256 x 128) or narrow (256 x 224) launches, and
# the whole-round FFN-down shape that stays plain.
SCHEDULE_SHAPES = [
    ("int8", 9914, 4096, 4096), ("int8", 4096, 6144, 4096), ("int8", 4096, 5376, 5376),
    ("int8", 4096, 14336, 5376), ("int8", 9914, 7168, 5376), ("int8", 4096, 7168, 5376),
    ("int8", 2048, 5376, 5376), ("bf16", 4096, 5376, 5376), ("bf16", 4096, 7168, 5376),
    ("int8", 4096, 4096, 16384),
]


def schedules_probe(torch, dev, rounds=6, reps=20):
    """Each shape's library schedule against the plain launch (M5K_GEMM_MIXED_TILES=0 and
    M5K_GEMM_NARROW_TILES=0), through the C ABI: bit equality, then ABBA rounds of `reps`
    back-to-back calls between one event pair; medians."""
    from m5kernels_amd import _lib
    from m5kernels_amd.hip import launch_plan

    off = {"M5K_GEMM_MIXED_TILES": "0", "M5K_GEMM_NARROW_TILES": "0"}
    g = torch.Generator(device=dev).manual_seed(SEED)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    out = []
    for mode, m, n, k in SCHEDULE_SHAPES:
        if mode == "int8":
            a = torch.randint(-127, 128, (m, k), generator=g, device=dev, dtype=torch.int8)
            b = torch.randint(-127, 128, (n, k), generator=g, device=dev, dtype=torch.int8)
            sa = torch.rand(m, generator=g, device=dev) * 0.01 + 1e-3
            sb = torch.rand(n, generator=g, device=dev) * 0.01 + 1e-3
        else:
            a = torch.randn((m, k), generator=g, device=dev).to(torch.bfloat16)
            b = torch.randn((n, k), generator=g, device=dev).to(torch.bfloat16)
        c = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
        st = _lib.stream_of(c)
        if mode == "int8":
            args = ("m5k_gemm_i8", _lib.ptr(a), _lib.ptr(b), m, n, k, _lib.ptr(sa), _lib.ptr(sb), _lib.ptr(c),
                    _lib.BF16, None, None, None, None, None, st)
        else:
            args = ("m5k_gemm_float", _lib.ptr(a), _lib.ptr(b), _lib.BF16, m, n, k, _lib.ptr(c), _lib.BF16, None,
                    None, None, st)

        def run(plain):
            saved = {v: os.environ.pop(v, None) for v in off}
            if plain:
                os.environ.update(off)
            try:
                _lib.call(*args)
            finally:
                for v, old in saved.items():
                    if old is None:
                        os.environ.pop(v, None)
                    else:
                        os.environ[v] = old

        outs = []
        for plain in (False, True):
            c.fill_(7.0)
            run(plain)
            torch.cuda.synchronize()
            outs.append(c.clone())
        same = bool(torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16)))
        # ~50 ms of load first: the clocks settle to their sustained state (as in the headline run).
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < 0.05:
            for _ in range(20):
                run(False)
            torch.cuda.synchronize()
        times = {False: [], True: []}
        for r in range(rounds):
            for plain in ((False, True) if r % 2 == 0 else (True, False)):
                for _ in range(5):
                    run(plain)
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                torch.cuda.synchronize()
                torch.cuda._sleep(20_000_000)
                e0.record()
                for _ in range(reps):
                    run(plain)
                e1.record()
                torch.cuda.synchronize()
                times[plain].append(e0.elapsed_time(e1) / reps)
        sched_ms, plain_ms = statistics.median(times[False]), statistics.median(times[True])
        plan, full = launch_plan(mode, m, n, cus)
        out.append({"mode": mode, "m": m, "n": n, "k": k, "schedule": plan, "mixed_full_tiles": full,
                    "schedule_ms": sched_ms, "plain_ms": plain_ms, "speedup": plain_ms / sched_ms,
                    "bit_identical": same})
        log(f"[bench] schedules {mode} {m}x{n}x{k}: {plan} {sched_ms * 1e3:.1f} us, plain {plain_ms * 1e3:.1f} us, "
            f"x{plain_ms / sched_ms:.3f}, bit-identical {same}")
        del a, b, c, outs
    return out


def settle(torch, fn, seconds):
    """Run fn back to back for at least `seconds` of device time, synchronizing every 50 calls
    and once at the end: MI355X ramps its clocks over the first ~100 ms of sustained MFMA load
    after idle, and an idle gap of tens of milliseconds (as the first timing-event creation of
    a process takes) drops them again, so the caller starts timing right after this returns."""
    t0, calls = time.perf_counter(), 0
    while time.perf_counter() - t0 < seconds:
        for _ in range(50):
            fn()
        calls += 50
        torch.cuda.synchronize()
    return calls


VENDOR_SHAPES = [("ffn_down", 4096, 4096, 16384), ("ffn_up", 4096, 16384, 4096), ("q_proj", 4096, 4096, 4096),
                 ("m9914", 9914, 4096, 4096), ("h3_ffn_up", 4096, 14336, 5376)]


def vendor_probe(torch, dev, rounds=8, reps=10):
    """Our INT8 and FP8 GEMMs against hipBLASLt on the same codes: torch._int_mm (INT32 out, no
    epilogue) and torch._scaled_mm on the FP8 codes viewed as float8_e4m3fn, with per-row and
    per-column FP32 scales (the reference's scaling) and with scalar scales.  Inputs as the
    headline (A ~ N(0,1), W ~ N(0, 0.02), bf16, seed 29) at each shape; ABBA rounds of `reps`
    launches between one event pair, medians in ms."""
    from m5kernels_amd import gemm, quantize

    bf = torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(SEED)
    out = []
    for name, m, n, k in VENDOR_SHAPES:
        a = torch.randn((m, k), generator=g, device=dev).to(bf)
        w = (torch.randn((n, k), generator=g, device=dev) * 0.02).to(bf)
        aq, sa = quantize(a, "int8")
        wq, ws = quantize(w, "int8")
        a8, sa8 = quantize(a, "fp8")
        w8, ws8 = quantize(w, "fp8")
        wq_t = wq.t()
        fns = {
            "m5k_int8": lambda: gemm(aq, wq, "int8", a_scales=sa, b_scales=ws, output_dtype=bf),
            "hipblaslt_int8": lambda: torch._int_mm(aq, wq_t),
            "m5k_fp8": lambda: gemm(a8, w8, "fp8", a_scales=sa8, b_scales=ws8, output_dtype=bf),
        }
        af, wf = a8.view(torch.float8_e4m3fn), w8.view(torch.float8_e4m3fn)
        one = torch.ones((), device=dev)
        sa_col, sb_row = sa8.view(m, 1).float(), ws8.view(1, n).float()
        for key, fn in (("hipblaslt_fp8_rowwise",
                         lambda: torch._scaled_mm(af, wf.t(), scale_a=sa_col, scale_b=sb_row, out_dtype=bf)),
                        ("hipblaslt_fp8_scalar",
                         lambda: torch._scaled_mm(af, wf.t(), scale_a=one, scale_b=one, out_dtype=bf))):
            try:
                fn()
                fns[key] = fn
            except Exception as e:  # not every torch build offers every scaling
                log(f"[bench] vendor probe: {key} unavailable ({str(e).splitlines()[0][:100]})")
        for fn in fns.values():
            for _ in range(20):
                fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        times = {key: [] for key in fns}
        names = list(fns)
        for r in range(rounds):
            for key in names if r % 2 == 0 else names[::-1]:
                e0.record()
                for _ in range(reps):
                    fns[key]()
                e1.record()
                torch.cuda.synchronize()
                times[key].append(e0.elapsed_time(e1) / reps)
        ops = 2 * m * n * k
        row = {"shape": name, "m": m, "n": n, "k": k}
        for key, v in times.items():
            ms = statistics.median(v)
            row[key] = {"ms": ms, "TOPS": ops / (ms * 1e-3) / 1e12}
        out.append(row)
        log(f"[bench] vendor probe {name}: " + ", ".join(f"{key} {row[key]['ms'] * 1e3:.1f} us" for key in times))
    return out


def _diag_lib():
    import ctypes

    from m5kernels_amd import build as hip_build

    if not hip_build.DIAG_LIB_PATH.exists():
        raise RuntimeError(f"{hip_build.DIAG_LIB_PATH} is missing: build it with `python -m m5kernels_amd.build`")
    lib = ctypes.CDLL(str(hip_build.DIAG_LIB_PATH))
    lib.m5k_diag_mfma_ceiling.restype = ctypes.c_int
    lib.m5k_diag_mfma_ceiling.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                          ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                          ctypes.c_void_p]
    lib.m5k_diag_stream_mix.restype = ctypes.c_int
    lib.m5k_diag_stream_mix.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                        ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    return lib


def ceiling_kernels(torch, dev, aq, wq):
    """name -> launcher of the MFMA ceiling kernels (libm5k_diag.so) on the FFN-down codes: the
    GEMM main loop's v_mfma_i32_16x16x64_i8 stream alone, register-resident fragments read from
    the bench's own A and W codes, K / 128 iterations = the GEMM's MFMA count; the same on
    constant codes (all 1); the v_mfma_i32_32x32x32_i8 form of the same work; and the 16 x 16 x 64
    stream on four waves (one per SIMD) instead of eight."""
    import ctypes

    lib = _diag_lib()
    out = torch.empty((M // 256) * (N // 256) * 512, dtype=torch.int32, device=dev)

    def launcher(md, constant):
        def run():
            stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
            rc = lib.m5k_diag_mfma_ceiling(aq.data_ptr(), wq.data_ptr(), M, N, K, K // 128, constant, md,
                                           out.data_ptr(), stream)
            if rc != 0:
                raise RuntimeError(f"m5k_diag_mfma_ceiling failed ({rc})")
        return run

    return {"mfma_ceiling_16x16x64": launcher(16, 0), "mfma_ceiling_16x16x64_constant": launcher(16, 1),
            "mfma_ceiling_32x32x32": launcher(32, 0), "mfma_ceiling_16x16x64_one_wave_per_simd": launcher(4, 0)}


def mfma_ceiling(torch, dev, rounds=8, reps=10):
    """--mfma-ceiling: the FFN-down INT8 GEMM beside the MFMA-only ceiling kernels on its own codes
    (ceiling_kernels), ABBA rounds of `reps` launches between one event pair after a 0.4 s clock
    settle; medians.  gemm_frac_of_ceiling = ceiling time / GEMM time."""
    from m5kernels_amd import gemm, quantize

    a, w = make_inputs(torch, dev)
    wq, ws = quantize(w, "int8")
    aq, sa = quantize(a, "int8")
    del a, w
    fns = {"gemm_i8": lambda: gemm(aq, wq, "int8", a_scales=sa, b_scales=ws, output_dtype=torch.bfloat16)}
    fns.update(ceiling_kernels(torch, dev, aq, wq))
    settle(torch, fns["gemm_i8"], 0.4)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    times = {key: [] for key in fns}
    names = list(fns)
    for r in range(rounds):
        for key in names if r % 2 == 0 else names[::-1]:
            e0.record()
            for _ in range(reps):
                fns[key]()
            e1.record()
            torch.cuda.synchronize()
            times[key].append(e0.elapsed_time(e1) / reps)
    ops = 2.0 * M * N * K
    res = {"workload": "ffn_down_w8a8 codes (bench inputs)", "m": M, "n": N, "k": K, "rounds": rounds, "reps": reps}
    for key, v in times.items():
        ms = statistics.median(v)
        tops = ops / (ms * 1e-3) / 1e12
        res[key] = {"us": ms * 1e3, "TOPS": tops, "frac_of_int8_peak": tops / PEAK_INT8_TOPS,
                    "p10_p90_us": [sorted(v)[len(v) // 10] * 1e3, sorted(v)[(9 * len(v)) // 10] * 1e3]}
        log(f"[bench] mfma ceiling: {key} {ms * 1e3:.1f} us = {tops:.0f} TOPS ({tops / PEAK_INT8_TOPS:.3f})")
    res["gemm_frac_of_ceiling"] = res["mfma_ceiling_16x16x64"]["us"] / res["gemm_i8"]["us"]
    res["quad_vs_eight_waves"] = quad_probe(torch, dev, aq, wq, sa, ws, rounds, reps)
    return res


def quad_probe(torch, dev, aq, wq, sa, ws, rounds, reps):
    """The four-wave grid (forced quad schedule: 128 x 128 per wave, one wave per SIMD) against the
    library's eight-wave launch on the FFN-down codes, FFN-up and 4096^3 (seeded INT8 codes):
    bit equality, then ABBA rounds of `reps` launches between one event pair, queued behind a
    short GPU spin; medians."""
    from m5kernels_amd import gemm
    from m5kernels_amd.hip import launch_override

    g = torch.Generator(device=dev).manual_seed(SEED)
    up_a = torch.randint(-127, 128, (4096, 4096), generator=g, device=dev, dtype=torch.int8)
    up_w = torch.randint(-127, 128, (16384, 4096), generator=g, device=dev, dtype=torch.int8)
    up_sa = torch.rand(4096, generator=g, device=dev) * 0.01 + 1e-3
    up_ws = torch.rand(16384, generator=g, device=dev) * 0.01 + 1e-3
    shapes = {"ffn_down_4096x4096x16384": (aq, wq, sa, ws), "ffn_up_4096x16384x4096": (up_a, up_w, up_sa, up_ws),
              "q_4096x4096x4096": (up_a, up_w[:4096], up_sa, up_ws[:4096])}
    out = {}
    for name, (a, w, s_a, s_w) in shapes.items():
        def run(quad, a=a, w=w, s_a=s_a, s_w=s_w):
            if quad:
                with launch_override("quad"):
                    return gemm(a, w, "int8", a_scales=s_a, b_scales=s_w, output_dtype=torch.bfloat16)
            with launch_override("plain"):
                return gemm(a, w, "int8", a_scales=s_a, b_scales=s_w, output_dtype=torch.bfloat16)

        same = bool(torch.equal(run(False).view(torch.int16), run(True).view(torch.int16)))
        settle(torch, lambda: run(False), 0.2)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        times = {False: [], True: []}
        for r in range(rounds):
            for quad in ((False, True) if r % 2 == 0 else (True, False)):
                torch.cuda._sleep(2_000_000)  # the host queues every launch before the first runs
                e0.record()
                for _ in range(reps):
                    run(quad)
                e1.record()
                torch.cuda.synchronize()
                times[quad].append(e0.elapsed_time(e1) / reps)
        eight, quad = statistics.median(times[False]) * 1e3, statistics.median(times[True]) * 1e3
        out[name] = {"bit_identical": same, "eight_waves_us": eight, "quad_us": quad, "quad_over_eight": quad / eight}
        log(f"[bench] quad vs eight waves: {name} {eight:.1f} / {quad:.1f} us (x{quad / eight:.3f}), "
            f"bit-identical {same}")
    return out


# Traffic mixes of the row kernels for hbm_ceiling: (name, rows, K, inputs, full-size output).
# Every mix writes the INT8 codes (half the BF16 input's bytes).
STREAM_MIXES = (
    ("quantize_ffn_down", M, K, 1, False),      # A bf16 -> codes
    ("prep_ungated_m4096", 4096, 4096, 1, False),  # X -> codes
    ("prep_gated_m4096", 4096, 4096, 2, True),     # X, branch -> R_next, codes
    ("prep_gated_m9914", 9914, 4096, 2, True),
)


STREAM_POLICIES = ("plain", "nt_stores", "nt_loads_stores")


def hbm_ceiling(torch, dev, grid_blocks=2048):
    """--hbm-ceiling: the HBM rate of each row kernel's read/write mix with no compute
    (libm5k_diag.so's stream_mix: 16-byte loads, one XOR, 16- and 8-byte stores), timed like the
    row kernels: time_op on one repeated input set and time_streaming over independent sets,
    for each cache policy of STREAM_POLICIES; the top-level figures are the fastest policy's.
    The row kernels' parameter tables and per-row scales (under 3% of their bytes) are left out."""
    import ctypes

    lib = _diag_lib()
    res = {"grid_blocks": grid_blocks}

    def launcher(x, b, full, half, policy=0):
        def run():
            stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
            rc = lib.m5k_diag_stream_mix(x.data_ptr(), None if b is None else b.data_ptr(),
                                         None if full is None else full.data_ptr(), half.data_ptr(), x.numel() // 8,
                                         grid_blocks, policy, stream)
            if rc != 0:
                raise RuntimeError(f"m5k_diag_stream_mix failed ({rc})")
        return run

    for name, rows, k, n_in, full_out in STREAM_MIXES:
        nbytes = rows * k * (2 * n_in + (2 if full_out else 0) + 1)

        def make_set():
            x = torch.randint(-2**15, 2**15, (rows, k), dtype=torch.int16, device=dev).view(torch.bfloat16)
            b = torch.randint(-2**15, 2**15, (rows, k), dtype=torch.int16, device=dev).view(torch.bfloat16) \
                if n_in == 2 else None
            full = torch.empty((rows, k), dtype=torch.bfloat16, device=dev) if full_out else None
            half = torch.empty((rows, k), dtype=torch.int8, device=dev)
            return x, b, full, half

        s0 = make_set()
        x, b, full, half = s0
        xw = x.view(torch.int16).view(-1, 8)
        bw = b.view(torch.int16).view(-1, 8) if b is not None else torch.zeros_like(xw)
        r = xw ^ bw
        r32 = r.view(torch.int32)
        h = torch.stack([r32[:, 0] ^ r32[:, 1], r32[:, 2] ^ r32[:, 3]], 1)
        for policy in range(len(STREAM_POLICIES)):
            if full is not None:
                full.zero_()
            half.zero_()
            launcher(*s0, policy)()
            torch.cuda.synchronize()
            if full is not None:
                assert torch.equal(full.view(torch.int16).view(-1, 8), r), (name, policy)
            assert torch.equal(half.view(torch.int32).view(-1, 2), h), (name, policy)
        del xw, bw, r, r32, h
        n = _sets_for(nbytes)
        sets = [s0] + [make_set() for _ in range(n - 1)]
        gbs = lambda t: nbytes / (t * 1e-3) / 1e9  # noqa: E731
        entry = {"bytes": nbytes, "streaming_input_sets": n, "policies": {}}
        for policy, pname in enumerate(STREAM_POLICIES):
            one = time_op(torch, launcher(*s0, policy))["avg_ms"]
            st = time_streaming(torch, [launcher(*st_, policy) for st_ in sets])
            entry["policies"][pname] = {"one_set_us": one * 1e3, "streaming_us": st * 1e3}
            log(f"[bench] hbm ceiling: {name} {pname} {nbytes / 1e6:.1f} MB one set {one * 1e3:.1f} us "
                f"({gbs(one) / PEAK_HBM_GBS:.3f}), streaming {st * 1e3:.1f} us ({gbs(st) / PEAK_HBM_GBS:.3f})")
        del sets, s0, x, b, full, half
        one = min(v["one_set_us"] for v in entry["policies"].values()) * 1e-3
        st = min(v["streaming_us"] for v in entry["policies"].values()) * 1e-3
        entry.update({"one_set_us": one * 1e3, "one_set_GBps": gbs(one), "one_set_frac_of_hbm_peak": gbs(one) / PEAK_HBM_GBS,
                      "streaming_us": st * 1e3, "streaming_GBps": gbs(st),
                      "streaming_frac_of_hbm_peak": gbs(st) / PEAK_HBM_GBS})
        res[name] = entry
    return res


def counter_workload(torch, dev, reps):
    """The kernels whose hardware counters the profiles quote, `reps` launches each after a
    clock-settling run, in this order: the FFN-down INT8 GEMM (ours), the same GEMM on constant
    codes, hipBLASLt's INT8 GEMM (torch._int_mm) on the bench's codes, the FFN-down FP8 GEMM,
    the INT8 and FP8 quantizers on
    the FFN-down activation, the MFMA ceiling kernels on the same codes (ceiling_kernels), the fused
    gated and ungated prep (M 4096, K 4096, H128) and the
    RMS quantizer (M 4096, K 4096, H256).  For rocprofv3 --pmc runs; prints nothing else."""
    from m5kernels_amd import (fused_gated_residual_norm_hadamard_quantize, fused_norm_hadamard_quantize, gemm,
                               quantize, rms_quantize)

    a, w = make_inputs(torch, dev)
    wq, ws = quantize(w, "int8")
    aq, sa = quantize(a, "int8")
    w8, ws8 = quantize(w, "fp8")
    a8, sa8 = quantize(a, "fp8")
    wq_t = wq.t()
    bf = torch.bfloat16
    ours = lambda: gemm(aq, wq, "int8", a_scales=sa, b_scales=ws, output_dtype=bf)  # noqa: E731
    settle(torch, ours, 0.3)
    # The same kernel on constant codes (every A and W code 1): identical instruction stream and
    # memory traffic, with the MFMA array's data switching removed, to expose the power limit.
    ones_a, ones_w = torch.ones_like(aq), torch.ones_like(wq)
    runs = [
        ("gemm_i8", ours),
        ("gemm_i8_constant_codes", lambda: gemm(ones_a, ones_w, "int8", a_scales=sa, b_scales=ws, output_dtype=bf)),
        ("hipblaslt_int_mm", lambda: torch._int_mm(aq, wq_t)),
        ("gemm_f8", lambda: gemm(a8, w8, "fp8", a_scales=sa8, b_scales=ws8, output_dtype=bf)),
        ("quantize_int8", lambda: quantize(a, "int8")),
        ("quantize_fp8", lambda: quantize(a, "fp8")),
    ]
    runs += list(ceiling_kernels(torch, dev, aq, wq).items())
    g = torch.Generator(device=dev).manual_seed(SEED)
    m, k, tables = 4096, 4096, 2
    res = torch.randn((m, k), generator=g, device=dev).to(bf)
    branch = torch.randn((m, k), generator=g, device=dev).to(bf)
    gate, scale, shift = ((torch.randn((tables, k), generator=g, device=dev) * 0.1).to(bf) for _ in range(3))
    gamma = (1 + 0.1 * torch.randn((k,), generator=g, device=dev)).to(bf)
    row_map = (torch.arange(m, device=dev, dtype=torch.int32) * tables // m).to(torch.int32)
    signs = torch.ones(k, dtype=torch.int8, device=dev)
    kw = dict(norm="layer", epsilon=1e-5, round_output="input", row_map=row_map)
    gamma32 = gamma.float()
    runs += [
        ("prep_gated", lambda: fused_gated_residual_norm_hadamard_quantize(
            res, branch, gate, gamma, scale, shift, signs, 128, gate_row_map=row_map, **kw)),
        ("prep_ungated", lambda: fused_norm_hadamard_quantize(res, gamma, scale, shift, signs, 128, **kw)),
        ("rms_quantize", lambda: rms_quantize(res, gamma32, signs, 256)),
    ]
    for name, fn in runs:
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
        log(f"[bench] counter workload: {name} x{reps}")


def main():
    p = argparse.ArgumentParser(description=__doc__)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=200)
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="target CPU-baseline sample duration")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline (profiling runs)")
    p.add_argument("--no-torch", action="store_true", help="skip the BF16 torch baseline (profiling runs)")
    p.add_argument("--no-extras", action="store_true", help="skip the other configurations (profiling runs)")
    p.add_argument("--copy-probe", action="store_true",
                   help="only run a 256 MiB device copy x5 (calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    p.add_argument("--schedules", action="store_true",
                   help="only compare the library's GEMM schedules (mixed / narrow) with the plain launch")
    p.add_argument("--vs-hipblaslt", action="store_true",
                   help="only time the INT8 and FP8 GEMMs against hipBLASLt on five shapes")
    p.add_argument("--prep-mixed", type=int, default=0, metavar="REPS",
                   help="REPS mixed-dtype gated prep calls (one dispatch each), then their timing; prints nothing else")
    p.add_argument("--mfma-ceiling", action="store_true",
                   help="only time the FFN-down GEMM beside MFMA-only kernels on its own codes (the ceiling)")
    p.add_argument("--hbm-ceiling", action="store_true",
                   help="only time each row kernel's read/write mix with no compute (one set and streaming)")
    p.add_argument("--counter-workload", type=int, default=0, metavar="REPS",
                   help="only launch each profiled kernel REPS times (for rocprofv3 --pmc runs)")
    p.add_argument("--op-settle", type=float, default=OP_SETTLE_S,
                   help="device seconds each timed extra runs before timing (0 for counter runs)")
    p.add_argument("--settle-seconds", type=float, default=0.4,
                   help="minimum device time of the warmup, whatever --warmup says (clock ramp)")
    args = p.parse_args()
    _set_op_settle(args.op_settle)
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(
            "bench.py measures one MI355X: this build has no multi-GPU path (every box has one GPU); "
            "run with --gpus 1",
            file=sys.stderr,
        )
        sys.exit(2)

    import torch

    from m5kernels_amd import _lib, gemm, quantize

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_probe:
        src = torch.ones(128 * 1024 * 1024, dtype=torch.bfloat16, device=dev)  # 256 MiB
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("[bench] copied 256 MiB x5")
        return
    if args.mfma_ceiling:
        print(json.dumps({"mfma_ceiling": mfma_ceiling(torch, dev)}))
        return
    if args.prep_mixed:
        print(json.dumps({"prep_mixed": prep_mixed(torch, dev, args.prep_mixed)}))
        return
    if args.hbm_ceiling:
        print(json.dumps({"hbm_ceiling": hbm_ceiling(torch, dev)}))
        return
    if args.counter_workload:
        counter_workload(torch, dev, args.counter_workload)
        return
    if args.vs_hipblaslt:
        print(json.dumps({"vs_hipblaslt": vendor_probe(torch, dev)}))
        return
    if args.schedules:
        res = schedules_probe(torch, dev)
        print(json.dumps({"schedules": res}))
        if not all(r["bit_identical"] for r in res):
            sys.exit(1)
        return
    log(f"[bench] inputs: A bf16 [{M},{K}], W bf16 [{N},{K}], seed {SEED}")
    a, w = make_inputs(torch, dev)
    wq, ws = quantize(w, "int8")  # offline weight preparation, untimed
    torch.cuda.synchronize()

    def step():
        aq, sa = quantize(a, "int8")
        return gemm(aq, wq, "int8", a_scales=sa, b_scales=ws, output_dtype=torch.bfloat16)

    steps = args.steps
    # Timing events exist before the warmup: the first creation in a process costs tens of ms.
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    log(f"[bench] warmup {args.warmup} steps, then at least {args.settle_seconds} s of steps; timing {steps} steps")
    # Each step's output is released before the next step runs, as in the reference's timing loop
    # (engine.py:70-92: `y = fn()` builds a lazy MLX graph, dropping the previous output, before
    # mx.eval computes the new one).  Kept alive across the next step, the 32 MB output alternates
    # between two allocator blocks and the working set outgrows the 256 MB Infinity Cache: 12 us
    # more per step (rocprof: GEMM +8.5 us, quantizer +3.8 us).
    y = None
    for _ in range(args.warmup):
        y = None
        y = step()
    torch.cuda.synchronize()
    settle_steps = settle(torch, step, args.settle_seconds)  # ends synchronized
    t0 = time.perf_counter()
    start.record()
    for i in range(steps):
        y = None
        y = step()
    end.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    total_ms = start.elapsed_time(end)
    # Per-kernel durations without an event between the two kernels: any event packet there (even
    # one without a system fence, or hipExtLaunchKernel's own pair) slows the kernels it separates
    # (rocprofv3 kernel trace of the step, one box: quantizer 30.4 -> 31.7-33.2 us, GEMM 189.1 ->
    # 200.2-217.7 us).  The GEMM: K launches back to back on one set of codes, one event pair around
    # them; its average matches the GEMM's rocprof duration inside the step.  The quantizer's share
    # of the step is the step minus that average (the two kernels run back to back, no gap between
    # them in the kernel trace).  For reference, K quantizer launches cycling over independent
    # activation sets beyond the Infinity Cache, each output kept for a cycle, give its streaming rate.
    log(f"[bench] per-kernel passes, {steps} launches each")
    aq, sa = quantize(a, "int8")
    g0, g1 = FenceFreeEvent(), FenceFreeEvent()
    stream = torch.cuda.current_stream(dev)
    for _ in range(5):
        y = None
        y = gemm(aq, wq, "int8", a_scales=sa, b_scales=ws, output_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    g0.record(stream)
    for _ in range(steps):
        y = None
        y = gemm(aq, wq, "int8", a_scales=sa, b_scales=ws, output_dtype=torch.bfloat16)
    g1.record(stream)
    torch.cuda.synchronize()
    gemm_avg = g0.elapsed_time(g1) / steps
    del aq, sa
    y = None
    n_sets = _sets_for(3 * M * K)
    a_sets = [a] + [torch.randn((M, K), device=dev).to(torch.bfloat16) for _ in range(n_sets - 1)]
    quant_streaming = time_streaming(torch, [lambda i=i: quantize(a_sets[i], "int8") for i in range(n_sets)],
                                     reps=steps)
    del a_sets
    host = []
    for _ in range(min(steps, 20)):  # synchronized host wall per step (the reference's measure)
        h0 = time.perf_counter()
        y = step()
        torch.cuda.synchronize()
        host.append((time.perf_counter() - h0) * 1e3)
    host.sort()
    ms_per_step = max(total_ms, wall_ms) / steps
    ops = 2.0 * M * N * K
    tops = ops / (ms_per_step * 1e-3) / 1e12
    gemm_tops = ops / (gemm_avg * 1e-3) / 1e12
    quant_avg = ms_per_step - gemm_avg
    quant_bytes = 2 * M * K + M * K + 4 * M
    quant_gbs = quant_bytes / (quant_avg * 1e-3) / 1e9
    log(f"[bench] step {ms_per_step:.4f} ms ({tops:.1f} TOPS); gemm {gemm_avg:.4f} ms ({gemm_tops:.1f} TOPS); "
        f"quant {quant_avg:.4f} ms ({quant_gbs:.0f} GB/s)")

    traffic = None
    quant_traffic = None
    if TRAFFIC_FILE.exists():  # scaled FETCH_SIZE + WRITE_SIZE per launch from the rocprofv3 --pmc runs
        measured = json.loads(TRAFFIC_FILE.read_text())
        traffic = measured.get("gemm_i8_ffn_down", {}).get("l2_miss_bytes_per_launch")
        quant_traffic = measured.get("quantize_rows_int8_ffn_down", {}).get("l2_miss_bytes_per_launch")

    result = {
        "metric": "W8A8 TOPS and ms at M=4096 FFN-down incl. online quant; % INT8 MFMA peak",
        "value": tops,
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "settle_steps": settle_steps,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded torch.randn on device; 0.1% activation channels x50)",
        "config": {
            "workload": "ffn_down_w8a8_online",
            "m": M,
            "k": K,
            "n": N,
            "seed": SEED,
            "activation_quant": "per-token symmetric INT8, online (timed)",
            "weight_quant": "per-output-channel symmetric INT8, offline (untimed)",
            "output": "bf16",
            "parallelism": "single GPU",
        },
        "pct_int8_mfma_peak_online": 100.0 * tops / PEAK_INT8_TOPS,
        "roofline": {
            "bound": "mfma",
            "kernel": "m5k_gemm_i8 (gemm_kernel<I8>)",
            "achieved": gemm_tops,
            "peak": PEAK_INT8_TOPS,
            "unit": "TFLOP/s",
            "unit_note": "integer ops (TOPS): 2*M*N*K per launch, dense INT8 MFMA peak 5.0 POP/s",
            "frac": gemm_tops / PEAK_INT8_TOPS,
            "traffic": traffic,
            "traffic_note": ("L2-miss bytes per launch (scaled FETCH_SIZE + WRITE_SIZE); the Infinity Cache serves "
                             "part of them, so HBM bytes are at most this"),
            "avg_launch_ms": gemm_avg,
        },
        "kernels": {
            "quantize_rows_int8": {
                "avg_ms": quant_avg,
                "avg_ms_method": "step minus the GEMM's back-to-back average",
                "streaming_ms": quant_streaming,
                "streaming_frac_of_hbm_peak": quant_bytes / (quant_streaming * 1e-3) / 1e9 / PEAK_HBM_GBS,
                "bound": "hbm",
                "bytes_per_launch": quant_bytes,
                "achieved_GBps": quant_gbs,
                "frac_of_hbm_peak": quant_gbs / PEAK_HBM_GBS,
                "traffic": quant_traffic,
            },
            "gemm_i8": {"avg_ms": gemm_avg, "achieved_TOPS": gemm_tops, "frac_of_int8_peak": gemm_tops / PEAK_INT8_TOPS},
        },
        "timing": {
            "event_total_ms": total_ms,
            "wall_ms": wall_ms,
            "method": ("after the warmup, K steps between one pair of HIP events on the launch stream; value uses "
                       "max(event, host wall).  Per-kernel averages, with no event between two kernels: the GEMM "
                       "from K back-to-back launches on one set of codes between one event pair; the quantizer as "
                       "the step minus that (kernels.quantize_rows_int8.streaming_ms: K launches cycling over "
                       "independent activation sets beyond the Infinity Cache)"),
            "quantizer_streaming_input_sets": n_sets,
            "host_sync_ms_per_step": {"median": host[len(host) // 2], "p10": host[len(host) // 10],
                                      "p90": host[(9 * len(host)) // 10]},
        },
    }

    if not args.no_torch:
        import torch.nn.functional as F

        # hipBLASLt INT8 GEMM on the same quantized operands (INT32 output, no scale epilogue),
        # interleaved with ours in rounds of 10 launches so both see the same clock state.
        wq_t = wq.t()
        aq, sa = quantize(a, "int8")
        ours_fn = lambda: gemm(aq, wq, "int8", a_scales=sa, b_scales=ws, output_dtype=torch.bfloat16)  # noqa: E731
        theirs_fn = lambda: torch._int_mm(aq, wq_t)  # noqa: E731
        for _ in range(20):
            theirs_fn()
        torch.cuda.synchronize()
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        rounds = {"ours": [], "hipblaslt": []}
        for r in range(6):
            for name, fn in ((("ours", ours_fn), ("hipblaslt", theirs_fn)) if r % 2 == 0
                             else (("hipblaslt", theirs_fn), ("ours", ours_fn))):
                s0.record()
                for _ in range(10):
                    fn()
                s1.record()
                torch.cuda.synchronize()
                rounds[name].append(s0.elapsed_time(s1) / 10)
        i8_ms = statistics.median(rounds["hipblaslt"])
        ours_ms = statistics.median(rounds["ours"])
        result["hipblaslt_int8_int_mm"] = {
            "ms": i8_ms, "TOPS": ops / (i8_ms * 1e-3) / 1e12, "m5k_gemm_ms_same_rounds": ours_ms,
            "m5k_gemm_speedup": i8_ms / ours_ms,
            "method": "6 alternating rounds of 10 launches each (ABBA order), medians",
        }
        for _ in range(20):
            F.linear(a, w)
        torch.cuda.synchronize()
        s0.record()
        for _ in range(50):
            F.linear(a, w)
        s1.record()
        torch.cuda.synchronize()
        bf16_ms = s0.elapsed_time(s1) / 50
        result["bf16_torch_linear"] = {"ms": bf16_ms, "TFLOPs": ops / (bf16_ms * 1e-3) / 1e12,
                                       "speedup_of_w8a8_online": bf16_ms / ms_per_step}

    if not args.no_extras:
        result["extras"] = extras(torch, dev)

    if not args.no_cpu:
        log("[bench] cpu baseline")
        result["cpu_baseline"] = cpu_baseline(torch, a, wq, ws, y, args.cpu_seconds)
        result["cpu_baseline"]["cpu_model"] = cpu_model()
        log("[bench] cpu baseline, NumPy variant")
        result["cpu_baseline"]["numpy_variant"] = numpy_baseline(torch, a, wq, ws, y, args.cpu_seconds / 2)

    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
