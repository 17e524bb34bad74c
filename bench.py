#!/usr/bin/env python3
"""W8A8 FFN-down on one MI355X, online activation quantization included.

Workload (the headline metric: FFN-down of the FFN up/down configuration): A bf16 [4096, 16384] ~N(0,1)
with 0.1% of channels (every 1024th) scaled x50, W bf16 [4096, 16384] ~N(0, 0.02), seed 29,
synthetic.  Offline (untimed): W -> per-output-channel INT8 codes + FP32 scales.  One step
= quantize(A) (per-token INT8) + W8A8 MFMA GEMM with the FP32 scale epilogue -> BF16 C.

Prints ONE JSON line: value = TOPS = 2*M*N*K / (ms per online step), the roofline of the
dominant kernel (the GEMM, dense INT8 MFMA peak), per-kernel HIP-event timings and the CPU
baseline (the oracle's C/OpenMP W8A8 on a bounded row sample, rank 0 only).
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


def main():
    p = argparse.ArgumentParser(description=__doc__)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="target CPU-baseline sample duration")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline (profiling runs)")
    p.add_argument("--no-torch", action="store_true", help="skip the BF16 torch baseline (profiling runs)")
    p.add_argument("--copy-probe", action="store_true",
                   help="only run a 256 MiB device copy x5 (calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = p.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(
            "bench.py measures one MI355X: this build has no multi-GPU path (every box has one GPU); "
            "run with --gpus 1",
            file=sys.stderr,
        )
        sys.exit(2)

    import torch

    from m5kernels_amd import gemm, quantize

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
    log(f"[bench] inputs: A bf16 [{M},{K}], W bf16 [{N},{K}], seed {SEED}")
    a, w = make_inputs(torch, dev)
    wq, ws = quantize(w, "int8")  # offline weight preparation, untimed
    torch.cuda.synchronize()

    def step():
        aq, sa = quantize(a, "int8")
        return gemm(aq, wq, "int8", a_scales=sa, b_scales=ws, output_dtype=torch.bfloat16)

    log(f"[bench] warmup {args.warmup}")
    for _ in range(args.warmup):
        y = step()
    torch.cuda.synchronize()

    steps = args.steps
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    log(f"[bench] timing {steps} steps")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for i in range(steps):
        ev[i][0].record()
        aq, sa = quantize(a, "int8")
        ev[i][1].record()
        y = gemm(aq, wq, "int8", a_scales=sa, b_scales=ws, output_dtype=torch.bfloat16)
        ev[i][2].record()
    end.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    total_ms = start.elapsed_time(end)
    quant_ms = [e[0].elapsed_time(e[1]) for e in ev]
    gemm_ms = [e[1].elapsed_time(e[2]) for e in ev]
    ms_per_step = max(total_ms, wall_ms) / steps
    ops = 2.0 * M * N * K
    tops = ops / (ms_per_step * 1e-3) / 1e12
    gemm_avg = statistics.fmean(gemm_ms)
    quant_avg = statistics.fmean(quant_ms)
    gemm_tops = ops / (gemm_avg * 1e-3) / 1e12
    quant_bytes = 2 * M * K + M * K + 4 * M
    quant_gbs = quant_bytes / (quant_avg * 1e-3) / 1e9
    log(f"[bench] step {ms_per_step:.4f} ms ({tops:.1f} TOPS); gemm {gemm_avg:.4f} ms ({gemm_tops:.1f} TOPS); "
        f"quant {quant_avg:.4f} ms ({quant_gbs:.0f} GB/s)")

    traffic = None
    quant_traffic = None
    if TRAFFIC_FILE.exists():  # scaled FETCH_SIZE + WRITE_SIZE per launch from the rocprofv3 --pmc runs
        measured = json.loads(TRAFFIC_FILE.read_text())
        traffic = measured.get("gemm_i8_ffn_down", {}).get("hbm_bytes_per_launch")
        quant_traffic = measured.get("quantize_rows_int8_ffn_down", {}).get("hbm_bytes_per_launch")

    result = {
        "metric": "W8A8 TOPS and ms at M=4096 FFN-down incl. online quant; % INT8 MFMA peak",
        "value": tops,
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
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
            "avg_launch_ms": gemm_avg,
        },
        "kernels": {
            "quantize_rows_int8": {
                "avg_ms": quant_avg,
                "bound": "hbm",
                "bytes_per_launch": quant_bytes,
                "achieved_GBps": quant_gbs,
                "frac_of_hbm_peak": quant_gbs / PEAK_HBM_GBS,
                "traffic": quant_traffic,
            },
            "gemm_i8": {"avg_ms": gemm_avg, "achieved_TOPS": gemm_tops, "frac_of_int8_peak": gemm_tops / PEAK_INT8_TOPS},
        },
        "timing": {"event_total_ms": total_ms, "wall_ms": wall_ms, "method": "HIP events on the launch stream"},
    }

    if not args.no_torch:
        import torch.nn.functional as F

        for _ in range(3):
            F.linear(a, w)
        torch.cuda.synchronize()
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record()
        for _ in range(10):
            F.linear(a, w)
        s1.record()
        torch.cuda.synchronize()
        bf16_ms = s0.elapsed_time(s1) / 10
        result["bf16_torch_linear"] = {"ms": bf16_ms, "TFLOPs": ops / (bf16_ms * 1e-3) / 1e12,
                                       "speedup_of_w8a8_online": bf16_ms / ms_per_step}
        # hipBLASLt INT8 GEMM on the same quantized operands (INT32 output, no scale epilogue).
        wq_t = wq.t()
        for _ in range(3):
            torch._int_mm(aq, wq_t)
        torch.cuda.synchronize()
        s0.record()
        for _ in range(10):
            torch._int_mm(aq, wq_t)
        s1.record()
        torch.cuda.synchronize()
        i8_ms = s0.elapsed_time(s1) / 10
        result["hipblaslt_int8_int_mm"] = {"ms": i8_ms, "TOPS": ops / (i8_ms * 1e-3) / 1e12,
                                           "m5k_gemm_speedup": i8_ms / gemm_avg}

    if not args.no_cpu:
        log("[bench] cpu baseline")
        result["cpu_baseline"] = cpu_baseline(torch, a, wq, ws, y, args.cpu_seconds)

    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
