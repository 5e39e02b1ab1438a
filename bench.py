#!/usr/bin/env python3
"""Benchmark of the lanternl MI355X backend on one GPU.

Default: times the hot path on synthetic data and prints ONE JSON line with the
metric of BASELINE.json, a `roofline` object for the dominant kernel (timed
live with hipEvents on the library stream) and a `cpu_baseline` object (the
CPU oracle -- a single-threaded C restatement of lanternl's pure-Lua loops --
timed on a bounded sample on this host).

  python bench.py [--steps K] [--warmup W] [--workload gemm4096]
  python bench.py --suite gemm       # config C5 sweep, one JSON line per shape

Only one GPU is used; --gpus above 1 exits with a message.
"""
import argparse
import ctypes
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_FP32_MFMA_TFLOPS = 157.3   # MI355X dense fp32 matrix, published
PEAK_HBM_GBPS = 8000.0          # MI355X HBM3E, published
METRIC = "fp32 GEMM TFLOP/s and % of MFMA peak; LMTrain steps/sec at 1 MI355X"


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def time_launches(fn, steps, warmup):
    """Average ms per call of fn() over `steps` back-to-back calls, bracketed by
    hipEvents recorded on the library stream (where fn enqueues its kernels)."""
    from lanternl_amd import device
    for _ in range(warmup):
        fn()
    device.sync()
    t = device.Timer()
    t.start()
    for _ in range(steps):
        fn()
    t.stop()
    device.sync()
    return t.ms() / steps


def bench_gemm(m, n, k, ta=False, tb=False, steps=20, warmup=3, seed=0):
    from lanternl_amd import device, kernels
    rng = np.random.default_rng(seed)
    a_shape = (k, m) if ta else (m, k)
    b_shape = (n, k) if tb else (k, n)
    A = device.Buffer.from_numpy(rng.uniform(-1, 1, a_shape).astype(np.float32))
    B = device.Buffer.from_numpy(rng.uniform(-1, 1, b_shape).astype(np.float32))
    C = device.Buffer((m, n))

    def run():
        kernels.sgemm(A, B, C, transa=ta, transb=tb)
    ms = time_launches(run, steps, warmup)
    flops = 2.0 * m * n * k
    tflops = flops / (ms * 1e-3) / 1e12
    return {"m": m, "n": n, "k": k, "op": ("T" if ta else "N") + ("T" if tb else "N"),
            "ms": ms, "tflops": tflops, "frac": tflops / PEAK_FP32_MFMA_TFLOPS,
            "bytes": 4.0 * (m * k + k * n + m * n)}


def cpu_baseline_gemm(n=512, reps=2):
    """The CPU oracle's matrix.lua `mm` loop order (double, 1 thread), n^3."""
    import oracle as O
    rng = np.random.default_rng(0)
    a = rng.uniform(-1, 1, (n, n)).astype(np.float32).astype(np.float64)
    b = rng.uniform(-1, 1, (n, n)).astype(np.float32).astype(np.float64)
    O.mm(a, b)
    t0 = time.perf_counter()
    for _ in range(reps):
        O.mm(a, b)
    dt = (time.perf_counter() - t0) / reps
    return {"value": 2.0 * n ** 3 / dt / 1e12, "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": f"{reps}x {n}^3 double GEMM, matrix.lua mm i-p-j order (C restatement, "
                      f"not LuaJIT), {_cpu_model()}"}


def run_gemm_workload(args):
    from lanternl_amd import device
    device.init(0)
    r = bench_gemm(4096, 4096, 4096, steps=args.steps, warmup=args.warmup)
    cpu = cpu_baseline_gemm()
    line = {
        "metric": METRIC, "value": r["tflops"], "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": r["ms"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic uniform[-1,1] seeded",
        "config": {"workload": "gemm_nn_4096^3 (config C5)", "m": 4096, "n": 4096, "k": 4096},
        "roofline": {"bound": "mfma", "achieved": r["tflops"], "peak": PEAK_FP32_MFMA_TFLOPS,
                     "unit": "TFLOP/s", "frac": r["frac"], "traffic": None},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def run_gemm_suite(args):
    from lanternl_amd import device
    device.init(0)
    cases = [(n, n, n, False, False) for n in (1024, 2048, 4096, 8192)]
    cases += [(m, 4096, 4096, False, False) for m in (1, 16, 64)]
    cases += [(4096, 4096, 4096, True, False), (4096, 4096, 4096, False, True)]
    cases += [(256, 256, 128, False, False), (256, 256, 128, True, False), (256, 256, 128, False, True)]
    for m, n, k, ta, tb in cases:
        steps = max(3, min(args.steps, int(2e12 / (2.0 * m * n * k)) + 3))
        r = bench_gemm(m, n, k, ta, tb, steps=steps, warmup=args.warmup)
        if m < 128:
            r["hbm_gbps"] = r["bytes"] / (r["ms"] * 1e-3) / 1e9
        print(json.dumps({"suite": "gemm", **r}), flush=True)


def main():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--workload", default="gemm4096", choices=["gemm4096"])
    p.add_argument("--suite", default=None, choices=["gemm"])
    args = p.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py: this build measures ONE GPU only (asked for {args.gpus}); "
              "the multi-GPU path is a design (see the sharding notes), not a measured run.",
              file=sys.stderr, flush=True)
        sys.exit(2)
    if args.suite == "gemm":
        run_gemm_suite(args)
    else:
        run_gemm_workload(args)


if __name__ == "__main__":
    main()
