#!/usr/bin/env python3
"""Benchmark of the lanternl MI355X backend on one GPU.

Default workload ("C2"): one full LMTrain step --
forward, cross-entropy, backward and the SGD update -- for vocab 2000, dim 128,
4 layers, 8 heads, ffn 256, 8 windows x 64 tokens, resident on the GPU,
launched eagerly on the library stream (`--graph`: replayed from a captured
hipGraph instead).  Prints ONE JSON line: steps/s, a `roofline` object
for the step's dominant kernel (timed live on the library stream with the
library's kernel timer), a `gemm4096` object (the 4096^3 NN GEMM measured in the same run),
a `gemm_shapes` object (the GEMM suite's other C1/C3/C5 shapes, same run),
a `bandwidth` object (the C3/C4 bandwidth kernels measured in the same run)
and a `cpu_baseline` object (the CPU oracle -- a single-threaded C
restatement of lanternl's pure-Lua loops in double -- timed on this host).
Kernel times (`kernel_ms`, `ms`) are dispatch start-to-end, as a kernel trace
reports them; `*_events` figures are hipEvents around back-to-back launches.

  python bench.py [--steps K] [--warmup W]
  python bench.py --workload gemm4096      # the 4096^3 fp32 GEMM (C5) instead
  python bench.py --workload dh2           # only the step's dominant kernel (counter passes)
  python bench.py --suite gemm             # C1/C3/C5 GEMM shapes, one JSON line each
  python bench.py --suite bandwidth        # C3/C4 bandwidth kernels, one JSON line each
  python bench.py --suite copy             # plain streaming kernel of known bytes (counter calibration)
  python bench.py --suite cpu              # CPU baselines: C1, C3, C4 and C5 1024^3 on the oracle (no GPU)

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
C2 = dict(vocab=2000, dim=128, layers=4, heads=8, ffn=256, batch=8, seq=64)
MALL_BYTES = 256 << 20          # Infinity Cache: rotate working sets past it


def _lscpu():
    """Host CPU facts from lscpu: model name and total core count (sockets x
    cores per socket) with the logical CPU count."""
    import subprocess
    info = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if ":" in line:
                k, v = line.split(":", 1)
                info[k.strip()] = v.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        cores = int(info.get("Socket(s)", "0")) * int(info.get("Core(s) per socket", "0"))
    except ValueError:
        cores = 0
    return {"model": info.get("Model name", _cpu_model()), "cores": cores or None,
            "logical_cpus": int(info["CPU(s)"]) if info.get("CPU(s)", "").isdigit() else os.cpu_count()}


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


SETTLE_MS = 30.0                # back-to-back GPU time before a per-call measurement (time_launches)


def time_launches(fn, steps, warmup, recorded=False, settle_ms=0.0):
    """Average ms per call of fn(i) over `steps` back-to-back calls, bracketed by
    hipEvents recorded on the library stream (where fn enqueues its kernels).

    recorded=True: after the eager warm-up (at least one call, which also sizes
    the library workspace), the `steps` calls are recorded once as a program
    (lhip_program_begin/end) and the timed region is one replay of it, so the
    kernels run back to back on the device with no Python or host launch cost
    between them.  fn must then only enqueue work.

    settle_ms (recorded only): before the timed replay, launch the calls
    eagerly until at least this much back-to-back GPU time has run.  The
    GPU's clocks follow its recent load, so without it the timed replay and a
    per-call measurement right after it (kernel_ms) would depend on `steps`:
    1024^3 NN read 26.3 us per call after a 20-call replay, 24.1-24.7 us after
    10 ms of back-to-back calls and 23.0-23.3 us after 30, 60 or 100 ms (the
    C3 logits product 53-55, 49-50 and 46.2 us), from the first call on."""
    from lanternl_amd import device
    for i in range(max(warmup, 1 if recorded else 0)):
        fn(i)
    device.sync()
    t = device.Timer()
    if recorded:
        prog = device.Program.record(lambda: [fn(i) for i in range(steps)])
        prog.replay()            # first replay uploads the graph
        device.sync()
        # the settling calls are eager launches, not replays: thousands of
        # graph launches under rocprofv3 --kernel-trace ended in a host
        # SIGSEGV inside hipGraphLaunch, where two replays per case never had
        busy = 0.0
        for _ in range(100000):
            if busy >= settle_ms:
                break
            t.start()
            for i in range(steps):
                fn(i)
            t.stop()
            device.sync()
            busy += t.ms()
        t.start()
        prog.replay()
        t.stop()
        device.sync()
        prog.free()
        return t.ms() / steps
    t.start()
    for i in range(steps):
        fn(i)
    t.stop()
    device.sync()
    return t.ms() / steps


def kernel_ms(fn, calls, warmup=1):
    """Kernel time per call of fn(i) the way a kernel trace (rocprofv3
    --kernel-trace) reports it: the library's kernel timer records each
    dispatch's start and end timestamps (lhip_ktimer_*), and a call's time is
    the sum over the kernels it launched.  Launch gaps are not included.
    Returns (median ms per call, kernels per call)."""
    from lanternl_amd import device
    for i in range(warmup):
        fn(i)
    device.sync()
    per_call, kpc = [], None
    for i in range(calls):   # one call at a time: no launch waits behind another in the queue
        t = device.kernel_times(lambda: fn(i), capacity=64)
        if not t or (kpc is not None and len(t) != kpc):
            raise RuntimeError(f"kernel timer: call {i} timed {len(t)} dispatches")
        kpc = len(t)
        per_call.append(sum(t))
    # the median: a call that lands on a clock or power-state change is an outlier
    return float(np.median(per_call)), kpc


# Operand arena.  Every GEMM and bandwidth case carves its buffer sets from one
# device allocation made once per process, so no case allocates or frees
# device memory: freeing a case's sets (hundreds of MB) and allocating the
# next case's slowed that next case's first calls -- the first 20 calls of an
# in-place RoPE case right after the RMSNorm backward had freed its 528 MB of
# sets took 7.0 us each against 6.44 us from the 25th call on, whichever RoPE
# case came first, while a RoPE case after another RoPE case did not show it.
_ARENA = {"buf": None, "top": 0, "cls": None}
_ARENA_BYTES = 1 << 30          # the largest case (8192^3 GEMM, 3 x 256 MB) fits
_ARENA_ALIGN = 2 << 20          # each array starts on a 2 MB boundary, as hipMalloc places large ones


def arena_reset():
    """Make the whole arena free again: the previous case's arrays are dead."""
    from lanternl_amd import device
    if _ARENA["buf"] is None:
        _ARENA["buf"] = device.Buffer((_ARENA_BYTES // 4,))

        class ArenaBuffer(device.Buffer):
            """A device array inside the arena.  Same interface as Buffer; the
            arena owns the memory, so free() only drops the address."""

            def __init__(self, addr, shape, dtype):
                self.shape = tuple(int(s) for s in shape)
                self.dtype = np.dtype(dtype)
                self.size = int(np.prod(self.shape)) if self.shape else 1
                self.nbytes = self.size * self.dtype.itemsize
                self._p = ctypes.c_void_p(addr)

            def free(self):
                self._p = None
        _ARENA["cls"] = ArenaBuffer
    _ARENA["top"] = 0


def arena_take(shape, dtype=np.float32, host=None):
    """A device array of `shape` from the arena, filled from `host` if given."""
    shape = shape if isinstance(shape, tuple) else (shape,)
    nbytes = int(np.prod(shape)) * np.dtype(dtype).itemsize
    top = _ARENA["top"]
    if top + nbytes > _ARENA_BYTES:
        raise RuntimeError(f"bench arena: {top + nbytes} bytes needed, the arena holds {_ARENA_BYTES}")
    _ARENA["top"] = top + -(-max(nbytes, 4) // _ARENA_ALIGN) * _ARENA_ALIGN
    buf = _ARENA["cls"](_ARENA["buf"].ptr + top, shape, dtype)
    return buf.upload(host) if host is not None else buf


def xcd_traffic_floor(m, n, k, xcds=8):
    """Least bytes an m x n x k fp32 product moves between the XCDs' L2s and
    memory when each XCD computes a block of the output: an XCD taking 1/q of
    the rows and 1/p of the columns (p*q = xcds) fetches A/q and B/p, so A is
    fetched p times and B q times in all; C is written once."""
    a, b, c = 4 * m * k, 4 * n * k, 4 * m * n
    return min(p * a + (xcds // p) * b for p in (1, 2, 4, 8) if xcds % p == 0) + c


def profile_figure(name, key):
    """A figure recorded in a committed profile (profiles/<name>), on a line
    `key: value` (the profile says how and at which commit it was measured)."""
    import re
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None, f"profiles/{name} is missing"
    with open(path) as f:
        text = f.read()
    m = re.search(r"^" + re.escape(key) + r":\s*([0-9.]+)", text, re.M)
    c = re.search(r"^measured_at_commit:\s*(\w+)", text, re.M)
    if not m:
        return None, f"profiles/{name} has no `{key}:` line"
    return float(m.group(1)), f"profiles/{name}" + (f" (commit {c.group(1)})" if c else "")


# ----------------------------------------------------------------------- GEMM
def bench_gemm(m, n, k, ta=False, tb=False, steps=20, warmup=3, seed=0, rotate=False):
    """fp32 GEMM timed with the kernel timer (`ms`, the kernel-trace figure
    that `frac` uses) and with hipEvents around a recorded replay (`ms_events`).
    rotate=True cycles over enough operand sets that one pass exceeds twice the
    256 MB Infinity Cache, so an HBM-bound shape reads HBM, not the cache."""
    from lanternl_amd import device, kernels
    rng = np.random.default_rng(seed)
    a_shape = (k, m) if ta else (m, k)
    b_shape = (n, k) if tb else (k, n)
    nbytes = 4.0 * (m * k + k * n + m * n)
    nsets = max(1, -(-2 * MALL_BYTES // int(nbytes))) if rotate else 1
    arena_reset()
    sets = []
    for _ in range(nsets):
        A = arena_take(a_shape, host=rng.uniform(-1, 1, a_shape).astype(np.float32))
        B = arena_take(b_shape, host=rng.uniform(-1, 1, b_shape).astype(np.float32))
        sets.append((A, B, arena_take((m, n))))

    def run(i):
        A, B, C = sets[i % nsets]
        kernels.sgemm(A, B, C, transa=ta, transb=tb)
    # one call on every set before timing (a fresh set's first use pays its
    # address translations; a shorter warm-up left that in the timed calls)
    for i in range(nsets):
        run(i)
    ms_events = time_launches(run, steps, warmup, recorded=True, settle_ms=SETTLE_MS)
    ms, kpc = kernel_ms(run, steps)
    flops = 2.0 * m * n * k
    tflops = flops / (ms * 1e-3) / 1e12
    return {"m": m, "n": n, "k": k, "op": ("T" if ta else "N") + ("T" if tb else "N"),
            "ms": ms, "ms_events": ms_events, "kernels_per_call": kpc, "tflops": tflops,
            "frac": tflops / PEAK_FP32_MFMA_TFLOPS, "bytes": nbytes, "buffer_sets": nsets}


def cpu_baseline_gemm(n=512, reps=4):
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
            "sample": f"{reps}x {n}^3 double GEMM in matrix.lua's mm loop order (C restatement of the "
                      f"Lua loop, not LuaJIT: LuaJIT is not installed), {_cpu_model()}"}


# ------------------------------------------------------------ LMTrain step (C2)
# The step's dominant kernel at C2 (largest share of kernel time in the
# rocprofv3 trace of this workload, profiles/lmtrain_c2_step.md): the
# batch-reduce NT GEMM of the backward, here in its dh2 form
# dh2 = dz1 . W1^T + du . W3^T, [B*T, ffn] x [ffn, dim] twice into one
# [B*T, dim] output.  It is timed alone, with the step's shapes and layout
# (the two gradients and the two weights adjacent), with hipEvents on the
# library stream it runs on.
# HBM bytes per launch come from that kernel's rocprofv3 FETCH_SIZE /
# WRITE_SIZE passes (scaled by the copy-kernel calibration), read from
# profiles/sgemm_batched_reduce_dh2.md.


def dominant_kernel_c2(steps, warmup):
    from lanternl_amd import device, kernels
    rng = np.random.default_rng(5)
    N, D, F = C2["batch"] * C2["seq"], C2["dim"], C2["ffn"]
    dzu = device.Buffer.from_numpy(rng.standard_normal((2, N, F)).astype(np.float32))
    w13 = device.Buffer.from_numpy((rng.standard_normal((2, D, F)) * 0.02).astype(np.float32))
    out = device.Buffer((N, D))

    def run(_):
        kernels.sgemm_batched_reduce(0, 1, N, D, F, 1.0, dzu.ptr, F, N * F, w13.ptr, F, D * F, 0.0, out.ptr, D, 2)
    calls = max(steps, 50)
    ms_events = time_launches(run, calls, warmup, recorded=True, settle_ms=SETTLE_MS)
    ms, kpc = kernel_ms(run, calls)
    flops = 2.0 * N * D * (2 * F)
    tflops = flops / (ms * 1e-3) / 1e12
    return {"ms": ms, "ms_events": ms_events, "kernels_per_call": kpc, "tflops": tflops,
            "frac": tflops / PEAK_FP32_MFMA_TFLOPS, "m": N, "n": D, "k": 2 * F, "flops": flops}


def dispatch_floor_ms(calls=50):
    """Kernel-timer duration of a kernel that does almost nothing (a one-
    workgroup fill of 16 bytes): the floor under every launch of the step."""
    from lanternl_amd import device
    from lanternl_amd._lib import call
    buf = device.Buffer((4,))
    ms, _ = kernel_ms(lambda _: call("lhip_zero", buf.ptr, 16), calls)
    buf.free()
    return ms


def cpu_baseline_lm(nsteps=5):
    import oracle as O
    cfg = O.lm_cfg(C2["vocab"], C2["dim"], C2["layers"], C2["heads"], C2["ffn"])
    rng = np.random.default_rng(0)
    n = O.lm_num_params(cfg)
    p = rng.normal(0, 0.02, n).astype(np.float32).astype(np.float64)
    v = np.zeros(n)
    ids = rng.integers(0, C2["vocab"], (C2["batch"], C2["seq"])).astype(np.int32)
    tgt = rng.integers(0, C2["vocab"], (C2["batch"], C2["seq"])).astype(np.int32)
    t0 = time.perf_counter()
    for _ in range(nsteps):
        O.lm_step_sgd(cfg, p, v, ids, tgt, 0.1)
    dt = (time.perf_counter() - t0) / nsteps
    host = _lscpu()
    return {"value": 1.0 / dt, "unit": "steps/s", "cores": 1, "kind": "port",
            "host_cpu": host["model"], "host_cores": host["cores"], "host_logical_cpus": host["logical_cpus"],
            "sample": f"{nsteps} full C2 LMTrain SGD steps (8 windows x 64 tokens, fwd+bwd+update) of the "
                      f"double-precision C restatement of the Lua CPU path (not LuaJIT: LuaJIT is not "
                      f"installed), single-threaded on 1 of the host's {host['cores']} cores "
                      f"({host['logical_cpus']} logical CPUs), {host['model']}"}


def run_lm_workload(args):
    from lanternl_amd import device, lmtrain
    device.init(0)
    rng = np.random.default_rng(0)
    gpu = lmtrain.GpuLMStep(**C2)
    gpu.set_params(lmtrain.init_params(gpu.cfg, rng, 0.02))
    gpu.set_batch(rng.integers(0, C2["vocab"], (C2["batch"], C2["seq"])),
                  rng.integers(0, C2["vocab"], (C2["batch"], C2["seq"])))
    gpu.use_graph(args.graph)

    def step(_):
        gpu.step(0.1, 0.9, 0.01, 1.0)
    ms = time_launches(step, args.steps, args.warmup)
    st = gpu.stats()
    if not np.isfinite(st["loss"]):
        raise RuntimeError(f"non-finite loss after the timed steps: {st}")
    dom = dominant_kernel_c2(args.steps, args.warmup)
    floor_ms = dispatch_floor_ms()
    dom_traffic, dom_src = profile_figure("sgemm_batched_reduce_dh2.md", "traffic_bytes_per_launch")
    xcd_floor = xcd_traffic_floor(dom["m"], dom["n"], dom["k"])
    g4 = gemm4096_object(args)
    flops = 3 * 1_000_341_504 * 1.0   # GEMM flops of one fwd+bwd step (forward x 3)
    line = {
        "metric": METRIC, "value": 1000.0 / ms, "unit": "steps/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: token ids/targets uniform in [0,2000), weights N(0,0.02), gains 1",
        "config": {"workload": "lmtrain_step_c2 (BASELINE configs[1]): one SGD step, fwd+CE+bwd+update",
                   **C2, "optimizer": "sgd(lr=0.1, momentum=0.9, wd=0.01, clip=1.0)",
                   "graph_replay": bool(args.graph), "streams": 1},
        "step_gemm_tflops": flops / (ms * 1e-3) / 1e12,
        "last_step": {"loss": st["loss"], "grad_norm": st["grad_norm"], "applied": st["applied"]},
        "roofline": {"bound": "mfma", "achieved": dom["tflops"], "peak": PEAK_FP32_MFMA_TFLOPS,
                     "unit": "TFLOP/s", "frac": dom["frac"], "traffic": dom_traffic,
                     "traffic_source": dom_src,
                     "traffic_floor_8xcd": xcd_floor,
                     "traffic_floor_method": "least L2-miss bytes any placement of the output tiles over the "
                                             "8 XCDs (each with its own L2) can reach: min over p*q = 8 of "
                                             "p*A + q*B + C, an XCD taking 1/q of the rows and 1/p of the "
                                             "columns; algorithmic bytes assume one shared cache",
                     "kernel": f"batch-reduce sgemm NT {dom['m']}x{dom['n']}x(2x{dom['k'] // 2}) "
                               f"(dh2 = dz1 . W1^T + du . W3^T), {dom['flops']:.0f} flop per launch",
                     "kernel_ms": dom["ms"], "kernel_ms_events": dom["ms_events"],
                     "dispatch_floor_ms": floor_ms,
                     "dispatch_floor_method": "the same kernel timer on a one-workgroup fill of 16 bytes "
                                              "(lhip_zero), launched alone: what any kernel costs on this "
                                              "timer before it does work",
                     "kernel_ms_method": "kernel_ms: median over calls of the dispatch start-to-end timestamps "
                                         "(library kernel timer), as rocprofv3 --kernel-trace reports them; "
                                         "kernel_ms_events: hipEvents around a recorded replay of back-to-back "
                                         "launches (includes launch gaps)"},
        "gemm4096": g4,
        "gemm_shapes": gemm_shapes_object(args),
        "bandwidth": bandwidth_object(args),
        "cpu_baseline": cpu_baseline_lm(),
    }
    gpu.close()
    print(json.dumps(line), flush=True)


def gemm4096_object(args):
    """NN 4096^3 (config C5) in the same run: kernel-trace time, TFLOP/s and
    fraction of the fp32 MFMA peak; HBM bytes per launch from the committed
    FETCH_SIZE / WRITE_SIZE passes (profiles/sgemm_nn_4096.md)."""
    r = bench_gemm(4096, 4096, 4096, steps=min(max(args.steps, 5), 20), warmup=min(args.warmup, 3) or 1)
    traffic, src = profile_figure("sgemm_nn_4096.md", "traffic_bytes_per_launch")
    return {"op": "NN", "m": 4096, "n": 4096, "k": 4096, "ms": r["ms"], "ms_events": r["ms_events"],
            "tflops": r["tflops"], "frac": r["frac"], "peak": PEAK_FP32_MFMA_TFLOPS, "traffic": traffic,
            "traffic_source": src}


def run_gemm_workload(args):
    from lanternl_amd import device
    device.init(0)
    r = bench_gemm(4096, 4096, 4096, steps=args.steps, warmup=args.warmup)
    traffic, src = profile_figure("sgemm_nn_4096.md", "traffic_bytes_per_launch")
    line = {
        "metric": METRIC, "value": r["tflops"], "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": r["ms"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic uniform[-1,1] seeded",
        "config": {"workload": "gemm_nn_4096^3 (config C5)", "m": 4096, "n": 4096, "k": 4096},
        "roofline": {"bound": "mfma", "achieved": r["tflops"], "peak": PEAK_FP32_MFMA_TFLOPS,
                     "unit": "TFLOP/s", "frac": r["frac"], "traffic": traffic, "traffic_source": src,
                     "kernel_ms": r["ms"], "kernel_ms_events": r["ms_events"]},
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline_gemm()
    print(json.dumps(line), flush=True)


def pcie_rates(nbytes=64 << 20, reps=10):
    """Pinned-host <-> device copy rates (GB/s) on this box, through the HIP
    runtime directly: the floor of the host-table path's transfers."""
    hip = ctypes.CDLL("libamdhip64.so")
    h, d = ctypes.c_void_p(), ctypes.c_void_p()
    if hip.hipHostMalloc(ctypes.byref(h), ctypes.c_size_t(nbytes), 0) or hip.hipMalloc(ctypes.byref(d),
                                                                                       ctypes.c_size_t(nbytes)):
        raise RuntimeError("pcie_rates: allocation failed")
    out = {}
    try:
        for name, dst, src, kind in (("h2d", d, h, 1), ("d2h", h, d, 2)):
            for _ in range(2):
                hip.hipMemcpy(dst, src, ctypes.c_size_t(nbytes), kind)
            t0 = time.perf_counter()
            for _ in range(reps):
                hip.hipMemcpy(dst, src, ctypes.c_size_t(nbytes), kind)
            out[name] = nbytes * reps / (time.perf_counter() - t0) / 1e9
    finally:
        hip.hipFree(d)
        hip.hipHostFree(h)
    return out


def bench_host_gemm(m, k, n, op=0, reps=20, rates=None, gemm_ms=None):
    """lhip_matmul_host (the flat-table adapter contract, luatl_adapter.lua:128-135):
    double host arrays in, fp32 conversion, upload, GEMM, download, double host
    array out, synchronous -- timed with the host clock around whole calls.
    This is the PCIe-inclusive rate of the boundary; it is never `value`."""
    from lanternl_amd._lib import call
    rng = np.random.default_rng(0)
    a = rng.uniform(-1, 1, m * k)
    nb = k * n if op == 0 else (n * k if op == 1 else m * n)
    b = rng.uniform(-1, 1, nb)
    rows = k if op == 2 else m
    c = np.empty(rows * n)
    args = (op, a.ctypes.data, b.ctypes.data, c.ctypes.data, m, k, n, 0)
    call("lhip_matmul_host", *args)
    t0 = time.perf_counter()
    for _ in range(reps):
        call("lhip_matmul_host", *args)
    dt = (time.perf_counter() - t0) / reps
    nbytes = 8.0 * (m * k + nb + rows * n)
    r = {"suite": "gemm_host", "op": ["NN", "NT", "TN"][op], "m": m, "k": k, "n": n, "ms": dt * 1e3,
         "tflops": 2.0 * m * k * n / dt / 1e12, "host_bytes": nbytes, "host_gbps": nbytes / dt / 1e9}
    if rates:
        # the fp32 bytes that must cross PCIe (A and B up, C down) at the pinned rates
        floor = 4.0 * (m * k + nb) / (rates["h2d"] * 1e9) + 4.0 * rows * n / (rates["d2h"] * 1e9)
        r["pcie_floor_ms"] = floor * 1e3
        if gemm_ms is not None:
            r["gemm_ms"] = gemm_ms
            r["vs_floor_plus_gemm"] = r["ms"] / (r["pcie_floor_ms"] + gemm_ms)
    return r


def bench_host_spin(m=256, k=128, n=256, reps=200, gap_us=200.0):
    """The C1 host-table call with the conversion workers spinning between
    calls (lhip_set_host_spin 1000 us, the default) and sleeping at once (0),
    back to back and with `gap_us` of single-threaded host work between calls
    (a LuaJIT host's own work).  Reports the call's wall time and the process
    CPU time it costs per call (all threads; the gap's own work excluded)."""
    import ctypes as ct
    from lanternl_amd._lib import call
    rng = np.random.default_rng(1)
    a, b = rng.uniform(-1, 1, m * k), rng.uniform(-1, 1, k * n)
    c = np.empty(m * n)
    args_ = (0, a.ctypes.data, b.ctypes.data, c.ctypes.data, m, k, n, 0)
    prev = ct.c_int()
    call("lhip_set_host_spin", 1000, ct.byref(prev))

    def gap():
        t_end = time.perf_counter() + gap_us * 1e-6
        while time.perf_counter() < t_end:
            pass
    out = []
    try:
        for spin in (1000, 0):
            call("lhip_set_host_spin", spin, None)
            for with_gap in (False, True):
                for _ in range(5):
                    call("lhip_matmul_host", *args_)
                wall, cpu0, g_cpu = 0.0, time.process_time(), 0.0
                for _ in range(reps):
                    if with_gap:
                        g0 = time.thread_time()          # the calling thread's own work only
                        gap()
                        g_cpu += time.thread_time() - g0
                    t0 = time.perf_counter()
                    call("lhip_matmul_host", *args_)
                    wall += time.perf_counter() - t0
                cpu = time.process_time() - cpu0 - g_cpu
                out.append({"suite": "gemm_host_spin", "op": "NN", "m": m, "k": k, "n": n, "spin_us": spin,
                            "host_work_between_calls_us": gap_us if with_gap else 0.0,
                            "ms": wall / reps * 1e3, "cpu_ms_per_call": cpu / reps * 1e3,
                            "note": "cpu_ms_per_call: process CPU time (every thread) per call, the calling "
                                    "thread's host work between calls excluded (workers spinning through the "
                                    "gaps are counted)"})
    finally:
        call("lhip_set_host_spin", prev.value, None)
    return out


def gemm_cases(big=True):
    """The GEMM suite's shapes (m, n, k, transa, transb): C5 squares (8192^3
    with `big`), skinny M against a 4096x4096 operand, 4096^3 transposed,
    C1 and the C3 LM-head products."""
    cases = [(n, n, n, False, False) for n in ((1024, 2048, 4096, 8192) if big else (1024, 2048))]
    cases += [(m, 4096, 4096, False, False) for m in (1, 16, 64)]
    cases += [(4096, 4096, 4096, True, False), (4096, 4096, 4096, False, True)]
    cases += [(256, 256, 128, False, False), (256, 256, 128, True, False), (256, 256, 128, False, True)]
    # C3: LM head logits, dW (A^T.B) and dhidden (A.B^T)
    cases += [(512, 32000, 128, False, False), (128, 32000, 512, True, False), (512, 128, 32000, False, True)]
    return cases


def bench_gemm_case(m, n, k, ta, tb, steps, warmup):
    """bench_gemm with the suite's call count (fewer calls for the long
    products) and operand rotation for the HBM-bound shapes (skinny M, C3's
    32000-wide operands), plus the algorithmic HBM rate."""
    steps = max(5, min(steps, int(4e12 / (2.0 * m * n * k)) + 5))
    hbm = m <= 64 or max(m, n, k) == 32000
    r = bench_gemm(m, n, k, ta, tb, steps=max(steps, 20) if hbm else steps, warmup=warmup, rotate=hbm)
    r["hbm_gbps_algorithmic"] = r["bytes"] / (r["ms"] * 1e-3) / 1e9
    r["hbm_frac"] = r["hbm_gbps_algorithmic"] / PEAK_HBM_GBPS
    return r


def gemm_shapes_object(args):
    """The GEMM suite's shapes other than 4096^3 NN (in `gemm4096`) and
    8192^3, measured in the default run with the suite's method: kernel-timer
    ms per call (every kernel the call launches), TFLOP/s and fraction of the
    fp32 MFMA peak, algorithmic HBM fraction."""
    t0 = time.perf_counter()
    out = {}
    for m, n, k, ta, tb in gemm_cases(big=False):
        r = bench_gemm_case(m, n, k, ta, tb, min(max(args.steps, 5), 20), min(args.warmup, 3) or 1)
        out[f"{m}x{n}x{k} {r['op']}"] = {"ms": round(r["ms"], 6), "tflops": round(r["tflops"], 2),
                                         "frac": round(r["frac"], 4), "hbm_frac": round(r["hbm_frac"], 4),
                                         "kernels_per_call": r["kernels_per_call"],
                                         "buffer_sets": r["buffer_sets"]}
    return {"peak_tflops": PEAK_FP32_MFMA_TFLOPS, "peak_gbps": PEAK_HBM_GBPS,
            "method": "kernel timer (dispatch start to end, median over calls each launched alone, summed over "
                      "the call's kernels, after at least 30 ms of back-to-back replays); operand sets rotated past the 256 MB Infinity Cache for M <= 64 and "
                      "the 32000-wide C3 products; hbm_frac = (A + B + C fp32 bytes) / ms / 8 TB/s",
            "seconds": round(time.perf_counter() - t0, 2), "shapes": out}


def run_gemm_suite(args):
    from lanternl_amd import device
    device.init(0)
    for m, n, k, ta, tb in gemm_cases():
        r = bench_gemm_case(m, n, k, ta, tb, args.steps, args.warmup)
        print(json.dumps({"suite": "gemm", **r}), flush=True)
    # the host-table boundary (PCIe and fp64 <-> fp32 conversions included),
    # against the PCIe floor of its fp32 bytes plus the device GEMM
    rates = pcie_rates()
    print(json.dumps({"suite": "pcie", "h2d_gbps": rates["h2d"], "d2h_gbps": rates["d2h"],
                      "bytes": 64 << 20, "memory": "pinned host"}), flush=True)
    dev = {}
    for m, k, n, op, reps in [(256, 128, 256, 0, 200), (256, 128, 256, 1, 200), (256, 128, 256, 2, 200),
                              (1024, 1024, 1024, 0, 20), (4096, 4096, 4096, 0, 5)]:
        key = (m, k, n, op)
        if key not in dev:
            ta, tb = op == 2, op == 1
            gm, gn, gk = (k, n, m) if op == 2 else (m, n, k)
            dev[key] = bench_gemm(gm, gn, gk, ta, tb, steps=10, warmup=2)["ms"]
        print(json.dumps(bench_host_gemm(m, k, n, op, reps, rates, dev[key])), flush=True)
    for r in bench_host_spin():
        print(json.dumps(r), flush=True)


# ------------------------------------------------------------ bandwidth kernels
def bench_bandwidth(name, nbytes, make_set, launch, steps, warmup, only=None):
    """Rotate over enough independent buffer sets that one pass over them
    exceeds the 256 MB Infinity Cache, so the timed traffic is HBM traffic.
    make_set(i) builds set i from the operand arena (arena_take)."""
    if only and only not in name:
        return None
    nsets = max(2, -(-2 * MALL_BYTES // int(nbytes)))
    arena_reset()
    sets = [make_set(i) for i in range(nsets)]

    def run(i):
        launch(sets[i % nsets])
    # one call on every set first: a set's first use pays its address
    # translations, which a warm-up over fewer calls than sets left inside
    # the timed calls
    for i in range(nsets):
        run(i)
    ms_events = time_launches(run, steps, warmup, recorded=True, settle_ms=SETTLE_MS)
    ms, kpc = kernel_ms(run, steps)
    gbps = nbytes / (ms * 1e-3) / 1e9
    return {"suite": "bandwidth", "kernel": name, "ms": ms, "ms_events": ms_events, "kernels_per_call": kpc,
            "bytes": nbytes, "gbps": gbps, "frac": gbps / PEAK_HBM_GBPS, "buffer_sets": nsets}


def bandwidth_cases(steps, warmup, only=None, references=True):
    """The C3/C4 bandwidth kernels (and, with `references`, the library's
    plainest streaming kernels at the same sizes and stream counts), each
    timed with bench_bandwidth; returns their result dicts.  Inputs are
    seeded N(0, 1)-shaped host arrays (one per shape, uploaded into every
    buffer set: the timing needs non-zero data, not distinct data)."""
    from lanternl_amd import device
    from lanternl_amd._lib import call
    device.init(0)
    rng = np.random.default_rng(0)
    B = device.Buffer
    T, Dm, Fm = 4096, 1024, 4096
    host = {}

    def host_arr(shape, scale, loc):
        key = (shape, scale, loc)
        if key not in host:
            host[key] = (rng.standard_normal(shape) * scale + loc).astype(np.float32)
        return host[key]

    def arr(*shape, scale=1.0, loc=0.0):   # a buffer set's input, in the arena
        return arena_take(shape, host=host_arr(shape, scale, loc))
    new = arena_take                       # a buffer set's output, in the arena

    out = []
    # RMSNorm 4096 x 1024 (eps 1e-6, gain N(1, 0.1))
    w = B.from_numpy(host_arr((Dm,), 0.1, 1.0))
    nb = 4 * (2 * T * Dm + Dm + T)
    out.append(bench_bandwidth("rmsnorm_fwd 4096x1024", nb,
                               lambda i: (arr(T, Dm), new((T, Dm)), new((T,))),
                               lambda s: call("lhip_rmsnorm_fwd", s[0].ptr, w.ptr, s[1].ptr, s[2].ptr, T, Dm, 1e-6),
                               steps, warmup, only))
    nb = 4 * (3 * T * Dm + 2 * Dm + T)
    inv = B.from_numpy(np.ones(T, np.float32))
    dw = B((Dm,))
    out.append(bench_bandwidth("rmsnorm_bwd 4096x1024", nb,
                               lambda i: (arr(T, Dm), arr(T, Dm, scale=0.5), new((T, Dm))),
                               lambda s: call("lhip_rmsnorm_bwd", s[0].ptr, w.ptr, inv.ptr, s[1].ptr, s[2].ptr,
                                              dw.ptr, T, Dm, 0),
                               steps, warmup, only))
    # RoPE 4096 tokens x 16 heads x 64, base 1e4, in place (fwd and inverse),
    # interleaved pairs (the CPU path's layout) and half-split pairs
    nb = 4 * 2 * T * 16 * 64
    for il in (1, 0):
        for inverse in (0, 1):
            out.append(bench_bandwidth(f"rope_{'bwd' if inverse else 'fwd'} 4096x16x64 "
                                       f"{'interleaved' if il else 'half-split'}", nb,
                                       lambda i: (arr(T, 16 * 64),),
                                       lambda s, inv_=inverse, il_=il: call("lhip_rope", s[0].ptr, None, T, 16, 64,
                                                                            16 * 64, 0, 0, 10000.0, il_, inv_),
                                       steps, warmup, only))
    # SwiGLU 4096 x 4096
    n = T * Fm
    out.append(bench_bandwidth("swiglu_fwd 4096x4096", 4 * 3 * n,
                               lambda i: (arr(T, Fm), arr(T, Fm, scale=0.5), new((T, Fm))),
                               lambda s: call("lhip_swiglu_fwd", s[0].ptr, Fm, s[1].ptr, Fm, s[2].ptr, Fm, T, Fm),
                               steps, warmup, only))
    out.append(bench_bandwidth("swiglu_bwd 4096x4096", 4 * 5 * n,
                               lambda i: (arr(T, Fm), arr(T, Fm, scale=0.5), arr(T, Fm, scale=0.25), new((T, Fm)),
                                          new((T, Fm))),
                               lambda s: call("lhip_swiglu_bwd", s[0].ptr, Fm, s[1].ptr, Fm, s[2].ptr, Fm, s[3].ptr,
                                              Fm, s[4].ptr, Fm, T, Fm, 0),
                               steps, warmup, only))
    # row softmax 4096 x 4096, scores N(0, 4) (sigma 2)
    out.append(bench_bandwidth("softmax_fwd 4096x4096", 4 * 2 * n,
                               lambda i: (arr(T, T, scale=2.0), new((T, T))),
                               lambda s: call("lhip_softmax_fwd", s[0].ptr, s[1].ptr, T, T, 1.0, 0, 0, 0),
                               steps, warmup, only))
    out.append(bench_bandwidth("softmax_bwd 4096x4096", 4 * 3 * n,
                               lambda i: (arr(T, T, scale=0.01, loc=1.0 / T), arr(T, T), new((T, T))),
                               lambda s: call("lhip_softmax_bwd", s[0].ptr, s[1].ptr, s[2].ptr, T, T, 1.0, 0, 0, 0, 0),
                               steps, warmup, only))
    # C3 fused softmax + CE: 512 x 32000 logits, labels uniform
    R, V = 512, 32000
    labels = B.from_numpy(rng.integers(0, V, R).astype(np.int32), np.int32)
    out.append(bench_bandwidth("ce_fused 512x32000", 4 * (2 * R * V + 2 * R),
                               lambda i: (arr(R, V), new((R, V)), new((R,))),
                               lambda s: call("lhip_ce_fused", s[0].ptr, labels.ptr, s[2].ptr, s[1].ptr, R, V, -1,
                                              1.0 / R),
                               steps, warmup, only))
    if references:
        # size-matched streaming references: what a kernel with no arithmetic
        # to speak of and the same number of read and written streams reaches
        for rows, cols in ((T, Dm), (T, Fm)):
            n = rows * cols
            out.append(bench_bandwidth(f"reference silu {rows}x{cols} (1 read + 1 write)", 4 * 2 * n,
                                       lambda i, r_=rows, c_=cols: (arr(r_, c_), new((r_ * c_,))),
                                       lambda s, n_=n: call("lhip_silu", s[0].ptr, s[1].ptr, n_),
                                       steps, warmup, only))
            out.append(bench_bandwidth(f"reference silu in place {rows}x{cols} (1 read + 1 write)", 4 * 2 * n,
                                       lambda i, r_=rows, c_=cols: (arr(r_, c_),),
                                       lambda s, n_=n: call("lhip_silu", s[0].ptr, s[0].ptr, n_),
                                       steps, warmup, only))
            out.append(bench_bandwidth(f"reference add {rows}x{cols} (2 reads + 1 write)", 4 * 3 * n,
                                       lambda i, r_=rows, c_=cols: (arr(r_, c_), arr(r_, c_, scale=0.5),
                                                                    new((r_ * c_,))),
                                       lambda s, n_=n: call("lhip_add", s[0].ptr, s[1].ptr, s[2].ptr, n_),
                                       steps, warmup, only))
    return [r for r in out if r is not None]


def bandwidth_object(args):
    """The C3/C4 bandwidth kernels measured in the default run: kernel-timer
    ms, GB/s and fraction of the 8 TB/s HBM peak per kernel (buffer sets
    rotated past the Infinity Cache), 20 timed calls each."""
    t0 = time.perf_counter()
    res = bandwidth_cases(steps=20, warmup=5, references=False)
    kernels = {r["kernel"]: {"ms": round(r["ms"], 6), "bytes": r["bytes"], "gbps": round(r["gbps"], 1),
                             "frac": round(r["frac"], 4), "kernels_per_call": r["kernels_per_call"]} for r in res}
    return {"peak_gbps": PEAK_HBM_GBPS, "method": "kernel timer (dispatch start to end, median of 20 calls each "
            "launched alone, after at least 30 ms of back-to-back replays), buffer sets rotated past the 256 MB Infinity Cache; bytes = each input read once "
            "plus each output written once (fp32)", "seconds": round(time.perf_counter() - t0, 2),
            "kernels": kernels}


def run_bandwidth_suite(args):
    for r in bandwidth_cases(max(args.steps, 20), args.warmup, args.only):
        print(json.dumps(r), flush=True)


def run_cpu_suite(args):
    """CPU baselines of the stand-in for the reference's pure-Lua path (the
    oracle: single-threaded C restatements of its loops in double; LuaJIT is
    not installed): C1's three GEMM variants, each C4 kernel, C3's fused CE and
    C5 1024^3, each a bounded sample timed on this host, one JSON line each."""
    import oracle as O
    host = _lscpu()
    rng = np.random.default_rng(0)

    def timed(fn, min_s=0.5, max_reps=50):
        fn()
        reps, t0 = 0, time.perf_counter()
        while True:
            fn()
            reps += 1
            dt = time.perf_counter() - t0
            if dt >= min_s or reps >= max_reps:
                return dt / reps, reps

    def line(case, dt, reps, value, unit, sample, gpu_ref):
        print(json.dumps({"suite": "cpu", "case": case, "value": value, "unit": unit, "s_per_call": dt,
                          "reps": reps, "cores": 1, "kind": "port", "sample": sample,
                          "host_cpu": host["model"], "host_cores": host["cores"],
                          "host_logical_cpus": host["logical_cpus"], "gpu_line": gpu_ref}), flush=True)

    u = lambda *sh: rng.uniform(-1, 1, sh)   # noqa: E731
    # C1: 256x128 . 128x256 and the transposed variants at matching shapes
    a, b, at, bt = u(256, 128), u(128, 256), u(128, 256), u(256, 128)
    for name, fn in (("C1 NN 256x128 . 128x256", lambda: O.mm(a, b)),
                     ("C1 TN (128x256)^T . 128x256", lambda: O.matmul_tn(at, b)),
                     ("C1 NT 256x128 . (256x128)^T", lambda: O.matmul_nt(a, bt))):
        dt, reps = timed(fn)
        line(name, dt, reps, 2.0 * 256 * 128 * 256 / dt / 1e9, "GFLOP/s", f"{reps} calls, double", "--suite gemm C1")
    # C5 1024^3
    a, b = u(1024, 1024), u(1024, 1024)
    dt, reps = timed(lambda: O.mm(a, b), min_s=1.0, max_reps=3)
    line("C5 NN 1024^3", dt, reps, 2.0 * 1024 ** 3 / dt / 1e9, "GFLOP/s", f"{reps} calls, double",
         "--suite gemm NN 1024")
    # C4 kernels on a 512-row sample of the 4096-row shapes (GB/s of the fp32
    # bytes the GPU kernel moves for the same rows, so the two lines compare)
    R, D, F = 512, 1024, 4096
    x, w = rng.standard_normal((R, D)), rng.normal(1, 0.1, D)
    y, inv = O.rmsnorm_fwd(x, w, 1e-6)
    g = rng.standard_normal((R, D))
    cases = [
        ("C4 rmsnorm_fwd 512x1024 (of 4096x1024)", lambda: O.rmsnorm_fwd(x, w, 1e-6), 4 * (2 * R * D + D + R)),
        ("C4 rmsnorm_bwd 512x1024 (of 4096x1024)", lambda: O.rmsnorm_bwd(x, w, inv, g), 4 * (3 * R * D + 2 * D + R)),
        ("C4 rope_fwd 512x16x64 interleaved (of 4096)",
         lambda: O.rope_heads(x, 16, 64, interleaved=True), 4 * 2 * R * D),
        ("C4 rope_bwd 512x16x64 interleaved (of 4096)",
         lambda: O.rope_heads(x, 16, 64, interleaved=True, inverse=True), 4 * 2 * R * D),
    ]
    gt, up, dh = rng.standard_normal((R, F)), rng.standard_normal((R, F)), rng.standard_normal((R, F))
    sc = rng.normal(0, 2, (R, F))
    sm = O.softmax_fwd(sc)
    cases += [
        ("C4 swiglu_fwd 512x4096 (of 4096x4096)", lambda: O.swiglu_fwd(gt, up), 4 * 3 * R * F),
        ("C4 swiglu_bwd 512x4096 (of 4096x4096)", lambda: O.swiglu_bwd(gt, up, dh), 4 * 5 * R * F),
        ("C4 softmax_fwd 512x4096 (of 4096x4096)", lambda: O.softmax_fwd(sc), 4 * 2 * R * F),
        ("C4 softmax_bwd 512x4096 (of 4096x4096)", lambda: O.softmax_bwd(sm, dh), 4 * 3 * R * F),
    ]
    lg = rng.standard_normal((64, 32000))
    tg = rng.integers(0, 32000, 64).astype(np.int32)
    cases += [("C3 ce_fused 64x32000 (of 512x32000)", lambda: O.ce_fused(lg, tg, -1, 1.0 / 64),
               4 * (2 * 64 * 32000 + 2 * 64))]
    for name, fn, nbytes in cases:
        dt, reps = timed(fn)
        line(name, dt, reps, nbytes / dt / 1e9, "GB/s", f"{reps} calls, double arithmetic, fp32-equivalent bytes",
             "--suite bandwidth")


def run_copy_suite(args):
    """out = a + b over 64 Mi floats (768 MiB of traffic per launch: two 256 MiB
    reads, one 256 MiB write), the reference for scaling FETCH_SIZE/WRITE_SIZE."""
    from lanternl_amd import device
    from lanternl_amd._lib import call
    device.init(0)
    n = 64 << 20
    a = device.Buffer((n,)).zero()
    b = device.Buffer((n,)).zero()
    o = device.Buffer((n,))

    def run(_):
        call("lhip_add", a.ptr, b.ptr, o.ptr, n)
    ms = time_launches(run, max(args.steps, 5), args.warmup)
    nbytes = 3 * 4 * n
    print(json.dumps({"suite": "copy", "kernel": "add_kernel 64Mi floats", "ms": ms, "bytes": nbytes,
                      "read_bytes": 2 * 4 * n, "write_bytes": 4 * n,
                      "gbps": nbytes / (ms * 1e-3) / 1e9}), flush=True)


def main():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--workload", default="lmtrain_c2", choices=["lmtrain_c2", "gemm4096", "dh2"],
                   help="dh2: only the step's dominant kernel (for counter passes)")
    p.add_argument("--no-cpu", action="store_true", help="gemm4096: skip the CPU baseline (counter passes)")
    p.add_argument("--graph", action="store_true",
                   help="replay the LM step from a captured hipGraph (default: eager launches on the library "
                        "stream)")
    p.add_argument("--suite", default=None, choices=["gemm", "bandwidth", "copy", "cpu"])
    p.add_argument("--only", default=None, help="bandwidth suite: run only kernels whose name contains this")
    args = p.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py: this build measures ONE GPU only (asked for {args.gpus}); "
              "the multi-GPU path is a design (see the sharding notes), not a measured run.",
              file=sys.stderr, flush=True)
        sys.exit(2)
    if args.suite == "gemm":
        run_gemm_suite(args)
    elif args.suite == "bandwidth":
        run_bandwidth_suite(args)
    elif args.suite == "copy":
        run_copy_suite(args)
    elif args.suite == "cpu":
        run_cpu_suite(args)
    elif args.workload == "gemm4096":
        run_gemm_workload(args)
    elif args.workload == "dh2":
        from lanternl_amd import device
        device.init(0)
        print(json.dumps({"workload": "dh2", **dominant_kernel_c2(args.steps, args.warmup)}), flush=True)
    else:
        run_lm_workload(args)


if __name__ == "__main__":
    main()
