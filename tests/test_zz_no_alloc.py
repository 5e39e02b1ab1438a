"""lhip_sgemm_noalloc: the GEMM entry point that allocates nothing.

Its split-K partials live in a fixed 64 MiB device array instead of the
library workspace.  It must give exactly what lhip_sgemm gives (same kernels,
same K slices, same summation order), on consecutive calls whose sizes shrink
(the array keeps the previous call's contents), refuse a shape whose partials
would not fit before launching anything, allocate nothing (the library's
workspace and buffer counters do not move), and be recordable into a program.
"""
import ctypes

import numpy as np
import pytest

from tests.gpu_util import announce, rel_fro, to_dev
from lanternl_amd import _lib, device
from lanternl_amd._lib import MemStats, call, lib

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20


def _mem():
    s = MemStats()
    call("lhip_mem_stats", ctypes.byref(s))
    return s.workspace_bytes, s.live_buffers, s.n_alloc


def _operands(rng, m, n, k, ta, tb):
    a = rng.uniform(-1, 1, (k, m) if ta else (m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (n, k) if tb else (k, n)).astype(np.float32)
    return a, b


def _run(name, ta, tb, m, n, k, A, B, C, alpha=1.0, beta=0.0):
    lda = m if ta else k
    ldb = k if tb else n
    call(name, ta, tb, m, n, k, alpha, A.ptr, lda, B.ptr, ldb, beta, C.ptr, n)


# (m, n, k, ta, tb): the first uses the whole 64 MiB (2048^3: four 512-deep
# slices of 2048x2048), each later one is smaller, so it runs over what the
# previous call left in the array
SEQUENCE = [
    (2048, 2048, 2048, 0, 0),   # 256x256 tiles, 4 K slices: 64 MiB of partials
    (256, 256, 8192, 1, 0),     # 64x64 tiles, 32 K slices (Aᵀ.B)
    (64, 4096, 4096, 0, 0),     # one band of 64x64 tiles on four wave sets, 4 K slices
    (16, 4096, 4096, 0, 0),     # skinny rows, K slices
    (96, 80, 3000, 0, 1),       # A.Bᵀ, ragged edges
    (64, 64, 64, 0, 0),         # unsplit
]


def test_noalloc_matches_sgemm_on_shrinking_calls():
    device.init(0)
    rng = np.random.default_rng(71)
    for i, (m, n, k, ta, tb) in enumerate(SEQUENCE):
        announce("noalloc", i, (m, n, k, ta, tb))
        a, b = _operands(rng, m, n, k, ta, tb)
        A, B = to_dev(a), to_dev(b)
        c0 = rng.uniform(-1, 1, (m, n)).astype(np.float32)
        Cn, Cr = to_dev(c0), to_dev(c0)
        beta = 0.5 if i % 2 else 0.0
        device.sync()
        before = _mem()
        _run("lhip_sgemm_noalloc", ta, tb, m, n, k, A, B, Cn, 1.0, beta)
        device.sync()
        after = _mem()
        # nothing allocated by the call: workspace and buffer counters unchanged
        assert after == before, (before, after)
        _run("lhip_sgemm", ta, tb, m, n, k, A, B, Cr, 1.0, beta)
        device.sync()
        got, ref = Cn.download(), Cr.download()
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"call {i}: differs from lhip_sgemm"
        # and both meet the GEMM bar against float64
        a64, b64 = a.astype(np.float64), b.astype(np.float64)
        exact = (a64.T if ta else a64) @ (b64.T if tb else b64) + beta * c0.astype(np.float64)
        assert rel_fro(got, exact) <= 1e-4


def test_noalloc_refuses_oversized_split_before_launch():
    device.init(0)
    # 4096 x 3840 x 4096: 240 tiles of 256x256, split in two K slices of
    # 4096x3840 floats each (126 MB of partials) on 256 CUs -- beyond the
    # 64 MiB array, so the host refuses it before anything launches.  The
    # operands are allocated at their real sizes (A 64 MiB, B and C 60 MiB),
    # so that if a plan on another CU count needs no split (nothing to
    # refuse), the call still runs in bounds and the assertion fails on the
    # return code instead of a memory fault.
    m, n, k = 4096, 3840, 4096
    A, B, Cc = device.Buffer((m, k)), device.Buffer((k, n)), device.Buffer((m, n))
    for buf in (A, B, Cc):
        buf.zero()
    device.sync()
    rc = lib().lhip_sgemm_noalloc(0, 0, m, n, k, 1.0, A.ptr, k, B.ptr, n, 0.0, Cc.ptr, n)
    device.sync()
    assert rc == -7, f"expected LHIP_E_CAPACITY (-7), got {rc} on {device.info()['compute_units']} CUs"
    msg = _lib.last_error()
    assert "scratch" in msg and str(SCRATCH_BYTES) in msg, msg
    lib().lhip_clear_error()


def test_noalloc_recorded_program_replays_exactly():
    device.init(0)
    rng = np.random.default_rng(72)
    m, n, k = 256, 256, 8192          # 32 K slices through the scratch array
    a, b = _operands(rng, m, n, k, 0, 0)
    A, B = to_dev(a), to_dev(b)
    Cp, Cr = device.Buffer((m, n)), device.Buffer((m, n))
    _run("lhip_sgemm", 0, 0, m, n, k, A, B, Cr)
    device.sync()
    ref = Cr.download()
    call("lhip_program_begin")
    try:
        _run("lhip_sgemm_noalloc", 0, 0, m, n, k, A, B, Cp)
    except Exception:
        lib().lhip_program_end(None)
        raise
    h = ctypes.c_void_p()
    call("lhip_program_end", ctypes.byref(h))
    try:
        # eager work that also uses the scratch array between the replays
        small = to_dev(rng.uniform(-1, 1, (16, 4096)).astype(np.float32))
        big = to_dev(rng.uniform(-1, 1, (4096, 4096)).astype(np.float32))
        out = device.Buffer((16, 4096))
        for rep in range(3):
            announce("noalloc replay", rep)
            Cp.zero()
            call("lhip_program_replay", h, 1)
            device.sync()
            got = Cp.download()
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"replay {rep}"
            _run("lhip_sgemm_noalloc", 0, 0, 16, 4096, 4096, small, big, out)
            device.sync()
    finally:
        call("lhip_program_free", h)
