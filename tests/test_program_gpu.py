"""GPU tests of recorded programs (lhip_program_*): a sequence of compute calls
recorded once from the library stream and replayed as a hipGraph, the
counterpart of luaTL.Program's capture/replay (ai/gpu/luaTL_train.lua:327-627,
tests/test.lua:383-439 "Program buffer" and "CUDA Graph capture + replay").

Every replay is checked against the eager result of the same calls (bit-exact:
the kernels are deterministic) with eager work and synchronisations between the
replays, and the eager result against the oracle at the usual bars.
"""
import ctypes

import numpy as np
import pytest

import oracle as O
from lanternl_amd import device
from lanternl_amd._lib import LanternlHipError, call, lib
from tests.gpu_util import announce, f32, rel_fro, to_dev

pytestmark = pytest.mark.gpu

E_UNSUPPORTED = -8


@pytest.fixture(scope="module", autouse=True)
def _dev():
    device.init(0)
    yield
    assert not device.recording()


def dl(buf):
    device.sync()
    return buf.download()


def _chain(rng):
    """GEMM (split-K shape) -> RMSNorm -> causal softmax -> fused CE, on fresh buffers."""
    m, k, n = 256, 8192, 128
    a = f32(rng.uniform(-1, 1, (m, k)))
    b = f32(rng.uniform(-1, 1, (k, n)))
    w = f32(rng.normal(1.0, 0.1, n))
    labels = rng.integers(0, n, m).astype(np.int32)
    bufs = dict(A=to_dev(a), B=to_dev(b), W=to_dev(w), L=to_dev(labels, np.int32),
                C=device.Buffer((m, n)), Y=device.Buffer((m, n)), INV=device.Buffer((m,)),
                P=device.Buffer((m, n)), LOSS=device.Buffer((m,)), DL=device.Buffer((m, n)))

    def run():
        call("lhip_sgemm", 0, 0, m, n, k, 1.0, bufs["A"].ptr, k, bufs["B"].ptr, n, 0.0, bufs["C"].ptr, n)
        call("lhip_rmsnorm_fwd", bufs["C"].ptr, bufs["W"].ptr, bufs["Y"].ptr, bufs["INV"].ptr, m, n, 1e-5)
        call("lhip_softmax_fwd", bufs["Y"].ptr, bufs["P"].ptr, m, n, 0.25, 1, 0, 64)
        call("lhip_ce_fused", bufs["Y"].ptr, bufs["L"].ptr, bufs["LOSS"].ptr, bufs["DL"].ptr, m, n, -1, 1.0 / m)

    def outputs():
        return {k_: dl(bufs[k_]) for k_ in ("C", "Y", "INV", "P", "LOSS", "DL")}

    return a, b, w, labels, bufs, run, outputs


def test_program_replays_match_eager_and_oracle():
    announce("program", "gemm+rmsnorm+softmax+ce")
    rng = np.random.default_rng(7)
    a, b, w, labels, bufs, run, outputs = _chain(rng)
    run()                                  # eager: sizes the workspace
    eager = outputs()
    c_ref = O.mm(a, b)
    assert rel_fro(eager["C"], c_ref) <= 1e-4
    y_ref, _ = O.rmsnorm_fwd(eager["C"].astype(np.float64), w, 1e-5)
    assert rel_fro(eager["Y"], y_ref) <= 1e-5
    prog = device.Program.record(run)
    # recording executed nothing: clear the outputs, then replay
    for k_ in ("C", "Y", "INV", "P", "LOSS", "DL"):
        bufs[k_].zero()
    scratch = device.Buffer((1 << 20,))
    for rep in range(4):
        prog.replay()
        got = outputs()
        for k_, v in eager.items():
            assert np.array_equal(got[k_], v), f"replay {rep}: {k_} differs from the eager result"
        # eager work and a synchronisation between replays
        call("lhip_fill", scratch.ptr, scratch.size, float(rep))
        for k_ in ("C", "P", "DL"):
            bufs[k_].zero()
        device.sync()
    prog.free()


def test_program_reads_current_inputs_and_replays_back_to_back():
    announce("program", "new inputs, times=3")
    rng = np.random.default_rng(8)
    a, b, w, labels, bufs, run, outputs = _chain(rng)
    run()
    prog = device.Program.record(run)
    a2 = f32(rng.uniform(-1, 1, a.shape))
    bufs["A"].upload(a2)                   # a program keeps pointers, not values
    prog.replay(3)                         # idempotent chain: three replays, one result
    got = outputs()
    run()
    eager = outputs()
    for k_, v in eager.items():
        assert np.array_equal(got[k_], v), k_
    assert rel_fro(got["C"], O.mm(a2, b)) <= 1e-4
    prog.free()


def test_recording_refuses_synchronising_and_allocating_calls():
    announce("program", "refusals")
    L = lib()
    x = device.Buffer((256,)).zero()
    host = np.zeros(256, np.float32)
    call("lhip_program_begin")
    try:
        assert device.recording()
        assert L.lhip_sync() == E_UNSUPPORTED
        assert L.lhip_upload(x.ptr, host.ctypes.data, host.nbytes) == E_UNSUPPORTED
        assert L.lhip_download(host.ctypes.data, x.ptr, host.nbytes) == E_UNSUPPORTED
        p = ctypes.c_void_p()
        assert L.lhip_malloc(ctypes.byref(p), 1024) == E_UNSUPPORTED
        assert L.lhip_free(x.ptr) == E_UNSUPPORTED
        assert L.lhip_program_begin() == -6        # already recording
        # a workspace that would have to grow (4 GiB of dw partials) is refused
        big = 1 << 20
        rc = L.lhip_rmsnorm_bwd(x.ptr, x.ptr, x.ptr, x.ptr, x.ptr, x.ptr, 4096, big, 0)
        assert rc == E_UNSUPPORTED, rc
        call("lhip_fill", x.ptr, 256, 3.0)          # an ordinary call is recorded
    finally:
        prog = device.Program()
        call("lhip_program_end", ctypes.byref(prog._h))
    assert not device.recording()
    np.testing.assert_array_equal(x.download(), 0.0)   # recorded, not executed
    prog.replay()
    np.testing.assert_array_equal(dl(x), 3.0)
    prog.free()


def test_discarded_recording_leaves_library_usable():
    announce("program", "discard")
    x = device.Buffer((64,)).zero()

    def bad():
        call("lhip_fill", x.ptr, 64, 5.0)
        raise ValueError("abandon")
    with pytest.raises(ValueError):
        device.Program.record(bad)
    assert not device.recording()
    np.testing.assert_array_equal(dl(x), 0.0)
    call("lhip_fill", x.ptr, 64, 2.0)
    np.testing.assert_array_equal(dl(x), 2.0)
    with pytest.raises(LanternlHipError, match="ARG"):
        call("lhip_program_end", None)               # nothing is being recorded
    with pytest.raises(LanternlHipError, match="NULL"):
        call("lhip_program_replay", None, 1)


def test_program_survives_workspace_growth():
    """A program keeps the workspace pointer it was recorded with.  An eager
    call that grows the library workspace while the program is live must not
    free that memory under it: the old workspace is retired until the last
    program is freed, and the replay still matches the eager result."""
    announce("program", "workspace growth between record and replay")
    from lanternl_amd._lib import MemStats
    rng = np.random.default_rng(9)

    def ws_bytes():
        s = MemStats()
        call("lhip_mem_stats", ctypes.byref(s))
        return s.workspace_bytes

    m, n, k = 256, 128, 8192                       # split-K through the workspace
    a, b = f32(rng.uniform(-1, 1, (m, k))), f32(rng.uniform(-1, 1, (k, n)))
    A, B, Cp = to_dev(a), to_dev(b), device.Buffer((m, n))
    call("lhip_sgemm", 0, 0, m, n, k, 1.0, A.ptr, k, B.ptr, n, 0.0, Cp.ptr, n)
    eager = dl(Cp)
    assert rel_fro(eager, O.mm(a, b)) <= 1e-4
    prog = device.Program.record(
        lambda: call("lhip_sgemm", 0, 0, m, n, k, 1.0, A.ptr, k, B.ptr, n, 0.0, Cp.ptr, n))
    w0 = ws_bytes()
    # 4096 x 3840 x 4096 splits K in two slices of 4096x3840 floats (126 MB of
    # partials), more than any earlier call of this suite needs
    gm, gn, gk = 4096, 3840, 4096
    ga = to_dev(rng.uniform(-1, 1, (gm, gk)).astype(np.float32))
    gb = to_dev(rng.uniform(-1, 1, (gk, gn)).astype(np.float32))
    gc = device.Buffer((gm, gn))
    call("lhip_sgemm", 0, 0, gm, gn, gk, 1.0, ga.ptr, gk, gb.ptr, gn, 0.0, gc.ptr, gn)
    device.sync()
    if ws_bytes() <= w0:
        prog.free()
        pytest.skip(f"workspace already {w0} bytes: the growing call did not grow it")
    grown = ws_bytes()          # the new workspace, plus the retired one held for the program
    assert grown > w0
    del ga, gb, gc
    for rep in range(3):
        Cp.zero()
        prog.replay()
        got = dl(Cp)
        assert np.array_equal(got, eager), f"replay {rep} after the workspace grew"
        # the eager path on the grown workspace still agrees too
        call("lhip_sgemm", 0, 0, m, n, k, 1.0, A.ptr, k, B.ptr, n, 0.0, Cp.ptr, n)
        assert np.array_equal(dl(Cp), eager)
    prog.free()
    # the retired workspace is released with the last live program
    assert ws_bytes() == grown - w0
