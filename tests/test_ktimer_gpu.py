"""GPU tests of the library's kernel timer (lhip_ktimer_start / lhip_ktimer_stop),
which bench.py uses for kernel-trace comparable kernel times: one duration per
kernel launched while it is on, in launch order, and the rules that keep it
out of recorded programs."""
import ctypes

import numpy as np
import pytest

from lanternl_amd import device, kernels
from lanternl_amd._lib import LanternlHipError, call
from tests.gpu_util import announce

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _dev():
    device.init(0)
    yield


def test_one_duration_per_kernel_in_launch_order():
    announce("ktimer order")
    nb, ns = 64 << 20, 1024
    big = [device.Buffer((nb,)).zero() for _ in range(3)]
    small = [device.Buffer((ns,)).zero() for _ in range(3)]
    device.sync()

    def add(bufs, n):
        call("lhip_add", bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, n)
    t = device.kernel_times(lambda: (add(small, ns), add(big, nb), add(small, ns)))
    assert len(t) == 3
    assert all(x > 0 for x in t)
    # 768 MiB of traffic (~100 us at HBM rates) take far longer than 12 KiB
    # (a few us: a dispatch's start-to-end span across the eight XCDs)
    assert t[1] > 8 * max(t[0], t[2])


def test_capacity_limits_the_timed_launches_and_stop_reports_the_rest():
    """Launches past the capacity run untimed; stop counts them all and returns
    LHIP_E_CAPACITY, so a caller cannot sum a partial list unknowingly."""
    announce("ktimer capacity")
    a = device.Buffer.from_numpy(np.ones((32, 32), np.float32))
    c = device.Buffer((32, 32))
    call("lhip_ktimer_start", 2)
    for _ in range(5):
        kernels.sgemm(a, a, c)
    ms = (ctypes.c_float * 2)()
    n = ctypes.c_int()
    with pytest.raises(LanternlHipError, match="5 kernels were launched but only 2 timed"):
        call("lhip_ktimer_stop", ms, 2, ctypes.byref(n))
    assert n.value == 5 and ms[0] > 0 and ms[1] > 0
    np.testing.assert_array_equal(c.download(), np.full((32, 32), 32, np.float32))
    # the Python wrapper raises instead of returning a short list
    with pytest.raises(LanternlHipError, match="only 3 timed"):
        device.kernel_times(lambda: [kernels.sgemm(a, a, c) for _ in range(4)], capacity=3)
    # within the capacity: one entry per launch, stop returns OK
    assert len(device.kernel_times(lambda: [kernels.sgemm(a, a, c) for _ in range(3)], capacity=3)) == 3


def test_graph_mode_lm_step_refused_while_the_timer_is_on():
    """A graph replay's kernels cannot be timed, so a graph-mode step is refused
    (as lhip_program_begin is) rather than leaving the timer to count captured
    launches as dispatches."""
    announce("ktimer vs lm graph step")
    from lanternl_amd import lmtrain
    step = lmtrain.GpuLMStep(vocab=32, dim=16, layers=1, heads=2, ffn=32, batch=2, seq=8)
    rng = np.random.default_rng(0)
    step.set_params(rng.normal(0, 0.02, step.n).astype(np.float32))
    step.set_batch(rng.integers(0, 32, (2, 8)), rng.integers(0, 32, (2, 8)))
    step.use_graph(True)
    call("lhip_ktimer_start", 64)
    try:
        with pytest.raises(LanternlHipError, match="graph mode while the kernel timer is on"):
            step.step(lr=0.1)
    finally:
        call("lhip_ktimer_stop", None, 0, None)
    step.step(lr=0.1)          # timer off: the graph step runs
    device.sync()
    step.close()


def test_timer_and_program_recording_exclude_each_other():
    announce("ktimer vs program")
    call("lhip_ktimer_start", 4)
    try:
        with pytest.raises(LanternlHipError):
            call("lhip_program_begin")
    finally:
        call("lhip_ktimer_stop", None, 0, None)
    call("lhip_program_begin")
    try:
        with pytest.raises(LanternlHipError):
            call("lhip_ktimer_start", 4)
    finally:
        call("lhip_program_end", None)
    with pytest.raises(LanternlHipError):
        call("lhip_ktimer_stop", None, 0, None)   # not on
