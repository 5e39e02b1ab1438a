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


def test_capacity_limits_the_timed_launches_and_count_reports_them():
    announce("ktimer capacity")
    a = device.Buffer.from_numpy(np.ones((32, 32), np.float32))
    c = device.Buffer((32, 32))
    call("lhip_ktimer_start", 2)
    for _ in range(5):
        kernels.sgemm(a, a, c)
    ms = (ctypes.c_float * 2)()
    n = ctypes.c_int()
    call("lhip_ktimer_stop", ms, 2, ctypes.byref(n))
    assert n.value == 2 and ms[0] > 0 and ms[1] > 0
    np.testing.assert_array_equal(c.download(), np.full((32, 32), 32, np.float32))


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
