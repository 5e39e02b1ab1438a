"""Device lifecycle, buffers and timing over the C ABI.

``Buffer`` is the Python analogue of the reference's resident handle
(ai/gpu/luatl_adapter.lua:46-101): a device allocation with a shape, an
element type, ``upload``/``download`` of host arrays and ``zero``.  It owns its
memory and frees it when collected (after lhip_shutdown that is a no-op,
like luaTL_tensor_release_safe, cuda/luaTL_train.cu:47-53).
"""
import ctypes

import numpy as np

from ._lib import DevInfo, call, lib

_DTYPES = {np.dtype(np.float32): "f32", np.dtype(np.int32): "i32"}


def init(device=0):
    """Initialise the library on `device` (idempotent)."""
    call("lhip_init", device)


def shutdown():
    call("lhip_shutdown")


def ready():
    return bool(lib().lhip_is_ready())


def sync():
    call("lhip_sync")


def info():
    d = DevInfo()
    call("lhip_device_info", ctypes.byref(d))
    return {
        "name": d.name.decode(), "arch": d.arch.decode(), "device": d.device,
        "compute_units": d.compute_units, "clock_khz": d.clock_khz,
        "total_mem": d.total_mem, "lds_per_block": d.lds_per_block, "l2_bytes": d.l2_bytes,
        "peak_fp32_matrix_tflops": d.peak_fp32_matrix_tflops, "peak_hbm_gbps": d.peak_hbm_gbps,
    }


class Buffer:
    """A device array (row-major, float32 or int32)."""

    def __init__(self, shape, dtype=np.float32):
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        if self.dtype not in _DTYPES:
            raise TypeError(f"unsupported dtype {self.dtype}")
        self.size = int(np.prod(self.shape)) if self.shape else 1
        self.nbytes = self.size * self.dtype.itemsize
        self._p = ctypes.c_void_p()
        call("lhip_malloc", ctypes.byref(self._p), max(self.nbytes, 4))

    @classmethod
    def from_numpy(cls, arr, dtype=None):
        arr = np.asarray(arr)
        dt = np.dtype(dtype) if dtype is not None else (np.dtype(np.int32) if arr.dtype.kind in "iu" else np.dtype(np.float32))
        b = cls(arr.shape, dt)
        b.upload(arr)
        return b

    @classmethod
    def zeros(cls, shape, dtype=np.float32):
        b = cls(shape, dtype)
        b.zero()
        return b

    @property
    def ptr(self):
        if self._p is None or self._p.value is None:
            raise RuntimeError("buffer has been freed")
        return self._p.value

    def offset(self, elems):
        """Device address `elems` elements into the buffer (a strided view's base)."""
        if not 0 <= elems <= self.size:
            raise IndexError(f"offset {elems} outside buffer of {self.size} elements")
        return self.ptr + elems * self.dtype.itemsize

    def upload(self, arr):
        a = np.ascontiguousarray(arr, dtype=self.dtype)
        if a.size != self.size:
            raise ValueError(f"upload: {a.size} elements into a buffer of {self.size}")
        call("lhip_upload", self.ptr, a.ctypes.data, self.nbytes)
        return self

    def download(self):
        out = np.empty(self.shape, dtype=self.dtype)
        call("lhip_download", out.ctypes.data, self.ptr, self.nbytes)
        return out

    def zero(self):
        call("lhip_zero", self.ptr, self.nbytes)
        return self

    def free(self):
        if self._p is not None and self._p.value:
            try:
                lib().lhip_free(self._p)
            finally:
                self._p = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Timer:
    """hipEvent pair recorded on the library stream."""

    def __init__(self):
        self._a = ctypes.c_void_p()
        self._b = ctypes.c_void_p()
        call("lhip_event_create", ctypes.byref(self._a))
        call("lhip_event_create", ctypes.byref(self._b))

    def start(self):
        call("lhip_event_record", self._a)

    def stop(self):
        call("lhip_event_record", self._b)

    def ms(self):
        v = ctypes.c_float()
        call("lhip_event_elapsed_ms", self._a, self._b, ctypes.byref(v))
        return float(v.value)

    def __del__(self):
        try:
            lib().lhip_event_destroy(self._a)
            lib().lhip_event_destroy(self._b)
        except Exception:
            pass


def kernel_times(fn, capacity=4096):
    """Run fn() with the library's kernel timer on and return the duration
    (ms) of each kernel it launched, in launch order: dispatch start to end,
    as a kernel trace reports them (lhip_ktimer_start / lhip_ktimer_stop)."""
    call("lhip_ktimer_start", capacity)
    try:
        fn()
    finally:
        buf = (ctypes.c_float * capacity)()
        n = ctypes.c_int()
        call("lhip_ktimer_stop", buf, capacity, ctypes.byref(n))
    return [float(buf[i]) for i in range(min(n.value, capacity))]


class Program:
    """A recorded sequence of library calls, replayed as one hipGraph launch.

    The counterpart of luaTL.Program's capture/replay
    (ai/gpu/luaTL_train.lua:327-627): ``record(fn)`` runs ``fn()`` while the
    library stream is being captured, so the compute calls fn makes are
    recorded rather than executed; ``replay(times)`` enqueues the recording.
    Calls that synchronise or allocate are refused while recording (run fn
    once eagerly first so that the library workspace is already sized).
    """

    def __init__(self):
        self._h = ctypes.c_void_p()

    @classmethod
    def record(cls, fn):
        prog = cls()
        call("lhip_program_begin")
        try:
            fn()
        except BaseException:
            lib().lhip_program_end(None)   # discard the partial recording
            raise
        call("lhip_program_end", ctypes.byref(prog._h))
        return prog

    def replay(self, times=1):
        if not self._h.value:
            raise RuntimeError("program has been freed")
        call("lhip_program_replay", self._h, int(times))

    def free(self):
        if self._h is not None and self._h.value:
            try:
                lib().lhip_program_free(self._h)
            finally:
                self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def recording():
    return bool(lib().lhip_is_recording())
