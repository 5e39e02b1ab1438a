"""The `luatl_adapter` backend module, restated in Python over the C ABI.

Mirrors the module contract that ai/core/matrix.lua probes (matrix.lua:28-48):
a module with ``available``, ``reason`` and ``matmul(a, m, k, b, n)`` taking
flat row-major sequences and returning a NEW flat list of m*n numbers
(luatl_adapter.lua:128-135).  ``matmul_nt`` / ``matmul_tn`` serve the
transposed products (matrix.lua:597-660) with the same calling convention:

    matmul_nt(a, m, k, b, n) -> a(m x k) . b(n x k)^T   (m*n numbers)
    matmul_tn(a, m, k, b, n) -> a(m x k)^T . b(m x n)   (k*n numbers)

Inputs are rounded to fp32, the product runs on the GPU (v_mfma fp32) and the
result comes back as doubles.  Nothing here falls back to the CPU: a failure
raises, and the registry above decides what to do with it.
"""
import ctypes

import numpy as np

from . import device
from ._lib import call

name = "luatl_adapter"
available = False
reason = "not loaded"


def _probe():
    global available, reason
    try:
        device.init(0)
    except Exception as e:  # noqa: BLE001 -- surfaced through matrix.backends()
        available, reason = False, str(e).splitlines()[0]
        return
    available, reason = True, "ready"


_probe()


def _flat(x, n, what):
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float64).reshape(-1))
    if a.size < n:
        raise ValueError(f"{name}: {what}: expected {n} elements, got {a.size}")
    return a


def _host(op, a, m, k, b, n, rows, nb):
    if not available:
        raise RuntimeError(f"{name}: backend unavailable: {reason}")
    ad = _flat(a, m * k, "a")
    bd = _flat(b, nb, "b")
    out = np.empty(rows * n, dtype=np.float64)
    call("lhip_matmul_host", op, ad.ctypes.data_as(ctypes.c_void_p), bd.ctypes.data_as(ctypes.c_void_p),
         out.ctypes.data_as(ctypes.c_void_p), m, k, n, 0)
    return out.tolist()


def matmul(a, m, k, b, n):
    """a(m x k) . b(k x n) -> new flat list (luatl_adapter.lua:128-135)."""
    return _host(0, a, m, k, b, n, m, k * n)


def matmul_nt(a, m, k, b, n):
    """a(m x k) . b(n x k)^T -> new flat list of m*n (matrix.lua:597-625 semantics)."""
    return _host(1, a, m, k, b, n, m, n * k)


def matmul_tn(a, m, k, b, n):
    """a(m x k)^T . b(m x n) -> new flat list of k*n (matrix.lua:627-660 semantics)."""
    return _host(2, a, m, k, b, n, k, m * n)
