"""Python wrappers of the device entry points (device Buffers in, device Buffers out).

Each wrapper checks shapes on the host, then calls the C ABI, which enqueues
the kernel on the library stream and returns; ``device.sync()`` waits.
"""
from ._lib import call
from .device import Buffer


def _dims2(buf, name):
    if len(buf.shape) != 2:
        raise ValueError(f"{name} must be 2-D, got shape {buf.shape}")
    return buf.shape


def sgemm(a: Buffer, b: Buffer, c: Buffer, transa=False, transb=False, alpha=1.0, beta=0.0):
    """c = alpha * op(a) @ op(b) + beta * c on whole 2-D buffers."""
    ar, ac = _dims2(a, "a")
    br, bc = _dims2(b, "b")
    m, k = (ac, ar) if transa else (ar, ac)
    kb, n = (bc, br) if transb else (br, bc)
    if kb != k:
        raise ValueError(f"inner dimensions differ: op(a) is {m}x{k}, op(b) is {kb}x{n}")
    if c.shape != (m, n):
        raise ValueError(f"c is {c.shape}, expected {(m, n)}")
    call("lhip_sgemm", int(bool(transa)), int(bool(transb)), m, n, k, float(alpha),
         a.ptr, ac, b.ptr, bc, float(beta), c.ptr, n)
    return c


def sgemm_raw(transa, transb, m, n, k, alpha, a_ptr, lda, b_ptr, ldb, beta, c_ptr, ldc):
    """lhip_sgemm on raw device addresses (strided views)."""
    call("lhip_sgemm", int(bool(transa)), int(bool(transb)), m, n, k, float(alpha),
         a_ptr, lda, b_ptr, ldb, float(beta), c_ptr, ldc)


def sgemm_strided_batched(transa, transb, m, n, k, alpha, a_ptr, lda, sa, b_ptr, ldb, sb,
                          beta, c_ptr, ldc, sc, batch):
    call("lhip_sgemm_strided_batched", int(bool(transa)), int(bool(transb)), m, n, k, float(alpha),
         a_ptr, lda, sa, b_ptr, ldb, sb, float(beta), c_ptr, ldc, sc, batch)


def sgemm_batched_reduce(transa, transb, m, n, k, alpha, a_ptr, lda, sa, b_ptr, ldb, sb, beta, c_ptr, ldc, count):
    """C = alpha * sum_j op(A_j) op(B_j) + beta * C over `count` strided operand pairs (raw pointers)."""
    call("lhip_sgemm_batched_reduce", int(bool(transa)), int(bool(transb)), m, n, k, float(alpha),
         a_ptr, lda, sa, b_ptr, ldb, sb, float(beta), c_ptr, ldc, count)
