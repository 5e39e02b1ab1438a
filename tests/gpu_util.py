"""Helpers shared by the GPU parity tests (no oracle logic here)."""
import numpy as np

from lanternl_amd import device


def rel_fro(x, ref):
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.linalg.norm(ref)
    num = np.linalg.norm(x - ref)
    return num / den if den > 0 else num


def f32(a):
    """fp32-representable float64 copy (both sides see identical inputs)."""
    return np.asarray(a, dtype=np.float32).astype(np.float64)


def to_dev(a, dtype=np.float32):
    return device.Buffer.from_numpy(np.asarray(a), dtype=dtype)


def announce(*what):
    print("[gpu-case]", *what, flush=True)
