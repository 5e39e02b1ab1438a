"""ai.Matrix's backend registry and GEMM entry points, restated in Python.

Follows ai/core/matrix.lua: the registry (BACKEND_NAMES :25, probe :28-48,
backends :127-135, reset_backends :137-142, use :144-167, backend_failed
:169-176, try_backend :178-202), ``accel`` and ``strict`` (:18-19), and the
three products ``multiply`` (:541-595), ``matmul_nt`` (:597-625) and
``matmul_tn`` (:627-660).

What is new relative to the reference: every product is offloaded above
the threshold, including the calls that write into a caller's matrix.
  * ``out`` absent, ``acc`` off: the backend entry ``matmul`` / ``matmul_nt`` /
    ``matmul_tn`` returns a NEW flat table, adopted as the result's data
    (``multiply``'s rule, matrix.lua:571-585, carried over to the transposed
    products, which are pure Lua in the reference, matrix.lua:597-660).
  * ``out`` given (the autograd backward, tensor2.lua:206-211,222-227, passes
    ``grad_of(x)`` and ``acc = true``): the backend entry
    ``matmul_into(op, a, m, k, b, n, rd, acc)`` computes the product on the
    device and then, on the host in double, stores it into ``rd = out.data``
    (acc off) or adds it to ``rd`` (acc on), the Lua-side add of the Lua
    loops.  ``rd`` is touched only after the device call has succeeded, so a
    failed call leaves it as it was and the Lua loop that follows does the
    whole product once.
  * ``out`` absent with ``acc`` on targets a fresh zero matrix, so it is the
    plain product and takes the first rule.
A backend without the entry a call needs is skipped for that call, not
counted as failed.  The gate is otherwise the reference's: accel enabled,
not forced to "lua", and m*k*n >= threshold or a forced backend.  The CPU
loops below the threshold keep the reference's order (i-p-j with the a==0
skip for multiply and matmul_tn; a p-ordered dot product for matmul_nt).

Matrices are ``Matrix(rows, cols, data)`` with ``data`` a flat row-major
sequence (a list or a 1-D float64 numpy array); 0-based, unlike Lua.
"""
import importlib

import numpy as np

strict = False
accel = {"enabled": True, "threshold": 4096, "max_errors": 3, "force": None}
last_backend = "lua"

BACKEND_NAMES = ("luatl_adapter", "gpu", "blas")
# Python modules that implement each registry name.  "gpu" (cuBLAS) and "blas"
# (OpenBLAS) are vendor-BLAS backends of the reference that this build does
# not provide, so they probe as "not installed".
MODULES = {"luatl_adapter": "lanternl_amd.backend"}

_backends = []


class Matrix:
    __slots__ = ("rows", "cols", "data")

    def __init__(self, rows, cols, data=None):
        if not (isinstance(rows, int) and isinstance(cols, int)) or rows < 0 or cols < 0:
            raise ValueError(f"matrix.new: rows and cols must be non-negative integers (got {rows}, {cols})")
        self.rows, self.cols = rows, cols
        self.data = np.zeros(rows * cols) if data is None else data

    def to_numpy(self):
        return np.asarray(self.data, dtype=np.float64).reshape(self.rows, self.cols)

    @classmethod
    def from_numpy(cls, a):
        a = np.asarray(a, dtype=np.float64)
        return cls(a.shape[0], a.shape[1], a.reshape(-1).copy())


def _probe(name, overrides):
    entry = {"name": name, "available": False, "errors": 0, "reason": "not loaded", "module": None,
             "last_error": None}
    try:
        if name in overrides:
            mod = overrides[name]
        elif name in MODULES:
            mod = importlib.import_module(MODULES[name])
        else:
            raise ImportError(f"module '{name}' not found")
    except Exception as e:  # noqa: BLE001 -- the reason is the product here
        entry["reason"] = f"not installed ({str(e).splitlines()[0] if str(e) else type(e).__name__})"
        return entry
    entry["module"] = mod
    if getattr(mod, "available", None) is not True:
        entry["reason"] = getattr(mod, "reason", None) or f"module reports available = {getattr(mod, 'available', None)}"
    elif not callable(getattr(mod, "matmul", None)):
        entry["reason"] = "module is available but exposes no matmul() function"
    else:
        entry["available"] = True
        entry["reason"] = "ready"
    return entry


def reset_backends(overrides=None):
    """Re-probe every backend (matrix.lua:137-142).  `overrides` maps a
    registry name to a module object, the way a Lua test pre-loads a stub."""
    global _backends
    _backends = [_probe(n, overrides or {}) for n in BACKEND_NAMES]
    return backends()


def backends():
    if not _backends:
        reset_backends()
    return [{k: e[k] for k in ("name", "available", "reason", "errors", "last_error")} for e in _backends]


def adapter():
    for e in _backends:
        if e["name"] == "luatl_adapter":
            return e["module"]
    return None


def use(name=None):
    """Force a backend, "lua", or back to "auto" (matrix.lua:144-167)."""
    if not _backends:
        reset_backends()
    if name is None or name == "auto":
        accel["force"] = None
        accel["enabled"] = True
        return "auto"
    if name == "lua" or name is False:
        accel["force"] = "lua"
        return "lua"
    for e in _backends:
        if e["name"] == name:
            if not e["available"]:
                raise RuntimeError(f"matrix.use: backend '{name}' is not usable: {e['reason']}")
            accel["force"] = name
            accel["enabled"] = True
            return name
    raise ValueError(f"matrix.use: unknown backend '{name}' (expected 'auto', 'lua', {', '.join(BACKEND_NAMES)})")


def _backend_failed(entry, msg):
    entry["errors"] += 1
    entry["last_error"] = msg
    if entry["errors"] >= (accel.get("max_errors") or 3):
        entry["available"] = False
        entry["reason"] = f"disabled after {entry['errors']} failures: {msg}"


def _is_number(v):
    return isinstance(v, (int, float, np.floating, np.integer)) and not isinstance(v, bool)


def _try_backend(entry, fn_name, args, last):
    """pcall one backend entry and validate its flat result (matrix.lua:178-202)."""
    fn = getattr(entry["module"], fn_name, None)
    if not callable(fn):
        return None  # backend does not serve this call: not a failure
    try:
        res = fn(*args)
    except Exception as e:  # noqa: BLE001 -- counted, as the Lua pcall does
        msg = str(e).splitlines()[0] if str(e) else type(e).__name__
        _backend_failed(entry, msg)
        return None
    if not isinstance(res, (list, tuple, np.ndarray)):
        _backend_failed(entry, f"{fn_name} returned {type(res).__name__}, expected flat table")
        return None
    if strict:
        for i in range(last):
            if i >= len(res) or not _is_number(res[i]):
                _backend_failed(entry, f"{fn_name} result index {i + 1} is {type(res[i]).__name__ if i < len(res) else 'nil'}")
                return None
    elif len(res) < last or not _is_number(res[0]) or not _is_number(res[last - 1]):
        _backend_failed(entry, f"{fn_name} returned a malformed result (expected {last} numbers)")
        return None
    return res


# op names of the into-entry, per product
_OPS = {"matmul": "nn", "matmul_nt": "nt", "matmul_tn": "tn"}


def _dispatch(fn_name, who, ad, m, k, bd, n, last, out, acc):
    """The gate of matrix.lua:571-590, extended to every product and to `out`.

    Returns the flat data the result adopts (a new table, or ``out.data``
    written in place by ``matmul_into``), or None for the Lua loops."""
    global last_backend
    if not _backends:
        reset_backends()
    force = accel.get("force")
    if accel.get("enabled") and force != "lua":
        work = m * k * n
        if force is not None or work >= (accel.get("threshold") or 0):
            if out is None:
                name, args = fn_name, (ad, m, k, bd, n)
            else:
                name, args = "matmul_into", (_OPS[fn_name], ad, m, k, bd, n, out.data, bool(acc))
            for e in _backends:
                if e["available"] and (force is None or force == e["name"]):
                    res = _try_backend(e, name, args, last)
                    if res is not None:
                        last_backend = e["name"]
                        return res
            if force is not None and force != "lua":
                raise RuntimeError(f"matrix.{who}: backend '{force}' was forced via matrix.use() but is unavailable")
    last_backend = "lua"
    return None


def _check(m, who, arg):
    if not isinstance(m, Matrix):
        raise TypeError(f"matrix.{who}: {arg} must be a matrix table, got {type(m).__name__}")
    n = m.rows * m.cols
    if n and len(m.data) < n:
        raise ValueError(f"matrix.{who}: {arg} is malformed (expected {n} numbers, first/last check failed)")


def _target(out, rows, cols, who):
    if out is None:
        return Matrix(rows, cols)
    if out.rows != rows or out.cols != cols:
        raise ValueError(f"matrix.{who}: out is {out.rows}x{out.cols} but result is {rows}x{cols}")
    return out


def multiply(a, b, out=None, acc=False):
    """a . b (matrix.lua:541-595)."""
    global last_backend
    _check(a, "multiply", "a"); _check(b, "multiply", "b")
    if a.cols != b.rows:
        raise ValueError(f"matrix.multiply: inner dimension mismatch, a is {a.rows}x{a.cols} and b is "
                         f"{b.rows}x{b.cols} (a.cols {a.cols} must equal b.rows {b.rows})")
    m, k, n = a.rows, a.cols, b.cols
    r = _target(out, m, n, "multiply")
    if r is a or r is b:
        raise ValueError("matrix.multiply: out must not alias a or b")
    if m == 0 or n == 0:
        last_backend = "lua"
        return r
    if k == 0:
        last_backend = "lua"
        if not acc:
            r.data = np.zeros(m * n)
        return r
    res = _dispatch("matmul", "multiply", a.data, m, k, b.data, n, m * n, out, acc)
    if res is not None:
        r.data = res
        return r
    A, B = a.to_numpy(), b.to_numpy()
    R = r.to_numpy().copy() if acc else np.zeros((m, n))
    for i in range(m):                      # mm, matrix.lua:514-539
        row = R[i]
        for p in range(k):
            av = A[i, p]
            if av != 0:
                row += av * B[p]
    r.data = R.reshape(-1)
    return r


def matmul_nt(a, b, out=None, acc=False):
    """a . b^T (matrix.lua:597-625), offloaded above the threshold."""
    _check(a, "matmul_nt", "a"); _check(b, "matmul_nt", "b")
    if a.cols != b.cols:
        raise ValueError(f"matrix.matmul_nt: inner dimension mismatch, a is {a.rows}x{a.cols} and b is {b.rows}x{b.cols}")
    m, k, n = a.rows, a.cols, b.rows
    r = _target(out, m, n, "matmul_nt")
    if r is a or r is b:
        raise ValueError("matrix.matmul_nt: out must not alias a or b")
    if m == 0 or n == 0:
        return r
    res = _dispatch("matmul_nt", "matmul_nt", a.data, m, k, b.data, n, m * n, out, acc) if k > 0 else None
    if res is not None:
        r.data = res
        return r
    A, B = a.to_numpy(), b.to_numpy()
    S = np.zeros((m, n))
    for p in range(k):                       # s = s + a[i][p]*b[j][p], p ascending
        S += np.outer(A[:, p], B[:, p])
    r.data = (r.to_numpy() + S).reshape(-1) if acc else S.reshape(-1)
    return r


def matmul_tn(a, b, out=None, acc=False):
    """a^T . b (matrix.lua:627-660), offloaded above the threshold."""
    _check(a, "matmul_tn", "a"); _check(b, "matmul_tn", "b")
    if a.rows != b.rows:
        raise ValueError(f"matrix.matmul_tn: outer dimension mismatch, a is {a.rows}x{a.cols} and b is {b.rows}x{b.cols}")
    m, k, n = a.rows, a.cols, b.cols
    r = _target(out, k, n, "matmul_tn")
    if r is a or r is b:
        raise ValueError("matrix.matmul_tn: out must not alias a or b")
    if not acc:
        r.data = np.zeros(k * n)
    if m == 0 or k == 0 or n == 0:
        return r
    res = _dispatch("matmul_tn", "matmul_tn", a.data, m, k, b.data, n, k * n, out, acc)
    if res is not None:
        r.data = res
        return r
    A, B = a.to_numpy(), b.to_numpy()
    R = r.to_numpy().copy()
    for i in range(m):
        for p in range(k):
            av = A[i, p]
            if av != 0:
                R[p] += av * B[i]
    r.data = R.reshape(-1)
    return r
