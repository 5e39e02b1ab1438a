"""The `luatl_adapter` backend module, restated in Python over the C ABI.

The Python mirror of ``lanternl_amd/lua/luatl_adapter.lua``, which is the Lua
module itself (the LuaJIT FFI binding that ai/core/matrix.lua requires).  Both
follow the reference adapter, ai/gpu/luatl_adapter.lua, call for call: the
same names, the same argument lists and the same return conventions.  A
reference caller that uses only the adapter's own functions (the registry,
tests/test.lua:436-475) reads the same here.  Callers that reach past the
adapter into the reference's low-level module (``adapter.luaTL``:
ai/gpu/gpu_transformer.lua:58-60, ai/benchmarks/bench_gpu_transformer.lua:41,
and ai/optim/lmtrain_gpu.lua through gpu_transformer) do not: that field has
no counterpart here and is None.

* Module contract (matrix.lua:28-48): ``available``, ``reason``/``error`` and
  ``matmul(a, m, k, b, n)``.  ``a`` and ``b`` are flat row-major sequences or
  resident handles; with two handles the result is a new handle, otherwise a
  NEW flat list of m*n numbers (luatl_adapter.lua:102-135).  ``matmul_nt`` /
  ``matmul_tn`` serve the transposed products with the same convention:

      matmul_nt(a, m, k, b, n) -> a(m x k) . b(n x k)^T   (m*n numbers)
      matmul_tn(a, m, k, b, n) -> a(m x k)^T . b(m x n)   (k*n numbers)

  ``matmul_into(op, a, m, k, b, n, rd, acc)`` serves the products that write
  into a caller's flat sequence (matrix.multiply / matmul_nt / matmul_tn with
  ``out``, which the autograd backward passes with ``acc = true``,
  tensor2.lua:206-211,222-227): ``rd`` receives the product, or has it added
  in double with ``acc``, after the device call has succeeded.
* Legacy flat calls (luatl_adapter.lua:137-159): ``rmsnorm(x, rows, cols, w,
  eps)``, ``softmax(x, rows, cols)``, ``softmax_causal(x, rows, cols, scale,
  group)``, each taking a flat table or a handle.
* Resident calls (:161-187): ``gemm(hA, hB, hC, opts)``, ``gemm_dx``,
  ``gemm_dw``, ``add_inplace``, ``silu_inplace``, ``gelu_inplace``,
  ``scale_inplace``, ``rope(h, o)``, ``swiglu(ha, hb, ho, o)``,
  ``rmsnorm_bwd(hx, hg, hdy, hdx, hdg, eps)``, ``softmax_bwd(hy, hdy, hdx, o)``,
  ``program(cap, timing)``, ``sync``, ``stats``, ``hardware``, ``shutdown``,
  and the resident-tensor toolkit (:188-246).
* ``program(cap, timing)`` returns a ``Program`` with luaTL.Program's op list
  (ai/gpu/luaTL_train.lua:332-632): ops are queued, ``run`` executes them on the
  library stream, ``capture`` records them once into a hipGraph and ``replay``
  launches it.

Inputs of the flat-table calls are rounded to fp32, the work runs on the GPU
and results come back as doubles.  Nothing here falls back to the CPU: a
failure raises, and the registry above decides what to do with it.  Handles
and tensors expose ``.t.data`` (the device address), ``rows`` and ``cols`` as
the reference's do; ``luaTL`` (the reference's own low-level module) has no
counterpart and is None.
"""
import ctypes

import numpy as np

from . import device as _device
from ._lib import MemStats, call, lib

name = "luatl"
priority = 100
available = False
reason = "not loaded"
error = None
device = None               # the reference's M.device (a device name string)
C = None                    # the reference's M.C: here the ctypes library
luaTL = None                # the reference's M.luaTL: no counterpart (this is not luaTL)

F32 = 0                     # luaTL.F32: the only element type of this build

# luaTL.EW codes (cuda/luaTL_core.cu:49-72) = LHIP_EW_* of include/lanternl_hip.h
EW = {"COPY": 0, "ADD": 1, "SUB": 2, "MUL": 3, "DIV": 4, "SCALE": 5, "AXPY": 6, "FILL": 7, "RELU": 8,
      "GELU": 9, "SILU": 10, "TANH": 11, "SIGMOID": 12, "EXP": 13, "SQRT": 14, "RSQRT": 15, "NEG": 16,
      "RECIP": 17, "ABS": 18, "CLAMP": 19, "DRELU": 20, "DSILU": 21, "DGELU": 22}
ACT = {"NONE": 0, "RELU": 1, "GELU": 2, "SILU": 3, "TANH": 4, "SIGMOID": 5}
PRE = {"NONE": 0, "RMSNORM": 1, "GELU": 2, "SILU": 3, "RELU": 4}


def _probe():
    global available, reason, error, device, C
    try:
        _device.init(0)
        device = _device.info()["name"]
    except Exception as e:  # noqa: BLE001 -- surfaced through matrix.backends()
        available, reason = False, str(e).splitlines()[0]
        error = reason
        return
    available, reason, error, C = True, "ready", None, lib()


_probe()


def _require():
    if not available:
        raise RuntimeError(f"luatl adapter: backend unavailable: {reason}")


# ------------------------------------------------------------------ tensors
class Tensor:
    """A device fp32 matrix: the role of a luaTL tensor (``data`` is the device
    address, ``rows``/``cols``/``nelem``/``nbytes``/``dtype``).  Owning tensors
    hold a device.Buffer; ``wrap`` makes non-owning ones."""

    __slots__ = ("data", "rows", "cols", "dtype", "_buf")

    def __init__(self, rows, cols, data=None, buf=None):
        self.rows, self.cols, self.dtype = int(rows), int(cols), F32
        self._buf = buf
        self.data = int(data) if data is not None else (buf.ptr if buf is not None else 0)

    @property
    def nelem(self):
        return self.rows * self.cols

    @property
    def nbytes(self):
        return 4 * self.nelem

    @classmethod
    def new(cls, rows, cols):
        buf = _device.Buffer((max(rows * cols, 1),))
        return cls(rows, cols, buf=buf)

    def t(self):
        """Logical transpose as a stride view (luaTL_train.lua:120-122)."""
        return view(self.data, self.cols, self.rows, 1, self.cols, 0)

    def free(self):
        if self._buf is not None:
            self._buf.free()
            self._buf = None
        self.data = 0


def _fetch_f32(ptr, n):
    """n fp32 values at a device address, as a new list of floats."""
    buf = np.empty(n, np.float32)
    call("lhip_download", buf.ctypes.data, ptr, 4 * n)
    return buf.astype(np.float64).tolist()


def _put_f32(ptr, seq, n, what):
    """The first n numbers of a flat sequence, rounded to fp32, to a device address."""
    vals = np.asarray(seq, dtype=np.float32).reshape(-1)
    if vals.size < n:
        raise ValueError(f"lanternl_hip: {what} needs {n} numbers, the table holds {vals.size}")
    vals = np.ascontiguousarray(vals[:n])
    call("lhip_upload", ptr, vals.ctypes.data, 4 * n)


class Handle:
    """A resident GPU matrix exposed to lanternl (luatl_adapter.lua:46-101)."""

    def __init__(self, t, rows, cols):
        self.t, self.rows, self.cols = t, rows, cols

    def toflat(self):
        return _fetch_f32(self.t.data, self.rows * self.cols)

    def upload(self, flat):
        _put_f32(self.t.data, flat, self.rows * self.cols, f"Handle:upload into {self.rows}x{self.cols}")
        return self

    def zero(self):
        call("lhip_zero", self.t.data, 4 * self.rows * self.cols)
        return self

    def free(self):
        t, self.t = self.t, None
        if t is not None:
            t.free()

    def tensor(self):
        return self.t

    def shape(self):
        return self.rows, self.cols


HandleClass = Handle


def is_handle(x):
    return isinstance(x, Handle)


def new_handle(t, rows, cols):
    return Handle(t, rows, cols)


def pin(flat, rows, cols):
    """Upload a flat sequence once and keep it resident (luatl_adapter.lua:63-73):
    it must hold exactly rows*cols numbers."""
    _require()
    n = rows * cols
    if len(flat) != n:
        raise ValueError(f"lanternl_hip.pin: a {rows}x{cols} matrix takes exactly {n} numbers, "
                         f"the table holds {len(flat)}")
    h = Handle(Tensor.new(rows, cols), rows, cols)
    _put_f32(h.t.data, flat, n, "pin")
    return h


def alloc(rows, cols):
    """A resident zero matrix (luatl_adapter.lua:75-78)."""
    _require()
    return Handle(Tensor.new(rows, cols), rows, cols).zero()


# Device lanes for the flat-table calls: one grow-only buffer per operand lane
# (0 = first operand, 1 = second, 2 = result), sized to the next power of two
# that fits; each call gets a non-owning tensor shaped for it.
LANE_A, LANE_B, LANE_C = 0, 1, 2
_lanes = {}


def _pow2_at_least(n):
    c = 256
    while c < n:
        c *= 2
    return c


def _dev_lane(lane, rows, cols):
    need = max(rows * cols, 1)
    store = _lanes.get(lane)
    if store is None or store.nelem < need:
        if store is not None:
            store.free()
        store = Tensor.new(_pow2_at_least(need), 1)
        _lanes[lane] = store
    return Tensor(rows, cols, data=store.data)


def _operand(x, rows, cols, lane):
    """(tensor, resident): a handle's tensor, or a flat sequence copied into a device lane."""
    if is_handle(x):
        return x.t, True
    t = _dev_lane(lane, rows, cols)
    _put_f32(t.data, x, rows * cols, f"a {rows}x{cols} operand")
    return t, False


def _deliver(t, rows, cols, resident):
    """A new handle over t for resident inputs, otherwise a new flat list read back from t."""
    return Handle(t, rows, cols) if resident else _fetch_f32(t.data, rows * cols)


def _row_call(x, rows, cols, launch):
    """launch(X, O) on a flat sequence or a handle; the output takes the input's form."""
    X, resident = _operand(x, rows, cols, LANE_A)
    O = Tensor.new(rows, cols) if resident else _dev_lane(LANE_C, rows, cols)
    launch(X, O)
    return _deliver(O, rows, cols, resident)


# the flat-table products through lhip_matmul_host (double in and out)
_OPCODE = {"nn": 0, "nt": 1, "tn": 2}
_OPNAME = ("matmul", "matmul_nt", "matmul_tn")


def _extents(code, m, k, n):
    return ((m * k, k * n, m * n), (m * k, n * k, m * n), (m * k, m * n, k * n))[code]


def _doubles(x, need, what):
    vals = np.ascontiguousarray(np.asarray(x, dtype=np.float64).reshape(-1))
    if vals.size < need:
        raise ValueError(f"lanternl_hip: {what} needs {need} numbers, the table holds {vals.size}")
    return vals


def _host_product(code, a, m, k, b, n):
    """The product as a float64 array of its rows*cols numbers."""
    for d in (m, k, n):
        if isinstance(d, bool) or not isinstance(d, (int, float, np.integer, np.floating)) or d < 0 or d % 1:
            raise ValueError(f"lanternl_hip: {_OPNAME[code]} dimensions must be non-negative integers, "
                             f"got {m} x {k} x {n}")
    m, k, n = int(m), int(k), int(n)
    na, nb, nc = _extents(code, m, k, n)
    ad = _doubles(a, na, f"{_OPNAME[code]} operand a")
    bd = _doubles(b, nb, f"{_OPNAME[code]} operand b")
    res = np.empty(nc, dtype=np.float64)
    call("lhip_matmul_host", code, ad.ctypes.data_as(ctypes.c_void_p), bd.ctypes.data_as(ctypes.c_void_p),
         res.ctypes.data_as(ctypes.c_void_p), m, k, n, 0)
    return res


# ------------------------------------------------------------------ legacy entry points
def matmul(a, m, k, b, n):
    """a(m x k) . b(k x n) (luatl_adapter.lua:128-135): flat tables -> new flat
    list; two handles -> new handle; a handle and a table -> flat list."""
    _require()
    if not (is_handle(a) or is_handle(b)):
        return _host_product(0, a, m, k, b, n).tolist()
    A, ra = _operand(a, m, k, LANE_A)
    B, rb = _operand(b, k, n, LANE_B)
    resident = ra and rb
    out = Tensor.new(m, n) if resident else _dev_lane(LANE_C, m, n)
    gemm_ex(A, B, out)
    return _deliver(out, m, n, resident)


def matmul_nt(a, m, k, b, n):
    """a(m x k) . b(n x k)^T -> new flat list of m*n (matrix.lua:597-625 semantics)."""
    _require()
    return _host_product(1, a, m, k, b, n).tolist()


def matmul_tn(a, m, k, b, n):
    """a(m x k)^T . b(m x n) -> new flat list of k*n (matrix.lua:627-660 semantics)."""
    _require()
    return _host_product(2, a, m, k, b, n).tolist()


def matmul_into(op, a, m, k, b, n, rd, acc):
    """The product `op` ("nn", "nt", "tn"; shapes as in matmul / matmul_nt /
    matmul_tn) of two flat sequences, written into the caller's flat sequence
    ``rd``: the product itself, or ``rd + product`` in double when ``acc``.
    ``rd`` is written only after the device call has succeeded.  Returns rd."""
    _require()
    code = _OPCODE.get(op)
    if code is None:
        raise ValueError(f'lanternl_hip.matmul_into: op must be "nn", "nt" or "tn", got {op!r}')
    nc = _extents(code, m, k, n)[2]
    if len(rd) < nc:
        raise ValueError(f"lanternl_hip.matmul_into: rd holds {len(rd)} numbers, the product {nc}")
    res = _host_product(code, a, m, k, b, n)
    if isinstance(rd, np.ndarray):
        if acc:
            rd[:nc] += res
        else:
            rd[:nc] = res
    else:
        prev = np.asarray(rd[:nc], dtype=np.float64) if acc else 0.0
        rd[:nc] = (prev + res).tolist()
    return rd


def rmsnorm(x, rows, cols, w=None, eps=None):
    """luatl_adapter.lua:137-145: y = x * w / rms(x) per row (w None: gain 1)."""
    _require()
    gain = _operand(w, 1, cols, LANE_B)[0] if w is not None else None
    e = 1e-5 if eps is None else eps
    return _row_call(x, rows, cols, lambda X, O: call("lhip_rmsnorm_ex", X.data, gain.data if gain else None,
                                                      O.data, rows, cols, e))


def softmax(x, rows, cols):
    """luatl_adapter.lua:147-152: row softmax, no mask."""
    _require()
    return _row_call(x, rows, cols, lambda X, O: call("lhip_softmax_ex", X.data, None, O.data, rows, cols,
                                                      1.0, 0, 0, 0))


def softmax_causal(x, rows, cols, scale=None, group=None):
    """luatl_adapter.lua:154-159: causal row softmax of scale*x, mask restarting every `group` rows."""
    _require()
    sc = 1.0 if scale is None else scale
    return _row_call(x, rows, cols, lambda X, O: call("lhip_softmax_ex", X.data, None, O.data, rows, cols,
                                                      sc, 1, group or 0, 0))


# ------------------------------------------------------------------ views and gemm_ex
class View:
    """A stride view (luaTL_train.lua:113-118): data, rows, cols, rs, cs, bs."""

    __slots__ = ("data", "rows", "cols", "rs", "cs", "bs", "dtype")

    def __init__(self, data, rows, cols, rs, cs, bs=0):
        self.data, self.rows, self.cols = int(data), int(rows), int(cols)
        self.rs, self.cs, self.bs, self.dtype = int(rs), int(cs), int(bs), F32

    @property
    def nelem(self):
        return self.rows * self.cols


def _base(t):
    if is_handle(t):
        return t.t.data
    if isinstance(t, (Tensor, View)):
        return t.data
    return int(t)


def _coerce(x):
    """A tensor, handle or view as a stride view (luaTL_train.lua:143-150)."""
    if is_handle(x):
        x = x.t
    if isinstance(x, View):
        return x
    return View(x.data, x.rows, x.cols, x.cols, 1, 0)


def gemm_ex(A, B, Cc, o=None):
    """luaTL.gemm_ex (luaTL_train.lua:154-172): Cc = act(alpha*(pre(A) @ B) + bias) + beta*Cc
    on tensors or stride views; opts alpha, beta, bias, gamma, rowscale, batch, eps, pre, act."""
    o = o or {}
    a, b, c = _coerce(A), _coerce(B), _coerce(Cc)
    if b.rows != a.cols:
        raise ValueError(f"gemm_ex: inner dim mismatch {a.rows}x{a.cols} @ {b.rows}x{b.cols}")
    call("lhip_gemm_ex", a.data, b.data, c.data,
         _base(o["bias"]) if o.get("bias") is not None else None,
         _base(o["gamma"]) if o.get("gamma") is not None else None,
         _base(o["rowscale"]) if o.get("rowscale") is not None else None,
         a.rows, b.cols, a.cols, a.rs, a.cs, b.rs, b.cs, c.rs, c.cs, a.bs, b.bs, c.bs,
         int(o.get("batch", 1)), float(o.get("alpha", 1.0)), float(o.get("beta", 0.0)),
         float(o.get("eps", 1e-5)), int(o.get("pre", 0)), int(o.get("act", 0)))
    return Cc


def _t(x):
    """Logical transpose of a handle/tensor (W:t(), luaTL_train.lua:120-122)."""
    if is_handle(x):
        x = x.t
    return view(x.data, x.cols, x.rows, 1, x.cols, 0)


# ------------------------------------------------------------------ resident calls
def gemm(hA, hB, hC, opts=None):
    """luatl_adapter.lua:163: hC = gemm_ex(hA, hB, hC, opts)."""
    gemm_ex(hA.t, hB.t, hC.t, opts)
    return hC


def gemm_dx(hdY, hW, hdX, beta=None):
    """luatl_adapter.lua:164 (luaTL.matmul_dx): dX = dY . W^T + beta*dX (beta default 0)."""
    gemm_ex(hdY.t, _t(hW), hdX.t, {"beta": 0.0 if beta is None else beta})
    return hdX


def gemm_dw(hX, hdY, hdW, beta=None):
    """luatl_adapter.lua:165 (luaTL.matmul_dw): dW = X^T . dY + beta*dW (beta default 1)."""
    gemm_ex(_t(hX), hdY.t, hdW.t, {"beta": 1.0 if beta is None else beta})
    return hdW


def add_inplace(hDst, hSrc, alpha=None):
    """luatl_adapter.lua:167 (Tensor:add_inplace, luaTL.lua:633-638): the AXPY
    operator with a = dst, b = src, so dst = alpha*dst + src."""
    call("lhip_elementwise", hDst.t.data, hSrc.t.data, hDst.t.data, hDst.t.nelem, EW["AXPY"],
         1.0 if alpha is None else alpha, 0.0)
    return hDst


def silu_inplace(h):
    call("lhip_elementwise", h.t.data, None, h.t.data, h.t.nelem, EW["SILU"], 0.0, 0.0)
    return h


def gelu_inplace(h):
    call("lhip_elementwise", h.t.data, None, h.t.data, h.t.nelem, EW["GELU"], 0.0, 0.0)
    return h


def scale_inplace(h, a):
    """luatl_adapter.lua:170: h = a*h (the SCALE operator with beta 0)."""
    call("lhip_elementwise", h.t.data, None, h.t.data, h.t.nelem, EW["SCALE"], float(a), 0.0)
    return h


def _rope_call(x, o):
    o = o or {}
    heads = int(o.get("heads", 1))
    hd = int(o.get("head_dim", x.cols // heads))
    rs = int(o.get("row_stride", x.cols))
    pos = o.get("pos_ids")
    call("lhip_rope", x.data, _base(pos) if pos is not None else None, x.rows, heads, hd,
         rs if rs > 0 else heads * hd, int(o.get("pos_offset", 0)), 0, float(o.get("theta", 10000.0)),
         1 if o.get("interleaved") else 0, 1 if o.get("inverse") else 0)


def rope(h, o=None):
    """luatl_adapter.lua:172 (Tensor:rope, luaTL_train.lua:225-234): in place; half-split pairs
    unless o.interleaved; o.heads, head_dim, row_stride, pos_ids, pos_offset, theta, inverse."""
    _rope_call(h.t, o)
    return h


def _swiglu_call(a, b, out, o):
    o = o or {}
    call("lhip_swiglu_fwd", a.data, int(o.get("lda", a.cols)), b.data, int(o.get("ldb", b.cols)), out.data,
         int(o.get("ldo", out.cols)), out.rows, out.cols)


def swiglu(ha, hb, ho, o=None):
    """luatl_adapter.lua:173 (luaTL.swiglu): ho = silu(ha) * hb, leading dims from o."""
    _swiglu_call(ha.t, hb.t, ho.t, o)
    return ho


def rmsnorm_bwd(hx, hg, hdy, hdx, hdg, eps=None):
    """luatl_adapter.lua:175-178: dx from x, gain and dy (dx overwritten), dgamma accumulated."""
    x = hx.t
    call("lhip_rmsnorm_bwd_ex", x.data, hg.t.data if hg is not None else None, hdy.t.data, hdx.t.data,
         hdg.t.data if hdg is not None else None, x.rows, x.cols, 1e-5 if eps is None else eps)
    return hdx


def _softmax_bwd_call(y, dy, dx, o):
    o = o or {}
    call("lhip_softmax_bwd_ex", y.data, dy.data, dx.data, y.rows, y.cols, float(o.get("scale", 1.0)),
         1 if o.get("causal") else 0, int(o.get("group", 0)), int(o.get("mask_offset", 0)))


def softmax_bwd(hy, hdy, hdx, o=None):
    """luatl_adapter.lua:180: dx = scale * y * (dy - <dy, y>) on the kept columns."""
    _softmax_bwd_call(hy.t, hdy.t, hdx.t, o)
    return hdx


def program(cap=None, timing=None):
    """luatl_adapter.lua:182: a luaTL.Program (capacity ops, optional event timing)."""
    _require()
    return Program(cap, timing)


def sync():
    call("lhip_sync")


def stats():
    """Memory statistics under the reference's keys (luaTL.pool_stats, luaTL.lua:308-325).
    There is no caching pool: every allocation is a hipMalloc."""
    s = MemStats()
    call("lhip_mem_stats", ctypes.byref(s))
    return {"reserved": s.bytes_in_use + s.workspace_bytes + s.staging_bytes, "in_use": s.bytes_in_use,
            "peak": s.peak_in_use, "blocks": s.live_buffers, "free_blocks": 0, "allocs": s.n_alloc,
            "frees": s.n_free, "cuda_malloc": s.n_alloc, "cuda_free": s.n_free, "cache_hit": 0,
            "cache_miss": s.n_alloc, "trims": 0, "workspace": s.workspace_bytes, "staging": s.staging_bytes}


def hardware():
    """Device description under the reference's keys (luaTL.hardware, luaTL.lua:279-305)."""
    d = _device.info()
    free, total = mem()
    cus = d["compute_units"]
    return {"name": d["name"], "sm": d["arch"].split(":")[0], "major": 9, "minor": 5,
            "multiprocessors": cus, "cores_per_sm": 64, "cuda_cores": 64 * cus, "warp_size": 64,
            "max_threads_block": 1024, "max_threads_sm": 2048, "shared_per_block": d["lds_per_block"],
            "shared_per_sm": 160 * 1024, "total_vram": total, "free_vram": free, "l2_cache": d["l2_bytes"],
            "bandwidth_gbs": d["peak_hbm_gbps"], "gflops_fp32": d["peak_fp32_matrix_tflops"] * 1000.0,
            "gflops_fp16": 0.0, "tensor_cores": True, "fp16": False, "bf16": False}


def shutdown():
    global available, reason
    for lane in list(_lanes):
        _lanes.pop(lane).free()
    call("lhip_shutdown")
    available, reason = False, "shut down"


# ------------------------------------------------------------------ resident-tensor toolkit
def offset(t, elems):
    """Device address `elems` floats into a tensor/handle/view (luatl_adapter.lua:194-196)."""
    return _base(t) + 4 * int(elems)


def view(ptr, rows, cols, rs, cs, bs=0):
    """Explicit stride view (luatl_adapter.lua:200-203)."""
    return View(_base(ptr), rows, cols, rs, cs, bs)


def cols(t, col0, w):
    """Column slice [col0, col0 + w) keeping the parent's leading dimension (luatl_adapter.lua:206-209)."""
    base = t.t if is_handle(t) else t
    return View(_base(base) + 4 * int(col0), base.rows, w, base.cols, 1, 0)


def wrap(ptr, rows, cols_):
    """Non-owning tensor over a raw device address (luatl_adapter.lua:212)."""
    return Tensor(rows, cols_, data=_base(ptr))


def ids(n):
    """A zeroed device buffer for n int32 ids: an n x 1 tensor, since ids and
    fp32 values are both 4 bytes wide (luatl_adapter.lua:215-219)."""
    return alloc(n, 1)


def upload_i32(t, cbuf, n):
    a = np.ascontiguousarray(np.asarray(cbuf, dtype=np.int32).reshape(-1)[:n])
    call("lhip_upload", _base(t), a.ctypes.data, 4 * n)


def download_i32(t, cbuf, n):
    out = np.empty(n, np.int32)
    call("lhip_download", out.ctypes.data, _base(t), 4 * n)
    cbuf[:n] = out
    return cbuf


def download_f32(ptr, cbuf, n):
    out = np.empty(n, np.float32)
    call("lhip_download", out.ctypes.data, _base(ptr), 4 * n)
    cbuf[:n] = out
    return cbuf


def scalar(t):
    """The first fp32 value of a device tensor, handle or view (a loss, a norm) (luatl_adapter.lua:236-241)."""
    return _fetch_f32(_base(t), 1)[0]


def mem():
    f, t = ctypes.c_ulonglong(), ctypes.c_ulonglong()
    call("lhip_mem_info", ctypes.byref(f), ctypes.byref(t))
    return f.value, t.value


# ------------------------------------------------------------------ Program (luaTL.Program)
class ProgramFull(RuntimeError):
    pass


class Program:
    """luaTL.Program's op list (ai/gpu/luaTL_train.lua:332-632) over this library.

    Each op method queues one library call; ``run(keep)`` issues the queue on
    the library stream (then, unless ``async_(True)``, waits and, with timing,
    reads the elapsed time) and clears it unless ``keep``; ``capture()`` records
    the queue once into a hipGraph (run it first: a recording cannot allocate);
    ``replay()`` launches the graph, or runs the queue when nothing is captured.
    ``barrier()`` waits for the stream when run and is skipped in a capture, as
    luaTL_prog_capture skips SYNC ops (luaTL_train.cu:1614-1660)."""

    def __init__(self, capacity=None, timing=None):
        self.capacity = int(capacity) if capacity and capacity > 0 else 4096
        self.timing = bool(timing)
        self.ops = []
        self.flags = 1
        self.last_ms = -1.0
        self.total_runs = 0
        self._graph = None
        self._timer = _device.Timer() if self.timing else None

    # queue management
    def reset(self):
        self.ops = []
        return self

    def _push(self, fn, sync=False):
        if len(self.ops) >= self.capacity:
            raise ProgramFull(f"luaTL.Program full ({self.capacity})")
        self.ops.append((fn, sync))
        return self

    def size(self):
        return len(self.ops)

    def async_(self, on):
        self.flags = 0 if on else 1
        return self

    # ops (luaTL_train.lua:365-606)
    def gemm(self, A, B, Cc, o=None):
        o = dict(o or {})
        return self._push(lambda: gemm_ex(A, B, Cc, o))

    def matmul(self, A, B, Cc, o=None):
        return self.gemm(A, B, Cc, o)

    def dx(self, dY, W, dX, beta=None):
        return self.gemm(dY, _t(W), dX, {"beta": 0.0 if beta is None else beta})

    def dw(self, X, dY, dW, beta=None):
        return self.gemm(_t(X), dY, dW, {"beta": 1.0 if beta is None else beta})

    def ew(self, op, A, B, out, alpha=None, beta=None):
        al, be = 1.0 if alpha is None else alpha, 0.0 if beta is None else beta
        return self._push(lambda: call("lhip_elementwise", _base(A) if A is not None else None,
                                       _base(B) if B is not None else None, _base(out), out.nelem, op, al, be))

    def add(self, A, B, out):
        return self.ew(EW["ADD"], A, B, out, 1, 1)

    def axpy(self, dst, B, a=None):
        return self.ew(EW["AXPY"], dst, B, dst, 1 if a is None else a, 0)

    def scale(self, dst, a):
        return self.ew(EW["SCALE"], dst, None, dst, a, 0)

    def dsilu(self, x, dy, out):
        return self.ew(EW["DSILU"], x, dy, out, 1, 0)

    def dgelu(self, x, dy, out):
        return self.ew(EW["DGELU"], x, dy, out, 1, 0)

    def rmsnorm(self, x, w, out, eps=None):
        e = 1e-5 if eps is None else eps
        return self._push(lambda: call("lhip_rmsnorm_ex", x.data, _base(w) if w is not None else None, out.data,
                                       x.rows, x.cols, e))

    def rmsnorm_bwd(self, x, gamma, dy, dx, dgamma=None, eps=None):
        e = 1e-5 if eps is None else eps
        return self._push(lambda: call("lhip_rmsnorm_bwd_ex", x.data, _base(gamma) if gamma is not None else None,
                                       dy.data, dx.data, _base(dgamma) if dgamma is not None else None,
                                       x.rows, x.cols, e))

    def softmax(self, x, out, o=None):
        o = dict(o or {})
        bias = o.get("bias")
        return self._push(lambda: call("lhip_softmax_ex", x.data, _base(bias) if bias is not None else None,
                                       out.data, x.rows, x.cols, float(o.get("scale", 1.0)),
                                       1 if o.get("causal") else 0, int(o.get("group", 0)),
                                       int(o.get("mask_offset", 0))))

    def softmax_bwd(self, y, dy, dx, o=None):
        o = dict(o or {})
        return self._push(lambda: _softmax_bwd_call(y, dy, dx, o))

    def swiglu(self, a, b, out, o=None):
        o = dict(o or {})
        return self._push(lambda: _swiglu_call(a, b, out, o))

    def swiglu_bwd(self, a, b, dout, da, db, o=None):
        o = dict(o or {})
        return self._push(lambda: call("lhip_swiglu_bwd_ex", a.data, b.data, dout.data,
                                       _base(da) if da is not None else None, _base(db) if db is not None else None,
                                       dout.rows, dout.cols, int(o.get("lda", a.cols)), int(o.get("ldb", b.cols)),
                                       int(o.get("ldo", dout.cols))))

    def rope(self, x, o=None):
        o = dict(o or {})
        return self._push(lambda: _rope_call(x, o))

    def embed(self, ids_, tbl, out):
        return self._push(lambda: call("lhip_embed_fwd", tbl.data, _base(ids_), out.data, out.rows, out.cols,
                                       tbl.rows))

    def embed_bwd(self, ids_, dout, dtable, scale=None):
        s = 1.0 if scale is None else scale
        return self._push(lambda: call("lhip_embed_bwd", dout.data, _base(ids_), dtable.data, dout.rows,
                                       dout.cols, dtable.rows, s, 1))

    def cross_entropy(self, logits, targets, losses, dlogits=None, o=None):
        o = dict(o or {})
        gs = float(o.get("grad_scale", 1.0 / logits.rows))
        return self._push(lambda: call("lhip_ce_fused", logits.data, _base(targets), _base(losses),
                                       _base(dlogits) if dlogits is not None else None, logits.rows, logits.cols,
                                       int(o.get("ignore_index", -1)), gs))

    def reduce_cols(self, x, out, alpha=None, beta=None, rs=None):
        return self._push(lambda: call("lhip_reduce_cols", x.data, _base(out), x.rows, x.cols,
                                       x.cols if not rs else rs, 1.0 if alpha is None else alpha,
                                       0.0 if beta is None else beta))

    def l2(self, x, acc):
        return self._push(lambda: call("lhip_l2_accum", x.data, x.nelem, _base(acc)))

    def clip(self, x, nsq, max_norm):
        return self._push(lambda: call("lhip_clip_by_nsq", x.data, x.nelem, _base(nsq), float(max_norm)))

    def adamw(self, w, g, m, v, w_lp=None, o=None):
        o = dict(o or {})
        return self._push(lambda: call("lhip_adamw_elementwise", w.data, g.data, m.data, v.data,
                                       _base(w_lp) if w_lp is not None else None, w.nelem, int(o.get("step", 1)),
                                       float(o.get("lr", 1e-3)), float(o.get("beta1", 0.9)),
                                       float(o.get("beta2", 0.999)), float(o.get("eps", 1e-8)),
                                       float(o.get("wd", 0.0)), float(o.get("clip", 0.0))))

    def zero(self, t):
        return self._push(lambda: call("lhip_zero", t.data, t.nbytes))

    def copy(self, src, dst):
        return self._push(lambda: call("lhip_copy", dst.data, src.data, src.nbytes))

    def cast(self, src, dst):
        if getattr(src, "dtype", F32) != F32 or getattr(dst, "dtype", F32) != F32:
            raise NotImplementedError("luaTL.Program:cast: this build holds fp32 only")
        return self.copy(src, dst)

    def transpose(self, x, out):
        return self._push(lambda: call("lhip_transpose", x.data, out.data, x.rows, x.cols))

    def bcast_add(self, x, vec, out, alpha=None):
        a = 1.0 if alpha is None else alpha
        return self._push(lambda: call("lhip_bcast_add", x.data, _base(vec) if vec is not None else None,
                                       out.data, x.rows, x.cols, a))

    def barrier(self):
        return self._push(lambda: call("lhip_sync"), sync=True)

    def argmax(self, x, out):
        return self._push(lambda: call("lhip_argmax_rows", x.data, _base(out), x.rows, x.cols))

    def sum(self, x, acc, scale=None):
        s = 1.0 if scale is None else scale
        return self._push(lambda: call("lhip_sum_accum", x.data, x.nelem, s, _base(acc)))

    def gather(self, src, idx, dst):
        return self._push(lambda: call("lhip_embed_fwd", src.data, _base(idx), dst.data, dst.rows, dst.cols,
                                       src.rows))

    def row_rms(self, x, out, eps=None, rs=None, cs=None):
        e = 1e-5 if eps is None else eps
        return self._push(lambda: call("lhip_row_rms", x.data, _base(out), x.rows, x.cols,
                                       rs if rs else x.cols, cs if cs else 1, e))

    # execution (luaTL_train.lua:607-632; luaTL_train.cu:1563-1700)
    def _finish(self):
        if self.flags & 1:
            if self._timer is not None:
                self.last_ms = self._timer.ms()
            else:
                _device.sync()
        self.total_runs += 1

    def run(self, keep=False):
        if not self.ops:
            return self
        if self._timer is not None:
            self._timer.start()
        for fn, _ in self.ops:
            fn()
        if self._timer is not None:
            self._timer.stop()
        self._finish()
        if not keep:
            self.ops = []
        return self

    def capture(self):
        """Record the current queue as a hipGraph (barriers skipped).  Run it first."""
        if not self.ops:
            raise ValueError("Program:capture: the op list is empty (ARG)")
        self.free_graph()
        _device.sync()
        self._graph = _device.Program.record(lambda: [fn() for fn, sync in self.ops if not sync])
        return self

    def replay(self):
        if self._graph is None:
            return self.run(keep=True)
        if self._timer is not None:
            self._timer.start()
        self._graph.replay()
        if self._timer is not None:
            self._timer.stop()
        self._finish()
        return self

    def wait(self):
        _device.sync()
        if self._timer is not None:
            self.last_ms = self._timer.ms()
        return self

    def elapsed_ms(self):
        return self.last_ms

    def is_captured(self):
        return self._graph is not None

    def free_graph(self):
        if self._graph is not None:
            self._graph.free()
            self._graph = None
        return self
