"""GPU tests of lanternl_amd/lua/luatl_adapter.lua itself, executed (in
tests/lua_vm.py, over ctypes) against liblanternl_hip.so, as LuaJIT would run
it: `require("luatl_adapter")`, its ffi.cdef, its helper layer and every call
it makes.

* tests/test.lua:436-475 (the reference adapter test) replayed as Lua;
* the flat-table products (matmul, matmul_nt, matmul_tn, matmul_into with and
  without acc) against the oracle, and the error paths that leave `rd` alone;
* the matrix.lua patch (lanternl_amd/lua/matrix_patch.lua), run with this adapter as the
  `luatl_adapter` backend: the CPU backward's calls with `out` and `acc = true`
  at config C1 and at config C2's per-window shapes are served by the backend
  and agree with the oracle;
* the legacy row calls, gemm_ex on stride views, the resident row and
  elementwise calls, and luaTL.Program's op list (run, captured, replayed)
  against the oracle.

Bars as for the Python mirror (tests/test_adapter_gpu.py): GEMM results
relative Frobenius <= 1e-4, row and elementwise results <= 1e-5, argmax
bit-exact, a captured replay bit-identical to the eager run.
"""
import os

import numpy as np
import pytest

import oracle as O
from lanternl_amd import device
from tests import lua_registry as R
from tests.gpu_util import announce, f32, rel_fro
from tests.lua_vm import LuaError, LuaTable, LuaVM

pytestmark = pytest.mark.gpu
GEMM, ROW = 1e-4, 1e-5
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LUA_DIR = os.path.join(ROOT, "lanternl_amd", "lua")


class Lua:
    """The adapter module loaded by `require` in a fresh interpreter."""

    def __init__(self):
        self.vm = LuaVM()
        self.vm.search_dirs.append(LUA_DIR)
        self.M = self.vm.call(self.vm.G.rawget("require"), "luatl_adapter")[0]

    def __call__(self, name, *args):
        return self.vm.call(self.vm.index(self.M, name), *args)

    def method(self, obj, name, *args):
        return self.vm.call(self.vm.index(obj, name), obj, *args)

    def run(self, src, *args):
        return self.vm.call(self.vm.load(src, "test chunk"), *args)

    def pin(self, a):
        a = np.asarray(a, np.float32)
        r, c = (a.shape if a.ndim == 2 else (a.size, 1))
        return self("pin", flat(a), float(r), float(c))[0]

    def dl(self, x):
        """A tensor, handle or view's rows x cols elements (contiguous from its data)."""
        self("sync")
        t = self.vm.index(x, "t") if self("is_handle", x)[0] else x
        rows, cols = int(t.rawget("rows")), int(t.rawget("cols"))
        buf = self.vm.ffi.new("float[?]", rows * cols)
        self("download_f32", t, buf, float(rows * cols))
        return np.frombuffer(buf.obj, np.float32).reshape(rows, cols).astype(np.float64)


def flat(a):
    return LuaTable.from_list([float(v) for v in np.asarray(a, np.float64).ravel()])


def arr(t, *shape):
    return np.array(t.to_list(), np.float64).reshape(shape)


def opts(**kw):
    return LuaTable({k: (float(v) if isinstance(v, (int, float)) and not isinstance(v, bool) else v)
                     for k, v in kw.items()})


@pytest.fixture(scope="module")
def L():
    device.init(0)
    lua = Lua()
    assert lua.M.rawget("available") is True, lua.M.rawget("reason")
    return lua


# ----------------------------------------------------------- module contract
def test_module_fields(L):
    M = L.M
    assert M.rawget("name") == "luatl" and M.rawget("reason") == "ready" and M.rawget("error") is None
    from lanternl_amd import backend as mirror
    assert isinstance(M.rawget("device"), str) and M.rawget("device") == mirror.device   # hipDeviceProp_t.name
    assert M.rawget("luaTL") is None
    for fn in ("matmul", "matmul_nt", "matmul_tn", "matmul_into", "rmsnorm", "softmax", "softmax_causal", "gemm",
               "gemm_dx", "gemm_dw", "program", "pin", "alloc", "hardware", "stats", "shutdown"):
        assert callable(M.rawget(fn)), fn


# ----------------------------------------------------------- tests/test.lua:436-475
REPLAY = r'''
local ad = require("luatl_adapter")
assert(ad.available, ad.error)
local function near(x, y, tol)
    if #x ~= #y then return false end
    for i = 1, #x do
        if math.abs(x[i] - y[i]) > tol then return false end
    end
    return true
end
local a = { 1, 2, 3, 4, 5, 6 }            -- 2x3
local b = { 1, 0, 0, 1, 1, 1 }            -- 3x2
local c = ad.matmul(a, 2, 3, b, 2)
assert(near(c, { 4, 5, 10, 11 }, 1e-4), "flat matmul")
assert(type(c) == "table" and getmetatable(c) == nil and c[1] ~= nil, "a plain table comes back")
local hA, hB = ad.pin(a, 2, 3), ad.pin(b, 3, 2)
local hC = ad.matmul(hA, 2, 3, hB, 2)
assert(ad.is_handle(hC), "two handles give a handle")
assert(near(hC:toflat(), c, 1e-4), "the handle holds the same product")
local hdY = ad.pin({ 1, 1, 1, 1 }, 2, 2)
local hdX = ad.alloc(2, 3)
ad.gemm_dx(hdY, hB, hdX)                  -- ones(2x2) . B^T
assert(near(hdX:toflat(), { 1, 1, 2, 1, 1, 2 }, 1e-5), "gemm_dx")
local hdW = ad.alloc(3, 2)
ad.gemm_dw(hA, hdY, hdW, 0.0)             -- A^T . ones(2x2)
assert(near(hdW:toflat(), { 5, 5, 7, 7, 9, 9 }, 1e-5), "gemm_dw")
local sm = ad.softmax_causal({ 1, 2, 3, 4 }, 2, 2, 1.0)
assert(math.abs(sm[2]) < 1e-6 and math.abs(sm[1] - 1.0) < 1e-6, "causal mask")
local mixed = ad.matmul(hA, 2, 3, b, 2)
assert(not ad.is_handle(mixed) and near(mixed, c, 1e-4), "a handle with a table gives a table")
for _, h in ipairs({ hA, hB, hC, hdY, hdX, hdW }) do h:free() end
assert(hA.t == nil, "free drops the tensor")
return #c, ad.device
'''


def test_reference_adapter_test_replayed_in_lua(L):
    announce("lua module", "tests/test.lua:436-475")
    n, dev = L.run(REPLAY)
    assert n == 4.0 and dev == L.M.rawget("device")


def test_count_errors_and_pin_messages(L):
    with pytest.raises(LuaError, match="takes exactly 4 numbers, the table holds 3"):
        L("pin", flat([1, 2, 3]), 2.0, 2.0)
    with pytest.raises(LuaError, match="takes exactly 4 numbers, the table holds 5"):
        L("pin", flat([1, 2, 3, 4, 5]), 2.0, 2.0)
    with pytest.raises(LuaError, match="matmul operand a needs 6 numbers, the table holds 4"):
        L("matmul", flat([1, 2, 3, 4]), 2.0, 3.0, flat([1, 0, 0, 1, 1, 1]), 2.0)
    h = L.pin(np.ones((2, 2)))
    with pytest.raises(LuaError, match="needs 4 numbers, the table holds 1"):
        L.method(h, "upload", flat([1.0]))
    L.method(h, "free")


# ----------------------------------------------------------- flat-table products
OPS = {"nn": (O.mm, lambda m, k, n: ((m, k), (k, n), (m, n))),
       "nt": (O.matmul_nt, lambda m, k, n: ((m, k), (n, k), (m, n))),
       "tn": (O.matmul_tn, lambda m, k, n: ((m, k), (m, n), (k, n)))}
ENTRY = {"nn": "matmul", "nt": "matmul_nt", "tn": "matmul_tn"}


@pytest.mark.parametrize("op", ["nn", "nt", "tn"])
@pytest.mark.parametrize("mkn", [(33, 17, 29), (1, 64, 1), (256, 128, 256)])
def test_flat_products_vs_oracle(L, op, mkn):
    announce("lua module", f"{ENTRY[op]} {mkn}")
    m, k, n = mkn
    fn, shapes = OPS[op]
    sa, sb, sc = shapes(m, k, n)
    rng = np.random.default_rng(m * 7 + k * 3 + n)
    a, b = f32(rng.standard_normal(sa)), f32(rng.standard_normal(sb))
    got = L(ENTRY[op], flat(a), float(m), float(k), flat(b), float(n))[0]
    assert isinstance(got, LuaTable) and got.meta is None
    assert rel_fro(arr(got, *sc), fn(a, b)) <= GEMM
    # matmul_into: overwrite, then accumulate onto a non-zero table, in double
    rd0 = rng.standard_normal(sc)
    rd = flat(rd0)
    assert L("matmul_into", op, flat(a), float(m), float(k), flat(b), float(n), rd, False)[0] is rd
    assert rel_fro(arr(rd, *sc), fn(a, b)) <= GEMM
    rd = flat(rd0)
    L("matmul_into", op, flat(a), float(m), float(k), flat(b), float(n), rd, True)
    want = fn(a, b, rd0.copy(), acc=True)
    assert rel_fro(arr(rd, *sc), want) <= GEMM
    assert rel_fro(arr(rd, *sc) - rd0, fn(a, b)) <= GEMM      # the added product alone


def test_matmul_into_errors_leave_rd_untouched(L):
    rd0 = [float(i) for i in range(6)]
    rd = LuaTable.from_list(list(rd0))
    a, b = flat(np.ones((2, 3))), flat(np.ones((3, 3)))
    with pytest.raises(LuaError, match='op must be "nn", "nt" or "tn", got xx'):
        L("matmul_into", "xx", a, 2.0, 3.0, b, 3.0, rd, True)
    with pytest.raises(LuaError, match="rd must be a flat table of 6 numbers"):
        L("matmul_into", "nn", a, 2.0, 3.0, b, 3.0, LuaTable.from_list([0.0] * 5), True)
    with pytest.raises(LuaError, match="matmul operand b needs 9 numbers, the table holds 4"):
        L("matmul_into", "nn", a, 2.0, 3.0, flat(np.ones(4)), 3.0, rd, True)
    with pytest.raises(LuaError, match="matmul_tn dimensions must be non-negative integers, got 2 x 3 x 1.5"):
        L("matmul_into", "tn", a, 2.0, 3.0, b, 1.5, rd, True)
    assert rd.to_list() == rd0
    with pytest.raises(LuaError, match="matmul dimensions must be non-negative integers, got 2.5 x 3 x 3"):
        L("matmul", a, 2.5, 3.0, b, 3.0)
    with pytest.raises(LuaError, match="matmul_nt dimensions must be non-negative integers, got -1 x 3 x 3"):
        L("matmul_nt", a, -1.0, 3.0, b, 3.0)


# ----------------------------------------------------------- the matrix.lua patch with this backend
# forward products and their backward calls (tensor2.lua:206-211,222-227):
# (name, kind, x shape, w shape)
FORWARD = [
    ("C1 a.b", "matmul", (256, 128), (128, 256)),
    ("C2 q/k/v/o", "matmul", (64, 128), (128, 128)),
    ("C2 W2", "matmul", (64, 256), (256, 128)),
    ("C2 P.V", "matmul", (64, 64), (64, 16)),
    ("C2 tied head", "matmul_nt", (64, 128), (2000, 128)),
    ("C2 QK^T", "matmul_nt", (64, 16), (64, 16)),
]


@pytest.fixture(scope="module")
def patched(L):
    matrix, backends = R.build(L.vm, [("luatl_adapter", L.M)])
    assert backends.rawget(1).rawget("available") is True
    return matrix


@pytest.mark.parametrize("name,kind,xs,ws", FORWARD, ids=[f[0] for f in FORWARD])
def test_patch_serves_backward_calls_with_out_and_acc(L, patched, name, kind, xs, ws):
    announce("lua module + matrix.lua patch", name)
    rng = np.random.default_rng(sum(xs) * 31 + sum(ws))
    x, w = f32(rng.standard_normal(xs)), f32(rng.standard_normal(ws))
    ys = (xs[0], ws[1]) if kind == "matmul" else (xs[0], ws[0])
    g = f32(rng.standard_normal(ys))
    gx0, gw0 = rng.standard_normal(xs), rng.standard_normal(ws)
    call = lambda fname, p, q, out: L.vm.call(L.vm.index(patched, fname), R.lua_matrix(p), R.lua_matrix(q),  # noqa: E731
                                              out, True)
    gx, gw = R.lua_matrix(gx0), R.lua_matrix(gw0)
    if kind == "matmul":        # y = x.w: dx += g.w^T, dw += x^T.g
        call("matmul_nt", g, w, gx)
        assert patched.rawget("last_backend") == "luatl_adapter"
        call("matmul_tn", x, g, gw)
        want_x, want_w = O.matmul_nt(g, w, gx0.copy(), acc=True), O.matmul_tn(x, g, gw0.copy(), acc=True)
    else:                       # s = x.w^T: dx += g.w, dw += g^T.x
        call("multiply", g, w, gx)
        assert patched.rawget("last_backend") == "luatl_adapter"
        call("matmul_tn", g, x, gw)
        want_x, want_w = O.mm(g, w, gx0.copy(), acc=True), O.matmul_tn(g, x, gw0.copy(), acc=True)
    assert patched.rawget("last_backend") == "luatl_adapter"
    got_x = arr(gx.rawget("data"), *xs)
    got_w = arr(gw.rawget("data"), *ws)
    assert rel_fro(got_x, want_x) <= GEMM and rel_fro(got_w, want_w) <= GEMM
    assert rel_fro(got_x - gx0, want_x - gx0) <= GEMM and rel_fro(got_w - gw0, want_w - gw0) <= GEMM


def test_patch_small_call_stays_in_lua(L, patched):
    a, b = np.arange(6.0).reshape(2, 3), np.arange(12.0).reshape(3, 4)
    out = R.lua_matrix(np.ones((2, 4)))
    L.vm.call(L.vm.index(patched, "multiply"), R.lua_matrix(a), R.lua_matrix(b), out, True)
    assert patched.rawget("last_backend") == "lua"
    np.testing.assert_array_equal(arr(out.rawget("data"), 2, 4), 1 + a @ b)


# ----------------------------------------------------------- legacy row calls
def test_legacy_rmsnorm_and_softmax_vs_oracle(L):
    announce("lua module", "legacy rmsnorm/softmax")
    rng = np.random.default_rng(31)
    rows, cols = 24, 40
    x = f32(rng.standard_normal((rows, cols)))
    w = f32(rng.normal(1, 0.1, cols))
    r, c = float(rows), float(cols)
    y = arr(L("rmsnorm", flat(x), r, c, flat(w), 1e-6)[0], rows, cols)
    assert rel_fro(y, O.rmsnorm_fwd(x, w, 1e-6)[0]) <= ROW
    y1 = arr(L("rmsnorm", flat(x), r, c)[0], rows, cols)
    assert rel_fro(y1, O.rmsnorm_fwd(x, np.ones(cols), 1e-5)[0]) <= ROW
    hy = L("rmsnorm", L.pin(x), r, c, L.pin(w), 1e-6)[0]
    assert L("is_handle", hy)[0] and rel_fro(L.dl(hy), O.rmsnorm_fwd(x, w, 1e-6)[0]) <= ROW
    s = arr(L("softmax", flat(x), r, c)[0], rows, cols)
    assert rel_fro(s, O.softmax_ex(x)) <= ROW
    sc = arr(L("softmax_causal", flat(x), r, c, 0.25, 8.0)[0], rows, cols)
    assert rel_fro(sc, O.softmax_ex(x, None, 0.25, True, 8, 0)) <= ROW


# ----------------------------------------------------------- gemm_ex on stride views
@pytest.mark.parametrize("case", ["plain", "alpha_beta_cm", "bias_gelu", "pre_rmsnorm", "heads_batched"])
def test_gemm_ex_on_views_vs_oracle(L, case):
    announce("lua module gemm_ex", case)
    rng = np.random.default_rng(sum(map(ord, case)) + 1)
    M_, N, K = 37, 29, 45
    kw, extras_on, batch = {}, (), 1
    strides = (K, 1, N, 1, N, 1, 0, 0, 0)
    if case == "alpha_beta_cm":
        strides, kw = (1, M_, N, 1, 1, M_, 0, 0, 0), dict(alpha=0.5, beta=-2.0)
    elif case == "bias_gelu":
        kw, extras_on = dict(alpha=1.5, beta=0.5, act=2), ("bias",)
    elif case == "pre_rmsnorm":
        kw, extras_on = dict(pre=1, eps=1e-6), ("gamma",)
    elif case == "heads_batched":
        T, H, hd = 64, 8, 16
        M_, N, K, batch = T, T, hd, H
        strides, kw = (H * hd, 1, 1, H * hd, T, 1, hd, hd, T * T), dict(alpha=0.25)
    a_rs, a_cs, b_rs, b_cs, c_rs, c_cs, a_bs, b_bs, c_bs = strides
    na = (M_ - 1) * a_rs + (K - 1) * a_cs + (batch - 1) * a_bs + 1
    nb = (K - 1) * b_rs + (N - 1) * b_cs + (batch - 1) * b_bs + 1
    nc = (M_ - 1) * c_rs + (N - 1) * c_cs + (batch - 1) * c_bs + 1
    A, B, C0 = (f32(rng.standard_normal(n)) for n in (na, nb, nc))
    extras = {k: f32(rng.normal(1 if k == "gamma" else 0, 0.3, N if k == "bias" else K)) for k in extras_on}
    ref = C0.copy()
    O.gemm_ex(A, B, ref, M_, N, K, strides, batch=batch, bias=extras.get("bias"), gamma=extras.get("gamma"),
              **kw)
    hA, hB, hC = L.pin(A), L.pin(B), L.pin(C0)
    o = opts(batch=batch, **kw)
    for k, v in extras.items():
        o.rawset(k, L.pin(v))
    fl = float
    av = L("view", hA, fl(M_), fl(K), fl(a_rs), fl(a_cs), fl(a_bs))[0]
    bv = L("view", hB, fl(K), fl(N), fl(b_rs), fl(b_cs), fl(b_bs))[0]
    cv = L("view", hC, fl(M_), fl(N), fl(c_rs), fl(c_cs), fl(c_bs))[0]
    assert L("gemm_ex", av, bv, cv, o)[0] is cv
    got = L.dl(hC).ravel()
    idx = np.array([z * c_bs + i * c_rs + j * c_cs for z in range(batch) for i in range(M_) for j in range(N)])
    assert rel_fro(got[idx], ref[idx]) <= GEMM
    with pytest.raises(LuaError, match="inner dim mismatch"):
        L("gemm_ex", av, av, cv, o)


# ----------------------------------------------------------- resident row and elementwise calls
def test_resident_row_and_elementwise_calls_vs_oracle(L):
    announce("lua module", "resident rmsnorm_bwd/softmax_bwd/swiglu/rope/inplace")
    rng = np.random.default_rng(32)
    rows, cols = 48, 64
    x = f32(rng.standard_normal((rows, cols))); g = f32(rng.normal(1, 0.1, cols))
    dy = f32(rng.standard_normal((rows, cols)))
    hx, hg, hdy = L.pin(x), L.pin(g.reshape(1, -1)), L.pin(dy)
    hdx = L("alloc", float(rows), float(cols))[0]
    dg0 = f32(rng.standard_normal(cols))
    hdg = L.pin(dg0.reshape(1, -1))
    L("rmsnorm_bwd", hx, hg, hdy, hdx, hdg, 1e-6)
    dg_ref = dg0.copy()
    dx_ref = O.rmsnorm_bwd_luatl(x, g, dy, 1e-6, dg_ref)
    assert rel_fro(L.dl(hdx), dx_ref) <= ROW and rel_fro(L.dl(hdg).ravel(), dg_ref) <= ROW
    L("rmsnorm_bwd", hx, None, hdy, hdx, None)
    assert rel_fro(L.dl(hdx), O.rmsnorm_bwd_luatl(x, None, dy, 1e-5)) <= ROW
    for o in ({}, {"scale": 0.5, "causal": True, "group": 16}, {"causal": True, "mask_offset": -3}):
        y = O.softmax_ex(x, None, o.get("scale", 1.0), o.get("causal", False), o.get("group", 0),
                         o.get("mask_offset", 0))
        L("softmax_bwd", L.pin(y), hdy, hdx, opts(**o))
        ref = O.softmax_bwd_ex(f32(y), dy, o.get("scale", 1.0), o.get("causal", False), o.get("group", 0),
                               o.get("mask_offset", 0))
        assert rel_fro(L.dl(hdx), ref) <= ROW, o
    # swiglu on the packed [rows, 2F] layout: b is a wrapped offset into the same buffer
    F = 32
    packed = f32(rng.standard_normal((rows, 2 * F)))
    hp = L.pin(packed)
    ho = L("alloc", float(rows), float(F))[0]
    tb = L("wrap", L("offset", hp, float(F))[0], float(rows), float(F))[0]
    hb = L("new_handle", tb, float(rows), float(F))[0]
    L("swiglu", hp, hb, ho, opts(lda=2 * F, ldb=2 * F))
    assert rel_fro(L.dl(ho), O.swiglu_fwd(packed[:, :F], packed[:, F:])) <= ROW
    H, hd = 4, 16
    q = f32(rng.standard_normal((rows, H * hd)))
    for o in ({"heads": H}, {"heads": H, "interleaved": True, "pos_offset": 5, "theta": 500.0},
              {"heads": H, "inverse": True}):
        hq = L.pin(q)
        L("rope", hq, opts(**o))
        ref = O.rope_heads(q, H, hd, H * hd, o.get("pos_offset", 0), o.get("theta", 10000.0),
                           o.get("interleaved", False), o.get("inverse", False))
        assert rel_fro(L.dl(hq), ref) <= ROW, o
    a = f32(rng.standard_normal((16, 20))); b = f32(rng.standard_normal((16, 20)))
    ha, hb2 = L.pin(a), L.pin(b)
    L("add_inplace", ha, hb2, 0.5)
    assert rel_fro(L.dl(ha), 0.5 * a + b) <= ROW
    for fn, arg, want in (("scale_inplace", (-3.0,), -3.0 * a), ("silu_inplace", (), O.ew("SILU", a, None)),
                          ("gelu_inplace", (), O.ew("GELU", a, None))):
        L.method(ha, "upload", flat(a))
        L(fn, ha, *arg)
        assert rel_fro(L.dl(ha), want) <= ROW, fn


def test_ids_scalar_and_column_views(L):
    n = 10
    ids = L("ids", float(n))[0]
    src = L.vm.ffi.new("int[?]", n, *[float(3 * i - 7) for i in range(n)])
    L("upload_i32", ids, src, float(n))
    back = L.vm.ffi.new("int[?]", n)
    L("download_i32", ids, back, float(n))
    assert list(np.frombuffer(back.obj, np.int32)) == [3 * i - 7 for i in range(n)]
    x = f32(np.arange(12).reshape(3, 4))
    hx = L.pin(x)
    assert L("scalar", hx)[0] == 0.0
    cv = L("cols", hx, 1.0, 2.0)[0]                       # columns 1..2, leading dimension 4
    assert cv.rawget("rs") == 4.0 and cv.rawget("cols") == 2.0
    out = L("alloc", 3.0, 2.0)[0]
    L("gemm_ex", cv, L("view", L.pin(np.eye(2)), 2.0, 2.0, 2.0, 1.0)[0], L.vm.index(out, "t"))
    np.testing.assert_array_equal(L.dl(out), x[:, 1:3])


# ----------------------------------------------------------- luaTL.Program
PROGRAM = r'''
local ad, x, w, g, tgt, N, D, V = ...
local ffi = require("ffi")
local T = {}
local shapes = { x = { N, D }, w = { D, V }, g = { 1, D }, h = { N, D }, logits = { N, V }, p = { N, V },
                 loss = { N, 1 }, dlog = { N, V }, l2 = { 1, 1 }, lsum = { 1, 1 }, am = { N, 1 }, dw = { D, V } }
for k, s in pairs(shapes) do T[k] = ad.alloc(s[1], s[2]):tensor() end
ad.new_handle(T.x, N, D):upload(x)
ad.new_handle(T.w, D, V):upload(w)
ad.new_handle(T.g, 1, D):upload(g)
local ids = ad.ids(N)
local ib = ffi.new("int[?]", N)
for i = 0, N - 1 do ib[i] = tgt[i + 1] end
ad.upload_i32(ids, ib, N)
local function queue(P)
    P:zero(T.l2):zero(T.lsum)
    P:rmsnorm(T.x, T.g, T.h, 1e-5)
    P:gemm(T.h, T.w, T.logits)
    P:softmax(T.logits, T.p, { scale = 0.5 })
    P:cross_entropy(T.logits, ids.t, T.loss, T.dlog, { grad_scale = 1 / N })
    P:argmax(T.logits, T.am)
    P:dw(T.h, T.dlog, T.dw, 0.0)
    P:l2(T.dw, T.l2)
    P:sum(T.loss, T.lsum, 1 / N)
    P:barrier()
    P:axpy(T.w, T.dw, 1.0)
    return P
end
local function argmax_back()
    local b = ffi.new("int[?]", N)
    ad.download_i32(T.am, b, N)
    local t = {}
    for i = 0, N - 1 do t[i + 1] = b[i] end
    return t
end
return T, queue, argmax_back
'''


def test_program_op_list_run_capture_replay(L):
    announce("lua module", "luaTL.Program ops")
    rng = np.random.default_rng(35)
    N, D, V = 64, 32, 50
    x = f32(rng.standard_normal((N, D))); w = f32(rng.standard_normal((D, V)) * 0.2)
    gam = f32(rng.normal(1, 0.1, D)); tgt = rng.integers(0, V, N).astype(np.int32)
    T, queue, argmax_back = L.run(PROGRAM, L.M, flat(x), flat(w), flat(gam), flat(tgt), float(N), float(D),
                                  float(V))
    P = L("program", 64.0, True)[0]
    L.vm.call(queue, P)
    assert L.method(P, "size")[0] == 12.0 and L.method(P, "is_captured")[0] is False
    L.method(P, "run", True)
    assert L.method(P, "elapsed_ms")[0] > 0
    keys = ("h", "logits", "p", "loss", "dlog", "dw", "l2", "lsum", "w")
    eager = {k: L.dl(T.rawget(k)) for k in keys}
    am = np.array(L.vm.call(argmax_back)[0].to_list(), np.int64)
    assert rel_fro(eager["h"], O.rmsnorm_fwd(x, gam, 1e-5)[0]) <= ROW
    assert rel_fro(eager["logits"], O.mm(f32(eager["h"]), w)) <= GEMM
    assert rel_fro(eager["p"], O.softmax_ex(f32(eager["logits"]), None, 0.5)) <= ROW
    l_ref, d_ref = O.ce_fused(f32(eager["logits"]), tgt, -1, 1.0 / N)
    assert np.max(np.abs(eager["loss"].ravel() - l_ref)) <= 1e-5 and rel_fro(eager["dlog"], d_ref) <= ROW
    assert np.array_equal(am, O.argmax_rows(f32(eager["logits"])))
    assert rel_fro(eager["dw"], O.matmul_tn(f32(eager["h"]), f32(eager["dlog"]))) <= GEMM
    assert abs(eager["l2"][0, 0] - np.sum(eager["dw"] ** 2)) <= 1e-5 * np.sum(eager["dw"] ** 2)
    assert abs(eager["lsum"][0, 0] - np.mean(eager["loss"])) <= 1e-6
    assert rel_fro(eager["w"], w + eager["dw"]) <= ROW
    # a captured replay runs one more step from the current weights; the eager
    # run of the same queue from the same weights matches it bit for bit
    L.method(P, "capture")
    assert L.method(P, "is_captured")[0] is True
    W = L("new_handle", T.rawget("w"), float(D), float(V))[0]
    scratch = device.Buffer((1 << 16,))
    from lanternl_amd._lib import call
    for rep in range(3):
        L.method(W, "upload", flat(w))
        L.method(P, "replay")
        got = {k: L.dl(T.rawget(k)) for k in ("loss", "dw", "l2", "w")}
        L.method(W, "upload", flat(w))
        P2 = L("program", 64.0)[0]
        L.method(L.vm.call(queue, P2)[0], "run")
        for k in got:
            assert np.array_equal(got[k], L.dl(T.rawget(k))), (rep, k)
        call("lhip_fill", scratch.ptr, scratch.size, float(rep))     # eager work between replays
    L.method(P, "free_graph")
    assert L.method(P, "is_captured")[0] is False
    L.method(P, "run")
    assert L.method(P, "size")[0] == 0.0
    small = L("program", 2.0)[0]
    L.method(L.method(small, "zero", T.rawget("l2"))[0], "zero", T.rawget("lsum"))
    with pytest.raises(LuaError, match=r"luaTL.Program full \(2\)"):
        L.method(small, "zero", T.rawget("am"))
    with pytest.raises(LuaError, match="the op list is empty"):
        L.method(L("program", 4.0)[0], "capture")


def test_hardware_stats_and_mem(L):
    hw = L("hardware")[0]
    for k in ("name", "sm", "multiprocessors", "warp_size", "total_vram", "free_vram", "l2_cache", "bandwidth_gbs",
              "gflops_fp32"):
        assert hw.rawget(k) is not None, k
    assert hw.rawget("warp_size") == 64.0 and hw.rawget("sm") == "gfx950" and hw.rawget("gflops_fp32") > 1e5
    st = L("stats")[0]
    for k in ("reserved", "in_use", "peak", "blocks", "allocs", "frees"):
        assert isinstance(st.rawget(k), float), k
    free, total = L("mem")
    assert 0 < free <= total
