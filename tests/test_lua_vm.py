"""CPU tests of the Lua side run in tests/lua_vm.py (no Lua runtime exists in
this image or on the GPU box):

* the interpreter itself, pinned on facts the Lua 5.1 manual fixes (operator
  precedence and arithmetic, multiple results, closures over loop variables,
  metatables, error positions, string library) and on LuaJIT FFI behaviour
  (arrays, structs, pointer arithmetic, finalisers, a call into libc);
* lanternl_amd/lua/luatl_adapter.lua, executed: its ffi.cdef declares each
  function and struct exactly as include/lanternl_hip.h does, every declared
  symbol resolves in liblanternl_hip.so, and without a GPU the module loads
  and reports itself unavailable with the library's reason;
* the matrix.lua patch (lanternl_amd/lua/matrix_patch.lua), executed in a harness that plays
  matrix.lua, with a pure-Lua backend: the dispatch rules (out/acc to
  matmul_into, threshold, force, failure counting) and the products' values.
"""
import ctypes
import ctypes.util
import gc
import os
import re

import numpy as np
import pytest

from tests import lua_registry as R
from tests.lua_vm import FFI, LuaError, LuaTable, LuaVM, run_module
from tests.lua_lint import LuaSyntaxError

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ADAPTER = os.path.join(ROOT, "lanternl_amd", "lua", "luatl_adapter.lua")
HEADER = os.path.join(ROOT, "include", "lanternl_hip.h")
LIB = os.path.join(ROOT, "lanternl_amd", "liblanternl_hip.so")


def run(src, *args):
    vm = LuaVM()
    return vm.call(vm.load(src, "t"), *args)


# ----------------------------------------------------------------- the language
@pytest.mark.parametrize("expr,want", [
    ("7 % -3", -2.0), ("-7 % 3", 2.0), ("5.5 % 2", 1.5),         # a % b == a - floor(a/b)*b
    ("2^3^2", 512.0), ("-2^2", -4.0), ("2^-1", 0.5),            # ^ is right-assoc, binds tighter than unary -
    ("1 + 2 * 3 - 4 / 8", 6.5), ("(1 + 2) * 3", 9.0),
    ('"10" + 1', 11.0), ('"0x10" * 1', 16.0),                   # string -> number coercion
    ("1 .. 2 .. 3", "123"), ('"a" .. 1.5', "a1.5"), ("10 / 4", 2.5),
    ("not 1 == 2", False), ("not nil", True), ("1 and 2", 2.0), ("nil or false", False),
    ("false and nil", False), ('"a" < "b"', True), ("#\"abc\" + #{1, 2, nil, 4}", None),
    ("tostring(1e100)", "1e+100"), ("tostring(0.1)", "0.1"), ("tostring(-0.5)", "-0.5"),
    ("tostring(2^53)", "9.007199254741e+15"), ("tostring(3)", "3"), ("math.floor(-0.5)", -1.0),
    ("select('#', nil, nil)", 2.0), ("select(2, 'a', 'b', 'c')", "b"), ("select(-1, 'a', 'b')", "b"),
    ("type(print)", "function"), ("type(nil)", "nil"), ("type({})", "table"),
    ("tonumber('  12  ')", 12.0), ("tonumber('z')", None), ("tonumber('ff', 16)", 255.0),
    ("1e300 * 1e10 == math.huge", True), ("0/0 ~= 0/0", True),
])
def test_expressions(expr, want):
    if want is None and "#" in expr:       # border of a table with a hole: only check it runs
        run("return " + expr)
        return
    got = run("return " + expr)[0]
    assert got == want and type(got) is type(want), (expr, got)


def test_multiple_results_and_varargs():
    src = r'''
    local function f() return 1, 2, 3 end
    local function g(...) return select("#", ...), ... end
    local a, b, c, d = f()
    local t1 = { f(), f() }           -- only the last call expands
    local t2 = { (f()) }              -- parentheses keep one value
    local n, x, y = g(nil, 5)
    local function tail(...) local t = {...} return #t end
    return a, b, c, d, #t1, #t2, n, x, y, tail(f())
    '''
    assert run(src) == [1.0, 2.0, 3.0, None, 4.0, 1.0, 2.0, None, 5.0, 3.0]


def test_closures_capture_per_iteration_and_shared_upvalues():
    src = r'''
    local fs = {}
    for i = 1, 3 do fs[i] = function() return i end end
    local function mk()
        local n = 0
        return function() n = n + 1 return n end, function() return n end
    end
    local inc, get = mk()
    inc() inc()
    local w = {}
    local j = 0
    while j < 3 do j = j + 1 local k = j * 10 w[j] = function() return k end end
    local function fact(n) if n <= 1 then return 1 end return n * fact(n - 1) end
    return fs[1]() + fs[3](), get(), w[1]() + w[3](), fact(10)
    '''
    assert run(src) == [4.0, 2.0, 40.0, 3628800.0]


def test_loops_and_scopes():
    src = r'''
    local c = 0
    for x = 1, 2, 0.5 do c = c + 1 end          -- 1, 1.5, 2
    for x = 3, 1 do c = c + 100 end             -- no iterations
    local r = 0
    repeat local z = r r = r + 1 until z >= 2  -- the condition sees the body's locals
    local keys = { a = 1, b = 2, c = 3, 4, 5 }
    local seen = 0
    for k, v in pairs(keys) do seen = seen + 1 keys[k] = nil end   -- clearing fields while traversing
    local s = 0
    for i, v in ipairs({ 1, 2, nil, 4 }) do s = s + v end           -- stops at the hole
    local x = 1
    do local x = 2 end
    local out = {}
    for i = 1, 10 do if i > 3 then break end out[#out + 1] = i end
    return c, r, seen, next(keys) == nil, s, x, #out
    '''
    assert run(src) == [3.0, 3.0, 5.0, True, 3.0, 1.0, 3.0]


def test_metatables():
    src = r'''
    local log = {}
    local base = { greet = function(self) return "hi " .. self.name end }
    local obj = setmetatable({ name = "x" }, { __index = base })
    local dyn = setmetatable({}, { __index = function(t, k) return k .. "?" end,
                                  __newindex = function(t, k, v) log[#log + 1] = k rawset(t, k, v) end })
    dyn.a = 1
    dyn.a = 2                      -- existing field: no __newindex
    local callable = setmetatable({}, { __call = function(self, a, b) return a + b end })
    return obj:greet(), dyn.zz, rawget(dyn, "zz"), dyn.a, #log, callable(2, 3), getmetatable(obj).__index == base
    '''
    assert run(src) == ["hi x", "zz?", None, 2.0, 1.0, 5.0, True]


def test_errors_and_positions():
    src = r'''
    local function inner() error("boom", 2) end
    local function outer()
        inner()
    end
    local ok1, e1 = pcall(outer)
    local ok2, e2 = pcall(function() local t = nil return t.x end)
    local ok3, e3 = pcall(error, { code = 7 })
    local ok4, e4 = pcall(error, "plain", 0)
    local ok5, e5 = pcall(function() return 1 + {} end)
    local ok6, e6 = pcall(function() return ("x"):bad() end)
    return ok1, e1, ok2, e2, ok3, e3.code, e4, e5, e6
    '''
    r = run(src)
    assert r[0] is False and r[1] == '[string "t"]:4: boom'          # level 2: the caller's line
    assert r[2] is False and r[3] == '[string "t"]:7: attempt to index a nil value'
    assert r[4] is False and r[5] == 7.0 and r[6] == "plain"
    assert "attempt to perform arithmetic on a table value" in r[7]
    assert "attempt to call a nil value" in r[8]
    with pytest.raises(LuaError, match="boom"):
        run("error('boom')")


def test_string_library():
    src = r'''
    local s = "/usr/lib/x/liblanternl_hip.so"
    return ("%5.2f|%-4d|%s|%x|%q"):format(3.14159, 7, "ok", 255, 'a"b'),
           s:match("^(.*)[/\\]"), s:sub(-3), s:sub(2, 4), s:find("lib", 1, true),
           ("a,b;c"):match("([^,]+),([^;]+)"), ("ab"):rep(3, "-"), ("x"):upper(), #s
    '''
    r = run(src)
    assert r[0] == ' 3.14|7   |ok|ff|"a\\"b"'
    assert r[1] == "/usr/lib/x" and r[2] == ".so" and r[3] == "usr"
    # calls inside an expression list give one value; only the last one expands
    assert r[4:] == [6.0, "a", "ab-ab-ab", "X", 29.0]
    assert run('return ("/usr/lib"):find("lib", 1, true)') == [6.0, 8.0]
    assert run('return ("a,b;c"):match("([^,]+),([^;]+)")') == ["a", "b"]
    assert run('return ("abc"):find("(b)(c)")') == [2.0, 3.0, "b", "c"]
    assert run('return ("abc"):match("x")') == [None]


def test_strings_long_brackets_and_escapes():
    r = run('return [[\nline1\nline2]], [==[a]]b]==], "t\\tq\\"\\65\\n", \'\\\\\'')
    assert r == ["line1\nline2", "a]]b", 't\tq"A\n', "\\"]


@pytest.mark.parametrize("src,msg", [
    ("goto done", "goto is not supported"),
    ("local function f() return ... end", "outside a vararg function"),
    ("x = = 1", "unexpected symbol"),
])
def test_unsupported_or_invalid_code_is_rejected(src, msg):
    with pytest.raises(LuaSyntaxError, match=msg):
        LuaVM().load(src)


def test_table_keys_normalise_integral_floats():
    assert run("local t = {} t[1] = 'a' t[1.0] = 'b' t[2] = 'c' return #t, t[1]") == [2.0, "b"]
    with pytest.raises(LuaError, match="table index is nil"):
        run("local t = {} t[nil] = 1")
    assert run("local t = {} return t[0/0]") == [None]
    with pytest.raises(LuaError, match="table index is NaN"):
        run("local t = {} t[0/0] = 1")


# ----------------------------------------------------------------- the FFI
def test_ffi_arrays_structs_pointers():
    src = r'''
    local ffi = require("ffi")
    ffi.cdef[[
    typedef struct { int a; double b; char name[8]; unsigned long long big; } rec_t;
    ]]
    local arr = ffi.new("double[?]", 4)
    for i = 0, 3 do arr[i] = i * 1.5 end
    local p = ffi.cast("double*", arr) + 2
    local r = ffi.new("rec_t")
    r.a = 7.0 r.b = 0.25 r.big = 2^40
    local pp = ffi.new("void*[1]")
    local f = ffi.new("float[3]", 1, 2, 3)
    local cp = ffi.cast("char*", arr) + 8
    local dp = ffi.cast("double*", cp)
    return p[0], p[1], r.a, r.b, tonumber(r.big), pp[0] == nil, f[2], dp[0], ffi.sizeof == nil
    '''
    with pytest.raises(LuaError, match="ffi.sizeof is not supported"):
        run(src)
    r = run(src.replace(", ffi.sizeof == nil", ""))
    assert r == [3.0, 4.5, 7.0, 0.25, 2.0 ** 40, True, 3.0, 1.5]


def test_ffi_64bit_integers_are_boxed_as_luajit_does():
    """A long long read from C is an int64 cdata: tonumber() converts it;
    arithmetic with numbers stays 64-bit; math, 'for' limits, concatenation and
    table keys need tonumber() first."""
    src = r'''
    local ffi = require("ffi")
    local a = ffi.new("long long[2]")
    local u = ffi.new("unsigned long long[1]")
    a[0] = 2^40 a[1] = -3
    u[0] = 5
    local x = a[0]
    return type(x), tonumber(x), x == 2^40, x + 1 == 2^40 + 1, tostring(a[1]), tostring(u[0] - 6),
           x > 1, tonumber(a[1] * 2), ("%d"):format(a[1])
    '''
    r = run(src)
    assert r[:4] == ["cdata", 2.0 ** 40, True, True]
    assert r[4] == "-3LL" and r[5] == "18446744073709551615ULL"
    assert r[6] is True and r[7] == -6.0 and r[8] == "-3"
    for bad, msg in [("math.max(a[0], 1)", "not supported between"), ("for i = 1, a[0] do end", "'for' initial value"),
                     ("local t = {} t[a[0]] = 1", "table key"), ("local s = 'n=' .. a[0]", "concatenate")]:
        with pytest.raises(Exception, match=msg):
            run('local ffi = require("ffi") local a = ffi.new("long long[1]") ' + bad)


def test_ffi_arrays_are_bounds_checked():
    with pytest.raises(IndexError):
        run('local a = require("ffi").new("float[?]", 4) a[4] = 1')


def test_ffi_call_into_libc_and_string():
    libc = ctypes.util.find_library("c")
    src = r'''
    local ffi = require("ffi")
    ffi.cdef[[
    size_t strlen(const char* s);
    void* memset(void* s, int c, size_t n);
    ]]
    local C = ffi.load(...)
    local buf = ffi.new("char[16]")
    C.memset(buf, 65, 5)
    return tonumber(C.strlen(buf)), type(C.strlen(buf)), ffi.string(buf), ffi.string(buf, 3)
    '''
    assert run(src, libc) == [5.0, "cdata", "AAAAA", "AAA"]     # size_t comes back boxed
    with pytest.raises(LuaError, match="missing declaration"):
        run('local ffi = require("ffi") local C = ffi.load(...) return C.strlen', libc)
    assert run('return pcall(require("ffi").load, "no_such_library_here")')[0] is False


def test_ffi_gc_finaliser_runs_once_and_can_be_cancelled():
    vm = LuaVM()
    f = vm.load(r'''
    local ffi = require("ffi")
    local log = ...
    local a = ffi.gc(ffi.new("int[1]"), function(p) log[#log + 1] = "a" end)
    local b = ffi.gc(ffi.new("int[1]"), function(p) log[#log + 1] = "b" end)
    ffi.gc(b, nil)
    return a, b
    ''', "gc")
    log = LuaTable()
    a, b = vm.call(f, log)
    assert log.length() == 0
    del a, b
    gc.collect()
    assert log.to_list() == ["a"]


# ----------------------------------------------------------------- the adapter module
def _header_ffi():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/|//[^\n]*", "", text, flags=re.S)
    text = "\n".join(ln for ln in text.splitlines() if not ln.lstrip().startswith("#"))
    text = text.replace('extern "C" {', "").replace("LHIP_API", "")
    hf = FFI()
    hf.cdef(text)
    return hf


def _sig(ct):
    return (ct.base.__name__ if ct.base is not None else "void", ct.ptr)


LUA_MODULES = [ADAPTER, os.path.join(ROOT, "lanternl_amd", "lua", "lanternl_lm.lua")]


@pytest.mark.parametrize("path", LUA_MODULES, ids=os.path.basename)
def test_module_cdef_matches_the_header_and_the_library(path):
    """Each module's ffi.cdef, declared as the module declares it, against the
    C header: every function's argument and return types, every struct's
    field names, types and offsets; and every symbol resolves in the library."""
    text = open(path).read()
    blocks = re.findall(r"ffi\.cdef\[\[(.*?)\]\]", text, re.S)
    assert len(blocks) == 1
    mf = FFI()
    mf.cdef(blocks[0])
    _compare_with_header(mf)


def _compare_with_header(mf):
    hf = _header_ffi()
    assert len(mf.funcs) >= 15
    for name, (ret, args) in mf.funcs.items():
        assert name in hf.funcs, f"{name} is declared in the adapter but not in lanternl_hip.h"
        hret, hargs = hf.funcs[name]
        assert _sig(ret) == _sig(hret), name
        assert [_sig(a) for a in args] == [_sig(a) for a in hargs], name
    def layout(cls):
        return [(f, t.__name__, getattr(cls, f).offset, getattr(cls, f).size) for f, t in cls._fields_]
    for tname, cls in mf.types.items():
        hcls = hf.types[tname]
        assert ctypes.sizeof(cls) == ctypes.sizeof(hcls), tname
        assert layout(cls) == layout(hcls), tname
    lib = ctypes.CDLL(LIB)
    for name in mf.funcs:
        assert hasattr(lib, name), name


def test_the_two_modules_declare_nothing_twice():
    """LuaJIT's C namespace is global: a second declaration of a name raises
    "attempt to redefine", so the modules loaded together must not overlap."""
    decls = []
    for path in LUA_MODULES:
        mf = FFI()
        mf.cdef(re.search(r"ffi\.cdef\[\[(.*?)\]\]", open(path).read(), re.S).group(1))
        decls.append(set(mf.funcs) | set(mf.types))
    assert not (decls[0] & decls[1])
    with pytest.raises(LuaError, match="attempt to redefine 'f'"):
        FFI().cdef("int f(int x);\nint f(int x);")


def test_lm_module_is_unavailable_with_the_adapter():
    vm = LuaVM()
    vm.search_dirs.append(os.path.dirname(ADAPTER))
    lm = vm.call(vm.G.rawget("require"), "lanternl_lm")[0]
    ad = vm.call(vm.G.rawget("require"), "luatl_adapter")[0]
    if ad.rawget("available"):
        pytest.skip("a GPU is visible: the GPU tests cover the available module")
    assert lm.rawget("available") is False and lm.rawget("reason") == ad.rawget("reason")
    assert lm.rawget("new") is None


def test_adapter_module_loads_and_reports_availability():
    vm, M = run_module(ADAPTER)
    assert M.rawget("name") == "luatl" and M.rawget("priority") == 100.0
    if M.rawget("available"):
        pytest.skip("a GPU is visible: the GPU tests cover the available module")
    reason = M.rawget("reason")
    assert "lanternl_hip[init]" in reason and "(DEVICE)" in reason and M.rawget("error") == reason
    # an unavailable module exposes no entry points (matrix.lua's probe skips it)
    assert M.rawget("matmul") is None and M.rawget("matmul_into") is None


def test_adapter_reports_a_missing_library(monkeypatch, tmp_path):
    """With the library nowhere on its search list the module returns
    available = false and the loader's message, as the registry expects."""
    lua_dir = tmp_path / "lua"
    lua_dir.mkdir()
    (lua_dir / "luatl_adapter.lua").write_text(open(ADAPTER).read())
    monkeypatch.setenv("LANTERNL_HIP_LIB", str(tmp_path / "nope.so"))
    vm, M = run_module(str(lua_dir / "luatl_adapter.lua"))
    assert M.rawget("available") is False
    assert M.rawget("reason").startswith("liblanternl_hip.so not found (cannot load library")


# ----------------------------------------------------------------- the matrix.lua patch, on the CPU
def _harness(*extra):
    vm = LuaVM()
    stub = R.stub_backend(vm)
    matrix, backends = R.build(vm, list(extra) + [("luatl_adapter", stub)])
    return vm, matrix, backends, stub


def _np(t, rows, cols):
    return np.array(t.to_list(), dtype=np.float64).reshape(rows, cols)


@pytest.mark.parametrize("acc", [False, True])
def test_patch_routes_out_and_acc_to_matmul_into(acc):
    vm, matrix, backends, stub = _harness()
    rng = np.random.default_rng(5)
    m, k, n = 12, 20, 18                              # 4320 multiply-adds: above the 4096 threshold
    a, b = rng.standard_normal((m, k)), rng.standard_normal((k, n))
    g = rng.standard_normal((m, n))
    cases = [
        ("multiply", a, b, rng.standard_normal((m, n)), lambda o: o * acc + a @ b),
        ("matmul_nt", a, rng.standard_normal((n, k)), rng.standard_normal((m, n)), None),
        ("matmul_tn", a, g, rng.standard_normal((k, n)), lambda o: o * acc + a.T @ g),
    ]
    for fname, x, y, out0, want in cases:
        if want is None:
            yy = y
            want = (lambda o, yy=yy: o * acc + a @ yy.T)
        out = R.lua_matrix(out0)
        res = vm.call(vm.index(matrix, fname), R.lua_matrix(x), R.lua_matrix(y), out, acc)[0]
        assert res is out and matrix.rawget("last_backend") == "luatl_adapter", fname
        got = _np(out.rawget("data"), *out0.shape)
        np.testing.assert_allclose(got, want(out0), rtol=1e-12, atol=1e-12)
    op = {"multiply": "nn", "matmul_nt": "nt", "matmul_tn": "tn"}
    assert stub.rawget("calls").to_list() == [f"matmul_into:{op[c[0]]}" + (":acc" if acc else "") for c in cases]


def test_patch_without_out_uses_the_plain_entries():
    vm, matrix, backends, stub = _harness()
    rng = np.random.default_rng(6)
    a, b, c = rng.standard_normal((16, 16)), rng.standard_normal((16, 16)), rng.standard_normal((16, 16))
    r1 = vm.call(vm.index(matrix, "multiply"), R.lua_matrix(a), R.lua_matrix(b))[0]
    r2 = vm.call(vm.index(matrix, "matmul_nt"), R.lua_matrix(a), R.lua_matrix(c))[0]
    r3 = vm.call(vm.index(matrix, "matmul_tn"), R.lua_matrix(a), R.lua_matrix(c))[0]
    np.testing.assert_allclose(_np(r1.rawget("data"), 16, 16), a @ b, rtol=1e-12)
    np.testing.assert_allclose(_np(r2.rawget("data"), 16, 16), a @ c.T, rtol=1e-12)
    np.testing.assert_allclose(_np(r3.rawget("data"), 16, 16), a.T @ c, rtol=1e-12)
    assert stub.rawget("calls").to_list() == ["matmul", "matmul_nt", "matmul_tn"]


def test_patch_threshold_and_force():
    vm, matrix, backends, stub = _harness()
    a, b = np.arange(6.0).reshape(2, 3), np.arange(12.0).reshape(3, 4)
    mul = vm.index(matrix, "multiply")
    r = vm.call(mul, R.lua_matrix(a), R.lua_matrix(b))[0]          # 24 multiply-adds: stays in Lua
    assert matrix.rawget("last_backend") == "lua" and stub.rawget("calls").length() == 0
    np.testing.assert_array_equal(_np(r.rawget("data"), 2, 4), a @ b)
    accel = matrix.rawget("accel")
    accel.rawset("force", "luatl_adapter")                           # forced: served below the threshold
    vm.call(mul, R.lua_matrix(a), R.lua_matrix(b))
    assert matrix.rawget("last_backend") == "luatl_adapter"
    accel.rawset("force", "blas")                                     # forced onto a backend not listed
    with pytest.raises(LuaError, match="backend 'blas' was forced via matrix.use\\(\\) but is unavailable"):
        vm.call(mul, R.lua_matrix(a), R.lua_matrix(b))
    accel.rawset("force", "lua")
    vm.call(mul, R.lua_matrix(a), R.lua_matrix(b))
    assert matrix.rawget("last_backend") == "lua"


def test_patch_counts_failures_and_falls_through():
    failing = r'''
    local M = { available = true }
    function M.matmul() error("device lost") end
    function M.matmul_into() return 42 end
    return M
    '''
    vm = LuaVM()
    bad = R.stub_backend(vm, failing)
    stub = R.stub_backend(vm)
    matrix, backends = R.build(vm, [("gpu", bad), ("luatl_adapter", stub)])
    rng = np.random.default_rng(7)
    a, b = rng.standard_normal((16, 16)), rng.standard_normal((16, 16))
    mul = vm.index(matrix, "multiply")
    vm.call(mul, R.lua_matrix(a), R.lua_matrix(b))
    e = backends.rawget(1)
    assert e.rawget("errors") == 1.0 and "device lost" in e.rawget("last_error")
    assert matrix.rawget("last_backend") == "luatl_adapter"
    out = R.lua_matrix(np.zeros((16, 16)))
    vm.call(mul, R.lua_matrix(a), R.lua_matrix(b), out, True)
    assert e.rawget("errors") == 2.0 and e.rawget("last_error") == "matmul_into returned number, expected flat table"
    np.testing.assert_allclose(_np(out.rawget("data"), 16, 16), a @ b, rtol=1e-12)
    vm.call(mul, R.lua_matrix(a), R.lua_matrix(b))
    assert e.rawget("errors") == 3.0 and e.rawget("available") is False
    assert e.rawget("reason").startswith("disabled after 3 failures")
    vm.call(mul, R.lua_matrix(a), R.lua_matrix(b))                   # a disabled backend is skipped
    assert e.rawget("errors") == 3.0 and matrix.rawget("last_backend") == "luatl_adapter"


def test_patch_skips_a_backend_without_the_entry():
    """A backend that has matmul but no matmul_into is skipped for calls with
    `out` (not counted as a failure); the next backend serves them."""
    old = r'''
    local M = { available = true }
    function M.matmul(a, m, k, b, n) error("must not be called for out calls") end
    return M
    '''
    vm = LuaVM()
    matrix, backends = R.build(vm, [("gpu", R.stub_backend(vm, old)), ("luatl_adapter", R.stub_backend(vm))])
    rng = np.random.default_rng(8)
    a, b = rng.standard_normal((16, 16)), rng.standard_normal((16, 16))
    out = R.lua_matrix(np.ones((16, 16)))
    vm.call(vm.index(matrix, "matmul_nt"), R.lua_matrix(a), R.lua_matrix(b), out, True)
    assert backends.rawget(1).rawget("errors") == 0.0 and matrix.rawget("last_backend") == "luatl_adapter"
    np.testing.assert_allclose(_np(out.rawget("data"), 16, 16), 1 + a @ b.T, rtol=1e-12)

