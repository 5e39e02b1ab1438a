"""CPU checks of lanternl_amd/lua/luatl_adapter.lua, which cannot run here (no
LuaJIT in this image or on the GPU box):
  * its ffi.cdef declares exactly the C ABI of include/lanternl_hip.h;
  * every function of the reference adapter (ai/gpu/luatl_adapter.lua), every
    Handle method and every luaTL.Program method (ai/gpu/luaTL_train.lua:
    332-632) exists with the reference's parameter list, name for name, and the
    module sets the reference's fields -- the reference's signatures come from
    tests/golden/adapter_signatures.json (tests/golden/make_adapter_signatures.py);
  * the Python mirror (lanternl_amd/backend.py), which the GPU tests drive,
    has the same functions with the same parameter counts."""
import inspect
import json
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ADAPTER = os.path.join(ROOT, "lanternl_amd", "lua", "luatl_adapter.lua")
HEADER = os.path.join(ROOT, "include", "lanternl_hip.h")
SIGS = json.load(open(os.path.join(ROOT, "tests", "golden", "adapter_signatures.json")))
# Prog:slot hands out the next slot of the reference's C op array; ops here are
# queued closures, so there is no slot to hand out (Prog:push plays that part)
PROGRAM_INTERNAL = {"slot"}


def _params(decl):
    inner = decl[decl.index("(") + 1: decl.rindex(")")].strip()
    return 0 if inner in ("", "void") else inner.count(",") + 1


def _decls(text, prefix=""):
    """name -> parameter count of every lhip_* function declared in text."""
    out = {}
    for m in re.finditer(prefix + r"[\w\s\*]+?\b(lhip_\w+)\s*\(([^;]*?)\)\s*;", text, re.S):
        out[m.group(1)] = _params("(" + m.group(2) + ")")
    return out


def _lua_sigs(text, owner):
    pat = re.compile(r"^function\s+" + re.escape(owner) + r"[.:](\w+)\s*\(([^)]*)\)", re.M)
    return {m.group(1): [p.strip() for p in m.group(2).split(",") if p.strip()] for m in pat.finditer(text)}


def test_cdef_functions_match_the_header():
    lua = open(ADAPTER).read()
    cdef = lua[lua.index("ffi.cdef[["): lua.index("]]", lua.index("ffi.cdef[["))]
    mine = _decls(cdef)
    header = _decls(open(HEADER).read(), prefix=r"LHIP_API\s+")
    assert len(mine) >= 45
    missing = sorted(set(mine) - set(header))
    assert not missing, f"cdef declares functions the header does not: {missing}"
    wrong = {f: (mine[f], header[f]) for f in mine if mine[f] != header[f]}
    assert not wrong, f"parameter counts differ (cdef, header): {wrong}"


def test_library_exports_every_cdef_function():
    import ctypes
    from lanternl_amd.build import LIB_PATH
    assert os.path.exists(LIB_PATH), "build the library first (__graft_entry__.build())"
    L = ctypes.CDLL(LIB_PATH)
    lua = open(ADAPTER).read()
    cdef = lua[lua.index("ffi.cdef[["): lua.index("]]", lua.index("ffi.cdef[["))]
    missing = [f for f in _decls(cdef) if not hasattr(L, f)]
    assert not missing, missing


def test_every_reference_adapter_function_has_its_parameter_list():
    mine = _lua_sigs(open(ADAPTER).read(), "M")
    ref = SIGS["module"]
    assert len(ref) >= 30
    missing = sorted(set(ref) - set(mine))
    assert not missing, f"reference adapter functions missing: {missing}"
    wrong = {f: (mine[f], ref[f]) for f in ref if mine[f] != ref[f]}
    assert not wrong, f"parameter lists differ (mine, reference): {wrong}"
    # the transposed products this backend adds, with matmul's convention
    assert mine["matmul_nt"] == mine["matmul_tn"] == ref["matmul"]


def test_handle_methods_and_program_methods_match():
    lua = open(ADAPTER).read()
    mine = _lua_sigs(lua, "Handle")
    wrong = {f: (mine.get(f), p) for f, p in SIGS["handle"].items() if mine.get(f) != p}
    assert not wrong, wrong
    prog = _lua_sigs(lua, "Prog")
    want = {k: v for k, v in SIGS["program"].items() if k not in PROGRAM_INTERNAL}
    assert len(want) >= 40
    wrong = {f: (prog.get(f), p) for f, p in want.items() if prog.get(f) != p}
    assert not wrong, f"Program methods differ (mine, reference): {wrong}"


# Reference module fields with no counterpart here.  `luaTL` is the reference's
# own low-level CUDA module (luatl_adapter.lua:17); callers that reach into it
# (gpu_transformer.lua:58-60, bench_gpu_transformer.lua:41) are not served.
ABSENT_FIELDS = {"luaTL"}


def test_module_sets_the_reference_fields():
    lua = open(ADAPTER).read()
    ctor = re.search(r"local M\s*=\s*\{([^}]*)\}", lua).group(1)
    # only assignments of a value count: `M.x = nil` does not set the field
    fields = set(re.findall(r"\bM\.(\w+)\s*=(?!=)[ \t]*(?![ \t]|nil\b)", lua)) | set(re.findall(r"(\w+)\s*=", ctor))
    missing = sorted(set(SIGS["fields"]) - ABSENT_FIELDS - fields)
    assert not missing, missing
    assert ABSENT_FIELDS <= set(SIGS["fields"])
    header = lua[:lua.index("local M =")]
    for f in ABSENT_FIELDS:
        assert f not in fields
        assert f"M.{f}" in header and "no counterpart" in header, f"absent field {f} is not documented"
    assert "reason" in fields      # matrix.lua:39-40 reads mod.reason
    assert re.search(r'name\s*=\s*"luatl"', ctor) and re.search(r"priority\s*=\s*100", ctor)


def test_matmul_into_entry_declared_in_both_modules():
    """The entry the registry's out=/acc dispatch calls (lanternl_amd/lua/matrix_patch.lua)."""
    mine = _lua_sigs(open(ADAPTER).read(), "M")
    assert mine["matmul_into"] == ["op", "a", "m", "k", "b", "n", "rd", "acc"]
    from lanternl_amd import backend as B
    assert list(inspect.signature(B.matmul_into).parameters) == mine["matmul_into"]


def test_python_mirror_has_the_same_calls():
    """lanternl_amd/backend.py is what the GPU tests drive: same functions, same arity."""
    from lanternl_amd import backend as B
    for f, params in SIGS["module"].items():
        fn = getattr(B, f, None)
        assert callable(fn), f
        sig = inspect.signature(fn)
        assert len(sig.parameters) == len(params), (f, list(sig.parameters), params)
    for f, params in SIGS["handle"].items():
        assert len(inspect.signature(getattr(B.Handle, f)).parameters) == len(params) + 1, f
    for f, params in SIGS["program"].items():
        if f in PROGRAM_INTERNAL:
            continue
        meth = getattr(B.Program, "async_" if f == "async" else f)
        assert len(inspect.signature(meth).parameters) == len(params) + 1, (f, params)
    for field in ("name", "priority", "available", "reason", "error", "C", "luaTL", "HandleClass",
                  "is_handle", "new_handle"):
        assert hasattr(B, field), field
    assert B.name == "luatl" and B.priority == 100
