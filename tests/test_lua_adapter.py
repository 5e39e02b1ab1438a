"""CPU checks of lanternl_amd/lua/luatl_adapter.lua, which cannot run here (no
LuaJIT in this image): its ffi.cdef must declare exactly the C ABI of
include/lanternl_hip.h, and it must define the module surface of the
reference adapter (ai/gpu/luatl_adapter.lua:63-246) that this backend serves."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ADAPTER = os.path.join(ROOT, "lanternl_amd", "lua", "luatl_adapter.lua")
HEADER = os.path.join(ROOT, "include", "lanternl_hip.h")


def _params(decl):
    inner = decl[decl.index("(") + 1: decl.rindex(")")].strip()
    return 0 if inner in ("", "void") else inner.count(",") + 1


def _decls(text, prefix=""):
    """name -> parameter count of every lhip_* function declared in text."""
    out = {}
    for m in re.finditer(prefix + r"[\w\s\*]+?\b(lhip_\w+)\s*\(([^;]*?)\)\s*;", text, re.S):
        out[m.group(1)] = _params("(" + m.group(2) + ")")
    return out


def test_cdef_functions_match_the_header():
    lua = open(ADAPTER).read()
    cdef = lua[lua.index("ffi.cdef[["): lua.index("]]", lua.index("ffi.cdef[["))]
    mine = _decls(cdef)
    header = _decls(open(HEADER).read(), prefix=r"LHIP_API\s+")
    assert len(mine) >= 30
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


# module contract (matrix.lua:28-48,178-202) and the resident-mode surface of
# ai/gpu/luatl_adapter.lua:63-246 (gelu_inplace and scale_inplace are not on
# the hot path: neither the CPU LMTrain step nor this backend uses them)
SURFACE = ["matmul", "matmul_nt", "matmul_tn", "pin", "alloc", "gemm", "gemm_dx", "gemm_dw", "rmsnorm",
           "rmsnorm_bwd", "softmax", "softmax_causal", "softmax_bwd", "swiglu", "rope", "add_inplace",
           "silu_inplace", "program", "sync", "stats", "hardware", "shutdown", "offset", "view", "cols", "wrap",
           "ids", "upload_i32", "download_i32", "download_f32", "scalar", "mem"]
HANDLE = ["toflat", "upload", "zero", "free", "shape"]


def test_adapter_defines_the_reference_surface():
    lua = open(ADAPTER).read()
    have = set(re.findall(r"^function M\.(\w+)\s*\(", lua, re.M))
    assert not [f for f in SURFACE if f not in have], [f for f in SURFACE if f not in have]
    hmeth = set(re.findall(r"^function Handle:(\w+)\s*\(", lua, re.M))
    assert not [f for f in HANDLE if f not in hmeth]
    assert re.search(r"available\s*=", lua) and re.search(r"reason\s*=", lua)
