"""Runs lanternl_amd/lua/matrix_patch.lua, the change ai/core/matrix.lua takes
(the `try_offload` helper and its three call sites), as Lua, in
tests/lua_vm.py.

The patch file has two parts, marked `-- [helper]` and `-- [call sites]`: the
helper, a local function inside matrix.lua, and the lines that go into
matrix.multiply / matmul_nt / matmul_tn.  ``build(vm, backends)`` wraps both in
a harness that stands in for the parts of matrix.lua they rely on: the
`matrix` table with `accel` and `strict` (matrix.lua:19-20), the `backends`
list of probe entries (:25-52), `backend_failed` (:169-176) and `sformat`; and
the three products with their `out`/`acc` handling and plain Lua loops for the
calls no backend serves (:540-590, :597-660).  It returns ``(matrix,
backends)`` as Lua tables; the caller chooses the backends.

Test infrastructure only.
"""
import os
import re

from tests.lua_vm import LuaTable, LuaVM

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PATCH = os.path.join(ROOT, "lanternl_amd", "lua", "matrix_patch.lua")

HEAD = r'''
local backend_list = ...
local sformat = string.format
local matrix = { strict = false, last_backend = "lua",
                 accel = { enabled = true, threshold = 4096, max_errors = 3, force = nil } }
-- probe entries as matrix.lua builds them: name, module, available, errors
local backends = {}
for i = 1, #backend_list do
    local b = backend_list[i]
    backends[i] = { name = b.name, module = b.module, available = b.module.available == true, errors = 0,
                    reason = b.module.available == true and "ready" or tostring(b.module.reason) }
end
-- a failure is counted; max_errors of them disable the backend
local function backend_failed(entry, msg)
    entry.errors = entry.errors + 1
    entry.last_error = msg
    if entry.errors >= (matrix.accel.max_errors or 3) then
        entry.available = false
        entry.reason = "disabled after " .. entry.errors .. " failures: " .. msg
    end
end
'''

PRODUCTS = r'''
local function target(out, rows, cols)
    if out ~= nil then return out end
    local d = {}
    for i = 1, rows * cols do d[i] = 0 end
    return { rows = rows, cols = cols, data = d }
end

function matrix.multiply(a, b, out, acc)
    local m, k, n = a.rows, a.cols, b.cols
    local result = target(out, m, n)
    local ad, bd = a.data, b.data
@@NN@@
    matrix.last_backend = "lua"
    local rd = result.data
    for i = 1, m do
        for j = 1, n do
            local s = 0
            for p = 1, k do s = s + ad[(i - 1) * k + p] * bd[(p - 1) * n + j] end
            local idx = (i - 1) * n + j
            if acc then rd[idx] = rd[idx] + s else rd[idx] = s end
        end
    end
    return result
end

function matrix.matmul_nt(a, b, out, acc)
    local m, k, n = a.rows, a.cols, b.rows
    local result = target(out, m, n)
    if m == 0 or n == 0 then return result end
@@NT@@
    matrix.last_backend = "lua"
    local ad, bd, rd = a.data, b.data, result.data
    for i = 1, m do
        for j = 1, n do
            local s = 0
            for p = 1, k do s = s + ad[(i - 1) * k + p] * bd[(j - 1) * k + p] end
            local idx = (i - 1) * n + j
            if acc then rd[idx] = rd[idx] + s else rd[idx] = s end
        end
    end
    return result
end

function matrix.matmul_tn(a, b, out, acc)
    local m, k, n = a.rows, a.cols, b.cols
    local result = target(out, k, n)
    local rd = result.data
    if not acc then
        for i = 1, k * n do rd[i] = 0 end
    end
    if m == 0 or k == 0 or n == 0 then return result end
@@TN@@
    matrix.last_backend = "lua"
    local ad, bd = a.data, b.data
    for i = 1, m do
        for p = 1, k do
            local av = ad[(i - 1) * k + p]
            for j = 1, n do
                local idx = (p - 1) * n + j
                rd[idx] = rd[idx] + av * bd[(i - 1) * n + j]
            end
        end
    end
    return result
end

return matrix, backends
'''


def patch_parts(text=None):
    """(helper, {"nn": site, "nt": site, "tn": site}) from the patch file."""
    text = text if text is not None else open(PATCH).read()
    _, rest = text.split("-- [helper]\n", 1)
    helper, sites_block = rest.split("-- [call sites]\n", 1)
    sites = {}
    for sec in re.split(r"^-- (?=matrix\.)", sites_block, flags=re.M)[1:]:
        head, _, body = sec.partition("\n")
        code = "\n".join(ln for ln in body.splitlines() if not ln.lstrip().startswith("--"))
        key = {"matrix.multiply": "nn", "matrix.matmul_nt": "nt", "matrix.matmul_tn": "tn"}[head.split(":")[0]]
        sites[key] = code
    assert set(sites) == {"nn", "nt", "tn"}, sites.keys()
    return helper, sites


def source():
    helper, sites = patch_parts()
    body = PRODUCTS.replace("@@NN@@", sites["nn"]).replace("@@NT@@", sites["nt"]).replace("@@TN@@", sites["tn"])
    return HEAD + helper + body


def build(vm, backend_list):
    """Run the harness with [(name, module table)] as the backends, in order."""
    lst = LuaTable.from_list([LuaTable({"name": n, "module": m}) for n, m in backend_list])
    fn = vm.load(source(), "matrix.lua (patched, harness)")
    matrix, backends = vm.call(fn, lst)
    return matrix, backends


def lua_matrix(a):
    """A matrix.lua matrix {rows, cols, data} from a 2-D array."""
    rows, cols = a.shape
    return LuaTable({"rows": float(rows), "cols": float(cols),
                     "data": LuaTable.from_list([float(v) for v in a.ravel()])})


# a pure-Lua backend with the adapter's product entries (for CPU runs of the patch)
LUA_STUB_BACKEND = r'''
local M = { available = true, reason = "ready", calls = {} }
local function extents(op, m, k, n)
    if op == "nn" then return m * k, k * n, m * n end
    if op == "nt" then return m * k, n * k, m * n end
    return m * k, m * n, k * n
end
local function product(op, a, m, k, b, n)
    local r = {}
    if op == "tn" then
        for i = 1, k * n do r[i] = 0 end
        for i = 1, m do for p = 1, k do for j = 1, n do
            r[(p - 1) * n + j] = r[(p - 1) * n + j] + a[(i - 1) * k + p] * b[(i - 1) * n + j]
        end end end
        return r
    end
    for i = 1, m do for j = 1, n do
        local s = 0
        for p = 1, k do
            local bv = op == "nn" and b[(p - 1) * n + j] or b[(j - 1) * k + p]
            s = s + a[(i - 1) * k + p] * bv
        end
        r[(i - 1) * n + j] = s
    end end
    return r
end
function M.matmul(a, m, k, b, n) M.calls[#M.calls + 1] = "matmul" return product("nn", a, m, k, b, n) end
function M.matmul_nt(a, m, k, b, n) M.calls[#M.calls + 1] = "matmul_nt" return product("nt", a, m, k, b, n) end
function M.matmul_tn(a, m, k, b, n) M.calls[#M.calls + 1] = "matmul_tn" return product("tn", a, m, k, b, n) end
function M.matmul_into(op, a, m, k, b, n, rd, acc)
    M.calls[#M.calls + 1] = "matmul_into:" .. op .. (acc and ":acc" or "")
    local r = product(op, a, m, k, b, n)
    local _, _, nc = extents(op, m, k, n)
    for i = 1, nc do rd[i] = acc and rd[i] + r[i] or r[i] end
    return rd
end
return M
'''


def stub_backend(vm, code=LUA_STUB_BACKEND):
    return vm.call(vm.load(code, "stub backend"))[0]


__all__ = ["LuaVM", "PATCH", "build", "lua_matrix", "patch_parts", "source", "stub_backend"]
