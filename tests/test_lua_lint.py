"""The Lua side, checked without a Lua runtime (none exists in this image or on
the GPU box): lanternl_amd/lua/luatl_adapter.lua, lanternl_amd/lua/lanternl_lm.lua
and the matrix.lua patch (lanternl_amd/lua/matrix_patch.lua) must parse as Lua 5.1 / LuaJIT, and every
name they use must be a local in scope or a Lua builtin (a misspelt local, or
a local function used above its declaration, would otherwise only fail when
LuaJIT runs it).  The parser itself (tests/lua_lint.py) is checked on
constructs it must accept and mistakes it must reject."""
import os
import re

import pytest

from tests import lua_lint as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ADAPTER = os.path.join(ROOT, "lanternl_amd", "lua", "luatl_adapter.lua")

LUA_BUILTINS = {"assert", "collectgarbage", "debug", "error", "getmetatable", "io", "ipairs", "math", "next", "os",
                "pairs", "pcall", "print", "rawequal", "rawget", "rawset", "require", "select", "setmetatable",
                "string", "table", "tonumber", "tostring", "type", "unpack", "xpcall", "jit", "bit"}

GRAMMAR_OK = r'''
local a, b = 1, 0x1F
local s = "x\"y" .. 'z' .. [[long
string]] .. [==[ ]] ]==]
--[[ block
comment ]] -- line comment
local t = { 1, 2; x = 3, ["k"] = 4, [a + 1] = -b, f = function(...) return select("#", ...) end, }
local function fact(n) if n <= 1 then return 1 else return n * fact(n - 1) end end
local M = {}
function M.f(x, y) return x ^ 2 ^ y, not x == y, #t, -x % 3 end
function M:g(v) self.v = v; return self end
for i = 10, 1, -1 do a = a + i end
for k, v in pairs(t) do b = b + (tonumber(v) or 0) end
while a > 0 do a = a - 1 if a == 3 then break end end
repeat local z = a; a = a + 1 until z >= 5
do local u = M:g(1).v; t[#t + 1] = u end
local c = M.f(1, 2); print(("%d"):format(c), type{}, tostring"x")
goto done
::done::
return M
'''


def test_parser_accepts_the_grammar_and_resolves_scopes():
    free = L.free_names(GRAMMAR_OK)
    assert set(free) == {"select", "pairs", "tonumber", "print", "type", "tostring"}


@pytest.mark.parametrize("src,where", [
    ("if x then y = 1", "expected end"),
    ("local function f() return 1", "expected end"),
    ("x + 1 = 2", "syntax error|cannot assign"),
    ("f() = 1", "cannot assign"),
    ('local s = "abc', "unfinished string"),
    ("local t = {1, 2", "expected }"),
    ("for i = 1 do end", "expected ,"),
    ("return 1 end", "expected eof"),
])
def test_parser_rejects_mistakes(src, where):
    with pytest.raises(L.LuaSyntaxError, match=where):
        L.parse(src)


def test_resolver_finds_use_before_local_and_misspelt_locals():
    src = "local function a() return helper() end\nlocal function helper() return 1 end\nlocal v = 1\nreturn vv"
    free = L.free_names(src)
    assert free == {"helper": 1, "vv": 4}
    # a local's own initialiser does not see it; a local function sees itself
    assert L.free_names("local x = x") == {"x": 1}
    assert L.free_names("local function r(n) return r(n) end") == {}
    # loop variables and parameters are scoped to their bodies
    assert L.free_names("for i = 1, 2 do end return i") == {"i": 1}
    assert L.free_names("local function f(p) end return p") == {"p": 1}


@pytest.mark.parametrize("name", ["luatl_adapter.lua", "lanternl_lm.lua"])
def test_module_parses_and_uses_only_locals_and_builtins(name):
    text = open(os.path.join(os.path.dirname(ADAPTER), name)).read()
    free = L.free_names(text)
    unknown = {k: v for k, v in free.items() if k not in LUA_BUILTINS}
    assert not unknown, f"names used as globals in {name} (first line): {unknown}"


def test_matrix_lua_patch_parses():
    """The helper and the three call sites the patch adds to matrix.lua."""
    from tests.lua_registry import PATCH, patch_parts
    text = open(PATCH).read()
    L.parse(text)                                    # the file as a whole is valid Lua
    helper, sites = patch_parts(text)
    # matrix.lua's own locals the helper relies on (ai/core/matrix.lua:1-25,169-176)
    matrix_locals = {"matrix", "backends", "backend_failed", "sformat"}
    free = L.free_names(helper)
    assert set(free) <= LUA_BUILTINS | matrix_locals, free
    # the call sites are statements inside the three functions: wrap them in one
    wrapped = ("local function try_offload(...) end\nlocal function body(a, b, ad, bd, m, k, n, result, out, acc)\n"
               + "\n".join(sites.values()) + "\nend")
    free = L.free_names(wrapped)
    assert not free, free


def test_integration_notes_show_the_patch_file_verbatim():
    """The ```lua blocks the integration notes give maintainers are the patch
    file's two parts, character for character."""
    from tests.lua_registry import PATCH
    text = open(PATCH).read()
    helper = text.split("-- [helper]\n", 1)[1].split("-- [call sites]\n", 1)[0]
    sites = text.split("-- [call sites]\n", 1)[1]
    notes = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    blocks = re.findall(r"```lua\n(.*?)```", notes, re.S)
    assert helper.rstrip("\n") + "\n" in [b for b in blocks]
    assert sites in blocks
