"""GPU tests of lanternl_amd/lua/lanternl_lm.lua, executed (tests/lua_vm.py)
against liblanternl_hip.so: the LMTrain step driven from Lua, with the
reference's data structures (a Transformer's parameters() as Tensors over
{rows, cols, data} matrices; build_windows' {inp, tgt, n} windows with 1-based
ids), against the Python mirror (lanternl_amd.lmtrain.GpuLMStep) on the same
library with the same inputs.

Both drive the same device step, which is deterministic, so the bar is
bit-for-bit equality of parameters, statistics, argmax, AdamW state and
checkpoints.  The step itself is checked against the oracle in
tests/test_lm_gpu.py.
"""
import os

import numpy as np
import pytest

from lanternl_amd import device, lmtrain
from tests.gpu_util import announce
from tests.lua_vm import LuaError, LuaTable, LuaVM

pytestmark = pytest.mark.gpu
LUA_DIR = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "lanternl_amd", "lua")
TINY = dict(vocab=32, dim=16, layers=1, heads=2, ffn=32, batch=2, seq=8)


class LuaLM:
    def __init__(self):
        self.vm = LuaVM()
        self.vm.search_dirs.append(LUA_DIR)
        self.lm = self.vm.call(self.vm.G.rawget("require"), "lanternl_lm")[0]

    def new(self, cfg):
        return self.vm.call(self.lm.rawget("new"), opts(cfg))[0]

    def m(self, obj, name, *args):
        return self.vm.call(self.vm.index(obj, name), obj, *args)

    def run(self, src, *args):
        return self.vm.call(self.vm.load(src, "test chunk"), *args)


def opts(d):
    return LuaTable({k: (float(v) if isinstance(v, (int, float)) and not isinstance(v, bool) else v)
                     for k, v in d.items()})


def flat(a):
    return LuaTable.from_list([float(v) for v in np.asarray(a, np.float64).ravel()])


def arr32(t):
    return np.array(t.to_list(), np.float32)


# a Transformer stand-in: parameters() returns Tensors whose .data is a matrix
MODEL = r'''
local layout, flat = ...
local params = {}
for i, L in ipairs(layout) do
    local d = {}
    for j = 1, L.rows * L.cols do d[j] = flat[L.offset + j] end
    params[i] = { data = { rows = L.rows, cols = L.cols, data = d } }
end
local model = {}
function model:parameters() return params end
return model
'''


def windows_lua(ids, tgt, lens):
    """build_windows' {inp, tgt, n} with 1-based ids, one per row of (ids, tgt)."""
    out = []
    for b, n in enumerate(lens):
        out.append(LuaTable.from_list([LuaTable.from_list([float(v + 1) for v in ids[b, :n]]),
                                       LuaTable.from_list([float(v + 1) for v in tgt[b, :n]]), float(n)]))
    return LuaTable.from_list(out)


@pytest.fixture(scope="module")
def L():
    device.init(0)
    lua = LuaLM()
    assert lua.lm.rawget("available") is True, lua.lm.rawget("reason")
    return lua


def _pair(L, cfg, seed):
    rng = np.random.default_rng(seed)
    py = lmtrain.GpuLMStep(**cfg)
    p0 = lmtrain.init_params(py.cfg, rng, 0.02)
    py.set_params(p0)
    step = L.new(cfg)
    layout = L.vm.call(L.lm.rawget("layout"), opts(cfg))[0]
    model = L.run(MODEL, layout, flat(p0))[0]
    L.m(step, "load_model", model)
    return py, step, model, p0, rng


def _stats_equal(st_lua, st_py):
    assert np.float32(st_lua.rawget("loss")) == np.float32(st_py["loss"])
    assert np.float32(st_lua.rawget("grad_norm")) == np.float32(st_py["grad_norm"])
    assert st_lua.rawget("applied") is st_py["applied"] and st_lua.rawget("correct") == st_py["correct"]
    assert arr32(st_lua.rawget("window_losses")).tolist() == st_py["window_losses"].astype(np.float32).tolist()


def test_layout_is_transformer_parameters_order(L):
    layout = L.vm.call(L.lm.rawget("layout"), opts(TINY))[0].to_list()
    names = [e.rawget("name") for e in layout]
    assert names == ["emb", "ln1.1", "wq.1", "wk.1", "wv.1", "wo.1", "ln2.1", "w1.1", "w3.1", "w2.1", "lnf"]
    table = lmtrain.param_table(lmtrain.config(**TINY))
    for e, (name, off, rows, cols) in zip(layout, table):
        assert (e.rawget("offset"), e.rawget("rows"), e.rawget("cols")) == (off, rows, cols)


def test_sgd_steps_match_the_python_mirror(L):
    announce("lua lm", "sgd x3, full and ragged batches")
    py, step, model, p0, rng = _pair(L, TINY, 5)
    B, T, V = TINY["batch"], TINY["seq"], TINY["vocab"]
    for it, (lens, nw) in enumerate([([T, T], 2), ([T, 5], 2), ([6, 0], 1)]):
        ids = rng.integers(0, V, (B, T)); tgt = rng.integers(0, V, (B, T))
        for bb in range(B):       # the slots past a window's tokens hold 0 on both sides
            n_b = lens[bb] if bb < nw else 0
            ids[bb, n_b:] = 0
            tgt[bb, n_b:] = 0
        L.m(step, "set_windows", windows_lua(ids, tgt, lens[:nw]))
        if lens == [T, T]:
            py.set_batch(ids, tgt)
        else:
            py.set_batch(ids, tgt, lengths=lens, n_windows=nw)
        L.m(step, "sgd", opts(dict(lr=0.1, momentum=0.9, weight_decay=0.01, clip=1.0)))
        py.step(0.1, 0.9, 0.01, 1.0)
        _stats_equal(L.m(step, "stats")[0], py.stats())
        np.testing.assert_array_equal(arr32(L.m(step, "params")[0]), py.params(), err_msg=f"step {it}")
        np.testing.assert_array_equal(arr32(L.m(step, "velocity")[0]), py.velocity())
        np.testing.assert_array_equal(arr32(L.m(step, "grads")[0]), py.grads())
        am = np.array(L.m(step, "argmax")[0].to_list(), np.int64)
        np.testing.assert_array_equal(am - 1, py.argmax())
    # the device weights back into the Transformer's tensors
    L.m(step, "store_model", model)
    params = L.m(model, "parameters")[0].to_list()
    got = np.concatenate([arr32(p.rawget("data").rawget("data")) for p in params])
    np.testing.assert_array_equal(got, py.params())
    py.close()
    L.m(step, "free")


def test_adamw_steps_state_and_graph_replay(L):
    announce("lua lm", "adamw x2 and graph replay")
    py, step, model, p0, rng = _pair(L, TINY, 6)
    B, T, V = TINY["batch"], TINY["seq"], TINY["vocab"]
    ids = rng.integers(0, V, (B, T)); tgt = rng.integers(0, V, (B, T))
    L.m(step, "set_windows", windows_lua(ids, tgt, [T, T]))
    py.set_batch(ids, tgt)
    L.m(step, "use_graph", True)
    py.use_graph(False)                      # the graph replay must equal the eager step
    for _ in range(3):
        L.m(step, "adamw", opts(dict(lr=1e-2)))
        py.step_adamw(lr=1e-2)
        _stats_equal(L.m(step, "stats")[0], py.stats())
    np.testing.assert_array_equal(arr32(L.m(step, "params")[0]), py.params())
    m_l, v_l, t_l = L.m(step, "adam_state")
    m_p, v_p, t_p = py.adam_state()
    np.testing.assert_array_equal(arr32(m_l), m_p)
    np.testing.assert_array_equal(arr32(v_l), v_p)
    assert t_l == t_p == 3
    # resume: moments and step count set from Lua, one more step on each side
    L.m(step, "set_adam_state", flat(m_p), flat(v_p), float(t_p))
    L.m(step, "adamw", opts(dict(lr=1e-2)))
    py.step_adamw(lr=1e-2)
    np.testing.assert_array_equal(arr32(L.m(step, "params")[0]), py.params())
    py.close()
    L.m(step, "free")


def test_checkpoints_cross_between_lua_and_python(L, tmp_path):
    announce("lua lm", "checkpoints")
    cfg_np = lmtrain.config(**TINY)
    py, step, model, p0, rng = _pair(L, TINY, 7)
    for fmt in ("bin", "text"):
        path = str(tmp_path / f"lua_{fmt}.ckpt")
        L.m(step, "save", path, opts(dict(format=fmt, epoch=3, loss=1.25, backend="luatl_adapter")))
        params, header = lmtrain.load_checkpoint(path, cfg_np)
        np.testing.assert_array_equal(params, p0.astype(np.float32))
        assert header["epoch"] == 3 and header["loss"] == 1.25 and header["version"] == 3
    # a Python-written checkpoint into the Lua step
    p1 = lmtrain.init_params(cfg_np, rng, 0.02)
    path = str(tmp_path / "py.ckpt")
    lmtrain.save_checkpoint(path, cfg_np, p1, epoch=9)
    h = L.m(step, "load", path)[0]
    assert h.rawget("version") == 3.0 and h.rawget("epoch") == 9.0 and h.rawget("format") == "bin"
    np.testing.assert_array_equal(arr32(L.m(step, "params")[0]), p1.astype(np.float32))
    py.close()
    L.m(step, "free")


def test_errors(L):
    step = L.new(TINY)
    layout = L.vm.call(L.lm.rawget("layout"), opts(TINY))[0]
    n = int(step.rawget("n"))
    model = L.run(MODEL, layout, flat(np.zeros(n)))[0]
    params = L.m(model, "parameters")[0]
    params.rawget(3.0).rawget("data").rawset("cols", 17.0)      # wq.1 is 16x16
    with pytest.raises(LuaError, match=r"tensor 3 \(wq.1\) is 16x17, the configuration needs 16x16"):
        L.m(step, "load_model", model)
    params.rawset(12.0, params.rawget(11.0))                     # an extra tensor (e.g. an untied head)
    with pytest.raises(LuaError, match="the model has 12 parameter tensors, this configuration 11"):
        L.m(step, "load_model", model)
    bad = windows_lua(np.full((1, 8), 40), np.zeros((1, 8), np.int64), [8])
    with pytest.raises(LuaError, match="id 41 / target 1 outside 1..32"):
        L.m(step, "set_windows", bad)
    three = windows_lua(np.zeros((3, 8), np.int64), np.zeros((3, 8), np.int64), [8, 8, 8])
    with pytest.raises(LuaError, match="3 windows for a batch of 2"):
        L.m(step, "set_windows", three)
    one = windows_lua(np.zeros((1, 8), np.int64), np.zeros((1, 8), np.int64), [8])
    with pytest.raises(LuaError, match=r"window 2 is not an \{ inp, tgt, n \} table"):
        L.m(step, "set_windows", one, 1.0, 2.0)          # hi past the list's end
    half = windows_lua(np.zeros((1, 8), np.int64), np.zeros((1, 8), np.int64), [8])
    half.rawget(1.0).rawset(3.0, 2.5)                               # n = 2.5 tokens
    with pytest.raises(LuaError, match=r"window 1 holds 2.5 tokens"):
        L.m(step, "set_windows", half)
    params.rawset(12.0, None)
    params.rawget(3.0).rawget("data").rawset("cols", 16.0)
    params.rawget(5.0).rawget("data").rawget("data").rawset(256.0, None)   # wv.1 short by one value
    with pytest.raises(LuaError, match=r"tensor 5 \(wv.1\) holds 255 values, its 16x16 shape needs 256"):
        L.m(step, "load_model", model)
    with pytest.raises(LuaError, match="option layers must be a positive integer, got 1.5"):
        L.new(dict(TINY, layers=1.5))
    with pytest.raises(LuaError, match="o.lr is required"):
        L.m(step, "sgd", opts({}))
    with pytest.raises(LuaError, match=r"lanternl_lm\[load\]: .*\((ARG|SHAPE|UNSUPPORTED|NULL|DEVICE)\)"):
        L.m(step, "load", "/nonexistent/dir/x.ckpt")
    L.m(step, "free")
    with pytest.raises(LuaError, match="the step has been freed"):
        L.m(step, "params")
