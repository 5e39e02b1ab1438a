"""CPU tests of the ai.Matrix registry restatement (lanternl_amd/matrix.py):
probe reasons, threshold gate, fault counting and disablement, forced
backends, strict validation, and that the CPU loops agree with the oracle
(ai/core/matrix.lua:19-202, 514-660).  Backends are stubs, as a Lua test would
pre-load them: the registry's own degradation path is the hook for a fake backend."""
import types

import numpy as np
import pytest

import oracle as O
from lanternl_amd import matrix as MX


def stub(matmul=None, available=True, reason=None, **extra):
    m = types.SimpleNamespace(available=available, reason=reason, matmul=matmul, calls=0)
    for k, v in extra.items():
        setattr(m, k, v)
    return m


@pytest.fixture(autouse=True)
def _reset():
    saved = dict(MX.accel), MX.strict
    yield
    MX.accel.clear(); MX.accel.update(saved[0]); MX.strict = saved[1]
    MX.reset_backends({"luatl_adapter": stub(available=False, reason="reset")})


def M(a):
    return MX.Matrix.from_numpy(np.asarray(a, dtype=np.float64))


def test_probe_reasons():
    lst = MX.reset_backends({"luatl_adapter": stub(available=False, reason="no device")})
    by = {e["name"]: e for e in lst}
    assert [e["name"] for e in lst] == ["luatl_adapter", "gpu", "blas"]
    assert by["luatl_adapter"]["reason"] == "no device" and not by["luatl_adapter"]["available"]
    assert by["gpu"]["reason"].startswith("not installed")
    lst = MX.reset_backends({"luatl_adapter": stub(matmul=None)})
    assert lst[0]["reason"] == "module is available but exposes no matmul() function"
    lst = MX.reset_backends({"luatl_adapter": stub(matmul=lambda *a: None)})
    assert lst[0]["available"] and lst[0]["reason"] == "ready"


def test_threshold_gate_and_fallback_equals_lua_loops():
    seen = []

    def mm(a, m, k, b, n):
        seen.append((m, k, n))
        return list((np.asarray(a).reshape(m, k) @ np.asarray(b).reshape(k, n)).ravel())
    MX.reset_backends({"luatl_adapter": stub(matmul=mm)})
    rng = np.random.default_rng(0)
    small_a, small_b = rng.uniform(-1, 1, (4, 8)), rng.uniform(-1, 1, (8, 16))   # 512 < 4096
    r = MX.multiply(M(small_a), M(small_b))
    assert MX.last_backend == "lua" and not seen
    np.testing.assert_array_equal(r.to_numpy(), O.mm(small_a, small_b))   # same loop order: exact
    big_a, big_b = rng.uniform(-1, 1, (16, 16)), rng.uniform(-1, 1, (16, 16))   # 4096 >= 4096
    MX.multiply(M(big_a), M(big_b))
    assert MX.last_backend == "luatl_adapter" and seen == [(16, 16, 16)]
    # a backend without matmul_into is skipped (not failed) for out=: the Lua loop runs
    out = M(np.ones((16, 16)))
    MX.multiply(M(big_a), M(big_b), out=out, acc=True)
    assert MX.last_backend == "lua" and len(seen) == 1 and MX.backends()[0]["errors"] == 0
    np.testing.assert_array_equal(out.to_numpy(), O.mm(big_a, big_b, out=np.ones((16, 16)), acc=True))


def _into_stub(log):
    """A backend whose matmul_into computes in float64 and follows the contract:
    rd = product, or rd += product with acc, written in place; returns rd."""
    def into(op, a, m, k, b, n, rd, acc):
        log.append((op, m, k, n, acc))
        A = np.asarray(a, dtype=np.float64).reshape(m, k)
        if op == "nn":
            P = A @ np.asarray(b, dtype=np.float64).reshape(k, n)
        elif op == "nt":
            P = A @ np.asarray(b, dtype=np.float64).reshape(n, k).T
        else:
            P = A.T @ np.asarray(b, dtype=np.float64).reshape(m, n)
        P = P.reshape(-1)
        if acc:
            rd[:] = np.asarray(rd) + P
        else:
            rd[:] = P
        return rd
    return stub(matmul=lambda *a: None, matmul_into=into)


@pytest.mark.parametrize("acc", [True, False])
def test_out_and_acc_offload_through_matmul_into(acc):
    """The backward's calls (tensor2.lua:206-211,222-227) pass out=grad_of(x), acc=true:
    above the threshold all three products go to the backend's matmul_into and land
    in out.data; the result equals the Lua loops on the same operands."""
    log = []
    MX.reset_backends({"luatl_adapter": _into_stub(log)})
    rng = np.random.default_rng(3)
    g = rng.uniform(-1, 1, (16, 24)); w = rng.uniform(-1, 1, (20, 24)); x = rng.uniform(-1, 1, (16, 20))
    base_x = rng.uniform(-1, 1, (16, 20)); base_w = rng.uniform(-1, 1, (20, 24))
    # BACKWARD.matmul for y = x.w: gx += g.w^T, gw += x^T.g
    gx, gw = M(base_x), M(base_w)
    data_x = gx.data
    MX.matmul_nt(M(g), M(w), out=gx, acc=acc)
    assert MX.last_backend == "luatl_adapter" and gx.data is data_x     # written in place
    MX.matmul_tn(M(x), M(g), out=gw, acc=acc)
    assert MX.last_backend == "luatl_adapter"
    # BACKWARD.matmul_nt for s = x.w^T (w 24x20 here): gx += g.w, gw += g^T.x
    s_g = rng.uniform(-1, 1, (16, 24)); w2 = rng.uniform(-1, 1, (24, 20))
    gx2 = M(base_x)
    MX.multiply(M(s_g), M(w2), out=gx2, acc=acc)
    assert MX.last_backend == "luatl_adapter"
    assert [e[0] for e in log] == ["nt", "tn", "nn"] and all(e[4] == acc for e in log)
    MX.use("lua")
    try:
        rx, rw, rx2 = M(base_x), M(base_w), M(base_x)
        MX.matmul_nt(M(g), M(w), out=rx, acc=acc)
        MX.matmul_tn(M(x), M(g), out=rw, acc=acc)
        MX.multiply(M(s_g), M(w2), out=rx2, acc=acc)
    finally:
        MX.use("auto")
    for got, want in ((gx, rx), (gw, rw), (gx2, rx2)):
        np.testing.assert_allclose(got.to_numpy(), want.to_numpy(), rtol=1e-12, atol=1e-12)


def test_matmul_into_failure_falls_back_once_and_counts():
    """A failing matmul_into is counted like a failing matmul; the Lua loop then
    does the whole product once into out (the backend leaves rd untouched on error)."""
    def boom(*a):
        raise RuntimeError("into exploded")
    MX.reset_backends({"luatl_adapter": stub(matmul=lambda *a: None, matmul_into=boom)})
    a = np.ones((16, 16)); out = M(np.full((16, 16), 2.0))
    MX.multiply(M(a), M(a), out=out, acc=True)
    assert MX.last_backend == "lua"
    np.testing.assert_array_equal(out.to_numpy(), np.full((16, 16), 18.0))
    e = MX.backends()[0]
    assert e["errors"] == 1 and e["last_error"] == "into exploded"


def test_below_threshold_out_stays_in_lua_and_acc_without_out_is_plain():
    log, seen = [], []
    st = _into_stub(log)

    def mm(a, m, k, b, n):
        seen.append((m, k, n))
        return list((np.asarray(a).reshape(m, k) @ np.asarray(b).reshape(k, n)).ravel())
    st.matmul = mm
    MX.reset_backends({"luatl_adapter": st})
    small = np.ones((4, 8)); out = M(np.zeros((4, 4)))
    MX.matmul_nt(M(small), M(small), out=out, acc=True)            # 4*8*4 < 4096
    assert MX.last_backend == "lua" and not log
    big = np.ones((16, 16))
    r = MX.multiply(M(big), M(big), acc=True)                       # out=nil: fresh zeros, plain entry
    assert MX.last_backend == "luatl_adapter" and seen == [(16, 16, 16)] and not log
    np.testing.assert_array_equal(r.to_numpy(), np.full((16, 16), 16.0))


def test_transposed_cpu_loops_match_oracle_exactly():
    MX.use("lua")
    rng = np.random.default_rng(1)
    a = rng.uniform(-1, 1, (7, 5)); b = rng.uniform(-1, 1, (9, 5)); c = rng.uniform(-1, 1, (7, 3))
    a[2, 3] = 0.0
    np.testing.assert_array_equal(MX.matmul_nt(M(a), M(b)).to_numpy(), O.matmul_nt(a, b))
    np.testing.assert_array_equal(MX.matmul_tn(M(a), M(c)).to_numpy(), O.matmul_tn(a, c))
    acc0 = rng.uniform(-1, 1, (7, 9))
    out = M(acc0)
    MX.matmul_nt(M(a), M(b), out=out, acc=True)
    np.testing.assert_array_equal(out.to_numpy(), O.matmul_nt(a, b, out=acc0.copy(), acc=True))


def test_zero_skip_semantics_of_lua_loops():
    # matrix.lua:521,530: a==0 terms are skipped, so 0 * inf does not poison the row
    MX.use("lua")
    a = np.array([[0.0, 1.0]]); b = np.array([[np.inf, 2.0], [3.0, 4.0]])
    np.testing.assert_array_equal(MX.multiply(M(a), M(b)).to_numpy(), [[3.0, 4.0]])


def test_failures_counted_then_disabled():
    def boom(*a):
        raise RuntimeError("device exploded\nsecond line")
    MX.reset_backends({"luatl_adapter": stub(matmul=boom)})
    a = np.ones((16, 16))
    for i in range(1, 4):
        r = MX.multiply(M(a), M(a))
        assert MX.last_backend == "lua"
        np.testing.assert_array_equal(r.to_numpy(), np.full((16, 16), 16.0))
        e = MX.backends()[0]
        assert e["errors"] == i and e["last_error"] == "device exploded"
    e = MX.backends()[0]
    assert not e["available"] and e["reason"] == "disabled after 3 failures: device exploded"


def test_malformed_results_are_failures():
    MX.reset_backends({"luatl_adapter": stub(matmul=lambda *a: "nope")})
    MX.multiply(M(np.ones((16, 16))), M(np.ones((16, 16))))
    assert MX.backends()[0]["last_error"] == "matmul returned str, expected flat table"
    MX.reset_backends({"luatl_adapter": stub(matmul=lambda a, m, k, b, n: [1.0] * (m * n - 1))})
    MX.multiply(M(np.ones((16, 16))), M(np.ones((16, 16))))
    assert "malformed" in MX.backends()[0]["last_error"]
    MX.strict = True
    MX.reset_backends({"luatl_adapter": stub(matmul=lambda a, m, k, b, n: [1.0] * 5 + [None] + [1.0] * (m * n - 6))})
    MX.multiply(M(np.ones((16, 16))), M(np.ones((16, 16))))
    assert MX.backends()[0]["last_error"] == "matmul result index 6 is NoneType"


def test_use_forcing_rules():
    MX.reset_backends({"luatl_adapter": stub(available=False, reason="no device")})
    with pytest.raises(RuntimeError, match="not usable: no device"):
        MX.use("luatl_adapter")
    with pytest.raises(ValueError, match="unknown backend"):
        MX.use("cuda")
    assert MX.use("lua") == "lua" and MX.use() == "auto"
    # a forced backend that disables itself mid-run raises from multiply (matrix.lua:586-588)
    MX.reset_backends({"luatl_adapter": stub(matmul=lambda *a: 1 / 0)})
    MX.use("luatl_adapter")
    MX.accel["max_errors"] = 1
    with pytest.raises(RuntimeError, match="was forced"):
        MX.multiply(M(np.ones((2, 2))), M(np.ones((2, 2))))


def test_transposed_products_offload_through_their_own_entry():
    calls = []

    def nt(a, m, k, b, n):
        calls.append("nt")
        return list((np.asarray(a).reshape(m, k) @ np.asarray(b).reshape(n, k).T).ravel())

    def tn(a, m, k, b, n):
        calls.append("tn")
        return list((np.asarray(a).reshape(m, k).T @ np.asarray(b).reshape(m, n)).ravel())
    MX.reset_backends({"luatl_adapter": stub(matmul=lambda *a: None, matmul_nt=nt, matmul_tn=tn)})
    rng = np.random.default_rng(2)
    a, b = rng.uniform(-1, 1, (16, 16)), rng.uniform(-1, 1, (16, 16))
    np.testing.assert_allclose(MX.matmul_nt(M(a), M(b)).to_numpy(), O.matmul_nt(a, b), rtol=1e-12)
    np.testing.assert_allclose(MX.matmul_tn(M(a), M(b)).to_numpy(), O.matmul_tn(a, b), rtol=1e-12)
    assert calls == ["nt", "tn"]
    # a backend without matmul_nt is skipped, not counted as failed
    MX.reset_backends({"luatl_adapter": stub(matmul=lambda *a: None)})
    MX.matmul_nt(M(a), M(b))
    assert MX.last_backend == "lua" and MX.backends()[0]["errors"] == 0
