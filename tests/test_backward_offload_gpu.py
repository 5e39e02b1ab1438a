"""GPU parity of the CPU LMTrain backward's GEMM calls, served through the registry.

The autograd backward of ai/core/tensor2.lua issues its products with the
caller's gradient buffer as `out` and `acc = true`:
  * BACKWARD.matmul    (tensor2.lua:206-211): matmul_nt(g, b, grad_of(a), true)
                                              matmul_tn(a, g, grad_of(b), true)
  * BACKWARD.matmul_nt (tensor2.lua:222-227): multiply(g, b, grad_of(a), true)
                                              matmul_tn(g, a, grad_of(b), true)
Each call is replayed through lanternl_amd.matrix (the ai.Matrix registry with
the real backend, not forced) on a non-zero `out`, at config C1 and at the
per-window shapes of config C2's forward products (transformer.lua:196-257):
q/k/v/o, W1/W3, W2, the tied head, QK^T and P.V.  Each must be served by the
backend (`last_backend == "luatl_adapter"`) and agree with the oracle's
restatement of the Lua loops (or_mm / or_matmul_nt / or_matmul_tn with acc):
relative Frobenius <= 1e-4 on the accumulated result and on the added product
alone.
"""
import numpy as np
import pytest

import oracle as O
from lanternl_amd import device
from lanternl_amd import matrix as MX
from tests.gpu_util import announce, f32, rel_fro

pytestmark = pytest.mark.gpu
TOL = 1e-4

# forward products y = x . w (Tensor.matmul) and s = x . w^T (Tensor.matmul_nt):
# (name, kind, x shape, w shape)
FORWARD = [
    ("C1 a.b", "matmul", (256, 128), (128, 256)),
    ("C2 q/k/v/o", "matmul", (64, 128), (128, 128)),
    ("C2 W1/W3", "matmul", (64, 128), (128, 256)),
    ("C2 W2", "matmul", (64, 256), (256, 128)),
    ("C2 P.V", "matmul", (64, 64), (64, 16)),
    ("C2 tied head", "matmul_nt", (64, 128), (2000, 128)),
    ("C2 QK^T", "matmul_nt", (64, 16), (64, 16)),
]


@pytest.fixture(scope="module", autouse=True)
def _dev():
    device.init(0)
    MX.reset_backends()
    assert MX.backends()[0]["available"], MX.backends()[0]["reason"]
    MX.use("auto")
    yield
    MX.use("auto")


def _mat(a):
    return MX.Matrix.from_numpy(a)


def _check(call, who, out0, want_fn, acc):
    """call(out) runs the registry product into `out`; want_fn(out0) is the oracle."""
    out = _mat(out0)
    call(out, acc)
    assert MX.last_backend == "luatl_adapter", f"{who}: served by {MX.last_backend}"
    got = out.to_numpy()
    want = want_fn(out0.copy(), acc)
    e_total = rel_fro(got, want)
    e_prod = rel_fro(got - (out0 if acc else 0.0), want - (out0 if acc else 0.0))
    print(f"  {who} acc={acc}: rel_fro total {e_total:.2e} product {e_prod:.2e}", flush=True)
    assert e_total <= TOL and e_prod <= TOL, (who, e_total, e_prod)


@pytest.mark.parametrize("acc", [True, False])
@pytest.mark.parametrize("name,kind,xs,ws", FORWARD, ids=[f[0] for f in FORWARD])
def test_backward_calls_offload_with_out_and_acc(name, kind, xs, ws, acc):
    announce("backward offload", name, kind, xs, ws, "acc" if acc else "out")
    rng = np.random.default_rng(2 * [f[0] for f in FORWARD].index(name) + int(acc))
    x = f32(rng.uniform(-1, 1, xs))
    w = f32(rng.normal(0, 0.02 if name == "C2 tied head" else 0.5, ws))
    ys = (xs[0], ws[1]) if kind == "matmul" else (xs[0], ws[0])
    g = f32(rng.normal(0, 1, ys))
    gx0 = rng.uniform(-1, 1, xs)                 # non-zero gradient buffers (doubles)
    gw0 = rng.uniform(-1, 1, ws)
    if kind == "matmul":
        # BACKWARD.matmul: gx (+)= g . w^T ; gw (+)= x^T . g
        _check(lambda out, a: MX.matmul_nt(_mat(g), _mat(w), out, a), f"{name} dx=g.w^T",
               gx0, lambda o, a: O.matmul_nt(g, w, out=o, acc=a), acc)
        _check(lambda out, a: MX.matmul_tn(_mat(x), _mat(g), out, a), f"{name} dw=x^T.g",
               gw0, lambda o, a: O.matmul_tn(x, g, out=o, acc=a), acc)
    else:
        # BACKWARD.matmul_nt: gx (+)= g . w ; gw (+)= g^T . x
        _check(lambda out, a: MX.multiply(_mat(g), _mat(w), out, a), f"{name} dx=g.w",
               gx0, lambda o, a: O.mm(g, w, out=o, acc=a), acc)
        _check(lambda out, a: MX.matmul_tn(_mat(g), _mat(x), out, a), f"{name} dw=g^T.x",
               gw0, lambda o, a: O.matmul_tn(g, x, out=o, acc=a), acc)


def test_backward_chain_accumulates_over_windows():
    """LMTrain sums every window's gradient into one buffer (lmtrain.lua:1183-1212):
    eight acc=true products into the same out, as eight windows' dW of W1."""
    announce("backward offload: 8-window accumulation")
    rng = np.random.default_rng(11)
    gw = _mat(np.zeros((128, 256)))
    want = np.zeros((128, 256))
    for _ in range(8):
        x = f32(rng.uniform(-1, 1, (64, 128)))
        g = f32(rng.normal(0, 1, (64, 256)))
        MX.matmul_tn(_mat(x), _mat(g), gw, True)
        assert MX.last_backend == "luatl_adapter"
        want = O.matmul_tn(x, g, out=want, acc=True)
    assert rel_fro(gw.to_numpy(), want) <= TOL


def test_below_threshold_backward_call_stays_in_lua():
    """m*k*n < 4096 keeps the Lua loop (matrix.lua:19,575-576), exactly the oracle."""
    announce("backward offload: below threshold")
    rng = np.random.default_rng(12)
    g = f32(rng.normal(0, 1, (8, 8))); w = f32(rng.uniform(-1, 1, (8, 8)))
    out0 = rng.uniform(-1, 1, (8, 8))
    out = _mat(out0)
    MX.matmul_nt(_mat(g), _mat(w), out, True)
    assert MX.last_backend == "lua"
    np.testing.assert_array_equal(out.to_numpy(), O.matmul_nt(g, w, out=out0.copy(), acc=True))


def test_matmul_into_list_tables_and_errors_leave_rd_untouched():
    """The entry itself, as the Lua module's caller sees it: Python lists in and out
    (Lua tables), rd written in place; a failing call (short operand) raises and
    leaves rd as it was."""
    announce("backend.matmul_into lists")
    from lanternl_amd import backend as B
    rd = [1.0, 1.0, 1.0, 1.0]
    got = B.matmul_into("nn", [1, 2, 3, 4, 5, 6], 2, 3, [1, 0, 0, 1, 1, 1], 2, rd, True)
    assert got is rd and rd == [5.0, 6.0, 11.0, 12.0]               # tests/test.lua:445-449 + 1
    B.matmul_into("nt", [1, 2, 3, 4, 5, 6], 2, 3, [1, 0, 0, 0, 1, 1], 2, rd, False)
    assert rd == [1.0, 5.0, 4.0, 11.0]
    rd6 = [0.5] * 6
    B.matmul_into("tn", [1, 2, 3, 4, 5, 6], 2, 3, [1, 0, 0, 1], 2, rd6, True)   # a^T . I
    assert rd6 == [1.5, 4.5, 2.5, 5.5, 3.5, 6.5]
    with pytest.raises(ValueError, match="rd holds 4"):
        B.matmul_into("tn", [1, 2, 3, 4, 5, 6], 2, 3, [1, 0, 0, 1], 2, rd, True)
    before = list(rd)
    with pytest.raises(ValueError, match="needs 6 numbers"):
        B.matmul_into("nn", [1, 2, 3], 2, 3, [1, 0, 0, 1, 1, 1], 2, rd, True)
    with pytest.raises(ValueError, match="op must be"):
        B.matmul_into("tt", [1, 2, 3, 4, 5, 6], 2, 3, [1, 0, 0, 1, 1, 1], 2, rd, True)
    assert rd == before
