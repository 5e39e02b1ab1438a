"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the parity checker.

Every check below is independent of the oracle's own formula: reference known
answers (cited), library routines (numpy/scipy/torch float64), closed forms,
invariants and central finite differences.  CPU only.
"""
import math

import numpy as np
import pytest
import scipy.special as sps

import oracle as O

RNG = np.random.default_rng(1234)


def fd_grad(f, x, h=1e-6):
    """Central finite-difference gradient of scalar f at x (float64)."""
    x = np.array(x, dtype=np.float64)
    g = np.zeros_like(x)
    it = np.nditer(x, flags=["multi_index"])
    for _ in it:
        idx = it.multi_index
        old = x[idx]
        x[idx] = old + h; fp = f(x)
        x[idx] = old - h; fm = f(x)
        x[idx] = old
        g[idx] = (fp - fm) / (2 * h)
    return g


# ------------------------------------------------------------------ GEMM family
def test_mm_reference_known_answers():
    # tests/core_test.lua:31-34
    c = O.mm(np.array([[1, 2], [3, 4]]), np.array([[5, 6], [7, 8]]))
    assert c.ravel().tolist() == [19, 22, 43, 50]
    # tests/test.lua:445-449 (adapter legacy flat contract)
    c = O.mm(np.arange(1, 7).reshape(2, 3), np.array([1, 0, 0, 1, 1, 1]).reshape(3, 2))
    assert c.ravel().tolist() == [4, 5, 10, 11]


@pytest.mark.parametrize("m,k,n", [(37, 53, 41), (128, 96, 160), (1, 7, 1), (5, 1, 9)])
def test_gemm_family_vs_numpy(m, k, n):
    a = RNG.uniform(-1, 1, (m, k)); b = RNG.uniform(-1, 1, (k, n))
    np.testing.assert_allclose(O.mm(a, b), a @ b, rtol=1e-12, atol=1e-12)
    bt = np.ascontiguousarray(b.T)
    np.testing.assert_allclose(O.matmul_nt(a, bt), a @ b, rtol=1e-12, atol=1e-12)
    at = np.ascontiguousarray(a.T)            # (k, m) -> A^T B with A stored k x m
    np.testing.assert_allclose(O.matmul_tn(at, b), a @ b, rtol=1e-12, atol=1e-12)
    # (AB)^T = B^T A^T
    np.testing.assert_allclose(O.mm(bt, at), (a @ b).T, rtol=1e-12, atol=1e-12)


def test_gemm_accumulate_doubles():
    # tests/test.lua:115-122: beta = 1 accumulation doubles the product
    a = RNG.uniform(-1, 1, (6, 4)); b = RNG.uniform(-1, 1, (4, 5))
    for fn, bb in ((O.mm, b), (O.matmul_nt, np.ascontiguousarray(b.T))):
        r = fn(a, bb)
        r2 = fn(a, bb, out=r.copy(), acc=True)
        np.testing.assert_allclose(r2, 2 * r, rtol=1e-14)
    at = np.ascontiguousarray(a.T)
    r = O.matmul_tn(at, b); r2 = O.matmul_tn(at, b, out=r.copy(), acc=True)
    np.testing.assert_allclose(r2, 2 * r, rtol=1e-14)


def test_mm_zero_skip_semantics():
    # matrix.lua:521,530,650: a==0 terms are skipped, so 0*inf never makes NaN
    a = np.array([[0.0, 1.0]]); b = np.array([[np.inf], [2.0]])
    assert O.mm(a, b)[0, 0] == 2.0
    # matmul_tn: a^T (1x2) . b (2x1) with a[0] = 0 facing b[0] = inf -> the term is skipped
    assert O.matmul_tn(np.ascontiguousarray(a.T), np.array([[np.inf], [0.0]]))[0, 0] == 0.0
    # matmul_nt has no skip: 0*inf is NaN (matrix.lua:617-619)
    assert np.isnan(O.matmul_nt(a, np.array([[np.inf, 2.0]]))[0, 0])
    # inf propagates through a non-zero term (tests/core_test.lua:95-100 intent)
    assert np.isinf(O.mm(np.array([[np.inf, np.inf]]), np.array([[0.5], [0.5]]))[0, 0])


# ------------------------------------------------------------------ RMSNorm
def test_rmsnorm_forward_invariants():
    x = RNG.normal(0, 1, (5, 16)); w = np.ones(16)
    y, inv = O.rmsnorm_fwd(x, w, eps=0.0)
    np.testing.assert_allclose((y * y).mean(1), 1.0, rtol=1e-12)       # unit RMS
    y2, _ = O.rmsnorm_fwd(7.5 * x, w, eps=0.0)
    np.testing.assert_allclose(y2, y, rtol=1e-12)                        # scale invariant
    np.testing.assert_allclose(inv, 1 / np.sqrt((x * x).mean(1)), rtol=1e-12)
    wr = RNG.normal(1, 0.1, 16)
    yw, _ = O.rmsnorm_fwd(x, wr, eps=0.0)
    np.testing.assert_allclose(yw, y * wr, rtol=1e-12)                   # gain per column


def test_rmsnorm_backward_finite_difference():
    # tests/test.lua:209-243 pattern, but on a random upstream gradient and for dw too
    rows, cols, eps = 3, 8, 1e-5
    x = RNG.normal(0, 1, (rows, cols)); w = RNG.normal(1, 0.3, cols); g = RNG.normal(0, 1, (rows, cols))
    _, inv = O.rmsnorm_fwd(x, w, eps)
    dx, dw = O.rmsnorm_bwd(x, w, inv, g)
    fx = lambda xv: float((O.rmsnorm_fwd(xv, w, eps)[0] * g).sum())
    fw = lambda wv: float((O.rmsnorm_fwd(x, wv, eps)[0] * g).sum())
    np.testing.assert_allclose(dx, fd_grad(fx, x), rtol=1e-6, atol=1e-8)
    np.testing.assert_allclose(dw, fd_grad(fw, w), rtol=1e-6, atol=1e-8)


# ------------------------------------------------------------------ softmax
def test_softmax_known_answers_and_invariants():
    # tests/core_test.lua:48-51: three equal (huge) logits -> 1/3 each
    y = O.softmax_fwd(np.array([[1000.0, 1000.0, 1000.0]]))
    np.testing.assert_allclose(y, 1 / 3, rtol=1e-15)
    x = RNG.normal(0, 2, (9, 9))
    y = O.softmax_fwd(x)
    np.testing.assert_allclose(y.sum(1), 1.0, rtol=1e-14)
    np.testing.assert_allclose(y, sps.softmax(x, axis=1), rtol=1e-13)
    yc = O.softmax_fwd(x, causal=True)
    assert np.all(yc[np.triu_indices(9, 1)] == 0.0)                       # mask is exact zero
    np.testing.assert_allclose(yc.sum(1), 1.0, rtol=1e-14)
    for i in range(9):
        np.testing.assert_allclose(yc[i, :i + 1], sps.softmax(x[i, :i + 1]), rtol=1e-13)
    yo = O.softmax_fwd(x[:4], causal=True, offset=2)                      # offset widens the window
    assert np.all(yo[0, 3:] == 0) and yo[0, 2] > 0
    # tests/test.lua:260-262 adapter softmax_causal({1,2,3,4}, 2x2): [1,0; p,1-p]
    y = O.softmax_fwd(np.array([[1.0, 2.0], [3.0, 4.0]]), causal=True)
    assert y[0, 0] == 1.0 and y[0, 1] == 0.0


@pytest.mark.parametrize("causal", [False, True])
def test_softmax_backward(causal):
    x = RNG.normal(0, 1, (6, 6)); g = RNG.normal(0, 1, (6, 6))
    y = O.softmax_fwd(x, causal=causal)
    dx = O.softmax_bwd(y, g, causal=causal)
    f = lambda xv: float((O.softmax_fwd(xv, causal=causal) * g).sum())
    np.testing.assert_allclose(dx, fd_grad(f, x), rtol=1e-6, atol=1e-9)


# ------------------------------------------------------------------ SiLU / SwiGLU
def test_silu_swiglu_library_and_fd():
    x = np.concatenate([RNG.normal(0, 3, 50), [0.0, 40.0, -40.0, -800.0, 800.0]])
    y, s = O.silu_fwd(x)
    np.testing.assert_allclose(s, sps.expit(x), rtol=1e-14)              # library sigmoid
    np.testing.assert_allclose(y, x * sps.expit(x), rtol=1e-14)
    assert not np.any(np.isnan(y))                                         # stable by sign
    up = RNG.normal(0, 1, x.size)
    np.testing.assert_allclose(O.swiglu_fwd(x, up), x * sps.expit(x) * up, rtol=1e-14)
    gate = RNG.normal(0, 2, (4, 5)); up = RNG.normal(0, 1, (4, 5)); dh = RNG.normal(0, 1, (4, 5))
    dg, du = O.swiglu_bwd(gate, up, dh)
    fg = lambda gv: float((O.swiglu_fwd(gv, up) * dh).sum())
    fu = lambda uv: float((O.swiglu_fwd(gate, uv) * dh).sum())
    np.testing.assert_allclose(dg, fd_grad(fg, gate), rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(du, fd_grad(fu, up), rtol=1e-6, atol=1e-9)
    dx = O.silu_bwd(gate, sps.expit(gate), dh)
    fs = lambda gv: float((O.silu_fwd(gv)[0] * dh).sum())
    np.testing.assert_allclose(dx, fd_grad(fs, gate), rtol=1e-6, atol=1e-9)


# ------------------------------------------------------------------ RoPE
def test_rope_angles_and_rotation():
    c, s = O.rope_angles(10000.0, 4, 0)
    # tests/core_test.lua:88-92: position 0 is the identity
    assert c[0, 0] == 1.0 and s[0, 0] == 0.0
    hd, T = 16, 12
    c, s = O.rope_angles(10000.0, hd, T - 1)
    theta = np.arange(T)[:, None] * 10000.0 ** (-np.arange(0, hd, 2) / hd)[None, :]
    np.testing.assert_allclose(c, np.cos(theta), rtol=1e-13, atol=1e-15)
    np.testing.assert_allclose(s, np.sin(theta), rtol=1e-13, atol=1e-15)
    x = RNG.normal(0, 1, (T, hd))
    y = O.rope_fwd(x, c, s)
    np.testing.assert_allclose(y[0], x[0], rtol=0, atol=0)               # pos 0 identity
    pn = lambda a: a[:, 0::2] ** 2 + a[:, 1::2] ** 2                       # per-pair norms
    np.testing.assert_allclose(pn(y), pn(x), rtol=1e-12)
    # complex-number statement of an interleaved rotation
    z = (x[:, 0::2] + 1j * x[:, 1::2]) * np.exp(1j * theta)
    np.testing.assert_allclose(y[:, 0::2], z.real, atol=1e-12)
    np.testing.assert_allclose(y[:, 1::2], z.imag, atol=1e-12)
    # backward is the transpose (= inverse) rotation: <R x, g> = <x, R^T g>
    g = RNG.normal(0, 1, (T, hd))
    np.testing.assert_allclose((y * g).sum(), (x * O.rope_bwd(g, c, s)).sum(), rtol=1e-12)
    np.testing.assert_allclose(O.rope_bwd(y, c, s), x, atol=1e-12)       # tests/test.lua:277-289
    # odd width: trailing column passes through
    x5 = RNG.normal(0, 1, (T, 5)); c2, s2 = O.rope_angles(10000.0, 4, T - 1)
    assert np.array_equal(O.rope_fwd(x5, c2, s2, 2)[:, 4], x5[:, 4])


def test_rope_heads_contract():
    T, H, hd = 7, 2, 8
    x = RNG.normal(0, 1, (T, H * hd))
    c, s = O.rope_angles(10000.0, hd, T - 1)
    yi = O.rope_heads(x, H, hd, interleaved=True)
    for h in range(H):                                                    # same as tensor2 rope
        np.testing.assert_allclose(yi[:, h * hd:(h + 1) * hd], O.rope_fwd(x[:, h * hd:(h + 1) * hd], c, s),
                                   atol=1e-12)
    # half-split is the interleaved rotation under the pair permutation
    # (half-split slot p holds interleaved element 2p, slot p+hd/2 holds 2p+1)
    perm = np.concatenate([np.arange(0, hd, 2), np.arange(1, hd, 2)])
    xs = x.copy()
    for h in range(H):
        xs[:, h * hd:(h + 1) * hd] = x[:, h * hd + perm]
    ys = O.rope_heads(xs, H, hd, interleaved=False)
    for h in range(H):
        np.testing.assert_allclose(ys[:, h * hd:(h + 1) * hd], yi[:, h * hd + perm], atol=1e-12)
    back = O.rope_heads(yi, H, hd, interleaved=True, inverse=True)       # inverse = identity
    np.testing.assert_allclose(back, x, atol=1e-12)
    pos = np.array([5, 0, 3, 3, 1, 2, 6], dtype=np.int32)
    yp = O.rope_heads(x, H, hd, interleaved=True, pos_ids=pos)
    np.testing.assert_allclose(yp[1], x[1], atol=0)                       # pos 0 untouched


# ------------------------------------------------------------------ cross-entropy
def test_cross_entropy_known_answer_and_library():
    # tests/core_test.lua:54-57: CE([2, 1, 0.1], target 1 (1-based)) = 0.417
    loss, sm, cnt = O.cross_entropy(np.array([[2.0, 1.0, 0.1]]), [0])
    assert cnt == 1
    assert abs(loss - 0.417) < 1e-2                                        # the reference's own bar
    assert abs(loss - (math.log(math.exp(2) + math.exp(1) + math.exp(0.1)) - 2)) < 1e-15
    x = RNG.normal(0, 3, (6, 11)); t = RNG.integers(0, 11, 6)
    loss, sm, cnt = O.cross_entropy(x, t)
    ref = np.mean(sps.logsumexp(x, axis=1) - x[np.arange(6), t])
    assert abs(loss - ref) < 1e-13
    np.testing.assert_allclose(sm, sps.softmax(x, axis=1), rtol=1e-13)
    dl = O.cross_entropy_bwd(sm, t, cnt)
    np.testing.assert_allclose(dl.sum(1), 0, atol=1e-15)                  # tests/test.lua:347-355
    f = lambda xv: O.cross_entropy(xv, t)[0]
    np.testing.assert_allclose(dl, fd_grad(f, x), rtol=1e-6, atol=1e-9)
    # uniform logits give ln V
    assert abs(O.cross_entropy(np.zeros((3, 2000)), [5, 6, 7])[0] - math.log(2000)) < 1e-12


def test_cross_entropy_ignore_and_fused_contract():
    x = RNG.normal(0, 1, (5, 7)); t = np.array([1, 6, 0, 3, 2])
    loss_i, sm, cnt = O.cross_entropy(x, t, ignore_index=0)
    assert cnt == 4 and np.all(sm[2] == 0)
    keep = [0, 1, 3, 4]
    assert abs(loss_i - O.cross_entropy(x[keep], t[keep])[0]) < 1e-14
    # fused per-row contract (tests/test.lua:322-357)
    tt = np.array([2, -1, 7, 3, 9], dtype=np.int32)   # -1 ignored, 7/9 out of range for V=7
    losses, d = O.ce_fused(x, tt, ignore_index=3, gscale=0.25)
    assert losses[1] == 0 and losses[2] == 0 and losses[3] == 0 and losses[4] == 0
    assert np.all(d[1:] == 0)
    assert abs(losses[0] - (sps.logsumexp(x[0]) - x[0, 2])) < 1e-13
    np.testing.assert_allclose(d[0], 0.25 * (sps.softmax(x[0]) - np.eye(7)[2]), rtol=1e-13, atol=1e-16)


# ------------------------------------------------------------------ argmax / embed
def test_argmax_known_answer_and_ties():
    # tests/test.lua:375-379
    assert O.argmax_rows(np.array([[1, 9, 2], [8, 3, 4]], dtype=float)).tolist() == [1, 0]
    x = np.array([[3, 7, 7, 1], [np.nan, 2, np.nan, 2], [-np.inf] * 4, [np.nan] * 4,
                  [-np.inf, -5, np.inf, np.inf]])
    assert O.argmax_rows(x).tolist() == [1, 1, 0, 0, 2]
    r = RNG.normal(0, 1, (50, 33))
    assert np.array_equal(O.argmax_rows(r), np.argmax(r, 1))


def test_embed_gather_scatter():
    # tests/test.lua:291-320: ids {3,0,7,3,1} (0-based on device)
    V, D = 10, 4
    tbl = RNG.uniform(-1, 1, (V, D)); ids = np.array([3, 0, 7, 3, 1])
    out = O.embed_fwd(tbl, ids)
    assert np.array_equal(out, tbl[ids])
    dt = O.embed_bwd(np.ones((5, D)), ids, V)
    assert np.all(dt[3] == 2) and np.all(dt[0] == 1) and np.all(dt[2] == 0)


# ------------------------------------------------------------------ optimizer
def test_grad_norm_and_sgd_closed_form():
    assert O.grad_norm(np.array([3.0, 4.0])) == 5.0                       # tests/test.lua:157-161
    p = np.array([1.0, -2.0]); v = np.zeros(2); g = np.array([0.5, 0.25])
    O.sgd_step(p, g, v, lr=0.1, momentum=0.9, wd=0.01)
    # step 1: g' = g + wd p = [0.51, 0.23]; v = g'; p -= lr v
    np.testing.assert_allclose(v, [0.51, 0.23], rtol=1e-15)
    np.testing.assert_allclose(p, [0.949, -2.023], rtol=1e-15)
    O.sgd_step(p, g, v, lr=0.1, momentum=0.9, wd=0.01)
    # step 2: g' = [0.50949, 0.22977]; v = 0.9*[0.51,0.23] + g' = [0.96849, 0.43677]
    np.testing.assert_allclose(v, [0.96849, 0.43677], rtol=1e-14)
    np.testing.assert_allclose(p, [0.949 - 0.096849, -2.023 - 0.043677], rtol=1e-14)


def test_sgd_nesterov_and_plain_closed_form():
    """optim2.lua:84-97: Nesterov steps by g' + momentum*v instead of v, and
    momentum 0 is plain SGD on g' = g + wd*p (hand-computed values)."""
    g = np.array([0.5, 0.25])
    p = np.array([1.0, -2.0]); v = np.zeros(2)
    O.sgd_step(p, g, v, lr=0.1, momentum=0.9, wd=0.01, nesterov=True)
    # step 1: g' = [0.51, 0.23] = v; p -= 0.1 * (g' + 0.9 v) = 0.1 * 1.9 g'
    np.testing.assert_allclose(v, [0.51, 0.23], rtol=1e-15)
    np.testing.assert_allclose(p, [0.9031, -2.0437], rtol=1e-14)
    O.sgd_step(p, g, v, lr=0.1, momentum=0.9, wd=0.01, nesterov=True)
    # step 2: g' = g + 0.01 p = [0.509031, 0.229563]; v = 0.9 v + g' = [0.968031, 0.436563];
    # p -= 0.1 * (g' + 0.9 v) = 0.1 * [1.3802589, 0.6224697]
    np.testing.assert_allclose(v, [0.968031, 0.436563], rtol=1e-14)
    np.testing.assert_allclose(p, [0.76507411, -2.10594697], rtol=1e-14)
    # momentum 0: no velocity, p -= lr * (g + wd p); v untouched
    p = np.array([1.0, -2.0]); v = np.array([7.0, 7.0])
    O.sgd_step(p, g, v, lr=0.1, momentum=0.0, wd=0.01)
    np.testing.assert_allclose(p, [1.0 - 0.051, -2.0 - 0.023], rtol=1e-15)
    assert np.array_equal(v, [7.0, 7.0])


def test_adamw_closed_forms():
    """optim2.lua:116-147.  No reference test holds AdamW vectors, so the
    restatement is pinned by what the algorithm fixes: with a constant
    gradient the bias corrections make m/bc1 = g and v/bc2 = g^2 exactly at
    every t, so each step is p <- p(1 - lr*wd) - lr*g/(|g| + eps); with a zero
    gradient p decays as (1 - lr*wd)^t and the moments stay 0; the moments
    follow their recurrences (a wrong beta, a missing or misplaced bias
    correction, or coupled decay fails one of these)."""
    lr, b1, b2, eps, wd = 0.1, 0.9, 0.95, 1e-8, 0.01
    g = np.array([2.0, -0.5, 1e-3, 0.0])
    p = np.array([1.0, 3.0, -2.0, 0.5]); m = np.zeros(4); v = np.zeros(4)
    pexp = p.copy()
    for t in range(1, 8):
        O.adamw_step(p, g, m, v, t, lr, b1, b2, eps, wd)
        pexp = pexp * (1 - lr * wd) - lr * g / (np.abs(g) + eps)
        np.testing.assert_allclose(p, pexp, rtol=1e-13, atol=1e-15)
        np.testing.assert_allclose(m, (1 - b1 ** t) * g, rtol=1e-13, atol=0)
        np.testing.assert_allclose(v, (1 - b2 ** t) * g * g, rtol=1e-13, atol=0)
    # zero gradient: pure decoupled decay
    p = np.array([1.0, -4.0]); m = np.zeros(2); v = np.zeros(2)
    for t in range(1, 6):
        O.adamw_step(p, np.zeros(2), m, v, t, lr, b1, b2, eps, wd)
    np.testing.assert_allclose(p, np.array([1.0, -4.0]) * (1 - lr * wd) ** 5, rtol=1e-14)
    assert np.all(m == 0) and np.all(v == 0)
    # changing gradient, two steps by hand: t=1 then t=2
    p = np.array([1.0]); m = np.zeros(1); v = np.zeros(1)
    O.adamw_step(p, np.array([1.0]), m, v, 1, lr, b1, b2, eps, wd)
    O.adamw_step(p, np.array([-3.0]), m, v, 2, lr, b1, b2, eps, wd)
    m2 = b1 * (1 - b1) * 1.0 + (1 - b1) * -3.0          # = -0.21
    v2 = b2 * (1 - b2) * 1.0 + (1 - b2) * 9.0            # = 0.4975
    p1 = (1.0 - lr * wd) - lr * 1.0 / (1.0 + eps)
    p2 = p1 * (1 - lr * wd) - lr / (1 - b1 ** 2) * m2 / (np.sqrt(v2 / (1 - b2 ** 2)) + eps)
    assert abs(m[0] - m2) < 1e-15 and abs(v[0] - v2) < 1e-15
    assert abs(p[0] - p2) < 1e-14


# ------------------------------------------------------------------ LMTrain
TINY = dict(vocab=32, dim=16, layers=2, heads=2, ffn=24)


def _tiny_params(cfg, scale=0.3, seed=7):
    rng = np.random.default_rng(seed)
    tab = O.lm_param_table(cfg)
    p = np.zeros(O.lm_num_params(cfg))
    for (name, off, r, c) in tab:
        if name.startswith("ln"):
            p[off:off + r * c] = rng.normal(1, 0.1, r * c)
        else:
            p[off:off + r * c] = rng.normal(0, scale, r * c)
    return p, tab


def test_lm_param_layout():
    cfg = O.lm_cfg(2000, 128, 4, 8, 256)
    # config-2 parameter count: 2000*128 + 4*(2*128 + 4*128*128 + 3*128*256) + 128
    assert O.lm_num_params(cfg) == 912512
    tab = O.lm_param_table(cfg)
    assert tab[0][0] == "emb" and tab[-1][0] == "lnf" and len(tab) == 38
    assert sum(r * c for (_, _, r, c) in tab) == 912512


def test_lm_window_vs_torch_autograd():
    torch = pytest.importorskip("torch")
    from tests import lm_torch_ref as ref
    cfg = O.lm_cfg(**TINY)
    p, tab = _tiny_params(cfg)
    rng = np.random.default_rng(3)
    T = 9
    ids = rng.integers(0, cfg.vocab, T); tgt = rng.integers(0, cfg.vocab, T)
    loss, g, logits, corr = O.lm_window(cfg, p, ids, tgt)
    tl, tg, tlog = ref.window_grad(cfg, p, tab, ids, tgt)
    assert abs(loss - tl) < 1e-12
    np.testing.assert_allclose(logits, tlog, rtol=1e-11, atol=1e-13)
    np.testing.assert_allclose(g, tg, rtol=1e-9, atol=1e-12)
    assert corr == int((np.argmax(tlog, 1) == tgt).sum())
    del torch


def test_lm_window_finite_difference_spot():
    cfg = O.lm_cfg(vocab=11, dim=8, layers=1, heads=2, ffn=6)
    p, tab = _tiny_params(cfg, scale=0.5, seed=11)
    ids = np.array([1, 4, 4, 9, 0]); tgt = np.array([4, 4, 9, 0, 2])
    _, g, _, _ = O.lm_window(cfg, p, ids, tgt)
    rng = np.random.default_rng(5)
    for idx in rng.choice(p.size, 25, replace=False):
        h = 1e-6
        pp = p.copy(); pp[idx] += h; lp = O.lm_window(cfg, pp, ids, tgt)[0]
        pm = p.copy(); pm[idx] -= h; lm = O.lm_window(cfg, pm, ids, tgt)[0]
        assert abs((lp - lm) / (2 * h) - g[idx]) < 1e-7 + 1e-5 * abs(g[idx])


def test_lm_uniform_logits_give_ln_vocab():
    cfg = O.lm_cfg(**TINY)
    p, tab = _tiny_params(cfg)
    p[tab[0][1]:tab[0][1] + cfg.vocab * cfg.dim] = 0.0                   # zero tied embedding
    loss = O.lm_window(cfg, p, np.arange(5), np.arange(5))[0]
    assert abs(loss - math.log(cfg.vocab)) < 1e-13


def test_lm_step_sgd_semantics():
    """lmtrain.lua:1183-1227: mean of window grads, clip, SGD(mom, wd)."""
    cfg = O.lm_cfg(**TINY)
    p0, tab = _tiny_params(cfg)
    rng = np.random.default_rng(9)
    B, T = 3, 6
    ids = rng.integers(0, cfg.vocab, (B, T)); tgt = rng.integers(0, cfg.vocab, (B, T))
    gsum = np.zeros(p0.size); losses = []
    for b in range(B):
        l, gsum, _, _ = O.lm_window(cfg, p0, ids[b], tgt[b], grads=gsum)
        losses.append(l)
    gmean = gsum / B
    norm = float(np.sqrt((gmean ** 2).sum()))
    for clip in (1e9, 0.5 * norm):
        p = p0.copy(); v = np.zeros_like(p)
        out = O.lm_step_sgd(cfg, p, v, ids, tgt, lr=0.05, momentum=0.9, wd=0.01, clip_norm=clip)
        assert out["applied"]
        np.testing.assert_allclose(out["losses"], losses, rtol=1e-14)
        assert abs(out["gnorm"] - norm) < 1e-12 * norm
        gexp = gmean * (clip / norm if norm > clip else 1.0)
        np.testing.assert_allclose(out["grads"], gexp, rtol=1e-12, atol=1e-16)
        gp = gexp + 0.01 * p0
        np.testing.assert_allclose(v, gp, rtol=1e-12, atol=1e-16)
        np.testing.assert_allclose(p, p0 - 0.05 * gp, rtol=1e-12, atol=1e-16)
    # a non-finite gradient norm skips the step (lmtrain.lua:1214-1218)
    bad = p0.copy(); bad[tab[1][1]] = np.nan
    v = np.zeros_like(bad); before = bad.copy()
    out = O.lm_step_sgd(cfg, bad, v, ids, tgt, lr=0.05)
    assert not out["applied"]
    assert np.array_equal(np.isnan(bad), np.isnan(before)) and np.all(v == 0)


def test_lm_step_adamw_semantics():
    """lmtrain.lua:1183-1227 with optimizer "adamw": the same batch gradient as
    the SGD step (scale 1/B, clip), then AdamW with t advanced only for an
    applied step; a skipped step leaves params, moments and t unchanged."""
    cfg = O.lm_cfg(**TINY)
    p0, tab = _tiny_params(cfg)
    rng = np.random.default_rng(19)
    B, T = 2, 5
    ids = rng.integers(0, cfg.vocab, (B, T)); tgt = rng.integers(0, cfg.vocab, (B, T))
    ps = p0.copy(); vs = np.zeros_like(ps)
    ref = O.lm_step_sgd(cfg, ps, vs, ids, tgt, lr=0.0, momentum=0.0, wd=0.0, clip_norm=0.3)
    p = p0.copy(); m = np.zeros_like(p); v = np.zeros_like(p)
    out = O.lm_step_adamw(cfg, p, m, v, 0, ids, tgt, lr=1e-2, beta1=0.9, beta2=0.95, eps=1e-8, wd=0.01,
                          clip_norm=0.3)
    assert out["applied"] and out["t"] == 1
    np.testing.assert_allclose(out["grads"], ref["grads"], rtol=1e-14, atol=0)
    pe = p0.copy(); me = np.zeros_like(pe); ve = np.zeros_like(pe)
    O.adamw_step(pe, ref["grads"], me, ve, 1, 1e-2, 0.9, 0.95, 1e-8, 0.01)
    np.testing.assert_allclose(p, pe, rtol=1e-14, atol=0)
    np.testing.assert_allclose(m, me, rtol=1e-14, atol=0)
    bad = p.copy(); bad[tab[1][1]] = np.nan
    mb, vb = m.copy(), v.copy()
    out = O.lm_step_adamw(cfg, bad, mb, vb, 1, ids, tgt, lr=1e-2)
    assert not out["applied"] and out["t"] == 1
    assert np.array_equal(mb, m) and np.array_equal(vb, v)


# ------------------------------------------------- luaTL operation set (GPU reference path)
def test_ew_unary_operators_against_libraries():
    """cuda/luaTL_core.cu:909-934, unary half: each against a library routine."""
    x = np.linspace(-40, 40, 801)
    assert np.allclose(O.ew("SIGMOID", x, None), sps.expit(x), rtol=1e-14, atol=1e-300)
    assert np.allclose(O.ew("SILU", x, None), x * sps.expit(x), rtol=1e-14, atol=1e-300)
    assert np.allclose(O.ew("TANH", x, None), np.tanh(x), rtol=1e-14)
    xs = np.linspace(-5, 5, 101)
    assert np.allclose(O.ew("EXP", xs, None), np.exp(xs), rtol=1e-14)
    assert np.array_equal(O.ew("RELU", x, None), np.maximum(x, 0))
    assert np.array_equal(O.ew("ABS", x, None), np.abs(x))
    assert np.array_equal(O.ew("NEG", x, None), -x)
    assert np.array_equal(O.ew("COPY", x, None), x)
    assert np.allclose(O.ew("SQRT", x, None), np.sqrt(np.maximum(x, 0)), rtol=1e-15)
    assert O.ew("RSQRT", np.array([4.0]), None)[0] == 0.5 and O.ew("RECIP", np.array([4.0]), None)[0] == 0.25
    # the tanh form approximates x * Phi(x) to within 1e-3 everywhere (its
    # published accuracy); a wrong coefficient or a missing 0.5 breaks this
    xg = np.linspace(-8, 8, 3201)
    assert np.max(np.abs(O.ew("GELU", xg, None) - xg * sps.ndtr(xg))) < 1e-3


def test_ew_derivative_operators_against_central_differences():
    """DSILU / DGELU / DRELU: b times the derivative of the unary operator."""
    a = np.linspace(-6, 6, 241)
    b = RNG.uniform(-2, 2, a.size)
    h = 1e-6
    for dop, op in (("DSILU", "SILU"), ("DGELU", "GELU")):
        fd = (O.ew(op, a + h, None) - O.ew(op, a - h, None)) / (2 * h)
        assert np.allclose(O.ew(dop, a, b), b * fd, atol=1e-8), dop
    assert np.array_equal(O.ew("DRELU", a, b), np.where(a > 0, b, 0.0))


def test_ew_binary_operators_hand_values():
    """The binary rows of luaTL's table on hand-picked values.  AXPY is
    alpha*a + b (luaTL_core.cu:921): Tensor:add_inplace(B, alpha) runs it with
    a = self, b = B (luaTL.lua:634-638), so it computes alpha*self + B."""
    one = lambda op, a, b, al, be: O.ew(op, np.array([a]), np.array([b]), al, be)[0]  # noqa: E731
    assert one("ADD", 2, 3, 2.0, 0.5) == 5.5
    assert one("SUB", 2, 3, 2.0, 0.5) == 2.5
    assert one("MUL", 2, 3, 0.5, 9.0) == 3.0
    assert abs(one("DIV", 3, 4, 2.0, 9.0) - 1.5) < 1e-15
    assert one("SCALE", 3, 99, 2.0, 1.0) == 7.0
    assert one("AXPY", 3, 4, 2.0, 9.0) == 10.0
    assert one("FILL", 3, 4, 2.5, 9.0) == 2.5
    assert one("CLAMP", 5, 0, -1.0, 2.0) == 2.0 and one("CLAMP", -5, 0, -1.0, 2.0) == -1.0
    # a missing operand reads as 0
    assert O.ew("ADD", np.array([2.0]), None, 1.0, 1.0)[0] == 2.0


def _np_gemm_ref(a, b, c0, alpha, beta, bias=None, act=None):
    v = alpha * (a @ b)
    if bias is not None:
        v = v + bias[None, :]
    if act is not None:
        v = act(v)
    return v + beta * c0 if beta != 0 else v


def test_gemm_ex_strides_batches_and_epilogue():
    """cuda/luaTL_train.cu:127-234 against numpy products of explicit copies."""
    M, N, K = 7, 5, 6
    # A given transposed (stored K x M: a_rs = 1, a_cs = M), C column-major
    at = RNG.standard_normal((K, M))
    b = RNG.standard_normal((K, N))
    c0 = RNG.standard_normal((N, M))                 # C^T stored
    C = c0.copy().ravel()
    O.gemm_ex(at.ravel(), b.ravel(), C, M, N, K, (1, M, N, 1, 1, M, 0, 0, 0), alpha=0.5, beta=2.0)
    ref = _np_gemm_ref(at.T, b, c0.T, 0.5, 2.0)
    assert np.allclose(C.reshape(N, M).T, ref, rtol=1e-13)
    # bias + GELU + beta, row-major; beta == 0 never reads C
    a = RNG.standard_normal((M, K))
    bias = RNG.standard_normal(N)
    c1 = RNG.standard_normal((M, N))
    C = c1.copy().ravel()
    O.gemm_ex(a.ravel(), b.ravel(), C, M, N, K, (K, 1, N, 1, N, 1, 0, 0, 0), alpha=1.5, beta=-1.0, act=2,
              bias=bias)
    gelu = lambda v: O.ew("GELU", v, None)  # noqa: E731 (pinned above)
    assert np.allclose(C.reshape(M, N), _np_gemm_ref(a, b, c1, 1.5, -1.0, bias, gelu), rtol=1e-12)
    C = np.full(M * N, np.nan)
    O.gemm_ex(a.ravel(), b.ravel(), C, M, N, K, (K, 1, N, 1, N, 1, 0, 0, 0), act=5)
    assert np.allclose(C.reshape(M, N), sps.expit(a @ b), rtol=1e-13)
    # batched per-head views: q (T x H*hd) . k^T per head into S (H x T x T)
    T, H, hd = 5, 3, 4
    q = RNG.standard_normal((T, H * hd)); k = RNG.standard_normal((T, H * hd))
    S = np.zeros(H * T * T)
    O.gemm_ex(q.ravel(), k.ravel(), S, T, T, hd, (H * hd, 1, 1, H * hd, T, 1, hd, hd, T * T), batch=H)
    S = S.reshape(H, T, T)
    for h in range(H):
        qs, ks = q[:, h * hd:(h + 1) * hd], k[:, h * hd:(h + 1) * hd]
        assert np.allclose(S[h], qs @ ks.T, rtol=1e-13)


def test_gemm_ex_prologues():
    """pre RMSNORM equals or_rmsnorm_fwd's rows (pinned by finite differences)
    times B, with rowscale computed or given; pre SILU/RELU map A elementwise."""
    M, N, K = 6, 4, 8
    a = RNG.standard_normal((M, K)); b = RNG.standard_normal((K, N)); g = RNG.normal(1, 0.1, K)
    eps = 1e-5
    y, inv = O.rmsnorm_fwd(a, g, eps)
    C = np.zeros(M * N)
    O.gemm_ex(a.ravel(), b.ravel(), C, M, N, K, (K, 1, N, 1, N, 1, 0, 0, 0), pre=1, gamma=g, eps=eps)
    assert np.allclose(C.reshape(M, N), y @ b, rtol=1e-12)
    rs = RNG.uniform(0.5, 2, M)
    C = np.zeros(M * N)
    O.gemm_ex(a.ravel(), b.ravel(), C, M, N, K, (K, 1, N, 1, N, 1, 0, 0, 0), pre=1, rowscale=rs)
    assert np.allclose(C.reshape(M, N), (a * rs[:, None]) @ b, rtol=1e-12)
    for pre, f in ((3, lambda v: v * sps.expit(v)), (4, lambda v: np.maximum(v, 0))):
        C = np.zeros(M * N)
        O.gemm_ex(a.ravel(), b.ravel(), C, M, N, K, (K, 1, N, 1, N, 1, 0, 0, 0), pre=pre)
        assert np.allclose(C.reshape(M, N), f(a) @ b, rtol=1e-12)


def _kept_softmax(v, lim):
    out = np.zeros_like(v)
    if lim > 0:
        out[:lim] = sps.softmax(v[:lim])
    return out


def test_softmax_ex_against_scipy_and_the_cpu_form():
    rows, cols = 9, 7
    x = RNG.standard_normal((rows, cols)) * 2
    bias = RNG.standard_normal(cols)
    for causal, group, moff, scale, bb in ((False, 0, 0, 0.5, None), (True, 3, 0, 1.0, None),
                                           (True, 0, 2, 0.7, bias), (True, 4, -2, 1.0, None)):
        y = O.softmax_ex(x, bb, scale, causal, group, moff)
        for r in range(rows):
            lrow = r % group if group > 0 else r
            lim = min(max(lrow + moff + 1, 0), cols) if causal else cols
            v = x[r] * scale + (bb if bb is not None else 0)
            assert np.allclose(y[r], _kept_softmax(v, lim), rtol=1e-13, atol=1e-300)
    # a negative offset masks whole rows: all zero
    y = O.softmax_ex(x, None, 1.0, True, 0, -3)
    assert not y[:3].any() and np.allclose(y[3:].sum(1), 1)
    # where the contracts coincide (offset >= 0, group = rows) it equals the
    # CPU path's or_softmax_fwd
    assert np.allclose(O.softmax_ex(x, None, 1.0, True, 0, 1), O.softmax_fwd(x, causal=True, offset=1), rtol=1e-14)


def test_softmax_bwd_ex_by_central_differences():
    rows, cols = 5, 6
    x = RNG.standard_normal((rows, cols))
    dy = RNG.standard_normal((rows, cols))
    for causal, group, moff, scale in ((False, 0, 0, 0.8), (True, 2, 1, 1.3), (True, 0, -2, 1.0)):
        y = O.softmax_ex(x, None, scale, causal, group, moff)
        dx = O.softmax_bwd_ex(y, dy, scale, causal, group, moff)
        f = lambda xx: float(np.sum(dy * O.softmax_ex(xx, None, scale, causal, group, moff)))  # noqa: E731
        assert np.allclose(dx, fd_grad(f, x), atol=1e-8)


def test_rmsnorm_bwd_luatl_matches_the_cpu_form():
    rows, cols, eps = 6, 10, 1e-5
    x = RNG.standard_normal((rows, cols)); g = RNG.normal(1, 0.1, cols); dy = RNG.standard_normal((rows, cols))
    _, inv = O.rmsnorm_fwd(x, g, eps)
    dx_ref, dg_ref = O.rmsnorm_bwd(x, g, inv, dy)
    dg = np.zeros(cols)
    dx = O.rmsnorm_bwd_luatl(x, g, dy, eps, dg)
    assert np.allclose(dx, dx_ref, rtol=1e-12) and np.allclose(dg, dg_ref, rtol=1e-12)
    O.rmsnorm_bwd_luatl(x, g, dy, eps, dg)            # dgamma accumulates
    assert np.allclose(dg, 2 * dg_ref, rtol=1e-12)
    assert np.allclose(O.rmsnorm_bwd_luatl(x, None, dy, eps), O.rmsnorm_bwd_luatl(x, np.ones(cols), dy, eps))


def test_adamw_luatl_closed_forms():
    """Constant gradient: m*bc1 = g and v*bc2 = g^2 at every t, so each step is
    w(1 - lr*wd) - lr*g/(|g| + eps); clip clamps g first."""
    lr, b1, b2, eps, wd = 0.05, 0.9, 0.999, 1e-8, 0.01
    g = np.array([2.0, -0.5, 1e-3, 0.0, 7.0])
    w = RNG.standard_normal(5); m = np.zeros(5); v = np.zeros(5)
    wexp = w.copy()
    gc = np.clip(g, -3.0, 3.0)
    for t in range(1, 6):
        O.adamw_luatl(w, g, m, v, t, lr, b1, b2, eps, wd, clip=3.0)
        wexp = wexp * (1 - lr * wd) - lr * gc / (np.abs(gc) + eps)
    assert np.allclose(w, wexp, rtol=1e-12, atol=1e-15)
    assert np.allclose(m, (1 - b1 ** 5) * gc, rtol=1e-12) and np.allclose(v, (1 - b2 ** 5) * gc ** 2, rtol=1e-12)


def test_reduce_cols_and_clip():
    x = RNG.standard_normal((11, 6))
    out = RNG.standard_normal(6)
    ref = 0.5 * x.sum(0) + 2.0 * out
    assert np.allclose(O.reduce_cols(x, out.copy(), 0.5, 2.0), ref, rtol=1e-13)
    wide = RNG.standard_normal((4, 10))           # row stride 10, 6 columns summed
    assert np.allclose(O.reduce_cols(wide[:, :6].copy(), np.zeros(6)), wide[:, :6].sum(0))
    y = RNG.standard_normal(50)
    nsq = float(np.sum(y * y)); nrm = math.sqrt(nsq)
    z = O.clip_by_nsq(y.copy(), nsq, nrm / 4)
    assert abs(np.linalg.norm(z) - (nrm / 4) * nrm / (nrm + 1e-6)) < 1e-12
    assert np.array_equal(O.clip_by_nsq(y.copy(), nsq, 2 * nrm), y)     # below the bound: unchanged


def test_lm_ragged_batch_vs_torch_autograd():
    """lmtrain.lua:535-558 (a short last window) and :1183-1212 (a short last
    batch): each window's loss is the mean over its own tokens, the gradients
    of the n_in_batch windows are summed and scaled by 1/n_in_batch.  Checked
    against float64 torch autograd of each truncated window; the content past
    a window's length and in the unused slots must not matter."""
    pytest.importorskip("torch")
    from tests import lm_torch_ref as ref
    cfg = O.lm_cfg(**TINY)
    p0, tab = _tiny_params(cfg)
    rng = np.random.default_rng(21)
    B, T = 4, 8
    ids = rng.integers(0, cfg.vocab, (B, T)); tgt = rng.integers(0, cfg.vocab, (B, T))
    lens, nwin = np.array([8, 3, 5, 8]), 3
    gsum = np.zeros(p0.size); losses = []; corr = 0
    for b in range(nwin):
        tl, tg, tlog = ref.window_grad(cfg, p0, tab, ids[b, :lens[b]], tgt[b, :lens[b]])
        gsum += tg
        losses.append(tl)
        corr += int((np.argmax(tlog, 1) == tgt[b, :lens[b]]).sum())
    gexp = gsum / nwin
    p = p0.copy(); v = np.zeros_like(p)
    out = O.lm_step_sgd(cfg, p, v, ids, tgt, lr=0.0, momentum=0.0, wd=0.0, clip_norm=1e9, lens=lens, nwin=nwin)
    np.testing.assert_allclose(out["losses"][:nwin], losses, rtol=1e-12)
    np.testing.assert_allclose(out["grads"], gexp, rtol=1e-9, atol=1e-12)
    assert out["correct"] == corr
    # padding and unused slots do not matter
    ids2, tgt2 = ids.copy(), tgt.copy()
    ids2[1, 3:] = (ids2[1, 3:] + 5) % cfg.vocab; tgt2[2, 5:] = 0; ids2[3] = 1
    p2 = p0.copy(); v2 = np.zeros_like(p2)
    out2 = O.lm_step_sgd(cfg, p2, v2, ids2, tgt2, lr=0.0, momentum=0.0, wd=0.0, clip_norm=1e9, lens=lens, nwin=nwin)
    assert np.array_equal(out2["grads"], out["grads"]) and np.array_equal(out2["losses"], out["losses"])
    # one window in the batch: no scaling (lmtrain.lua:1211 scales only when n_in_batch > 1)
    out1 = O.lm_step_sgd(cfg, p0.copy(), np.zeros_like(p0), ids, tgt, lr=0.0, momentum=0.0, wd=0.0,
                         clip_norm=1e9, lens=lens, nwin=1)
    np.testing.assert_allclose(out1["grads"], ref.window_grad(cfg, p0, tab, ids[0], tgt[0])[1], rtol=1e-9,
                               atol=1e-12)
    # full lengths are the full-window step
    pa, pb = p0.copy(), p0.copy()
    fa = O.lm_step_sgd(cfg, pa, np.zeros_like(pa), ids, tgt, lr=0.05)
    fb = O.lm_step_sgd(cfg, pb, np.zeros_like(pb), ids, tgt, lr=0.05, lens=np.full(B, T), nwin=B)
    assert np.array_equal(pa, pb) and np.array_equal(fa["grads"], fb["grads"])
