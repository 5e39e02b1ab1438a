"""GPU parity of the bandwidth-bound kernels against the CPU oracle.

Each kernel runs through the C ABI on identical fp32-representable inputs and
is compared with the double-precision restatement of the Lua path
(oracle/oracle.c, which tests/test_oracle.py pins).  Tolerances are written
per test: fp32 elementwise results are held to a relative Frobenius error of
1e-5 (the fp32 rounding of a handful of operations), the cross-entropy loss to
1e-5 absolute, indices and gathers bit-exactly.
Sizes include the C4 shapes (tokens=4096, dim=1024, ffn=4096) and C3
(512 x 32000 logits).
"""
import numpy as np
import pytest

import oracle as O
from lanternl_amd import device
from lanternl_amd._lib import LanternlHipError, call
from tests.gpu_util import announce, f32, rel_fro, to_dev

pytestmark = pytest.mark.gpu
EW = 1e-5          # relative Frobenius bar for fp32 elementwise / row kernels


@pytest.fixture(scope="module", autouse=True)
def _dev():
    device.init(0)
    yield


def dl(buf):
    device.sync()
    return buf.download().astype(np.float64)


# ------------------------------------------------------------------ RMSNorm
@pytest.mark.parametrize("rows,cols,eps", [(64, 128, 1e-5), (512, 128, 1e-5), (4096, 1024, 1e-6),
                                           (7, 13, 1e-5), (3, 5000, 1e-6), (5, 4100, 1e-5), (9, 2048, 1e-6),
                                          (11, 3072, 1e-6), (6, 4096, 1e-5),
                                          # two rows per wave (rows >= 4096): a last wave with one row,
                                          # and rows shorter than a wave's float4 lanes (clamped loads)
                                          (4099, 100, 1e-5), (4101, 1024, 1e-6)])
def test_rmsnorm_fwd_bwd(rows, cols, eps):
    announce("rmsnorm", rows, cols)
    rng = np.random.default_rng(rows * 31 + cols)
    x = f32(rng.standard_normal((rows, cols)))
    w = f32(rng.normal(1.0, 0.1, cols))
    g = f32(rng.standard_normal((rows, cols)))
    y_ref, inv_ref = O.rmsnorm_fwd(x, w, eps)
    X, W, Y, INV = to_dev(x), to_dev(w), device.Buffer((rows, cols)), device.Buffer((rows,))
    call("lhip_rmsnorm_fwd", X.ptr, W.ptr, Y.ptr, INV.ptr, rows, cols, eps)
    assert rel_fro(dl(Y), y_ref) <= EW
    assert rel_fro(dl(INV), inv_ref) <= EW
    dx_ref, dw_ref = O.rmsnorm_bwd(x, w, inv_ref, g)
    G, DX, DW = to_dev(g), device.Buffer((rows, cols)), device.Buffer((cols,))
    call("lhip_rmsnorm_bwd", X.ptr, W.ptr, INV.ptr, G.ptr, DX.ptr, DW.ptr, rows, cols, 0)
    assert rel_fro(dl(DX), dx_ref) <= EW
    assert rel_fro(dl(DW), dw_ref) <= EW
    # accumulate: a second call adds the same amounts
    call("lhip_rmsnorm_bwd", X.ptr, W.ptr, INV.ptr, G.ptr, DX.ptr, DW.ptr, rows, cols, 1)
    assert rel_fro(dl(DX), 2 * dx_ref) <= EW
    assert rel_fro(dl(DW), 2 * dw_ref) <= EW
    # dw = NULL: dx only (no partials are written)
    DX2 = device.Buffer((rows, cols))
    call("lhip_rmsnorm_bwd", X.ptr, W.ptr, INV.ptr, G.ptr, DX2.ptr, None, rows, cols, 0)
    assert rel_fro(dl(DX2), dx_ref) <= EW


def test_rmsnorm_bwd_finite_differences_of_gpu_forward():
    """tests/test.lua:209-243 pattern on the GPU forward itself: d/dx of
    sum(g * rmsnorm(x)) by central differences (fp64 host evaluation of the
    fp32 kernel is too coarse, so the check uses the oracle forward in double
    and the GPU backward)."""
    rng = np.random.default_rng(11)
    rows, cols = 3, 8
    x = f32(rng.standard_normal((rows, cols))); w = f32(rng.normal(1, 0.1, cols))
    g = f32(rng.standard_normal((rows, cols)))
    _, inv = O.rmsnorm_fwd(x, w, 1e-5)
    X, W, INV, G = to_dev(x), to_dev(w), to_dev(inv), to_dev(g)
    DX, DW = device.Buffer((rows, cols)), device.Buffer((cols,))
    call("lhip_rmsnorm_bwd", X.ptr, W.ptr, INV.ptr, G.ptr, DX.ptr, DW.ptr, rows, cols, 0)
    dx = dl(DX)
    h = 1e-6
    fd = np.zeros_like(x)
    for i in range(rows):
        for j in range(cols):
            xp = x.copy(); xp[i, j] += h
            xm = x.copy(); xm[i, j] -= h
            fd[i, j] = (np.sum(g * O.rmsnorm_fwd(xp, w, 1e-5)[0]) - np.sum(g * O.rmsnorm_fwd(xm, w, 1e-5)[0])) / (2 * h)
    assert rel_fro(dx, fd) <= 1e-5


# ------------------------------------------------------------------ softmax
def softmax_ref(x, scale, causal, offset=0, group=None):
    rows = x.shape[0]
    group = group or rows
    out = np.zeros_like(x)
    for r0 in range(0, rows, group):
        out[r0:r0 + group] = O.softmax_fwd(scale * x[r0:r0 + group], causal, offset)
    return out


def softmax_bwd_ref(y, g, scale, causal, offset=0, group=None):
    rows = y.shape[0]
    group = group or rows
    out = np.zeros_like(y)
    for r0 in range(0, rows, group):
        out[r0:r0 + group] = scale * O.softmax_bwd(y[r0:r0 + group], g[r0:r0 + group], causal, offset)
    return out


@pytest.mark.parametrize("rows,cols,scale,causal,offset,group", [
    (4096, 4096, 1.0, 0, 0, 0),          # config C4: scores N(0, 4)
    (64, 64, 0.25, 1, 0, 0),             # one C2 head (T=64, hd=16 -> 1/sqrt(16))
    (8 * 8 * 64, 64, 0.25, 1, 0, 64),    # all C2 heads batched, group-causal
    (37, 53, 1.0, 1, 2, 0),              # generic path (cols % 4 != 0), offset
    (5, 5000, 0.5, 0, 0, 0),             # generic path (row too long for registers)
    (16, 20, 1.0, 1, -3, 8),             # negative offset: lim clamps to 1
    (96, 3072, 0.5, 1, 5, 40),           # workgroup-per-row forward (3 float4 per thread), group-causal
    (64, 4096, 1.0, 1, 0, 0),            # workgroup-per-row forward, causal prefix of a long row
    (32, 3072, 0.7, 0, 0, 0),            # workgroup-per-row, no mask (unconditional loads), 3 float4 per thread
])
def test_softmax_fwd_bwd(rows, cols, scale, causal, offset, group):
    announce("softmax", rows, cols, causal, group)
    rng = np.random.default_rng(rows + cols)
    x = f32(rng.normal(0, 2.0, (rows, cols)))
    g = f32(rng.standard_normal((rows, cols)))
    y_ref = softmax_ref(x, scale, causal, offset, group or None)
    X, Y = to_dev(x), device.Buffer((rows, cols))
    call("lhip_softmax_fwd", X.ptr, Y.ptr, rows, cols, scale, causal, offset, group)
    y = dl(Y)
    assert rel_fro(y, y_ref) <= EW
    assert np.array_equal(y == 0, y_ref == 0) or not causal   # masked entries are exactly zero
    np.testing.assert_allclose(y.sum(axis=1), 1.0, atol=1e-5)
    dx_ref = softmax_bwd_ref(y_ref, g, scale, causal, offset, group or None)
    G, DX = to_dev(g), device.Buffer((rows, cols))
    call("lhip_softmax_bwd", Y.ptr, G.ptr, DX.ptr, rows, cols, scale, causal, offset, group, 0)
    assert rel_fro(dl(DX), dx_ref) <= EW
    # accumulate: a second call adds the same gradient
    call("lhip_softmax_bwd", Y.ptr, G.ptr, DX.ptr, rows, cols, scale, causal, offset, group, 1)
    assert rel_fro(dl(DX), 2 * dx_ref) <= EW


def test_softmax_equal_logits_known_answer():
    """tests/core_test.lua:48-51: softmax of three equal large logits is 1/3 each."""
    X = to_dev(np.full((1, 3), 1000.0)); Y = device.Buffer((1, 3))
    call("lhip_softmax_fwd", X.ptr, Y.ptr, 1, 3, 1.0, 0, 0, 0)
    np.testing.assert_allclose(dl(Y), 1 / 3, rtol=1e-6)
    X = to_dev(np.full((2, 8), 1000.0)); Y = device.Buffer((2, 8))
    call("lhip_softmax_fwd", X.ptr, Y.ptr, 2, 8, 1.0, 0, 0, 0)
    np.testing.assert_allclose(dl(Y), 1 / 8, rtol=1e-6)


# ------------------------------------------------------------------ SwiGLU
# widths on both sides of every size class of the row kernels: float4s per
# lane (1, 2, 4, 8, 16: 256, 512, 1024, 2048 and 4096 columns), the
# workgroup-per-row forms (3072, 4096), the generic path past 4096 and for
# widths that are not a multiple of 4
SWEEP_COLS = [1, 3, 252, 255, 256, 260, 508, 512, 516, 1020, 1024, 1028, 2044, 2048, 2052, 3068, 3072, 3076,
              4092, 4096, 4100]


def test_row_kernels_size_class_sweep():
    """RMSNorm, softmax (random scale, causal prefix, offset and group) and
    SwiGLU, forward and backward, at every SWEEP_COLS width with random row
    counts (one width with enough rows for two rows per wave), against the
    oracle at the row bar."""
    rng = np.random.default_rng(1202)
    for i, cols in enumerate(SWEEP_COLS):
        rows = 4099 if cols == 1020 else int(rng.integers(1, 130))
        announce("row sweep", i, rows, cols)
        x = f32(rng.standard_normal((rows, cols)))
        w = f32(rng.normal(1.0, 0.1, cols))
        g = f32(rng.standard_normal((rows, cols)))
        eps = float(rng.choice([1e-5, 1e-6]))
        y_ref, inv_ref = O.rmsnorm_fwd(x, w, eps)
        X, W, Y, INV, G = to_dev(x), to_dev(w), device.Buffer((rows, cols)), device.Buffer((rows,)), to_dev(g)
        call("lhip_rmsnorm_fwd", X.ptr, W.ptr, Y.ptr, INV.ptr, rows, cols, eps)
        assert rel_fro(dl(Y), y_ref) <= EW and rel_fro(dl(INV), inv_ref) <= EW, ("rmsnorm", rows, cols)
        dx_ref, dw_ref = O.rmsnorm_bwd(x, w, inv_ref, g)
        DX, DW = device.Buffer((rows, cols)), device.Buffer((cols,))
        call("lhip_rmsnorm_bwd", X.ptr, W.ptr, INV.ptr, G.ptr, DX.ptr, DW.ptr, rows, cols, 0)
        assert rel_fro(dl(DX), dx_ref) <= EW and rel_fro(dl(DW), dw_ref) <= EW, ("rmsnorm bwd", rows, cols)
        scale = float(rng.choice([1.0, 0.25, 0.7]))
        causal = int(rng.integers(0, 2))
        offset = int(rng.integers(-2, 4)) if causal else 0
        group = int(rng.choice([0, max(1, rows // 2)])) if causal else 0
        xs = f32(rng.normal(0, 2.0, (rows, cols)))
        ys_ref = softmax_ref(xs, scale, causal, offset, group or None)
        XS, YS = to_dev(xs), device.Buffer((rows, cols))
        call("lhip_softmax_fwd", XS.ptr, YS.ptr, rows, cols, scale, causal, offset, group)
        ys = dl(YS)
        assert rel_fro(ys, ys_ref) <= EW, ("softmax", rows, cols, causal, offset, group)
        dxs_ref = softmax_bwd_ref(ys_ref, g, scale, causal, offset, group or None)
        DXS = device.Buffer((rows, cols))
        call("lhip_softmax_bwd", YS.ptr, G.ptr, DXS.ptr, rows, cols, scale, causal, offset, group, 0)
        assert rel_fro(dl(DXS), dxs_ref) <= EW, ("softmax bwd", rows, cols, causal, offset, group)
        gate = f32(rng.standard_normal((rows, cols)) * 3)
        GT, UP, H = to_dev(gate), to_dev(x), device.Buffer((rows, cols))
        call("lhip_swiglu_fwd", GT.ptr, cols, UP.ptr, cols, H.ptr, cols, rows, cols)
        assert rel_fro(dl(H), O.swiglu_fwd(gate, x)) <= EW, ("swiglu", rows, cols)
        dg_ref, du_ref = O.swiglu_bwd(gate, x, g)
        DG, DU = device.Buffer((rows, cols)), device.Buffer((rows, cols))
        call("lhip_swiglu_bwd", GT.ptr, cols, UP.ptr, cols, G.ptr, cols, DG.ptr, cols, DU.ptr, cols, rows, cols, 0)
        assert rel_fro(dl(DG), dg_ref) <= EW and rel_fro(dl(DU), du_ref) <= EW, ("swiglu bwd", rows, cols)


@pytest.mark.parametrize("rows,cols", [(64, 256), (4096, 4096), (17, 33), (3, 20), (7, 1028)])
def test_swiglu_fwd_bwd(rows, cols):
    announce("swiglu", rows, cols)
    rng = np.random.default_rng(rows * 3 + cols)
    gate = f32(rng.standard_normal((rows, cols)) * 3)
    up = f32(rng.standard_normal((rows, cols)))
    dh = f32(rng.standard_normal((rows, cols)))
    GT, UP, H = to_dev(gate), to_dev(up), device.Buffer((rows, cols))
    call("lhip_swiglu_fwd", GT.ptr, cols, UP.ptr, cols, H.ptr, cols, rows, cols)
    assert rel_fro(dl(H), O.swiglu_fwd(gate, up)) <= EW
    dg_ref, du_ref = O.swiglu_bwd(gate, up, dh)
    DH, DG, DU = to_dev(dh), device.Buffer((rows, cols)), device.Buffer((rows, cols))
    call("lhip_swiglu_bwd", GT.ptr, cols, UP.ptr, cols, DH.ptr, cols, DG.ptr, cols, DU.ptr, cols, rows, cols, 0)
    assert rel_fro(dl(DG), dg_ref) <= EW
    assert rel_fro(dl(DU), du_ref) <= EW
    # accumulate: a second call adds the same gradients
    call("lhip_swiglu_bwd", GT.ptr, cols, UP.ptr, cols, DH.ptr, cols, DG.ptr, cols, DU.ptr, cols, rows, cols, 1)
    assert rel_fro(dl(DG), 2 * dg_ref) <= EW
    assert rel_fro(dl(DU), 2 * du_ref) <= EW


def test_swiglu_strided_fused_w13_layout():
    """gate and up as the two halves of one [rows, 2F] buffer (a fused W1|W3 GEMM output)."""
    rng = np.random.default_rng(5)
    rows, F = 64, 256
    z = f32(rng.standard_normal((rows, 2 * F)))
    Z, H = to_dev(z), device.Buffer((rows, F))
    call("lhip_swiglu_fwd", Z.ptr, 2 * F, Z.offset(F), 2 * F, H.ptr, F, rows, F)
    assert rel_fro(dl(H), O.swiglu_fwd(z[:, :F], z[:, F:])) <= EW


def test_swiglu_closed_form_known_values():
    """tests/test.lua:245-275: silu(0)*u = 0; silu(a)*b at a few points."""
    a = np.array([[0.0, 1.0, -1.0, 20.0, -20.0, 0.5, -0.5, 3.0]])
    b = np.array([[5.0, 2.0, 2.0, 1.0, 1.0, -1.0, 4.0, 0.25]])
    A, B, H = to_dev(a), to_dev(b), device.Buffer((1, 8))
    call("lhip_swiglu_fwd", A.ptr, 8, B.ptr, 8, H.ptr, 8, 1, 8)
    expect = a / (1 + np.exp(-a)) * b
    np.testing.assert_allclose(dl(H), expect, rtol=1e-6, atol=1e-12)


# ------------------------------------------------------------------ RoPE
# access modes: interleaved float4 (hd % 4 == 0), half-split 2 x float4
# (hd % 8 == 0), half-split 2 x float2 (hd 12), scalar (odd pair counts)
@pytest.mark.parametrize("rows,heads,hd,interleaved", [(4096, 16, 64, 1), (4096, 16, 64, 0), (64, 8, 16, 1),
                                                       (50, 3, 6, 1), (50, 3, 6, 0), (10, 2, 10, 0),
                                                       (33, 5, 12, 0), (33, 5, 12, 1), (9, 3, 256, 0)])
def test_rope_vs_oracle_heads(rows, heads, hd, interleaved):
    announce("rope", rows, heads, hd, interleaved)
    rng = np.random.default_rng(rows + hd)
    x = f32(rng.standard_normal((rows, heads * hd)))
    for inverse in (0, 1):
        ref = O.rope_heads(x, heads, hd, interleaved=bool(interleaved), inverse=bool(inverse))
        X = to_dev(x)
        call("lhip_rope", X.ptr, None, rows, heads, hd, heads * hd, 0, 0, 10000.0, interleaved, inverse)
        assert rel_fro(dl(X), ref) <= EW


def test_rope_matches_cpu_path_tables_and_period():
    """CPU-path RoPE (per head slice, interleaved pairs, angle tables of
    transformer.lua:30-48) over B windows of T rows: pos = r % T."""
    rng = np.random.default_rng(8)
    B, T, H, hd = 3, 64, 8, 16
    x = f32(rng.standard_normal((B * T, H * hd)))
    cosr, sinr = O.rope_angles(10000.0, hd, T - 1)
    ref = np.zeros_like(x)
    for b in range(B):
        for h in range(H):
            ref[b * T:(b + 1) * T, h * hd:(h + 1) * hd] = O.rope_fwd(x[b * T:(b + 1) * T, h * hd:(h + 1) * hd], cosr, sinr)
    X = to_dev(x)
    call("lhip_rope", X.ptr, None, B * T, H, hd, H * hd, 0, T, 10000.0, 1, 0)
    assert rel_fro(dl(X), ref) <= EW
    # backward = BACKWARD.rope (tensor2.lua:451-473) on an upstream gradient
    g = f32(rng.standard_normal((B * T, H * hd)))
    bref = np.zeros_like(g)
    for b in range(B):
        for h in range(H):
            bref[b * T:(b + 1) * T, h * hd:(h + 1) * hd] = O.rope_bwd(g[b * T:(b + 1) * T, h * hd:(h + 1) * hd], cosr, sinr)
    G = to_dev(g)
    call("lhip_rope", G.ptr, None, B * T, H, hd, H * hd, 0, T, 10000.0, 1, 1)
    assert rel_fro(dl(G), bref) <= EW


def test_rope_identity_at_pos0_and_round_trip_and_pos_ids():
    rng = np.random.default_rng(9)
    x = f32(rng.standard_normal((32, 4 * 64)))
    # tests/core_test.lua:88-92: position 0 is the identity (pos_ids all 0)
    X = to_dev(x)
    Z0 = to_dev(np.zeros(32, np.int32), np.int32)      # keep the buffer alive across the call
    call("lhip_rope", X.ptr, Z0.ptr, 32, 4, 64, 256, 0, 0, 10000.0, 1, 0)
    assert np.array_equal(dl(X), x)
    # tests/test.lua:277-289: forward then inverse is the identity
    X = to_dev(x)
    for inv in (0, 1):
        call("lhip_rope", X.ptr, None, 32, 4, 64, 256, 100, 0, 10000.0, 0, inv)
    assert rel_fro(dl(X), x) <= 1e-6
    # explicit pos_ids equal the pos_offset form; norm of each pair preserved
    ids = (np.arange(32) + 7).astype(np.int32)
    A, Bf = to_dev(x), to_dev(x)
    IDS = to_dev(ids, np.int32)
    call("lhip_rope", A.ptr, IDS.ptr, 32, 4, 64, 256, 0, 0, 10000.0, 1, 0)
    call("lhip_rope", Bf.ptr, None, 32, 4, 64, 256, 7, 0, 10000.0, 1, 0)
    a = dl(A)
    assert np.array_equal(a, dl(Bf))
    pn = lambda v: np.hypot(v[:, 0::2], v[:, 1::2])  # noqa: E731
    np.testing.assert_allclose(pn(a), pn(x), rtol=1e-5)


def test_rope_rejects_odd_head_dim():
    X = device.Buffer((4, 6))
    with pytest.raises(LanternlHipError, match="even"):
        call("lhip_rope", X.ptr, None, 4, 2, 3, 6, 0, 0, 10000.0, 1, 0)


# ------------------------------------------------------------------ fused CE
@pytest.mark.parametrize("rows,V,gs", [(512, 32000, 1 / 512), (64, 2000, 1 / 64), (8, 1000, 1.0),
                                       (6, 9000, 0.5), (4, 33000, 1.0), (5, 37, 1.0)])
def test_ce_fused_vs_oracle(rows, V, gs):
    announce("ce", rows, V)
    rng = np.random.default_rng(rows + V)
    x = f32(rng.standard_normal((rows, V)) * 2)
    t = rng.integers(0, V, rows).astype(np.int32)
    t[1] = -1                      # ignored (t < 0)
    t[2] = V                       # ignored (t >= V)
    loss_ref, d_ref = O.ce_fused(x, t, ignore_index=-100, gscale=gs)
    X, T, L, D = to_dev(x), to_dev(t, np.int32), device.Buffer((rows,)), device.Buffer((rows, V))
    call("lhip_ce_fused", X.ptr, T.ptr, L.ptr, D.ptr, rows, V, -100, gs)
    loss = dl(L)
    assert np.max(np.abs(loss - loss_ref)) <= 1e-5
    assert loss[1] == 0 and loss[2] == 0
    d = dl(D)
    assert rel_fro(d, d_ref) <= EW
    assert not d[1].any() and not d[2].any()
    # tests/test.lua:347-355: each dlogits row sums to 0
    np.testing.assert_allclose(d.sum(axis=1), 0.0, atol=1e-5 * max(1.0, gs * 10))
    # in place: dlogits aliasing logits
    call("lhip_ce_fused", X.ptr, T.ptr, L.ptr, X.ptr, rows, V, -100, gs)
    assert rel_fro(dl(X), d_ref) <= EW


def test_ce_known_answer_and_uniform_logits():
    """tests/core_test.lua:54-57: CE([2,1,0.1], target 1 (Lua) = 0) = 0.41703;
    near-uniform logits give ln V (ln 2000, ln 32000)."""
    X = to_dev(np.array([[2.0, 1.0, 0.1]]))
    T, L = to_dev(np.array([0], np.int32), np.int32), device.Buffer((1,))
    call("lhip_ce_fused", X.ptr, T.ptr, L.ptr, None, 1, 3, -100, 1.0)
    expect = np.log(np.exp(2) + np.exp(1) + np.exp(0.1)) - 2
    assert abs(dl(L)[0] - expect) <= 1e-6 and abs(expect - 0.41703) < 1e-5
    for V in (2000, 32000):
        X = to_dev(np.zeros((4, V)))
        T, L = to_dev(np.arange(4, dtype=np.int32), np.int32), device.Buffer((4,))
        call("lhip_ce_fused", X.ptr, T.ptr, L.ptr, None, 4, V, -100, 1.0)
        np.testing.assert_allclose(dl(L), np.log(V), atol=1e-5)


# ------------------------------------------------------------------ argmax
def test_argmax_known_answer_and_edge_cases_bit_exact():
    # tests/test.lua:375-379
    X, OUT = to_dev(np.array([[1, 9, 2], [8, 3, 4]], np.float64)), device.Buffer((2,), np.int32)
    call("lhip_argmax_rows", X.ptr, OUT.ptr, 2, 3)
    device.sync()
    assert OUT.download().tolist() == [1, 0]
    rng = np.random.default_rng(3)
    for rows, cols in ((512, 2000), (512, 32000), (33, 7), (4, 1)):
        x = f32(rng.integers(-3, 4, (rows, cols)).astype(np.float64))   # many ties
        x[0, :] = -np.inf
        x[min(1, rows - 1), ::3] = np.nan
        if rows > 2:
            x[2, :] = np.nan
        X, OUT = to_dev(x), device.Buffer((rows,), np.int32)
        call("lhip_argmax_rows", X.ptr, OUT.ptr, rows, cols)
        device.sync()
        assert np.array_equal(OUT.download(), O.argmax_rows(x)), (rows, cols)


# ------------------------------------------------------------------ embedding
def test_embed_gather_exact_and_scatter_known_answer():
    rng = np.random.default_rng(4)
    V, D = 8, 4
    tab = f32(rng.standard_normal((V, D)))
    ids = np.array([3, 0, 7, 3, 1], np.int32)
    TB, IDS, OUT = to_dev(tab), to_dev(ids, np.int32), device.Buffer((5, D))
    call("lhip_embed_fwd", TB.ptr, IDS.ptr, OUT.ptr, 5, D, V)
    assert np.array_equal(dl(OUT), O.embed_fwd(tab, ids))
    # tests/test.lua:291-320: scatter of ones -> row3 = 2, row0 = 1, row2 = 0
    G, DT = to_dev(np.ones((5, D))), device.Buffer((V, D))
    call("lhip_embed_bwd", G.ptr, IDS.ptr, DT.ptr, 5, D, V, 1.0, 0)
    dt = dl(DT)
    assert dt[3].tolist() == [2] * D and dt[0].tolist() == [1] * D and dt[2].tolist() == [0] * D


@pytest.mark.parametrize("n,V,D", [(512, 2000, 128), (100, 50, 600), (64, 10, 3)])
def test_embed_fwd_bwd_vs_oracle(n, V, D):
    announce("embed", n, V, D)
    rng = np.random.default_rng(n + V + D)
    tab = f32(rng.standard_normal((V, D)))
    ids = rng.integers(0, V, n).astype(np.int32)
    g = f32(rng.standard_normal((n, D)))
    TB, IDS, OUT = to_dev(tab), to_dev(ids, np.int32), device.Buffer((n, D))
    call("lhip_embed_fwd", TB.ptr, IDS.ptr, OUT.ptr, n, D, V)
    assert np.array_equal(dl(OUT), O.embed_fwd(tab, ids))
    base = f32(rng.standard_normal((V, D)))
    ref = base + O.embed_bwd(g, ids, V, 0.5)
    G, DT = to_dev(g), to_dev(base)
    call("lhip_embed_bwd", G.ptr, IDS.ptr, DT.ptr, n, D, V, 0.5, 1)
    assert rel_fro(dl(DT), ref) <= EW


def test_embed_out_of_range_ids_give_zero_rows():
    tab = np.arange(12, dtype=np.float64).reshape(3, 4)
    ids = np.array([0, -1, 3, 2], np.int32)
    OUT = device.Buffer((4, 4))
    TB, IDS = to_dev(tab), to_dev(ids, np.int32)
    call("lhip_embed_fwd", TB.ptr, IDS.ptr, OUT.ptr, 4, 4, 3)
    out = dl(OUT)
    assert np.array_equal(out[0], tab[0]) and not out[1].any() and not out[2].any() and np.array_equal(out[3], tab[2])


# ------------------------------------------------------------------ optimizer
@pytest.mark.parametrize("clip,B,nan,mom,nest", [(1.0, 8, False, 0.9, 0), (1e6, 1, False, 0.9, 0),
                                                  (1.0, 4, True, 0.9, 0), (1.0, 8, False, 0.9, 1),
                                                  (1e6, 2, False, 0.0, 0)])
def test_sumsq_and_sgd_step_vs_oracle(clip, B, nan, mom, nest):
    """lhip_sgd_step: LMTrain's step logic around optim2.SGD (lmtrain.lua:1212-1226,
    optim2.lua:72-99), with momentum (plain and Nesterov) and without."""
    rng = np.random.default_rng(17)
    n = 912_512
    p = f32(rng.standard_normal(n) * 0.02)
    g = f32(rng.standard_normal(n) * 0.01)
    v = f32(rng.standard_normal(n) * 0.001)
    if nan:
        g[123] = np.nan
    P, G, Vb = to_dev(p), to_dev(g), to_dev(v)
    SS = device.Buffer((2,))          # 8 bytes: one device double
    NORM, APP = device.Buffer((1,)), device.Buffer((1,), np.int32)
    call("lhip_sumsq", G.ptr, n, SS.ptr)
    device.sync()
    ss = SS.download().view(np.float64)[0]
    if not nan:
        assert abs(ss - float(np.sum(g * g))) <= 1e-9 * ss
    lr, wd = 0.05, 0.01
    call("lhip_sgd_step", P.ptr, G.ptr, Vb.ptr, n, SS.ptr, lr, mom, wd, 1.0 / B, clip, nest, NORM.ptr, APP.ptr)
    device.sync()
    # oracle: scale_grads(1/B) (only when B > 1), norm, skip if non-finite, clip, SGD
    gg = g / B if B > 1 else g.copy()
    norm = O.grad_norm(gg)
    applied = bool(np.isfinite(norm))
    assert APP.download()[0] == int(applied)
    pr, vr = p.copy(), v.copy()
    if applied:
        if norm > clip:
            gg = gg * (clip / norm)
        O.sgd_step(pr, gg, vr, lr, mom, wd, nesterov=bool(nest))
        assert abs(NORM.download()[0] - norm) <= 1e-6 * norm
        assert rel_fro(dl(G), gg) <= EW
    assert rel_fro(dl(P), pr) <= EW and rel_fro(dl(Vb), vr) <= EW
    if not applied:
        assert np.array_equal(dl(P), p) and np.array_equal(dl(Vb), v)


@pytest.mark.parametrize("clip,B,nan,step", [(1.0, 8, False, 1), (1e6, 1, False, 5), (1.0, 4, True, 2)])
def test_adamw_step_vs_oracle(clip, B, nan, step):
    """lhip_adamw_step: the LMTrain step logic around optim2.AdamW.step at step count `step`."""
    rng = np.random.default_rng(18)
    n = 912_512
    p = f32(rng.standard_normal(n) * 0.02)
    g = f32(rng.standard_normal(n) * 0.01)
    m = f32(rng.standard_normal(n) * 0.001)
    v = f32(np.abs(rng.standard_normal(n)) * 1e-5)
    if nan:
        g[77] = np.inf
    P, G, M, Vb = to_dev(p), to_dev(g), to_dev(m), to_dev(v)
    SS = device.Buffer((2,))
    NORM, APP = device.Buffer((1,)), device.Buffer((1,), np.int32)
    call("lhip_sumsq", G.ptr, n, SS.ptr)
    lr, b1, b2, eps, wd = 1e-3, 0.9, 0.95, 1e-8, 0.01
    call("lhip_adamw_step", P.ptr, G.ptr, M.ptr, Vb.ptr, n, SS.ptr, lr, b1, b2, eps, wd, 1.0 / B, clip, step,
         NORM.ptr, APP.ptr)
    device.sync()
    gg = g / B if B > 1 else g.copy()
    norm = O.grad_norm(gg)
    applied = bool(np.isfinite(norm))
    assert APP.download()[0] == int(applied)
    if not applied:
        assert np.array_equal(dl(P), p) and np.array_equal(dl(M), m) and np.array_equal(dl(Vb), v)
        return
    if norm > clip:
        gg = gg * (clip / norm)
    pr, mr, vr = p.copy(), m.copy(), v.copy()
    O.adamw_step(pr, gg, mr, vr, step, lr, b1, b2, eps, wd)
    assert abs(NORM.download()[0] - norm) <= 1e-6 * norm
    assert rel_fro(dl(G), gg) <= EW
    assert rel_fro(dl(M), mr) <= EW and rel_fro(dl(Vb), vr) <= EW
    assert rel_fro(dl(P) - p, pr - p) <= 1e-4


def test_sum_and_fill_and_add():
    x = np.arange(1, 1001, dtype=np.float64)
    X, OUT = to_dev(x), device.Buffer((1,))
    call("lhip_sum", X.ptr, 1000, 0.5, OUT.ptr)
    assert dl(OUT)[0] == 250250.0
    call("lhip_fill", X.ptr, 999, 3.0)
    y = dl(X)
    assert (y[:999] == 3).all() and y[999] == 1000
    A, Bb, C = to_dev(np.ones(10)), to_dev(np.arange(10.0)), device.Buffer((10,))
    call("lhip_add", A.ptr, Bb.ptr, C.ptr, 10)
    assert dl(C).tolist() == list(np.arange(10.0) + 1)
    # lhip_zero on an odd byte count goes through the byte-fill kernel
    Z = to_dev(np.ones(10))
    call("lhip_zero", Z.ptr + 4, 7)
    z = Z.download().view(np.uint8)
    assert (z[4:11] == 0).all() and z[11] != 0


# ------------------------------------------------------------ silu, memory queries
@pytest.mark.parametrize("n", [1, 7, 4096, 1_000_003])
def test_silu_vs_closed_form_in_place_and_out(n):
    """lhip_silu (the adapter's silu_inplace): x * sigmoid(x) with the sigmoid by
    sign (tensor2.lua:272-291), against the float64 closed form, including large
    |x|; in place and out of place, on an unaligned view."""
    announce("silu", n)
    rng = np.random.default_rng(n)
    x = f32(rng.normal(0, 4, n))
    # large |x| (exp(80) overflows the naive sigmoid's intermediate in fp32 only
    # at ~89, but the sign form never forms it); silu(-80) ~ -1.4e-33 stays a
    # normal fp32 number, so the relative bar applies
    x[: min(n, 3)] = np.array([-80.0, 80.0, 0.0], np.float32)[: min(n, 3)]
    xd = x.astype(np.float64)
    ref = xd / (1.0 + np.exp(-np.clip(xd, -700, 700)))
    X, Y = to_dev(x), device.Buffer((n,))
    call("lhip_silu", X.ptr, Y.ptr, n)
    assert rel_fro(dl(Y), ref) <= EW
    call("lhip_silu", X.ptr, X.ptr, n)                       # in place
    assert rel_fro(dl(X), ref) <= EW
    if n > 1:                                                # unaligned view: scalar path
        Z = to_dev(x)
        call("lhip_silu", Z.offset(1), Z.offset(1), n - 1)
        got = dl(Z)
        assert got[0] == x[0]
        assert rel_fro(got[1:], ref[1:]) <= EW


def test_mem_info_and_allocation_accounting():
    """lhip_mem_info (luaTL_mem_info) and lhip_mem_stats (the adapter's stats())."""
    import ctypes
    from lanternl_amd._lib import MemStats, lib
    announce("mem info / stats")
    L = lib()
    free_b, total_b = ctypes.c_ulonglong(), ctypes.c_ulonglong()
    call("lhip_mem_info", ctypes.byref(free_b), ctypes.byref(total_b))
    assert 0 < free_b.value <= total_b.value
    assert abs(total_b.value - device.info()["total_mem"]) <= 0.01 * device.info()["total_mem"]
    before = MemStats()
    call("lhip_mem_stats", ctypes.byref(before))
    p = ctypes.c_void_p()
    call("lhip_malloc", ctypes.byref(p), 3 << 20)
    mid = MemStats()
    call("lhip_mem_stats", ctypes.byref(mid))
    assert mid.bytes_in_use == before.bytes_in_use + (3 << 20)
    assert mid.live_buffers == before.live_buffers + 1
    assert mid.n_alloc == before.n_alloc + 1
    assert mid.peak_in_use >= mid.bytes_in_use
    assert L.lhip_free(p) == 0
    after = MemStats()
    call("lhip_mem_stats", ctypes.byref(after))
    assert after.bytes_in_use == before.bytes_in_use
    assert after.live_buffers == before.live_buffers
    assert after.n_free == before.n_free + 1
    assert after.peak_in_use >= mid.bytes_in_use
