"""GPU tests of the reference adapter's surface as this backend serves it
(lanternl_amd/backend.py, the Python mirror of lanternl_amd/lua/luatl_adapter.lua),
through the C ABI: the reference adapter test (tests/test.lua:436-475)
replayed, every legacy and resident call against the oracle's restatement of
the luaTL kernel it stands for, and luaTL.Program's op list run, captured and
replayed.

Bars: GEMM results relative Frobenius <= 1e-4; row and elementwise results
<= 1e-5; argmax and gathers bit-exact; a captured replay bit-identical to the
eager run of the same ops.
"""
import numpy as np
import pytest

import oracle as O
from lanternl_amd import backend as ad
from lanternl_amd import device
from tests.gpu_util import announce, f32, rel_fro

pytestmark = pytest.mark.gpu
GEMM, ROW = 1e-4, 1e-5


@pytest.fixture(scope="module", autouse=True)
def _dev():
    device.init(0)
    assert ad.available, ad.reason
    yield


def close(a, b, tol):
    return all(abs(x - y) <= tol for x, y in zip(a, b)) and len(a) == len(b)


def pin(a):
    a = np.asarray(a, np.float32)
    r, c = (a.shape if a.ndim == 2 else (a.size, 1))
    return ad.pin(a.ravel().tolist(), r, c)


def dl(h):
    device.sync()
    t = h.t if ad.is_handle(h) else h
    out = np.empty(t.rows * t.cols, np.float32)
    ad.download_f32(t, out, out.size)
    return out.reshape(t.rows, t.cols).astype(np.float64)


# ----------------------------------------------------------- tests/test.lua:436-475
def test_reference_adapter_test_replayed():
    announce("adapter", "tests/test.lua:436-475")
    assert ad.available and ad.error is None and isinstance(ad.device, str)
    a = [1, 2, 3, 4, 5, 6]               # 2x3
    b = [1, 0, 0, 1, 1, 1]               # 3x2
    c = ad.matmul(a, 2, 3, b, 2)
    assert close(c, [4, 5, 10, 11], 1e-4) and isinstance(c, list) and c[0] is not None
    hA, hB = ad.pin(a, 2, 3), ad.pin(b, 3, 2)
    hC = ad.matmul(hA, 2, 3, hB, 2)
    assert ad.is_handle(hC)
    assert close(hC.toflat(), c, 1e-4)
    hdY = ad.pin([1, 1, 1, 1], 2, 2)
    hdX = ad.alloc(2, 3)
    ad.gemm_dx(hdY, hB, hdX)             # dX = dY @ B^T -> 2x3
    assert len(hdX.toflat()) == 6
    assert close(hdX.toflat(), (np.ones((2, 2)) @ np.array(b, float).reshape(3, 2).T).ravel(), 1e-5)
    hdW = ad.alloc(3, 2)
    ad.gemm_dw(hA, hdY, hdW, 0.0)        # dW = A^T @ dY -> 3x2
    assert len(hdW.toflat()) == 6
    assert close(hdW.toflat(), (np.array(a, float).reshape(2, 3).T @ np.ones((2, 2))).ravel(), 1e-5)
    sm = ad.softmax_causal([1, 2, 3, 4], 2, 2, 1.0)
    assert abs(sm[1]) < 1e-6 and abs(sm[0] - 1.0) < 1e-6
    # a handle with a flat table: the result is flat (resident only when both are)
    mixed = ad.matmul(hA, 2, 3, b, 2)
    assert isinstance(mixed, list) and close(mixed, c, 1e-4)
    for h in (hA, hB, hC, hdY, hdX, hdW):
        h.free()


def test_pin_rejects_a_wrong_element_count():
    """luatl_adapter.lua:63-67: pin takes exactly rows*cols numbers; short and
    long tables are both refused, and so is a short operand of a flat call."""
    with pytest.raises(ValueError, match="takes exactly 4 numbers, the table holds 3"):
        ad.pin([1, 2, 3], 2, 2)
    with pytest.raises(ValueError, match="takes exactly 4 numbers, the table holds 5"):
        ad.pin([1, 2, 3, 4, 5], 2, 2)
    with pytest.raises(ValueError, match="needs 6 numbers, the table holds 4"):
        ad.matmul([1, 2, 3, 4], 2, 3, [1, 0, 0, 1, 1, 1], 2)
    with pytest.raises(ValueError, match="matmul dimensions must be non-negative integers, got 2.5 x 3 x 2"):
        ad.matmul([1.0] * 6, 2.5, 3, [1.0] * 6, 2)
    rd = [0.0] * 6
    with pytest.raises(ValueError, match="matmul_tn dimensions must be non-negative integers, got 2 x 3 x -2"):
        ad.matmul_into("tn", [1.0] * 6, 2, 3, [1.0] * 6, -2, rd, True)
    assert rd == [0.0] * 6
    h = ad.pin([1.0, 2.0, 3.0, 4.0], 2, 2)
    with pytest.raises(ValueError, match="needs 4 numbers"):
        h.upload([1.0])
    h.free()


# ----------------------------------------------------------- legacy flat calls
def test_legacy_rmsnorm_and_softmax_vs_oracle():
    announce("adapter", "legacy rmsnorm/softmax")
    rng = np.random.default_rng(31)
    rows, cols = 24, 40
    x = f32(rng.standard_normal((rows, cols)))
    w = f32(rng.normal(1, 0.1, cols))
    y = np.array(ad.rmsnorm(x.ravel().tolist(), rows, cols, w.ravel().tolist(), 1e-6)).reshape(rows, cols)
    assert rel_fro(y, O.rmsnorm_fwd(x, w, 1e-6)[0]) <= ROW
    y1 = np.array(ad.rmsnorm(x.ravel().tolist(), rows, cols)).reshape(rows, cols)   # no gain, eps 1e-5
    assert rel_fro(y1, O.rmsnorm_fwd(x, np.ones(cols), 1e-5)[0]) <= ROW
    hx = pin(x)
    hy = ad.rmsnorm(hx, rows, cols, pin(w), 1e-6)                                   # resident in, resident out
    assert ad.is_handle(hy) and rel_fro(dl(hy), O.rmsnorm_fwd(x, w, 1e-6)[0]) <= ROW
    s = np.array(ad.softmax(x.ravel().tolist(), rows, cols)).reshape(rows, cols)
    assert rel_fro(s, O.softmax_ex(x)) <= ROW
    sc = np.array(ad.softmax_causal(x.ravel().tolist(), rows, cols, 0.25, 8)).reshape(rows, cols)
    assert rel_fro(sc, O.softmax_ex(x, None, 0.25, True, 8, 0)) <= ROW


# ----------------------------------------------------------- resident calls
def _gemm_case(rng, M, N, K, strides, batch=1, **kw):
    a_rs, a_cs, b_rs, b_cs, c_rs, c_cs, a_bs, b_bs, c_bs = strides
    na = (M - 1) * a_rs + (K - 1) * a_cs + (batch - 1) * a_bs + 1
    nb = (K - 1) * b_rs + (N - 1) * b_cs + (batch - 1) * b_bs + 1
    nc = (M - 1) * c_rs + (N - 1) * c_cs + (batch - 1) * c_bs + 1
    A = f32(rng.standard_normal(na)); B = f32(rng.standard_normal(nb)); C0 = f32(rng.standard_normal(nc))
    extras = {k: f32(rng.normal(1 if k == "gamma" else 0, 0.3, N if k == "bias" else (K if k == "gamma" else M)))
              for k in ("bias", "gamma", "rowscale") if kw.pop(k, False)}
    ref = C0.copy()
    O.gemm_ex(A, B, ref, M, N, K, strides, batch=batch, bias=extras.get("bias"), gamma=extras.get("gamma"),
              rowscale=extras.get("rowscale"), **kw)
    hA, hB, hC = pin(A.reshape(-1, 1)), pin(B.reshape(-1, 1)), pin(C0.reshape(-1, 1))
    o = {"batch": batch, **{k: v for k, v in kw.items()}}
    if "pre" in kw:
        o["pre"] = kw["pre"]
    if "act" in kw:
        o["act"] = kw["act"]
    for k, v in extras.items():
        o[k] = pin(v.reshape(-1, 1))
    av = ad.view(hA, M, K, a_rs, a_cs, a_bs)
    bv = ad.view(hB, K, N, b_rs, b_cs, b_bs)
    cv = ad.view(hC, M, N, c_rs, c_cs, c_bs)
    ad.gemm_ex(av, bv, cv, o)
    got = dl(hC).ravel()
    # compare only the addressed elements of C
    idx = np.array([z * c_bs + i * c_rs + j * c_cs for z in range(batch) for i in range(M) for j in range(N)])
    return got[idx], ref[idx]


@pytest.mark.parametrize("case", ["plain", "alpha_beta_cm", "bias_gelu", "pre_rmsnorm", "pre_rowscale",
                                  "pre_silu", "heads_batched", "big_split"])
def test_gemm_ex_vs_oracle(case):
    announce("adapter gemm_ex", case)
    rng = np.random.default_rng(sum(map(ord, case)))
    M, N, K = 37, 29, 45
    rm = (K, 1, N, 1, N, 1, 0, 0, 0)
    if case == "plain":
        got, ref = _gemm_case(rng, M, N, K, rm)
    elif case == "alpha_beta_cm":       # A transposed, C column-major
        got, ref = _gemm_case(rng, M, N, K, (1, M, N, 1, 1, M, 0, 0, 0), alpha=0.5, beta=-2.0)
    elif case == "bias_gelu":
        got, ref = _gemm_case(rng, M, N, K, rm, alpha=1.5, beta=0.5, act=2, bias=True)
    elif case == "pre_rmsnorm":
        got, ref = _gemm_case(rng, M, N, K, rm, pre=1, eps=1e-6, gamma=True)
    elif case == "pre_rowscale":
        got, ref = _gemm_case(rng, M, N, K, rm, pre=1, rowscale=True, act=3)
    elif case == "pre_silu":
        got, ref = _gemm_case(rng, M, N, K, (1, M, 1, K, N, 1, 0, 0, 0), pre=3)   # A^T, B^T views
    elif case == "heads_batched":       # per-head Q.K^T of a [T, H*hd] activation
        T, H, hd = 64, 8, 16
        got, ref = _gemm_case(rng, T, T, hd, (H * hd, 1, 1, H * hd, T, 1, hd, hd, T * T), batch=H, alpha=0.25)
    else:                               # K long enough to split
        got, ref = _gemm_case(rng, 64, 48, 6000, (6000, 1, 48, 1, 48, 1, 0, 0, 0), beta=1.0)
    assert rel_fro(got, ref) <= GEMM


def test_gemm_ex_rejects_general_strides():
    from lanternl_amd._lib import LanternlHipError
    h = ad.alloc(64, 1)
    with pytest.raises(LanternlHipError, match="UNSUPPORTED"):
        ad.gemm_ex(ad.view(h, 4, 4, 8, 2), ad.view(h, 4, 4, 4, 1), ad.view(h, 4, 4, 4, 1))


def test_resident_row_ops_vs_oracle():
    announce("adapter", "resident rmsnorm_bwd/softmax_bwd/swiglu/rope")
    rng = np.random.default_rng(32)
    rows, cols = 48, 64
    x = f32(rng.standard_normal((rows, cols))); g = f32(rng.normal(1, 0.1, cols))
    dy = f32(rng.standard_normal((rows, cols)))
    hx, hg, hdy = pin(x), pin(g.reshape(1, -1)), pin(dy)
    hdx = ad.alloc(rows, cols)
    dg0 = f32(rng.standard_normal(cols))
    hdg = pin(dg0.reshape(1, -1))
    ad.rmsnorm_bwd(hx, hg, hdy, hdx, hdg, 1e-6)
    dg_ref = dg0.copy()
    dx_ref = O.rmsnorm_bwd_luatl(x, g, dy, 1e-6, dg_ref)
    assert rel_fro(dl(hdx), dx_ref) <= ROW and rel_fro(dl(hdg).ravel(), dg_ref) <= ROW
    ad.rmsnorm_bwd(hx, None, hdy, hdx, None)                  # gain-free, eps 1e-5
    assert rel_fro(dl(hdx), O.rmsnorm_bwd_luatl(x, None, dy, 1e-5)) <= ROW
    # softmax backward, including an offset that masks whole rows
    for o in ({}, {"scale": 0.5, "causal": True, "group": 16}, {"causal": True, "mask_offset": -3}):
        y = O.softmax_ex(x, None, o.get("scale", 1.0), o.get("causal", False), o.get("group", 0),
                         o.get("mask_offset", 0))
        hy = pin(y)
        ad.softmax_bwd(hy, hdy, hdx, o)
        ref = O.softmax_bwd_ex(f32(y), dy, o.get("scale", 1.0), o.get("causal", False), o.get("group", 0),
                               o.get("mask_offset", 0))
        assert rel_fro(dl(hdx), ref) <= ROW, o
    # swiglu on the packed [rows, 2*F] layout (a = base, b = base + F, lda = ldb = 2F)
    F = 32
    packed = f32(rng.standard_normal((rows, 2 * F)))
    hp = pin(packed)
    ho = ad.alloc(rows, F)
    hb = ad.wrap(ad.offset(hp, F), rows, F)
    ad.swiglu(hp, ad.new_handle(hb, rows, F), ho, {"lda": 2 * F, "ldb": 2 * F})
    gate, up = packed[:, :F], packed[:, F:]
    assert rel_fro(dl(ho), O.swiglu_fwd(gate, up)) <= ROW
    # rope, half-split (the reference default) and interleaved, with heads
    H, hd = 4, 16
    q = f32(rng.standard_normal((rows, H * hd)))
    for o in ({"heads": H}, {"heads": H, "interleaved": True, "pos_offset": 5, "theta": 500.0},
              {"heads": H, "inverse": True}):
        hq = pin(q)
        ad.rope(hq, o)
        ref = O.rope_heads(q, H, hd, H * hd, o.get("pos_offset", 0), o.get("theta", 10000.0),
                           o.get("interleaved", False), o.get("inverse", False))
        assert rel_fro(dl(hq), ref) <= ROW, o


def test_inplace_elementwise_calls():
    announce("adapter", "add/scale/silu/gelu inplace")
    rng = np.random.default_rng(33)
    a = f32(rng.standard_normal((16, 20))); b = f32(rng.standard_normal((16, 20)))
    ha, hb = pin(a), pin(b)
    ad.add_inplace(ha, hb, 0.5)          # AXPY with a = dst: dst = 0.5*dst + src
    assert rel_fro(dl(ha), 0.5 * a + b) <= ROW
    ha.upload(a.ravel())
    ad.add_inplace(ha, hb)               # alpha 1: dst + src
    assert rel_fro(dl(ha), a + b) <= ROW
    ha.upload(a.ravel())
    ad.scale_inplace(ha, -3.0)
    assert rel_fro(dl(ha), -3.0 * a) <= ROW
    ha.upload(a.ravel())
    ad.silu_inplace(ha)
    assert rel_fro(dl(ha), O.ew("SILU", a, None)) <= ROW
    ha.upload(a.ravel())
    ad.gelu_inplace(ha)
    assert rel_fro(dl(ha), O.ew("GELU", a, None)) <= ROW


@pytest.mark.parametrize("op", list(O.EW))
def test_elementwise_operator_table(op):
    rng = np.random.default_rng(40 + O.EW[op])
    n = 4099                                     # a float4 body and a scalar tail
    a = f32(rng.uniform(-4, 4, n))
    b = f32(rng.uniform(-4, 4, n))
    if op in ("DIV", "RECIP"):                   # keep denominators away from 0
        b = f32(np.where(np.abs(b) < 0.5, 0.5, b))
        a = f32(np.where(np.abs(a) < 0.5, 0.5, a)) if op == "RECIP" else a
    alpha, beta = (-1.0, 2.0) if op == "CLAMP" else (0.75, -1.25)
    from lanternl_amd._lib import call
    A, B, Cb = device.Buffer.from_numpy(a), device.Buffer.from_numpy(b), device.Buffer((n,))
    call("lhip_elementwise", A.ptr, B.ptr, Cb.ptr, n, O.EW[op], alpha, beta)
    device.sync()
    ref = O.ew(op, a, b, alpha, beta)
    got = Cb.download().astype(np.float64)
    if op == "FILL":
        assert np.all(got == np.float32(alpha))
    else:
        assert rel_fro(got, ref) <= ROW, op
    # in place on an unaligned view (the scalar path)
    call("lhip_elementwise", A.offset(1), B.offset(1), A.offset(1), n - 1, O.EW[op], alpha, beta)
    device.sync()
    got = A.download().astype(np.float64)[1:]
    assert rel_fro(got, O.ew(op, a[1:], b[1:], alpha, beta)) <= ROW or op == "FILL"


def test_luatl_reductions_and_small_ops():
    announce("adapter", "reduce_cols/l2/clip/sum/transpose/bcast_add/row_rms/adamw")
    from lanternl_amd._lib import call
    rng = np.random.default_rng(34)
    R, Cn = 300, 70
    x = f32(rng.standard_normal((R, Cn)))
    X = device.Buffer.from_numpy(x)
    out0 = f32(rng.standard_normal(Cn))
    OUT = device.Buffer.from_numpy(out0)
    call("lhip_reduce_cols", X.ptr, OUT.ptr, R, Cn, Cn, 0.5, 2.0)
    assert rel_fro(OUT.download(), O.reduce_cols(x, out0.copy(), 0.5, 2.0)) <= ROW
    ACC = device.Buffer.from_numpy(np.array([1.5], np.float32))
    call("lhip_l2_accum", X.ptr, R * Cn, ACC.ptr)
    device.sync()
    assert abs(ACC.download()[0] - (1.5 + np.sum(x * x))) <= 1e-6 * np.sum(x * x)
    S = device.Buffer.from_numpy(np.array([0.25], np.float32))
    call("lhip_sum_accum", X.ptr, R * Cn, 2.0, S.ptr)
    device.sync()
    assert abs(S.download()[0] - (0.25 + 2.0 * np.sum(x))) <= 1e-4 * np.sum(np.abs(x))
    nsq = float(np.sum(x * x))
    NSQ = device.Buffer.from_numpy(np.array([nsq], np.float32))
    Y = device.Buffer.from_numpy(x)
    call("lhip_clip_by_nsq", Y.ptr, R * Cn, NSQ.ptr, 1.0)
    assert rel_fro(Y.download(), O.clip_by_nsq(x.copy(), float(np.float32(nsq)), 1.0)) <= ROW
    T = device.Buffer((Cn, R))
    call("lhip_transpose", X.ptr, T.ptr, R, Cn)
    device.sync()
    assert np.array_equal(T.download(), x.T.astype(np.float32))
    v = f32(rng.standard_normal(Cn))
    V, BO = device.Buffer.from_numpy(v), device.Buffer((R, Cn))
    call("lhip_bcast_add", X.ptr, V.ptr, BO.ptr, R, Cn, -0.5)
    assert rel_fro(BO.download(), x - 0.5 * v[None, :]) <= ROW
    RR = device.Buffer((R,))
    call("lhip_row_rms", X.ptr, RR.ptr, R, Cn, Cn, 1, 1e-5)
    assert rel_fro(RR.download(), O.rmsnorm_fwd(x, np.ones(Cn), 1e-5)[1]) <= ROW
    call("lhip_row_rms", X.ptr, RR.ptr, Cn, R, 1, Cn, 1e-5)          # the columns, as strided rows
    assert rel_fro(RR.download()[:Cn], O.rmsnorm_fwd(np.ascontiguousarray(x.T), np.ones(R), 1e-5)[1]) <= ROW
    n = 5000
    w = f32(rng.standard_normal(n)); gr = f32(rng.standard_normal(n) * 3)
    m = f32(rng.standard_normal(n) * 0.1); vv = f32(np.abs(rng.standard_normal(n)))
    Wb, Gb, Mb, Vb, Wm = (device.Buffer.from_numpy(a) for a in (w, gr, m, vv, np.zeros(n, np.float32)))
    call("lhip_adamw_elementwise", Wb.ptr, Gb.ptr, Mb.ptr, Vb.ptr, Wm.ptr, n, 3, 1e-2, 0.9, 0.999, 1e-8, 0.01, 2.0)
    wr, mr, vr = w.copy(), m.copy(), vv.copy()
    O.adamw_luatl(wr, gr, mr, vr, 3, 1e-2, 0.9, 0.999, 1e-8, 0.01, 2.0)
    assert rel_fro(Wb.download(), wr) <= ROW and rel_fro(Mb.download(), mr) <= ROW
    assert rel_fro(Vb.download(), vr) <= ROW and np.array_equal(Wm.download(), Wb.download())


# ----------------------------------------------------------- luaTL.Program
def _program_model(rng):
    """A small forward + loss + update written as luaTL.Program ops."""
    N, D, V = 64, 32, 50
    x = f32(rng.standard_normal((N, D))); w = f32(rng.standard_normal((D, V)) * 0.2)
    gam = f32(rng.normal(1, 0.1, D)); tgt = rng.integers(0, V, N).astype(np.int32)
    T = {k: ad.Tensor.new(*s) for k, s in dict(x=(N, D), w=(D, V), g=(1, D), h=(N, D), logits=(N, V),
                                                 p=(N, V), loss=(N, 1), dlog=(N, V), l2=(1, 1), lsum=(1, 1),
                                                 am=(N, 1), dw=(D, V)).items()}
    for k, a in (("x", x), ("w", w), ("g", gam.reshape(1, -1))):
        ad.Handle(T[k], *a.shape).upload(a.ravel())
    ids = ad.ids(N)
    ad.upload_i32(ids, tgt, N)
    return T, ids, (x, w, gam, tgt)


def _queue(P, T, ids):
    P.zero(T["l2"]).zero(T["lsum"])
    P.rmsnorm(T["x"], T["g"], T["h"], 1e-5)
    P.gemm(T["h"], T["w"], T["logits"])
    P.softmax(T["logits"], T["p"], {"scale": 0.5})
    P.cross_entropy(T["logits"], ids.t, T["loss"], T["dlog"], {"grad_scale": 1.0 / 64})
    P.argmax(T["logits"], T["am"])
    P.dw(T["h"], T["dlog"], T["dw"], 0.0)
    P.l2(T["dw"], T["l2"])
    P.sum(T["loss"], T["lsum"], 1.0 / 64)
    P.barrier()
    P.axpy(T["w"], T["dw"], 1.0)         # w = 1*w + dw  (AXPY with a = dst)
    return P


def test_program_op_list_run_capture_replay():
    announce("adapter", "luaTL.Program ops")
    rng = np.random.default_rng(35)
    T, ids, (x, w, gam, tgt) = _program_model(rng)
    P = ad.program(64, True)
    _queue(P, T, ids)
    assert P.size() == 12 and not P.is_captured()
    P.run(keep=True)                    # eager, kept for capture
    assert P.elapsed_ms() > 0
    eager = {k: dl(T[k]) for k in ("h", "logits", "p", "loss", "dlog", "dw", "l2", "lsum", "w")}
    am_e = np.empty(64, np.int32)
    ad.download_i32(T["am"], am_e, 64)
    # oracle for the first step
    h = O.rmsnorm_fwd(x, gam, 1e-5)[0]
    assert rel_fro(eager["h"], h) <= ROW
    logits = O.mm(f32(eager["h"]), w)
    assert rel_fro(eager["logits"], logits) <= GEMM
    assert rel_fro(eager["p"], O.softmax_ex(f32(eager["logits"]), None, 0.5)) <= ROW
    l_ref, d_ref = O.ce_fused(f32(eager["logits"]), tgt, -1, 1.0 / 64)
    assert np.max(np.abs(eager["loss"].ravel() - l_ref)) <= 1e-5 and rel_fro(eager["dlog"], d_ref) <= ROW
    assert np.array_equal(am_e, O.argmax_rows(f32(eager["logits"])))
    assert rel_fro(eager["dw"], O.matmul_tn(f32(eager["h"]), f32(eager["dlog"]))) <= GEMM
    assert abs(eager["l2"][0, 0] - np.sum(eager["dw"] ** 2)) <= 1e-5 * np.sum(eager["dw"] ** 2)
    assert abs(eager["lsum"][0, 0] - np.mean(eager["loss"])) <= 1e-6
    assert rel_fro(eager["w"], w + eager["dw"]) <= ROW
    # capture: each replay runs one more step from the current weights; the
    # eager run of the same queue from the same weights must match bit for bit
    P.capture()
    assert P.is_captured()
    W = ad.Handle(T["w"], 32, 50)
    scratch = device.Buffer((1 << 16,))
    from lanternl_amd._lib import call
    for rep in range(3):
        W.upload(w.ravel())
        P.replay()
        got = {k: dl(T[k]) for k in ("loss", "dw", "l2", "w")}
        W.upload(w.ravel())
        P2 = ad.program(64)
        _queue(P2, T, ids).run()
        for k in got:
            assert np.array_equal(got[k], dl(T[k])), (rep, k)
        call("lhip_fill", scratch.ptr, scratch.size, float(rep))   # eager work between replays
    P.free_graph()
    assert not P.is_captured()
    # run() without keep clears the queue; capacity is enforced
    P.run()
    assert P.size() == 0
    small = ad.program(2)
    small.zero(T["l2"]).zero(T["lsum"])
    with pytest.raises(ad.ProgramFull, match="full"):
        small.zero(T["am"])
    with pytest.raises(ValueError):
        ad.program(4).capture()


def test_hardware_stats_and_mem_keys():
    hw = ad.hardware()
    for k in ("name", "sm", "multiprocessors", "warp_size", "total_vram", "free_vram", "l2_cache",
              "bandwidth_gbs", "gflops_fp32"):
        assert k in hw, k
    assert hw["warp_size"] == 64 and hw["multiprocessors"] > 0 and hw["gflops_fp32"] > 1e5
    st = ad.stats()
    for k in ("reserved", "in_use", "peak", "blocks", "allocs", "frees"):
        assert k in st, k
    free, total = ad.mem()
    assert 0 < free <= total
