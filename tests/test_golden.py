"""CPU: the committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py) are reproduced by the oracle from their stored
inputs -- a regression pin on the double-precision restatement of the Lua
loops, which tests/test_oracle.py pins against the reference's known answers,
library routines and closed forms.  Outputs were stored as fp32, so the bar is
fp32 rounding (2e-7 relative per element, scaled by magnitude); integer
results (argmax) are exact."""
import os

import numpy as np
import pytest

import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"))


def close32(got, want):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape
    assert np.all(np.isfinite(got) == np.isfinite(want))
    fin = np.isfinite(want)
    scale = np.maximum(np.abs(want[fin]), np.max(np.abs(want[fin])) * 1e-3 if fin.any() else 1.0)
    assert np.all(np.abs(got[fin] - want[fin]) <= 4e-7 * scale + 1e-30)


def d(x):
    return np.asarray(x, dtype=np.float64)


def test_fixtures_present_and_generator_committed():
    for name in ("gemm_c1", "gemm_odd", "ops_tiny", "lm_tiny_step"):
        assert os.path.exists(os.path.join(GOLDEN, name + ".npz")), name
    assert os.path.exists(os.path.join(GOLDEN, "make_golden.py"))


def test_golden_gemm_c1_and_odd_shapes():
    g = load("gemm_c1")
    a, b = d(g["a"]), d(g["b"])
    assert g["a"].shape == (256, 128) and g["b"].shape == (128, 256)
    close32(O.mm(a, b), g["c_nn"])
    close32(O.matmul_nt(a, np.ascontiguousarray(b.T)), g["c_nt"])
    close32(O.matmul_tn(np.ascontiguousarray(a.T), b), g["c_tn"])
    # an independent library product agrees with the fixture to double rounding
    close32(a @ b, g["c_nn"])
    o = load("gemm_odd")
    for tag in ("s1", "s2"):
        close32(O.mm(d(o[f"{tag}_a"]), d(o[f"{tag}_b"])), o[f"{tag}_c"])
        close32(d(o[f"{tag}_a"]) @ d(o[f"{tag}_b"]), o[f"{tag}_c"])


def test_golden_row_and_elementwise_ops():
    g = load("ops_tiny")
    y, inv = O.rmsnorm_fwd(d(g["rms_x"]), d(g["rms_w"]), 1e-5)
    close32(y, g["rms_y"]); close32(inv, g["rms_inv"])
    dx, dw = O.rmsnorm_bwd(d(g["rms_x"]), d(g["rms_w"]), inv, d(g["rms_g"]))
    close32(dx, g["rms_dx"]); close32(dw, g["rms_dw"])
    for tag, causal in (("sm", False), ("smc", True)):
        p = O.softmax_fwd(d(g["sm_x"]), causal=causal)
        close32(p, g[f"{tag}_y"])
        close32(O.softmax_bwd(p, d(g["sm_g"]), causal=causal), g[f"{tag}_dx"])
    # causal rows keep exactly their prefix
    assert np.all(np.triu(g["smc_y"], 1) == 0) and np.allclose(g["smc_y"].sum(1), 1, atol=1e-6)
    close32(O.swiglu_fwd(d(g["sw_g"]), d(g["sw_u"])), g["sw_h"])
    dg, du = O.swiglu_bwd(d(g["sw_g"]), d(g["sw_u"]), d(g["sw_dh"]))
    close32(dg, g["sw_dg"]); close32(du, g["sw_du"])
    for tag, il in (("il", True), ("hs", False)):
        close32(O.rope_heads(d(g["rope_x"]), 3, 8, interleaved=il), g[f"rope_{tag}_fwd"])
        close32(O.rope_heads(d(g["rope_x"]), 3, 8, interleaved=il, inverse=True), g[f"rope_{tag}_bwd"])
    loss, dl = O.ce_fused(d(g["ce_logits"]), g["ce_tgt"], -1, 0.25)
    close32(loss, g["ce_loss"]); close32(dl, g["ce_dlogits"])
    assert g["ce_loss"][2] == 0 and np.all(g["ce_dlogits"][2] == 0)        # ignored row
    assert np.array_equal(O.argmax_rows(d(g["am_x"])), g["am_idx"])
    assert list(g["am_idx"][1:4]) == [2, 0, 4]                              # tie, all -inf, NaN
    close32(O.embed_fwd(d(g["emb_table"]), g["emb_ids"]), g["emb_out"])
    close32(O.embed_bwd(d(g["emb_g"]), g["emb_ids"], 9), g["emb_dtable"])


def test_golden_lm_tiny_step():
    g = load("lm_tiny_step")
    V, D, L, H, F, B, T = (int(x) for x in g["cfg"])
    cfg = O.lm_cfg(V, D, L, H, F)
    p = d(g["params"]).copy()
    v = np.zeros_like(p)
    lr, mom, wd, clip = (float(x) for x in g["lr_mom_wd_clip"])
    ref = O.lm_step_sgd(cfg, p, v, g["ids"], g["tgt"], lr, mom, wd, clip)
    close32(ref["losses"], g["losses"])
    close32(ref["grads"], g["grads"])
    assert ref["gnorm"] == pytest.approx(float(g["gnorm"]), rel=1e-12)
    assert int(ref["applied"]) == int(g["applied"])
    close32(p, g["params_after"])
    close32(v, g["velocity_after"])
