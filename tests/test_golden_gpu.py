"""GPU parity against the committed golden fixtures (tests/golden/*.npz, written
by tests/golden/make_golden.py from the pinned oracle): the HIP path on the
stored fp32 inputs against the stored outputs, through the C ABI.

Bars as in the other parity tests: GEMM products relative Frobenius <= 1e-4;
fp32 row / elementwise kernels <= 1e-5; CE losses 1e-5 absolute; argmax and
embedding gathers bit-exact; the LM step's losses 1e-5 absolute, gradients,
update and velocity 1e-4 relative, global norm 1e-5 relative."""
import os

import numpy as np
import pytest

from lanternl_amd import device, kernels, lmtrain
from lanternl_amd._lib import call
from tests.gpu_util import announce, rel_fro, to_dev

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module", autouse=True)
def _dev():
    device.init(0)
    yield


def load(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"))


def dl(buf):
    device.sync()
    return buf.download()


def _gemm(ta, tb, a, b):
    A, B = to_dev(a), to_dev(b)
    m = a.shape[1] if ta else a.shape[0]
    n = b.shape[0] if tb else b.shape[1]
    C = device.Buffer((m, n))
    kernels.sgemm(A, B, C, transa=ta, transb=tb)
    return dl(C)


def test_golden_gemm_family():
    announce("golden gemm")
    g = load("gemm_c1")
    a, b = g["a"], g["b"]
    assert rel_fro(_gemm(False, False, a, b), g["c_nn"]) <= 1e-4
    assert rel_fro(_gemm(False, True, a, np.ascontiguousarray(b.T)), g["c_nt"]) <= 1e-4
    assert rel_fro(_gemm(True, False, np.ascontiguousarray(a.T), b), g["c_tn"]) <= 1e-4
    o = load("gemm_odd")
    for tag in ("s1", "s2"):
        assert rel_fro(_gemm(False, False, o[f"{tag}_a"], o[f"{tag}_b"]), o[f"{tag}_c"]) <= 1e-4


def test_golden_row_and_elementwise_ops():
    announce("golden ops")
    g = load("ops_tiny")
    r, c = g["rms_x"].shape
    X, W, Y, INV = to_dev(g["rms_x"]), to_dev(g["rms_w"]), device.Buffer((r, c)), device.Buffer((r,))
    call("lhip_rmsnorm_fwd", X.ptr, W.ptr, Y.ptr, INV.ptr, r, c, 1e-5)
    assert rel_fro(dl(Y), g["rms_y"]) <= 1e-5 and rel_fro(dl(INV), g["rms_inv"]) <= 1e-5
    G, DX, DW = to_dev(g["rms_g"]), device.Buffer((r, c)), device.Buffer((c,))
    call("lhip_rmsnorm_bwd", X.ptr, W.ptr, INV.ptr, G.ptr, DX.ptr, DW.ptr, r, c, 0)
    assert rel_fro(dl(DX), g["rms_dx"]) <= 1e-5 and rel_fro(dl(DW), g["rms_dw"]) <= 1e-5
    r, c = g["sm_x"].shape
    for tag, causal in (("sm", 0), ("smc", 1)):
        S, P, GS, DS = to_dev(g["sm_x"]), device.Buffer((r, c)), to_dev(g["sm_g"]), device.Buffer((r, c))
        call("lhip_softmax_fwd", S.ptr, P.ptr, r, c, 1.0, causal, 0, 0)
        p = dl(P)
        assert rel_fro(p, g[f"{tag}_y"]) <= 1e-5
        if causal:
            assert np.all(np.triu(p, 1) == 0)
        call("lhip_softmax_bwd", P.ptr, GS.ptr, DS.ptr, r, c, 1.0, causal, 0, 0, 0)
        assert rel_fro(dl(DS), g[f"{tag}_dx"]) <= 1e-5
    r, c = g["sw_g"].shape
    GA, UP, H = to_dev(g["sw_g"]), to_dev(g["sw_u"]), device.Buffer((r, c))
    call("lhip_swiglu_fwd", GA.ptr, c, UP.ptr, c, H.ptr, c, r, c)
    assert rel_fro(dl(H), g["sw_h"]) <= 1e-5
    DH, DG, DU = to_dev(g["sw_dh"]), device.Buffer((r, c)), device.Buffer((r, c))
    call("lhip_swiglu_bwd", GA.ptr, c, UP.ptr, c, DH.ptr, c, DG.ptr, c, DU.ptr, c, r, c, 0)
    assert rel_fro(dl(DG), g["sw_dg"]) <= 1e-5 and rel_fro(dl(DU), g["sw_du"]) <= 1e-5
    r, c = g["rope_x"].shape
    for tag, il in (("il", 1), ("hs", 0)):
        for inv, key in ((0, "fwd"), (1, "bwd")):
            XR = to_dev(g["rope_x"])
            call("lhip_rope", XR.ptr, None, r, 3, 8, c, 0, 0, 10000.0, il, inv)
            assert rel_fro(dl(XR), g[f"rope_{tag}_{key}"]) <= 1e-5
    r, v = g["ce_logits"].shape
    LG, TG, LS, DLG = to_dev(g["ce_logits"]), to_dev(g["ce_tgt"], np.int32), device.Buffer((r,)), device.Buffer((r, v))
    call("lhip_ce_fused", LG.ptr, TG.ptr, LS.ptr, DLG.ptr, r, v, -1, 0.25)
    assert np.max(np.abs(dl(LS).astype(np.float64) - g["ce_loss"])) <= 1e-5
    assert rel_fro(dl(DLG), g["ce_dlogits"]) <= 1e-5
    r, c = g["am_x"].shape
    AM, IDX = to_dev(g["am_x"]), device.Buffer((r,), np.int32)
    call("lhip_argmax_rows", AM.ptr, IDX.ptr, r, c)
    assert np.array_equal(dl(IDX), g["am_idx"])
    n, dim = g["emb_g"].shape
    vocab = g["emb_table"].shape[0]
    TB, IDS, OUT = to_dev(g["emb_table"]), to_dev(g["emb_ids"], np.int32), device.Buffer((n, dim))
    call("lhip_embed_fwd", TB.ptr, IDS.ptr, OUT.ptr, n, dim, vocab)
    assert np.array_equal(dl(OUT), g["emb_out"])
    GE, DT = to_dev(g["emb_g"]), device.Buffer((vocab, dim)).zero()
    call("lhip_embed_bwd", GE.ptr, IDS.ptr, DT.ptr, n, dim, vocab, 1.0, 0)
    assert rel_fro(dl(DT), g["emb_dtable"]) <= 1e-5


def test_golden_lm_tiny_step():
    announce("golden lm step")
    g = load("lm_tiny_step")
    V, D, L, H, F, B, T = (int(x) for x in g["cfg"])
    lr, mom, wd, clip = (float(x) for x in g["lr_mom_wd_clip"])
    gpu = lmtrain.GpuLMStep(V, D, L, H, F, B, T)
    gpu.set_params(g["params"])
    gpu.set_batch(g["ids"], g["tgt"])
    gpu.step(lr, mom, wd, clip)
    st = gpu.stats()
    assert st["applied"] == bool(g["applied"])
    assert np.max(np.abs(st["window_losses"] - g["losses"])) <= 1e-5
    assert abs(st["grad_norm"] - float(g["gnorm"])) <= 1e-5 * float(g["gnorm"])
    p0 = g["params"].astype(np.float64)
    assert rel_fro(gpu.grads(), g["grads"]) <= 1e-4
    assert rel_fro(gpu.params().astype(np.float64) - p0, g["params_after"].astype(np.float64) - p0) <= 1e-4
    assert rel_fro(gpu.velocity(), g["velocity_after"]) <= 1e-4
    gpu.close()
