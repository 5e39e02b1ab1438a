"""Writes the golden fixtures of tests/golden/ (run: python tests/golden/make_golden.py).

The reference's CPU path cannot run here (no Lua runtime; its CUDA half needs
nvcc), so the vectors come from this repository's double-precision restatement
of the Lua loops (oracle/, pinned in tests/test_oracle.py against the
reference's own known answers, library routines, finite differences and
closed forms).  Once committed they freeze that pinned behaviour: the CPU
tests check that the oracle still reproduces them, the GPU tests check the HIP
path against them.

Inputs are drawn from numpy's PCG64 with fixed seeds, rounded to fp32 and
stored as fp32 (so both sides see identical values); expected outputs are
stored as fp32 too (their rounding, ~6e-8 relative, is far below every bar).

Fixtures (each an .npz):
  gemm_c1.npz        config C1: A 256x128, B 128x256 ~U[-1,1]; C = A.B, and
                     the transposed products on the stored transposes
                     (matrix.lua:514-539, :597-625, :627-660)
  gemm_odd.npz       37x53.53x41 and 128x96.96x160 (shapes of tests/test.lua:42,65)
  ops_tiny.npz       forward and backward of every row/elementwise op at tiny
                     sizes: RMSNorm, causal/non-causal softmax, SwiGLU, RoPE
                     (interleaved and half-split), fused CE with an ignored
                     row, argmax with ties / -inf / NaN rows, embedding
                     gather and scatter-add with duplicate ids
  lm_tiny_step.npz   one LMTrain SGD step, V=32 D=16 L=1 H=2 F=32, B=2 windows
                     of T=8: parameters, ids, targets before; per-window
                     losses, gradients, global norm, parameters and velocity after
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import oracle as O  # noqa: E402  (test infrastructure: the checker)


def f32(a):
    return np.asarray(a, dtype=np.float32)


def gemm_c1():
    rng = np.random.default_rng(101)
    a = f32(rng.uniform(-1, 1, (256, 128)))
    b = f32(rng.uniform(-1, 1, (128, 256)))
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    return dict(a=a, b=b, c_nn=f32(O.mm(a64, b64)),
                c_nt=f32(O.matmul_nt(a64, np.ascontiguousarray(b64.T))),
                c_tn=f32(O.matmul_tn(np.ascontiguousarray(a64.T), b64)))


def gemm_odd():
    rng = np.random.default_rng(102)
    out = {}
    for tag, (m, k, n) in {"s1": (37, 53, 41), "s2": (128, 96, 160)}.items():
        a = f32(rng.uniform(-1, 1, (m, k)))
        b = f32(rng.uniform(-1, 1, (k, n)))
        out[f"{tag}_a"], out[f"{tag}_b"] = a, b
        out[f"{tag}_c"] = f32(O.mm(a.astype(np.float64), b.astype(np.float64)))
    return out


def ops_tiny():
    rng = np.random.default_rng(103)
    d = {}
    # RMSNorm (tensor2.lua:609-666), eps 1e-5
    x = f32(rng.standard_normal((6, 20)))
    w = f32(rng.normal(1.0, 0.1, 20))
    g = f32(rng.standard_normal((6, 20)))
    y, inv = O.rmsnorm_fwd(x.astype(np.float64), w.astype(np.float64), 1e-5)
    dx, dw = O.rmsnorm_bwd(x.astype(np.float64), w.astype(np.float64), inv, g.astype(np.float64))
    d.update(rms_x=x, rms_w=w, rms_g=g, rms_y=f32(y), rms_inv=f32(inv), rms_dx=f32(dx), rms_dw=f32(dw))
    # softmax (tensor2.lua:332-408), non-causal and causal
    s = f32(rng.normal(0, 2, (7, 9)))
    gs = f32(rng.standard_normal((7, 9)))
    for tag, causal in (("sm", False), ("smc", True)):
        p = O.softmax_fwd(s.astype(np.float64), causal=causal)
        d[f"{tag}_y"] = f32(p)
        d[f"{tag}_dx"] = f32(O.softmax_bwd(p, gs.astype(np.float64), causal=causal))
    d.update(sm_x=s, sm_g=gs)
    # SwiGLU (tensor2.lua:167-183, 272-303)
    ga = f32(rng.normal(0, 2, (5, 12)))
    up = f32(rng.standard_normal((5, 12)))
    dh = f32(rng.standard_normal((5, 12)))
    h = O.swiglu_fwd(ga.astype(np.float64), up.astype(np.float64))
    dg, du = O.swiglu_bwd(ga.astype(np.float64), up.astype(np.float64), dh.astype(np.float64))
    d.update(sw_g=ga, sw_u=up, sw_dh=dh, sw_h=f32(h), sw_dg=f32(dg), sw_du=f32(du))
    # RoPE over 3 heads of 8 (transformer.lua:30-48; tensor2.lua:410-473), base 1e4, positions 0..9
    xr = f32(rng.standard_normal((10, 24)))
    d["rope_x"] = xr
    for tag, il in (("il", True), ("hs", False)):
        d[f"rope_{tag}_fwd"] = f32(O.rope_heads(xr.astype(np.float64), 3, 8, interleaved=il))
        d[f"rope_{tag}_bwd"] = f32(O.rope_heads(xr.astype(np.float64), 3, 8, interleaved=il, inverse=True))
    # fused softmax + CE (tensor2.lua:809-882): row 2 ignored (-1), grad scale 1/4
    lg = f32(rng.normal(0, 3, (4, 11)))
    tg = np.array([3, 0, -1, 10], np.int32)
    loss, dlog = O.ce_fused(lg.astype(np.float64), tg, -1, 0.25)
    d.update(ce_logits=lg, ce_tgt=tg, ce_loss=f32(loss), ce_dlogits=f32(dlog))
    # argmax (lmtrain.lua:1200-1209): ties -> first, NaN never wins, all -inf -> 0
    am = f32(rng.standard_normal((5, 7)))
    am[1, 2] = am[1, 5] = 9.0
    am[2, :] = -np.inf
    am[3, 0] = np.nan
    am[3, 4] = 5.0
    d.update(am_x=am, am_idx=O.argmax_rows(am.astype(np.float64)).astype(np.int32))
    # embedding gather and scatter-add with duplicate ids (tensor2.lua:572-607)
    table = f32(rng.standard_normal((9, 6)))
    ids = np.array([3, 0, 7, 3, 1, 3], np.int32)
    ge = f32(rng.standard_normal((6, 6)))
    d.update(emb_table=table, emb_ids=ids, emb_g=ge,
             emb_out=f32(O.embed_fwd(table.astype(np.float64), ids)),
             emb_dtable=f32(O.embed_bwd(ge.astype(np.float64), ids, 9)))
    return d


def lm_tiny_step():
    V, D, L, H, F, B, T = 32, 16, 1, 2, 32, 2, 8
    rng = np.random.default_rng(104)
    cfg = O.lm_cfg(V, D, L, H, F)
    n = O.lm_num_params(cfg)
    p0 = f32(rng.normal(0, 0.3, n))
    # norm gains at 1 (Transformer.new), the rest N(0, 0.3)
    for name, off, rows, cols in O.lm_param_table(cfg):
        if name.startswith("ln"):
            p0[off:off + rows * cols] = 1.0
    ids = rng.integers(0, V, (B, T)).astype(np.int32)
    tgt = rng.integers(0, V, (B, T)).astype(np.int32)
    p = p0.astype(np.float64)
    v = np.zeros(n)
    ref = O.lm_step_sgd(cfg, p, v, ids, tgt, 0.1, 0.9, 0.01, 1.0)
    return dict(cfg=np.array([V, D, L, H, F, B, T], np.int32), params=p0, ids=ids, tgt=tgt,
                lr_mom_wd_clip=np.array([0.1, 0.9, 0.01, 1.0]),
                losses=f32(ref["losses"]), grads=f32(ref["grads"]), gnorm=np.float64(ref["gnorm"]),
                applied=np.int32(ref["applied"]), params_after=f32(p), velocity_after=f32(v))


FIXTURES = {"gemm_c1": gemm_c1, "gemm_odd": gemm_odd, "ops_tiny": ops_tiny, "lm_tiny_step": lm_tiny_step}


def main():
    for name, make in FIXTURES.items():
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **make())
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
