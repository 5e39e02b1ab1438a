"""ctypes wrapper around liboracle.so -- TEST INFRASTRUCTURE ONLY.

All arrays are numpy float64 (int32 for ids/labels), row-major, 0-based ids.
See oracle.h for the reference file:line each function restates.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_D = ctypes.POINTER(ctypes.c_double)
_I = ctypes.POINTER(ctypes.c_int)


class LmCfg(ctypes.Structure):
    """or_lm_cfg (oracle.h); defaults follow ai/nn/transformer.lua:88-98."""
    _fields_ = [("vocab", ctypes.c_int), ("dim", ctypes.c_int), ("layers", ctypes.c_int),
                ("heads", ctypes.c_int), ("ffn", ctypes.c_int), ("causal", ctypes.c_int),
                ("eps", ctypes.c_double), ("rope_base", ctypes.c_double)]


def build():
    """Compile liboracle.so from oracle.c (gcc, strict IEEE double)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


def _declare(L):
    c_int, c_long, c_double = ctypes.c_int, ctypes.c_long, ctypes.c_double
    sig = {
        "or_mm": (None, [_D, _D, _D, c_int, c_int, c_int, c_int]),
        "or_matmul_nt": (None, [_D, _D, _D, c_int, c_int, c_int, c_int]),
        "or_matmul_tn": (None, [_D, _D, _D, c_int, c_int, c_int, c_int]),
        "or_rmsnorm_fwd": (None, [_D, _D, _D, _D, c_int, c_int, c_double]),
        "or_rmsnorm_bwd": (None, [_D, _D, _D, _D, _D, _D, c_int, c_int]),
        "or_softmax_fwd": (None, [_D, _D, c_int, c_int, c_int, c_int]),
        "or_softmax_bwd": (None, [_D, _D, _D, c_int, c_int, c_int, c_int]),
        "or_silu_fwd": (None, [_D, _D, _D, c_long]),
        "or_silu_bwd": (None, [_D, _D, _D, _D, c_long]),
        "or_swiglu_fwd": (None, [_D, _D, _D, c_long]),
        "or_swiglu_bwd": (None, [_D, _D, _D, _D, _D, c_long]),
        "or_rope_angles": (None, [c_double, c_int, c_int, _D, _D]),
        "or_rope_fwd": (None, [_D, _D, c_int, c_int, _D, _D, c_int]),
        "or_rope_bwd": (None, [_D, _D, c_int, c_int, _D, _D, c_int]),
        "or_rope_heads": (None, [_D, _I, c_int, c_int, c_int, c_int, c_int, c_double, c_int, c_int]),
        "or_cross_entropy": (c_double, [_D, _I, c_int, c_int, c_int, c_int, _D, _I]),
        "or_cross_entropy_bwd": (None, [_D, _I, c_int, c_int, c_int, c_int, c_double, c_int, _D]),
        "or_ce_fused": (None, [_D, _I, _D, _D, c_int, c_int, c_int, c_double]),
        "or_argmax_rows": (None, [_D, _I, c_int, c_int]),
        "or_embed_fwd": (None, [_D, _I, _D, c_int, c_int]),
        "or_embed_bwd": (None, [_D, _I, _D, c_int, c_int, c_double]),
        "or_grad_norm": (c_double, [_D, c_long]),
        "or_scale": (None, [_D, c_long, c_double]),
        "or_sgd_step": (None, [_D, _D, _D, c_long, c_double, c_double, c_double, c_int]),
        "or_adamw_step": (None, [_D, _D, _D, _D, c_long, c_double, c_double, c_double, c_double,
                                 c_double, c_int]),
        "or_ew": (None, [c_int, _D, _D, _D, c_long, c_double, c_double]),
        "or_gemm_ex": (None, [_D, _D, _D, _D, _D, _D, c_int, c_int, c_int, c_long, c_long, c_long, c_long,
                              c_long, c_long, c_long, c_long, c_long, c_int, c_double, c_double, c_double,
                              c_int, c_int]),
        "or_softmax_ex": (None, [_D, _D, _D, c_int, c_int, c_double, c_int, c_int, c_int]),
        "or_softmax_bwd_ex": (None, [_D, _D, _D, c_int, c_int, c_double, c_int, c_int, c_int]),
        "or_rmsnorm_bwd_luatl": (None, [_D, _D, _D, _D, _D, c_int, c_int, c_double]),
        "or_adamw_luatl": (None, [_D, _D, _D, _D, c_long, c_int, c_double, c_double, c_double, c_double,
                                  c_double, c_double]),
        "or_reduce_cols": (None, [_D, _D, c_int, c_int, c_long, c_double, c_double]),
        "or_clip_by_nsq": (None, [_D, c_long, c_double, c_double]),
        "or_lm_num_params": (c_long, [ctypes.POINTER(LmCfg)]),
        "or_lm_param_offsets": (c_int, [ctypes.POINTER(LmCfg), ctypes.POINTER(c_long), _I, _I]),
        "or_lm_window": (c_double, [ctypes.POINTER(LmCfg), _D, _I, _I, c_int, _D, _D, _I]),
        "or_lm_step_sgd": (c_int, [ctypes.POINTER(LmCfg), _D, _D, _I, _I, c_int, c_int,
                                   c_double, c_double, c_double, c_double, _D, _D, _I, _D]),
        "or_lm_step_adamw": (c_int, [ctypes.POINTER(LmCfg), _D, _D, _D, _I, _I, _I, c_int, c_int,
                                     c_double, c_double, c_double, c_double, c_double, c_double,
                                     _D, _D, _I, _D]),
        "or_lm_step_sgd_ex": (c_int, [ctypes.POINTER(LmCfg), _D, _D, _I, _I, c_int, c_int, _I,
                                      c_double, c_double, c_double, c_double, _D, _D, _I, _D]),
        "or_lm_step_adamw_ex": (c_int, [ctypes.POINTER(LmCfg), _D, _D, _D, _I, _I, _I, c_int, c_int, _I,
                                        c_double, c_double, c_double, c_double, c_double, c_double,
                                        _D, _D, _I, _D]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _d(a):
    """float64 C-contiguous view/copy and its pointer."""
    a = np.ascontiguousarray(a, dtype=np.float64)
    return a, a.ctypes.data_as(_D)


def _i(a):
    a = np.ascontiguousarray(a, dtype=np.int32)
    return a, a.ctypes.data_as(_I)


def _nul(kind):
    return ctypes.cast(None, kind)


# ---------------------------------------------------------------- GEMM family
def mm(a, b, out=None, acc=False):
    """matrix.multiply CPU path (matrix.lua:514-539): a (m,k) . b (k,n)."""
    a, pa = _d(a); b, pb = _d(b)
    m, k = a.shape; n = b.shape[1]
    assert b.shape[0] == k, (a.shape, b.shape)
    r = np.zeros((m, n)) if out is None else out
    assert r.dtype == np.float64 and r.flags.c_contiguous and r.shape == (m, n)
    lib().or_mm(pa, pb, r.ctypes.data_as(_D), m, k, n, int(acc))
    return r


def matmul_nt(a, b, out=None, acc=False):
    """matrix.matmul_nt (matrix.lua:597-625): a (m,k) . b(n,k)^T."""
    a, pa = _d(a); b, pb = _d(b)
    m, k = a.shape; n = b.shape[0]
    assert b.shape[1] == k, (a.shape, b.shape)
    r = np.zeros((m, n)) if out is None else out
    assert r.dtype == np.float64 and r.flags.c_contiguous and r.shape == (m, n)
    lib().or_matmul_nt(pa, pb, r.ctypes.data_as(_D), m, k, n, int(acc))
    return r


def matmul_tn(a, b, out=None, acc=False):
    """matrix.matmul_tn (matrix.lua:627-660): a (m,k)^T . b (m,n) -> (k,n)."""
    a, pa = _d(a); b, pb = _d(b)
    m, k = a.shape; n = b.shape[1]
    assert b.shape[0] == m, (a.shape, b.shape)
    r = np.zeros((k, n)) if out is None else out
    assert r.dtype == np.float64 and r.flags.c_contiguous and r.shape == (k, n)
    lib().or_matmul_tn(pa, pb, r.ctypes.data_as(_D), m, k, n, int(acc))
    return r


# ---------------------------------------------------------------- row ops
def rmsnorm_fwd(x, w, eps=1e-5):
    x, px = _d(x); w, pw = _d(w)
    rows, cols = x.shape
    out = np.zeros_like(x); inv = np.zeros(rows)
    lib().or_rmsnorm_fwd(px, pw, out.ctypes.data_as(_D), inv.ctypes.data_as(_D), rows, cols, eps)
    return out, inv


def rmsnorm_bwd(x, w, inv, g):
    """Returns (dx, dw) starting from zeros (tensor2.lua:641-666)."""
    x, px = _d(x); w, pw = _d(w); inv, pi = _d(inv); g, pg = _d(g)
    rows, cols = x.shape
    dx = np.zeros_like(x); dw = np.zeros(cols)
    lib().or_rmsnorm_bwd(px, pw, pi, pg, dx.ctypes.data_as(_D), dw.ctypes.data_as(_D), rows, cols)
    return dx, dw


def softmax_fwd(x, causal=False, offset=0):
    x, px = _d(x)
    rows, cols = x.shape
    y = np.zeros_like(x)
    lib().or_softmax_fwd(px, y.ctypes.data_as(_D), rows, cols, int(causal), offset)
    return y


def softmax_bwd(y, g, causal=False, offset=0):
    y, py = _d(y); g, pg = _d(g)
    rows, cols = y.shape
    dx = np.zeros_like(y)
    lib().or_softmax_bwd(py, pg, dx.ctypes.data_as(_D), rows, cols, int(causal), offset)
    return dx


def silu_fwd(x):
    x, px = _d(x)
    y = np.zeros_like(x); s = np.zeros_like(x)
    lib().or_silu_fwd(px, y.ctypes.data_as(_D), s.ctypes.data_as(_D), x.size)
    return y, s


def silu_bwd(x, sig, g):
    x, px = _d(x); sig, ps = _d(sig); g, pg = _d(g)
    dx = np.zeros_like(x)
    lib().or_silu_bwd(px, ps, pg, dx.ctypes.data_as(_D), x.size)
    return dx


def swiglu_fwd(gate, up):
    gate, pg = _d(gate); up, pu = _d(up)
    h = np.zeros_like(gate)
    lib().or_swiglu_fwd(pg, pu, h.ctypes.data_as(_D), gate.size)
    return h


def swiglu_bwd(gate, up, dh):
    gate, pg = _d(gate); up, pu = _d(up); dh, pd = _d(dh)
    dg = np.zeros_like(gate); du = np.zeros_like(gate)
    lib().or_swiglu_bwd(pg, pu, pd, dg.ctypes.data_as(_D), du.ctypes.data_as(_D), gate.size)
    return dg, du


def rope_angles(base, hd, maxpos):
    npairs = hd // 2
    c = np.zeros((maxpos + 1, npairs)); s = np.zeros((maxpos + 1, npairs))
    lib().or_rope_angles(base, hd, maxpos, c.ctypes.data_as(_D), s.ctypes.data_as(_D))
    return c, s


def rope_fwd(x, cosr, sinr, npairs=None):
    x, px = _d(x); cosr, pc = _d(cosr); sinr, ps = _d(sinr)
    rows, cols = x.shape
    npairs = cols // 2 if npairs is None else npairs
    assert cosr.shape[1] == npairs
    y = np.zeros_like(x)
    lib().or_rope_fwd(px, y.ctypes.data_as(_D), rows, cols, pc, ps, npairs)
    return y


def rope_bwd(g, cosr, sinr, npairs=None):
    g, pg = _d(g); cosr, pc = _d(cosr); sinr, ps = _d(sinr)
    rows, cols = g.shape
    npairs = cols // 2 if npairs is None else npairs
    dx = np.zeros_like(g)
    lib().or_rope_bwd(pg, dx.ctypes.data_as(_D), rows, cols, pc, ps, npairs)
    return dx


def rope_heads(x, heads, hd, row_stride=None, pos_offset=0, theta=10000.0,
               interleaved=False, inverse=False, pos_ids=None):
    """luaTL_rope contract in double; returns a rotated copy."""
    x = np.array(x, dtype=np.float64, copy=True, order="C")
    rows = x.shape[0]
    row_stride = x.shape[1] if row_stride is None else row_stride
    if pos_ids is not None:
        pid, pp = _i(pos_ids)
    else:
        pid, pp = None, _nul(_I)
    lib().or_rope_heads(x.ctypes.data_as(_D), pp, rows, heads, hd, row_stride, pos_offset,
                        theta, int(interleaved), int(inverse))
    return x


def cross_entropy(logits, tgt, ignore_index=None):
    """Tensor.cross_entropy (tensor2.lua:809-857); tgt 0-based. Returns (loss, sm, count)."""
    x, px = _d(logits); t, pt = _i(tgt)
    rows, cols = x.shape
    sm = np.zeros_like(x); cnt = ctypes.c_int(0)
    loss = lib().or_cross_entropy(px, pt, rows, cols, int(ignore_index is not None),
                                  int(ignore_index or 0), sm.ctypes.data_as(_D), ctypes.byref(cnt))
    return loss, sm, cnt.value


def cross_entropy_bwd(sm, tgt, count, g=1.0, ignore_index=None):
    sm, ps = _d(sm); t, pt = _i(tgt)
    rows, cols = sm.shape
    lg = np.zeros_like(sm)
    lib().or_cross_entropy_bwd(ps, pt, rows, cols, int(ignore_index is not None),
                               int(ignore_index or 0), g, count, lg.ctypes.data_as(_D))
    return lg


def ce_fused(logits, tgt, ignore_index=-1, gscale=1.0):
    """luaTL_cross_entropy contract: per-row losses and dlogits."""
    x, px = _d(logits); t, pt = _i(tgt)
    rows, V = x.shape
    losses = np.zeros(rows); d = np.zeros_like(x)
    lib().or_ce_fused(px, pt, losses.ctypes.data_as(_D), d.ctypes.data_as(_D), rows, V,
                      ignore_index, gscale)
    return losses, d


def argmax_rows(x):
    x, px = _d(x)
    rows, cols = x.shape
    out = np.zeros(rows, dtype=np.int32)
    lib().or_argmax_rows(px, out.ctypes.data_as(_I), rows, cols)
    return out


def embed_fwd(w, ids):
    w, pw = _d(w); ids, pi = _i(ids)
    out = np.zeros((ids.size, w.shape[1]))
    lib().or_embed_fwd(pw, pi, out.ctypes.data_as(_D), ids.size, w.shape[1])
    return out


def embed_bwd(g, ids, vocab, scale=1.0):
    g, pg = _d(g); ids, pi = _i(ids)
    wg = np.zeros((vocab, g.shape[1]))
    lib().or_embed_bwd(pg, pi, wg.ctypes.data_as(_D), ids.size, g.shape[1], scale)
    return wg


def grad_norm(g):
    g, pg = _d(g)
    return lib().or_grad_norm(pg, g.size)


def sgd_step(p, g, v, lr, momentum=0.0, wd=0.0, nesterov=False):
    """In place on float64 arrays p and v (optim2.lua:72-99)."""
    assert p.dtype == np.float64 and v.dtype == np.float64
    g, pg = _d(g)
    lib().or_sgd_step(p.ctypes.data_as(_D), pg, v.ctypes.data_as(_D), p.size, lr, momentum,
                      wd, int(nesterov))


def adamw_step(p, g, m, v, t, lr, beta1=0.9, beta2=0.95, eps=1e-8, wd=0.01):
    """In place on float64 p, m, v; t is the already advanced step count
    (optim2.lua:116-147)."""
    for a in (p, m, v):
        assert a.dtype == np.float64
    g, pg = _d(g)
    lib().or_adamw_step(p.ctypes.data_as(_D), pg, m.ctypes.data_as(_D), v.ctypes.data_as(_D), p.size,
                        lr, beta1, beta2, eps, wd, int(t))


# ---------------------------------------------------------------- LMTrain step
def lm_cfg(vocab, dim, layers, heads, ffn, causal=True, eps=1e-5, rope_base=10000.0):
    return LmCfg(vocab, dim, layers, heads, ffn, int(causal), eps, rope_base)


def lm_num_params(cfg):
    return lib().or_lm_num_params(ctypes.byref(cfg))


def lm_param_table(cfg):
    """[(name, offset, rows, cols)] in Transformer:parameters() order."""
    n = 2 + 9 * cfg.layers
    offs = (ctypes.c_long * n)(); rows = (ctypes.c_int * n)(); cols = (ctypes.c_int * n)()
    lib().or_lm_param_offsets(ctypes.byref(cfg), offs, rows, cols)
    names = ["emb"]
    for l in range(cfg.layers):
        names += [f"{nm}.{l}" for nm in ("ln1", "wq", "wk", "wv", "wo", "ln2", "w1", "w3", "w2")]
    names.append("lnf")
    return [(names[i], offs[i], rows[i], cols[i]) for i in range(n)]


def lm_window(cfg, params, ids, tgt, grads=None):
    """One window fwd+bwd; returns (loss, grads (accumulated), logits, correct)."""
    params, pp = _d(params)
    ids, pi = _i(ids); tgt, pt = _i(tgt)
    T = ids.size
    if grads is None:
        grads = np.zeros(params.size)
    logits = np.zeros((T, cfg.vocab))
    corr = ctypes.c_int(0)
    loss = lib().or_lm_window(ctypes.byref(cfg), pp, pi, pt, T, grads.ctypes.data_as(_D),
                              logits.ctypes.data_as(_D), ctypes.byref(corr))
    return loss, grads, logits, corr.value


def _ragged(ids, lens, nwin):
    B, T = ids.shape
    nwin = B if nwin is None else int(nwin)
    assert 1 <= nwin <= B
    if lens is None:
        return nwin, None, _nul(_I)
    lens, pl = _i(lens)
    assert lens.size >= nwin and np.all((lens[:nwin] >= 1) & (lens[:nwin] <= T))
    return nwin, lens, pl


def lm_step_sgd(cfg, params, vel, ids, tgt, lr, momentum=0.9, wd=0.01, clip_norm=1.0, lens=None, nwin=None):
    """One LMTrain batch step (optimizer="sgd"); params/vel float64 updated in place.

    ids/tgt are (B, T) 0-based; windows b < nwin (default B), window b holding
    lens[b] tokens (default T).  Returns dict(losses, gnorm, correct, grads, applied).
    """
    assert params.dtype == np.float64 and vel.dtype == np.float64
    ids, pi = _i(ids); tgt, pt = _i(tgt)
    B, T = ids.shape
    nwin, lens_keep, pl = _ragged(ids, lens, nwin)
    losses = np.zeros(B); grads = np.zeros(params.size)
    gn = ctypes.c_double(0); corr = ctypes.c_int(0)
    applied = lib().or_lm_step_sgd_ex(ctypes.byref(cfg), params.ctypes.data_as(_D),
                                      vel.ctypes.data_as(_D), pi, pt, nwin, T, pl, lr, momentum, wd,
                                      clip_norm, losses.ctypes.data_as(_D), ctypes.byref(gn),
                                      ctypes.byref(corr), grads.ctypes.data_as(_D))
    return dict(losses=losses, gnorm=gn.value, correct=corr.value, grads=grads,
                applied=bool(applied))


def lm_step_adamw(cfg, params, m, v, t, ids, tgt, lr, beta1=0.9, beta2=0.95, eps=1e-8, wd=0.01,
                  clip_norm=1.0, lens=None, nwin=None):
    """One LMTrain batch step (optimizer="adamw"); params, m, v float64 updated in
    place.  t is the AdamW step count before the call; lens/nwin as lm_step_sgd.
    Returns dict(losses, gnorm, correct, grads, applied, t) with t advanced when
    the step applied."""
    for a in (params, m, v):
        assert a.dtype == np.float64
    ids, pi = _i(ids); tgt, pt = _i(tgt)
    B, T = ids.shape
    nwin, lens_keep, pl = _ragged(ids, lens, nwin)
    losses = np.zeros(B); grads = np.zeros(params.size)
    gn = ctypes.c_double(0); corr = ctypes.c_int(0); tc = ctypes.c_int(int(t))
    applied = lib().or_lm_step_adamw_ex(ctypes.byref(cfg), params.ctypes.data_as(_D), m.ctypes.data_as(_D),
                                        v.ctypes.data_as(_D), ctypes.byref(tc), pi, pt, nwin, T, pl, lr, beta1,
                                        beta2, eps, wd, clip_norm, losses.ctypes.data_as(_D),
                                        ctypes.byref(gn), ctypes.byref(corr), grads.ctypes.data_as(_D))
    return dict(losses=losses, gnorm=gn.value, correct=corr.value, grads=grads,
                applied=bool(applied), t=tc.value)


# ---------------------------------------------------------------- luaTL operation set
# The reference GPU path's kernels restated in double (oracle.c, "The luaTL
# operation set"); the adapter's resident calls and Program ops are checked
# against these.
EW = {"COPY": 0, "ADD": 1, "SUB": 2, "MUL": 3, "DIV": 4, "SCALE": 5, "AXPY": 6, "FILL": 7, "RELU": 8,
      "GELU": 9, "SILU": 10, "TANH": 11, "SIGMOID": 12, "EXP": 13, "SQRT": 14, "RSQRT": 15, "NEG": 16,
      "RECIP": 17, "ABS": 18, "CLAMP": 19, "DRELU": 20, "DSILU": 21, "DGELU": 22}


def ew(op, a, b, alpha=1.0, beta=0.0, n=None):
    """luaTL_elementwise's operator table (cuda/luaTL_core.cu:909-934); a/b may be None."""
    if isinstance(op, str):
        op = EW[op]
    ref = a if a is not None else b
    n = int(np.size(ref)) if n is None else n
    pa = pb = _nul(_D)
    if a is not None:
        a, pa = _d(a)
    if b is not None:
        b, pb = _d(b)
    c = np.empty(n)
    lib().or_ew(op, pa, pb, c.ctypes.data_as(_D), n, alpha, beta)
    return c if ref is None else c.reshape(np.shape(ref))


def gemm_ex(A, B, C, M, N, K, strides, batch=1, alpha=1.0, beta=0.0, eps=1e-5, pre=0, act=0, bias=None,
            gamma=None, rowscale=None):
    """luaTL_gemm_ex_kernel (cuda/luaTL_train.cu:127-234) on flat float64 buffers;
    strides = (a_rs, a_cs, b_rs, b_cs, c_rs, c_cs, a_bs, b_bs, c_bs).  C is updated in place."""
    A, pA = _d(A); B, pB = _d(B)
    assert C.dtype == np.float64 and C.flags.c_contiguous
    keep, ptrs = [], []
    for v in (bias, gamma, rowscale):
        if v is None:
            ptrs.append(_nul(_D))
        else:
            v, p = _d(v)
            keep.append(v)
            ptrs.append(p)
    lib().or_gemm_ex(pA, pB, C.ctypes.data_as(_D), ptrs[0], ptrs[1], ptrs[2], M, N, K, *strides, batch, alpha,
                     beta, eps, pre, act)
    return C


def softmax_ex(x, bias=None, scale=1.0, causal=False, group=0, moff=0):
    """luaTL_softmax_ex_kernel (cuda/luaTL_train.cu:545-585)."""
    x, px = _d(x)
    rows, cols = x.shape
    y = np.empty_like(x)
    pb = _nul(_D)
    if bias is not None:
        bias, pb = _d(bias)
    lib().or_softmax_ex(px, pb, y.ctypes.data_as(_D), rows, cols, scale, int(causal), group, moff)
    return y


def softmax_bwd_ex(y, dy, scale=1.0, causal=False, group=0, moff=0):
    """luaTL_softmax_bwd_kernel (cuda/luaTL_train.cu:589-619)."""
    y, py = _d(y); dy, pdy = _d(dy)
    rows, cols = y.shape
    dx = np.empty_like(y)
    lib().or_softmax_bwd_ex(py, pdy, dx.ctypes.data_as(_D), rows, cols, scale, int(causal), group, moff)
    return dx


def rmsnorm_bwd_luatl(x, g, dy, eps, dgamma=None):
    """luaTL_rmsnorm_bwd_kernel (cuda/luaTL_train.cu:489-526): returns dx; dgamma (float64,
    may be None) accumulates."""
    x, px = _d(x); dy, pdy = _d(dy)
    rows, cols = x.shape
    pg = _nul(_D)
    if g is not None:
        g, pg = _d(g)
    dx = np.empty_like(x)
    pdg = _nul(_D)
    if dgamma is not None:
        assert dgamma.dtype == np.float64 and dgamma.flags.c_contiguous
        pdg = dgamma.ctypes.data_as(_D)
    lib().or_rmsnorm_bwd_luatl(px, pg, pdy, dx.ctypes.data_as(_D), pdg, rows, cols, eps)
    return dx


def adamw_luatl(w, g, m, v, step, lr=1e-3, b1=0.9, b2=0.999, eps=1e-8, wd=0.0, clip=0.0):
    """luaTL_adamw_kernel (cuda/luaTL_core.cu:1346-1380), in place on float64 w, m, v."""
    for a in (w, m, v):
        assert a.dtype == np.float64 and a.flags.c_contiguous
    g, pg = _d(g)
    lib().or_adamw_luatl(w.ctypes.data_as(_D), pg, m.ctypes.data_as(_D), v.ctypes.data_as(_D), w.size, step,
                         lr, b1, b2, eps, wd, clip)


def reduce_cols(x, out, alpha=1.0, beta=0.0, rs=None):
    """luaTL_reduce_cols_kernel (cuda/luaTL_train.cu:895-906), out updated in place."""
    x, px = _d(x)
    rows, cols = x.shape
    assert out.dtype == np.float64 and out.flags.c_contiguous
    lib().or_reduce_cols(px, out.ctypes.data_as(_D), rows, cols, cols if rs is None else rs, alpha, beta)
    return out


def clip_by_nsq(x, nsq, max_norm):
    """luaTL_clip_kernel (cuda/luaTL_train.cu:947-965), in place on float64 x."""
    assert x.dtype == np.float64 and x.flags.c_contiguous
    lib().or_clip_by_nsq(x.ctypes.data_as(_D), x.size, nsq, max_norm)
    return x
