"""The CPU LMTrain step (optimizer "sgd" or "adamw") run on the GPU through lhip_lm_*.

Host-side mirror of the parts of ai/optim/lmtrain.lua that feed one optimizer
step: ``build_windows`` (lmtrain.lua:535-558) cuts token sequences into
(input, target) windows, and ``GpuLMStep.step`` / ``step_adamw`` run the batch
body of LMTrain:run (lmtrain.lua:1183-1227) for ``batch`` windows: forward,
mean CE per window, backward, grads scaled by 1/batch, global-norm skip and
clip, and the SGD (optim2.lua:48-102) or AdamW (optim2.lua:104-164) update,
all on the device.  ``save_checkpoint`` / ``load_checkpoint`` and
``GpuLMStep.save`` / ``load`` read and write the lmio v3 checkpoint format
(ai/optim/lmio.lua).  Ids are 0-based here (Lua's are 1-based).

Batches may be ragged as LMTrain's are: ``pack_windows`` lays out up to
``batch`` windows of up to ``seq`` tokens each (the short trailing window that
build_windows cuts at a sequence's end, and the short last batch of an epoch)
for ``GpuLMStep.set_batch``.  Each window's loss is the mean over its own
tokens and the summed gradients are scaled by 1/n_in_batch, as in
lmtrain.lua:1183-1212.
"""
import ctypes

import numpy as np

from . import device
from ._lib import LmConfig, LmStats, call, lib

PARAM_NAMES_PER_LAYER = ("ln1", "wq", "wk", "wv", "wo", "ln2", "w1", "w3", "w2")


def build_windows(sequences, max_seq, stride=None):
    """[(inp, tgt, n)] exactly as lmtrain.lua:535-558 (0-based lists)."""
    stride = stride or max_seq
    windows = []
    for seq in sequences:
        n_tok = len(seq)
        start = 0
        while start < n_tok - 1:
            stop = min(start + max_seq, n_tok - 1)
            inp = list(seq[start:stop])
            tgt = list(seq[start + 1:stop + 1])
            if inp:
                windows.append((inp, tgt, len(inp)))
            if stop >= n_tok - 1:
                break
            start += stride
    return windows


def pack_windows(windows, batch, seq):
    """Lay out up to `batch` windows [(inp, tgt, n)] (build_windows' tuples) as
    (ids, targets, lengths, n_windows) for GpuLMStep.set_batch: window b at row
    b, its n tokens first, the rest of the row and the unused rows zero."""
    if not 1 <= len(windows) <= batch:
        raise ValueError(f"{len(windows)} windows for a batch of {batch}")
    ids = np.zeros((batch, seq), np.int32)
    tgt = np.zeros((batch, seq), np.int32)
    lens = np.zeros(batch, np.int32)
    for b, (inp, out, n) in enumerate(windows):
        if not 1 <= n <= seq or len(inp) < n or len(out) < n:
            raise ValueError(f"window {b}: {n} tokens, expected 1..{seq}")
        ids[b, :n] = inp[:n]
        tgt[b, :n] = out[:n]
        lens[b] = n
    return ids, tgt, lens, len(windows)


def config(vocab, dim, layers, heads, ffn, batch, seq, causal=True, eps=1e-5, rope_base=10000.0):
    return LmConfig(vocab, dim, layers, heads, ffn, int(bool(causal)), eps, rope_base, batch, seq)


def param_table(cfg):
    """[(name, offset, rows, cols)] in Transformer:parameters() order."""
    n = 2 + 9 * cfg.layers
    offs = (ctypes.c_longlong * n)()
    rows = (ctypes.c_int * n)()
    cols = (ctypes.c_int * n)()
    call("lhip_lm_param_offsets", ctypes.byref(cfg), offs, rows, cols)
    names = ["emb"] + [f"{p}.{l}" for l in range(cfg.layers) for p in PARAM_NAMES_PER_LAYER] + ["lnf"]
    return [(names[i], offs[i], rows[i], cols[i]) for i in range(n)]


def num_params(cfg):
    n = lib().lhip_lm_num_params(ctypes.byref(cfg))
    if n < 0:
        raise ValueError("invalid LM config")
    return n


def init_params(cfg, rng, std=0.02):
    """All weight matrices N(0, std), RMSNorm gains 1 (the synthetic C2 init)."""
    p = np.zeros(num_params(cfg), dtype=np.float32)
    for name, off, r, c in param_table(cfg):
        if name.startswith(("ln1", "ln2", "lnf")):
            p[off:off + r * c] = 1.0
        else:
            p[off:off + r * c] = rng.normal(0.0, std, r * c)
    return p


def _ckpt_info(fmt="bin", keep=1, epoch=0, loss=float("nan"), best_loss=float("nan"), backend=None, extra=None):
    from ._lib import CkptInfo
    if fmt not in ("bin", "text"):
        raise ValueError("format must be 'bin' or 'text'")
    return CkptInfo(0 if fmt == "bin" else 1, int(keep), int(epoch), float(loss), float(best_loss),
                    backend.encode() if backend else None, extra.encode() if extra else None)


def _ckpt_header_dict(h):
    return {"version": h.version, "format": "bin" if h.format == 0 else "text",
            "dtype": "f32" if h.dtype_bytes == 4 else "f64", "epoch": h.epoch, "loss": h.loss,
            "best_loss": h.best_loss, "causal": h.causal, "tie": h.tie, "max_seq": h.max_seq,
            "rope_base": h.rope_base}


def save_checkpoint(path, cfg, params, **info):
    """Write the flat parameter vector in the lmio v3 checkpoint format
    (ai/optim/lmio.lua; host side, no device).  info: fmt ('bin'|'text'), keep,
    epoch, loss, best_loss, backend, extra."""
    p = np.ascontiguousarray(params, dtype=np.float32).reshape(-1)
    ci = _ckpt_info(**info)
    call("lhip_ckpt_save_host", str(path).encode(), ctypes.byref(cfg), ctypes.byref(ci), p.ctypes.data, p.size)


def load_checkpoint(path, cfg):
    """Read an lmio checkpoint (v1/v2/v3, bin/text, f32/f64) into a flat fp32
    vector for cfg; returns (params, header dict)."""
    from ._lib import CkptHeader
    out = np.empty(num_params(cfg), dtype=np.float32)
    h = CkptHeader()
    call("lhip_ckpt_load_host", str(path).encode(), ctypes.byref(cfg), out.ctypes.data, out.size, ctypes.byref(h))
    return out, _ckpt_header_dict(h)


class GpuLMStep:
    """Device-resident model + optimizer state (SGD or AdamW) for one LMTrain configuration."""

    def __init__(self, vocab, dim, layers, heads, ffn, batch, seq, causal=True, eps=1e-5, rope_base=10000.0):
        device.init(0)
        self.cfg = config(vocab, dim, layers, heads, ffn, batch, seq, causal, eps, rope_base)
        self.batch, self.seq = batch, seq
        self.n = num_params(self.cfg)
        self._h = ctypes.c_void_p()
        call("lhip_lm_create", ctypes.byref(self.cfg), ctypes.byref(self._h))

    # -- state ---------------------------------------------------------------
    def _vec(self, name, arr=None):
        if arr is None:
            out = np.empty(self.n, dtype=np.float32)
            call(name, self._h, out.ctypes.data, self.n)
            return out
        a = np.ascontiguousarray(arr, dtype=np.float32).reshape(-1)
        if a.size != self.n:
            raise ValueError(f"{a.size} values given, model has {self.n}")
        call(name, self._h, a.ctypes.data, self.n)
        return None

    def set_params(self, p):
        self._vec("lhip_lm_set_params", p)

    def params(self):
        return self._vec("lhip_lm_get_params")

    def grads(self):
        return self._vec("lhip_lm_get_grads")

    def set_velocity(self, v):
        self._vec("lhip_lm_set_velocity", v)

    def velocity(self):
        return self._vec("lhip_lm_get_velocity")

    def set_batch(self, ids, targets, lengths=None, n_windows=None):
        """(batch, seq) ids and targets; optionally each window's token count
        (`lengths`, tokens first in its row) and the number of windows used
        (`n_windows`), for LMTrain's short last window and short last batch."""
        ids = np.ascontiguousarray(ids, dtype=np.int32).reshape(-1)
        tgt = np.ascontiguousarray(targets, dtype=np.int32).reshape(-1)
        if ids.size != self.batch * self.seq or tgt.size != ids.size:
            raise ValueError(f"expected {self.batch}x{self.seq} ids and targets")
        if lengths is None and n_windows is None:
            call("lhip_lm_set_batch", self._h, ids.ctypes.data, tgt.ctypes.data)
            return
        nw = self.batch if n_windows is None else int(n_windows)
        lens = None if lengths is None else np.ascontiguousarray(lengths, dtype=np.int32).reshape(-1)
        if lens is not None and lens.size < nw:
            raise ValueError(f"{lens.size} lengths for {nw} windows")
        call("lhip_lm_set_batch_ex", self._h, ids.ctypes.data, tgt.ctypes.data,
             None if lens is None else lens.ctypes.data, nw)

    def use_graph(self, on=True):
        call("lhip_lm_use_graph", self._h, int(bool(on)))

    # -- the step --------------------------------------------------------------
    def step(self, lr, momentum=0.9, weight_decay=0.01, clip_norm=1.0, nesterov=False):
        """Enqueue one SGD step (asynchronous; stats() waits)."""
        call("lhip_lm_step_sgd", self._h, float(lr), float(momentum), float(weight_decay),
             float(clip_norm), int(bool(nesterov)))

    def step_adamw(self, lr=1e-3, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.01, clip_norm=1.0):
        """Enqueue one AdamW step (LMTrain's default optimizer; asynchronous)."""
        call("lhip_lm_step_adamw", self._h, float(lr), float(beta1), float(beta2), float(eps),
             float(weight_decay), float(clip_norm))

    def set_adam_state(self, m=None, v=None, step=0):
        arrs = []
        for a in (m, v):
            if a is None:
                arrs.append(None)
                continue
            a = np.ascontiguousarray(a, dtype=np.float32).reshape(-1)
            if a.size != self.n:
                raise ValueError(f"{a.size} values given, model has {self.n}")
            arrs.append(a)
        call("lhip_lm_set_adam_state", self._h, None if arrs[0] is None else arrs[0].ctypes.data,
             None if arrs[1] is None else arrs[1].ctypes.data, self.n, int(step))

    def save(self, path, **info):
        """Checkpoint the device parameters (lmio v3; see save_checkpoint for info)."""
        ci = _ckpt_info(**info)
        call("lhip_lm_save", self._h, str(path).encode(), ctypes.byref(ci))

    def load(self, path):
        """Load a checkpoint into the device parameters; returns its header dict."""
        from ._lib import CkptHeader
        h = CkptHeader()
        call("lhip_lm_load", self._h, str(path).encode(), ctypes.byref(h))
        return _ckpt_header_dict(h)

    def adam_state(self):
        """(m, v, step) of the AdamW optimizer."""
        m = np.empty(self.n, dtype=np.float32); v = np.empty(self.n, dtype=np.float32)
        t = ctypes.c_int(0)
        call("lhip_lm_get_adam_state", self._h, m.ctypes.data, v.ctypes.data, self.n, ctypes.byref(t))
        return m, v, int(t.value)

    def stats(self):
        st = LmStats()
        wl = np.zeros(self.batch, dtype=np.float32)
        call("lhip_lm_stats", self._h, ctypes.byref(st), wl.ctypes.data, self.batch)
        return {"loss": float(st.loss), "window_losses": wl.astype(np.float64), "grad_norm": float(st.grad_norm),
                "applied": bool(st.applied), "correct": int(st.correct), "steps": int(st.steps)}

    def argmax(self):
        out = np.empty(self.batch * self.seq, dtype=np.int32)
        call("lhip_lm_get_argmax", self._h, out.ctypes.data, out.size)
        return out

    def close(self):
        if self._h is not None and self._h.value:
            lib().lhip_lm_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
