"""Float64 torch.autograd statement of the CPU Transformer (ai/nn/transformer.lua:196-257).

Independent of the oracle's hand-derived backward: the gradients here come
from torch's autograd, so agreement pins the oracle's BACKWARD restatement.
Runs on the CPU only (no GPU use).
"""
import math

import numpy as np
import torch


def forward_loss(cfg, params, ids, tgt):
    """params: list of float64 leaf tensors in Transformer:parameters() order."""
    V, D, L, H, F = cfg.vocab, cfg.dim, cfg.layers, cfg.heads, cfg.ffn
    hd = D // H
    npairs = hd // 2
    T = len(ids)
    it = iter(params)
    emb = next(it)
    layers = []
    for _ in range(L):
        layers.append([next(it) for _ in range(9)])
    lnf = next(it)

    inv = torch.tensor([1.0 / (cfg.rope_base ** ((2 * k) / hd)) for k in range(npairs)],
                       dtype=torch.float64)
    pos = torch.arange(T, dtype=torch.float64)
    ang = pos[:, None] * inv[None, :]
    cs, sn = torch.cos(ang), torch.sin(ang)

    def rms(x, w):
        r = 1.0 / torch.sqrt((x * x).sum(1, keepdim=True) / x.shape[1] + cfg.eps)
        return x * r * w

    def rope(x):  # interleaved pairs (2k, 2k+1)
        x0, x1 = x[:, 0::2][:, :npairs], x[:, 1::2][:, :npairs]
        y0 = x0 * cs - x1 * sn
        y1 = x0 * sn + x1 * cs
        out = torch.stack([y0, y1], dim=2).reshape(T, 2 * npairs)
        if x.shape[1] > 2 * npairs:
            out = torch.cat([out, x[:, 2 * npairs:]], 1)
        return out

    mask = torch.tril(torch.ones(T, T, dtype=torch.bool))
    x = emb[torch.as_tensor(ids, dtype=torch.long)]
    for (ln1, wq, wk, wv, wo, ln2, w1, w3, w2) in layers:
        h = rms(x, ln1)
        q, k, v = h @ wq, h @ wk, h @ wv
        outs = []
        for hh in range(H):
            sl = slice(hh * hd, (hh + 1) * hd)
            qh, kh = rope(q[:, sl]), rope(k[:, sl])
            sc = (qh @ kh.T) * (1.0 / math.sqrt(hd))
            if cfg.causal:
                sc = sc.masked_fill(~mask, float("-inf"))
            pr = torch.softmax(sc, dim=1)
            outs.append(pr @ v[:, sl])
        x = x + torch.cat(outs, 1) @ wo
        h2 = rms(x, ln2)
        g = h2 @ w1
        x = x + (torch.nn.functional.silu(g) * (h2 @ w3)) @ w2
    xf = rms(x, lnf)
    logits = xf @ emb.T
    loss = torch.nn.functional.cross_entropy(logits, torch.as_tensor(tgt, dtype=torch.long))
    return loss, logits


def window_grad(cfg, flat_params, table, ids, tgt):
    """Loss and flat gradient for one window via autograd."""
    ps = []
    for (_, off, r, c) in table:
        t = torch.tensor(flat_params[off:off + r * c].reshape(r, c), dtype=torch.float64,
                         requires_grad=True)
        ps.append(t)
    loss, logits = forward_loss(cfg, ps, ids, tgt)
    loss.backward()
    g = np.concatenate([p.grad.numpy().ravel() for p in ps])
    return loss.item(), g, logits.detach().numpy()
