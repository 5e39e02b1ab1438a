"""GPU parity of the device-resident LMTrain SGD step against the CPU oracle.

The oracle (oracle.c: or_lm_step_sgd) restates ai/optim/lmtrain.lua:1183-1227
with optimizer "sgd" over ai/nn/transformer.lua in double precision; it is
pinned against float64 torch autograd and finite differences in
tests/test_oracle.py.  Both sides get identical fp32-representable
parameters, ids and targets.

Bars: per-window CE losses within 1e-5 absolute (north star), gradients and
the parameter update within a relative Frobenius error of 1e-4, the global
norm within 1e-5 relative, argmax indices bit-exact against the oracle's
argmax of the GPU's own logits.  lr is explicit (the cosine schedule gives
lr = 0 for a one-step run, lmtrain.lua:1036-1052).
"""
import numpy as np
import pytest

import oracle as O
from lanternl_amd import lmtrain
from tests.gpu_util import announce, rel_fro

pytestmark = pytest.mark.gpu


def _run_case(V, D, L, H, F, B, T, steps, lr, std, seed, graph=False, clip=1.0, mom=0.9, wd=0.01, causal=True,
              id_hi=None):
    rng = np.random.default_rng(seed)
    cfg = O.lm_cfg(V, D, L, H, F, causal=causal)
    gpu = lmtrain.GpuLMStep(V, D, L, H, F, B, T, causal=causal)
    p32 = lmtrain.init_params(gpu.cfg, rng, std)
    gpu.set_params(p32)
    if graph:
        gpu.use_graph(True)
    results = []
    for _ in range(steps):
        ids = rng.integers(0, id_hi or V, (B, T)).astype(np.int32)
        tgt = rng.integers(0, V, (B, T)).astype(np.int32)
        gpu.set_batch(ids, tgt)
        # the oracle starts every step from the GPU's own state (no drift between the sides)
        p_before = gpu.params().astype(np.float64)
        v_before = gpu.velocity().astype(np.float64)
        gpu.step(lr, mom, wd, clip)
        st = gpu.stats()
        p_ref, v_ref = p_before.copy(), v_before.copy()
        ref = O.lm_step_sgd(cfg, p_ref, v_ref, ids, tgt, lr, mom, wd, clip)
        results.append((st, ref, p_before, gpu.params().astype(np.float64), gpu.grads().astype(np.float64),
                        gpu.velocity().astype(np.float64), p_ref, v_ref))
    return gpu, results


def _check(results, loss_tol=1e-5):
    for st, ref, before, after, grads, vel, p_ref, v_ref in results:
        assert st["applied"] == ref["applied"]
        assert np.max(np.abs(st["window_losses"] - ref["losses"])) <= loss_tol
        assert abs(st["loss"] - ref["losses"].mean()) <= loss_tol
        assert abs(st["grad_norm"] - ref["gnorm"]) <= 1e-5 * ref["gnorm"]
        assert rel_fro(grads, ref["grads"]) <= 1e-4
        assert rel_fro(after - before, p_ref - before) <= 1e-4
        assert rel_fro(vel, v_ref) <= 1e-4


def test_lm_step_tiny_three_steps():
    """V=32 D=16 L=1 H=2 F=32, B=2 windows of T=8: three chained SGD steps."""
    announce("lm tiny")
    gpu, res = _run_case(32, 16, 1, 2, 32, 2, 8, steps=3, lr=0.1, std=0.3, seed=1)
    _check(res)
    gpu.close()


def test_lm_step_two_layers_clip_active():
    """Larger weights so the global norm exceeds clip_norm = 1 and the clip scales the grads."""
    announce("lm clip")
    gpu, res = _run_case(64, 32, 2, 4, 64, 3, 16, steps=2, lr=0.05, std=0.5, seed=2)
    assert res[0][1]["gnorm"] > 1.0
    _check(res)
    gpu.close()


def test_lm_step_eight_layers_weight_gradient_batches():
    """Eight layers: the deferred weight gradients (1 + 7 x 8 products, 17
    norm-gain column sums) exceed one grouped launch and one column-sum launch,
    so they are issued in several batches."""
    announce("lm 8 layers")
    gpu, res = _run_case(40, 16, 8, 2, 32, 2, 8, steps=2, lr=0.1, std=0.3, seed=6)
    _check(res)
    gpu.close()


@pytest.mark.parametrize("D,H,T", [(12, 2, 7), (16, 2, 7), (24, 2, 12), (64, 2, 20), (96, 2, 36), (128, 2, 64)])
def test_lm_step_attention_load_paths(D, H, T):
    """The fused attention's operand loads: float4 (head_dim and T multiples of
    4), float4 forward with element-wise backward (T = 7), and element-wise
    both ways (head_dim 6); the one-wave forward over one to four 16-wide
    head-dimension groups (head_dim 12 (partial group), 32, 48 and 64)."""
    announce("lm attention loads", D, H, T)
    gpu, res = _run_case(30, D, 1, H, 2 * D, 2, T, steps=1, lr=0.1, std=0.3, seed=7 + D + T)
    _check(res)
    gpu.close()


@pytest.mark.parametrize("D,H", [(32, 2), (12, 2)])
def test_lm_step_non_causal(D, H):
    """Non-causal attention over T = 40 (three 16-row blocks, the last ragged):
    every key block is visible from every query block, so the backward's dq
    and dk/dv jobs each sum shares from all three waves; float4 (head_dim 16)
    and element-wise (head_dim 6) loads."""
    announce("lm non-causal", D, H)
    gpu, res = _run_case(30, D, 1, H, 2 * D, 2, 40, steps=1, lr=0.1, std=0.3, seed=11 + D, causal=False)
    _check(res)
    gpu.close()


def test_lm_step_config_c2():
    """Config C2: vocab 2000, dim 128, 4 layers, 8 heads (hd 16), ffn 256, batch 8 x seq 64,
    weights N(0, 0.02); one SGD step (lr 0.1, momentum 0.9, wd 0.01, clip 1)."""
    announce("lm C2")
    gpu, res = _run_case(2000, 128, 4, 8, 256, 8, 64, steps=1, lr=0.1, std=0.02, seed=3)
    _check(res)
    st, ref = res[0][0], res[0][1]
    # near-uniform logits at init: loss ~ ln V
    assert abs(st["loss"] - np.log(2000)) < 0.05
    assert ref["applied"]
    gpu.close()


@pytest.mark.parametrize("B,id_hi", [(16, 40), (8, 2000), (16, 2000)])
def test_lm_step_c2_embedding_scatter(B, id_hi):
    """C2's dimensions, where the last grouped weight-gradient launch also
    scatters dx_0 into the tied table's rows and leaves the squared-norm
    partials: ids crowded into 40 rows (hundreds of tokens per 32-row block,
    past the first batch of matches) and 16 windows (1024 tokens, two listing
    rounds), as well as spread ids at 512 and 1024 tokens."""
    announce("lm C2 scatter", B, id_hi)
    gpu, res = _run_case(2000, 128, 4, 8, 256, B, 64, steps=2, lr=0.1, std=0.02, seed=31 + B + id_hi,
                         id_hi=id_hi)
    _check(res)
    gpu.close()


@pytest.mark.parametrize("B,T", [(8, 60), (9, 60)])
def test_lm_step_c2_token_counts_off_the_chunk_grid(B, T):
    """C2's dimensions with 480 and 540 tokens: the grouped weight-gradient
    launch (224 tiles of 64x64) reduces over K = 480 on two wave sets of
    64-deep chunks (7.5 chunks) and K = 540 on four sets of 32-deep chunks
    (16.9), so its last chunk is partial and every load past K, including the
    loads issued beyond the last chunk, must read zeros."""
    announce("lm C2 tokens", B, T)
    gpu, res = _run_case(2000, 128, 4, 8, 256, B, T, steps=2, lr=0.1, std=0.02, seed=71 + B)
    _check(res)
    gpu.close()


def _random_configs(seed, count):
    rng = np.random.default_rng(seed)
    for _ in range(count):
        H = int(rng.choice([1, 2, 3, 4, 8]))
        hd = 2 * int(rng.integers(1, 49))
        F = int(rng.integers(1, 97)) * 4 if rng.uniform() < 0.75 else int(rng.integers(3, 300))
        yield dict(V=int(rng.integers(5, 3000)), D=H * hd, H=H, F=F, L=int(rng.integers(1, 4)),
                   B=int(rng.integers(1, 11)), T=int(rng.integers(1, 81)), causal=bool(rng.integers(2)))


@pytest.mark.parametrize("i,cfg", list(enumerate(_random_configs(2024, 12))))
def test_lm_step_random_configurations(i, cfg):
    """Seeded random shapes away from the hand-picked ones: any head count
    and even head_dim up to 96, ffn widths that are not multiples of 4 (a
    quarter of the draws), any vocabulary, 1-3 layers, 1-10 windows of 1-80
    tokens, causal or not; two SGD steps each against the oracle."""
    announce("lm random", i, cfg)
    c = cfg
    gpu, res = _run_case(c["V"], c["D"], c["L"], c["H"], c["F"], c["B"], c["T"], steps=2, lr=0.1, std=0.02,
                         seed=500 + i, causal=c["causal"])
    _check(res)
    gpu.close()


def test_lm_argmax_and_correct_count_bit_exact():
    announce("lm argmax")
    V, D, L, H, F, B, T = 50, 16, 1, 2, 32, 2, 8
    rng = np.random.default_rng(4)
    cfg = O.lm_cfg(V, D, L, H, F)
    gpu = lmtrain.GpuLMStep(V, D, L, H, F, B, T)
    p = lmtrain.init_params(gpu.cfg, rng, 0.5)
    gpu.set_params(p)
    ids = rng.integers(0, V, (B, T)).astype(np.int32)
    tgt = rng.integers(0, V, (B, T)).astype(np.int32)
    gpu.set_batch(ids, tgt)
    gpu.step(0.0, 0.0, 0.0, 0.0)
    st = gpu.stats()
    am = gpu.argmax().reshape(B, T)
    correct = 0
    for b in range(B):
        _, _, logits, corr = O.lm_window(cfg, p.astype(np.float64), ids[b], tgt[b])
        assert np.array_equal(am[b], O.argmax_rows(logits))
        correct += corr
    assert st["correct"] == correct
    gpu.close()


def test_lm_graph_replay_matches_eager_every_step():
    """hipGraph replay of the step gives bit-identical parameters to eager
    launches, checked after every replay with eager work in between."""
    announce("lm graph")
    V, D, L, H, F, B, T = 2000, 128, 2, 8, 256, 4, 64
    rng = np.random.default_rng(5)
    eager = lmtrain.GpuLMStep(V, D, L, H, F, B, T)
    graph = lmtrain.GpuLMStep(V, D, L, H, F, B, T)
    p = lmtrain.init_params(eager.cfg, rng, 0.02)
    eager.set_params(p)
    graph.set_params(p)
    graph.use_graph(True)
    for s in range(4):
        ids = rng.integers(0, V, (B, T)).astype(np.int32)
        tgt = rng.integers(0, V, (B, T)).astype(np.int32)
        eager.set_batch(ids, tgt)
        graph.set_batch(ids, tgt)
        lr = 0.1 / (s + 1)                      # hyper-parameters change between replays
        eager.step(lr)
        graph.step(lr)
        se, sg = eager.stats(), graph.stats()
        assert se["loss"] == sg["loss"] and se["grad_norm"] == sg["grad_norm"]
        assert np.array_equal(eager.params(), graph.params()), s
        assert np.array_equal(eager.velocity(), graph.velocity()), s
    eager.close()
    graph.close()


def test_lm_nonfinite_norm_skips_the_step():
    """lmtrain.lua:1214-1218: a non-finite gradient norm skips the update."""
    announce("lm skip")
    V, D, L, H, F, B, T = 32, 16, 1, 2, 32, 2, 8
    rng = np.random.default_rng(6)
    gpu = lmtrain.GpuLMStep(V, D, L, H, F, B, T)
    p = lmtrain.init_params(gpu.cfg, rng, 0.3)
    p[5] = np.inf                       # an embedding entry -> inf logits -> NaN loss/grads
    gpu.set_params(p)
    gpu.set_batch(rng.integers(0, V, (B, T)), rng.integers(0, V, (B, T)))
    gpu.step(0.1)
    st = gpu.stats()
    assert not st["applied"] and not np.isfinite(st["grad_norm"])
    assert np.array_equal(gpu.params(), p, equal_nan=True)
    assert not gpu.velocity().any()
    gpu.close()


def test_lm_loss_decreases_over_steps():
    """tests/test.lua:511-574 pattern: repeated steps on one batch drive the loss down."""
    announce("lm descent")
    V, D, L, H, F, B, T = 200, 64, 2, 4, 128, 4, 32
    rng = np.random.default_rng(7)
    gpu = lmtrain.GpuLMStep(V, D, L, H, F, B, T)
    gpu.set_params(lmtrain.init_params(gpu.cfg, rng, 0.05))
    gpu.set_batch(rng.integers(0, V, (B, T)), rng.integers(0, V, (B, T)))
    gpu.use_graph(True)
    gpu.step(0.5)
    first = gpu.stats()["loss"]
    for _ in range(40):
        gpu.step(0.5)
    last = gpu.stats()["loss"]
    assert last < 0.9 * first, (first, last)
    gpu.close()


def test_lm_rejects_out_of_range_ids():
    from lanternl_amd._lib import LanternlHipError
    gpu = lmtrain.GpuLMStep(32, 16, 1, 2, 32, 1, 4)
    with pytest.raises(LanternlHipError, match="outside"):
        gpu.set_batch(np.array([[0, 1, 32, 2]]), np.zeros((1, 4)))
    with pytest.raises(LanternlHipError, match="no batch"):
        gpu.step(0.1)
    gpu.close()


def test_lm_step_unfused_attention_path():
    """Windows longer than 64 tokens take the unfused attention path (separate
    RoPE, score GEMM, softmax, PV GEMM and their backwards); same parity bars."""
    announce("lm unfused attention")
    gpu, res = _run_case(48, 16, 1, 2, 32, 2, 80, steps=2, lr=0.1, std=0.3, seed=12)
    _check(res)
    gpu.close()


def test_lm_step_unfused_gemm_path():
    """dim 6 (not a multiple of 4) takes the separate RMSNorm, projection GEMM,
    SwiGLU and SwiGLU-backward launches instead of the fused GEMMs."""
    announce("lm unfused gemm")
    gpu, res = _run_case(40, 6, 2, 1, 10, 2, 5, steps=2, lr=0.1, std=0.3, seed=14)
    _check(res)
    gpu.close()


def test_lm_step_head_dim_64_fused_limit():
    """head_dim 64 and T 64: the largest fused attention configuration."""
    announce("lm hd64")
    gpu, res = _run_case(64, 128, 1, 2, 64, 2, 64, steps=1, lr=0.05, std=0.1, seed=13)
    _check(res)
    gpu.close()


# ------------------------------------------------------------------ AdamW
def _run_adamw(V, D, L, H, F, B, T, steps, lr, std, seed, graph=False, clip=1.0, b1=0.9, b2=0.95, eps=1e-8,
               wd=0.01, poison_step=None):
    """Chained AdamW steps; before each, the oracle takes the GPU's params,
    moments and step count, so each step is compared on its own."""
    rng = np.random.default_rng(seed)
    cfg = O.lm_cfg(V, D, L, H, F)
    gpu = lmtrain.GpuLMStep(V, D, L, H, F, B, T)
    gpu.set_params(lmtrain.init_params(gpu.cfg, rng, std))
    if graph:
        gpu.use_graph(True)
    out = []
    for s in range(steps):
        ids = rng.integers(0, V, (B, T)).astype(np.int32)
        tgt = rng.integers(0, V, (B, T)).astype(np.int32)
        if poison_step == s:
            p = gpu.params()
            p[V * D + 3] = np.nan            # a first-layer norm gain: every gradient turns NaN
            gpu.set_params(p)
        gpu.set_batch(ids, tgt)
        p0 = gpu.params().astype(np.float64)
        m0, v0, t0 = gpu.adam_state()
        gpu.step_adamw(lr, b1, b2, eps, wd, clip)
        st = gpu.stats()
        m1, v1, t1 = gpu.adam_state()
        pr, mr, vr = p0.copy(), m0.astype(np.float64), v0.astype(np.float64)
        ref = O.lm_step_adamw(cfg, pr, mr, vr, t0, ids, tgt, lr, b1, b2, eps, wd, clip)
        out.append(dict(st=st, ref=ref, p0=p0, p1=gpu.params().astype(np.float64), m1=m1, v1=v1, t1=t1,
                        pr=pr, mr=mr, vr=vr, grads=gpu.grads().astype(np.float64)))
    return gpu, out


def _check_adamw(out, loss_tol=1e-5):
    for r in out:
        st, ref = r["st"], r["ref"]
        assert st["applied"] == ref["applied"]
        assert r["t1"] == ref["t"]
        if not ref["applied"]:
            continue
        assert np.max(np.abs(st["window_losses"] - ref["losses"])) <= loss_tol
        assert abs(st["grad_norm"] - ref["gnorm"]) <= 1e-5 * ref["gnorm"]
        assert rel_fro(r["grads"], ref["grads"]) <= 1e-4
        assert rel_fro(r["m1"], r["mr"]) <= 1e-4
        assert rel_fro(r["v1"], r["vr"]) <= 1e-4
        # Adam's update is ~lr*sign(g) per element: compare the update itself
        assert rel_fro(r["p1"] - r["p0"], r["pr"] - r["p0"]) <= 1e-3


def test_lm_adamw_tiny_chained_steps():
    """AdamW (optim2.lua:104-164) over three chained steps: bias corrections at t = 1, 2, 3."""
    announce("lm adamw tiny")
    gpu, out = _run_adamw(32, 16, 1, 2, 32, 2, 8, steps=3, lr=1e-2, std=0.3, seed=21)
    assert [r["t1"] for r in out] == [1, 2, 3]
    _check_adamw(out)
    gpu.close()


def test_lm_adamw_config_c2_graph():
    """Config C2 with LMTrain's AdamW defaults (lr 1e-3, betas 0.9/0.95, eps 1e-8, wd 0.01,
    lmtrain.lua:25-26), replayed from a captured graph."""
    announce("lm adamw C2 graph")
    gpu, out = _run_adamw(2000, 128, 4, 8, 256, 8, 64, steps=2, lr=1e-3, std=0.02, seed=22, graph=True)
    _check_adamw(out)
    gpu.close()


def test_lm_adamw_skip_keeps_step_count():
    """A non-finite norm skips the update and leaves the AdamW step count where it was
    (optim2's self.t advances inside step(), which LMTrain does not call then)."""
    announce("lm adamw skip")
    gpu, out = _run_adamw(32, 16, 1, 2, 32, 2, 8, steps=2, lr=1e-2, std=0.3, seed=23, poison_step=1)
    assert out[0]["ref"]["applied"] and not out[1]["ref"]["applied"]
    assert out[1]["t1"] == 1
    _check_adamw(out)
    gpu.close()


def test_lm_adamw_graph_matches_eager_and_state_round_trip():
    """Graph replay and eager launches agree bit for bit over AdamW steps (the
    step-count slots alternate per call); set/get of the AdamW state round-trips;
    switching optimizers re-captures."""
    announce("lm adamw graph==eager")
    V, D, L, H, F, B, T = 64, 32, 2, 4, 64, 2, 16
    rng = np.random.default_rng(24)
    p = lmtrain.init_params(lmtrain.config(V, D, L, H, F, B, T), rng, 0.1)
    a = lmtrain.GpuLMStep(V, D, L, H, F, B, T)
    b = lmtrain.GpuLMStep(V, D, L, H, F, B, T)
    a.set_params(p); b.set_params(p)
    b.use_graph(True)
    for s in range(4):
        ids = rng.integers(0, V, (B, T)); tgt = rng.integers(0, V, (B, T))
        a.set_batch(ids, tgt); b.set_batch(ids, tgt)
        if s == 2:      # one SGD step in between: the graph is captured again for it
            a.step(0.01); b.step(0.01)
        else:
            a.step_adamw(2e-3); b.step_adamw(2e-3)
        assert np.array_equal(a.params(), b.params())
    ma, va, ta = a.adam_state(); mb, vb, tb = b.adam_state()
    assert ta == tb == 3 and np.array_equal(ma, mb) and np.array_equal(va, vb)
    m = rng.standard_normal(a.n).astype(np.float32); v = np.abs(rng.standard_normal(a.n)).astype(np.float32)
    a.set_adam_state(m, v, 7)
    m2, v2, t2 = a.adam_state()
    assert t2 == 7 and np.array_equal(m2, m) and np.array_equal(v2, v)
    a.close(); b.close()


def test_lm_checkpoint_save_load_device(tmp_path):
    """lhip_lm_save streams the device parameters into an lmio v3 file identical
    to the host writer's; lhip_lm_load puts them back, and a step from the
    loaded model equals a step from set_params."""
    announce("lm checkpoint")
    V, D, L, H, F, B, T = 64, 32, 2, 4, 64, 2, 16
    rng = np.random.default_rng(31)
    a = lmtrain.GpuLMStep(V, D, L, H, F, B, T)
    p = lmtrain.init_params(a.cfg, rng, 0.1)
    a.set_params(p)
    for fmt in ("bin", "text"):
        path = tmp_path / f"dev.{fmt}"
        a.save(path, fmt=fmt, epoch=3, loss=1.5)
        ref = tmp_path / f"host.{fmt}"
        lmtrain.save_checkpoint(ref, a.cfg, p, fmt=fmt, epoch=3, loss=1.5)
        assert path.read_bytes() == ref.read_bytes()
    b = lmtrain.GpuLMStep(V, D, L, H, F, B, T)
    hdr = b.load(tmp_path / "dev.bin")
    assert hdr["epoch"] == 3 and hdr["loss"] == 1.5
    assert np.array_equal(b.params(), p)
    ids = rng.integers(0, V, (B, T)); tgt = rng.integers(0, V, (B, T))
    a.set_batch(ids, tgt); b.set_batch(ids, tgt)
    a.step(0.05); b.step(0.05)
    assert np.array_equal(a.params(), b.params())
    with pytest.raises(Exception):
        lmtrain.GpuLMStep(V, 48, L, H, F, B, T).load(tmp_path / "dev.bin")
    a.close(); b.close()


# ------------------------------------------------- ragged batches (LMTrain's last window / last batch)
def _ragged_case(V, D, L, H, F, B, T, plan, graph, causal=True, opt="sgd", seed=77):
    """plan: per step (lengths, n_windows) or None for a full batch."""
    rng = np.random.default_rng(seed)
    cfg = O.lm_cfg(V, D, L, H, F, causal=causal)
    gpu = lmtrain.GpuLMStep(V, D, L, H, F, B, T, causal=causal)
    gpu.set_params(lmtrain.init_params(gpu.cfg, rng, 0.02))
    if graph:
        gpu.use_graph(True)
    t = 0
    for k, item in enumerate(plan):
        announce("lm ragged", k, item, "graph" if graph else "eager", opt, "causal" if causal else "full")
        ids = rng.integers(0, V, (B, T)).astype(np.int32)
        tgt = rng.integers(0, V, (B, T)).astype(np.int32)
        if item is None:
            lens, nw = np.full(B, T, np.int32), B
            gpu.set_batch(ids, tgt)
        else:
            lens = np.zeros(B, np.int32)
            lens[:len(item)] = item
            nw = len(item)
            # junk past each window's length and in the unused slots must not matter
            gpu.set_batch(ids, tgt, lens, nw)
        p_before = gpu.params().astype(np.float64)
        if opt == "sgd":
            v_before = gpu.velocity().astype(np.float64)
            gpu.step(0.05, 0.9, 0.01, 1.0)
            ref_p, ref_v = p_before.copy(), v_before.copy()
            ref = O.lm_step_sgd(cfg, ref_p, ref_v, ids, tgt, 0.05, 0.9, 0.01, 1.0, lens=lens, nwin=nw)
        else:
            m0, v0, t0 = gpu.adam_state()
            gpu.step_adamw(1e-3, 0.9, 0.95, 1e-8, 0.01, 1.0)
            ref_p, ref_m, ref_v = p_before.copy(), m0.astype(np.float64), v0.astype(np.float64)
            ref = O.lm_step_adamw(cfg, ref_p, ref_m, ref_v, t0, ids, tgt, 1e-3, lens=lens, nwin=nw)
        st = gpu.stats()
        wl = st["window_losses"]
        assert np.max(np.abs(wl[:nw] - ref["losses"][:nw])) <= 1e-5
        assert np.all(wl[nw:] == 0)
        tok = lens[:nw].astype(np.float64)
        assert abs(st["loss"] - float(np.sum(ref["losses"][:nw] * tok) / tok.sum())) <= 1e-5
        assert st["applied"] == ref["applied"] and st["correct"] == ref["correct"]
        assert abs(st["grad_norm"] - ref["gnorm"]) <= 1e-5 * ref["gnorm"]
        assert rel_fro(gpu.grads(), ref["grads"]) <= 1e-4
        after = gpu.params().astype(np.float64)
        if opt == "sgd":
            assert rel_fro(after - p_before, ref_p - p_before) <= 1e-4
            assert rel_fro(gpu.velocity(), ref_v) <= 1e-4
        else:
            assert rel_fro(after - p_before, ref_p - p_before) <= 1e-3
            m1, v1, t1 = gpu.adam_state()
            assert t1 == ref["t"] and rel_fro(m1, ref_m) <= 1e-4 and rel_fro(v1, ref_v) <= 1e-4
        t += 1
    gpu.close()


RAGGED = [None, [64, 64, 64, 64, 17], None, [17], [64, 3, 64, 40, 64, 64, 64, 1]]


@pytest.mark.parametrize("graph", [False, True])
def test_lm_step_ragged_batches_c2(graph):
    """Config C2 (B=8, T=64) with LMTrain's ragged batches: 5 windows of
    {64, 64, 64, 64, 17} tokens, one 17-token window, 8 windows with short
    ones, between full batches, eager and replayed from the captured graph."""
    _ragged_case(2000, 128, 4, 8, 256, 8, 64, RAGGED, graph)


def test_lm_step_ragged_adamw_and_noncausal():
    _ragged_case(2000, 128, 2, 8, 256, 8, 64, [None, [64, 64, 64, 64, 17]], False, opt="adamw", seed=78)
    # a non-causal model: the fused attention masks keys past each window's length
    _ragged_case(64, 32, 1, 2, 48, 4, 16, [None, [16, 5, 9]], True, causal=False, seed=79)
    # the unfused attention path (seq > 64), causal
    _ragged_case(64, 32, 1, 2, 48, 2, 80, [[80, 33]], False, seed=80)


def test_lm_set_batch_rejects_bad_windows():
    from lanternl_amd._lib import LanternlHipError
    gpu = lmtrain.GpuLMStep(64, 32, 1, 2, 48, 4, 16)
    ids = np.zeros((4, 16), np.int32)
    for lens, nw in (([16, 0], 2), ([17], 1), ([16] * 5, 5), ([4], 0)):
        with pytest.raises(LanternlHipError):
            gpu.set_batch(ids, ids, np.array(lens + [0] * (5 - len(lens)), np.int32), nw)
    bad = ids.copy(); bad[0, 3] = 99                       # a counted id outside the vocabulary
    with pytest.raises(LanternlHipError, match="ids"):
        gpu.set_batch(bad, ids, np.array([8, 0, 0, 0], np.int32), 1)
    bad[0, 3] = 0; bad[0, 12] = 99                         # past the window's length: ignored
    gpu.set_batch(bad, ids, np.array([8, 0, 0, 0], np.int32), 1)
    ncg = lmtrain.GpuLMStep(64, 32, 1, 2, 48, 2, 80, causal=False)   # unfused and non-causal
    with pytest.raises(LanternlHipError, match="UNSUPPORTED"):
        ncg.set_batch(np.zeros((2, 80), np.int32), np.zeros((2, 80), np.int32), np.array([80, 7], np.int32), 2)
    ncg.set_batch(np.zeros((2, 80), np.int32), np.zeros((2, 80), np.int32))   # full windows are fine
    gpu.close(); ncg.close()
