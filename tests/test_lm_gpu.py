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


def _run_case(V, D, L, H, F, B, T, steps, lr, std, seed, graph=False, clip=1.0, mom=0.9, wd=0.01):
    rng = np.random.default_rng(seed)
    cfg = O.lm_cfg(V, D, L, H, F)
    gpu = lmtrain.GpuLMStep(V, D, L, H, F, B, T)
    p32 = lmtrain.init_params(gpu.cfg, rng, std)
    gpu.set_params(p32)
    if graph:
        gpu.use_graph(True)
    results = []
    for _ in range(steps):
        ids = rng.integers(0, V, (B, T)).astype(np.int32)
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


def test_lm_step_head_dim_64_fused_limit():
    """head_dim 64 and T 64: the largest fused attention configuration."""
    announce("lm hd64")
    gpu, res = _run_case(64, 128, 1, 2, 64, 2, 64, steps=1, lr=0.05, std=0.1, seed=13)
    _check(res)
    gpu.close()
