"""The decoder training step (the benchmark transformer at a small size) compiled for hip against the CPU
oracle running the same traced graph: loss, every gradient, and the SGD-updated weights."""

import numpy as np
import pytest

import lumen_amd as L
from lumen_amd import dtypes as D
from lumen_amd import workloads as W
from lumen_amd.graph.trace import trace
from oracle import oracle

pytestmark = pytest.mark.gpu


def _grads(model, ids, targets):
    loss = W.loss_fn(model, ids, targets)
    loss.backward()
    return [loss] + [p.grad for p in model.parameters()]


def _setup(cfg, fn, *extra):
    model, opt = W.build(cfg, lr=1.0)
    weights = W.init_weights(model)
    W.load(model, weights)
    ids, targets = W.batch(cfg)
    args = (model,) + extra + (L.from_numpy(ids), L.from_numpy(targets))
    return model, opt, weights, ids, targets, args


def _oracle_inputs(traced, ids, targets, weights, names, scalars=()):
    ins = []
    by_id = {id(p): names[id(p)] for p in traced.weights}
    args = [ids, targets]
    for kind, k in traced.layout:
        if kind == "arg":
            ins.append(args[k])
        elif kind == "scalar":
            ins.append(np.array(scalars[k], np.float64))
        else:
            ins.append(weights[by_id[id(traced.weights[k])]])
    return ins


@pytest.mark.parametrize("hfuse", [True, False])
def test_transformer_gradients_match_oracle(hip, hfuse):
    """Loss within 1e-2 relative, every gradient within 5% relative norm of the oracle's (the reference's
    transformer test bounds, tests/test_transformer_example.py:318-331). Without horizontal fusion the
    concatenated attention gradients feeding the merged projection dots are written in place by the flash
    backward kernel (``alias`` steps)."""
    cfg = W.TINY
    model, opt, weights, ids, targets, args = _setup(cfg, _grads)
    names = {id(p): n for n, p in model.named_parameters()}
    with L.config.compiler.patch(horizontal_fusion=hfuse):
        f = L.compile(_grads, device="hip")
        got = [L.to_numpy(t) for t in f(*args)]
    if not hfuse:
        assert "alias" in [s["kind"] for s in f.plan.describe()]
    traced = trace(_grads, args)
    want = oracle.values(traced.graph, _oracle_inputs(traced, ids, targets, weights, names))
    assert abs(got[0] - want[0]) <= 1e-2 * abs(want[0]), (got[0], want[0])
    pnames = [n for n, _ in model.named_parameters()]
    for name, a, b in zip(pnames, got[1:], want[1:]):
        err = np.linalg.norm(a.astype(np.float64) - b) / max(np.linalg.norm(b), 1e-30)
        assert err <= 5e-2, (name, err)


@pytest.mark.parametrize("lce_chunk", [None, 128])
def test_transformer_train_step_updates_weights(hip, lce_chunk):
    """One SGD step (lr 1.0): the loss, and the written-back weights within bf16 rounding of the oracle's;
    also with the fused linear cross entropy backward (two row chunks), against the oracle on the same
    (substituted) traced graph."""
    cfg = W.TINY
    model, opt, weights, ids, targets, args = _setup(cfg, W.train_step)
    args = (model, opt) + args[1:]
    names = {id(p): n for n, p in model.named_parameters()}
    with L.config.compiler.patch(fused_linear_cross_entropy_chunk_size=lce_chunk):
        f = L.compile(W.train_step, device="hip")
        loss = float(L.to_numpy(f(*args)))
        traced = trace(W.train_step, args)
    want = oracle.values(traced.graph, _oracle_inputs(traced, ids, targets, weights, names, scalars=[1.0]))
    assert abs(loss - want[0]) <= 1e-2 * abs(want[0])
    for j, k in enumerate(traced.written):
        p = traced.weights[k]
        got = D.bf16_to_f32(p._placed("hip:0").raw())
        w = want[1 + j]
        tol = 2e-2 * np.abs(w) + 1e-2 * np.abs(w).max()
        assert (np.abs(got - w) <= tol).mean() > 0.999, names[id(p)]


def test_hip_graph_replays_match_uncaptured_runs(hip):
    """With hip_graphs the third and later calls of a compiled function replay one captured HIP graph whose
    arguments and runtime scalars are staged into its own buffers: several calls with new inputs, new
    scalars and eager device work in between, each equal bit for bit to the same call run uncaptured; then
    the training step (weights written back every call) for three steps, equal to the uncaptured steps."""
    import lumen_amd.functional as F

    def fn(x, w, s):
        return F.relu(F.matmul(x, w, "float32", "float32")) * s + x.float().sum()

    rng = np.random.default_rng(5)
    w = L.tensor(D.bf16_to_f32(D.bf16_bits(rng.standard_normal((256, 320)) * 0.1)), "bfloat16")
    xs = [L.tensor(D.bf16_to_f32(D.bf16_bits(rng.standard_normal((512, 256)))), "bfloat16") for _ in range(5)]
    with L.config.compiler.patch(hip_graphs=True):
        f = L.compile(fn, device="hip")
        got = []
        for i, x in enumerate(xs):
            got.append(np.asarray(L.to_numpy(f(x, w, 0.5 + i)), np.float32))
            L.from_numpy(np.full(1 << 20, float(i), np.float32)).to("hip")  # eager work between calls
        assert f._graphs[id(f.plan)] not in (None, "warm")  # captured
    with L.config.compiler.patch(hip_graphs=False):
        u = L.compile(fn, device="hip")
        want = [np.asarray(L.to_numpy(u(x, w, 0.5 + i)), np.float32) for i, x in enumerate(xs)]
    for g_, w_ in zip(got, want):
        assert np.array_equal(g_, w_)

    losses = {}
    for graphs in (True, False):
        cfg = W.TINY
        model, opt, weights, ids, targets, args = _setup(cfg, W.train_step)
        args = (model, opt) + args[1:]
        with L.config.compiler.patch(hip_graphs=graphs):
            step = L.compile(W.train_step, device="hip")
            losses[graphs] = [float(L.to_numpy(step(*args))) for _ in range(4)]
            losses[graphs].append(D.bf16_to_f32(model.head._placed("hip:0").raw()).copy())
    assert losses[True][:4] == losses[False][:4]
    assert np.array_equal(losses[True][4], losses[False][4])
