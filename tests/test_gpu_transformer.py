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


def _bf16_step(w):
    """The spacing of bf16 values at |w| (8 significant bits)."""
    a = np.abs(np.asarray(w, np.float64))
    e = np.floor(np.log2(np.where(a > 0, a, 2.0**-133)))
    return 2.0 ** (np.maximum(e, -133) - 7)


def _grad_bound(want):
    """The bf16 bound on a gradient, element by element: rtol 2e-2 plus 1e-2 of the gradient's largest
    magnitude (the absolute part scaled to the tensor, as the reference scales its attention-gradient atol,
    tests/functional/test_attention.py:413-416)."""
    w = np.asarray(want, np.float64)
    return 2e-2 * np.abs(w) + 1e-2 * np.abs(w).max()


@pytest.mark.parametrize("hfuse", [True, False])
def test_transformer_gradients_match_oracle(hip, hfuse):
    """Loss within 1e-2 relative (tests/test_transformer_example.py:316); every element of every gradient
    within the bf16 bound (rtol 2e-2 plus 1e-2 of its largest magnitude) and each gradient's norm within 2e-2
    of the oracle's. Without horizontal fusion the concatenated attention gradients feeding the merged
    projection dots are written in place by the flash backward kernel (``alias`` steps)."""
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
        a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
        err = np.abs(a - b)
        assert np.all(err <= _grad_bound(b)), (name, float(err.max()), float(np.abs(b).max()))
        assert abs(np.linalg.norm(a) - np.linalg.norm(b)) <= 2e-2 * np.linalg.norm(b), name


@pytest.mark.parametrize("lce_chunk", [None, 128])
def test_transformer_train_step_updates_weights(hip, lce_chunk):
    """One SGD step (lr 1.0): the loss, and every written-back weight within one bf16 step of the oracle's
    plus the learning rate times the gradient bound (the update differs only through the gradient, then by
    one rounding: the reference's rule of exact agreement where the gradient is clear of zero and a bounded
    update where it is not, tests/test_transformer_example.py:318-331, restated for SGD); also with the fused
    linear cross entropy backward (two row chunks), against the oracle on the same (substituted) graph."""
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
    # the oracle's gradients at the same weights bound the updates
    gmodel, _, _, _, _, gargs = _setup(cfg, _grads)
    gtraced = trace(_grads, gargs)
    gnames = {id(p): n for n, p in gmodel.named_parameters()}
    grads = oracle.values(gtraced.graph, _oracle_inputs(gtraced, ids, targets, weights, gnames))[1:]
    grad_of = dict(zip([n for n, _ in gmodel.named_parameters()], grads))
    for j, k in enumerate(traced.written):
        p = traced.weights[k]
        got = D.bf16_to_f32(p._placed("hip:0").raw()).astype(np.float64)
        w = np.asarray(want[1 + j], np.float64)
        limit = _bf16_step(w) + 1.0 * _grad_bound(grad_of[names[id(p)]])
        assert np.all(np.abs(got - w) <= limit), (names[id(p)], float(np.abs(got - w).max()))


def test_hip_graph_reads_large_arguments_in_place(hip, monkeypatch):
    """Arguments of 1 MiB and more are read in place by the captured graph (no staging copy): one graph per set
    of their addresses, the newest kept (here two); inputs taken in rotation, a new address evicting the oldest
    graph and an old one captured again, each call equal bit for bit to the same call run uncaptured."""
    import lumen_amd.functional as F
    from lumen_amd.graph.compiled import Compiled

    monkeypatch.setattr(Compiled, "GRAPHS_PER_PLAN", 2)
    monkeypatch.setattr(Compiled, "GRAPH_MIN_STEPS", 1)

    def fn(x, s):
        return F.softmax(x.float() * s, -1).bfloat16()

    rng = np.random.default_rng(8)
    xs = [L.tensor(D.bf16_to_f32(D.bf16_bits(rng.standard_normal((1024, 1024)))), "bfloat16").to("hip")
          for _ in range(3)]
    order = [0, 1, 0, 1, 2, 0, 2, 1]
    with L.config.compiler.patch(hip_graphs=True):
        f = L.compile(fn, device="hip")
        got = []
        for n, i in enumerate(order):
            got.append(np.asarray(L.to_numpy(f(xs[i], 0.5 + n)), np.float32))
            L.from_numpy(np.full(1 << 20, float(n), np.float32)).to("hip")  # eager work between calls
        graphs = f._graphs[id(f.plan)]
        assert len(graphs) == 2 and all(xs[i].data_ptr() in key for key, i in zip(graphs, (2, 1)))
    with L.config.compiler.patch(hip_graphs=False):
        u = L.compile(fn, device="hip")
        want = [np.asarray(L.to_numpy(u(xs[i], 0.5 + n)), np.float32) for n, i in enumerate(order)]
    for g_, w_ in zip(got, want):
        assert np.array_equal(g_, w_)


def test_hip_graph_replays_match_uncaptured_runs(hip, monkeypatch):
    """With hip_graphs the third and later calls of a compiled function replay one captured HIP graph whose
    arguments and runtime scalars are staged into its own buffers: several calls with new inputs, new
    scalars and eager device work in between, each equal bit for bit to the same call run uncaptured; then
    the training step (weights written back every call) for three steps, equal to the uncaptured steps."""
    import lumen_amd.functional as F

    def fn(x, w, s):
        return F.relu(F.matmul(x, w, "float32", "float32")) * s + x.float().sum()

    from lumen_amd.graph.compiled import Compiled

    with L.config.compiler.patch(hip_graphs=True):  # a short plan runs uncaptured by default
        f = L.compile(fn, device="hip")
        ones = [L.tensor(np.ones(shape, np.float32), "bfloat16") for shape in ((512, 256), (256, 320))]
        for _ in range(3):
            f(*ones, 1.0)
        assert len(f.plan.native_steps) < Compiled.GRAPH_MIN_STEPS and not f._graphs.get(id(f.plan))
    monkeypatch.setattr(Compiled, "GRAPH_MIN_STEPS", 1)
    rng = np.random.default_rng(5)
    w = L.tensor(D.bf16_to_f32(D.bf16_bits(rng.standard_normal((256, 320)) * 0.1)), "bfloat16")
    xs = [L.tensor(D.bf16_to_f32(D.bf16_bits(rng.standard_normal((512, 256)))), "bfloat16") for _ in range(5)]
    with L.config.compiler.patch(hip_graphs=True):
        f = L.compile(fn, device="hip")
        got = []
        for i, x in enumerate(xs):
            got.append(np.asarray(L.to_numpy(f(x, w, 0.5 + i)), np.float32))
            L.from_numpy(np.full(1 << 20, float(i), np.float32)).to("hip")  # eager work between calls
        assert len(f._graphs[id(f.plan)]) == 1  # captured once: the small arguments are staged
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


def test_runtime_scalars_are_uploaded_once_per_value(hip, monkeypatch):
    """A runtime scalar is uploaded once per value and kept on the device (the upload synchronizes, so a
    per-call upload would stall every call on the previous one): calls alternating two values keep two
    device copies, captured and replayed, each call equal bit for bit to the same call run uncaptured."""
    import lumen_amd.functional as F
    from lumen_amd.graph.compiled import Compiled

    monkeypatch.setattr(Compiled, "GRAPH_MIN_STEPS", 1)

    def fn(x, s):
        return F.relu(x.float() * s - 0.25)

    rng = np.random.default_rng(11)
    x = L.tensor(D.bf16_to_f32(D.bf16_bits(rng.standard_normal((256, 512)))), "bfloat16")
    values = [0.5, 1.5, 0.5, 1.5, 0.5, 1.5]
    with L.config.compiler.patch(hip_graphs=True):
        f = L.compile(fn, device="hip")
        got = [np.asarray(L.to_numpy(f(x, v)), np.float32) for v in values]
        assert len(f._scalars) == 2 and len(f._graphs[id(f.plan)]) == 1
    with L.config.compiler.patch(hip_graphs=False):
        u = L.compile(fn, device="hip")
        want = [np.asarray(L.to_numpy(u(x, v)), np.float32) for v in values]
    for g_, w_ in zip(got, want):
        assert np.array_equal(g_, w_)
    assert not np.array_equal(got[0], got[1])


@pytest.mark.parametrize("cfg_name", ["TINY", "CONFIG4"])
def test_weights_updated_in_place_match_copied_updates(hip, cfg_name):
    """Every weight the training step assigns is computed over its old value (no workspace copy, no copy
    back), including the weight-gradient GEMMs whose epilogue applies the update (at config 4 they are large
    enough for the epilogue autotuner, which then writes them elsewhere while timing): three steps give the
    losses and weights of the same steps with the updates written to the workspace and copied back, to
    float32 rounding of the loss and one bf16 step of every weight (the column sums fused into some
    epilogues add with atomics, in no fixed order)."""
    cfg = getattr(W, cfg_name)
    got = {}
    for in_place in (True, False):
        model, opt, weights, ids, targets, args = _setup(cfg, W.train_step)
        args = (model, opt) + args[1:]
        with L.config.compiler.patch(update_in_place=in_place, hip_graphs=True):
            step = L.compile(W.train_step, device="hip")
            losses = [float(L.to_numpy(step(*args))) for _ in range(3)]
            traced = trace(W.train_step, args)
            if in_place:
                assert len(step.plan.in_place_outputs) == len(traced.written)
                assert not any(st.kind == "copy" for st in step.plan.steps)
            else:
                assert not step.plan.in_place_outputs
        got[in_place] = (losses, [D.bf16_to_f32(p._placed("hip:0").raw()).astype(np.float64)
                                  for _, p in model.named_parameters()])
    for a, b in zip(got[True][0], got[False][0]):
        assert abs(a - b) <= 1e-5 * abs(b), (a, b)
    for (name, _), a, b in zip(model.named_parameters(), got[True][1], got[False][1]):
        assert np.all(np.abs(a - b) <= _bf16_step(b)), (name, float(np.abs(a - b).max()))
