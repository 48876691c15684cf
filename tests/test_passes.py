"""Compiler passes preserve values (the reference's pass tests run rewritten graphs through
reference::run, lumen/graph_compiler/tests/mod.rs:140-148): cse, simplify, flash-attention matching and
the fusion grouping, checked bit for bit with the oracle."""

import numpy as np
import pytest

import lumen_amd as L
import lumen_amd.functional as F
from lumen_amd import dtypes as D
from lumen_amd import workloads as W
from lumen_amd.compiler import attention, fusion, passes
from lumen_amd.graph.trace import trace
from oracle import oracle


def _inputs(g, seed=0):
    rng = np.random.default_rng(seed)
    out = []
    for v in g.inputs:
        t = g.types[v]
        if t.dtype in ("int64", "int32"):
            out.append(rng.integers(0, 7, t.shape).astype(D.storage(t.dtype)))
        elif t.dtype == "bfloat16":
            out.append(D.bf16_bits(rng.standard_normal(t.shape).astype(np.float32)))
        else:
            out.append(rng.standard_normal(t.shape).astype(D.storage(t.dtype)))
    return out


def _same(g0, g1, seed=0):
    xs = _inputs(g0, seed)
    for a, b in zip(oracle.run(g0, xs), oracle.run(g1, xs)):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8))


PROGRAMS = {
    "mlp": (lambda x, w: F.softmax(F.relu(F.matmul(x, w, "float32", "float32")), -1) * 2.0,
            [((8, 16), "float32"), ((16, 8), "float32")]),
    "dup": (lambda x: F.exp(x) + F.exp(x) * F.exp(x), [((5, 3), "float32")]),
    "casts": (lambda x, w: F.matmul(x, w, "float32", "bfloat16").float().bfloat16(),
              [((4, 8), "bfloat16"), ((8, 4), "bfloat16")]),
    "layouts": (lambda x: x.t().t().reshape(6, 2).reshape(3, 4) + 1.0, [((3, 4), "float32")]),
}


@pytest.mark.parametrize("name", sorted(PROGRAMS))
def test_frontend_preserves_values(name):
    fn, shapes = PROGRAMS[name]
    g = L.make_graph(fn)(*[L.empty(list(s), d, "meta") for s, d in shapes])
    _same(g, passes.cse(g))
    _same(g, passes.frontend(g))
    assert len(passes.frontend(g).nodes) <= len(g.nodes)


def test_cse_merges_duplicates():
    fn, shapes = PROGRAMS["dup"]
    g = L.make_graph(fn)(*[L.empty(list(s), d, "meta") for s, d in shapes])
    assert sum(n.prim == "exp" for n in passes.cse(g).nodes) == 1


def test_simplify_folds_narrowing_cast_into_dot():
    fn, shapes = PROGRAMS["casts"]
    g = passes.frontend(L.make_graph(fn)(*[L.empty(list(s), d, "meta") for s, d in shapes]))
    dots = [n for n in g.nodes if n.prim == "dot_general"]
    assert dots[0].params["output_dtype"] == "bfloat16"


@pytest.mark.parametrize("causal", [False, True])
def test_flash_attention_match_preserves_values(causal):
    def grads(q, k, v, do):
        out, pull = L.vjp(lambda q, k, v: F.flash_attention(q, k, v, is_causal=causal), q, k, v)
        return (out,) + pull(do)

    g = L.make_graph(grads)(*[L.empty([1, 32, 2, 64], "bfloat16", "meta") for _ in range(4)])
    m = attention.match(passes.frontend(g))
    names = [n.params.get("name") for n in m.nodes if n.prim == "fusion"]
    assert names == ["flash_attention", "flash_attention_backward"]
    _same(g, m)


@pytest.mark.parametrize("causal", [False, True])
def test_grouped_query_attention_matches_with_the_key_value_heads_as_operands(causal):
    """Grouped heads (4 query heads over 2 key/value heads): the forward and the backward (dK and dV summed
    over each group) both become flash fusions whose K and V operands are the [B, S, 2, D] tensors
    themselves, not their expansion to every query head; the values are unchanged (oracle on both graphs)."""
    def grads(q, k, v, do):
        out, pull = L.vjp(lambda q, k, v: F.flash_attention(q, k, v, is_causal=causal), q, k, v)
        return (out,) + pull(do)

    metas = [L.empty(s, "bfloat16", "meta") for s in ([1, 40, 4, 64], [1, 40, 2, 64], [1, 40, 2, 64], [1, 40, 4, 64])]
    g = L.make_graph(grads)(*metas)
    m = attention.match(passes.frontend(g))
    fus = [n for n in m.nodes if n.prim == "fusion"]
    assert [n.params["name"] for n in fus] == ["flash_attention", "flash_attention_backward"]
    for f in fus:
        assert [tuple(m.types[u].shape) for u in f.inputs[1:3]] == [(1, 40, 2, 64)] * 2
    assert [tuple(m.types[v].shape) for v in m.outputs] == [(1, 40, 4, 64), (1, 40, 4, 64), (1, 40, 2, 64),
                                                            (1, 40, 2, 64)]
    _same(g, m)


def test_written_attention_matches():
    """Attention written as matmul -> scale -> causal mask -> softmax -> matmul is recognized too."""

    def attn(q, k, v):
        s = F.matmul(q, k.transpose(-1, -2), "float32", "float32") * 0.125
        rows = L.prims.iota("int64", s.shape, 2)
        cols = L.prims.iota("int64", s.shape, 3)
        s = F.where(cols <= rows, s, float("-inf"))
        p = F.softmax(s, -1).bfloat16()
        return F.matmul(p, v, "float32", "bfloat16")

    g = L.make_graph(attn)(*[L.empty([2, 2, 32, 64], "bfloat16", "meta") for _ in range(3)])
    m = attention.match(passes.frontend(g))
    assert [n.params.get("name") for n in m.nodes if n.prim == "fusion"] == ["flash_attention"]
    assert [n for n in m.nodes if n.prim == "fusion"][0].params["causal"] is True
    _same(g, m)


def test_fusion_of_the_training_step_preserves_dependencies():
    """Every step reads only values computed by earlier steps or graph inputs, and every graph output is
    written by some step (the tiny transformer step)."""
    model, opt = W.build(W.TINY)
    ids = L.empty([W.TINY.batch, W.TINY.seq], "int64", "meta")
    g = attention.match(passes.frontend(trace(W.train_step, (model, opt, ids, ids)).graph))
    steps = fusion.fuse(g)
    have = set(g.inputs)
    for st in steps:
        assert all(u in have for u in st.inputs), st.label()
        have.update(st.outputs)
    assert set(g.outputs) <= have
    kinds = {st.kind for st in steps}
    assert {"dot", "row", "flash_fwd", "flash_bwd", "scatter_add"} <= kinds


def test_merge_dots_packs_projections_and_their_gradients():
    """merge_dots (passes/merge_dots): the three projections of one activation become one dot against the
    packed weights, and their backward (the summed input gradient and the three weight gradients) one dot
    each; values stay within float32 reassociation of the unmerged graph."""
    from lumen_amd.compiler import merge

    def f(x, wq, wk, wv):
        q = F.matmul(x, wq.t(), "float32", "float32")
        k = F.matmul(x, wk.t(), "float32", "float32")
        v = F.matmul(x, wv.t(), "float32", "float32")
        return ((q * k + v) * x.sum()).sum()

    metas = [L.empty([16, 32], "float32", "meta")] + [L.empty([24, 32], "float32", "meta") for _ in range(3)]
    g0 = passes.frontend(L.make_graph(L.value_and_grad(f, argnums=(0, 1, 2, 3)))(*metas))
    g1, packs = merge.merge_dots(g0, {1, 2, 3})
    assert packs == [(1, 2, 3)]
    dots = lambda g: sum(n.prim == "dot_general" for n in g.nodes)
    assert dots(g0) == 9 and dots(g1) == 3
    xs = _inputs(g0)
    for a, b in zip(oracle.run(g0, xs), oracle.run(g1, xs)):
        np.testing.assert_allclose(np.asarray(a, np.float64), np.asarray(b, np.float64), rtol=1e-5,
                                   atol=1e-5 * max(1.0, float(np.abs(a).max())))


def _eval_ce(h, w, t):
    return F.mean(F.cross_entropy(F.matmul(h, w.t(), "float32", "float32"), t))


def test_linear_cross_entropy_pass_rewrites_an_eval_loss_and_keeps_its_value():
    """A cross entropy whose logits only it reads becomes one linear_cross_entropy node (the weight's
    transpose folded away); the oracle gives the same loss on both graphs (float32 rounding of the sums:
    the fused op sums exponentials in float64, the unfused graph in float32)."""
    from lumen_amd.compiler import passes
    from oracle import oracle

    rng = np.random.default_rng(3)
    b, v, d = 48, 300, 40
    h = D.bf16_bits(rng.standard_normal((b, d)).astype(np.float32))
    w = D.bf16_bits((rng.standard_normal((v, d)) * 0.3).astype(np.float32))
    t = rng.integers(0, v, b).astype(np.int64)
    args = [L.tensor(D.bf16_to_f32(h), "bfloat16"), L.tensor(D.bf16_to_f32(w), "bfloat16"), L.from_numpy(t)]
    g = passes.frontend(L.make_graph(_eval_ce)(*args))
    g2 = passes.linear_cross_entropy(g)
    prims_ = [n.prim for n in g2.nodes]
    assert "linear_cross_entropy" in prims_ and "dot_general" not in prims_ and "transpose" not in prims_
    (a,) = oracle.run(g, [h, w, t])
    (b_,) = oracle.run(g2, [h, w, t])
    np.testing.assert_allclose(b_, a, rtol=1e-6)


def test_linear_cross_entropy_pass_leaves_a_training_step():
    """With the gradient the backward reads the logits, so nothing is rewritten (as in the reference)."""
    from lumen_amd.compiler import passes

    h = L.empty([16, 8], "bfloat16", "meta")
    w = L.empty([40, 8], "bfloat16", "meta")
    t = L.empty([16], "int32", "meta")
    g = passes.frontend(L.make_graph(lambda h, w, t: L.value_and_grad(lambda h: _eval_ce(h, w, t))(h))(h, w, t))
    assert all(n.prim != "linear_cross_entropy" for n in passes.linear_cross_entropy(g).nodes)


def test_linear_cross_entropy_through_the_pipeline():
    """Through compile_graph (simplify twice, attention matching) the eval loss still becomes the fused
    step: the row max may reach the log-sum-exp without its reshape."""
    from lumen_amd.compiler.plan import Plan

    h = L.empty([512, 256], "bfloat16", "meta")
    w = L.empty([5000, 256], "bfloat16", "meta")
    t = L.empty([512], "int64", "meta")
    p = Plan(L.make_graph(_eval_ce)(h, w, t), build_kernels=False)
    assert [s.kind for s in p.steps][0] == "linear_cross_entropy"
    with L.config.compiler.patch(fused_linear_cross_entropy=False):
        p = Plan(L.make_graph(_eval_ce)(h, w, t), build_kernels=False)
    assert "linear_cross_entropy" not in [s.kind for s in p.steps]


def _prims(g):
    return [n.prim for n in g.nodes]


REWRITES = {
    # name: (program, input shapes, check of the simplified graph) — identities and compositions
    "mul_one": (lambda x: (x * 1.0) * (1.0 * x), [((4, 5), "float32")],
                lambda g: _prims(g).count("mul") == 1),
    "add_sub_div": (lambda x: ((x + 0.0) - 0.0) / 1.0 + (0.0 + x), [((3, 7), "bfloat16")],
                    lambda g: _prims(g) == ["add"]),
    "double_neg": (lambda x: -(-x) * 3.0, [((6,), "float32")], lambda g: "neg" not in _prims(g)),
    "select_same": (lambda x, y: F.where(x > y, x, x), [((4, 4), "float32"), ((4, 4), "float32")],
                    lambda g: "select" not in _prims(g)),
    "broadcasts": (lambda x: x.reshape(4, 1).expand(4, 6).reshape(1, 4, 6).expand(3, 4, 6) * 2.0,
                   [((4,), "float32")], lambda g: True),
    # structural (after matching): a transposed dot, transposed operands, moved casts and elementwise ops
    "dot_transposed": (lambda x, w: F.matmul(x, w, "float32", "float32").t() + 1.0,
                       [((8, 16), "float32"), ((16, 4), "float32")],
                       lambda g: "transpose" not in _prims(g)),
    "dot_operand_transposed": (lambda x, w: F.matmul(x.t(), w.t(), "float32", "float32"),
                               [((16, 8), "float32"), ((4, 16), "float32")],
                               lambda g: "transpose" not in _prims(g)),
    "widening_cast_after_layout": (lambda x: x.float().t().reshape(20) * 2.0, [((4, 5), "bfloat16")],
                                   lambda g: _prims(g).index("cast") > _prims(g).index("reshape")),
    "narrowing_cast_before_layout": (lambda x: (x * 3.0).t().bfloat16(), [((4, 5), "float32")],
                                     lambda g: _prims(g).index("cast") < _prims(g).index("transpose")),
    "elementwise_before_reshape": (lambda x, y: F.exp(x.reshape(10, 2) * y.reshape(10, 2)),
                                   [((4, 5), "float32"), ((4, 5), "float32")],
                                   lambda g: _prims(g)[-1] == "reshape"),
}


@pytest.mark.parametrize("name", sorted(REWRITES))
def test_simplify_rewrites_keep_values_bit_for_bit(name):
    """Each rewrite of simplify (``passes/simplify.rs``) on a program that exercises it: the rewritten graph
    has the expected structure and the oracle computes the same bits from both (random inputs, twice)."""
    fn, shapes, check = REWRITES[name]
    g = L.make_graph(fn)(*[L.empty(list(s), d, "meta") for s, d in shapes])
    s = passes.frontend(g, matched=True)
    assert check(s), str(s)
    for seed in (0, 1):
        _same(g, s, seed)


def test_attention_with_a_different_value_head_dim_is_matched():
    """A value head dim other than the query's (16 vs 24, one of the reference's backward cases,
    ``passes/attention/forward.rs:721-735`` checks each head dim on its own): the forward and the backward become
    flash fusions reading V, O and dO at head dim 24 and Q, K at 16; the values are unchanged."""
    def grads(q, k, v, do):
        out, pull = L.vjp(lambda q, k, v: F.flash_attention(q, k, v, is_causal=True), q, k, v)
        return (out,) + pull(do)

    metas = [L.empty(s, "bfloat16", "meta") for s in ([1, 3, 2, 16], [1, 50, 1, 16], [1, 50, 1, 24], [1, 3, 2, 24])]
    g = L.make_graph(grads)(*metas)
    m = attention.match(passes.frontend(g))
    assert [n.params["name"] for n in m.nodes if n.prim == "fusion"] == ["flash_attention", "flash_attention_backward"]
    _same(g, m)
