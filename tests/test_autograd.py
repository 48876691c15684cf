"""Reverse-mode rules checked against central finite differences: float64 programs traced with
``value_and_grad``, the gradient graph evaluated by the oracle, the differences from the forward graph."""

import numpy as np
import pytest

import lumen_amd as L
import lumen_amd.functional as F
from lumen_amd.graph import prims
from oracle import oracle

FNS = {
    "exp_log_tanh": lambda x, w: F.sum(F.tanh(F.exp(x * 0.3) * w[:4]) + F.log(x * x + 1.0)),
    "softmax_matmul": lambda x, w: F.sum(F.softmax(F.matmul(x, w, "float64", "float64"), -1) * w[:, :1].t()),
    "rms_norm": lambda x, w: F.sum(F.rms_norm(x, x.shape[-1], w[:, 0]) * F.sigmoid(x)),
    "layer_norm_gelu": lambda x, w: F.mean(F.gelu(F.layer_norm(x, x.shape[-1]) * w[:, 0])),
    "max_div_sqrt": lambda x, w: F.sum(F.maximum(x, w[:, 0]) / F.sqrt(x * x + 2.0)),
    "amax_transpose": lambda x, w: F.sum(F.amax(x.t(), -1) * 2.0) + F.sum(F.matmul(w, x.t(), "float64", "float64")),
    "cross_entropy": lambda x, w: F.mean(F.cross_entropy(F.matmul(x, w, "float64", "float64"), _targets(x.shape[0]))),
    "gather_slice_concat": lambda x, w: F.sum(F.cat([x[1:3], x[:1] * 3.0], 0) * x[1:4, :1]) + F.sum(x[_idx()] * 2.0),
}


def _targets(n):
    return prims.iota("int64", [n], 0) - prims.iota("int64", [n], 0) + prims.full([n], 2, "int64")


def _idx():
    return prims.iota("int64", [3], 0)


@pytest.mark.parametrize("name", sorted(FNS))
def test_gradients_match_finite_differences(name):
    fn = FNS[name]
    rng = np.random.default_rng(0)
    x = rng.standard_normal((4, 6)) + 0.5
    w = rng.standard_normal((6, 6)) * 0.5
    metas = [L.empty([4, 6], "float64", "meta"), L.empty([6, 6], "float64", "meta")]
    g_grad = L.make_graph(lambda a, b: L.value_and_grad(fn, (0, 1))(a, b))(*metas)
    outs = oracle.run(g_grad, [x, w])
    gx, gw = outs[1], outs[2]
    g_f = L.make_graph(fn)(*metas)

    def f(a, b):
        return float(oracle.run(g_f, [a, b])[0])

    h = 1e-6
    for arr, grad, which in ((x, gx, 0), (w, gw, 1)):
        num = np.zeros_like(arr)
        for i in np.ndindex(arr.shape):
            p, m = arr.copy(), arr.copy()
            p[i] += h
            m[i] -= h
            args_p = (p, w) if which == 0 else (x, p)
            args_m = (m, w) if which == 0 else (x, m)
            num[i] = (f(*args_p) - f(*args_m)) / (2 * h)
        np.testing.assert_allclose(grad, num, rtol=1e-5, atol=1e-7, err_msg=f"{name} d{'xw'[which]}")


def test_backward_accumulates_into_grad():
    """``loss.backward()`` twice adds the gradients (torch semantics inside the trace)."""

    def f(x):
        y = F.sum(x * x)
        y.backward()
        y2 = F.sum(x * 3.0)
        y2.backward()
        return x.grad

    (g,) = oracle.run(L.make_graph(f)(L.empty([3], "float64", "meta")), [np.array([1.0, 2.0, 3.0])])
    np.testing.assert_allclose(g, [5.0, 7.0, 9.0])


def test_function_backward_is_used():
    """A ``Function``'s hand-written backward replaces the rules of its forward's primitives."""

    class Twice(L.autograd.Function):
        @staticmethod
        def forward(ctx, x):
            return x * 2.0

        @staticmethod
        def backward(ctx, g):
            return g * 10.0

    def f(x):
        return L.grad(lambda v: F.sum(Twice.apply(v)))(x)

    (g,) = oracle.run(L.make_graph(f)(L.empty([2], "float64", "meta")), [np.array([1.0, 2.0])])
    np.testing.assert_allclose(g, [10.0, 10.0])


@pytest.mark.parametrize("transposed", [False, True])
def test_fused_linear_cross_entropy_backward_matches_the_plain_gradient(transposed):
    """With fused_linear_cross_entropy_chunk_size, the gradient of mean(cross_entropy(h @ w')) is taken a row
    chunk at a time from the saved log-sum-exp (the logits recomputed per chunk): the graph has the chunk
    dots, and the oracle's gradients equal the plain graph's within the bf16 rounding of the logits gradient
    (rtol 2e-2 / atol 1e-2 of the largest, the bf16 bound) — bit for bit for the loss."""
    import lumen_amd.functional as F
    from lumen_amd import dtypes as D

    rows, feat, classes = 96, 32, 80
    rng = np.random.default_rng(2)
    h = D.bf16_bits(rng.standard_normal((rows, feat)).astype(np.float32))
    w = D.bf16_bits((0.3 * rng.standard_normal((feat, classes) if transposed else (classes, feat))).astype(np.float32))
    t = rng.integers(0, classes, rows).astype(np.int64)

    def loss(h, w, t):
        logits = F.matmul(h, w if transposed else w.t(), "float32", "float32")
        return F.mean(F.cross_entropy(logits, t))

    metas = [L.empty(list(h.shape), "bfloat16", "meta"), L.empty(list(w.shape), "bfloat16", "meta"),
             L.empty([rows], "int64", "meta")]
    outs = {}
    for chunk in (None, 40):
        with L.config.compiler.patch(fused_linear_cross_entropy_chunk_size=chunk):
            g = L.make_graph(lambda a, b, c: L.value_and_grad(loss, (0, 1))(a, b, c))(*metas)
        dots = sum(1 for n in g.nodes if n.prim == "dot_general")
        outs[chunk] = (dots, oracle.run(g, [h, w, t]))
    assert outs[40][0] == 1 + 3 * 3 and outs[None][0] == 3  # forward + 3 chunks x (logits, dh, dw)
    assert np.array_equal(np.asarray(outs[None][1][0]), np.asarray(outs[40][1][0]))  # the loss
    for a, b in zip(outs[None][1][1:], outs[40][1][1:]):
        a = D.bf16_to_f32(a) if a.dtype == np.uint16 else np.asarray(a, np.float32)
        b = D.bf16_to_f32(b) if b.dtype == np.uint16 else np.asarray(b, np.float32)
        np.testing.assert_allclose(b, a, rtol=2e-2, atol=1e-2 * np.abs(a).max())
