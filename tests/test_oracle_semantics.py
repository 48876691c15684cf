"""Each primitive of the oracle against an independent closed form (NumPy), on small traced programs:
float rounding per result dtype, integer wraparound and XLA's division/remainder-by-zero rules, saturating
casts, NaN-propagating max, the sequential float32 dot fold, reductions in input order, index ops with
clamped indices."""

import numpy as np

import lumen_amd as L
import lumen_amd.functional as F
from lumen_amd import dtypes as D
from lumen_amd.graph import prims
from oracle import oracle


def _run(fn, *arrays):
    metas = [L.empty(list(a.shape), D.canonical(a.dtype) if a.dtype != np.uint16 else "bfloat16", "meta") for a in arrays]
    g = L.make_graph(fn)(*metas)
    return oracle.run(g, list(arrays))


def test_float32_arithmetic_is_correctly_rounded():
    rng = np.random.default_rng(0)
    x, y = rng.standard_normal((2, 1000)).astype(np.float32)
    for op, ref in ((prims.add, np.add), (prims.sub, np.subtract), (prims.mul, np.multiply), (prims.div, np.divide)):
        (got,) = _run(lambda a, b, op=op: op(a, b), x, y)
        np.testing.assert_array_equal(got, ref(x, y))


def test_bf16_arithmetic_rounds_the_exact_result_once():
    rng = np.random.default_rng(1)
    x = D.bf16_bits(rng.standard_normal(500).astype(np.float32))
    y = D.bf16_bits(rng.standard_normal(500).astype(np.float32))
    (got,) = _run(lambda a, b: a * b + a, x, y)
    xf, yf = D.bf16_to_f32(x).astype(np.float64), D.bf16_to_f32(y).astype(np.float64)
    prod = D.bf16_bits(xf * yf)
    want = D.bf16_bits(D.bf16_to_f32(prod).astype(np.float64) + xf)
    np.testing.assert_array_equal(got, want)


def test_integer_wraparound_and_division_by_zero():
    a = np.array([2**31 - 1, -(2**31), 7, -7, 5], np.int32)
    b = np.array([1, -1, 0, 2, 0], np.int32)
    (s,) = _run(prims.add, a, b)
    np.testing.assert_array_equal(s, (a.astype(np.int64) + b).astype(np.int32))
    (q,) = _run(prims.div, a, b)
    np.testing.assert_array_equal(q, [2**31 - 1, -(2**31), -1, -3, -1])  # truncation; x / 0 = -1
    (r,) = _run(prims.rem, a, b)
    np.testing.assert_array_equal(r, [0, 0, 7, -1, 5])  # x % 0 = x


def test_saturating_casts_and_nan_to_zero():
    x = np.array([1e10, -1e10, np.nan, 3.7, -3.7, 255.5], np.float32)
    (i,) = _run(lambda v: prims.cast(v, "int32"), x)
    np.testing.assert_array_equal(i, [2**31 - 1, -(2**31), 0, 3, -3, 255])
    (u,) = _run(lambda v: prims.cast(v, "uint8"), x)
    np.testing.assert_array_equal(u, [255, 0, 0, 3, 0, 255])


def test_max_propagates_nan():
    x = np.array([1.0, np.nan, 2.0], np.float32)
    y = np.array([np.nan, 0.0, 1.0], np.float32)
    (m,) = _run(prims.max, x, y)
    assert np.isnan(m[0]) and np.isnan(m[1]) and m[2] == 2.0


def test_f32_dot_is_the_sequential_fold():
    rng = np.random.default_rng(2)
    a = rng.standard_normal((5, 37)).astype(np.float32)
    b = rng.standard_normal((37, 3)).astype(np.float32)
    (got,) = _run(lambda x, y: F.matmul(x, y, "float32", "float32"), a, b)
    acc = np.zeros((5, 3), np.float32)
    for k in range(37):
        acc = (acc + (a[:, k : k + 1] * b[k : k + 1, :]).astype(np.float32)).astype(np.float32)
    np.testing.assert_array_equal(got, acc)


def test_bf16_dot_equals_float64_einsum_rounded():
    """bf16 x bf16 products are exact in float32; the fold then differs from float64 by float32 rounding."""
    rng = np.random.default_rng(3)
    a = D.bf16_bits(rng.standard_normal((4, 64)).astype(np.float32))
    b = D.bf16_bits(rng.standard_normal((64, 6)).astype(np.float32))
    (got,) = _run(lambda x, y: F.matmul(x, y, "float32", "float32"), a, b)
    want = D.bf16_to_f32(a).astype(np.float64) @ D.bf16_to_f32(b).astype(np.float64)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def test_reduce_sum_folds_in_input_order():
    x = np.array([[1e8, 1.0, -1e8, 1.0]], np.float32)
    (s,) = _run(lambda v: prims.reduce_sum(v, (1,), "float32"), x)
    assert s[0] == np.float32(np.float32(np.float32(1e8 + 1.0) - 1e8) + 1.0)


def test_layout_ops():
    x = np.arange(24, dtype=np.float32).reshape(2, 3, 4)
    (t,) = _run(lambda v: prims.transpose(v, (2, 0, 1)), x)
    np.testing.assert_array_equal(t, x.transpose(2, 0, 1))
    (b,) = _run(lambda v: prims.broadcast_in_dim(v[:, :1, :], (2, 5, 4), (0, 1, 2)), x)
    np.testing.assert_array_equal(b, np.broadcast_to(x[:, :1, :], (2, 5, 4)))
    (c,) = _run(lambda v: prims.concatenate([v, v[:, :1]], 1), x)
    np.testing.assert_array_equal(c, np.concatenate([x, x[:, :1]], 1))
    (i,) = _run(lambda v: prims.add(prims.iota("float32", v.shape, 2), v), x)
    np.testing.assert_array_equal(i, x + np.arange(4))


def test_gather_and_scatter_add_clamp_indices():
    x = np.arange(12, dtype=np.float32).reshape(4, 3)
    idx = np.array([[0, 3], [5, -2]], np.int64)
    (g,) = _run(lambda v, k: prims.gather(v, k, 0), x, idx)
    np.testing.assert_array_equal(g, x[np.clip(idx, 0, 3)])
    u = np.ones((2, 2, 3), np.float32)
    (s,) = _run(lambda v, k, w: prims.scatter_add(v, k, w, 0), x, idx, u)
    want = x.copy()
    for k in np.clip(idx, 0, 3).ravel():
        want[k] += 1
    np.testing.assert_array_equal(s, want)


def test_softmax_and_cross_entropy_closed_forms():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((6, 10)).astype(np.float64)
    t = rng.integers(0, 10, 6).astype(np.int64)
    (p,) = _run(lambda v: F.softmax(v, -1), x)
    e = np.exp(x - x.max(-1, keepdims=True))
    np.testing.assert_allclose(p, e / e.sum(-1, keepdims=True), rtol=1e-14)
    (ce,) = _run(lambda v, k: F.cross_entropy(v, k), x, t)
    lse = np.log(np.exp(x).sum(-1))
    np.testing.assert_allclose(ce, lse - x[np.arange(6), t], rtol=1e-12)
