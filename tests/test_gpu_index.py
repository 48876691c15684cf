"""Integer and indexing primitives on the GPU, bit for bit against the CPU oracle (the reference
interpreter's semantics, ``lumen/reference/mod.rs:415-462,738-856``): gathers and take_along_axis with
indices clamped into the axis, integer scatter_add, argmax/argmin with ties and NaN
(``functional/functions.py:613-638``), iota/compare masks, static slices (contiguous blocks and windows), dynamic slices with traced starts, integer
reductions with two's-complement wrap, saturating float-to-int casts and integer bit operations."""

import numpy as np
import pytest

import lumen_amd as L
import lumen_amd.functional as F
from lumen_amd import dtypes as D
from lumen_amd.graph import prims
from oracle import oracle

pytestmark = pytest.mark.gpu


def _tensor(a):
    if a.dtype == np.uint16:  # bf16 bit patterns
        return L.tensor(D.bf16_to_f32(a), "bfloat16")
    return L.from_numpy(a)


def _check(fn, *arrays, kinds=None):
    """Runs ``fn`` compiled for hip and through the oracle; every output must be identical bit for bit."""
    args = [_tensor(a) for a in arrays]
    f = L.compile(fn, device="hip")
    got = f(*args)
    got = [np.asarray(t.raw()) for t in (got if isinstance(got, (tuple, list)) else [got])]  # storage
    want = oracle.run(L.make_graph(fn)(*args), list(arrays))  # storage (bf16 as its 16-bit pattern)
    assert len(got) == len(want)
    for i, (g, w) in enumerate(zip(got, want)):
        assert g.shape == w.shape and g.dtype == w.dtype, (i, g.shape, g.dtype, w.shape, w.dtype)
        if w.dtype.kind == "f":  # compare bit patterns (NaN payloads and signed zeros included)
            g, w = g.view(f"u{w.dtype.itemsize}"), w.view(f"u{w.dtype.itemsize}")
        np.testing.assert_array_equal(g, w, err_msg=f"output {i}")
    if kinds is not None:
        assert {s["kind"] for s in f.plan.describe()} <= set(kinds)
    return got


def _bf16(a):
    return D.bf16_bits(np.asarray(a, np.float32))


def test_static_slices_in_loops(hip):
    """Static slices read inside loop kernels, bit for bit: contiguous blocks of their operand (rows of a
    packed [6144, 2048] bf16 weight gradient, whose flat index is the slice's plus an aligned offset and takes
    vector loads; a block of a float32 [3, 7, 10] at an offset of 90 elements, off the vector width; one row of
    an odd-width [5, 33]) and a window that is not one block ([5, 8] rows 1-3, columns 2-5)."""
    rng = np.random.default_rng(3)
    g = _bf16(rng.standard_normal((6144, 2048)))
    w = _bf16(rng.standard_normal((2048, 2048)))
    got = _check(lambda g, w: w - prims.slice(g, [4096, 0], [6144, 2048]) * 0.25, g, w, kinds=["loop"])
    assert got[0].shape == (2048, 2048)
    x = rng.standard_normal((3, 7, 10)).astype(np.float32)
    _check(lambda x: prims.slice(x, [1, 2, 0], [2, 5, 10]) * 3.0 + 1.0, x)
    y = rng.standard_normal((5, 33)).astype(np.float32)
    _check(lambda y: prims.slice(y, [2, 0], [3, 33]) * 2.0 - 1.0, y)
    z = rng.standard_normal((5, 8)).astype(np.float32)
    _check(lambda z: prims.slice(z, [1, 2], [4, 6]) - 0.5, z)


def test_embedding_gather_clamps_ids(hip):
    """A token-embedding gather ([vocab, d] table, [b, s] ids), with ids below 0 and past the vocabulary
    that both sides clamp to the first and last row; bf16 and int32 tables, int64 and int32 ids."""
    rng = np.random.default_rng(0)
    table = _bf16(rng.standard_normal((1000, 64)))
    ids = rng.integers(-20, 1020, (8, 300)).astype(np.int64)
    ids[0, :4] = [-1, 0, 999, 1000]
    _check(lambda t, i: prims.gather(t, i, 0), table, ids, kinds=["loop"])
    itab = rng.integers(-(2**31), 2**31 - 1, (50, 24), dtype=np.int64).astype(np.int32)
    ids32 = rng.integers(-3, 55, (7, 5)).astype(np.int32)
    _check(lambda t, i: prims.gather(t, i, 0), itab, ids32)
    # along a middle axis
    x = rng.standard_normal((4, 30, 6)).astype(np.float32)
    k = rng.integers(-2, 33, (3, 9)).astype(np.int64)
    _check(lambda t, i: prims.gather(t, i, 1), x, k)


def test_take_along_axis_clamps_each_index(hip):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((64, 100)).astype(np.float32)
    k = rng.integers(-5, 105, (64, 7)).astype(np.int32)
    _check(lambda v, i: prims.take_along_axis(v, i, 1), x, k)
    xi = rng.integers(-1000, 1000, (9, 33)).astype(np.int64)
    k0 = rng.integers(-2, 12, (4, 33)).astype(np.int64)
    _check(lambda v, i: prims.take_along_axis(v, i, 0), xi, k0)


def test_integer_scatter_add_is_exact(hip):
    """Integer scatter_add (wrapping int32 sums, repeated and clamped indices) and a float32 one whose
    updates are small integers (every partial sum exact, so the GPU's accumulation order cannot show)."""
    rng = np.random.default_rng(2)
    x = rng.integers(-(2**31), 2**31 - 1, (100, 16), dtype=np.int64).astype(np.int32)
    ids = rng.integers(-3, 103, 500).astype(np.int64)
    upd = rng.integers(-(2**30), 2**30, (500, 16)).astype(np.int32)
    _check(lambda a, i, u: prims.scatter_add(a, i, u, 0), x, ids, upd)
    xf = np.zeros((64, 8), np.float32)
    idf = rng.integers(0, 64, (40, 30)).astype(np.int32)
    uf = rng.integers(-8, 9, (40, 30, 8)).astype(np.float32)
    _check(lambda a, i, u: prims.scatter_add(a, i, u, 0), xf, idf, uf)


def test_float_scatter_add_of_rows(hip):
    """float32 scatter_add of whole rows along axis 0 (an embedding gradient's form: [B, S] ids, [B, S, D]
    updates into [V, D]) with repeated ids and ids clamped from below and above: bit for bit with small-integer
    updates (every partial sum exact), and within float32 reassociation (rtol 1e-5 of the summed magnitudes)
    with normal ones."""
    rng = np.random.default_rng(4)
    x = rng.integers(-4, 5, (300, 512)).astype(np.float32)
    ids = rng.integers(-5, 305, (7, 90)).astype(np.int64)
    ids[0, :40] = 17  # one row hit 40 times
    upd = rng.integers(-8, 9, (7, 90, 512)).astype(np.float32)
    got = _check(lambda a, i, u: prims.scatter_add(a, i, u, 0), x, ids, upd, kinds={"scatter_add", "copy", "fill"})
    uf = rng.standard_normal((7, 90, 512)).astype(np.float32)
    fn = lambda a, i, u: prims.scatter_add(a, i, u, 0)  # noqa: E731
    f = L.compile(fn, device="hip")
    out = np.asarray(L.to_numpy(f(L.from_numpy(x), L.from_numpy(ids), L.from_numpy(uf))), np.float64)
    (want,) = oracle.run(L.make_graph(fn)(*[L.from_numpy(a) for a in (x, ids, uf)]), [x, ids, uf])
    mag = np.abs(x).astype(np.float64)
    np.add.at(mag, np.clip(ids, 0, 299).ravel(), np.abs(uf).reshape(-1, 512))
    assert np.all(np.abs(out - want) <= 1e-5 * mag + 1e-6)
    del got


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_argmax_argmin_ties_and_nan(hip, dtype):
    """The first index of the maximum / minimum: ties resolve to the smallest position, a row holding NaN
    has no equal element (its maximum is NaN) and yields the axis length, as in the reference."""
    rng = np.random.default_rng(3)
    x = rng.integers(-3, 4, (96, 257)).astype(np.float32)  # many ties
    x[5, 17] = np.nan
    x[7] = 2.0
    x[9, 100:] = np.inf
    a = _bf16(x) if dtype == "bfloat16" else x

    def fn(v):
        return F.argmax(v, -1), F.argmin(v, 1, keepdim=True), F.argmax(v, 0), F.argmin(v)

    got = _check(fn, a)
    assert got[0][7] == 0 and got[0][5] == 257 and got[0][9] == 100  # ties, NaN row, first +inf


def test_integer_argmax_and_reductions_wrap(hip):
    rng = np.random.default_rng(4)
    x = rng.integers(-(2**31), 2**31 - 1, (33, 129), dtype=np.int64).astype(np.int32)
    x[3] = 7

    def fn(v):
        return (F.argmax(v, 1), prims.reduce_sum(v, (1,), "int32"), prims.reduce_max(v, (0,)),
                F.amin(v, 1))

    _check(fn, x)


def test_iota_compare_masks_and_select(hip):
    """A causal mask built from iotas (``k <= q + offset``), equality and less-than masks on integers,
    and a select through them: the boolean and integer results bit for bit."""
    rng = np.random.default_rng(5)
    s = rng.standard_normal((2, 64, 96)).astype(np.float32)

    def fn(x):
        q = prims.iota("int32", x.shape, 1)
        k = prims.iota("int32", x.shape, 2)
        allowed = prims.lt(k, q + 33)  # k <= q + 32
        m = prims.select(allowed, x, prims.full(x.shape, float("-inf"), "float32"))
        same = prims.eq(prims.rem(k, prims.full(x.shape, 7, "int32")), prims.rem(q, prims.full(x.shape, 7, "int32")))
        return m, allowed, same, prims.cast(allowed, "int32") + prims.cast(same, "int32")

    _check(fn, s)


def test_dynamic_slice_with_traced_clamped_start(hip):
    rng = np.random.default_rng(6)
    x = rng.standard_normal((12, 80)).astype(np.float32)
    for start in (0, 17, 70, 1000, -5):
        k = np.array(start, np.int32)
        _check(lambda v, i: prims.dynamic_slice(v, [3, i], (4, 16)), x, k)


def test_casts_bitwise_and_shifts(hip):
    """Saturating float-to-int casts (NaN to 0, out-of-range to the limits), integer bit operations and
    shifts with amounts outside the width (0, or -1 for arithmetic shifts of negatives)."""
    f = np.array([1e10, -1e10, np.nan, 3.7, -3.7, 255.5, -0.5, 2.0**31, np.inf, -np.inf] * 13, np.float32)
    _check(lambda v: (prims.cast(v, "int32"), prims.cast(v, "uint8"), prims.cast(v, "int64"), prims.cast(v, "int8")), f)
    rng = np.random.default_rng(7)
    a = rng.integers(-(2**31), 2**31 - 1, 777, dtype=np.int64).astype(np.int32)
    b = rng.integers(-3, 36, 777).astype(np.int32)

    def ops(x, y):
        return (prims.shift_left(x, y), prims.shift_right_logical(x, y), prims.shift_right_arithmetic(x, y),
                prims.and_(x, y), prims.or_(x, y), prims.xor(x, y), prims.not_(x), prims.div(x, y), prims.rem(x, y),
                x * y, x - y)

    _check(ops, a, b)
    u = rng.integers(0, 2**32 - 1, 513, dtype=np.uint64).astype(np.uint32)
    v = rng.integers(0, 40, 513).astype(np.uint32)
    _check(lambda x, y: (prims.shift_right_logical(x, y), prims.shift_left(x, y), x + y, prims.cast(x, "float32")), u, v)
