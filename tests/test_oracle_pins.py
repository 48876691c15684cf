"""Pins of the oracle's remaining primitives, each against something independent of its code: NumPy's
float64 functions rounded once to the result dtype, mathematical identities and special values, Python's
unbounded integers for bit operations, and NumPy's index routines with the reference's clamping
(``lumen/reference/mod.rs:415-424`` clamps gathered indices into the axis; ``:498-600`` the unary and
binary families; ``:715-729,809-833`` dynamic slices; ``:834-870`` cumsum)."""

import numpy as np
import pytest

import lumen_amd as L
from lumen_amd import dtypes as D
from lumen_amd.graph import prims
from oracle import oracle


def _run(fn, *arrays, uint16_is_bf16=True):
    def dt(a):
        return "bfloat16" if (a.dtype == np.uint16 and uint16_is_bf16) else D.canonical(a.dtype)

    metas = [L.empty(list(a.shape), dt(a), "meta") for a in arrays]
    g = L.make_graph(fn)(*metas)
    return oracle.run(g, list(arrays))


def _f32_ulps(a, b):
    def key(v):
        u = np.asarray(v, np.float32).view(np.int32).astype(np.int64)
        return np.where(u < 0, -(u & 0x7FFFFFFF), u)
    return np.abs(key(a) - key(b))


_UNARY = {
    "sin": (np.sin, (-10, 10)), "cos": (np.cos, (-10, 10)), "tan": (np.tan, (-1.5, 1.5)),
    "asin": (np.arcsin, (-1, 1)), "acos": (np.arccos, (-1, 1)), "atan": (np.arctan, (-20, 20)),
    "sinh": (np.sinh, (-5, 5)), "cosh": (np.cosh, (-5, 5)), "asinh": (np.arcsinh, (-50, 50)),
    "acosh": (np.arccosh, (1, 50)), "atanh": (np.arctanh, (-0.999, 0.999)),
    "log1p": (np.log1p, (-0.999, 10)), "expm1": (np.expm1, (-5, 5)), "exp2": (np.exp2, (-30, 30)),
    "log2": (np.log2, (1e-3, 1e3)), "cbrt": (np.cbrt, (-100, 100)),
    "rsqrt": (lambda v: 1.0 / np.sqrt(v), (1e-3, 1e3)),
    "logistic": (lambda v: 1.0 / (1.0 + np.exp(-v)), (-30, 30)),
}


@pytest.mark.parametrize("name", sorted(_UNARY))
def test_float_unary_is_float64_function_rounded_once(name):
    """Each float unary evaluated in float64 and rounded once: float32 results within one ulp of NumPy's
    float64 function rounded to float32 (libm implementations may differ in the last float64 bit, which
    can move a tie-adjacent float32 rounding by one), and exactly equal on at least 99.9% of inputs."""
    ref, (lo, hi) = _UNARY[name]
    rng = np.random.default_rng(len(name))
    x = rng.uniform(lo, hi, 4000).astype(np.float32)
    op = getattr(prims, name)
    (got,) = _run(op, x)
    want = ref(x.astype(np.float64)).astype(np.float32)
    assert _f32_ulps(got, want).max() <= 1
    assert (got == want).mean() >= 0.999


def test_float_unary_identities_and_special_values():
    """Values the mathematics fixes, so a swapped function (sin for cos, log2 for log1p) or a dropped term
    fails: identities on random inputs and the special points of each function."""
    rng = np.random.default_rng(9)
    x = rng.uniform(-3, 3, 256)
    (s,) = _run(prims.sin, x)
    (c,) = _run(prims.cos, x)
    np.testing.assert_allclose(s * s + c * c, 1.0, rtol=1e-15)
    (e,) = _run(prims.expm1, x)
    (l,) = _run(prims.log1p, e)
    np.testing.assert_allclose(l, x, rtol=1e-14, atol=1e-15)
    (t,) = _run(prims.exp2, x)
    (u,) = _run(prims.log2, t)
    np.testing.assert_allclose(u, x, rtol=1e-14, atol=1e-15)
    (sh,) = _run(prims.sinh, x)
    (ash,) = _run(prims.asinh, sh)
    np.testing.assert_allclose(ash, x, rtol=1e-13, atol=1e-15)
    (cb,) = _run(prims.cbrt, x)
    np.testing.assert_allclose(cb * cb * cb, x, rtol=1e-14, atol=1e-15)
    (rs,) = _run(prims.rsqrt, np.abs(x) + 0.5)
    np.testing.assert_allclose(rs * rs * (np.abs(x) + 0.5), 1.0, rtol=1e-15)
    (lg,) = _run(prims.logistic, x)
    (lg_neg,) = _run(prims.logistic, -x)
    np.testing.assert_allclose(lg + lg_neg, 1.0, rtol=1e-15)  # logistic(x) + logistic(-x) = 1

    sp = np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan, 8.0, -8.0, 2.0], np.float64)
    with np.errstate(all="ignore"):
        checks = {
            "cbrt": [0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan, 2.0, -2.0, np.cbrt(2.0)],
            "rsqrt": [np.inf, -np.inf, 1.0, np.nan, 0.0, np.nan, np.nan, 8.0 ** -0.5, np.nan, 0.5 ** 0.5],
            "log2": [-np.inf, -np.inf, 0.0, np.nan, np.inf, np.nan, np.nan, 3.0, np.nan, 1.0],
            "exp2": [1.0, 1.0, 2.0, 0.5, np.inf, 0.0, np.nan, 256.0, 1 / 256.0, 4.0],
            "log1p": [0.0, -0.0, np.log(2.0), -np.inf, np.inf, np.nan, np.nan, np.log(9.0), np.nan, np.log(3.0)],
            "logistic": [0.5, 0.5, 1 / (1 + np.exp(-1.0)), 1 / (1 + np.e), 1.0, 0.0, np.nan,
                         1 / (1 + np.exp(-8.0)), 1 / (1 + np.exp(8.0)), 1 / (1 + np.exp(-2.0))],
            "asin": [0.0, -0.0, np.pi / 2, -np.pi / 2, np.nan, np.nan, np.nan, np.nan, np.nan, np.nan],
            "acosh": [np.nan, np.nan, 0.0, np.nan, np.inf, np.nan, np.nan, np.arccosh(8.0), np.nan, np.arccosh(2.0)],
            "atanh": [0.0, -0.0, np.inf, -np.inf, np.nan, np.nan, np.nan, np.nan, np.nan, np.nan],
        }
    for name, want in checks.items():
        (got,) = _run(getattr(prims, name), sp)
        np.testing.assert_allclose(got, want, rtol=1e-15, err_msg=name)
        zeros = np.asarray(want[:2]) == 0  # the sign of a zero result is part of the closed form
        assert np.array_equal(np.signbit(got[:2])[zeros], np.signbit(np.asarray(want[:2]))[zeros]), name


def test_round_floor_ceil_ties_and_signs():
    """``round`` rounds halves to even (``round_ties_even``, reference ``mod.rs:530``), keeping the sign of
    zero; floor and ceil toward -inf and +inf."""
    x = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 2.4999, -2.6, 1e300, -0.0, 3.0], np.float64)
    (r,) = _run(prims.round, x)
    np.testing.assert_array_equal(r, [0.0, 2.0, 2.0, -0.0, -2.0, -2.0, 2.0, -3.0, 1e300, -0.0, 3.0])
    assert np.signbit(r[3]) and np.signbit(r[9])
    (f,) = _run(prims.floor, x)
    np.testing.assert_array_equal(f, np.floor(x))
    (c,) = _run(prims.ceil, x)
    np.testing.assert_array_equal(c, np.ceil(x))
    assert np.signbit(c[3])  # ceil(-0.5) = -0
    xb = D.bf16_bits(np.array([2.5, -3.5, 0.75], np.float32))
    (rb,) = _run(prims.round, xb)
    np.testing.assert_array_equal(D.bf16_to_f32(rb), [2.0, -4.0, 1.0])


_INT_TYPES = [(np.int8, 8, True), (np.uint8, 8, False), (np.int16, 16, True), (np.uint16, 16, False),
              (np.int32, 32, True), (np.uint32, 32, False), (np.int64, 64, True)]


def _bits(v, w):
    return int(v) & ((1 << w) - 1)


def _to_dtype(u, w, signed):
    u &= (1 << w) - 1
    return u - (1 << w) if signed and u >> (w - 1) else u


@pytest.mark.parametrize("dt,w,signed", _INT_TYPES)
def test_clz_and_population_count_on_the_bit_pattern(dt, w, signed):
    info = np.iinfo(dt)
    vals = [0, 1, 2, 3, info.max, info.min, info.max // 3, 5]
    if signed:
        vals += [-1, -2, -(2 ** (w - 2))]
    x = np.array(vals, dt)
    (pc,) = _run(prims.population_count, x, uint16_is_bf16=False)
    (lz,) = _run(prims.clz, x, uint16_is_bf16=False)
    for v, p, z in zip(vals, pc, lz):
        u = _bits(v, w)
        assert int(p) == bin(u).count("1"), (v, p)
        assert int(z) == w - u.bit_length(), (v, z)


@pytest.mark.parametrize("dt,w,signed", _INT_TYPES)
def test_shifts_saturate_outside_the_width(dt, w, signed):
    """Shift amounts in [0, width) shift; amounts below 0 or at least the width give 0, or -1 for an
    arithmetic right shift of a negative value (reference ``mod.rs:571-578``)."""
    info = np.iinfo(dt)
    base = [1, info.max, info.min, 5, 0] + ([-1, -7] if signed else [])
    amounts = [-1, 0, 1, w // 2, w - 1, w, w + 3]
    a = np.array([v for v in base for _ in amounts], dt)
    b = np.array([s % (1 << w) if (s < 0 and not signed) else s for _ in base for s in amounts], dt)
    (sl,) = _run(prims.shift_left, a, b, uint16_is_bf16=False)
    (srl,) = _run(prims.shift_right_logical, a, b, uint16_is_bf16=False)
    (sra,) = _run(prims.shift_right_arithmetic, a, b, uint16_is_bf16=False)
    for i in range(a.size):
        v, s = int(a[i]), int(b[i])
        u = _bits(v, w)
        sv = _to_dtype(u, w, True)
        if 0 <= s < w:
            want_l = _to_dtype(u << s, w, signed)
            want_rl = _to_dtype(u >> s, w, signed)
            want_ra = _to_dtype(sv >> s, w, signed)
        else:
            want_l = want_rl = 0
            want_ra = _to_dtype(-1, w, signed) if sv < 0 else 0
        assert (int(sl[i]), int(srl[i]), int(sra[i])) == (want_l, want_rl, want_ra), (dt, v, s)


def test_cumsum_forward_reverse_and_integer_wrap():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 5, 4)).astype(np.float32)
    for axis in range(3):
        (f,) = _run(lambda v, a=axis: prims.cumsum(v, a, False, "float32"), x)
        np.testing.assert_array_equal(f, np.add.accumulate(x, axis=axis, dtype=np.float32))
        (r,) = _run(lambda v, a=axis: prims.cumsum(v, a, True, "float32"), x)
        flip = np.flip(np.add.accumulate(np.flip(x, axis), axis=axis, dtype=np.float32), axis)
        np.testing.assert_array_equal(r, flip)
    # rounded after every add: 2^24 + 1 + 1 stays 2^24 in float32
    y = np.array([2.0 ** 24, 1.0, 1.0, 4.0], np.float32)
    (c,) = _run(lambda v: prims.cumsum(v, 0, False, "float32"), y)
    np.testing.assert_array_equal(c, [2.0 ** 24, 2.0 ** 24, 2.0 ** 24, 2.0 ** 24 + 4])
    z = np.array([2**31 - 2, 1, 1, 5], np.int32)
    (ci,) = _run(lambda v: prims.cumsum(v, 0, False, "int32"), z)
    np.testing.assert_array_equal(ci, [2**31 - 2, 2**31 - 1, -(2**31), -(2**31) + 5])


def test_dynamic_slice_and_update_clamp_the_start():
    """Starts are clamped so the window lies inside the operand (XLA's rule, reference ``mod.rs:715-729``):
    a start past the end reads the last full window, a negative one the first."""
    x = np.arange(60, dtype=np.float32).reshape(5, 12)
    for (i, j) in [(0, 0), (2, 5), (4, 11), (-3, 100), (1, -1)]:
        si, sj = min(max(i, 0), 5 - 3), min(max(j, 0), 12 - 4)
        (d,) = _run(lambda v, i=i, j=j: prims.dynamic_slice(v, [i, j], (3, 4)), x)
        np.testing.assert_array_equal(d, x[si : si + 3, sj : sj + 4])
        u = -np.arange(12, dtype=np.float32).reshape(3, 4) - 1
        (w,) = _run(lambda v, t, i=i, j=j: prims.dynamic_update_slice(v, t, [i, j]), x, u)
        want = x.copy()
        want[si : si + 3, sj : sj + 4] = u
        np.testing.assert_array_equal(w, want)
    # traced (array) start indices behave the same
    idx = np.array(7, np.int32)
    (d,) = _run(lambda v, k: prims.dynamic_slice(v, [0, k], (5, 6)), x, idx)
    np.testing.assert_array_equal(d, x[:, 6:12])


def test_take_along_axis_clamps_each_index():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((4, 7)).astype(np.float32)
    idx = rng.integers(-3, 10, (4, 5)).astype(np.int64)
    for axis in (0, 1):
        ix = idx if axis == 1 else rng.integers(-2, 6, (6, 7)).astype(np.int64)
        (t,) = _run(lambda v, k, a=axis: prims.take_along_axis(v, k, a), x, ix)
        np.testing.assert_array_equal(t, np.take_along_axis(x, np.clip(ix, 0, x.shape[axis] - 1), axis))
    xi = np.arange(28, dtype=np.int32).reshape(4, 7) * -3
    (ti,) = _run(lambda v, k: prims.take_along_axis(v, k, 1), xi, idx)
    np.testing.assert_array_equal(ti, np.take_along_axis(xi, np.clip(idx, 0, 6), 1))


def test_float_binary_pow_rem_min_nextafter():
    """pow in float64 rounded once; float ``rem`` truncates like C's fmod (sign of the dividend); ``min``
    propagates NaN; ``nextafter`` steps one ulp of the result dtype, from zero to the smallest subnormal
    (reference ``mod.rs:344-372``)."""
    rng = np.random.default_rng(11)
    a = rng.uniform(0.1, 4, 500).astype(np.float32)
    b = rng.uniform(-3, 3, 500).astype(np.float32)
    (p,) = _run(prims.pow, a, b)
    want = np.power(a.astype(np.float64), b.astype(np.float64)).astype(np.float32)
    assert _f32_ulps(p, want).max() <= 1
    x = np.array([5.5, -5.5, 5.5, -5.5, 1.0, 0.0], np.float64)
    y = np.array([2.0, 2.0, -2.0, -2.0, np.inf, 3.0], np.float64)
    (r,) = _run(prims.rem, x, y)
    np.testing.assert_array_equal(r, [1.5, -1.5, 1.5, -1.5, 1.0, 0.0])
    (m,) = _run(prims.min, np.array([1.0, np.nan, -0.5], np.float32), np.array([0.5, 2.0, np.nan], np.float32))
    assert m[0] == 0.5 and np.isnan(m[1]) and np.isnan(m[2])
    f = np.array([1.0, 1.0, 0.0, 0.0, -1.0, 3.0, np.nan], np.float32)
    g = np.array([2.0, 0.0, 1.0, -1.0, -2.0, 3.0, 1.0], np.float32)
    (n,) = _run(prims.nextafter, f, g)
    want = np.nextafter(f, g)
    np.testing.assert_array_equal(n[:6], want[:6])
    assert np.isnan(n[6])
    (pi,) = _run(prims.pow, np.array([2.0, -3.0, 0.5], np.float32), np.array([10, 3, -2], np.int32))
    np.testing.assert_array_equal(pi, [1024.0, -27.0, 4.0])


def test_integer_bitwise_min_abs_sign_not_and_is_finite():
    a = np.array([5, -6, 2**31 - 1, -(2**31), 0], np.int32)
    b = np.array([3, 3, -1, 1, -7], np.int32)
    for op, ref in ((prims.and_, np.bitwise_and), (prims.or_, np.bitwise_or), (prims.xor, np.bitwise_xor),
                    (prims.min, np.minimum)):
        (got,) = _run(op, a, b)
        np.testing.assert_array_equal(got, ref(a, b))
    (n,) = _run(prims.not_, a)
    np.testing.assert_array_equal(n, ~a)
    (ab,) = _run(prims.abs, a)
    np.testing.assert_array_equal(ab, [5, 6, 2**31 - 1, -(2**31), 0])  # |int min| wraps to itself
    (sg,) = _run(prims.sign, a)
    np.testing.assert_array_equal(sg, [1, -1, 1, -1, 0])
    fb = np.array([True, False])
    (nb,) = _run(prims.not_, fb)
    np.testing.assert_array_equal(nb, [False, True])
    x = np.array([1.0, np.inf, -np.inf, np.nan, -0.0], np.float32)
    (fin,) = _run(prims.is_finite, x)
    np.testing.assert_array_equal(fin, [True, False, False, False, True])
    (fs,) = _run(prims.sign, x)
    np.testing.assert_array_equal(fs[:3], [1.0, 1.0, -1.0])
    assert np.isnan(fs[3]) and fs[4] == 0 and np.signbit(fs[4])


def test_swap_pairs_slice_and_select():
    x = np.arange(24, dtype=np.float32).reshape(3, 8)
    (s,) = _run(prims.swap_pairs, x)
    np.testing.assert_array_equal(s, x.reshape(3, 4, 2)[:, :, ::-1].reshape(3, 8))
    (sl,) = _run(lambda v: prims.slice(v, (1, 2), (3, 7)), x)
    np.testing.assert_array_equal(sl, x[1:3, 2:7])
    c = np.array([[True, False] * 4] * 3)
    (se,) = _run(lambda p, v: prims.select(p, v, prims.neg(v)), c, x)
    np.testing.assert_array_equal(se, np.where(c, x, -x))


# ---- exp, log, sqrt, tanh at float32 rounding; reduce_max; eq and lt; the identity transfer ops ----------
# (reference ``lumen/reference/mod.rs:603-612`` evaluates Exp/Log/Sqrt/Tanh in float64 and rounds once;
# ``:645-717`` folds ReduceMax from the dtype's lowest value with NaN propagation; ``:498-530`` the
# comparisons; the transfer and wait primitives return their operand unchanged.)

_UNARY_CORE = {
    "exp": (np.exp, (-80, 80)), "log": (np.log, (1e-30, 1e30)),
    "sqrt": (np.sqrt, (0.0, 1e6)), "tanh": (np.tanh, (-12, 12)),
}


@pytest.mark.parametrize("name", sorted(_UNARY_CORE))
def test_float32_exp_log_sqrt_tanh_are_float64_rounded_once(name):
    """float32 results within one ulp of NumPy's float64 function rounded once to float32, and equal to it
    on at least 99.9% of inputs; ``sqrt`` is correctly rounded in both, so it must match everywhere.
    ``log`` draws its inputs log-uniformly so every binade from 2^-100 to 2^100 is covered."""
    ref, (lo, hi) = _UNARY_CORE[name]
    rng = np.random.default_rng(100 + len(name))
    if name == "log":
        x = np.exp(rng.uniform(np.log(lo), np.log(hi), 4000)).astype(np.float32)
    else:
        x = rng.uniform(lo, hi, 4000).astype(np.float32)
    (got,) = _run(getattr(prims, name), x)
    assert got.dtype == np.float32
    want = ref(x.astype(np.float64)).astype(np.float32)
    assert _f32_ulps(got, want).max() <= 1
    assert (got == want).mean() >= (1.0 if name == "sqrt" else 0.999)


def test_bf16_exp_log_sqrt_tanh_round_once_to_bf16():
    """With bf16 operands the float64 value is rounded once to bf16 (round to nearest even): compared bit
    for bit with NumPy's float64 function rounded by the reference test's bf16 helper, on every bf16
    pattern in each function's domain."""
    pats = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    with np.errstate(invalid="ignore"):
        vals = D.bf16_to_f32(pats).astype(np.float64)
    for name, ref, keep in [("exp", np.exp, np.abs(vals) < 80), ("log", np.log, vals > 0),
                            ("sqrt", np.sqrt, vals >= 0), ("tanh", np.tanh, np.isfinite(vals))]:
        sel = pats[keep & np.isfinite(vals)]
        (got,) = _run(getattr(prims, name), sel)
        want = D.bf16_bits(ref(D.bf16_to_f32(sel).astype(np.float64)))
        assert np.array_equal(got, want), name


def test_exp_log_sqrt_tanh_special_values():
    """The special points each function fixes: exp(±0) = 1, exp(-inf) = 0, log(0) = -inf, log of a
    negative is NaN, sqrt(-0) = -0, sqrt of a negative is NaN, tanh keeps the sign of zero and saturates
    to ±1 (in float32 already above 9.01), and NaN propagates through all four."""
    sp = np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan, 4.0, -4.0, 20.0], np.float64)
    with np.errstate(all="ignore"):
        checks = {
            "exp": [1.0, 1.0, np.e, 1 / np.e, np.inf, 0.0, np.nan, np.exp(4.0), np.exp(-4.0), np.exp(20.0)],
            "log": [-np.inf, -np.inf, 0.0, np.nan, np.inf, np.nan, np.nan, np.log(4.0), np.nan, np.log(20.0)],
            "sqrt": [0.0, -0.0, 1.0, np.nan, np.inf, np.nan, np.nan, 2.0, np.nan, np.sqrt(20.0)],
            "tanh": [0.0, -0.0, np.tanh(1.0), -np.tanh(1.0), 1.0, -1.0, np.nan, np.tanh(4.0), -np.tanh(4.0), 1.0],
        }
    for name, want in checks.items():
        (got,) = _run(getattr(prims, name), sp)
        np.testing.assert_allclose(got, want, rtol=1e-15, err_msg=name)
        assert np.array_equal(np.signbit(got[:2]), np.signbit(np.asarray(want[:2]))), name
    (t32,) = _run(prims.tanh, np.array([9.2, -9.2, 1e-30, -1e-30], np.float32))
    np.testing.assert_array_equal(t32, np.array([1.0, -1.0, 1e-30, -1e-30], np.float32))
    (s32,) = _run(prims.sqrt, np.array([2.0, 1e-40, 3.0e38], np.float32))
    np.testing.assert_array_equal(s32, np.sqrt(np.array([2.0, 1e-40, 3.0e38], np.float32)))


def _reduce_max(x, axes, **kw):
    return _run(lambda v: prims.reduce_max(v, axes), x, **kw)[0]


def test_float_reduce_max_matches_numpy_with_nan_and_negative_rows():
    """float32/float64 reduce_max equals ``np.max`` over each axis set: all-negative rows (an identity of
    0 instead of -inf would show), ``-inf``-only rows, a NaN anywhere in a row making the row NaN (NaN
    after larger values and before them), and ±0 mixes."""
    rng = np.random.default_rng(21)
    for dt in (np.float32, np.float64):
        x = rng.normal(size=(5, 7, 9)).astype(dt)
        x[0] = -np.abs(x[0]) - 1.0          # all negative
        x[1, 2] = -np.inf                   # a -inf-only row along the last axis
        x[2, 3, 0] = np.nan                 # NaN first in its row
        x[2, 4, 8] = np.nan                 # NaN last in its row
        x[3, 5] = np.where(np.arange(9) % 2 == 0, -0.0, 0.0).astype(dt)
        for axes in ([2], [1], [0], [0, 2], [1, 2], [0, 1, 2]):
            got = _reduce_max(x, axes)
            want = np.max(x, axis=tuple(axes))
            assert got.dtype == dt
            np.testing.assert_array_equal(got, want, err_msg=f"{dt} {axes}")
        row = _reduce_max(x, [2])
        assert np.isneginf(row[1, 2]) and np.isnan(row[2, 3]) and np.isnan(row[2, 4])
        assert (row[0] < 0).all()


def test_bf16_reduce_max_and_integer_identities():
    """bf16 reduce_max is the bf16 pattern of the largest value (NaN propagated); integer reduce_max
    starts from the type's lowest value (so an all-negative int8/int32/int64 row keeps its maximum) and
    unsigned types from 0; an empty reduced axis gives that identity."""
    rng = np.random.default_rng(22)
    v = rng.normal(size=(6, 33)).astype(np.float32) - 3.0
    v[4, 10] = np.nan
    b = D.bf16_bits(v)
    got = _reduce_max(b, [1])
    want = D.bf16_bits(np.max(D.bf16_to_f32(b), axis=1))
    assert np.array_equal(got[np.arange(6) != 4], want[np.arange(6) != 4])
    assert np.isnan(D.bf16_to_f32(got[4:5]))[0]
    for dt in (np.int8, np.int32, np.int64, np.uint8, np.uint32):
        info = np.iinfo(dt)
        x = rng.integers(info.min, info.max, size=(4, 17), endpoint=True, dtype=dt)
        if info.min < 0:
            x[1] = rng.integers(info.min, 0, size=17, dtype=dt)
            x[2] = info.min
        got = _reduce_max(x, [1])
        np.testing.assert_array_equal(got, np.max(x, axis=1), err_msg=str(dt))
        (empty,) = _run(lambda t: prims.reduce_max(t, [1]), np.zeros((3, 0), dt))
        np.testing.assert_array_equal(empty, np.full(3, info.min, dt), err_msg=str(dt))
    (fempty,) = _run(lambda t: prims.reduce_max(t, [0]), np.zeros((0, 2), np.float32))
    np.testing.assert_array_equal(fempty, np.full(2, -np.inf, np.float32))


def test_eq_and_lt_follow_ieee_and_integer_order():
    """eq and lt give bool: NaN compares unequal and unordered (even to itself), -0 == +0 and not
    -0 < +0, infinities order at the ends; integer comparisons use the full width (no wrap in a
    difference), including unsigned values above the signed range."""
    a = np.array([np.nan, np.nan, -0.0, 0.0, -np.inf, 1.0, 2.0, np.inf, 3.0], np.float32)
    b = np.array([np.nan, 1.0, 0.0, -0.0, np.inf, 1.0, 1.0, np.inf, np.nan], np.float32)
    (e,) = _run(prims.eq, a, b)
    (l,) = _run(prims.lt, a, b)
    assert e.dtype == np.bool_ and l.dtype == np.bool_
    np.testing.assert_array_equal(e, a == b)
    np.testing.assert_array_equal(l, a < b)
    for dt in (np.int8, np.int64, np.uint32, np.uint64):
        info = np.iinfo(dt)
        x = np.array([info.min, info.max, 0, info.max, info.min], dt)
        y = np.array([info.max, info.min, 0, info.max - 1, info.min], dt)
        (e,) = _run(prims.eq, x, y)
        (l,) = _run(prims.lt, x, y)
        np.testing.assert_array_equal(e, x == y, err_msg=str(dt))
        np.testing.assert_array_equal(l, x < y, err_msg=str(dt))


@pytest.mark.parametrize("name", ["to_host", "to_device", "host_wait", "device_wait"])
def test_transfer_and_wait_primitives_return_their_operand(name):
    """The transfer and wait primitives are the identity on values (only placement or ordering changes):
    float NaN payloads, -0 and bf16 patterns pass through bit for bit."""
    x = np.array([[np.nan, -0.0, 1.5], [np.inf, -3.25, 1e-40]], np.float32)
    (got,) = _run(lambda t: prims.bind(name, t), x)
    assert np.array_equal(got.view(np.uint32), x.view(np.uint32))
    b = np.array([0x7FC1, 0x8000, 0x3F80, 0xFF80], np.uint16)
    (gb,) = _run(lambda t: prims.bind(name, t), b)
    assert np.array_equal(gb, b)
