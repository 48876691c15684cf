"""Parity of compiled plans on the GPU against the CPU oracle (the reference interpreter's restatement)."""

import numpy as np
import pytest

import lumen_amd as L
import lumen_amd.functional as F
from lumen_amd import dtypes as D
from oracle import oracle

pytestmark = pytest.mark.gpu


def _bf16(a):
    return D.bf16_bits(np.asarray(a, np.float32))


def test_config1_relu_matmul_f32_is_bit_exact(hip):
    """relu(matmul(x, w)) in float32: the plan's dot is the reference's sequential fold, so the GPU result
    equals the oracle bit for bit."""
    rng = np.random.default_rng(0)
    x = rng.standard_normal((256, 512)).astype(np.float32)
    w = rng.standard_normal((512, 1024)).astype(np.float32)
    f = L.compile(lambda x, w: F.relu(F.matmul(x, w, "float32", "float32")), device="hip")
    got = L.to_numpy(f(L.from_numpy(x), L.from_numpy(w)))
    (want,) = oracle.run(L.make_graph(lambda x, w: F.relu(F.matmul(x, w, "float32", "float32")))(L.from_numpy(x), L.from_numpy(w)), [x, w])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _chain(x, a, b):
    t = (x * a + b).float()
    t = F.gelu(t)
    t = F.layer_norm(t, x.shape[-1])
    return F.softmax(t, -1).bfloat16()


def _chain2(x, a, b):
    """The config-2 chain with the layer norm's output as a second (bf16) result."""
    t = (x * a + b).float()
    t = F.gelu(t)
    n = F.layer_norm(t, x.shape[-1])
    return F.softmax(n, -1).bfloat16(), n.bfloat16()


def _ulps_bf16(got, want):
    """Distance in bf16 steps between two bf16-valued float32 arrays (monotone integer mapping)."""
    def key(v):
        u = D.bf16_bits(np.asarray(v, np.float32)).astype(np.int32)
        return np.where(u & 0x8000, 0x8000 - u, u)
    return np.abs(key(got) - key(want))


def check_softmax_rows(got, want):
    """A bf16 softmax output against the oracle, scaled to the values it holds (the entries of a 4096-wide
    row are ~2e-4, so a fixed atol of 1e-2 would accept zeros): every entry within rtol 2e-2 plus 1e-2 of
    its row's largest entry, every entry at most 2 bf16 steps from the oracle's, every row summing to 1
    within 1e-2."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    rowmax = np.abs(want).max(axis=-1, keepdims=True)
    assert np.all(np.abs(got - want) <= 2e-2 * np.abs(want) + 1e-2 * rowmax), "softmax entries off"
    assert _ulps_bf16(got, want).max() <= 2, "softmax entries more than 2 bf16 steps from the oracle"
    assert np.all(np.abs(got.sum(axis=-1) - 1.0) <= 1e-2), "softmax rows do not sum to 1"


@pytest.mark.parametrize("rows,cols", [(64, 4096), (37, 512), (16, 64), (8, 1000)])
def test_config2_fused_chain_matches_oracle(hip, rows, cols):
    """layernorm(gelu(x*a+b)) then softmax, bf16 in and out, float32 statistics: one row kernel, each
    softmax entry checked against the oracle relative to the row's own scale."""
    rng = np.random.default_rng(1)
    x = _bf16(rng.standard_normal((rows, cols)))
    a = _bf16(1.0 + 0.1 * rng.standard_normal(cols))
    b = _bf16(0.1 * rng.standard_normal(cols))
    args = [L.tensor(D.bf16_to_f32(v), "bfloat16") for v in (x, a, b)]
    f = L.compile(_chain, device="hip")
    got = L.to_numpy(f(*args))
    assert [s["kind"] for s in f.plan.describe()] == ["row"]
    (want,) = oracle.values(L.make_graph(_chain)(*args), [x, a, b])
    check_softmax_rows(got, want)
    with pytest.raises(AssertionError):  # the check rejects a kernel that wrote zeros
        check_softmax_rows(np.zeros_like(got), want)


def test_config2_at_full_size_matches_oracle_on_sampled_rows(hip):
    """Config 2 at its real size, x [8192, 4096] with a ~ N(1, 0.1) and b ~ N(0, 0.1): the whole input goes
    through the GPU plan once; 256 seeded rows (rows are independent) are compared with the oracle by the
    row-scaled softmax check, and every one of the 8192 rows must be finite and sum to 1 within 1e-2."""
    rows, cols = 8192, 4096
    rng = np.random.default_rng(2)
    x = _bf16(rng.standard_normal((rows, cols), np.float32))
    a = _bf16(1.0 + 0.1 * rng.standard_normal(cols))
    b = _bf16(0.1 * rng.standard_normal(cols))
    args = [L.tensor(D.bf16_to_f32(v), "bfloat16") for v in (x, a, b)]
    f = L.compile(_chain, device="hip")
    got = np.asarray(L.to_numpy(f(*args)), np.float64)
    assert [s["kind"] for s in f.plan.describe()] == ["row"]
    assert np.isfinite(got).all()
    assert np.all(np.abs(got.sum(axis=-1) - 1.0) <= 1e-2)
    pick = np.sort(rng.choice(rows, 256, replace=False))
    sub = [L.tensor(D.bf16_to_f32(v), "bfloat16") for v in (x[pick], a, b)]
    (want,) = oracle.values(L.make_graph(_chain)(*sub), [x[pick], a, b])
    check_softmax_rows(got[pick], want)


@pytest.mark.parametrize("rows,cols", [(64, 4096), (16, 1000)])
def test_config2_chain_with_layernorm_output_matches_oracle(hip, rows, cols):
    """The same chain also returning the layer norm's output (values of order 1, so the bf16 tolerance is
    meaningful at face value): the softmax by the row-scaled check and the layer norm within rtol 2e-2 /
    atol 1e-2 and (away from zero) 2 bf16 steps of the oracle."""
    rng = np.random.default_rng(5)
    x = _bf16(rng.standard_normal((rows, cols)))
    a = _bf16(1.0 + 0.1 * rng.standard_normal(cols))
    b = _bf16(0.1 * rng.standard_normal(cols))
    args = [L.tensor(D.bf16_to_f32(v), "bfloat16") for v in (x, a, b)]
    f = L.compile(_chain2, device="hip")
    sm, ln = (L.to_numpy(t) for t in f(*args))
    assert {s["kind"] for s in f.plan.describe()} == {"row"}
    want_sm, want_ln = oracle.values(L.make_graph(_chain2)(*args), [x, a, b])
    check_softmax_rows(sm, want_sm)
    np.testing.assert_allclose(ln, want_ln, rtol=2e-2, atol=1e-2)
    big = np.abs(np.asarray(want_ln, np.float64)) >= 1e-2  # near zero the float32 cancellation in x - mean dominates
    assert _ulps_bf16(ln, want_ln)[big].max() <= 2
    assert np.abs(np.asarray(want_ln, np.float64)).max() > 1.0  # the atol is small against these values


def test_horizontally_fused_loops_match_oracle_bit_for_bit(hip):
    """Small independent elementwise results computed in one hloop launch equal the oracle exactly (float32
    and bf16 elementwise ops are correctly rounded on both sides)."""
    rng = np.random.default_rng(7)
    a = rng.standard_normal((64, 64)).astype(np.float32)
    b = _bf16(rng.standard_normal(128))
    c = rng.standard_normal(1000).astype(np.float32)

    def fn(a, b, c):
        return a * 2.0 - 1.0, b + 1.0, c * c

    args = [L.from_numpy(a), L.tensor(D.bf16_to_f32(b), "bfloat16"), L.from_numpy(c)]
    f = L.compile(fn, device="hip")
    got = [L.to_numpy(t) for t in f(*args)]
    assert [s["kind"] for s in f.plan.describe()] == ["hloop"]
    want = oracle.values(L.make_graph(fn)(*args), [a, b, c])
    for g_, w_ in zip(got, want):
        assert np.array_equal(np.asarray(g_, np.float32), np.asarray(w_, np.float32))


def test_concatenated_dot_results_written_in_place_match_oracle(hip):
    """Two dots writing straight into their concatenation (strided GEMM stores, no copy launch), then a dot
    reading it, against the oracle (bf16 tolerance: the reference's bf16 bounds)."""
    rng = np.random.default_rng(3)

    def fn(x, w1, w2, w3):
        a = F.matmul(x, w1, "float32", "bfloat16")
        b = F.matmul(x, w2, "float32", "bfloat16")
        return F.matmul(F.cat([a, b], 1), w3, "float32", "bfloat16")

    shapes = [(2048, 256), (256, 512), (256, 512), (1024, 128)]
    xs = [_bf16(rng.standard_normal(s) * 0.5) for s in shapes]
    args = [L.tensor(D.bf16_to_f32(x), "bfloat16") for x in xs]
    f = L.compile(fn, device="hip")
    got = np.asarray(L.to_numpy(f(*args)), np.float32)
    assert "alias" in [s["kind"] for s in f.plan.describe()]
    (want,) = oracle.values(L.make_graph(fn)(*args), xs)
    np.testing.assert_allclose(got, want, rtol=2e-2, atol=1e-2 * np.abs(want).max())


def _epi_fn(x, w, h, b):
    y = F.matmul(x, w, "float32", "float32")
    return F.gelu(y) * b + y * h


def _epi_fn_keep(x, w, h, b):
    y = F.matmul(x, w, "float32", "float32")
    return F.gelu(y) * b + y * h, y


@pytest.mark.parametrize("fn", [_epi_fn, _epi_fn_keep])
@pytest.mark.parametrize("m,n,k", [(512, 512, 256), (1000, 776, 320)])
def test_gemm_epilogue_matches_oracle_and_unfused_plan(hip, fn, m, n, k, monkeypatch):
    """The dot with its elementwise consumer fused into the GEMM's store (gemm_epi kernel, ragged m and n
    included) against the oracle (float32: rtol 1e-4 of the largest value, the tolerance for float32
    results), and bit for bit against the same plan without epilogue fusion (same sums, same body). The
    fusion threshold (256 tiles) is lowered so that these small shapes take the fused path."""
    from lumen_amd.compiler.plan import Plan

    monkeypatch.setattr(Plan, "EPI_MIN_TILES", 1)
    rng = np.random.default_rng(11)
    x = _bf16(rng.standard_normal((m, k)) * 0.25)
    w = _bf16(rng.standard_normal((k, n)) * 0.25)
    h = rng.standard_normal((m, n)).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    args = [L.tensor(D.bf16_to_f32(x), "bfloat16"), L.tensor(D.bf16_to_f32(w), "bfloat16"), L.from_numpy(h),
            L.from_numpy(b)]
    with L.config.compiler.patch(horizontal_fusion=False):
        f = L.compile(fn, device="hip")
        got = f(*args)
        got = [np.asarray(L.to_numpy(t), np.float32) for t in (got if isinstance(got, tuple) else (got,))]
        assert [s["name"][:9] for s in f.plan.describe()] == ["gemm_epi_"]
    with L.config.compiler.patch(horizontal_fusion=False, epilogue_fusion=False, autotune=False):
        u = L.compile(fn, device="hip")
        ref = u(*args)
        ref = [np.asarray(L.to_numpy(t), np.float32) for t in (ref if isinstance(ref, tuple) else (ref,))]
        assert "loop" in [s["kind"] for s in u.plan.describe()]
    want = oracle.values(L.make_graph(fn)(*args), [x, w, h, b])
    for g_, r_, w_ in zip(got, ref, want):
        w_ = np.asarray(w_, np.float32)
        np.testing.assert_allclose(g_, w_, rtol=1e-4, atol=1e-4 * np.abs(w_).max())
        assert np.array_equal(g_, r_)


def _epi_colsum_fn(x, w, h, b):
    z = F.matmul(x, w, "float32", "float32") * h
    return F.sum(z, dim=(0,)), (z + b).bfloat16()


@pytest.mark.parametrize("fn", [_epi_fn_keep, _epi_colsum_fn])
def test_gemm_epilogue_k_loops_agree_and_autotune_keeps_values(hip, fn, monkeypatch):
    """The generated epilogue GEMM's first and last k loops (k tile 64 on eight waves; k tile 64 on four waves,
    two stages, placed by hand) give the same bits, ragged m and n included; and a plan whose autotuner times
    every k loop on its own buffers before the first run still gives those bits. Column sums, added atomically into zeros in no fixed
    order, agree within float32 reassociation (1e-5 of the sum of magnitudes)."""
    from lumen_amd.compiler import codegen
    from lumen_amd.compiler.plan import Plan

    monkeypatch.setattr(Plan, "EPI_MIN_TILES", 1)
    m, n, k = 1000, 776, 320
    rng = np.random.default_rng(23)
    x = _bf16(rng.standard_normal((m, k)) * 0.25)
    w = _bf16(rng.standard_normal((k, n)) * 0.25)
    h = rng.standard_normal((m, n)).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    args = [L.tensor(D.bf16_to_f32(x), "bfloat16"), L.tensor(D.bf16_to_f32(w), "bfloat16"), L.from_numpy(h),
            L.from_numpy(b)]

    def run(**patch):
        with L.config.compiler.patch(horizontal_fusion=False, **patch):
            f = L.compile(fn, device="hip")
            out = [np.asarray(L.to_numpy(t), np.float32) for t in f(*args)]
            assert any(s["name"].startswith("gemm_epi_") for s in f.plan.describe())
            return out, f.plan

    first, _ = run(autotune=False)
    monkeypatch.setattr(codegen.GemmEpilogueKernel, "VARIANTS", tuple(reversed(codegen.GemmEpilogueKernel.VARIANTS)))
    second, _ = run(autotune=False)
    monkeypatch.undo()
    monkeypatch.setattr(Plan, "EPI_MIN_TILES", 1)
    monkeypatch.setattr(Plan, "AUTOTUNE_MACS", 1)
    tuned, plan = run(autotune=True)
    assert plan.epi_alts and all(hasattr(plan.steps[si], "epi_variant") for si in plan.epi_alts)
    summed = fn is _epi_colsum_fn  # its first output: column sums added atomically, in no fixed order
    for i, (a, b_, c) in enumerate(zip(first, second, tuned)):
        if summed and i == 0:
            y = D.bf16_to_f32(x).astype(np.float64) @ D.bf16_to_f32(w).astype(np.float64)
            scale = np.abs(y * h).sum(axis=0)
            assert np.all(np.abs(a - b_) <= 1e-5 * scale) and np.all(np.abs(a - c) <= 1e-5 * scale)
        else:
            assert np.array_equal(a, b_) and np.array_equal(a, c)


@pytest.mark.parametrize("variant", [1, 2, 3, 4])
def test_each_gemm_epilogue_k_loop_gives_the_first_ones_bits(hip, variant, monkeypatch):
    """Every k loop a generated epilogue GEMM can be built with (k tile 32 cross-tile prefetch and ping-pong,
    k tile 64 two-stage on four and eight waves), forced as the only one, gives the bits of the default
    (k tile 64 on eight waves): ragged m and n, an odd number of k tiles of 64 (k = 320)."""
    from lumen_amd.compiler import codegen
    from lumen_amd.compiler.plan import Plan

    monkeypatch.setattr(Plan, "EPI_MIN_TILES", 1)
    m, n, k = 1000, 776, 320
    rng = np.random.default_rng(29)
    x = _bf16(rng.standard_normal((m, k)) * 0.25)
    w = _bf16(rng.standard_normal((k, n)) * 0.25)
    h = rng.standard_normal((m, n)).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    args = [L.tensor(D.bf16_to_f32(x), "bfloat16"), L.tensor(D.bf16_to_f32(w), "bfloat16"), L.from_numpy(h),
            L.from_numpy(b)]

    def run():
        with L.config.compiler.patch(horizontal_fusion=False, autotune=False):
            f = L.compile(_epi_fn_keep, device="hip")
            out = [np.asarray(L.to_numpy(t), np.float32) for t in f(*args)]
            assert any(s["name"].startswith("gemm_epi_") for s in f.plan.describe())
            return out

    first = run()
    variants = codegen.GemmEpilogueKernel.VARIANTS
    monkeypatch.setattr(codegen.GemmEpilogueKernel, "VARIANTS", (variants[variant],) + variants[1:])
    for a, b_ in zip(first, run()):
        assert np.array_equal(a, b_)


@pytest.mark.parametrize("shape,axes", [((1000, 2048), (0,)), ((3, 70, 1024), (0, 1)), ((130, 4100), (0,)),
                                        ((8192, 512), (0,)), ((1100, 260), (0,)), ((5, 600, 768), (0, 1))])
def test_leading_axis_sums_match_oracle(hip, shape, axes):
    """float32 sums over leading axes (the vectorized reduce kernel: four columns a thread, row chunks added
    atomically; 4100 columns is not a multiple of 4 x 256 threads; under 1024 columns a workgroup takes 64
    columns of 16 row lanes, 260 of them ragged) against the oracle's sequential sum (float32 reassociation:
    rtol 1e-4 of the sum of magnitudes)."""
    rng = np.random.default_rng(9)
    x = rng.standard_normal(shape).astype(np.float32)

    def fn(x):
        return F.sum(x * 2.0, dim=axes)

    f = L.compile(fn, device="hip")
    got = np.asarray(L.to_numpy(f(L.from_numpy(x))), np.float32)
    assert "reduce" in [s["kind"] for s in f.plan.describe()]
    (want,) = oracle.values(L.make_graph(fn)(L.from_numpy(x)), [x])
    scale = np.abs(x * 2.0).sum(axis=axes)
    assert np.all(np.abs(got - want) <= 1e-4 * scale + 1e-6)


def test_softmax_gradient_joins_its_statistics_row_kernel(hip):
    """Cross entropy forward + backward over [rows, classes] logits: the backward's softmax-minus-one-hot
    loop is absorbed into the forward's max/sum-exp row kernel (one launch reads the logits once), and the
    loss and logits gradient match the oracle (float32: rtol 1e-4)."""
    rng = np.random.default_rng(4)
    rows, classes = 512, 3000
    x = rng.standard_normal((rows, classes)).astype(np.float32)
    t = rng.integers(0, classes, rows).astype(np.int64)

    def fn(x, t):
        return L.value_and_grad(lambda x: F.mean(F.cross_entropy(x, t)))(x)

    f = L.compile(fn, device="hip")
    loss, dx = f(L.from_numpy(x), L.from_numpy(t))
    writers = [s.kind for s in f.plan.steps if any(f.plan.graph.types[v].shape == (rows, classes) for v in s.outputs)]
    assert writers == ["row"], writers
    want = oracle.values(L.make_graph(fn)(L.from_numpy(x), L.from_numpy(t)), [x, t])
    np.testing.assert_allclose(float(L.to_numpy(loss)), float(want[0]), rtol=1e-4)
    np.testing.assert_allclose(np.asarray(L.to_numpy(dx), np.float32), want[1], rtol=1e-4, atol=1e-4 * np.abs(want[1]).max())


def test_float32_tanh_is_within_4_ulp(hip):
    """The generated kernels' float32 tanh (odd series below 0.55, exp2/reciprocal form above) against float64
    tanh rounded to float32 over a log-spaced sweep of both signs, with zeros, infinities and NaN: at most 4
    ulp, and the special values exact."""
    mags = np.logspace(-30, 1.7, 200001).astype(np.float32)
    x = np.concatenate([mags, -mags, np.float32([0.0, -0.0, np.inf, -np.inf, np.nan, 0.55, -0.55, 44.0, 100.0])])
    f = L.compile(lambda x: F.tanh(x), device="hip")
    got = np.asarray(L.to_numpy(f(L.from_numpy(x))), np.float32)
    want = np.tanh(x.astype(np.float64))
    fin = np.isfinite(x)
    ulp = np.spacing(np.abs(want[fin]).astype(np.float32)).astype(np.float64)
    err = np.abs(got[fin].astype(np.float64) - want[fin]) / ulp
    assert err.max() <= 4.0, (err.max(), x[fin][err.argmax()])
    assert got[-7] == 1.0 and got[-6] == -1.0 and np.isnan(got[-5])
    assert np.array_equal(np.signbit(got[-9:-7]), [False, True]) and np.all(got[-9:-7] == 0)


def test_bf16_stores_round_to_nearest_even_bit_for_bit(hip):
    """float32 -> bfloat16 in generated kernels (the hardware conversion) against the reference's rounding
    restated on the host (round to nearest even; NaN -> its top 16 bits with the quiet bit): every tie and
    half-ulp neighbour of a sweep of exponents, NaN payloads of both signs, infinities, subnormals, the
    largest finite values, and 2^24 random bit patterns, bit for bit; stored as bfloat16 and rounded inside a
    kernel then widened back to float32."""
    rng = np.random.default_rng(12)
    hi = (np.arange(0, 1 << 16, 7, dtype=np.uint32) << 16)
    lows = np.uint32([0, 1, 0x7FFF, 0x8000, 0x8001, 0xFFFF, 0x4000, 0xC000])
    grid = (hi[:, None] | lows[None, :]).ravel()
    special = np.uint32([0x7F800000, 0xFF800000, 0x7F800001, 0xFF800001, 0x7FC00000, 0xFFC00000, 0x7FFFFFFF,
                         0xFFFFFFFF, 0x7F7FFFFF, 0xFF7FFFFF, 0x7F7F8000, 0x00000001, 0x80000001, 0x007FFFFF,
                         0x00008000, 0x00018000, 0x0, 0x80000000])
    bits = np.concatenate([grid, special, rng.integers(0, 1 << 32, 1 << 24, dtype=np.uint64).astype(np.uint32)])
    x = bits.view(np.float32)
    f = L.compile(lambda x: x.bfloat16(), device="hip")
    got = np.asarray(f(L.from_numpy(x)).raw()).view(np.uint16).ravel()
    assert np.array_equal(got, D.bf16_bits(x))
    # the rounding inside a kernel, widened back to float32 (r_bf16: one conversion of the pair {0, x}, whose
    # high half over a zero low half is the rounded value)
    f = L.compile(lambda x: x.bfloat16().float(), device="hip")
    got = np.asarray(f(L.from_numpy(x)).raw()).view(np.uint32).ravel()
    assert all("r_bf16(" in src for src in f.plan.sources.values())
    assert np.array_equal(got, D.bf16_bits(x).astype(np.uint32) << 16)


def test_float32_exp_is_within_4_ulp(hip):
    """The generated kernels' float32 exp (compensated x log2 e, hardware exp2) against float64 exp over a
    sweep of [-87.3, 88.7] (normal results): at most 4 ulp; below that results are within 2^-126 of exact
    (flushed), above it inf, and exp(-inf) = 0, exp(inf) = inf, exp(NaN) = NaN."""
    x = np.concatenate([np.linspace(-87.3, 88.7, 400001, dtype=np.float32),
                        np.float32([-1e-30, 0.0, -0.0, 1e-30, -100.0, -104.0, 89.0, -np.inf, np.inf, np.nan])])
    f = L.compile(lambda x: F.exp(x), device="hip")
    got = np.asarray(L.to_numpy(f(L.from_numpy(x))), np.float64)
    want = np.exp(x.astype(np.float64))
    n = 400001
    ulp = np.spacing(want[:n].astype(np.float32)).astype(np.float64)
    err = np.abs(got[:n] - want[:n]) / ulp
    assert err.max() <= 4.0, (err.max(), x[:n][err.argmax()])
    assert np.array_equal(got[n:n + 4], [1.0, 1.0, 1.0, 1.0])
    assert np.all(np.abs(got[n + 4:n + 6] - want[n + 4:n + 6]) <= 2.0 ** -126)
    assert got[n + 6] == np.inf and got[n + 7] == 0.0 and got[n + 8] == np.inf and np.isnan(got[n + 9])


@pytest.mark.parametrize("m,n,k", [(512, 512, 256), (1000, 776, 320)])
def test_gemm_epilogue_column_sums_match_oracle(hip, m, n, k, monkeypatch):
    """A row sum of a GEMM epilogue's float32 output (a bias / norm-weight gradient shape) computed inside the
    epilogue: per-wave column sums added atomically, the [m, n] product never stored (no reduce step left),
    ragged m and n. Against the oracle's sequential sums within float32 reassociation (1e-4 of the sum of
    magnitudes) and against the same plan without epilogue fusion."""
    from lumen_amd.compiler.plan import Plan

    monkeypatch.setattr(Plan, "EPI_MIN_TILES", 1)

    def fn(x, w, h):
        z = F.matmul(x, w, "float32", "float32") * h
        return F.sum(z, dim=(0,)), (z + 1.0).bfloat16()

    rng = np.random.default_rng(17)
    x = _bf16(rng.standard_normal((m, k)) * 0.25)
    w = _bf16(rng.standard_normal((k, n)) * 0.25)
    h = rng.standard_normal((m, n)).astype(np.float32)
    args = [L.tensor(D.bf16_to_f32(x), "bfloat16"), L.tensor(D.bf16_to_f32(w), "bfloat16"), L.from_numpy(h)]
    with L.config.compiler.patch(horizontal_fusion=False):
        f = L.compile(fn, device="hip")
        got = [np.asarray(L.to_numpy(t), np.float32) for t in f(*args)]
        kinds = [s["kind"] for s in f.plan.describe()]
        assert "reduce" not in kinds and any(s["name"].startswith("gemm_epi_") for s in f.plan.describe())
    with L.config.compiler.patch(horizontal_fusion=False, epilogue_fusion=False):
        u = L.compile(fn, device="hip")
        ref = [np.asarray(L.to_numpy(t), np.float32) for t in u(*args)]
    want = [np.asarray(v, np.float32) for v in oracle.values(L.make_graph(fn)(*args), [x, w, h])]
    y = D.bf16_to_f32(x).astype(np.float64) @ D.bf16_to_f32(w).astype(np.float64)
    scale = np.abs(y * h).sum(axis=0)
    assert np.all(np.abs(got[0] - want[0]) <= 1e-4 * scale + 1e-6)
    assert np.all(np.abs(got[0] - ref[0]) <= 1e-4 * scale + 1e-6)
    np.testing.assert_allclose(got[1], want[1], rtol=2e-2, atol=1e-2 * np.abs(want[1]).max())


def test_float32_division_is_within_1_ulp(hip):
    """Generated float32 division (refined hardware reciprocal plus one quotient correction) against the
    correctly rounded quotient: within 1 ulp everywhere, exact on at least 99% of random operands; zero,
    infinite and NaN operands and divisors near the ends of the exponent range follow IEEE division
    (signed zeros included)."""
    rng = np.random.default_rng(21)
    n = 1 << 20
    a = (rng.standard_normal(n) * np.exp2(rng.integers(-60, 60, n))).astype(np.float32)
    b = (rng.standard_normal(n) * np.exp2(rng.integers(-60, 60, n))).astype(np.float32)
    sa = np.float32([1.0, -0.0, 0.0, 3.0, -3.0, np.inf, 1.0, np.nan, 1.0, 1e-40, 5.0, 1.0, 2.0, -0.0])
    sb = np.float32([0.0, 2.0, -2.0, np.inf, -np.inf, 2.0, np.nan, 1.0, 1e-39, 3.0, 3e38, 1e-38, 2.0, -5.0])
    x, y = np.concatenate([a, sa]), np.concatenate([b, sb])
    f = L.compile(lambda x, y: x / y, device="hip")
    got = np.asarray(L.to_numpy(f(L.from_numpy(x), L.from_numpy(y))), np.float32)
    with np.errstate(all="ignore"):
        want = x / y  # NumPy float32 division: correctly rounded
    fin = np.isfinite(want[:n]) & (np.abs(want[:n]) >= np.float32(2.0 ** -126))
    ulp = np.spacing(np.abs(want[:n][fin])).astype(np.float64)
    err = np.abs(got[:n][fin].astype(np.float64) - want[:n][fin]) / ulp
    assert err.max() <= 1.0, (err.max(), x[:n][fin][err.argmax()], y[:n][fin][err.argmax()])
    assert (got[:n][fin] == want[:n][fin]).mean() >= 0.99
    tail_g, tail_w = got[n:], want[n:]
    same = (tail_g.view(np.uint32) == tail_w.view(np.uint32)) | (np.isnan(tail_g) & np.isnan(tail_w))
    assert same.all(), (tail_g, tail_w)


def test_gelu_tanh_form_matches_float64_and_oracle(hip):
    """The traced tanh GELU, evaluated in its sigmoid form x / (1 + 2^(x (k + k c2 x^2))): within 1e-5 relative of
    float64 GELU (tanh form) on [-10, 10] and within rtol 1e-4 (atol 1e-4 of the largest value) of the oracle,
    which evaluates the traced float32 graph (its 1 + tanh(u) loses relative accuracy as tanh(u) nears -1, so
    the oracle comparison is scaled by the largest value, as the float32 checks elsewhere). +inf gives inf,
    -inf NaN (0.5 x (1 + tanh u) is -inf * 0 in float32 too), NaN NaN."""
    x = np.concatenate([np.linspace(-10.0, 10.0, 200001, dtype=np.float32),
                        np.float32([0.0, -0.0, 1e-30, -1e-30, 1e-3, -1e-3, 30.0, -30.0, np.inf, -np.inf, np.nan])])
    f = L.compile(lambda x: F.gelu(x), device="hip")
    got = np.asarray(L.to_numpy(f(L.from_numpy(x))), np.float64)
    xd = x.astype(np.float64)
    with np.errstate(all="ignore"):  # 0.5 x (1 + tanh u) = x sigmoid(2u), without the cancellation
        want = xd / (1.0 + np.exp(-2.0 * 0.7978845608 * (xd + 0.044715 * xd ** 3)))
    n = 200001 + 8
    # the exponent's roundings (relative 2^-24 each, three of them) grow with its magnitude: 1e-5 relative down
    # to x = -8 (exponent -71 in base 2); below that the results are under 1e-18 and leave the float range
    # near x = -9.4 (-0), as the traced float32 form's do
    ok = xd[:n] >= -8.0
    rel = np.abs(got[:n] - want[:n]) / np.maximum(np.abs(want[:n]), 1e-300)
    assert rel[ok & (want[:n] != 0)].max() <= 1e-5, (rel[ok].max(), x[:n][ok][rel[ok].argmax()])
    assert np.abs(got[:n][~ok]).max() <= 1e-18
    assert got[n] == np.inf and np.isnan(got[n + 1]) and np.isnan(got[n + 2])
    g = L.make_graph(lambda x: F.gelu(x))(L.empty([n], "float32", "meta"))
    (ref,) = oracle.run(g, [x[:n]])
    np.testing.assert_allclose(got[:n], ref, rtol=1e-4, atol=1e-4 * np.abs(ref).max())


def test_float32_softmax_and_layer_norm_match_float64(hip):
    """A float32 row softmax (its shifted exponent as one exp2) and layer norm (its quotient as a multiply by
    the row's reciprocal) against float64 within 1e-5 relative (largest value of the row), and against the
    oracle within rtol 1e-4; rows with -inf entries give zeros there, a row of equal values a uniform row."""
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((64, 2048)) * 4.0).astype(np.float32)
    x[3, ::7] = -np.inf
    x[5] = 1.5
    f = L.compile(lambda x: (F.softmax(x, -1), F.layer_norm(x[1:], 2048)), device="hip")
    sm, ln = (np.asarray(L.to_numpy(t), np.float64) for t in f(L.from_numpy(x)))
    xd = x.astype(np.float64)
    e = np.exp(xd - xd.max(-1, keepdims=True))
    want_sm = e / e.sum(-1, keepdims=True)
    assert (np.abs(sm - want_sm) / want_sm.max(-1, keepdims=True)).max() <= 1e-5
    assert np.all(sm[3, ::7] == 0.0) and np.allclose(sm[5], 1.0 / 2048, rtol=1e-6)
    y = xd[1:]
    y = np.where(np.isinf(y), 0.0, y)  # the row with -inf entries normalizes to NaN: left out below
    mu = y.mean(-1, keepdims=True)
    want_ln = (y - mu) / np.sqrt(((y - mu) ** 2).mean(-1, keepdims=True) + 1e-5)
    keep = [r for r in range(63) if r != 2]
    err = np.abs(ln[keep] - want_ln[keep]) / np.maximum(np.abs(want_ln[keep]).max(-1, keepdims=True), 1e-30)
    assert err.max() <= 1e-5, err.max()
    g = L.make_graph(lambda x: (F.softmax(x, -1), F.layer_norm(x[1:], 2048)))(L.empty([64, 2048], "float32", "meta"))
    ref_sm, ref_ln = oracle.run(g, [x])
    np.testing.assert_allclose(sm, ref_sm, rtol=1e-4, atol=1e-4 * np.abs(ref_sm).max())
    np.testing.assert_allclose(ln[keep], ref_ln[keep], rtol=1e-4, atol=1e-4 * np.abs(ref_ln[keep]).max())


def test_gelu_gradient_matches_float64_and_oracle(hip):
    """The derivative of the traced tanh GELU (its tanh read in 1 + t and t * t, evaluated as
    1 - 2 / (1 + 2^(2u log2 e))) against float64 within 1e-4 absolute on [-10, 10] (the derivative is at most
    1.13 in magnitude) and against the oracle within rtol 1e-4 (atol 1e-4 of the largest value)."""
    x = np.linspace(-10.0, 10.0, 100001, dtype=np.float32)
    g = np.cos(x).astype(np.float32)

    def f(x, g):
        _, pull = L.vjp(lambda x: F.gelu(x), x)
        return pull(g)[0]

    fc = L.compile(f, device="hip")
    got = np.asarray(L.to_numpy(fc(L.from_numpy(x), L.from_numpy(g))), np.float64)
    xd = x.astype(np.float64)
    u = 0.7978845608 * (xd + 0.044715 * xd ** 3)
    t = np.tanh(u)
    want = g * (0.5 * (1.0 + t) + 0.5 * xd * (1.0 - t * t) * 0.7978845608 * (1.0 + 3.0 * 0.044715 * xd * xd))
    assert np.abs(got - want).max() <= 1e-4, np.abs(got - want).max()
    gr = L.make_graph(f)(*[L.empty([x.size], "float32", "meta")] * 2)
    (ref,) = oracle.run(gr, [x, g])
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4 * np.abs(ref).max())


def test_gelu_gradient_closed_form_matches_float64():
    """The GELU vjp's closed form (gelu_tanh_grad_f32: dy s (1 + 2 c1 x e s (1 + 3 c2 x^2)), s = 1 / (1 + e))
    against float64 on 2^20 points of [-8, 8] within 4e-6 of the value plus 4e-7 of |dy| (the absolute part
    for the derivative's zero near x = -0.75, where the sum cancels), and at the ends as the traced form
    gives: dy itself for large positive x, zero for large negative x (e = 2^(..) overflows there), NaN for
    +-inf and NaN."""
    n = 1 << 20
    x = np.concatenate([np.linspace(-8.0, 8.0, n, dtype=np.float32),
                        np.array([20.0, 90.0, -20.0, -90.0, np.inf, -np.inf, np.nan], np.float32)])
    g = (1.0 + 0.5 * np.sin(np.arange(x.size) * 0.37)).astype(np.float32) * np.where(np.arange(x.size) % 2, 1, -1)
    g = g.astype(np.float32)

    def f(x, g):
        _, pull = L.vjp(lambda x: F.gelu(x), x)
        return pull(g)[0]

    fc = L.compile(f, device="hip")
    got = np.asarray(L.to_numpy(fc(L.from_numpy(x), L.from_numpy(g))), np.float64)
    assert any("gelu_tanh_grad_f32(" in src for src in fc.plan.sources.values())
    xd, gd = x[:n].astype(np.float64), g.astype(np.float64)
    u = 0.7978845608028654 * (xd + 0.044715 * xd ** 3)
    t = np.tanh(u)
    want = gd[:n] * (0.5 * (1.0 + t) + 0.5 * xd * (1.0 - t * t) * 0.7978845608028654 * (1.0 + 3.0 * 0.044715 * xd * xd))
    bound = 4e-6 * np.abs(want) + 4e-7 * np.abs(gd[:n])
    err = np.abs(got[:n] - want)
    assert np.all(err <= bound), (float((err / bound).max()), float(xd[np.argmax(err / bound)]))
    np.testing.assert_array_equal(got[n:n + 2], gd[n:n + 2])
    assert np.all(got[n + 2:n + 4] == 0.0), got[n + 2:n + 4]
    assert np.all(np.isnan(got[n + 4:])), got[n + 4:]
