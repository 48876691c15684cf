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


@pytest.mark.parametrize("rows,cols", [(64, 4096), (37, 512), (16, 64), (8, 1000)])
def test_config2_fused_chain_matches_oracle(hip, rows, cols):
    """layernorm(gelu(x*a+b)) then softmax, bf16 in and out, float32 statistics: one row kernel, within
    the bf16 tolerance (rtol 2e-2, atol 1e-2)."""
    rng = np.random.default_rng(1)
    x = _bf16(rng.standard_normal((rows, cols)))
    a = _bf16(1.0 + 0.1 * rng.standard_normal(cols))
    b = _bf16(0.1 * rng.standard_normal(cols))
    args = [L.tensor(D.bf16_to_f32(v), "bfloat16") for v in (x, a, b)]
    f = L.compile(_chain, device="hip")
    got = L.to_numpy(f(*args))
    assert [s["kind"] for s in f.plan.describe()] == ["row"]
    (want,) = oracle.values(L.make_graph(_chain)(*args), [x, a, b])
    np.testing.assert_allclose(got, want, rtol=2e-2, atol=1e-2)


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
