"""The reference's own attention cases (``tests/functional/test_attention.py:51-67`` forward,
``:354-359`` backward) compiled for hip: grouped heads, one query row, fewer keys than queries, head dims
16/24/32/64/128 with a value head dim different from the query's, plus head dims 24, 40, 96 and 256. Shapes the
flash kernels take (a head dim that is a multiple of 8, up to 256 forward and 128 backward, as
``passes/attention/forward.rs:100,725`` and ``backward.rs:86,473`` allow, the value head dim checked on its own;
no query row left without keys) run as flash steps; the others run the unfused dot / row-softmax plan. Both are checked against
float64 attention at the reference's tolerances."""

import numpy as np
import pytest

import lumen_amd as L
import lumen_amd.functional as F
from oracle import oracle

pytestmark = pytest.mark.gpu

TOL = {"float32": 2e-6, "float16": 2e-3, "bfloat16": 2e-2}  # test_attention.py:51

CASES = [  # (b, sq, sk, n, nkv, h, hv), causal — test_attention.py:53-60
    ((2, 100, 100, 4, 4, 64, 64), False),
    ((1, 130, 77, 2, 2, 32, 32), False),
    ((2, 100, 100, 4, 2, 64, 64), True),
    ((1, 1, 300, 8, 2, 128, 128), True),
    ((2, 5, 40, 2, 1, 16, 24), False),
    ((1, 70, 200, 2, 2, 128, 128), True),
    # added here: the flash kernels' other head size with fewer keys than queries, non-causal; head dims the
    # kernels pad (96 to 128, 40 to 64) and the largest forward head dim
    ((1, 130, 77, 2, 1, 64, 64), False),
    ((1, 100, 100, 4, 2, 96, 96), True),
    ((2, 64, 70, 2, 2, 40, 40), False),
    ((1, 70, 90, 2, 1, 256, 256), True),
    ((1, 96, 96, 2, 2, 64, 128), True),  # value head dim above the query's
]

BACKWARD_CASES = [  # test_attention.py:354-359, plus two the hip flash backward takes
    ((1, 40, 40, 4, 2, 32, 32), True),
    ((1, 70, 20, 2, 2, 16, 16), False),
    ((1, 3, 50, 2, 1, 16, 24), True),
    ((1, 9, 24, 2, 2, 128, 128), True),
    ((1, 40, 40, 4, 2, 64, 64), True),
    ((2, 70, 150, 2, 2, 128, 128), False),
    ((1, 100, 100, 4, 2, 96, 96), True),
    ((1, 33, 47, 2, 2, 24, 24), False),
    ((1, 64, 64, 2, 2, 256, 256), True),  # forward flash, backward past MAX_BACKWARD_HEAD: unfused
]


def reference(q, k, v, causal):
    """Attention in float64 (test_attention.py:17-30): q [B, Sq, N, H], k and v [B, Sk, Nkv, *]."""
    q, k, v = (a.astype(np.float64) for a in (q, k, v))
    b, sq, n, h = q.shape
    sk, nkv = k.shape[1], k.shape[2]
    k, v = np.repeat(k, n // nkv, axis=2), np.repeat(v, n // nkv, axis=2)
    s = np.einsum("bqnh,bknh->bnqk", q, k) / np.sqrt(h)
    if causal:
        i, j = np.arange(sq)[:, None], np.arange(sk)[None, :]
        s = np.where(j <= i + sk - sq, s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    return np.einsum("bnqk,bknh->bqnh", p, v)


def _flash_ok(case, limit=256):
    (b, sq, sk, n, nkv, h, hv), causal = case
    return all(d % 8 == 0 and d <= limit for d in (h, hv)) and not (causal and sk < sq)


def _tensors(dtype, *shapes, seed=0):
    rng = np.random.default_rng(seed)
    arrays = [rng.standard_normal(s).astype(np.float32) for s in shapes]
    ts = [L.tensor(a, dtype) for a in arrays]
    return ts, [L.to_numpy(t).astype(np.float32) for t in ts]


def _ids(cases):
    return [f"{c[0]}{'-causal' if c[1] else ''}" for c in cases]


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("case", CASES, ids=_ids(CASES))
def test_flash_attention_cases(hip, case, dtype):
    (b, sq, sk, n, nkv, h, hv), causal = case
    (q, k, v), arrays = _tensors(dtype, (b, sq, n, h), (b, sk, nkv, h), (b, sk, nkv, hv))

    def f(q, k, v):
        return F.flash_attention(q, k, v, is_causal=causal)

    c = L.compile(f, device="hip")
    out = c(q, k, v)
    assert out.dtype == dtype and list(out.shape) == [b, sq, n, hv]
    got = L.to_numpy(out).astype(np.float32)
    np.testing.assert_allclose(got, reference(*arrays, causal=causal), rtol=TOL[dtype], atol=TOL[dtype])
    kinds = [s["kind"] for s in c.plan.describe()]
    if dtype != "float32" and _flash_ok(case):
        assert kinds == ["flash_fwd"] or kinds.count("flash_fwd") == 1, kinds
    else:
        assert "flash_fwd" not in kinds


@pytest.mark.parametrize("deterministic,store_ds", [(True, True), (True, False), (False, True)])
@pytest.mark.parametrize("case", BACKWARD_CASES, ids=_ids(BACKWARD_CASES))
def test_attention_backward_cases(hip, case, deterministic, store_ds):
    """The gradient of a weighted sum of flash attention's output with respect to q, k and v, in bf16,
    against the oracle on the same traced program, with the reference's tolerance: rtol 2e-2 and atol
    2e-2 times the largest magnitude of each gradient (test_attention.py:413-416); deterministic (the same
    bits every run: dQ from the stored dS, or recomputing S and dP) or with dQ added atomically (the
    reference's default)."""
    (b, sq, sk, n, nkv, h, hv), causal = case
    shapes = (b, sq, n, h), (b, sk, nkv, h), (b, sk, nkv, hv), (b, sq, n, hv)
    ts, _ = _tensors("bfloat16", *shapes)

    def loss(q, k, v, w):
        return F.sum((F.flash_attention(q, k, v, is_causal=causal) * w).float())

    grad = L.grad(loss, (0, 1, 2))
    with L.config.compiler.patch(deterministic=deterministic, attention_store_ds=store_ds):
        c = L.compile(grad, device="hip")
        got = [L.to_numpy(t).astype(np.float32) for t in c(*ts)]
        again = [L.to_numpy(t).astype(np.float32) for t in c(*ts)]
    raws = [t.raw() for t in ts]
    want = oracle.values(L.make_graph(grad)(*ts), raws)
    kinds = [s["kind"] for s in c.plan.describe()]
    if _flash_ok(case):
        assert "flash_fwd" in kinds, kinds
        # grouped heads too: the kernel sums dK and dV over each group of query heads
        assert ("flash_bwd" in kinds) == _flash_ok(case, 128), kinds
    for g_, w_ in zip(got, want):
        w_ = np.asarray(w_, np.float32)
        np.testing.assert_allclose(g_, w_, rtol=2e-2, atol=2e-2 * np.abs(w_).max())
    for g_, a_ in zip(got, again):
        if deterministic:  # the same bits each run
            np.testing.assert_array_equal(g_, a_)
        else:  # atomic dQ: the order of the adds varies, within float32 rounding of the bf16 results
            np.testing.assert_allclose(g_, a_, rtol=2e-2, atol=2e-2 * np.abs(a_).max())
