"""nhip_gemm (the dot_general kernel) through the C ABI: every operand layout, batches, edges and dtypes."""

import ctypes as C

import numpy as np
import pytest

from lumen_amd import dtypes as D
from lumen_amd import native as nv
from tests.hiputil import Dev

pytestmark = pytest.mark.gpu


def _desc(m, n, k, a_m, a_k, b_k, b_n, dt=nv.NHIP_BF16, out=nv.NHIP_F32, cfg=-1, batch=(), sa=(), sb=(), sd=()):
    d = nv.GemmDesc()
    d.m, d.n, d.k = m, n, k
    d.nbatch = len(batch)
    for i, (z, x, y, w) in enumerate(zip(batch, sa, sb, sd)):
        d.batch[i], d.a_batch[i], d.b_batch[i], d.d_batch[i] = z, x, y, w
    d.a_dtype = d.b_dtype = dt
    d.d_dtype = out
    d.a_m, d.a_k, d.b_k, d.b_n, d.d_m, d.d_n = a_m, a_k, b_k, b_n, n, 1
    d.config = cfg
    return d


@pytest.mark.parametrize("at,bt", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize(
    "m,n,k,cfg",
    [(512, 384, 256, -1), (264, 136, 200, 2), (64, 64, 64, 4), (520, 520, 72, 0), (520, 264, 192, 6), (264, 776, 128, 7),
     (264, 136, 96, 8), (200, 392, 192, 9), (520, 776, 192, 10), (520, 776, 160, 11), (520, 776, 160, 12),
     (264, 520, 32, 12), (264, 264, 64, 12), (520, 776, 160, 13), (264, 520, 32, 13), (520, 776, 192, 14),
     (264, 520, 64, 14), (264, 264, 128, 14), (520, 776, 192, 15), (264, 520, 64, 15)],
)
def test_gemm_layouts(hip, at, bt, m, n, k, cfg):
    """A as [m][k] or [k][m] in memory, B as [n][k] or [k][n]: float32 results within float32 rounding of
    the float64 product of the bf16 operands."""
    rng = np.random.default_rng(m + n + k)
    a = D.bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    b = D.bf16_bits(rng.standard_normal((k, n)).astype(np.float32))
    want = D.bf16_to_f32(a).astype(np.float64) @ D.bf16_to_f32(b).astype(np.float64)
    am = np.ascontiguousarray(a.T) if at else a
    bm = b if bt else np.ascontiguousarray(b.T)
    da, db, dd = Dev(am), Dev(bm), Dev(nbytes=m * n * 4)
    desc = _desc(m, n, k, 1 if at else k, m if at else 1, n if bt else 1, 1 if bt else k, cfg=cfg)
    nv.call("nhip_gemm", C.byref(desc), da.ptr, db.ptr, dd.ptr)
    got = dd.get((m, n), np.float32)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max() + 1e-4


def test_gemm_batched_bf16_output(hip):
    rng = np.random.default_rng(0)
    z, m, n, k = 3, 96, 80, 48
    a = D.bf16_bits(rng.standard_normal((z, m, k)).astype(np.float32))
    b = D.bf16_bits(rng.standard_normal((z, n, k)).astype(np.float32))
    want = np.einsum("zmk,znk->zmn", D.bf16_to_f32(a).astype(np.float64), D.bf16_to_f32(b).astype(np.float64))
    da, db, dd = Dev(a), Dev(b), Dev(nbytes=z * m * n * 2)
    desc = _desc(m, n, k, k, 1, 1, k, out=nv.NHIP_BF16, batch=(z,), sa=(m * k,), sb=(n * k,), sd=(m * n,))
    nv.call("nhip_gemm", C.byref(desc), da.ptr, db.ptr, dd.ptr)
    got = D.bf16_to_f32(dd.get((z, m, n), np.uint16))
    np.testing.assert_allclose(got, want, rtol=2e-2, atol=1e-2 * np.abs(want).max())


@pytest.mark.parametrize("cfg,out", [(6, nv.NHIP_BF16), (7, nv.NHIP_F16), (7, nv.NHIP_F32), (8, nv.NHIP_BF16),
                                     (9, nv.NHIP_BF16), (9, nv.NHIP_F32), (10, nv.NHIP_BF16), (11, nv.NHIP_BF16),
                                     (11, nv.NHIP_F32), (12, nv.NHIP_BF16), (12, nv.NHIP_F32), (13, nv.NHIP_BF16),
                                     (13, nv.NHIP_F32), (14, nv.NHIP_BF16), (14, nv.NHIP_F32),
                                     (15, nv.NHIP_BF16), (15, nv.NHIP_F32)])
def test_gemm_streamed_16bit_outputs_and_ragged_edges(hip, cfg, out):
    """The streamed kernels' LDS-staged row stores (256 x 256 tiles, configs 6-8, 11-15; 128 x 128, config 9):
    16-bit and float32 outputs, m and n not multiples of the tile, two batches."""
    rng = np.random.default_rng(cfg + out)
    z, m, n, k = 2, 300, 264, 128
    a = D.bf16_bits(rng.standard_normal((z, m, k)).astype(np.float32))
    b = D.bf16_bits(rng.standard_normal((z, n, k)).astype(np.float32))
    want = np.einsum("zmk,znk->zmn", D.bf16_to_f32(a).astype(np.float64), D.bf16_to_f32(b).astype(np.float64))
    es = 4 if out == nv.NHIP_F32 else 2
    da, db, dd = Dev(a), Dev(b), Dev(nbytes=z * m * n * es)
    desc = _desc(m, n, k, k, 1, 1, k, out=out, cfg=cfg, batch=(z,), sa=(m * k,), sb=(n * k,), sd=(m * n,))
    nv.call("nhip_gemm", C.byref(desc), da.ptr, db.ptr, dd.ptr)
    if out == nv.NHIP_F32:
        got = dd.get((z, m, n), np.float32)
        assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max() + 1e-4
    else:
        raw = dd.get((z, m, n), np.uint16)
        got = D.bf16_to_f32(raw) if out == nv.NHIP_BF16 else raw.view(np.float16).astype(np.float32)
        np.testing.assert_allclose(got, want, rtol=2e-2, atol=1e-2 * np.abs(want).max())


@pytest.mark.parametrize("m,n,k,at,bt,out", [(4300, 4400, 128, False, False, nv.NHIP_F32),
                                              (4352, 4401, 64, True, False, nv.NHIP_BF16),
                                              (4400, 4352, 192, False, True, nv.NHIP_F16),
                                              (4352, 4352, 128, True, True, nv.NHIP_BF16)])
def test_gemm_persistent_walks_every_tile(hip, m, n, k, at, bt, out):
    """The persistent 256 x 256 kernel (config 10) with more tiles than CUs, so each workgroup runs several
    and prefetches the next one's first k tile during its last: ragged m and n, a single k tile (k = 64),
    every layout, row stores staged through LDS as 16-byte vectors and, for a row length that is not a
    multiple of 4 (n = 4401), element by element."""
    rng = np.random.default_rng(m + n + k)
    a = D.bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    b = D.bf16_bits(rng.standard_normal((k, n)).astype(np.float32))
    want = D.bf16_to_f32(a).astype(np.float64) @ D.bf16_to_f32(b).astype(np.float64)
    am = np.ascontiguousarray(a.T) if at else a
    bm = b if bt else np.ascontiguousarray(b.T)
    es = 4 if out == nv.NHIP_F32 else 2
    da, db, dd = Dev(am), Dev(bm), Dev(nbytes=m * n * es)
    desc = _desc(m, n, k, 1 if at else k, m if at else 1, n if bt else 1, 1 if bt else k, out=out, cfg=10)
    nv.call("nhip_gemm", C.byref(desc), da.ptr, db.ptr, dd.ptr)
    if out == nv.NHIP_F32:
        got = dd.get((m, n), np.float32)
        assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max() + 1e-4
    else:
        raw = dd.get((m, n), np.uint16)
        got = D.bf16_to_f32(raw) if out == nv.NHIP_BF16 else raw.view(np.float16).astype(np.float32)
        np.testing.assert_allclose(got, want, rtol=2e-2, atol=1e-2 * np.abs(want).max())


@pytest.mark.parametrize("at,bt,splits,out", [(True, True, 4, nv.NHIP_BF16), (False, True, 2, nv.NHIP_F32),
                                              (True, False, 8, nv.NHIP_F16)])
@pytest.mark.parametrize("config", [-1, 9])
def test_gemm_splitk(hip, at, bt, splits, out, config):
    """Split-k (the weight-gradient shape: small output, deep k): partial products in the workspace, summed in
    split order; two batches, ragged m and n; partials from the 256 x 256 streamed kernel (default) and from
    the 128 x 128 one (config 9)."""
    rng = np.random.default_rng(splits)
    z, m, n, k = 2, 264, 200, 64 * splits * 3
    a = D.bf16_bits(rng.standard_normal((z, m, k)).astype(np.float32))
    b = D.bf16_bits(rng.standard_normal((z, k, n)).astype(np.float32))
    want = np.einsum("zmk,zkn->zmn", D.bf16_to_f32(a).astype(np.float64), D.bf16_to_f32(b).astype(np.float64))
    am = np.ascontiguousarray(a.transpose(0, 2, 1)) if at else a
    bm = b if bt else np.ascontiguousarray(b.transpose(0, 2, 1))
    es = 4 if out == nv.NHIP_F32 else 2
    da, db, dd = Dev(am), Dev(bm), Dev(nbytes=z * m * n * es)
    desc = _desc(m, n, k, 1 if at else k, m if at else 1, n if bt else 1, 1 if bt else k, out=out,
                 batch=(z,), sa=(m * k,), sb=(n * k,), sd=(m * n,))
    desc.splits = splits
    desc.config = config
    ws = C.c_size_t()
    nv.call("nhip_gemm_workspace", C.byref(desc), C.byref(ws))
    assert ws.value == splits * z * m * n * 4
    dw = Dev(nbytes=ws.value)
    nv.call("nhip_gemm_splitk", C.byref(desc), da.ptr, db.ptr, dd.ptr, dw.ptr)
    if out == nv.NHIP_F32:
        got = dd.get((z, m, n), np.float32)
        assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max() + 1e-4
    else:
        raw = dd.get((z, m, n), np.uint16)
        got = D.bf16_to_f32(raw) if out == nv.NHIP_BF16 else raw.view(np.float16).astype(np.float32)
        np.testing.assert_allclose(got, want, rtol=2e-2, atol=1e-2 * np.abs(want).max())


def test_gemm_f32_is_the_sequential_fold(hip):
    """float32 operands: every output equals the k-order fold rounded after each product and sum."""
    rng = np.random.default_rng(3)
    m, n, k = 33, 65, 129
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    acc = np.zeros((m, n), np.float32)
    for kk in range(k):
        acc = (acc + (a[:, kk : kk + 1] * b[kk : kk + 1, :]).astype(np.float32)).astype(np.float32)
    da, db, dd = Dev(a), Dev(b), Dev(nbytes=m * n * 4)
    desc = _desc(m, n, k, k, 1, n, 1, dt=nv.NHIP_F32)
    nv.call("nhip_gemm", C.byref(desc), da.ptr, db.ptr, dd.ptr)
    assert np.array_equal(dd.get((m, n), np.float32).view(np.uint32), acc.view(np.uint32))


@pytest.mark.parametrize("at,bt", [(False, False), (False, True), (True, False), (True, True)])
def test_gemm_throughput(hip, at, bt):
    """Times 8192^3 bf16 in every layout (random data) and prints TFLOP/s."""
    m = n = k = 8192
    rng = np.random.default_rng(0)
    a = D.bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    da, db, dd = Dev(a), Dev(a), Dev(nbytes=m * n * 2)
    desc = _desc(m, n, k, 1 if at else k, m if at else 1, n if bt else 1, 1 if bt else k, out=nv.NHIP_BF16)
    nv.call("nhip_gemm", C.byref(desc), da.ptr, db.ptr, dd.ptr)
    nv.sync()
    e0, e1 = nv.Event(), nv.Event()
    e0.record()
    for _ in range(5):
        nv.call("nhip_gemm", C.byref(desc), da.ptr, db.ptr, dd.ptr)
    e1.record()
    ms = e0.elapsed_ms(e1) / 5
    print(f"gemm 8192^3 at={at} bt={bt}: {ms * 1e3:.1f} us {2 * m * n * k / ms / 1e9:.1f} TFLOP/s")


def test_plan_autotunes_large_dots(hip):
    """A compiled dot of 2^30 multiply-adds is timed over the tile configs before its first run; the chosen
    config is kept per shape and the result matches the float64 product within bf16 rounding."""
    import lumen_amd as L
    import lumen_amd.functional as F
    from lumen_amd.compiler.plan import Plan

    rng = np.random.default_rng(5)
    x = D.bf16_bits(rng.standard_normal((1024, 1024)).astype(np.float32))
    w = D.bf16_bits(rng.standard_normal((1024, 1024)).astype(np.float32))
    fn = L.compile(lambda a, b: F.matmul(a, b.t(), "float32", "bfloat16"), device="hip")
    got = L.to_numpy(fn(L.tensor(D.bf16_to_f32(x), "bfloat16", "hip"), L.tensor(D.bf16_to_f32(w), "bfloat16", "hip")))
    want = D.bf16_to_f32(x).astype(np.float64) @ D.bf16_to_f32(w).astype(np.float64).T
    np.testing.assert_allclose(got, want, rtol=2e-2, atol=1e-2 * np.abs(want).max())
    dots = [st for st in fn.plan.steps if st.kind == "dot"]
    assert dots and all(getattr(st, "config", -1) >= 0 for st in dots)
    assert any(v >= 0 for v in Plan._tuned.values())


def test_gemm_persistent_f16_operands(hip):
    """The persistent kernel (config 10) with float16 operands (the f16 MFMA) and more tiles than CUs."""
    rng = np.random.default_rng(40)
    m, n, k = 4352, 4352, 128
    a = rng.standard_normal((m, k)).astype(np.float16)
    b = rng.standard_normal((n, k)).astype(np.float16)
    want = a.astype(np.float64) @ b.astype(np.float64).T
    da, db, dd = Dev(a.view(np.uint16)), Dev(b.view(np.uint16)), Dev(nbytes=m * n * 4)
    desc = _desc(m, n, k, k, 1, 1, k, dt=nv.NHIP_F16, cfg=10)
    nv.call("nhip_gemm", C.byref(desc), da.ptr, db.ptr, dd.ptr)
    got = dd.get((m, n), np.float32)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max() + 1e-4
