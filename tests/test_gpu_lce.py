"""The fused linear cross entropy (Primitive::LinearCrossEntropy, lumen/reference/mod.rs:1092-1120) on the GPU:
loss and log-sum-exp rows of h [b, d] . w [v, d]^T without the [b, v] logits, against the oracle."""

import ctypes as C

import numpy as np
import pytest

import lumen_amd as L
from lumen_amd import dtypes as D
from lumen_amd import native as nv
from lumen_amd.compiler.plan import Plan
from lumen_amd.graph import prims
from oracle import oracle
from tests.hiputil import Dev

pytestmark = pytest.mark.gpu


def _run(h, w, t, hdt):
    args = [L.tensor(D.bf16_to_f32(h) if hdt == "bfloat16" else h, hdt),
            L.tensor(D.bf16_to_f32(w) if hdt == "bfloat16" else w, hdt), L.from_numpy(t)]
    f = L.compile(lambda h, w, t: prims.linear_cross_entropy(h, w, t), device="hip")
    got = np.asarray(L.to_numpy(f(*args)), np.float32)
    assert [s["kind"] for s in f.plan.describe()] == ["linear_cross_entropy"]
    (want,) = oracle.values(L.make_graph(lambda h, w, t: prims.linear_cross_entropy(h, w, t))(*args), [h, w, t])
    return got, np.asarray(want, np.float32), f


def _within_lse_ulps(got, want):
    lse_ulp = np.spacing(np.abs(want[1]))
    assert np.all(np.abs(got[1] - want[1]) <= 2 * lse_ulp), np.abs(got[1] - want[1]).max()
    assert np.all(np.abs(got[0] - want[0]) <= 2 * lse_ulp + np.spacing(np.abs(want[0]))), np.abs(got[0] - want[0]).max()


@pytest.mark.parametrize("b,v,d", [(64, 1000, 96), (37, 4097, 64)])
def test_float32_loss_and_lse_are_within_2_ulp(hip, b, v, d):
    """float32 h and w: the logits are the reference's sequential k fold (the exact GEMM); the exponentials
    are float32 (within 2 ulp) summed in float64 where the reference takes float64 exponentials; the lse
    agrees with the oracle to 2 ulp, and the loss (lse minus a logit) to the lse's 2 ulp plus its own
    rounding."""
    rng = np.random.default_rng(b + v)
    h = rng.standard_normal((b, d)).astype(np.float32)
    w = rng.standard_normal((v, d)).astype(np.float32) * 0.2
    t = rng.integers(0, v, b).astype(np.int32)
    got, want, _ = _run(h, w, t, "float32")
    assert got.shape == (2, b)
    _within_lse_ulps(got, want)


def test_bf16_with_clamped_int64_targets_and_chunks(hip, monkeypatch):
    """bf16 operands (MFMA logits, float32 accumulation), int64 targets below 0 and past v (clamped to the
    first and last class, like the reference), and a scratch so small that the rows go in 13-row chunks with
    a ragged last one: float32 tolerance (rtol 1e-4 of the row's scale) against the oracle."""
    monkeypatch.setattr(Plan, "LCE_SCRATCH", 13 * 3000 * 4)
    rng = np.random.default_rng(5)
    b, v, d = 200, 3000, 128
    h = D.bf16_bits(rng.standard_normal((b, d)).astype(np.float32))
    w = D.bf16_bits((rng.standard_normal((v, d)) * 0.1).astype(np.float32))
    t = rng.integers(-5, v + 5, b).astype(np.int64)
    t[:3] = [-7, v, v + 100]
    got, want, f = _run(h, w, t, "bfloat16")
    assert f.plan._lce_desc(f.plan.steps[0].nodes[0]).chunk_rows == 13
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-4 * np.abs(want).max())


def _abi(h, w, t, chunk_rows, h_offset=0):
    """nhip_linear_cross_entropy through the C ABI with the workspace nhip_linear_cross_entropy_workspace asks
    for; h at ``h_offset`` bytes into its block. Returns (out [2, b], workspace bytes)."""
    b, d = h.shape
    desc = nv.LceDesc()
    desc.b, desc.v, desc.d, desc.chunk_rows = b, w.shape[0], d, chunk_rows
    desc.dtype, desc.target_dtype = nv.NHIP_BF16, nv.NHIP_LCE_I32 if t.dtype == np.int32 else nv.NHIP_LCE_I64
    ws = C.c_size_t()
    nv.call("nhip_linear_cross_entropy_workspace", C.byref(desc), C.byref(ws))
    dh = Dev(nbytes=h.nbytes + 16)
    nv.h2d(dh.ptr + h_offset, np.ascontiguousarray(h).ctypes.data, h.nbytes)
    dw, dt, do, dws = Dev(w), Dev(t), Dev(nbytes=2 * b * 4), Dev(nbytes=ws.value)
    nv.call("nhip_linear_cross_entropy", C.byref(desc), dh.ptr + h_offset, dw.ptr, dt.ptr, do.ptr, dws.ptr)
    return do.get((2, b), np.float32), ws.value


@pytest.mark.parametrize("v", [2048, 2000])
def test_c_abi_matches_plan(hip, v):
    """nhip_linear_cross_entropy through the C ABI against the compiled plan: with v a multiple of 64 both take
    the fused form (workspace: a (maximum, sum) pair a row and 64-class block plus a logit a row); otherwise
    the ABI call goes in 50-row chunks of float32 logits and the plan in one: the same float32 values up to
    the GEMM tile the row count selects (rtol 1e-5)."""
    rng = np.random.default_rng(8)
    b, d = 96, 64
    h = D.bf16_bits(rng.standard_normal((b, d)).astype(np.float32))
    w = D.bf16_bits((rng.standard_normal((v, d)) * 0.1).astype(np.float32))
    t = rng.integers(0, v, b).astype(np.int32)
    want, _, _ = _run(h, w, t, "bfloat16")
    got, ws = _abi(h, w, t, 50)
    assert ws == (b * (v // 64) * 8 + 255) // 256 * 256 + b * 4 if v % 64 == 0 else ws == 50 * v * 4
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5 * np.abs(want).max())


def test_fused_form_with_ragged_tiles_and_clamped_targets(hip):
    """The fused form (the GEMM's store reduces each 64-class block, a merge kernel the blocks) with rows and
    classes that fill neither 256-row nor 256-class tiles (b 300, v 4160 = 65 blocks), logits large enough
    that most exponentials underflow, and int64 targets below 0 and past v (clamped): against the oracle at
    float32 tolerance."""
    rng = np.random.default_rng(41)
    b, v, d = 300, 4160, 128
    h = D.bf16_bits(rng.standard_normal((b, d)).astype(np.float32) * 3.0)
    w = D.bf16_bits((rng.standard_normal((v, d)) * 0.6).astype(np.float32))
    t = rng.integers(-5, v + 5, b).astype(np.int64)
    t[:4] = [-1, v, v + 7, v - 1]
    got, want, f = _run(h, w, t, "bfloat16")
    assert Plan._lce_scratch(f.plan._lce_desc(f.plan.steps[0].nodes[0])) < b * v * 4 // 16
    assert np.ptp(want[1]) > 10  # rows of very different scales
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-4 * np.abs(want).max())


def test_fused_form_with_unaligned_operands_takes_the_row_kernel(hip):
    """h one bf16 element past a 16-byte boundary: the fused form's loads need 16-byte rows, so the call goes
    through float32 logit rows in chunks that fit the fused form's workspace, and agrees with the aligned call
    to float32 rounding of the two reductions (rtol 1e-5)."""
    rng = np.random.default_rng(43)
    b, v, d = 64, 1024, 64
    h = D.bf16_bits(rng.standard_normal((b, d)).astype(np.float32))
    w = D.bf16_bits((rng.standard_normal((v, d)) * 0.1).astype(np.float32))
    t = rng.integers(0, v, b).astype(np.int32)
    aligned, ws = _abi(h, w, t, 0)
    unaligned, ws2 = _abi(h, w, t, 0, h_offset=2)
    assert ws == ws2 and ws < b * v * 4
    np.testing.assert_allclose(unaligned, aligned, rtol=1e-5, atol=1e-5 * np.abs(aligned).max())


def test_compiled_eval_loss_uses_the_fused_step(hip):
    """mean(cross_entropy(h . w^T, t)) compiled for hip: the linear_cross_entropy pass (on by default) turns it
    into the fused step, and the loss equals the oracle's on the unfused graph within float32 tolerance."""
    import lumen_amd.functional as F

    def fn(h, w, t):
        return F.mean(F.cross_entropy(F.matmul(h, w.t(), "float32", "float32"), t))

    rng = np.random.default_rng(21)
    b, v, d = 512, 5000, 256
    h = D.bf16_bits(rng.standard_normal((b, d)).astype(np.float32))
    w = D.bf16_bits((rng.standard_normal((v, d)) * 0.05).astype(np.float32))
    t = rng.integers(0, v, b).astype(np.int64)
    args = [L.tensor(D.bf16_to_f32(h), "bfloat16"), L.tensor(D.bf16_to_f32(w), "bfloat16"), L.from_numpy(t)]
    f = L.compile(fn, device="hip")
    got = float(L.to_numpy(f(*args)))
    assert "linear_cross_entropy" in [s["kind"] for s in f.plan.describe()]
    (want,) = oracle.values(L.make_graph(fn)(*args), [h, w, t])
    np.testing.assert_allclose(got, float(want), rtol=1e-4)


def test_f16_operands_and_ragged_rows(hip):
    """float16 h and w (the f16 MFMA GEMM) with a class count that is not a multiple of 4 (the row kernel's
    element-by-element loads) against the oracle at float32 tolerance."""
    rng = np.random.default_rng(31)
    b, v, d = 130, 1003, 64
    h = (rng.standard_normal((b, d)) * 0.5).astype(np.float16)
    w = (rng.standard_normal((v, d)) * 0.2).astype(np.float16)
    t = rng.integers(0, v, b).astype(np.int32)
    args = [L.tensor(h.astype(np.float32), "float16"), L.tensor(w.astype(np.float32), "float16"), L.from_numpy(t)]
    f = L.compile(lambda h, w, t: prims.linear_cross_entropy(h, w, t), device="hip")
    got = np.asarray(L.to_numpy(f(*args)), np.float32)
    (want,) = oracle.values(L.make_graph(lambda h, w, t: prims.linear_cross_entropy(h, w, t))(*args),
                            [h.astype(np.float32), w.astype(np.float32), t])
    np.testing.assert_allclose(got, np.asarray(want, np.float32), rtol=1e-4, atol=1e-4 * np.abs(want).max())


@pytest.mark.parametrize("b,v", [(1, 1), (3, 2), (5, 7)])
def test_smallest_shapes(hip, b, v):
    """One row, one class (the loss is 0 and the lse the only logit), and other shapes below a 16-byte load
    (element-by-element row reads), float32 against the oracle to 2 ulp."""
    rng = np.random.default_rng(b * 10 + v)
    d = 8
    h = rng.standard_normal((b, d)).astype(np.float32)
    w = rng.standard_normal((v, d)).astype(np.float32)
    t = rng.integers(0, v, b).astype(np.int32)
    got, want, _ = _run(h, w, t, "float32")
    _within_lse_ulps(got, want)
    if v == 1:
        assert np.all(got[0] == 0.0)
