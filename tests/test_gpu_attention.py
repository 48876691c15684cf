"""Flash attention kernels through the C ABI against the oracle's unfused matmul-softmax-matmul graph."""

import ctypes as C
import math

import numpy as np
import pytest

import lumen_amd as L
import lumen_amd.functional as F
from lumen_amd import dtypes as D
from lumen_amd import native as nv
from oracle import oracle
from tests.hiputil import Dev, attn_desc

pytestmark = pytest.mark.gpu

CASES = [
    # b, sq, sk, n, nkv, d, causal
    (1, 128, 128, 2, 2, 64, False),
    (1, 128, 128, 2, 2, 64, True),
    (2, 200, 200, 2, 1, 128, True),
    (1, 64, 192, 4, 2, 128, True),
    (1, 96, 160, 1, 1, 64, False),
    (1, 1024, 1024, 2, 1, 128, True),
    # head dims padded to the kernels' 64 or 128 (zero columns past them)
    (1, 128, 160, 2, 2, 32, True),
    (2, 96, 96, 4, 2, 96, True),
    (1, 200, 136, 2, 1, 72, False),
]
# the forward alone also takes head dims up to 256
FWD_CASES = CASES + [(1, 200, 200, 2, 1, 256, True), (2, 64, 130, 2, 2, 192, False)]


def _inputs(b, sq, sk, n, nkv, d, seed=0):
    rng = np.random.default_rng(seed)
    q = D.bf16_bits(rng.standard_normal((b, sq, n, d)).astype(np.float32))
    k = D.bf16_bits(rng.standard_normal((b, sk, nkv, d)).astype(np.float32))
    v = D.bf16_bits(rng.standard_normal((b, sk, nkv, d)).astype(np.float32))
    return q, k, v


@pytest.mark.parametrize("b,sq,sk,n,nkv,d,causal", FWD_CASES)
def test_flash_forward_matches_unfused_graph(hip, b, sq, sk, n, nkv, d, causal):
    q, k, v = _inputs(b, sq, sk, n, nkv, d)
    scale = 1.0 / math.sqrt(d)
    dq, dk, dv = Dev(q), Dev(k), Dev(v)
    do_ = Dev(nbytes=q.nbytes)
    lse = Dev(nbytes=b * n * sq * 4)
    desc = attn_desc(b, sq, sk, n, nkv, d, causal, scale)
    nv.call("nhip_flash_fwd", C.byref(desc), dq.ptr, dk.ptr, dv.ptr, do_.ptr, lse.ptr)
    got = D.bf16_to_f32(do_.get(q.shape, np.uint16))
    got_lse = lse.get((b, n, sq), np.float32)

    def attn(q, k, v):
        return F.flash_attention(q, k, v, is_causal=causal)

    meta = [L.empty(list(x.shape), "bfloat16", "meta") for x in (q, k, v)]
    (want,) = oracle.values(L.make_graph(attn)(*meta), [q, k, v])
    np.testing.assert_allclose(got, want, rtol=2e-2, atol=1e-2)
    # log-sum-exp of the scaled, masked scores in float64
    qf, kf = (D.bf16_to_f32(x).astype(np.float64) for x in (q, k))
    kf = np.repeat(kf, n // nkv, axis=2)
    s = np.einsum("bqnd,bknd->bnqk", qf, kf) * scale
    if causal:
        mask = np.arange(sk)[None, :] <= np.arange(sq)[:, None] + (sk - sq)
        s = np.where(mask, s, -np.inf)
    m = s.max(-1)
    ref_lse = m + np.log(np.exp(s - m[..., None]).sum(-1))
    np.testing.assert_allclose(got_lse, ref_lse, rtol=1e-4, atol=1e-4)


def test_flash_forward_config3_throughput(hip):
    """B=8, H=16, S=2048, D=128 causal: runs, finite, and reports its time."""
    b, s, n, d = 8, 2048, 16, 128
    rng = np.random.default_rng(0)
    q = D.bf16_bits(rng.standard_normal((b, s, n, d)).astype(np.float32))
    dq, dk, dv = Dev(q), Dev(q), Dev(q)
    o = Dev(nbytes=q.nbytes)
    lse = Dev(nbytes=b * n * s * 4)
    desc = attn_desc(b, s, s, n, n, d, True, 1 / math.sqrt(d))
    flops = 2 * b * n * s * s * d  # causal half of 4 B N S^2 D
    for cfg, waves in enumerate((4, 8, 2)):
        desc.config = cfg
        nv.call("nhip_flash_fwd", C.byref(desc), dq.ptr, dk.ptr, dv.ptr, o.ptr, lse.ptr)
        nv.sync()
        e0, e1 = nv.Event(), nv.Event()
        e0.record()
        for _ in range(10):
            nv.call("nhip_flash_fwd", C.byref(desc), dq.ptr, dk.ptr, dv.ptr, o.ptr, lse.ptr)
        e1.record()
        ms = e0.elapsed_ms(e1) / 10
        print(f"flash fwd config3, {waves} waves a workgroup: {ms * 1e3:.1f} us, {flops / ms / 1e9:.1f} TFLOP/s")
    out = D.bf16_to_f32(o.get(q.shape, np.uint16))
    assert np.isfinite(out).all()


@pytest.mark.parametrize("deterministic", [1, 2, 0])
@pytest.mark.parametrize("b,sq,sk,n,nkv,d,causal", CASES)
def test_flash_backward_matches_unfused_graph(hip, b, sq, sk, n, nkv, d, causal, deterministic):
    """dQ, dK, dV from the backward kernels against the oracle running the traced FlashAttention-2 backward
    (recomputed probabilities from the saved log-sum-exp), bf16 tolerance; dQ from the stored dS tiles (1), by a
    kernel recomputing S and dP (2), or added atomically by the dK/dV kernel (0)."""
    q, k, v = _inputs(b, sq, sk, n, nkv, d, seed=1)
    rng = np.random.default_rng(2)
    g = D.bf16_bits(rng.standard_normal((b, sq, n, d)).astype(np.float32))
    scale = 1.0 / math.sqrt(d)
    desc = attn_desc(b, sq, sk, n, nkv, d, causal, scale, deterministic=deterministic)
    dq_, dk_, dv_, dg = Dev(q), Dev(k), Dev(v), Dev(g)
    o, lse = Dev(nbytes=q.nbytes), Dev(nbytes=b * n * sq * 4)
    nv.call("nhip_flash_fwd", C.byref(desc), dq_.ptr, dk_.ptr, dv_.ptr, o.ptr, lse.ptr)
    gq, gk, gv = Dev(nbytes=q.nbytes), Dev(nbytes=k.nbytes), Dev(nbytes=v.nbytes)
    ws_bytes = C.c_size_t()
    nv.call("nhip_flash_bwd_workspace", C.byref(desc), C.byref(ws_bytes))
    ws = Dev(nbytes=ws_bytes.value)
    nv.call("nhip_flash_bwd", C.byref(desc), dq_.ptr, dk_.ptr, dv_.ptr, o.ptr, dg.ptr, lse.ptr, gq.ptr, gk.ptr, gv.ptr, ws.ptr)
    got = [D.bf16_to_f32(t.get(x.shape, np.uint16)) for t, x in ((gq, q), (gk, k), (gv, v))]

    def grads(q, k, v, do):
        _, pull = L.vjp(lambda q, k, v: F.flash_attention(q, k, v, is_causal=causal), q, k, v)
        return pull(do)

    meta = [L.empty(list(x.shape), "bfloat16", "meta") for x in (q, k, v, g)]
    want = oracle.values(L.make_graph(grads)(*meta), [q, k, v, g])
    for name, a, w in zip(("dq", "dk", "dv"), got, want):
        scale_w = np.abs(w).max()
        np.testing.assert_allclose(a, w, rtol=2e-2, atol=1e-2 * max(1.0, scale_w), err_msg=name)


def test_flash_backward_config3_throughput(hip):
    b, s, n, d = 8, 2048, 16, 128
    rng = np.random.default_rng(0)
    q = D.bf16_bits(rng.standard_normal((b, s, n, d)).astype(np.float32))
    dq, dk, dv, g = Dev(q), Dev(q), Dev(q), Dev(q)
    o = Dev(nbytes=q.nbytes)
    lse = Dev(nbytes=b * n * s * 4)
    desc = attn_desc(b, s, s, n, n, d, True, 1 / math.sqrt(d))
    nv.call("nhip_flash_fwd", C.byref(desc), dq.ptr, dk.ptr, dv.ptr, o.ptr, lse.ptr)
    ws_bytes = C.c_size_t()
    nv.call("nhip_flash_bwd_workspace", C.byref(desc), C.byref(ws_bytes))
    gq, gk, gv, ws = Dev(nbytes=q.nbytes), Dev(nbytes=q.nbytes), Dev(nbytes=q.nbytes), Dev(nbytes=ws_bytes.value)
    flops = 2.5 * 2 * b * n * s * s * d
    for det in (1, 2, 0):
        desc.deterministic = det
        nv.call("nhip_flash_bwd_workspace", C.byref(desc), C.byref(ws_bytes))
        ws = Dev(nbytes=ws_bytes.value)
        args = (C.byref(desc), dq.ptr, dk.ptr, dv.ptr, o.ptr, g.ptr, lse.ptr, gq.ptr, gk.ptr, gv.ptr, ws.ptr)
        nv.call("nhip_flash_bwd", *args)
        nv.sync()
        e0, e1 = nv.Event(), nv.Event()
        e0.record()
        for _ in range(5):
            nv.call("nhip_flash_bwd", *args)
        e1.record()
        ms = e0.elapsed_ms(e1) / 5
        mode = {1: "dQ from stored dS", 2: "dQ recomputing S and dP", 0: "atomic dQ"}[det]
        print(f"flash bwd config3 ({mode}): {ms * 1e3:.1f} us, {flops / ms / 1e9:.1f} TFLOP/s (algorithmic 2.5x fwd)")
    assert np.isfinite(D.bf16_to_f32(gq.get(q.shape, np.uint16))).all()


@pytest.mark.parametrize("b,sq,sk,n,nkv,d,causal", [CASES[1], CASES[2], CASES[3], CASES[5], CASES[7], FWD_CASES[-2]])
def test_forward_tile_configs_agree_bit_for_bit(hip, b, sq, sk, n, nkv, d, causal):
    """Every forward tile config (4, 8 or 2 waves a workgroup) gives the same bits: each query is one lane's,
    its keys visited in the same tiles and order whatever the workgroup size (head dim 256 runs one tile)."""
    q, k, v = _inputs(b, sq, sk, n, nkv, d, seed=3)
    dq, dk, dv = Dev(q), Dev(k), Dev(v)
    count = C.c_int()
    nv.call("nhip_attn_config_count", C.byref(count))
    assert count.value == 3
    outs = []
    for cfg in range(count.value):
        desc = attn_desc(b, sq, sk, n, nkv, d, causal, 1.0 / math.sqrt(d))
        desc.config = cfg
        o, lse = Dev(nbytes=q.nbytes), Dev(nbytes=b * n * sq * 4)
        nv.call("nhip_flash_fwd", C.byref(desc), dq.ptr, dk.ptr, dv.ptr, o.ptr, lse.ptr)
        outs.append((o.get(q.shape, np.uint16), lse.get((b, n, sq), np.float32)))
    for o, lse in outs[1:]:
        assert np.array_equal(o, outs[0][0])
        assert np.array_equal(lse.view(np.uint32), outs[0][1].view(np.uint32))


def test_forced_configs_reach_the_plan(hip):
    """``autotune.use`` forces the GEMM and attention configs of a compiled plan, untimed; the results equal
    the autotuned plan's within the bf16 tolerance (and the attention bit for bit)."""
    from lumen_amd import autotune as A

    rng = np.random.default_rng(4)
    shapes = [(2, 256, 4, 64), (2, 256, 4, 64), (2, 256, 4, 64), (256, 256)]
    ts = [L.tensor(rng.standard_normal(s).astype(np.float32), "bfloat16") for s in shapes]

    def fn(q, k, v, w):
        o = F.flash_attention(q, k, v, is_causal=True)
        return F.matmul(o.reshape(512, 256), w, "float32", "bfloat16")

    free = L.compile(fn, device="hip")
    want = L.to_numpy(free(*ts))
    with A.use(A.HipGemmConfig(3), A.HipAttentionConfig(waves=2)):
        f = L.compile(fn, device="hip")
        got = L.to_numpy(f(*ts))
        steps = f.plan.steps
    assert [getattr(s, "config", None) for s in steps if s.kind == "flash_fwd"] == [2]
    assert [getattr(s, "config", None) for s in steps if s.kind == "dot"] == [3]
    np.testing.assert_allclose(got, want, rtol=2e-2, atol=1e-2 * np.abs(want).max())


def _attention_f64(q, k, v, g, scale, causal):
    """Float64 attention of one (batch, head) slice, [S, D] operands: the output, the natural-log LSE and the
    FlashAttention-2 gradients dQ, dK, dV of <O, g> (brute force on the whole score matrix)."""
    s = (q @ k.T) * scale
    if causal:
        s = np.where(np.tril(np.ones(s.shape, bool), s.shape[1] - s.shape[0]), s, -np.inf)
    m = s.max(-1, keepdims=True)
    e = np.exp(s - m)
    l_ = e.sum(-1, keepdims=True)
    p = e / l_
    o = p @ v
    dv = p.T @ g
    dp = g @ v.T
    ds = p * (dp - (g * o).sum(-1, keepdims=True))
    return o, (m + np.log(l_))[:, 0], ds @ k * scale, ds.T @ q * scale, dv


@pytest.mark.parametrize("deterministic", [1, 0])
def test_config3_full_size_slices_match_float64_attention(hip, deterministic):
    """Config 3 at its real size, [8, 2048, 16, 128] causal with independent N(0, 1) q, k, v and dO: the
    whole forward and backward run on the GPU; three (batch, head) slices of O and the LSE, and the dQ, dK,
    dV of two of them, are compared with float64 attention computed here from the same bf16 inputs (bf16
    tolerance: rtol 2e-2 plus 1e-2 of the slice's largest magnitude; LSE within 1e-3)."""
    b, s, n, d = 8, 2048, 16, 128
    rng = np.random.default_rng(33)
    q, k, v, g = (D.bf16_bits(rng.standard_normal((b, s, n, d), np.float32)) for _ in range(4))
    scale = 1.0 / math.sqrt(d)
    desc = attn_desc(b, s, s, n, n, d, True, scale, deterministic=deterministic)
    dq_, dk_, dv_, dg = Dev(q), Dev(k), Dev(v), Dev(g)
    o, lse = Dev(nbytes=q.nbytes), Dev(nbytes=b * n * s * 4)
    print("config3 full size fwd", flush=True)
    nv.call("nhip_flash_fwd", C.byref(desc), dq_.ptr, dk_.ptr, dv_.ptr, o.ptr, lse.ptr)
    ws_bytes = C.c_size_t()
    nv.call("nhip_flash_bwd_workspace", C.byref(desc), C.byref(ws_bytes))
    ws = Dev(nbytes=ws_bytes.value)
    gq, gk, gv = Dev(nbytes=q.nbytes), Dev(nbytes=k.nbytes), Dev(nbytes=v.nbytes)
    print("config3 full size bwd mode", deterministic, flush=True)
    nv.call("nhip_flash_bwd", C.byref(desc), dq_.ptr, dk_.ptr, dv_.ptr, o.ptr, dg.ptr, lse.ptr, gq.ptr, gk.ptr,
            gv.ptr, ws.ptr)
    got_o = D.bf16_to_f32(o.get(q.shape, np.uint16))
    got_lse = lse.get((b, n, s), np.float32)
    got_g = [D.bf16_to_f32(t.get(q.shape, np.uint16)) for t in (gq, gk, gv)]
    assert all(np.isfinite(x).all() for x in [got_o] + got_g)
    f = [D.bf16_to_f32(x).astype(np.float64) for x in (q, k, v, g)]
    for i, (bi, ni) in enumerate([(0, 0), (3, 7), (7, 15)]):
        sl = [x[bi, :, ni, :] for x in f]
        o64, lse64, dq64, dk64, dv64 = _attention_f64(*sl, scale, True)

        def close(a, w, what):
            np.testing.assert_allclose(a, w, rtol=2e-2, atol=1e-2 * np.abs(w).max(), err_msg=f"{what} b{bi} n{ni}")

        close(got_o[bi, :, ni, :], o64, "o")
        np.testing.assert_allclose(got_lse[bi, ni], lse64, rtol=1e-4, atol=1e-3)
        if i < 2:
            for name, a, w in zip(("dq", "dk", "dv"), got_g, (dq64, dk64, dv64)):
                close(a[bi, :, ni, :], w, name)


@pytest.mark.parametrize("d,dv,sq,sk,causal", [(16, 24, 5, 40, False), (32, 32, 70, 100, True), (96, 64, 64, 192, True),
                                               (64, 64, 40, 40, True)])
def test_partial_tiles_ignore_what_earlier_kernels_left_in_lds(hip, d, dv, sq, sk, causal):
    """The LDS chunks a partial tile leaves unloaded (rows past the sequence end, columns past a padded head
    dim) must not carry values an earlier kernel left in LDS: a forward and backward over all-NaN operands run
    first on every CU, then the partial shapes (value head dim apart from the query's included) in every dQ
    mode, checked finite and against the oracle."""
    nb, ns, nn = 8, 2048, 16  # poison: NaN Q, K, V and dO through the same kernels on every CU
    nanq = np.full((nb, ns, nn, 128), 0x7FC0, np.uint16)
    pq, po, pl = Dev(nanq), Dev(nbytes=nanq.nbytes), Dev(nbytes=nb * nn * ns * 4)
    pdesc = attn_desc(nb, ns, ns, nn, nn, 128, True, 0.1)
    nv.call("nhip_flash_fwd", C.byref(pdesc), pq.ptr, pq.ptr, pq.ptr, po.ptr, pl.ptr)
    rng = np.random.default_rng(d + dv + sk)
    b, n = 2, 2
    q, k = (D.bf16_bits(rng.standard_normal(s).astype(np.float32)) for s in ((b, sq, n, d), (b, sk, n, d)))
    v, g = (D.bf16_bits(rng.standard_normal(s).astype(np.float32)) for s in ((b, sk, n, dv), (b, sq, n, dv)))
    meta = [L.empty(list(x.shape), "bfloat16", "meta") for x in (q, k, v, g)]

    def grads(q, k, v, do):
        out, pull = L.vjp(lambda q, k, v: F.flash_attention(q, k, v, is_causal=causal), q, k, v)
        return (out,) + pull(do)

    want = oracle.values(L.make_graph(grads)(*meta), [q, k, v, g])
    for mode in (1, 2, 0):
        pws = C.c_size_t()
        pdesc.deterministic = mode
        nv.call("nhip_flash_bwd_workspace", C.byref(pdesc), C.byref(pws))
        pw = Dev(nbytes=pws.value)
        pg = Dev(nbytes=nanq.nbytes)
        nv.call("nhip_flash_bwd", C.byref(pdesc), pq.ptr, pq.ptr, pq.ptr, po.ptr, pq.ptr, pl.ptr, pg.ptr, pg.ptr,
                pg.ptr, pw.ptr)
        desc = attn_desc(b, sq, sk, n, n, d, causal, 1.0 / math.sqrt(d), deterministic=mode)
        desc.value_head_dim = dv
        for t in ("v", "o", "do", "dv"):
            rows = sk if t in ("v", "dv") else sq
            setattr(desc, f"{t}_b", rows * n * dv)
            setattr(desc, f"{t}_s", n * dv)
            setattr(desc, f"{t}_n", dv)
        dq_, dk_, dv_, dg = Dev(q), Dev(k), Dev(v), Dev(g)
        o, lse = Dev(nbytes=g.nbytes), Dev(nbytes=b * n * sq * 4)
        nv.call("nhip_flash_fwd", C.byref(desc), dq_.ptr, dk_.ptr, dv_.ptr, o.ptr, lse.ptr)
        ws_bytes = C.c_size_t()
        nv.call("nhip_flash_bwd_workspace", C.byref(desc), C.byref(ws_bytes))
        ws = Dev(nbytes=ws_bytes.value)
        gq, gk, gv = Dev(nbytes=q.nbytes), Dev(nbytes=k.nbytes), Dev(nbytes=v.nbytes)
        print("partial tiles", d, dv, sq, sk, causal, "mode", mode, flush=True)
        nv.call("nhip_flash_bwd", C.byref(desc), dq_.ptr, dk_.ptr, dv_.ptr, o.ptr, dg.ptr, lse.ptr, gq.ptr, gk.ptr,
                gv.ptr, ws.ptr)
        got = [D.bf16_to_f32(t.get(x.shape, np.uint16)) for t, x in ((o, g), (gq, q), (gk, k), (gv, v))]
        for name, a, w in zip(("o", "dq", "dk", "dv"), got, want):
            assert np.isfinite(a).all(), (name, mode)
            np.testing.assert_allclose(a, w, rtol=2e-2, atol=1e-2 * max(1.0, np.abs(w).max()), err_msg=f"{name} {mode}")
