"""The allocation-free flash backward (nhip_flash_bwd_noalloc, scratch in the library's own device array)
through the C ABI against nhip_flash_bwd with a caller workspace: identical bits on two calls in a row, the
second smaller, in each dQ mode (0 atomic, 1 stored dS, 2 recomputed), and a clear error above its scratch
limit."""

import ctypes as C
import math

import numpy as np
import pytest

from lumen_amd import dtypes as D
from lumen_amd import native as nv
from tests.hiputil import Dev, attn_desc

pytestmark = pytest.mark.gpu


def _run_both(b, s, n, nkv, d, causal, seed, mode):
    rng = np.random.default_rng(seed)

    def bf(*shape):
        return D.bf16_bits(rng.standard_normal(shape).astype(np.float32))

    q, k, v, g = bf(b, s, n, d), bf(b, s, nkv, d), bf(b, s, nkv, d), bf(b, s, n, d)
    desc = attn_desc(b, s, s, n, nkv, d, causal, 1.0 / math.sqrt(d))
    desc.deterministic = mode
    dq_, dk_, dv_, dg = Dev(q), Dev(k), Dev(v), Dev(g)
    o, lse = Dev(nbytes=q.nbytes), Dev(nbytes=b * n * s * 4)
    nv.call("nhip_flash_fwd", C.byref(desc), dq_.ptr, dk_.ptr, dv_.ptr, o.ptr, lse.ptr)
    ws_bytes = C.c_size_t()
    nv.call("nhip_flash_bwd_workspace", C.byref(desc), C.byref(ws_bytes))
    ws = Dev(nbytes=ws_bytes.value)
    outs = []
    for entry in ("nhip_flash_bwd", "nhip_flash_bwd_noalloc"):
        gq, gk, gv = Dev(nbytes=q.nbytes), Dev(nbytes=k.nbytes), Dev(nbytes=v.nbytes)
        args = [C.byref(desc), dq_.ptr, dk_.ptr, dv_.ptr, o.ptr, dg.ptr, lse.ptr, gq.ptr, gk.ptr, gv.ptr]
        nv.call(entry, *(args + [ws.ptr] if entry == "nhip_flash_bwd" else args))
        outs.append([t.get(x.shape, np.uint16) for t, x in ((gq, q), (gk, k), (gv, v))])
    return outs


@pytest.mark.parametrize("mode", [1, 2, 0])
def test_noalloc_flash_backward_matches_workspace_entry_point(hip, mode):
    """Modes 1 and 2 bit for bit. Mode 0 adds dQ with float32 atomics in no fixed order, so its dQ is compared
    within one bf16 rounding of each row's largest value (dK and dV bit for bit); the larger call runs first,
    so the smaller one starts on the stale accumulator it must clear itself."""
    for case in [(2, 512, 4, 2, 128, True, 0), (1, 130, 2, 2, 64, False, 1)]:  # the second call is smaller
        print("noalloc flash bwd mode", mode, case, flush=True)
        ref, got = _run_both(*case, mode)
        for name, a, w in zip(("dq", "dk", "dv"), got, ref):
            if mode == 0 and name == "dq":
                fa, fw = D.bf16_to_f32(a), D.bf16_to_f32(w)
                tol = 2.0 ** -7 * np.abs(fw).max(axis=-1, keepdims=True) + 1e-6
                assert (np.abs(fa - fw) <= tol).all(), name
            else:
                assert np.array_equal(a, w), name


def test_noalloc_flash_backward_rejects_sizes_above_its_scratch(hip):
    desc = attn_desc(64, 8192, 8192, 16, 16, 128, True, 0.1)  # 2^23 query rows > 2^21
    rc = nv.lib().nhip_flash_bwd_noalloc(C.byref(desc), *([None] * 9))
    assert rc != 0
    assert b"scratch" in nv.lib().nhip_last_error()
