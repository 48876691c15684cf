"""Helpers for GPU tests that call the C ABI directly: device copies of NumPy arrays."""

import ctypes as C

import numpy as np

from lumen_amd import native as nv


class Dev:
    """A device copy of a NumPy array (or an empty block of ``nbytes``), freed on deletion."""

    def __init__(self, arr=None, nbytes=None):
        nv.set_device(0)
        self.nbytes = arr.nbytes if arr is not None else nbytes
        self.ptr = nv.alloc(0, max(self.nbytes, 1))
        if arr is not None and arr.nbytes:
            a = np.ascontiguousarray(arr)
            nv.h2d(self.ptr, a.ctypes.data, a.nbytes)

    def get(self, shape, dtype):
        out = np.empty(shape, dtype)
        nv.d2h(out.ctypes.data, self.ptr, out.nbytes)
        return out

    def __del__(self):
        try:
            nv.free(0, self.ptr, self.nbytes)
        except Exception:
            pass


def attn_desc(b, sq, sk, n, nkv, d, causal, scale, dtype=1, deterministic=1):
    """Descriptor for contiguous [B, S, N, D] q/o/do/dq and [B, S, Nkv, D] k/v/dk/dv."""
    a = nv.AttnDesc()
    a.batch, a.heads, a.kv_heads, a.sq, a.sk, a.head_dim = b, n, nkv, sq, sk, d
    a.dtype, a.causal, a.scale, a.config = dtype, int(causal), scale, -1
    a.deterministic = int(deterministic)
    for t in ("q", "o", "do", "dq"):
        setattr(a, f"{t}_b", sq * n * d)
        setattr(a, f"{t}_s", n * d)
        setattr(a, f"{t}_n", d)
    for t in ("k", "v", "dk", "dv"):
        setattr(a, f"{t}_b", sk * nkv * d)
        setattr(a, f"{t}_s", nkv * d)
        setattr(a, f"{t}_n", d)
    return a


_ = C
