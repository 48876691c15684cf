"""Step-by-step parity of a compiled plan on the GPU: runs the plan one step at a time and compares every
value a step writes with the oracle's value of the same node of the compiled graph, so a wrong kernel is
named by its step rather than seen only in the final outputs. Test infrastructure (reads the oracle)."""

import numpy as np

from lumen_amd import dtypes as D
from lumen_amd import native as nv
from lumen_amd.compiler.plan import Plan
from lumen_amd.tensor import DeviceBuffer
from oracle import oracle


def _read(ptr_base, loc, dtype, shape):
    """The value at ``loc`` (element offset and strides from ``ptr_base``) as a NumPy array."""
    size = D.size_of(dtype)
    if not shape or int(np.prod(shape)) == 0:
        n = 1 if not shape else 0
        out = np.empty(shape, D.storage(dtype))
        if n:
            nv.d2h(out.ctypes.data, ptr_base + loc.offset * size, size)
        return out
    span = 1 + sum((s - 1) * st for s, st in zip(shape, loc.strides) if st > 0)
    flat = np.empty(span, D.storage(dtype))
    nv.d2h(flat.ctypes.data, ptr_base + loc.offset * size, span * size)
    view = np.lib.stride_tricks.as_strided(flat, shape=shape, strides=[st * size for st in loc.strides])
    return np.array(view)


def check_steps(graph, arrays, tolerance):
    """Compiles ``graph`` for hip:0, uploads ``arrays`` (its inputs, raw storage), runs the plan a step at a
    time and compares each written value with the oracle. ``tolerance(dtype, got, want)`` returns an error
    string or None. Returns a list of ``(step index, kind, label, value, message)`` for every mismatch."""
    plan = Plan(graph, "hip:0")
    g = plan.graph
    want = oracle.env(g, list(arrays))
    ins = [DeviceBuffer(0, max(1, np.asarray(a).nbytes)) for a in arrays]
    for buf, a in zip(ins, arrays):
        a = np.ascontiguousarray(a)
        if a.nbytes:
            nv.h2d(buf.ptr, a.ctypes.data, a.nbytes)
    ws = DeviceBuffer(0, max(1, plan.workspace_bytes))
    ptrs = [b.ptr for b in ins]
    plan._native_plan()
    bad = []
    for si, st in enumerate(plan.steps):
        if si in set(plan.native_steps):
            plan.run_steps(ws.ptr, ptrs, si)
        nv.call("nhip_stream_sync", 0)
        for v in st.outputs:
            loc = plan.loc[v]
            base = ws.ptr if loc.base[0] == "ws" else ptrs[loc.base[1]]
            ty = g.types[v]
            got = _read(base, loc, ty.dtype, tuple(ty.shape))
            msg = tolerance(ty.dtype, D.to_numpy_values(got, ty.dtype), np.asarray(want[v]))
            if msg:
                bad.append((si, st.kind, st.label(), v, msg))
    return bad
