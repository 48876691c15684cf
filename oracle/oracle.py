"""TEST INFRASTRUCTURE ONLY: ctypes front of ``liboracle.so`` (``oracle.c``), the CPU restatement of lumen's
reference interpreter (``lumen/reference/mod.rs``), and the text serialization of graphs it reads.

``run(graph, inputs)`` evaluates a ``lumen_amd`` graph on NumPy storage arrays (bfloat16 as uint16 bits) and
returns the outputs' storage arrays.
"""

from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

from lumen_amd import dtypes as D
from lumen_amd.graph.ir import Graph

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(HERE, "liboracle.so")
_lib = None


def build():
    """Compiles liboracle.so with the Makefile next to it."""
    subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY):
            build()
        _lib = C.CDLL(LIBRARY)
        _lib.oracle_run.argtypes = [C.c_char_p, C.POINTER(C.c_void_p), C.POINTER(C.c_void_p)]
        _lib.oracle_run.restype = C.c_int
        _lib.oracle_set_threads.argtypes = [C.c_int]
        _lib.oracle_set_threads.restype = None
        _lib.oracle_error.restype = C.c_char_p
        _lib.oracle_to_bf16.argtypes = [C.c_double]
        _lib.oracle_to_bf16.restype = C.c_uint16
        _lib.oracle_to_f16.argtypes = [C.c_double]
        _lib.oracle_to_f16.restype = C.c_uint16
        _lib.oracle_round_to_odd.argtypes = [C.c_double]
        _lib.oracle_round_to_odd.restype = C.c_float
        _lib.oracle_erf_inv.argtypes = [C.c_double]
        _lib.oracle_erf_inv.restype = C.c_double
        _lib.oracle_reduce_precision.argtypes = [C.c_double, C.c_int, C.c_int]
        _lib.oracle_reduce_precision.restype = C.c_double
        _lib.oracle_philox.argtypes = [C.c_uint64, C.c_uint64]
        _lib.oracle_philox.restype = C.c_uint32
        _lib.oracle_philox4x32.argtypes = [C.POINTER(C.c_uint32), C.POINTER(C.c_uint32), C.POINTER(C.c_uint32)]
        _lib.oracle_philox4x32.restype = None
    return _lib


def _param(key, v) -> list[str]:
    if isinstance(v, Graph):
        return [key, "g"] + [serialize(v)]
    if isinstance(v, bool):
        return [key, f"b:{int(v)}"]
    if isinstance(v, int):
        return [key, f"n:{v}"]
    if isinstance(v, float):
        return [key, f"f:{v.hex()}"]
    if isinstance(v, str):
        return [key, f"d:{v}"]
    if isinstance(v, (tuple, list)):
        return [key, f"i:{len(v)}:" + ",".join(str(int(x)) for x in v)]
    raise TypeError(f"cannot serialize parameter {key}={v!r}")


# Parameters the oracle does not read (labels, compiler annotations).
_SKIP = {"label", "name", "ty", "view", "in_place", "kernel", "role", "q_dims", "k_dims", "v_dims", "scale", "causal"}


def serialize(g: Graph) -> str:
    lines = ["graph", f"types {len(g.types)}"]
    for t in g.types:
        lines.append(f"{t.dtype} {len(t.shape)} " + " ".join(map(str, t.shape)))
    lines.append(f"inputs {len(g.inputs)} " + " ".join(map(str, g.inputs)))
    lines.append(f"nodes {len(g.nodes)}")
    for n in g.nodes:
        params = [(k, v) for k, v in sorted(n.params.items()) if k not in _SKIP]
        toks = [n.prim, str(n.output), str(len(n.inputs))] + [str(v) for v in n.inputs] + [str(len(params))]
        for k, v in params:
            toks += _param(k, v)
        lines.append(" ".join(toks))
    lines.append(f"outputs {len(g.outputs)} " + " ".join(map(str, g.outputs)))
    lines.append("end")
    return "\n".join(lines)


def set_threads(n: int) -> None:
    """Threads the oracle's dots may use (their output rows are independent; each fold is unchanged)."""
    lib().oracle_set_threads(int(n))


def run(graph: Graph, inputs: list) -> list:
    """Outputs (storage arrays) of ``graph`` on ``inputs`` (storage arrays or Tensors)."""
    if len(inputs) != len(graph.inputs):
        raise ValueError(f"the graph takes {len(graph.inputs)} inputs, got {len(inputs)}")
    arrays = []
    for v, x in zip(graph.inputs, inputs):
        ty = graph.types[v]
        if hasattr(x, "raw"):
            x = x.raw()
        a = np.ascontiguousarray(np.asarray(x), D.storage(ty.dtype)).reshape(np.asarray(x).shape)
        if tuple(a.shape) != tuple(ty.shape):
            raise ValueError(f"input %{v} must be {ty}, got shape {list(a.shape)}")
        arrays.append(a)
    outs = [np.empty(graph.types[v].shape, D.storage(graph.types[v].dtype)) for v in graph.outputs]
    ins = (C.c_void_p * max(1, len(arrays)))(*[a.ctypes.data for a in arrays])
    ous = (C.c_void_p * max(1, len(outs)))(*[o.ctypes.data for o in outs])
    if lib().oracle_run(serialize(graph).encode(), ins, ous) != 0:
        raise RuntimeError(lib().oracle_error().decode())
    return outs


def values(graph: Graph, inputs: list) -> list:
    """``run``'s outputs as NumPy values (bfloat16 widened to float32)."""
    return [D.to_numpy_values(o, graph.types[v].dtype) for o, v in zip(run(graph, inputs), graph.outputs)]


def philox4x32(key, counter):
    """Philox4x32-10 block of the oracle (for the Random123 known-answer tests)."""
    k = (C.c_uint32 * 2)(*key)
    c = (C.c_uint32 * 4)(*counter)
    o = (C.c_uint32 * 4)()
    lib().oracle_philox4x32(k, c, o)
    return list(o)


def env(graph: Graph, inputs: list) -> dict:
    """Every value of ``graph`` (inputs and each node's output) as NumPy values, keyed by value number: the
    oracle's view of each intermediate, for step-by-step comparisons."""
    import copy

    g2 = copy.copy(graph)
    g2.outputs = [n.output for n in graph.nodes]
    out = dict(zip(g2.outputs, values(g2, inputs)))
    for v, x in zip(graph.inputs, inputs):
        out[v] = D.to_numpy_values(np.asarray(x.raw() if hasattr(x, "raw") else x), graph.types[v].dtype)
    return out
