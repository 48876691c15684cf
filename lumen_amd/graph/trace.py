"""Tracing a Python function into a graph (``lumen/graph/tracer.py:371-500`` ``_trace``, ``:1144``
``make_graph``): tensor arguments and module weights become graph inputs, Python floats runtime float64
scalars (weakly typed, ``_scalar_dtype``), and weights the function assigns (``copy_``) extra outputs."""

from __future__ import annotations

from dataclasses import dataclass, field

from lumen_amd import nn
from lumen_amd.graph.ir import Graph
from lumen_amd.graph.tracer import TracedTensor, tracing
from lumen_amd.tensor import Tensor


@dataclass
class Traced:
    """A traced function: its graph, what it returned, and how the graph's inputs and outputs map back."""

    graph: Graph
    out: object                      # the returned structure, traced tensors as leaves
    layout: list                     # per graph input: ("arg", k) | ("scalar", k) | ("weight", k)
    weights: list                    # the weight tensors in input order
    written: list = field(default_factory=list)   # weight indices whose new values are extra outputs
    n_returned: int = 0
    static_writes: list = field(default_factory=list)  # (arg index, path, value) static scalars assigned


def tree_leaves(x):
    if isinstance(x, (TracedTensor, Tensor)):
        return [x]
    if isinstance(x, nn.Module):
        return [t for _, t in nn._leaves(x, "")]
    if isinstance(x, (list, tuple)):
        out = []
        for v in x:
            out += tree_leaves(v)
        return out
    if isinstance(x, dict):
        out = []
        for v in x.values():
            out += tree_leaves(v)
        return out
    return []


def tree_map(f, x):
    if isinstance(x, (TracedTensor, Tensor)):
        return f(x)
    if isinstance(x, (list, tuple)):
        return type(x)(tree_map(f, v) for v in x)
    if isinstance(x, dict):
        return {k: tree_map(f, v) for k, v in x.items()}
    return x


def weights_of(args):
    """Each module weight among ``args``, once, in field order (``tracer.py:236``)."""
    seen, out = set(), []

    def visit(x, in_module):
        if isinstance(x, Tensor):
            if in_module and id(x) not in seen:
                if not x._is_parameter:
                    raise TypeError(
                        f"a module's weights must be whole meta tensors, got a {x.device} tensor of shape {list(x.shape)}"
                    )
                seen.add(id(x))
                out.append(x)
        elif isinstance(x, nn.Module):
            import dataclasses

            for f in dataclasses.fields(x):
                visit(getattr(x, f.name), True)
        elif isinstance(x, (list, tuple)):
            for v in x:
                visit(v, in_module)

    for a in args:
        visit(a, False)
    return out


def trace(fn, args) -> Traced:
    graph = Graph()
    layout, k_arg = [], 0
    traced_args = []
    for a in args:
        if isinstance(a, Tensor):
            t = TracedTensor(graph, graph.input(a.dtype, a.shape))
            layout.append(("arg", k_arg))
            k_arg += 1
            traced_args.append(t)
        else:
            traced_args.append(a)
    # Top-level floats and module float fields are runtime scalars: float64 0-d inputs, weakly typed.
    scalars = {}
    k_scalar = 0

    def scalar(i, path, v):
        nonlocal k_scalar
        if not isinstance(v, float):
            return v
        t = TracedTensor(graph, graph.input("float64", ()))
        t.weak = True
        layout.append(("scalar", k_scalar))
        scalars[(i, path)] = v
        k_scalar += 1
        return t

    for i, a in enumerate(traced_args):
        if isinstance(a, float):
            traced_args[i] = scalar(i, (), a)
    # graph inputs in the reference's order: tensor arguments, runtime scalars, weights (tracer.py:371-500)
    created = {}
    for i, a in enumerate(traced_args):
        if isinstance(a, (nn.Module, list, tuple)):
            nn.map_tensors(a, lambda t: t, lambda path, v, i=i: created.setdefault((i, path), scalar(i, path, v)))
    weights = weights_of(args)
    winputs = {}
    for k, w in enumerate(weights):
        winputs[id(w)] = TracedTensor(graph, graph.input(w.dtype, w.shape))
        layout.append(("weight", k))
    mapped = [
        nn.map_tensors(a, lambda t: winputs.get(id(t), t), lambda path, v, i=i: created.get((i, path), v))
        if isinstance(a, (nn.Module, list, tuple))
        else a
        for i, a in enumerate(traced_args)
    ]
    leaves = [t for t in mapped if isinstance(t, TracedTensor) and not t.weak] + list(winputs.values())
    original = {id(w): winputs[id(w)].var for w in weights}
    with tracing(graph, leaves=leaves):
        out = fn(*mapped)
        # static scalars (ints, bools) the function assigned in a module: written back after each call
        static_writes = []
        for i, (a, m) in enumerate(zip(args, mapped)):
            if isinstance(a, nn.Module):
                for path in _int_paths(a):
                    now = nn.at(m, path)
                    if now != nn.at(a, path):
                        if isinstance(now, TracedTensor):
                            raise TypeError("an int field is static: it cannot be assigned a traced value")
                        static_writes.append((i, path, now))
    outs = tree_leaves(out)
    if not isinstance(out, (TracedTensor, list, tuple, dict)) or any(o.graph is not graph for o in outs):
        raise TypeError(f"a compiled function must return tensors computed from its inputs, got {out!r}")
    written = [k for k, w in enumerate(weights) if winputs[id(w)].var != original[id(w)]]
    graph.set_outputs([o.var for o in outs] + [winputs[id(weights[k])].var for k in written])
    graph.prune_map = graph.prune()
    return Traced(graph, out, layout, weights, written, len(outs), static_writes)


def _int_paths(x, path=()):
    import dataclasses

    if isinstance(x, nn.Module):
        for f in dataclasses.fields(x):
            v = getattr(x, f.name)
            if type(v) in (int, bool):
                yield (*path, f.name)
            elif isinstance(v, (nn.Module,)):
                yield from _int_paths(v, (*path, f.name))


def make_graph(fn):
    """A function returning ``fn``'s traced graph on given arguments (``tracer.py:1144``)."""

    def graph(*args):
        return trace(fn, args).graph

    return graph
