"""Value-preserving frontend passes: ``cse`` (``lumen/graph_compiler/passes/cse.rs:16-69``) and ``simplify``
(a subset of ``passes/simplify.rs:603-701``: identities, layout compositions, and folding a narrowing cast
into the dot that feeds it, the dot then rounding once to ``output_dtype``).

Both rebuild the graph; a rewrite never changes any value (the pass tests check it with the oracle)."""

from __future__ import annotations

from lumen_amd.graph.ir import Graph, TensorType

COMMUTATIVE = {"add", "mul", "max", "eq", "min", "and", "or", "xor"}


def _rebuild(graph: Graph, rewrite) -> Graph:
    """A new graph with each node passed through ``rewrite(g, node, ins) -> var`` (``ins`` remapped)."""
    g = Graph()
    remap = {}
    for v in graph.inputs:
        remap[v] = g.input(graph.types[v].dtype, graph.types[v].shape)
    for n in graph.nodes:
        ins = tuple(remap[v] for v in n.inputs)
        g.backward = n.backward
        remap[n.output] = rewrite(g, n, ins)
    g.backward = False
    g.set_outputs([remap[v] for v in graph.outputs])
    return g


def cse(graph: Graph) -> Graph:
    """Merges nodes applying one primitive with equal parameters to the same operands."""
    seen = {}

    def rewrite(g, n, ins):
        if n.prim in COMMUTATIVE:
            ins = tuple(sorted(ins))
        if n.prim in ("fusion", "fusion_output", "random_bits"):
            return g.add_node(n.prim, ins, n.params, graph.types[n.output], n.backward)
        key = (n.key(), ins)
        if key in seen:
            return seen[key]
        v = g.add_node(n.prim, ins, n.params, graph.types[n.output], n.backward)
        seen[key] = v
        return v

    return _rebuild(graph, rewrite)


def simplify(graph: Graph) -> Graph:
    """Identities and layout compositions; a narrowing cast folded into its only producer dot."""
    users = graph.users()
    prod = graph.producers()
    # casts that fold into their dot: the dot's only use is this cast, to a dtype it may output
    folded = {}
    for n in graph.nodes:
        if n.prim != "cast":
            continue
        p = prod.get(n.inputs[0])
        if p is None or p.prim != "dot_general" or len(users.get(p.output, [])) != 1 or p.output in graph.outputs:
            continue
        new = n.params["new_dtype"]
        ops = [graph.types[v].dtype for v in p.inputs]
        if p.params["output_dtype"] == p.params["accum_dtype"] and new in ops and new != p.params["accum_dtype"]:
            folded[p.output] = new
    skip = {n.output for n in graph.nodes if n.prim == "cast" and n.inputs[0] in folded}

    def rewrite(g, n, ins):
        t = graph.types[n.output]
        if n.prim == "dot_general" and n.output in folded:
            params = dict(n.params, output_dtype=folded[n.output])
            return g.add_node("dot_general", ins, params, TensorType(folded[n.output], t.shape), n.backward)
        if n.output in skip:
            return ins[0]
        src = g.types[ins[0]] if ins else None
        if n.prim in ("reshape", "transpose", "broadcast_in_dim", "cast", "host_wait", "device_wait") and src == t:
            if n.prim != "transpose" or list(n.params["permutation"]) == sorted(n.params["permutation"]):
                return ins[0]
        gp = {m.output: m for m in g.nodes}
        inner = gp.get(ins[0]) if ins else None
        if n.prim == "reshape" and inner is not None and inner.prim == "reshape":
            return g.add_node("reshape", inner.inputs, n.params, t, n.backward)
        if n.prim == "transpose" and inner is not None and inner.prim == "transpose":
            p1, p2 = inner.params["permutation"], n.params["permutation"]
            perm = tuple(p1[d] for d in p2)
            if list(perm) == sorted(perm):
                return inner.inputs[0]
            return g.add_node("transpose", inner.inputs, {"permutation": perm}, t, n.backward)
        if n.prim == "broadcast_in_dim" and inner is not None and inner.prim == "full" and inner.params["shape"] == ():
            return g.add_node("full", (), dict(inner.params, shape=tuple(t.shape)), t, n.backward)
        return g.add_node(n.prim, ins, n.params, t, n.backward)

    out = _rebuild(graph, rewrite)
    out.prune()
    return out


def frontend(graph: Graph) -> Graph:
    """cse, then simplify (``graph_compiler/mod.rs:82-98``)."""
    return simplify(cse(graph))
