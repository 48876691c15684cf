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


def _match_linear_cross_entropy(graph: Graph, dot, users, prod):
    """For a dot computing float32 logits h [b, d] . w^T that only a cross entropy reads (its max-shifted
    log-sum-exp over the classes and the gather of the target logits), ``(h, w [v, d], target [b], lse, loss)``;
    else None. The pattern and its conditions follow ``passes/linear_cross_entropy.rs:1-22``."""
    p = dot.params
    if p["lhs_batch"] or p["rhs_batch"] or p["accum_dtype"] != "float32" or p["output_dtype"] != "float32":
        return None
    lt, rt = graph.types[dot.inputs[0]], graph.types[dot.inputs[1]]
    if len(lt.shape) != 2 or len(rt.shape) != 2 or tuple(p["lhs_contracting"]) != (1,):
        return None
    if tuple(p["rhs_contracting"]) == (1,):
        w = dot.inputs[1]                                  # [v, d]
    elif tuple(p["rhs_contracting"]) == (0,):              # [d, v]: a transpose of the [v, d] weight
        t = prod.get(dot.inputs[1])
        if t is None or t.prim != "transpose" or tuple(t.params["permutation"]) != (1, 0):
            return None
        w = t.inputs[0]
    else:
        return None
    if graph.types[w].dtype != lt.dtype or lt.dtype not in ("float32", "bfloat16", "float16"):
        return None
    h = dot.inputs[0]
    if h in prod and prod[h].prim in ("transpose", "slice", "broadcast_in_dim"):
        return None                                        # the fused kernel reads row-major h
    logits = dot.output
    b, v = graph.types[logits].shape

    def one(var, prim=None):
        us = users.get(var, [])
        if len(us) != 1 or var in graph.outputs or (prim and us[0].prim != prim):
            return None
        return us[0]

    by = {}
    for u in users.get(logits, []):
        by.setdefault(u.prim, []).append(u)
    if logits in graph.outputs or sorted(by) != ["reduce_max", "reshape", "sub"] or any(len(x) != 1 for x in by.values()):
        return None
    mx, shift, flat = by["reduce_max"][0], by["sub"][0], by["reshape"][0]
    if tuple(mx.params["axes"]) != (1,) or shift.inputs[0] != logits or tuple(flat.params["new_sizes"]) != (b * v,):
        return None
    bc = prod.get(shift.inputs[1])
    if bc is None or bc.prim != "broadcast_in_dim" or one(bc.output) is not shift:
        return None
    keep = prod.get(bc.inputs[0])
    if keep is None or keep.prim != "reshape" or keep.inputs[0] != mx.output or one(keep.output) is not bc:
        return None
    e = one(shift.output, "exp")
    z = e and one(e.output, "reduce_sum")
    if z is None or tuple(z.params["axes"]) != (1,) or z.params.get("accum_dtype", "float32") != "float32":
        return None
    lg = one(z.output, "log")
    lse = lg and one(lg.output, "add")
    if lse is None:
        return None
    row_max = lse.inputs[0] if lse.inputs[1] == lg.output else lse.inputs[1]
    if row_max != mx.output:  # the row max reaches the add directly or through a reshape to [b]
        rm = prod.get(row_max)
        if rm is None or rm.prim != "reshape" or rm.inputs[0] != mx.output or one(rm.output) is not lse:
            return None
    if sorted(u.output for u in users.get(mx.output, [])) != sorted([keep.output, lse.output if row_max == mx.output
                                                                       else row_max]):
        return None
    pick = one(flat.output, "gather")
    if pick is None or pick.params.get("axis", 0) != 0 or pick.inputs[0] != flat.output:
        return None
    idx = prod.get(pick.inputs[1])
    if idx is None or idx.prim != "add":
        return None
    target = None
    for a, c in ((idx.inputs[0], idx.inputs[1]), (idx.inputs[1], idx.inputs[0])):
        m = prod.get(c)
        if m is None or m.prim != "mul":
            continue
        kinds = sorted(prod[x].prim if x in prod else "input" for x in m.inputs)
        if kinds != ["full", "iota"]:
            continue
        f = next(prod[x] for x in m.inputs if prod[x].prim == "full")
        io = next(prod[x] for x in m.inputs if prod[x].prim == "iota")
        if f.params["fill_value"] == v and io.params.get("dimension", 0) == 0:
            target = a
    if target is None or graph.types[target].dtype not in ("int32", "int64") or graph.types[target].shape != (b,):
        return None
    loss = one(pick.output, "sub")
    if loss is None or loss.inputs != (lse.output, pick.output):
        return None
    return h, w, target, lse.output, loss.output


def linear_cross_entropy(graph: Graph) -> Graph:
    """A cross entropy over logits h . w^T that nothing else reads becomes one ``linear_cross_entropy`` node
    (``passes/linear_cross_entropy.rs``, on by default like ``fused_linear_cross_entropy``): its [2, b] result's
    rows replace the loss and the log-sum-exp, and the [b, v] logits are never materialized. A training step
    does not match: the backward reads the logits."""
    users, prod = graph.users(), graph.producers()
    found = {}
    for n in graph.nodes:
        if n.prim == "dot_general":
            m = _match_linear_cross_entropy(graph, n, users, prod)
            if m is not None:
                found[m[3]] = m
                found[m[4]] = m
    if not found:
        return graph
    emitted = {}

    g = Graph()
    remap = {}
    for v in graph.inputs:
        remap[v] = g.input(graph.types[v].dtype, graph.types[v].shape)
    for n in graph.nodes:
        ins = tuple(remap[v] for v in n.inputs)
        g.backward = n.backward
        m = found.get(n.output)
        if m is None:
            remap[n.output] = g.add_node(n.prim, ins, n.params, graph.types[n.output], n.backward)
            continue
        h, w, target, lse, loss = m
        b = graph.types[h].shape[0]
        if id(m) not in emitted:  # at the first of the two results, where h, w and the targets all exist
            emitted[id(m)] = g.add_node("linear_cross_entropy", (remap[h], remap[w], remap[target]), {},
                                        TensorType("float32", (2, b)), n.backward)
        row = 1 if n.output == lse else 0
        sl = g.add_node("slice", (emitted[id(m)],), {"start_indices": (row, 0), "limit_indices": (row + 1, b)},
                        TensorType("float32", (1, b)), n.backward)
        remap[n.output] = g.add_node("reshape", (sl,), {"new_sizes": (b,)}, TensorType("float32", (b,)), n.backward)
    g.backward = False
    g.set_outputs([remap[v] for v in graph.outputs])
    g.prune()
    return g


def frontend(graph: Graph) -> Graph:
    """cse, then simplify (``graph_compiler/mod.rs:82-98``)."""
    return simplify(cse(graph))
