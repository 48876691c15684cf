"""Value-preserving frontend passes: ``cse`` (``lumen/graph_compiler/passes/cse.rs:16-69``) and ``simplify``
(a subset of ``passes/simplify.rs:603-701``: identities, layout compositions, and folding a narrowing cast
into the dot that feeds it, the dot then rounding once to ``output_dtype``).

Both rebuild the graph; a rewrite never changes any value (the pass tests check it with the oracle)."""

from __future__ import annotations

from lumen_amd import dtypes as D
from lumen_amd.graph.ir import ELEMENTWISE, Graph, InferError, TensorType, infer

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


_LAYOUT_MOVES = ("reshape", "transpose", "slice", "concatenate")


class _Builder:
    """The graph a rewrite pass builds: node of each new value, and whether a new value is read by one node
    only (values a rewrite creates for its own use are; a value standing for an original one is when that
    one was)."""

    def __init__(self, graph: Graph):
        self.g = Graph()
        self.node = {}
        self.once = {}
        self.remap = {v: self.g.input(graph.types[v].dtype, graph.types[v].shape) for v in graph.inputs}

    def add(self, prim, ins, params, backward=False, ty=None):
        if ty is None:
            ty = infer(prim, [self.g.types[v] for v in ins], params)
        v = self.g.add_node(prim, ins, params, ty, backward)
        self.node[v] = self.g.nodes[-1]
        return v

    def const(self, v):
        """The value a ``full`` (through broadcasts, reshapes and casts of it) fills ``v`` with, else None."""
        while v in self.node:
            n = self.node[v]
            if n.prim == "full":
                return float(n.params["fill_value"])
            if n.prim not in ("broadcast_in_dim", "reshape", "cast"):
                return None
            v = n.inputs[0]
        return None

    def producer(self, v, *prims):
        n = self.node.get(v)
        return n if n is not None and (not prims or n.prim in prims) else None


def _identity(b: _Builder, n, ins, t):
    """An existing value ``n`` equals (``x * 1``, ``x + 0``, ``x - 0``, ``x / 1``, ``-(-x)``, a select of one
    value, an update covering its whole operand, no-op casts and layouts), else None."""
    p = n.prim
    if p == "mul":
        if b.const(ins[1]) == 1.0:
            return ins[0]
        if b.const(ins[0]) == 1.0:
            return ins[1]
    if p == "div" and b.const(ins[1]) == 1.0:
        return ins[0]
    if p == "sub" and b.const(ins[1]) == 0.0:
        return ins[0]
    if p == "add":
        if b.const(ins[1]) == 0.0:
            return ins[0]
        if b.const(ins[0]) == 0.0:
            return ins[1]
    if p == "neg":
        inner = b.producer(ins[0], "neg")
        if inner is not None:
            return inner.inputs[0]
    if p == "select" and ins[1] == ins[2]:
        return ins[1]
    if p == "dynamic_update_slice" and b.g.types[ins[1]].shape == b.g.types[ins[0]].shape:
        return ins[1]  # its starts clamp to 0: the update overwrites all of the operand
    src = b.g.types[ins[0]] if ins else None
    if p in ("reshape", "transpose", "broadcast_in_dim", "cast", "host_wait", "device_wait") and src == t:
        if p != "transpose" or list(n.params["permutation"]) == sorted(n.params["permutation"]):
            return ins[0]
    return None


def _composed(b: _Builder, n, ins, t):
    """Consecutive layout ops as one (reshape of a reshape, transpose of a transpose, broadcast of a
    broadcast, a broadcast of a scalar constant as a constant), else None."""
    inner = b.producer(ins[0]) if ins else None
    if inner is None:
        return None
    if n.prim == "reshape" and inner.prim == "reshape":
        return b.add("reshape", inner.inputs, n.params, n.backward, t)
    if n.prim == "transpose" and inner.prim == "transpose":
        perm = tuple(inner.params["permutation"][d] for d in n.params["permutation"])
        if list(perm) == sorted(perm):
            return inner.inputs[0]
        return b.add("transpose", inner.inputs, {"permutation": perm}, n.backward, t)
    if n.prim == "broadcast_in_dim" and inner.prim == "full" and inner.params["shape"] == ():
        return b.add("full", (), dict(inner.params, shape=tuple(t.shape)), n.backward, t)
    if n.prim == "broadcast_in_dim" and inner.prim == "broadcast_in_dim":
        outer = n.params["broadcast_dimensions"]
        dims = tuple(outer[d] for d in inner.params["broadcast_dimensions"])
        params = {"shape": tuple(n.params["shape"]), "broadcast_dimensions": dims}
        try:
            infer("broadcast_in_dim", [b.g.types[inner.inputs[0]]], params)
        except InferError:
            return None
        return b.add("broadcast_in_dim", inner.inputs, params, n.backward, t)
    return None


def _dot_params(p, swap=False, lhs=None, rhs=None):
    q = dict(p)
    if swap:
        for a, c in (("lhs_contracting", "rhs_contracting"), ("lhs_batch", "rhs_batch")):
            q[a], q[c] = p[c], p[a]
    if lhs is not None:
        q["lhs_contracting"], q["lhs_batch"] = lhs
    if rhs is not None:
        q["rhs_contracting"], q["rhs_batch"] = rhs
    return q


def _swapped_dot(b: _Builder, n, ins, t):
    """``transpose(dot(x, y))`` whose permutation puts the rhs free axes before the lhs free ones, as
    ``dot(y, x)`` (the dot read by this transpose alone)."""
    d = b.producer(ins[0], "dot_general")
    if d is None or not b.once.get(ins[0]):
        return None
    p = d.params
    nb = len(p["lhs_batch"])
    fl = len(b.g.types[d.inputs[0]].shape) - nb - len(p["lhs_contracting"])
    fr = len(b.g.types[d.inputs[1]].shape) - nb - len(p["rhs_contracting"])
    want = tuple(range(nb)) + tuple(range(nb + fl, nb + fl + fr)) + tuple(range(nb, nb + fl))
    if tuple(n.params["permutation"]) != want:
        return None
    return b.add("dot_general", (d.inputs[1], d.inputs[0]), _dot_params(p, swap=True), n.backward, t)


def _folded_dot(b: _Builder, n, ins, t, graph_inputs):
    """A dot whose operand is a transpose (possibly under a cast) reads the transpose's input instead, its
    dimension numbers mapped through the permutation, when that keeps the operand's free axes in order.
    Before pattern matching only transposes of graph inputs fold (``graph_inputs`` is then a set)."""
    p = n.params
    sides = [(tuple(p["lhs_contracting"]), tuple(p["lhs_batch"])), (tuple(p["rhs_contracting"]), tuple(p["rhs_batch"]))]
    ops, changed = list(ins), False
    for side in (0, 1):
        cast = b.producer(ins[side], "cast")
        tv = cast.inputs[0] if cast is not None else ins[side]
        tr = b.producer(tv, "transpose")
        if tr is None or (graph_inputs is not None and tr.inputs[0] not in graph_inputs):
            continue
        perm = tr.params["permutation"]
        contracting, batch = sides[side]
        free = [perm[d] for d in range(len(perm)) if d not in contracting and d not in batch]
        if free != sorted(free):
            continue
        sides[side] = (tuple(perm[d] for d in contracting), tuple(perm[d] for d in batch))
        src = tr.inputs[0]
        ops[side] = b.add("cast", (src,), cast.params, n.backward) if cast is not None else src
        changed = True
    if not changed:
        return None
    return b.add("dot_general", tuple(ops), _dot_params(p, lhs=sides[0], rhs=sides[1]), n.backward, t)


def _moved(b: _Builder, n, ins, t):
    """Ops moved to the cheaper side of a rearrangement: an elementwise op whose operands are all the same
    reshape or transpose (of values read once) or constants runs before it; a widening cast of a layout
    op's operands runs after the layout op; a narrowing cast of a layout op's result runs before it. Values
    are unchanged: elementwise ops commute with rearrangements, and a cast with pure data movement."""
    p = n.prim
    if p in ELEMENTWISE and p != "cast":
        r = next((b.producer(v, "reshape", "transpose") for v in ins
                  if b.producer(v, "reshape", "transpose") is not None
                  and b.producer(b.producer(v).inputs[0], "full") is None), None)
        if r is None:
            return None
        shape = b.g.types[r.inputs[0]].shape
        before = []
        for v in ins:
            m = b.producer(v)
            if m is None:
                return None
            if m.prim == r.prim and m.params == r.params and b.g.types[m.inputs[0]].shape == shape and b.once.get(v):
                before.append(m.inputs[0])
            elif m.prim == "full":
                before.append(b.add("full", (), dict(m.params, shape=tuple(shape)), n.backward))
            else:
                return None
        x = b.add(p, tuple(before), n.params, n.backward)
        return b.add(r.prim, (x,), r.params, n.backward, t)
    if p in _LAYOUT_MOVES:
        casts = [b.producer(v, "cast") if b.once.get(v) else None for v in ins]
        c = next((c for c in casts if c is not None), None)
        if c is None:
            return None
        src, dst = b.g.types[c.inputs[0]].dtype, b.g.types[c.output].dtype
        if D.size_of(src) >= D.size_of(dst):
            return None
        if any(cc is None or b.g.types[cc.inputs[0]].dtype != src for cc in casts):
            return None
        x = b.add(p, tuple(cc.inputs[0] for cc in casts), n.params, n.backward)
        return b.add("cast", (x,), {"new_dtype": dst}, n.backward, t)
    if p == "cast":
        x = ins[0]
        lay = b.producer(x, *_LAYOUT_MOVES)
        if lay is None or not b.once.get(x) or D.size_of(b.g.types[x].dtype) <= D.size_of(n.params["new_dtype"]):
            return None
        cast_ins = tuple(b.add("cast", (u,), n.params, n.backward) for u in lay.inputs)
        return b.add(lay.prim, cast_ins, lay.params, n.backward, t)
    return None


def simplify(graph: Graph, matched: bool = False) -> Graph:
    """Value-preserving rewrites (``passes/simplify.rs:603-701``): identities and compositions of layout ops
    always; a narrowing cast that is a dot's only reader folded into the dot's ``output_dtype``; and, once
    pattern matching has run (``matched``), the structural ones — a transposed dot as the dot with swapped
    operands, operand transposes folded into a dot's dimension numbers, elementwise ops and casts moved
    across rearrangements. Before matching, only transposes of graph inputs fold into dots."""
    users = graph.users()
    prod = graph.producers()
    reads = {}
    for n in graph.nodes:
        for v in set(n.inputs):
            reads[v] = reads.get(v, 0) + 1
    for v in graph.outputs:
        reads[v] = reads.get(v, 0) + 1
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

    b = _Builder(graph)
    graph_inputs = None if matched else set(b.remap.values())
    for n in graph.nodes:
        ins = tuple(b.remap[v] for v in n.inputs)
        t = graph.types[n.output]
        b.g.backward = n.backward
        first = len(b.g.nodes)
        if n.prim == "dot_general" and n.output in folded:
            v = b.add("dot_general", ins, dict(n.params, output_dtype=folded[n.output]), n.backward,
                      TensorType(folded[n.output], t.shape))
        elif n.output in skip:
            v = ins[0]
        else:
            v = _identity(b, n, ins, t)
            if v is None:
                v = _composed(b, n, ins, t)
            if v is None and n.prim == "transpose" and matched:
                v = _swapped_dot(b, n, ins, t)
            if v is None and n.prim == "dot_general":
                v = _folded_dot(b, n, ins, t, graph_inputs)
            if v is None and matched:
                v = _moved(b, n, ins, t)
            if v is None:
                v = b.add(n.prim, ins, n.params, n.backward, t)
        for m in b.g.nodes[first:]:
            if m.output != v:
                b.once[m.output] = True
        fresh = v not in b.once
        b.once[v] = fresh and reads.get(n.output, 0) == 1
        b.remap[n.output] = v
    b.g.backward = False
    b.g.set_outputs([b.remap[v] for v in graph.outputs])
    b.g.prune()
    return b.g


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


def frontend(graph: Graph, matched: bool = False) -> Graph:
    """cse, then simplify (``graph_compiler/mod.rs:82-98``); ``matched``: pattern matching has run, so the
    structural rewrites are allowed."""
    return simplify(cse(graph), matched)
