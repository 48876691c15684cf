"""merge_dots: dots that share an operand and whose other operands are weights become one dot against the
weights packed into one block (``lumen/graph_compiler/passes/merge_dots/forward.rs:69-614``,
``backward.rs:310-330``).

* Forward: ``x . W_i^T`` for weights ``W_i`` [out_i, in] read by dots sharing ``x`` becomes one dot against
  ``concatenate(W_1, ..., W_k)`` [sum out_i, in], each member's result a slice of the merged one. The weights of
  a group form a *pack*: the plan asks its caller to store them back to back (``Plan.packs``), so the
  concatenation is a view of the first weight's memory and costs nothing.
* Backward: a sum of ``g_i . W_i`` over the weights of one pack (the input gradient of the projections)
  becomes one dot of ``concatenate(g_1, ..., g_k)`` against the packed block, and the weight gradients
  ``g_i^T . x`` become one dot sliced per weight.

The merged dot accumulates all of its k in one float32 sum, so results can differ from the unmerged graph by
float32 reassociation (as in the reference); every other value is unchanged.
"""

from __future__ import annotations

from lumen_amd.graph.ir import Graph, TensorType


class _Abandon(Exception):
    pass


def merge_dots(graph: Graph, packable: set) -> tuple[Graph, list]:
    """``(graph, packs)``: see the module docstring (the graph unchanged when a merge cannot be placed)."""
    try:
        return _merge_dots(graph, packable)
    except _Abandon:
        return graph, []


def _merge_dots(graph: Graph, packable: set) -> tuple[Graph, list]:
    """``(graph, packs)``: the rewritten graph and, per packed block, the graph-input positions of its weights
    in concatenation order. ``packable`` holds the input positions that are weights (parameters)."""
    types = graph.types
    pos = {v: i for i, v in enumerate(graph.inputs)}
    weights = {graph.inputs[i] for i in packable}
    users = graph.users()

    prod = graph.producers()

    def wref(v):
        """``(weight, transposed)`` when ``v`` is a rank-2 weight input or its transpose, else None."""
        if v in weights and len(types[v].shape) == 2:
            return v, False
        n = prod.get(v)
        if n is not None and n.prim == "transpose" and tuple(n.params["permutation"]) == (1, 0) and n.inputs[0] in weights:
            return n.inputs[0], True
        return None

    def contracted(n, side):
        """The dim of the weight (as stored) that dot ``n`` contracts on operand ``side``."""
        c = tuple(n.params["rhs_contracting" if side == 1 else "lhs_contracting"])
        if len(c) != 1:
            return None
        return (1 - c[0]) if wref(n.inputs[side])[1] else c[0]

    # ---- forward groups: dot(x, W_i) sharing x (lhs), each W_i contracted on its dim 1 (free dim 0 leading)
    groups: dict = {}
    for n in graph.nodes:
        if n.prim != "dot_general" or n.params["lhs_batch"] or n.params["rhs_batch"]:
            continue
        r = wref(n.inputs[1])
        if r is None or contracted(n, 1) != 1:
            continue
        p = n.params
        w = types[r[0]]
        key = (n.inputs[0], tuple(p["lhs_contracting"]), r[1], w.dtype, w.shape[1], p["accum_dtype"], p["output_dtype"])
        groups.setdefault(key, []).append(n)
    packs, pack_of = [], {}
    fwd = {}  # member output -> (group index, row offset)
    tr_of = {}  # pack -> whether its dots read the weights transposed
    for key, members in groups.items():
        ws = []
        for n in members:
            w = wref(n.inputs[1])[0]
            if w not in ws and w not in pack_of:
                ws.append(w)
        members = [n for n in members if wref(n.inputs[1])[0] in ws]
        if len(ws) < 2 or any(types[w].nbytes() % 256 for w in ws):
            continue
        k = len(packs)
        packs.append(tuple(pos[w] for w in ws))
        tr_of[k] = key[2]
        for w in ws:
            pack_of[w] = k
        off, offs = 0, {}
        for w in ws:
            offs[w] = off
            off += types[w].shape[0]
        for n in members:
            fwd[n.output] = (k, offs[wref(n.inputs[1])[0]])
    if not packs:
        return graph, []

    # ---- backward: add trees of dot(g_i, W_i) over a whole pack (dX), and dot(g_i, x) weight gradients
    def dx_leaf(v):
        """``(pack, weight)`` if ``v`` is a single-use dot(g, W) with W packed (read as in the pack's forward
        dots), contracting g's dim 1 with W's dim 0."""
        n = prod.get(v)
        if n is None or n.prim != "dot_general" or len(users.get(v, [])) != 1:
            return None
        r = wref(n.inputs[1])
        if r is None or r[0] not in pack_of or r[1] != tr_of[pack_of[r[0]]]:
            return None
        p = n.params
        if p["lhs_batch"] or p["rhs_batch"] or tuple(p["lhs_contracting"]) != (1,) or contracted(n, 1) != 0:
            return None
        if len(types[n.inputs[0]].shape) != 2:
            return None
        return pack_of[r[0]], r[0]

    add_roots = {}  # root add output -> (pack, {weight: cotangent}, dot params, other addends)
    inner = set()
    for n in graph.nodes:
        if n.prim != "add" or n.output in inner:
            continue
        leaves, others, stack, nodes_ = [], [], [n.output], []
        while stack:
            v = stack.pop()
            m = prod.get(v)
            if m is not None and m.prim == "add" and (v == n.output or len(users.get(v, [])) == 1):
                nodes_.append(v)
                stack.extend(m.inputs)
                continue
            leaf = dx_leaf(v)
            if leaf is None:
                others.append(v)
            else:
                leaves.append((leaf, prod[v]))
        if not leaves:
            continue
        k = leaves[0][0][0]
        ws = {w: dn for (kk, w), dn in leaves if kk == k}
        pack_ws = [graph.inputs[i] for i in packs[k]]
        if len(leaves) != len(pack_ws) or set(ws) != set(pack_ws):
            continue
        dts = {(dn.params["accum_dtype"], dn.params["output_dtype"]) for dn in ws.values()}
        if len(dts) != 1 or types[n.output].dtype != types[leaves[0][1].output].dtype:
            continue
        add_roots[n.output] = (k, {w: dn.inputs[0] for w, dn in ws.items()}, next(iter(ws.values())).params, others)
        inner.update(nodes_)

    # weight gradients: dot(g_i, x) contracting dim 0 of both, g_i the cotangents of a merged dX group
    dw = {}  # output -> (pack, row offset, merged-dot key)
    g_of = {}
    for k_root, (k, gmap, _, _) in add_roots.items():
        for w, gv in gmap.items():
            g_of[gv] = (k, w)
    dw_groups: dict = {}
    for n in graph.nodes:
        if n.prim != "dot_general" or n.inputs[0] not in g_of:
            continue
        p = n.params
        if p["lhs_batch"] or p["rhs_batch"] or tuple(p["lhs_contracting"]) != (0,) or tuple(p["rhs_contracting"]) != (0,):
            continue
        k, w = g_of[n.inputs[0]]
        dw_groups.setdefault((k, n.inputs[1], p["accum_dtype"], p["output_dtype"]), {})[w] = n
    gmaps = {k: gmap for (k, gmap, _, _) in add_roots.values()}
    for (k, x, _, _), byw in dw_groups.items():
        pack_ws = [graph.inputs[i] for i in packs[k]]
        if set(byw) != set(pack_ws):
            continue
        off = 0
        for w in pack_ws:
            dw[byw[w].output] = (k, off, (k, x))
            off += types[w].shape[0]

    # ---- rebuild
    out = Graph()
    remap = {}
    for v in graph.inputs:
        remap[v] = out.input(types[v].dtype, types[v].shape)
    blocks = {}    # pack -> concatenated weight block (transposed when its dots read the weights so)

    def block(k):
        if k not in blocks:
            b = _concat(out, [remap[graph.inputs[i]] for i in packs[k]], 0)
            if tr_of[k]:
                t = out.types[b]
                b = out.add_node("transpose", (b,), {"permutation": (1, 0)}, TensorType(t.dtype, t.shape[::-1]),
                                 out.backward)
            blocks[k] = b
        return blocks[k]

    merged = {}    # (pack, x) -> merged forward dot
    gcat = {}      # pack -> concatenated cotangents
    dwm = {}       # (pack, x) -> merged weight-gradient dot
    def ensure(v, depth=0):
        """Emits ``v``'s producers ahead of their place when a merged dot needs them early (the cotangents of a
        weight-gradient group are reshaped right before each one's use)."""
        if v in remap:
            return True
        m = prod.get(v)
        if m is None or depth > 8 or m.prim in ("dot_general", "fusion") or v in fwd or v in add_roots or v in dw:
            return False
        if not all(ensure(u, depth + 1) for u in m.inputs):
            return False
        out.backward = m.backward
        remap[v] = out.add_node(m.prim, tuple(remap[u] for u in m.inputs), m.params, types[v], m.backward)
        return True

    for n in graph.nodes:
        out.backward = n.backward
        v = n.output
        if v in remap:
            continue  # emitted early by ensure()
        if v in fwd:
            k, off = fwd[v]
            x = remap[n.inputs[0]]
            if (k, x) not in merged:
                merged[(k, x)] = _dot(out, x, block(k), n.params)
            remap[v] = _slice(out, merged[(k, x)], 1, off, types[v].shape[1])
            continue
        if v in add_roots:
            k, gmap, params, others = add_roots[v]
            if k not in gcat:
                gcat[k] = _concat(out, [remap[gmap[graph.inputs[i]]] for i in packs[k]], 1)
            acc = _dot(out, gcat[k], block(k), params)
            for o in others:
                acc = out.add_node("add", (remap[o], acc), {}, types[v], n.backward)
            remap[v] = acc
            continue
        if v in dw:
            k, off, key = dw[v]
            if not all(ensure(gmaps[k][graph.inputs[i]]) for i in packs[k]) or not ensure(key[1]):
                raise _Abandon()
            if k not in gcat:
                gcat[k] = _concat(out, [remap[gmaps[k][graph.inputs[i]]] for i in packs[k]], 1)
            if key not in dwm:
                dwm[key] = _dot(out, gcat[k], remap[key[1]], n.params)
            remap[v] = _slice(out, dwm[key], 0, off, types[v].shape[0])
            continue
        if any(u not in remap for u in n.inputs):
            continue  # interior of a merged add tree
        remap[v] = out.add_node(n.prim, tuple(remap[u] for u in n.inputs), n.params, types[v], n.backward)
    out.backward = False
    out.set_outputs([remap[v] for v in graph.outputs])
    out.prune()
    return out, packs


def _concat(g, vals, dim):
    ts = [g.types[v] for v in vals]
    shape = list(ts[0].shape)
    shape[dim] = sum(t.shape[dim] for t in ts)
    return g.add_node("concatenate", tuple(vals), {"dimension": dim}, TensorType(ts[0].dtype, tuple(shape)), g.backward)


def _dot(g, a, b, params):
    p = dict(params)
    ta, tb = g.types[a], g.types[b]
    lf = [d for d in range(len(ta.shape)) if d not in p["lhs_contracting"]]
    rf = [d for d in range(len(tb.shape)) if d not in p["rhs_contracting"]]
    shape = tuple(ta.shape[d] for d in lf) + tuple(tb.shape[d] for d in rf)
    return g.add_node("dot_general", (a, b), p, TensorType(p["output_dtype"], shape), g.backward)


def _slice(g, v, dim, start, size):
    t = g.types[v]
    st = [0] * len(t.shape)
    li = list(t.shape)
    st[dim], li[dim] = start, start + size
    shape = list(t.shape)
    shape[dim] = size
    return g.add_node("slice", (v,), {"start_indices": tuple(st), "limit_indices": tuple(li)},
                      TensorType(t.dtype, tuple(shape)), g.backward)
