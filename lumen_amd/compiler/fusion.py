"""Loop fusion: groups a graph's nodes into the steps of a plan (``lumen/graph_compiler/passes/fusion/mod.rs``,
``passes/diamonds.rs``, ``passes/alone.rs``).

Nodes are visited in reverse topological order. A dot, a flash-attention fusion or a scatter-add is a step
of its own (a built-in kernel). Every other node is fusible: it joins the loop kernel of its consumers when
all of them are in one kernel, so its value never reaches memory. A value with consumers in several kernels
is computed once (it gets a kernel, or becomes an extra output of the kernel it is in) unless it is index
math alone (``full``, ``iota``, layout ops of a kernel input), which each kernel recomputes.

A loop kernel with reductions is a row kernel: every reduction sums (or maxes) the trailing axes of one row
space ``R x C`` (a normalization diamond: softmax, layer norm, RMS norm, cross entropy's log-sum-exp), its
results flowing back to the rows only through size-1 reshapes and broadcasts of the trailing axes. Any
other reduction is a reduce step of its own.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

from lumen_amd.graph.ir import ELEMENTWISE, Graph

LAYOUT = {"reshape", "broadcast_in_dim", "transpose", "slice", "concatenate", "swap_pairs"}
VIEWABLE = {"reshape", "broadcast_in_dim", "transpose", "slice"}
INDEX_ONLY = {"full", "iota"}
FUSIBLE = ELEMENTWISE | LAYOUT | INDEX_ONLY | {"gather", "take_along_axis", "reduce_sum", "reduce_max",
                                               "dynamic_slice", "host_wait", "device_wait"}
# Built-in kernels: each node is a step of its own.
OWN_STEP = {"dot_general", "fusion", "scatter_add", "cumsum", "random_bits", "linear_cross_entropy",
            "dynamic_update_slice"}


@dataclass
class Step:
    """One launch (or view) of the plan."""

    kind: str                       # "loop", "row", "reduce", "dot", "flash_fwd", "flash_bwd", "scatter_add", "copy"
    nodes: list = field(default_factory=list)    # graph nodes computed, topological order
    outputs: list = field(default_factory=list)  # values this step writes to memory
    inputs: list = field(default_factory=list)   # values it reads from memory
    rows: tuple | None = None       # (R, C) of a row kernel
    name: str = ""
    scratch: int = 0                # bytes of workspace the step needs while it runs
    mode: int | None = None         # flash_bwd: the dQ mode (nhip_attn_desc.deterministic)

    def label(self):
        return " → ".join(n.prim for n in self.nodes[:6]) + (" → …" if len(self.nodes) > 6 else "")


def row_broadcast(src, out, dims, rows) -> bool:
    """Whether broadcasting ``src`` (numel R) to ``out`` (numel R x C) along ``dims`` repeats each row's
    value over that row's C elements of the row space ``rows`` = (R, C): the output's leading axes spanning R
    each come from a source axis of the same size (in order), and every other source axis has size 1."""
    R, C = rows
    if src.numel() != R or out.numel() != R * C:
        return False
    k = 0
    while k < len(out.shape) and math.prod(out.shape[:k]) < R:
        k += 1
    if math.prod(out.shape[:k]) != R:
        return False
    covered = set()
    for i, d in enumerate(dims):
        if d < k:
            if src.shape[i] != out.shape[d]:
                return False
            covered.add(d)
        elif src.shape[i] != 1:
            return False
    return all(out.shape[d] == 1 for d in range(k) if d not in covered)


def row_reads_ok(graph, nodes, rows) -> bool:
    """Whether a row kernel of ``nodes`` over ``rows`` reads every row statistic (its reductions and values
    computed from them alone) at its own row. The kernel holds a statistic for the current row only, so a
    statistic that reaches the elements through anything but a row broadcast (a transposed broadcast of a
    log-sum-exp, say) cannot be computed there."""
    if rows is None:
        return True
    R = rows[0]
    users = {}
    for m in nodes:
        for u in m.inputs:
            users.setdefault(u, []).append(m)
    stack = [m.output for m in nodes if m.prim in ("reduce_sum", "reduce_max")]
    seen = set(stack)
    while stack:
        v = stack.pop()
        for c in users.get(v, []):
            t = graph.types[c.output]
            if c.prim == "broadcast_in_dim" and t.numel() != R:
                if not row_broadcast(graph.types[v], t, c.params["broadcast_dimensions"], rows):
                    return False
                continue
            if t.numel() != R or not (c.prim in ("reshape", "broadcast_in_dim") or c.prim in ELEMENTWISE):
                return False
            if c.output not in seen:
                seen.add(c.output)
                stack.append(c.output)
    return True


def _row_space(graph, n):
    """``(R, C)`` of a reduction over trailing axes, or None."""
    x = graph.types[n.inputs[0]]
    axes = tuple(n.params["axes"])
    r = len(x.shape)
    if not axes or axes != tuple(range(r - len(axes), r)):
        return None
    c = math.prod(x.shape[r - len(axes):])
    return (math.prod(x.shape[: r - len(axes)]), c)


def fuse(graph: Graph, fuse_loops=True, packed=frozenset()) -> list:
    """The steps computing ``graph``'s outputs, in an order respecting dependencies. ``packed`` holds
    concatenations that are views (weights stored back to back)."""
    users = graph.users()
    prod = graph.producers()
    order = {n.output: i for i, n in enumerate(graph.nodes)}
    for i, v in enumerate(graph.inputs):
        order[v] = -1 - i
    is_input = set(graph.inputs)
    must = set(graph.outputs)
    views = set()
    # Operands of built-in steps live in memory; a layout op there is a strided view when it can be one.
    for n in graph.nodes:
        if n.prim in OWN_STEP:
            for j, u in enumerate(n.inputs):
                if n.prim == "scatter_add" and j == 0 and u in prod and prod[u].prim == "full":
                    continue
                while u in prod and (prod[u].prim in VIEWABLE or u in packed) and u not in graph.outputs:
                    views.add(u)
                    u = prod[u].inputs[0]
                must.add(u)
    for v in views:  # a view's base is in memory (or is itself a view of memory)
        for u in (prod[v].inputs if v in packed else prod[v].inputs[:1]):
            if u not in views:
                must.add(u)
    kernel_of: dict[int, int] = {}
    members: list[set] = []
    kinds: list[str] = []
    rows: list = []
    roots: list[list] = []

    def cheap(v):
        n = prod.get(v)
        if n is None:
            return True
        if n.prim in INDEX_ONLY:
            return True
        if n.prim in ("reshape", "broadcast_in_dim", "transpose", "slice"):
            return all(cheap(u) for u in n.inputs)
        return False

    def depends(v, target, memo):
        """Whether ``v`` transitively depends on ``target`` (pruned by topological order)."""
        if v == target:
            return True
        if order.get(v, -1) <= order.get(target, -1):
            return False
        if v in memo:
            return memo[v]
        n = prod.get(v)
        r = n is not None and any(depends(u, target, memo) for u in n.inputs)
        memo[v] = r
        return r

    extra_outs = {}
    for n in graph.nodes:
        if n.prim == "fusion_output":
            extra_outs.setdefault(n.inputs[0], []).append(n.output)
    for n in reversed(graph.nodes):
        v = n.output
        if v in kernel_of or n.prim == "fusion_output":
            continue
        if cheap(v) and v not in must and v not in views:
            continue
        if v in views and v not in must:
            k = len(members)
            members.append({v})
            kinds.append("view")
            rows.append(None)
            roots.append([v])
            kernel_of[v] = k
            continue
        if n.prim in OWN_STEP or n.prim not in FUSIBLE or not fuse_loops:
            k = len(members)
            members.append({v})
            kinds.append("own")
            rows.append(None)
            roots.append([v] + extra_outs.get(v, []))
            kernel_of[v] = k
            for x in extra_outs.get(v, []):
                kernel_of[x] = k
            continue
        k = len(members)
        mem = {v}
        members.append(mem)
        kinds.append("loop")
        rows.append(None)
        roots.append([v])
        kernel_of[v] = k
        if n.prim in ("reduce_sum", "reduce_max"):
            rs = _row_space(graph, n)
            if rs is not None:
                rows[k] = rs
            else:
                kinds[k] = "reduce"
                continue
        frontier = list(n.inputs)
        while frontier:
            frontier.sort(key=lambda u: -order.get(u, -1))
            u = frontier.pop(0)
            if u in is_input or u in mem or u in views:
                continue
            p = prod[u]
            if p.prim not in FUSIBLE or p.prim in OWN_STEP:
                continue
            if cheap(u) and u not in must:
                mem.add(u)
                frontier.extend(p.inputs)
                continue
            if u in kernel_of:
                continue
            outside = {c.output for c in users.get(u, []) if c.output not in mem}
            if p.prim in ("reduce_sum", "reduce_max"):
                rs = _row_space(graph, p)
                if rs is None or (rows[k] is not None and rows[k] != rs):
                    continue
                if not all(graph.types[r].numel() in (rs[0] * rs[1], rs[0]) for r in roots[k]):
                    continue
                if not row_reads_ok(graph, [m for m in graph.nodes if m.output in mem or m.output == u], rs):
                    continue
            if outside or u in must:
                if not _fits(graph, u, roots[k], rows[k] if p.prim not in ("reduce_sum", "reduce_max") else _row_space(graph, p)):
                    continue
                # computing u here must not make this kernel wait for a kernel that reads u: no member may
                # depend on anything another reader's kernel writes
                targets = set()
                for c in outside:
                    kc = kernel_of.get(c)
                    targets.update(roots[kc] if kc is not None else [c])
                cyc = False
                for tv in targets:
                    memo = {}
                    if any(depends(m, tv, memo) for m in mem):
                        cyc = True
                        break
                if cyc:
                    continue
                roots[k].append(u)
                must.add(u)
            mem.add(u)
            kernel_of[u] = k
            if p.prim in ("reduce_sum", "reduce_max"):
                rows[k] = _row_space(graph, p)
            frontier.extend(p.inputs)
    steps = []
    for k, mem in enumerate(members):
        nodes = [m for m in graph.nodes if m.output in mem]
        outs = list(roots[k])
        if kinds[k] == "own":
            node = nodes[0]
            kind = {"dot_general": "dot"}.get(node.prim, node.prim)
            if node.prim == "fusion":
                kind = {"flash_attention": "flash_fwd", "flash_attention_backward": "flash_bwd"}[node.params["name"]]
            st = Step(kind, nodes, outs)
            if kind in ("flash_fwd", "flash_bwd"):
                q = graph.types[node.inputs[0]]
                if kind == "flash_bwd":
                    from lumen_amd.compiler.attention import backward_mode, backward_workspace_bytes

                    b, sq, nh, hd = q.shape
                    sk, kvh = graph.types[node.inputs[1]].shape[1:3]
                    st.mode = backward_mode(b, nh, sq, sk)
                    hdv = graph.types[node.inputs[2]].shape[3]
                    st.scratch = backward_workspace_bytes(b, nh, sq, sk, hd, kvh, st.mode, hdv)
                elif len(outs) == 1:
                    st.scratch = graph.types[outs[0]].numel() // graph.types[outs[0]].shape[-1] * 4
        elif kinds[k] in ("view", "reduce"):
            st = Step(kinds[k], nodes, outs)
        else:
            st = Step("row" if rows[k] is not None else "loop", nodes, outs, rows=rows[k])
        produced = {m.output for m in nodes}
        ins = []
        for m in nodes:
            for u in m.inputs:
                if u not in produced and u not in ins:
                    ins.append(u)
        if st.kind == "scatter_add" and nodes[0].inputs[0] in prod and prod[nodes[0].inputs[0]].prim == "full":
            ins = [u for u in ins if u != nodes[0].inputs[0]]
        st.inputs = ins
        steps.append(st)
    for st in steps:
        if st.kind in ("loop", "row"):
            _pull_index_math(graph, st, prod, done_inputs=set(graph.inputs))
    if fuse_loops:
        steps = _rematerialize(graph, steps, prod)
    done, ordered = set(graph.inputs), []
    pending = steps[:]
    while pending:
        progressed = False
        for st in list(pending):
            if all(u in done for u in st.inputs):
                ordered.append(st)
                done.update(st.outputs)
                pending.remove(st)
                progressed = True
        if not progressed:
            raise RuntimeError("fusion produced a cycle: " + ", ".join(s.label() for s in pending))
    return ordered


REMAT = ELEMENTWISE | INDEX_ONLY | VIEWABLE
REMAT_BUDGET = 32  # nodes a kernel may recompute in place of one value it reads
REMAT_SMALL = 1 << 20  # operand bytes a recomputation may add regardless (per-row statistics)


def _inputs_of(nodes):
    produced = {m.output for m in nodes}
    ins = []
    for m in nodes:
        for u in m.inputs:
            if u not in produced and u not in ins:
                ins.append(u)
    return ins


def _rematerialize(graph, steps, prod):
    """Recomputes values instead of storing them (``passes/fusion/mod.rs`` duplicates cheap producers the
    same way). A loop or row kernel that reads a value computed elementwise from values already in memory
    computes it itself from the nearest stored ones, when the new operands it reads hold at most the replaced
    value's bytes (or at most 1 MiB): the training graph's backward kernels then recompute an activation's
    intermediates (GELU's tanh argument and friends) from its input instead of reading them back, read a norm's
    per-row statistic instead of its broadcast over the row, and the forward kernels stop writing them."""
    in_memory = set(graph.inputs)
    for st in steps:
        in_memory.update(st.outputs)
    for st in steps:
        if st.kind not in ("loop", "row"):
            continue
        changed = True
        while changed:
            changed = False
            for u in list(st.inputs):
                n = prod.get(u)
                if n is None or n.prim not in REMAT:
                    continue
                expr, leaves, stack = {}, set(), [u]
                ok = True
                while stack and ok:
                    v = stack.pop()
                    if v in expr:
                        continue
                    m = prod.get(v)
                    # a value some step stores already is read, not recomputed: a row statistic broadcast over
                    # the row ([R, 1] -> [R, C]) is read as the [R, 1] vector its kernel stores, a float32 copy
                    # of a stored bf16 value as that value, whatever computed them
                    if m is None or m.prim not in REMAT or (v != u and v in in_memory):
                        if v not in in_memory:
                            ok = False
                        leaves.add(v)
                        continue
                    expr[v] = m
                    if len(expr) > REMAT_BUDGET:
                        ok = False
                    stack.extend(m.inputs)
                if not ok:
                    continue
                new = [v for v in leaves if v not in st.inputs]
                if sum(graph.types[v].nbytes() for v in new) > max(graph.types[u].nbytes(), REMAT_SMALL):
                    # more bytes to read than the value it replaces (small per-row vectors are free): repeated
                    # one operand at a time this would unroll a running sum (a residual stream's gradient, bf16)
                    # into reads of every float32 term
                    continue
                have = {m.output for m in st.nodes}
                st.nodes.extend(m for v, m in expr.items() if v not in have)
                st.nodes.sort(key=lambda m: m.output)
                st.inputs = _inputs_of(st.nodes)
                changed = True
                break
    return _drop_unread(graph, steps)


def _drop_unread(graph, steps):
    """A loop or row kernel stops writing extra outputs nobody reads any more, and computing what fed only
    them."""
    read = set(graph.outputs)
    for st in steps:
        read.update(st.inputs)
    for st in steps:
        if st.kind in ("loop", "row") and len(st.outputs) > 1:
            outs = [st.outputs[0]] + [v for v in st.outputs[1:] if v in read]
            if len(outs) < len(st.outputs):
                st.outputs = outs
                by_out = {m.output: m for m in st.nodes}
                live, stack = set(), list(outs)
                while stack:
                    v = stack.pop()
                    if v in live or v not in by_out:
                        continue
                    live.add(v)
                    stack.extend(by_out[v].inputs)
                st.nodes = [m for m in st.nodes if m.output in live]
                st.inputs = _inputs_of(st.nodes)
    return steps


def _space(graph, st):
    """The [shape] a loop or row kernel's elementwise outputs share (a flat index of one is an element of
    the others), or None."""
    if st.kind == "row":
        if st.rows is None:
            return None
        numel = st.rows[0] * st.rows[1]
    elif st.kind == "loop" and st.outputs:
        numel = graph.types[st.outputs[0]].numel()
    else:
        return None
    shapes = {graph.types[v].shape for v in st.outputs if graph.types[v].numel() == numel}
    return next(iter(shapes)) if len(shapes) == 1 else None


def hoist_to_producers(graph, steps):
    """Moves an elementwise expression out of a kernel into the earlier loop or row kernel that writes the
    last of its operands, when the kernel then reads less: it reads the expression's value instead of its
    operands, and the producer computes it in its own pass over the same elements. A running sum whose only
    reader is a late kernel (a bf16 residual stream's gradient, summed term by term over the layers) becomes
    one term added per producer instead of every float32 term held in memory and read at the end."""
    def nbytes(v):
        return graph.types[v].nbytes()

    moved = True
    while moved:
        moved = False
        pos, readers = {}, {}
        for si, st in enumerate(steps):
            for v in st.outputs:
                pos[v] = si
            for u in st.inputs:
                readers.setdefault(u, set()).add(si)
        outputs = set(graph.outputs)
        for ki, kt in enumerate(steps):
            if kt.kind not in ("loop", "row"):
                continue
            inner = {m.output: m for m in kt.nodes}
            users = {}
            for m in kt.nodes:
                for u in m.inputs:
                    users.setdefault(u, set()).add(m.output)
            for n in kt.nodes:
                if n.prim not in ELEMENTWISE:
                    continue
                # n and the kernel's elementwise nodes feeding only it; leaves are the kernel's inputs
                tree, leaves, stack, ok = {n.output}, set(), list(n.inputs), True
                while stack and ok:
                    u = stack.pop()
                    m = inner.get(u)
                    if m is None:
                        leaves.add(u)
                    elif m.prim in ELEMENTWISE and users.get(u, set()) <= tree and u not in kt.outputs:
                        tree.add(u)
                        stack.extend(m.inputs)
                    else:
                        ok = False
                shape = graph.types[n.output].shape
                if not ok or not leaves or any(graph.types[u].shape != shape for u in leaves):
                    continue
                if any(u not in pos and u not in graph.inputs for u in leaves):
                    continue
                pi = max(pos.get(u, -1) for u in leaves)
                if pi < 0 or pi >= ki or _space(graph, steps[pi]) != shape:
                    continue
                pt = steps[pi]
                saved = sum(nbytes(u) for u in leaves if users[u] <= tree)
                have = set(pt.inputs) | {m.output for m in pt.nodes}
                extra = sum(nbytes(u) for u in leaves if u not in have)
                freed = sum(nbytes(u) for u in leaves if pos.get(u) == pi and users[u] <= tree
                            and readers.get(u, set()) == {ki} and u not in outputs)
                if saved - nbytes(n.output) + freed <= extra + nbytes(n.output):
                    continue
                moving = [m for m in kt.nodes if m.output in tree]
                kt.nodes = [m for m in kt.nodes if m.output not in tree]
                if n.output in kt.outputs:
                    kt.outputs = [v for v in kt.outputs if v != n.output]
                kt.inputs = _inputs_of(kt.nodes)
                pt.nodes = sorted(pt.nodes + moving, key=lambda m: m.output)
                pt.outputs = list(pt.outputs) + [n.output]
                pt.inputs = _inputs_of(pt.nodes)
                moved = True
                break
            if moved:
                break
    steps = [st for st in steps if st.kind not in ("loop", "row") or st.outputs]
    return _drop_unread(graph, steps)


def absorb_rows(graph, steps):
    """Merges a loop kernel into an earlier row kernel over the same row space when everything the loop
    reads is the row kernel's input, its output, or already in memory when the row kernel runs: the row
    kernel writes the loop's outputs in its writing pass, and the operands both read (a softmax's logits,
    say) are read once. Cross entropy's backward (softmax minus one-hot) joins the forward's max/sum-exp
    kernel this way."""
    pos = {}
    for si, st in enumerate(steps):
        for v in st.outputs:
            pos[v] = si
    merged = set()
    for li, lt in enumerate(steps):
        if lt.kind != "loop" or len(lt.outputs) == 0:
            continue
        numel = graph.types[lt.outputs[0]].numel()
        cands = {pos[u] for u in lt.inputs if u in pos and steps[pos[u]].kind == "row"}
        for ri in sorted(cands):
            rt = steps[ri]
            if ri in merged or ri >= li or rt.rows is None or rt.rows[0] * rt.rows[1] != numel:
                continue
            elem = [v for v in rt.outputs if graph.types[v].numel() == numel]
            shape = graph.types[(elem or rt.inputs)[0]].shape if (elem or rt.inputs) else None
            if any(graph.types[v].shape != shape for v in lt.outputs):
                continue
            ok = all(u in rt.inputs or u in rt.outputs or pos.get(u, -1) < ri for u in lt.inputs)
            if not ok:
                continue
            have = {m.output for m in rt.nodes}
            joined = sorted(rt.nodes + [m for m in lt.nodes if m.output not in have], key=lambda m: m.output)
            if not row_reads_ok(graph, joined, rt.rows):
                continue
            rt.nodes = joined
            rt.outputs = list(rt.outputs) + [v for v in lt.outputs if v not in rt.outputs]
            rt.inputs = _inputs_of(rt.nodes)
            for v in lt.outputs:
                pos[v] = ri
            merged.add(li)
            break
    return [st for i, st in enumerate(steps) if i not in merged]


# Horizontal fusion (``passes/horizontal.rs:40-49,79-393``): small independent loop kernels share one launch.
HFUSE_MAX_ELEMENTS = 1 << 20      # a member's outputs are at most this many elements each
HFUSE_MAX_MEMBERS = 32
HFUSE_MAX_HELD_BYTES = 16 << 20   # operand bytes a group may keep alive past their first use


def horizontal(graph, steps):
    """Groups small loop steps that do not read each other's results into ``hloop`` steps. A member runs
    late, at the group's launch, so the group is launched before the first later step that reads one of its
    results (or at the end); steps in between keep their order."""
    def small(st):
        return st.kind == "loop" and all(graph.types[v].numel() <= HFUSE_MAX_ELEMENTS for v in st.outputs)

    out, group, produced, held = [], [], set(), 0

    def flush():
        nonlocal group, produced, held
        if len(group) == 1:
            out.append(group[0])
        elif group:
            st = Step("hloop", [n for m in group for n in m.nodes], [v for m in group for v in m.outputs],
                      [v for m in group for v in m.inputs])
            st.members = group
            out.append(st)
        group, produced, held = [], set(), 0

    for st in steps:
        if group and any(u in produced for u in st.inputs):
            flush()
        if small(st):
            nbytes = sum(graph.types[u].nbytes() for u in st.inputs)
            if len(group) >= HFUSE_MAX_MEMBERS or held + nbytes > HFUSE_MAX_HELD_BYTES:
                flush()
            group.append(st)
            produced.update(st.outputs)
            held += nbytes
            continue
        out.append(st)
    flush()
    return out


def _index_only(v, prod, done):
    n = prod.get(v)
    if n is None:
        return False
    if n.prim in INDEX_ONLY:
        return True
    if n.prim in ("reshape", "broadcast_in_dim", "transpose", "slice"):
        return all(u in done or _index_only(u, prod, done) for u in n.inputs)
    return False


def _pull_index_math(graph, st, prod, done_inputs):
    materialized = set()
    for s in st.inputs:
        materialized.add(s)
    changed = True
    while changed:
        changed = False
        produced = {m.output for m in st.nodes}
        for u in list(st.inputs):
            n = prod.get(u)
            if n is not None and u not in produced and (n.prim in INDEX_ONLY) and u not in st.outputs:
                st.nodes.append(n)
                changed = True
        if changed:
            st.nodes.sort(key=lambda m: m.output)
            produced = {m.output for m in st.nodes}
            st.inputs = []
            for m in st.nodes:
                for u in m.inputs:
                    if u not in produced and u not in st.inputs:
                        st.inputs.append(u)


def _fits(graph, u, roots, rs):
    """Whether value ``u`` can be an extra output of a kernel with ``roots`` (and row space ``rs``)."""
    nu = graph.types[u].numel()
    base = graph.types[roots[0]].numel()
    if rs is None:
        return nu == base
    return nu in (rs[0] * rs[1], rs[0])


