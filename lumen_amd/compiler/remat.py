"""Rematerialization (``lumen/graph_compiler/remat.rs:1-200``; used by ``lumen/plan/compile.rs:37-44``): when a
plan's workspace exceeds ``config.compiler.memory_limit``, large values computed before the live-bytes
peak and read again after it are recomputed just before those later readers instead of being kept live.

Only cheap values are recomputed: elementwise and layout nodes (and, up to two levels back, such producers
of theirs) whose operands are still live at the later reader anyway, so a recomputation never extends
another value's life. Each round keeps a rewrite only if the real placement of the result needs less
workspace; values are bit-identical (a recomputation evaluates the same nodes on the same operands).
"""

from __future__ import annotations

from lumen_amd.graph.ir import ELEMENTWISE, Graph

RECOMPUTABLE = ELEMENTWISE | {"reshape", "transpose", "broadcast_in_dim", "slice", "full", "iota"}
MIN_BYTES = 64 << 10
MAX_DEPTH = 2
ROUNDS = 8
TRIES = 4  # candidates a round evaluates by placement


def usage(graph: Graph) -> list:
    """Live bytes at each node: a value counts from its node through its last reader (graph outputs to the
    end); graph inputs are the plan's inputs, not workspace."""
    n = len(graph.nodes)
    last = _last_readers(graph)
    delta = [0] * (n + 1)
    for i, nd in enumerate(graph.nodes):
        b = graph.types[nd.output].nbytes()
        delta[i] += b
        end = last.get(nd.output, i)
        if end < n:
            delta[end + 1] -= b
    live, out = 0, []
    for i in range(n):
        live += delta[i]
        out.append(live)
    return out


def _last_readers(graph):
    last = {}
    for i, nd in enumerate(graph.nodes):
        for v in nd.inputs:
            last[v] = i
    for v in graph.outputs:
        last[v] = len(graph.nodes)
    return last


def _plan_clone(graph, i, at, last, inputs):
    """Nodes to clone (producers first) so node ``i``'s value can be recomputed before node ``at``: ``i`` and,
    up to ``MAX_DEPTH`` levels, recomputable producers of operands not live at ``at``. None if impossible."""
    prod = {nd.output: k for k, nd in enumerate(graph.nodes)}
    chain = []

    def visit(k, depth):
        nd = graph.nodes[k]
        if nd.prim not in RECOMPUTABLE or depth > MAX_DEPTH:
            return False
        for v in nd.inputs:
            if v in inputs or last.get(v, -1) >= at:
                continue  # still live at the reader: read it
            p = prod.get(v)
            if p is None or not visit(p, depth + 1):
                return False
        if k not in chain:
            chain.append(k)
        return True

    return chain if visit(i, 1) else None


def recompute(graph: Graph, i: int, after: int) -> Graph | None:
    """A copy of ``graph`` whose readers of node ``i``'s value that come after node ``after`` read a
    recomputation of it placed before the first of them; None when it cannot be recomputed there."""
    v = graph.nodes[i].output
    readers = [k for k, nd in enumerate(graph.nodes) if k > after and v in nd.inputs]
    if not readers:
        return None
    at = readers[0]
    last = _last_readers(graph)
    chain = _plan_clone(graph, i, at, last, set(graph.inputs))
    if chain is None:
        return None
    g = Graph()
    remap = {u: g.input(graph.types[u].dtype, graph.types[u].shape) for u in graph.inputs}
    clone_of = {}  # original value -> its recomputation, read by nodes from `at` on
    for k, nd in enumerate(graph.nodes):
        if k == at:
            for c in chain:  # producers first
                m = graph.nodes[c]
                ins = tuple(clone_of.get(u, remap[u]) for u in m.inputs)
                clone_of[m.output] = g.add_node(m.prim, ins, m.params, graph.types[m.output], m.backward)
        ins = tuple((clone_of[u] if k >= at and u in clone_of else remap[u]) for u in nd.inputs)
        remap[nd.output] = g.add_node(nd.prim, ins, nd.params, graph.types[nd.output], nd.backward)
    g.set_outputs([remap[u] for u in graph.outputs])
    return g


def _step_live_ranges(plan):
    """``{value: (first step, last reading step, bytes)}`` of every value a plan step writes to the workspace
    (views extend their base's range), and the index of the step where the most bytes are live."""
    steps, g = plan.steps, plan.graph
    base = {}
    for st in steps:
        if st.kind == "view":
            v, src = st.outputs[0], st.nodes[0].inputs[0]
            base[v] = base.get(src, src)
    rng = {}
    for t, st in enumerate(steps):
        if st.kind == "view":
            continue
        for v in st.outputs:
            rng[v] = [t, t, g.types[v].nbytes()]
    for t, st in enumerate(steps):
        for u in st.inputs:
            r = rng.get(base.get(u, u))
            if r is not None:
                r[1] = max(r[1], t)
    for v in g.outputs:
        r = rng.get(base.get(v, v))
        if r is not None:
            r[1] = len(steps)
    live = [0] * (len(steps) + 1)
    for a, b, nbytes in rng.values():
        live[a] += nbytes
        live[min(b, len(steps) - 1) + 1] -= nbytes
    total, peak, at = 0, -1, 0
    for t in range(len(steps)):
        total += live[t]
        if total > peak:
            peak, at = total, t
    return rng, at


def rematerialize(graph: Graph, limit: int, plan_of) -> Graph:
    """``graph`` with values recomputed until ``plan_of(graph).workspace_bytes`` is at most ``limit`` or no
    candidate helps; the smallest found. Candidates are values plan steps write before the step where the
    most bytes are live and read again after it, largest first."""
    best_g, best_p = graph, plan_of(graph)
    for _ in range(ROUNDS):
        if best_p.workspace_bytes <= limit:
            break
        rng, peak = _step_live_ranges(best_p)
        peak_reads = set(best_p.steps[peak].inputs)
        pos = {nd.output: k for k, nd in enumerate(best_g.nodes)}
        done = [pos[m.output] for st in best_p.steps[: peak + 1] for m in st.nodes if m.output in pos]
        after = max(done) if done else -1
        cands = sorted(((b, v) for v, (a, e, b) in rng.items()
                        if a < peak < e and v not in peak_reads and b >= MIN_BYTES and v in pos
                        and best_g.nodes[pos[v]].prim in RECOMPUTABLE and v not in best_g.outputs), reverse=True)
        improved = False
        for _, v in cands[:TRIES]:
            g2 = recompute(best_g, pos[v], after)
            if g2 is None:
                continue
            p2 = plan_of(g2)
            if p2.workspace_bytes < best_p.workspace_bytes:
                best_g, best_p, improved = g2, p2, True
                break
        if not improved:
            break
    return best_g
