"""Step schedules of a plan (``lumen/graph_compiler/schedule.rs:90,161``; the choice among them,
``lumen/plan/compile.rs:19-47``): the plan keeps whichever order of its steps — as fused, in the graph's
node order, greedy list, or depth-first — needs the smallest workspace.

Both schedules work on steps (a fused kernel, a built-in kernel or a view), a step depending on the steps
that write the values it reads. Values reached through view steps count as their base's storage.
"""

from __future__ import annotations


def _deps(steps):
    """Per step, the sorted steps it must follow, and per step the steps following it."""
    writer = {}
    for i, st in enumerate(steps):
        for v in st.outputs:
            writer[v] = i
    operands = []
    for i, st in enumerate(steps):
        ops = sorted({writer[u] for u in st.inputs if u in writer and writer[u] != i})
        operands.append(ops)
    users = [[] for _ in steps]
    for i, ops in enumerate(operands):
        for o in ops:
            users[o].append(i)
    return operands, users


def _roots(graph, steps):
    """Per value, the value whose storage it is (a view step's output is its operand's)."""
    root = {}
    for st in steps:
        if st.kind == "view":
            v, src = st.outputs[0], st.nodes[0].inputs[0]
            root[v] = root.get(src, src)
    return lambda v: root.get(v, v)


def _out_bytes(graph, st):
    return 0 if st.kind == "view" else sum(graph.types[v].nbytes() for v in st.outputs)


def list_order(graph, steps):
    """Greedy list schedule: of the ready steps, run the one freeing the most bytes net of what it writes
    (views first, then more readers, then the earlier step)."""
    operands, users = _deps(steps)
    root = _roots(graph, steps)
    pinned = {root(v) for v in list(graph.inputs) + list(graph.outputs)}
    reads = [sorted({root(u) for u in st.inputs}) for st in steps]
    unread = {}
    for rs in reads:
        for r in rs:
            unread[r] = unread.get(r, 0) + 1
    waiting = [len(o) for o in operands]
    ready = [i for i in range(len(steps)) if waiting[i] == 0]
    order = []
    while ready:
        def priority(i):
            if steps[i].kind == "view":
                return (float("inf"), float("inf"), -i)
            freed = sum(graph.types[r].nbytes() for r in reads[i] if r not in pinned and unread[r] == 1)
            return (freed - _out_bytes(graph, steps[i]), len(users[i]), -i)

        k = max(range(len(ready)), key=lambda k: priority(ready[k]))
        i = ready.pop(k)
        order.append(i)
        for r in reads[i]:
            unread[r] -= 1
        for u in users[i]:
            waiting[u] -= 1
            if waiting[u] == 0:
                ready.append(u)
    return [steps[i] for i in order]


def dfs_order(graph, steps):
    """Depth-first post-order from the steps writing the graph's outputs, each step's heavier operand
    subgraphs (more extra readers, then more bytes written) visited first, so lighter ones run close to
    their use."""
    operands, users = _deps(steps)
    n = len(steps)
    cap = sum(_out_bytes(graph, st) for st in steps)
    stats = []
    for i in range(n):
        extra, nbytes = max(len(users[i]) - 1, 0), _out_bytes(graph, steps[i])
        for o in operands[i]:
            extra, nbytes = extra + stats[o][0], nbytes + stats[o][1]
        stats.append((min(extra, n), min(nbytes, cap)))
    writer = {}
    for i, st in enumerate(steps):
        for v in st.outputs:
            writer[v] = i
    starts = [writer[v] for v in graph.outputs if v in writer] + list(range(n))
    seen, order = [False] * n, []

    def by_weight(i):  # popped from the end: the heaviest operand first
        return sorted(operands[i], key=lambda o: (stats[o][0], stats[o][1], -o))

    for s in starts:
        if seen[s]:
            continue
        seen[s] = True
        stack = [(s, by_weight(s))]
        while stack:
            i, ops = stack[-1]
            if ops:
                o = ops.pop()
                if not seen[o]:
                    seen[o] = True
                    stack.append((o, by_weight(o)))
            else:
                order.append(i)
                stack.pop()
    return [steps[i] for i in order]


def traced_order(graph, steps):
    """The steps in the graph's own node order: of the ready steps, the one whose last node comes first in
    the graph (a recomputation placed late in the graph runs late)."""
    import heapq

    operands, users = _deps(steps)
    pos = {n.output: k for k, n in enumerate(graph.nodes)}
    key = [max((pos.get(m.output, -1) for m in st.nodes), default=-1) for st in steps]
    waiting = [len(o) for o in operands]
    heap = [(key[i], i) for i in range(len(steps)) if waiting[i] == 0]
    heapq.heapify(heap)
    order = []
    while heap:
        _, i = heapq.heappop(heap)
        order.append(i)
        for u in users[i]:
            waiting[u] -= 1
            if waiting[u] == 0:
                heapq.heappush(heap, (key[u], u))
    return [steps[i] for i in order]


SCHEDULES = {"traced": traced_order, "list": list_order, "dfs": dfs_order}
