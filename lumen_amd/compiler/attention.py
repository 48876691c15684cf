"""Flash-attention matching (``lumen/graph_compiler/passes/attention/forward.rs:58-423``,
``attention/backward.rs:56-237``) and its lowering to the built-in kernels.

Forward: ``softmax(scale * Q K^T [masked]) V`` written as primitives -- a dot, a multiply by a scalar, an
optional ``select`` against ``-inf``, ``reduce_max``, ``exp`` of the difference, ``reduce_sum``, the division,
a cast to the operands' dtype and the dot with V -- becomes one ``fusion`` named ``flash_attention`` whose
body keeps those primitives (so the oracle still evaluates the exact graph), with the log-sum-exp
``m + log(l)`` as an extra output when the backward reads it. The mask must be the bottom-right aligned
causal mask ``key <= query + Sk - Sq`` (checked by evaluating the mask's index graph) or absent.

Backward: FlashAttention-2's gradient (``lumen/functional/attention/flash.py:50-85``) -- probabilities
recomputed from the log-sum-exp, ``delta = rowsum(dO * O)``, the three gradient dots and their transposes and
casts -- becomes one ``flash_attention_backward`` fusion producing dQ, dK and dV.
"""

from __future__ import annotations

import numpy as np

from lumen_amd.graph.ir import Graph, Node, TensorType

FWD, BWD = "flash_attention", "flash_attention_backward"

# Largest head dims the flash kernels take (``forward.rs:100`` MAX_HEAD, ``backward.rs:86`` MAX_BACKWARD_HEAD):
# multiples of 8; the kernels run at 64, 128 or 256 with the columns past the head dim read as zeros.
MAX_HEAD, MAX_BACKWARD_HEAD = 256, 128


def _head_dim_ok(h, limit):
    return h > 0 and h % 8 == 0 and h <= limit


class _G:
    """Lookup helpers over a graph."""

    def __init__(self, g: Graph):
        self.g = g
        self.prod = g.producers()
        self.users = g.users()

    def node(self, v, prim=None):
        n = self.prod.get(v)
        if n is None or (prim is not None and n.prim != prim):
            return None
        return n

    def through(self, v, *prims):
        """Follows ``v`` back through producers of ``prims`` (reshape, broadcast...), returning the first
        value produced otherwise."""
        while True:
            n = self.prod.get(v)
            if n is None or n.prim not in prims:
                return v
            v = n.inputs[0]

    def const(self, v):
        """The fill value if ``v`` is a ``full`` (through broadcasts/reshapes), else None."""
        v = self.through(v, "broadcast_in_dim", "reshape")
        n = self.node(v, "full")
        return None if n is None else n.params["fill_value"]


def _scaled_scores(G, v):
    """``(dot, scale)`` if ``v`` is ``dot * full(scale)``."""
    n = G.node(v, "mul")
    if n is None:
        return None
    for a, b in ((0, 1), (1, 0)):
        d = G.node(n.inputs[a], "dot_general")
        s = G.const(n.inputs[b])
        if d is not None and s is not None:
            return d, float(s), n
    return None


def _mask(G, v):
    """``(scores, mask_nodes, pred)`` if ``v`` is ``select(pred, scores, -inf)``, else ``(v, [], None)``."""
    n = G.node(v, "select")
    if n is None:
        return v, [], None
    fill = G.const(n.inputs[2])
    if fill is None or fill != float("-inf"):
        return None
    return n.inputs[1], [n], n.inputs[0]


_MASK_PRIMS = {"iota", "full", "add", "sub", "lt", "eq", "select", "and", "or", "not", "broadcast_in_dim", "reshape",
               "max", "neg", "mul"}


def _mask_graph(G, pred):
    """The nodes computing ``pred`` if it is index math alone (iotas and constants), else None."""
    seen, stack, nodes = set(), [pred], []
    while stack:
        v = stack.pop()
        if v in seen:
            continue
        seen.add(v)
        n = G.prod.get(v)
        if n is None or n.prim not in _MASK_PRIMS:
            return None
        if n.prim == "iota" and n.params["dimension"] < len(n.params["shape"]) - 2:
            return None
        nodes.append(n)
        stack.extend(n.inputs)
    return sorted(nodes, key=lambda m: m.output)


def _eval_mask(G, nodes, pred, sq, sk):
    """``pred`` evaluated over one [sq, sk] score matrix (the mask reads only the last two indices)."""
    env = {}
    for n in nodes:
        t = G.g.types[n.output]
        shape = t.shape[:-2] + (sq, sk) if len(t.shape) >= 2 else t.shape
        shape = tuple(1 for _ in shape[:-2]) + shape[-2:] if len(shape) >= 2 else shape
        p = n.prim
        ins = [env[u] for u in n.inputs]
        if p == "iota":
            d = n.params["dimension"]
            r = np.arange(shape[d]).reshape([-1 if i == d else 1 for i in range(len(shape))])
            env[n.output] = np.broadcast_to(r, shape)
        elif p == "full":
            env[n.output] = np.broadcast_to(np.array(n.params["fill_value"]), shape)
        elif p in ("broadcast_in_dim", "reshape"):
            env[n.output] = np.broadcast_to(ins[0].reshape(ins[0].shape + (1,) * 0), shape) if ins[0].size in (1, np.prod(shape)) else None
            if env[n.output] is None:
                return None
        elif p == "add":
            env[n.output] = ins[0] + ins[1]
        elif p == "sub":
            env[n.output] = ins[0] - ins[1]
        elif p == "mul":
            env[n.output] = ins[0] * ins[1]
        elif p == "neg":
            env[n.output] = -ins[0]
        elif p == "max":
            env[n.output] = np.maximum(ins[0], ins[1])
        elif p == "lt":
            env[n.output] = ins[0] < ins[1]
        elif p == "eq":
            env[n.output] = ins[0] == ins[1]
        elif p == "select":
            env[n.output] = np.where(ins[0], ins[1], ins[2])
        elif p == "and":
            env[n.output] = ins[0] & ins[1]
        elif p == "or":
            env[n.output] = ins[0] | ins[1]
        elif p == "not":
            env[n.output] = ~ins[0]
    return np.asarray(env[pred]).reshape(sq, sk)


def _causal(G, pred, sq, sk):
    """True if ``pred`` is the bottom-right causal mask, False if absent, None if unrecognized."""
    if pred is None:
        return False
    nodes = _mask_graph(G, pred)
    if nodes is None:
        return None
    m = _eval_mask(G, nodes, pred, sq, sk)
    if m is None:
        return None
    want = np.arange(sk)[None, :] <= np.arange(sq)[:, None] + (sk - sq)
    return True if np.array_equal(m, want) else None


def _row_stat(G, v, prim):
    """The reduction behind ``broadcast(reshape(reduce(x, last)))``: ``(reduce node, reshape var)``."""
    b = G.node(v, "broadcast_in_dim")
    if b is None:
        return None
    r = G.node(b.inputs[0], "reshape")
    if r is None:
        return None
    red = G.node(r.inputs[0], prim)
    if red is None:
        return None
    x = G.g.types[red.inputs[0]]
    if tuple(red.params["axes"]) != (len(x.shape) - 1,):
        return None
    return red, r.output


def _dims_of_dot(n, side, ty):
    """``(batch dims, free dims, contracting dims)`` of a dot operand."""
    p = n.params
    c = p["lhs_contracting"] if side == 0 else p["rhs_contracting"]
    b = p["lhs_batch"] if side == 0 else p["rhs_batch"]
    f = [d for d in range(len(ty.shape)) if d not in c and d not in b]
    return tuple(b), tuple(f), tuple(c)


def _unexpand(G, v, batch_dims):
    """``(x, nodes)`` if ``v`` is grouped-query attention's head expansion of ``x`` [B, S, Nkv, H]
    (``expand_heads``: reshape to [B, S, Nkv, 1, H], broadcast to [B, S, Nkv, G, H], reshape to
    [B, S, Nkv G, H], so head n reads key/value head n / G) and a dot reads ``v`` with batch dims
    ``batch_dims`` = (0, 2); else ``(v, [])``. The kernels take ``x`` itself and the head ratio."""
    r2 = G.node(v, "reshape")
    bc = r2 and G.node(r2.inputs[0], "broadcast_in_dim")
    r1 = bc and G.node(bc.inputs[0], "reshape")
    if r1 is None or tuple(batch_dims) != (0, 2):
        return v, []
    x = r1.inputs[0]
    xt = G.g.types[x]
    if len(xt.shape) != 4:
        return v, []
    b, s, nkv, h = xt.shape
    t1, t2, t3 = (G.g.types[n.output].shape for n in (r1, bc, r2))
    grp = t2[3] if len(t2) == 5 else 0
    if (t1 != (b, s, nkv, 1, h) or len(t2) != 5 or t2 != (b, s, nkv, grp, h) or t3 != (b, s, nkv * grp, h)
            or tuple(bc.params["broadcast_dimensions"]) != (0, 1, 2, 3, 4)):
        return v, []
    return x, [r1, bc, r2]


def match_forward(g: Graph):
    """Each forward attention of ``g``: a dict of its nodes, operands, scale and mask."""
    G = _G(g)
    found = []
    for d2 in g.nodes:
        if d2.prim != "dot_general":
            continue
        cast = G.node(d2.inputs[0], "cast")
        if cast is None:
            continue
        div = G.node(cast.inputs[0], "div")
        if div is None:
            continue
        e = div.inputs[0]
        rs = _row_stat(G, div.inputs[1], "reduce_sum")
        if rs is None or rs[0].inputs[0] != e:
            continue
        exp = G.node(e, "exp")
        sub = exp and G.node(exp.inputs[0], "sub")
        if sub is None:
            continue
        rm = _row_stat(G, sub.inputs[1], "reduce_max")
        if rm is None or rm[0].inputs[0] != sub.inputs[0]:
            continue
        masked = _mask(G, sub.inputs[0])
        if masked is None:
            continue
        s1, mask_nodes, pred = masked
        sc = _scaled_scores(G, s1)
        if sc is None:
            continue
        d1, scale, mul = sc
        st = g.types[d1.output]
        if len(st.shape) != 4 or len(d1.params["lhs_batch"]) != 2 or len(d1.params["lhs_contracting"]) != 1:
            continue
        if tuple(d2.params["lhs_contracting"]) != (3,) or tuple(d2.params["lhs_batch"]) != (0, 1):
            continue
        if len(d2.params["rhs_contracting"]) != 1 or len(d2.params["rhs_batch"]) != 2:
            continue
        sq, sk = st.shape[2], st.shape[3]
        causal = _causal(G, pred, sq, sk)
        if causal is None or (causal and sk < sq):
            # causal with fewer keys than queries leaves the first sq - sk rows with no key: the written
            # attention gives NaN there, which the unfused plan reproduces and the flash kernel does not
            continue
        qt, kt, vt = (g.types[u] for u in (d1.inputs[0], d1.inputs[1], d2.inputs[1]))
        if qt.dtype not in ("bfloat16", "float16") or not (qt.dtype == kt.dtype == vt.dtype):
            continue
        if g.types[cast.output].dtype != qt.dtype or g.types[d2.output].dtype != qt.dtype:
            continue
        qb, qf, qc = _dims_of_dot(d1, 0, qt)
        kb, kf, kc = _dims_of_dot(d1, 1, kt)
        vb, vf, vc = _dims_of_dot(d2, 1, vt)
        if len(qf) != 1 or len(kf) != 1 or len(vf) != 1 or not _head_dim_ok(qt.shape[qc[0]], MAX_HEAD):
            continue
        if not _head_dim_ok(vt.shape[vf[0]], MAX_HEAD):  # the value head dim may differ from the query's
            continue
        # grouped heads: the kernel reads the key/value heads themselves (head n reads head n / G)
        k_in, k_exp = _unexpand(G, d1.inputs[1], kb)
        v_in, v_exp = _unexpand(G, d2.inputs[1], vb)
        if bool(k_exp) != bool(v_exp) or (k_exp and g.types[k_in].shape[2] != g.types[v_in].shape[2]):
            k_in, v_in, k_exp, v_exp = d1.inputs[1], d2.inputs[1], [], []
        # value nodes of the body (constants and mask math are copied)
        core = [*k_exp, *v_exp, d1, mul, *mask_nodes, rm[0], G.node(rm[1]), G.node(sub.inputs[1]), sub, exp, rs[0],
                G.node(rs[1]), G.node(div.inputs[1]), div, cast, d2]
        # the log-sum-exp read by a backward: add(reshape(max), log(reshape(sum)))
        lse = None
        for u in G.users.get(rs[1], []):
            if u.prim == "log":
                for a in G.users.get(u.output, []):
                    if a.prim == "add" and set(a.inputs) == {rm[1], u.output}:
                        lse = (u, a)
        if lse:
            core += list(lse)
        found.append(dict(core=core, d1=d1, d2=d2, q=d1.inputs[0], k=k_in, v=v_in, scale=scale,
                          causal=causal, lse=lse[1].output if lse else None, q_dims=(qb, qf[0], qc[0]),
                          k_dims=(kb, kf[0], kc[0]), v_dims=(vb, vc[0], vf[0]), mask_pred=pred,
                          shared={n.output for n in k_exp + v_exp}))
    return found


def match_backward(g: Graph):
    """Each FlashAttention-2 backward of ``g`` (as ``_FlashAttention.backward`` traces it)."""
    G = _G(g)
    found = []
    for dv in g.nodes:
        if dv.prim != "dot_general":
            continue
        c_pt = G.node(dv.inputs[0], "cast")
        if c_pt is None:
            continue
        pt_exp = G.node(c_pt.inputs[0], "exp")
        sub = pt_exp and G.node(pt_exp.inputs[0], "sub")
        if sub is None:
            continue
        b_l = G.node(sub.inputs[1], "broadcast_in_dim")
        r_l = b_l and G.node(b_l.inputs[0], "reshape")
        if r_l is None:
            continue
        lse = r_l.inputs[0]
        masked = _mask(G, sub.inputs[0])
        if masked is None:
            continue
        s1, mask_nodes, pred = masked
        sc = _scaled_scores(G, s1)
        if sc is None:
            continue
        dst_dot, scale, mul_s = sc
        pt = pt_exp.output
        # dS^T = (scale * (P^T * (dP^T - delta))) cast, read by dK and dQ dots
        dsts = []
        for u in G.users.get(pt, []):
            if u.prim != "mul" or u.output == c_pt.output:
                continue
            other = u.inputs[1] if u.inputs[0] == pt else u.inputs[0]
            sb = G.node(other, "sub")
            if sb is None:
                continue
            for u2 in G.users.get(u.output, []):
                if u2.prim == "mul" and G.const(u2.inputs[0] if u2.inputs[1] == u.output else u2.inputs[1]) is not None:
                    for u3 in G.users.get(u2.output, []):
                        if u3.prim == "cast":
                            dsts.append((u, sb, u2, u3))
        if len(dsts) != 1:
            continue
        mul_p, sub_d, mul_sc, c_ds = dsts[0]
        dpt = G.node(sub_d.inputs[0], "dot_general")
        bd = G.node(sub_d.inputs[1], "broadcast_in_dim")
        rd = bd and G.node(bd.inputs[0], "reshape")
        td = rd and G.node(rd.inputs[0], "transpose")
        ddot = td and G.node(td.inputs[0], "dot_general")
        if dpt is None or ddot is None:
            continue
        dk = dq = None
        for u in G.users.get(c_ds.output, []):
            if u.prim == "dot_general":
                if tuple(u.params["lhs_contracting"]) == (3,):
                    dk = u
                elif tuple(u.params["lhs_contracting"]) == (2,):
                    dq = u
        if dk is None or dq is None:
            continue
        k, q = dst_dot.inputs
        v, do = dpt.inputs
        if ddot.inputs[0] != do:
            continue
        o = ddot.inputs[1]
        if dv.inputs[1] != do or dk.inputs[1] != q or dq.inputs[1] != k:
            continue
        qt = g.types[q]
        if qt.dtype not in ("bfloat16", "float16") or len(qt.shape) != 4 or not _head_dim_ok(qt.shape[3], MAX_BACKWARD_HEAD):
            continue
        hv = g.types[v].shape[3] if len(g.types[v].shape) == 4 else 0
        if (len(g.types[k].shape) != 4 or g.types[k].shape[3] != qt.shape[3] or not _head_dim_ok(hv, MAX_BACKWARD_HEAD)
                or any(len(g.types[x].shape) != 4 or g.types[x].shape[3] != hv for x in (o, do))):
            continue  # one head dim for Q and K, one for V, O and dO
        if any(tuple(x.params["rhs_batch"]) != (0, 2) for x in (dv, dk, dq)):
            continue
        # grouped heads: K and V expanded to every query head, dK and dV summed over each group
        k_in, k_exp = _unexpand(G, k, dst_dot.params["lhs_batch"])
        v_in, v_exp = _unexpand(G, v, dpt.params["lhs_batch"])
        if bool(k_exp) != bool(v_exp):
            continue
        grouped = bool(k_exp)
        if grouped and g.types[k_in].shape[2] != g.types[v_in].shape[2]:
            continue
        sq_, sk_ = g.types[pt].shape[3], g.types[pt].shape[2]
        # the mask here is over [Sk, Sq]: evaluate transposed
        causal = _causal_t(G, pred, sk_, sq_)
        if causal is None or (causal and sk_ < sq_):  # rows with no key: left to the unfused plan
            continue
        outs = []
        tail = []
        ok = True
        for x in (dq, dk, dv):
            us = G.users.get(x.output, [])
            if len(us) != 1 or us[0].prim != "transpose" or tuple(us[0].params["permutation"]) != (0, 2, 1, 3):
                ok = False
                break
            hops = [us[0]]
            if grouped and x is not dq:  # reshape [B, Sk, Nkv, G, D], sum over the group axis
                r = G.users.get(us[0].output, [])
                red = len(r) == 1 and r[0].prim == "reshape" and G.users.get(r[0].output, [])
                if not (red and len(red) == 1 and red[0].prim == "reduce_sum" and tuple(red[0].params["axes"]) == (3,)
                        and g.types[r[0].output].shape[:3] == g.types[k_in].shape[:3]):
                    ok = False
                    break
                hops += [r[0], red[0]]
            us2 = G.users.get(hops[-1].output, [])
            if len(us2) != 1 or us2[0].prim != "cast" or g.types[us2[0].output].dtype != qt.dtype:
                ok = False
                break
            outs.append(us2[0].output)
            tail += hops + [us2[0]]
        if not ok:
            continue
        core = [*k_exp, *v_exp, dst_dot, mul_s, *mask_nodes, r_l, b_l, sub, pt_exp, ddot, td, rd, bd, dpt, sub_d, mul_p,
                mul_sc, c_ds, c_pt, dv, dk, dq] + tail
        found.append(dict(core=core, q=q, k=k_in, v=v_in, o=o, do=do, lse=lse, scale=scale, causal=causal, outs=outs,
                          mask_pred=pred, shared={n.output for n in k_exp + v_exp}))
    return found


def _causal_t(G, pred, sk, sq):
    """Like ``_causal`` for a mask over transposed scores ``[Sk, Sq]``."""
    if pred is None:
        return False
    nodes = _mask_graph(G, pred)
    if nodes is None:
        return None
    m = _eval_mask(G, nodes, pred, sk, sq)
    if m is None:
        return None
    want = np.arange(sk)[:, None] <= np.arange(sq)[None, :] + (sk - sq)
    return True if np.array_equal(m, want) else None


def _closure(G, core, inputs):
    """``core`` plus the constant/index nodes it reads (copied into a body), and the external inputs."""
    nodes = {n.output: n for n in core}
    stack = [u for n in core for u in n.inputs]
    while stack:
        u = stack.pop()
        if u in nodes or u in inputs:
            continue
        n = G.prod.get(u)
        if n is None:
            return None
        if n.prim in ("full", "iota") or (n.prim in _MASK_PRIMS and all(_is_index(G, w) for w in n.inputs)):
            nodes[u] = n
            stack.extend(n.inputs)
        else:
            return None
    return sorted(nodes.values(), key=lambda m: m.output)


def _is_index(G, v):
    n = G.prod.get(v)
    return n is not None and n.prim in _MASK_PRIMS and all(_is_index(G, w) for w in n.inputs)


def _body(g, nodes, inputs, outputs):
    body = Graph()
    remap = {}
    for v in inputs:
        t = g.types[v]
        remap[v] = body.input(t.dtype, t.shape)
    for n in nodes:
        remap[n.output] = body.add_node(n.prim, tuple(remap[u] for u in n.inputs), n.params, g.types[n.output])
    body.set_outputs([remap[v] for v in outputs])
    return body


def match(graph: Graph) -> Graph:
    """``graph`` with every recognized attention forward and backward replaced by flash fusions."""
    g = graph
    for kind in (BWD, FWD):
        G = _G(g)
        ms = match_backward(g) if kind == BWD else match_forward(g)
        if not ms:
            continue
        replace = {}   # var -> (fusion index, output index)
        fusions = []
        for m in ms:
            if kind == FWD:
                inputs = [m["q"], m["k"], m["v"]]
                outputs = [m["d2"].output] + ([m["lse"]] if m["lse"] is not None else [])
            else:
                inputs = [m["q"], m["k"], m["v"], m["o"], m["do"], m["lse"]]
                outputs = list(m["outs"])
            nodes = _closure(G, m["core"], set(inputs))
            if nodes is None:
                continue
            inner = {n.output for n in nodes}
            # interior values must not escape but through the outputs
            # (the head expansion of grouped K and V is a layout of an input: it stays for other readers too)
            escapes = any(
                u.output not in inner for n in nodes if n.output not in outputs and n.prim not in ("full", "iota")
                and not _is_index(G, n.output) and n.output not in m["shared"] for u in G.users.get(n.output, [])
            )
            if escapes:
                continue
            body = _body(g, nodes, inputs, outputs)
            params = dict(name=kind, body=body, scale=m["scale"], causal=bool(m["causal"]))
            if kind == FWD:
                params.update(q_dims=m["q_dims"], k_dims=m["k_dims"], v_dims=m["v_dims"])
            fusions.append((m, inputs, outputs, params, inner))
            for j, v in enumerate(outputs):
                replace[v] = (len(fusions) - 1, j)
        if not fusions:
            continue
        g = _rewrite(g, fusions, replace)
    return g


def _rewrite(g, fusions, replace):
    out = Graph()
    remap = {}
    for v in g.inputs:
        remap[v] = out.input(g.types[v].dtype, g.types[v].shape)
    anchor = {}
    for fi, (m, inputs, outputs, params, inner) in enumerate(fusions):
        anchor[max(outputs)] = fi
    done = set()
    removed = set()
    for fi, (_, _, outputs, _, inner) in enumerate(fusions):
        removed |= set(outputs)
    for n in g.nodes:
        if n.output in replace:
            fi, _ = replace[n.output]
            if fi in done:
                continue
            # emit the fusion where its last output was computed (all inputs exist by then)
            m, inputs, outputs, params, inner = fusions[fi]
            if n.output != min(outputs):
                continue
            done.add(fi)
            f = out.add_node("fusion", tuple(remap[u] for u in inputs), params, g.types[outputs[0]], n.backward)
            remap[outputs[0]] = f
            for j, v in enumerate(outputs[1:], 1):
                remap[v] = out.add_node("fusion_output", (f,), {"index": j, "ty": g.types[v]}, g.types[v], n.backward)
            continue
        if any(u not in remap for u in n.inputs):
            continue  # interior node of a fusion: dropped
        remap[n.output] = out.add_node(n.prim, tuple(remap[u] for u in n.inputs), n.params, g.types[n.output],
                                       n.backward)
    out.set_outputs([remap[v] for v in g.outputs])
    out.prune()
    return out


# ---- lowering to built-in steps ------------------------------------------------------------------------


def lower(plan, step):
    """``(kind, nhip_attn_desc, [locations])`` of a flash step of ``plan``."""
    from lumen_amd import native as nv

    g = plan.graph
    n = step.nodes[0]
    p = n.params
    body = p["body"]
    loc = plan.loc
    a = nv.AttnDesc()
    a.scale, a.causal = p["scale"], int(p["causal"])
    a.config = getattr(step, "config", -1) if p["name"] == FWD else -1  # the forward's tile (autotuned or forced)
    from lumen_amd.config import config

    a.deterministic = backward_mode() if step.mode is None else step.mode
    if p["name"] == FWD:
        q, k, v = n.inputs
        (qb, qs, qd), (kb, ks, kd), (vb, vs, vd) = p["q_dims"], p["k_dims"], p["v_dims"]
        ql, kl, vl = loc[q], loc[k], loc[v]
        qt = g.types[q]
        a.batch, a.heads = qt.shape[qb[0]], qt.shape[qb[1]]
        a.kv_heads = g.types[k].shape[kb[1]]
        a.sq, a.sk, a.head_dim = qt.shape[qs], g.types[k].shape[ks], qt.shape[qd]
        a.value_head_dim = g.types[v].shape[vd]
        a.dtype = 1 if qt.dtype == "bfloat16" else 2
        _need_unit(ql, qd, kl, kd, vl, vd)
        a.q_b, a.q_n, a.q_s = ql.strides[qb[0]], ql.strides[qb[1]], ql.strides[qs]
        a.k_b, a.k_n, a.k_s = kl.strides[kb[0]], kl.strides[kb[1]], kl.strides[ks]
        a.v_b, a.v_n, a.v_s = vl.strides[vb[0]], vl.strides[vb[1]], vl.strides[vs]
        ol = loc[step.outputs[0]]  # [B, N, Sq, D]
        a.o_b, a.o_n, a.o_s = ol.strides[0], ol.strides[1], ol.strides[2]
        if len(step.outputs) > 1:
            lse = loc[step.outputs[1]]
        else:
            lse = plan.scratch[id(step)]
        return nv.NHIP_STEP_FLASH_FWD, a, [ql, kl, vl, ol, lse]
    q, k, v, o, do, lse = n.inputs
    qt, kt = g.types[q], g.types[k]
    ls = {x: loc[x] for x in (q, k, v, o, do, lse)}
    a.batch, a.sq, a.heads, a.head_dim = qt.shape
    a.sk, a.kv_heads = kt.shape[1], kt.shape[2]
    a.value_head_dim = g.types[v].shape[3]
    a.dtype = 1 if qt.dtype == "bfloat16" else 2
    for name, x in (("q", q), ("k", k), ("v", v), ("o", o), ("do", do)):
        l_ = ls[x]
        if l_.strides[3] != 1:
            raise NotImplementedError("flash attention backward: head dim must be contiguous")
        setattr(a, f"{name}_b", l_.strides[0])
        setattr(a, f"{name}_s", l_.strides[1])
        setattr(a, f"{name}_n", l_.strides[2])
    outs = [loc[v_] for v_ in step.outputs[:3]]
    for name, l_ in zip(("dq", "dk", "dv"), outs):
        setattr(a, f"{name}_b", l_.strides[0])
        setattr(a, f"{name}_s", l_.strides[1])
        setattr(a, f"{name}_n", l_.strides[2])
    ws = plan.scratch[id(step)]
    return nv.NHIP_STEP_FLASH_BWD, a, [ls[q], ls[k], ls[v], ls[o], ls[do], ls[lse], outs[0], outs[1], outs[2], ws]


def _need_unit(*pairs):
    for loc, d in zip(pairs[::2], pairs[1::2]):
        if loc.strides[d] != 1:
            raise NotImplementedError("flash attention: the head dim of every operand must be contiguous")


_ = (Node, TensorType)


def backward_mode(batch=0, heads=0, sq=0, sk=0) -> int:
    """The flash backward's dQ mode (nhip_attn_desc.deterministic): 0 added atomically by the dK/dV kernel,
    1 from the dS tiles the dK/dV kernel stores, 2 by a kernel recomputing S and dP.

    Mode 1's dS tiles grow with Sq x Sk (2 GiB an attention at B 4, N 16, S 4096), so a shape whose tiles
    would exceed ``config.compiler.attention_ds_max_bytes`` (or an eighth of a set ``memory_limit``) takes
    mode 2, whose workspace is two floats a query row, as the reference's recomputing backward is."""
    from lumen_amd.config import config

    if not config.compiler.deterministic:
        return 0
    if not config.compiler.attention_store_ds:
        return 2
    cap = config.compiler.attention_ds_max_bytes
    if config.compiler.memory_limit:
        cap = min(cap, config.compiler.memory_limit // 8)
    return 2 if ds_bytes(batch, heads, sq, sk) > cap else 1


def ds_bytes(batch, heads, sq, sk) -> int:
    """Bytes of mode 1's 16-bit dS tiles, 128 keys x 64 queries each (attention.h flash_bwd_ds_bytes)."""
    return batch * heads * (-(-sk // 128)) * (-(-sq // 64)) * 128 * 64 * 2


def backward_workspace_bytes(b, nh, sq, sk, hd, kvh, mode, hdv=0) -> int:
    """Workspace bytes of nhip_flash_bwd for these sizes and mode, as the library itself reports them
    (nhip_flash_bwd_workspace), so the plan's scratch can never be smaller than what the kernels write."""
    import ctypes as C

    from lumen_amd import native as nv

    a = nv.AttnDesc()
    a.batch, a.sq, a.sk, a.heads, a.kv_heads, a.head_dim = b, sq, sk, nh, kvh, hd
    a.value_head_dim = hdv
    a.deterministic = mode
    n = C.c_size_t()
    nv.call("nhip_flash_bwd_workspace", C.byref(a), C.byref(n))
    return n.value
