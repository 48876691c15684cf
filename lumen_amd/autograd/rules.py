"""Reverse-mode rules: each differentiable primitive's cotangents of its operands given its result's.

Each rule is the composition of the reference's JVP rule and its transpose (``lumen/autograd/rules.py``), so
the backward graph computes the same primitives in the same order: ``mul``'s transpose multiplies by the
other operand, ``div`` by the reciprocal rule ``-(out / y)``, ``cast`` narrows or widens back (reusing the
wider value a narrowing cast came from, ``rules.py:22-68``), ``dot_general`` is JAX's
``_dot_general_transpose_lhs`` (``rules.py:428-489``), ``gather`` scatter-adds into a float32 accumulator.
"""

from __future__ import annotations

from lumen_amd.graph import prims as P
from lumen_amd.graph import tracer
from lumen_amd.graph.tracer import TracedTensor, accum_dtype, dot

RULES = {}


def _value(var):
    return TracedTensor(tracer.current_graph(), var)


def _full(like, value):
    from lumen_amd import dtypes as D

    return P.full(like.shape, float(value) if D.is_float(like.dtype) else int(value), like.dtype)


def rule(name):
    def deco(f):
        RULES[name] = f
        return f

    return deco


@rule("add")
def _add(ct, out, x, y, need, **p):
    return [ct if need[0] else None, ct if need[1] else None]


@rule("sub")
def _sub(ct, out, x, y, need, **p):
    return [ct if need[0] else None, P.neg(ct) if need[1] else None]


@rule("neg")
def _neg(ct, out, x, need, **p):
    return [P.neg(ct)]


@rule("mul")
def _mul(ct, out, x, y, need, **p):
    return [P.mul(ct, y) if need[0] else None, P.mul(x, ct) if need[1] else None]


@rule("div")
def _div(ct, out, x, y, need, **p):
    return [P.div(ct, y) if need[0] else None, P.mul(ct, P.neg(P.div(out, y))) if need[1] else None]


def _max_share(x, y):
    """1 where ``x`` is the max, 0.5 where tied (JAX's balanced share), else 0 (``rules.py:404-407``)."""
    one, half, zero = _full(x, 1), _full(x, 0.5), _full(x, 0)
    return P.select(P.lt(y, x), one, P.select(P.eq(x, y), half, zero))


@rule("max")
def _max(ct, out, x, y, need, **p):
    return [P.mul(ct, _max_share(x, y)) if need[0] else None, P.mul(ct, _max_share(y, x)) if need[1] else None]


@rule("exp")
def _exp(ct, out, x, need, **p):
    return [P.mul(ct, out)]


@rule("log")
def _log(ct, out, x, need, **p):
    return [P.div(ct, x)]


@rule("sqrt")
def _sqrt(ct, out, x, need, **p):
    return [P.div(ct, P.add(out, out))]


@rule("tanh")
def _tanh(ct, out, x, need, **p):
    return [P.mul(ct, P.sub(_full(out, 1), P.mul(out, out)))]


@rule("logistic")
def _logistic(ct, out, x, need, **p):
    return [P.mul(ct, P.mul(out, P.sub(_full(out, 1), out)))]


def _widened(var, dtype):
    """The ``dtype`` value a narrowing cast of ``var`` came from, through transposes and sums; or None."""
    node = tracer.producer(var)
    if node is None:
        return None
    name, ins, p = node
    if name == "transpose":
        inner = _widened(ins[0], dtype)
        return None if inner is None else P.transpose(inner, p["permutation"])
    if name == "add":
        a, b = (_widened(i, dtype) for i in ins)
        return None if a is None or b is None else P.add(a, b)
    if name == "cast" and tracer.current_graph().type_of(ins[0]).dtype == dtype:
        return _value(ins[0])
    return None


def _dot_tangent(var):
    node = tracer.producer(var) if var is not None else None
    if node is None or node[0] not in ("dot_general", "add"):
        return False
    return node[0] == "dot_general" or all((tracer.producer(v) or ("",))[0] == "dot_general" for v in node[1])


@rule("cast")
def _cast(ct, out, x, need, **p):
    """``ct`` back in ``x``'s dtype; a gradient dot rounded to a narrower dtype only for this is read at its
    accumulator instead (``rules.py:44-56``)."""
    if ct.dtype == x.dtype:
        return [ct]
    widened = _widened(ct.var, x.dtype) if not _dot_tangent(ct.var) else None
    return [P.cast(ct, x.dtype) if widened is None else widened]


@rule("reshape")
def _reshape(ct, out, x, need, **p):
    return [P.reshape(ct, x.shape)]


@rule("transpose")
def _transpose(ct, out, x, need, permutation, **p):
    inverse = sorted(range(len(permutation)), key=permutation.__getitem__)
    return [P.transpose(ct, inverse)]


@rule("swap_pairs")
def _swap(ct, out, x, need, **p):
    return [P.swap_pairs(ct)]


@rule("reduce_sum")
def _reduce_sum(ct, out, x, need, axes, **p):
    ct = P.cast(ct, x.dtype) if ct.dtype != x.dtype else ct
    kept = [d for d in range(x.ndim) if d not in axes]
    return [P.broadcast_in_dim(ct, x.shape, kept)]


@rule("broadcast_in_dim")
def _broadcast_in_dim(ct, out, x, need, shape, broadcast_dimensions, **p):
    dims = broadcast_dimensions
    stretched = [dims[i] for i, n in enumerate(x.shape) if n == 1 and shape[dims[i]] != 1]
    axes = sorted([d for d in range(len(shape)) if d not in dims] + stretched)
    if axes:
        ct = P.reduce_sum(ct, axes, accum_dtype(ct.dtype))
        ct = P.cast(ct, x.dtype) if ct.dtype != x.dtype else ct
    return [P.reshape(ct, x.shape) if ct.shape != x.shape else ct]


@rule("reduce_max")
def _reduce_max(ct, out, x, need, axes, **p):
    """The tangent averaged over positions equal to the max, transposed (``rules.py:420-425``)."""
    kept = [d for d in range(x.ndim) if d not in axes]
    where = P.cast(P.eq(x, P.broadcast_in_dim(out, x.shape, kept)), x.dtype)
    count = P.reduce_sum(where, axes, x.dtype)
    c = P.div(ct, count)
    c = P.broadcast_in_dim(c, x.shape, kept)
    return [P.mul(c, where)]


@rule("select")
def _select(ct, out, pred, x, y, need, **p):
    zeros = _full(ct, 0)
    return [None, P.select(pred, ct, zeros) if need[1] else None, P.select(pred, zeros, ct) if need[2] else None]


@rule("slice")
def _slice(ct, out, x, need, start_indices, limit_indices, **p):
    for d, (start, limit) in enumerate(zip(start_indices, limit_indices)):
        parts = []
        for size in (start, x.shape[d] - limit):
            shape = list(ct.shape)
            shape[d] = size
            parts.append(P.full(shape, 0.0, ct.dtype) if size else None)
        ops = [q for q in (parts[0], ct, parts[1]) if q is not None]
        ct = P.concatenate(ops, d) if len(ops) > 1 else ct
    return [ct]


@rule("concatenate")
def _concatenate(ct, out, *args, need, dimension, **p):
    cts, offset = [], 0
    for x, nd in zip(args, need):
        size = x.shape[dimension]
        if nd:
            start, limit = [0] * ct.ndim, list(ct.shape)
            start[dimension], limit[dimension] = offset, offset + size
            cts.append(P.slice(ct, start, limit))
        else:
            cts.append(None)
        offset += size
    return cts


@rule("gather")
def _gather(ct, out, x, indices, need, axis, **p):
    acc = accum_dtype(x.dtype)
    ct = ct if ct.dtype == acc else P.cast(ct, acc)
    o = P.scatter_add(P.full(x.shape, 0, acc), indices, ct, axis)
    return [o if acc == x.dtype else P.cast(o, x.dtype), None]


@rule("scatter_add")
def _scatter_add(ct, out, x, indices, updates, need, axis, **p):
    return [ct if need[0] else None, None, P.gather(ct, indices, axis) if need[2] else None]


@rule("dynamic_slice")
def _dynamic_slice(ct, out, x, *indices, need, slice_sizes, **p):
    return [P.dynamic_update_slice(_full(x, 0), ct, list(indices))] + [None] * len(indices)


@rule("dynamic_update_slice")
def _dynamic_update_slice(ct, out, x, update, *indices, need, **p):
    return [
        P.dynamic_update_slice(ct, _full(update, 0), list(indices)) if need[0] else None,
        P.dynamic_slice(ct, list(indices), update.shape) if need[1] else None,
    ] + [None] * len(indices)


@rule("cumsum")
def _cumsum(ct, out, x, need, axis, reverse, **p):
    c = P.cumsum(ct, axis, not reverse, ct.dtype)
    return [P.cast(c, x.dtype) if c.dtype != x.dtype else c]


def _narrowed(ct, dtype):
    """``ct`` in ``dtype``: the value a widening cast made it from, else a cast (``rules.py:442-451``)."""
    if ct.dtype == dtype:
        return ct
    node = tracer.producer(ct.var)
    if node is not None and node[0] == "cast" and tracer.current_graph().type_of(node[1][0]).dtype == dtype:
        return _value(node[1][0])
    return P.cast(ct, dtype)


def _ranges_like(*xs):
    start = 0
    for x in xs:
        yield list(range(start, start + len(x)))
        start += len(x)


def _dot_transpose_lhs(ct, x, y, dims, acc, swap_ans=False):
    (x_contract, y_contract), (x_batch, y_batch) = dims
    x_kept = [d for d in range(x.ndim) if d not in x_contract and d not in x_batch]
    y_kept = [d for d in range(y.ndim) if d not in y_contract and d not in y_batch]
    if swap_ans:
        ans_batch, ans_y, _ = _ranges_like(x_batch, y_kept, x_kept)
    else:
        ans_batch, _, ans_y = _ranges_like(x_batch, x_kept, y_kept)
    order = sorted(range(len(y_contract)), key=lambda i: y_contract[i])
    unsorted = list(x_batch) + x_kept + [x_contract[i] for i in order]
    out_axes = sorted(range(len(unsorted)), key=unsorted.__getitem__)
    ct = _narrowed(ct, y.dtype)
    x_bar = dot(ct, y, ((ans_y, y_kept), (ans_batch, y_batch)), acc, x.dtype)
    return x_bar if out_axes == list(range(len(out_axes))) else P.transpose(x_bar, out_axes)


@rule("dot_general")
def _dot_general(ct, out, x, y, need, lhs_contracting, rhs_contracting, lhs_batch, rhs_batch, accum_dtype, **p):
    xc, yc, xb, yb = lhs_contracting, rhs_contracting, lhs_batch, rhs_batch
    gx = _dot_transpose_lhs(ct, x, y, ((xc, yc), (xb, yb)), accum_dtype) if need[0] else None
    gy = _dot_transpose_lhs(ct, y, x, ((yc, xc), (yb, xb)), accum_dtype, swap_ans=True) if need[1] else None
    return [gx, gy]


# Primitives whose results carry no gradient (comparisons, integer and index producers).
NON_DIFFERENTIABLE = {"eq", "lt", "iota", "full", "random_bits", "is_finite", "not", "and", "or", "xor", "floor",
                      "ceil", "round", "sign"}
