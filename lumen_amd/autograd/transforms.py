"""Reverse-mode differentiation over the nodes recorded while tracing (``lumen/autograd/transforms.py``).

``backward`` walks the tape backwards from the output's cotangent, applying each node's rule
(``rules.RULES``) or a ``Function``'s ``backward``, and accumulates cotangents with ``add`` in tape order, as
``backward_pass`` does (``transforms.py:180-205``). Nodes it adds are marked as gradient nodes.
"""

from __future__ import annotations

import functools

from lumen_amd import dtypes as D
from lumen_amd.autograd import cross_entropy
from lumen_amd.autograd.function import FUNCTION
from lumen_amd.autograd.rules import NON_DIFFERENTIABLE, RULES
from lumen_amd.graph import prims as P
from lumen_amd.graph import tracer
from lumen_amd.graph.tracer import TracedTensor


def _value(var):
    return TracedTensor(tracer.current_graph(), var)


def _accumulate(cts, v, c):
    cts[v] = c if v not in cts else P.add(cts[v], c)


def backward(out, ct, tape, leaves):
    """The gradient of each of ``leaves`` (None where ``out`` does not depend on it) for cotangent ``ct``."""
    if (ct.dtype, tuple(ct.shape)) != (out.dtype, tuple(out.shape)):
        raise TypeError(f"backward: a gradient must have its value's type, got {ct.dtype}{list(ct.shape)} for {out!r}")
    graph = tracer.current_graph()
    tape = cross_entropy.substitute(tape)
    # Values that depend on a float leaf: only their nodes are differentiated.
    live = {p.var for p in leaves if D.is_float(p.dtype)}
    linear = []
    for node in tape:
        name, inputs, params, outv = node
        if any(v in live for v in inputs):
            outs = outv if name == FUNCTION else (outv,)
            if name != FUNCTION and (name in NON_DIFFERENTIABLE or not D.is_float(graph.type_of(outv).dtype)):
                continue
            live.update(outs)
            linear.append(node)
    if out.var not in live:
        return [None for _ in leaves]
    cts = {out.var: ct}
    saved = graph.backward
    graph.backward = True
    try:
        for name, inputs, params, outv in reversed(linear):
            if name == FUNCTION:
                _function_transpose(params, outv, cts, live)
                continue
            c = cts.pop(outv, None)
            if c is None:
                continue
            if name not in RULES:
                raise NotImplementedError(f"{name} has no gradient rule")
            need = [v in live for v in inputs]
            args = [_value(v) for v in inputs]
            grads = RULES[name](c, _value(outv), *args, need=need, **params)
            for v, g, nd in zip(inputs, grads, need):
                if g is not None and nd:
                    _accumulate(cts, v, g)
    finally:
        graph.backward = saved
    return [cts.get(p.var) if D.is_float(p.dtype) else None for p in leaves]


def _function_transpose(call, outs, cts, live):
    """A recorded ``FunctionCall`` in reverse: its ``backward`` on the outputs' cotangents (zeros for outputs
    without one), each gradient accumulated into its argument when that argument is differentiated."""
    cs = [cts.pop(o, None) for o in outs]
    if all(c is None for c in cs):
        return
    filled = [c if c is not None else _zeros(o) for c, o in zip(cs, outs)]
    returned = call.function.backward(call.ctx, *filled)
    for (_, v), g in zip(call.arguments, call.argument_gradients(returned)):
        if not (isinstance(v, TracedTensor) and g is not None and v.var in live):
            continue
        if (g.dtype, tuple(g.shape)) != (v.dtype, tuple(v.shape)):
            raise TypeError(f"{call.function.__name__}.backward: a {g.dtype}{list(g.shape)} gradient for a "
                            f"{v.dtype}{list(v.shape)} argument")
        _accumulate(cts, v.var, g)


def _zeros(var):
    ty = tracer.current_graph().type_of(var)
    return P.full(ty.shape, 0.0, ty.dtype)


def vjp(fn, *primals):
    """``fn(*primals)`` and a function from its cotangent to the primals' (``jax.vjp``)."""
    tape = []
    tracer._TAPES.append(tape)
    try:
        out = fn(*primals)
    finally:
        tracer._TAPES.pop()
    leaves = [p for p in primals if isinstance(p, TracedTensor)]

    def pullback(ct):
        return tuple(backward(out, ct, tape, leaves))

    return out, pullback


def value_and_grad(fn, argnums=0):
    def value_and_grad_fn(*args):
        nums = (argnums,) if isinstance(argnums, int) else tuple(argnums)

        def f(*diff):
            full = list(args)
            for i, d in zip(nums, diff):
                full[i] = d
            return fn(*full)

        out, pullback = vjp(f, *(args[i] for i in nums))
        if not isinstance(out, TracedTensor) or out.shape != () or not D.is_float(out.dtype):
            raise TypeError(f"grad: fn must return a float scalar, got {out!r}")
        grads = pullback(P.full((), 1.0, out.dtype))
        grads = tuple(g if g is not None else _zeros(a.var) for g, a in zip(grads, (args[i] for i in nums)))
        return out, grads[0] if isinstance(argnums, int) else grads

    return value_and_grad_fn


def grad(fn, argnums=0):
    vg = value_and_grad(fn, argnums)

    @functools.wraps(fn)
    def grad_fn(*args):
        return vg(*args)[1]

    return grad_fn
