"""User-defined differentiable operations (``lumen/autograd/function.py``'s interface).

A ``Function`` subclass writes a static ``forward(ctx, ...)`` in traced ops and a static
``backward(ctx, *output_cotangents)``. ``apply`` runs ``forward`` with taping paused, so its inner ops are not
differentiated one by one, and appends one ``FunctionCall`` record to every active tape; reverse mode later
calls ``backward`` on that record instead of the inner ops' rules.

``backward`` may return the positional arguments' gradients in order, a dict of gradients by parameter name
(keyword-only parameters included), or the leading positional gradients followed by such a dict; a None, or
an argument left out, has no gradient.
"""

from __future__ import annotations

import contextlib
import inspect
from dataclasses import dataclass

from lumen_amd.graph import tracer
from lumen_amd.graph.tracer import TracedTensor

FUNCTION = "autograd.Function"  # the tape entry name of a FunctionCall


class FunctionCtx:
    """Scratch state one ``apply`` shares between its ``forward`` and ``backward``."""

    def save_for_backward(self, *tensors, **named):
        self.saved_tensors = tensors
        self.saved_named_tensors = named


@contextlib.contextmanager
def _taping_paused():
    """Detaches the active tapes for the duration (yielding them) and restores them after."""
    active = list(tracer._TAPES)
    del tracer._TAPES[:]
    try:
        yield active
    finally:
        tracer._TAPES[:] = active


@dataclass
class FunctionCall:
    """One recorded ``Function.apply``: the subclass, its context and its arguments, each keyed by position
    (an int) or by keyword (a str); the first ``positional`` of them were positional."""

    function: type
    ctx: FunctionCtx
    arguments: list
    positional: int

    def traced_inputs(self) -> tuple:
        return tuple(value.var for _, value in self.arguments if isinstance(value, TracedTensor))

    def argument_gradients(self, returned) -> list:
        """What ``backward`` returned, as one gradient (or None) per argument, in argument order."""
        name = self.function.__name__
        if isinstance(returned, dict):
            leading, by_name = (), dict(returned)
        else:
            seq = tuple(returned) if isinstance(returned, (tuple, list)) else (returned,)
            trailing_dict = bool(seq) and isinstance(seq[-1], dict)
            leading, by_name = (seq[:-1], dict(seq[-1])) if trailing_dict else (seq, {})
        if len(leading) > self.positional or (not by_name and len(leading) != self.positional):
            raise ValueError(f"{name}.backward returned {len(leading)} gradients for {self.positional} positional "
                             "arguments")
        grads = dict(enumerate(leading))
        params = list(inspect.signature(self.function.forward).parameters)[1:]
        keys = {key for key, _ in self.arguments}
        for pname, g in by_name.items():
            key = params.index(pname) if pname in params[: self.positional] else pname
            if key not in keys:
                raise ValueError(f"{name}.backward returned a gradient for {pname!r}, which is not an argument")
            grads[key] = g
        return [grads.get(key) for key, _ in self.arguments]


def _bind(forward, args, kwargs):
    """``forward``'s arguments after binding (defaults filled in): ``[(key, value)]`` and the positional count."""
    bound = inspect.signature(forward).bind(None, *args, **kwargs)
    bound.apply_defaults()
    positional = list(bound.args[1:])
    return list(enumerate(positional)) + list(bound.kwargs.items()), len(positional)


class Function:
    """Base class of an op with a hand-written derivative (static ``forward`` and ``backward``)."""

    @staticmethod
    def forward(ctx, *args):
        raise NotImplementedError("a Function defines forward(ctx, *args)")

    @staticmethod
    def backward(ctx, *grads):
        raise NotImplementedError("a Function defines backward(ctx, *grads) for reverse mode")

    @classmethod
    def apply(cls, *args, **kwargs):
        tracer.current_graph()  # fails outside a trace
        arguments, npos = _bind(cls.forward, args, kwargs)
        call = FunctionCall(cls, FunctionCtx(), arguments, npos)
        with _taping_paused() as tapes:
            out = cls.forward(call.ctx, *(v for _, v in arguments[:npos]), **dict(arguments[npos:]))
        results = (out,) if isinstance(out, TracedTensor) else tuple(out)
        if not results or any(not isinstance(r, TracedTensor) for r in results):
            raise TypeError(f"{cls.__name__}.forward returns a tensor or a tuple of tensors, not {out!r}")
        entry = (FUNCTION, call.traced_inputs(), call, tuple(r.var for r in results))
        for tape in tapes:
            tape.append(entry)
        return out
