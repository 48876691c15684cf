"""Unreduced cross entropy on logits with a log-sum-exp gradient (``lumen/functional/cross_entropy/logits.py``)."""

from __future__ import annotations

import math

from lumen_amd.autograd.function import Function
from lumen_amd.functional.functions import amax, eq, exp, log, sum
from lumen_amd.graph import prims
from lumen_amd.graph.tracer import lift, require_float


def one_hot(target, n, dtype):
    """``target``'s classes of ``n`` as ``dtype`` rows of zeros and a one (``cross_entropy/utils.py``)."""
    hit = eq(target.reshape(*target.shape, 1), prims.iota(target.dtype, [n], 0))
    return prims.cast(hit, dtype)


class _CrossEntropy(Function):
    """Per-row ``logsumexp(x) - x[target]``, differentiated from the saved logsumexp (``logits.py:13-36``)."""

    @staticmethod
    def forward(ctx, x, target):
        m = amax(x, -1, keepdim=True)
        lse = m.reshape(*target.shape) + log(sum(exp(x - m), -1))
        ctx.save_for_backward(x, target, lse)
        rows, n = math.prod(target.shape), x.shape[-1]
        at = prims.iota(target.dtype, [rows], 0) * n + target.reshape(rows)
        return lse - prims.gather(x.reshape(rows * n), at, 0).reshape(*target.shape)

    @staticmethod
    def backward(ctx, g):
        x, target, lse = ctx.saved_tensors
        p = exp(x - lse.reshape(*target.shape, 1))
        return (p - one_hot(target, x.shape[-1], x.dtype)) * g.reshape(*target.shape, 1), None


def cross_entropy(input, target):
    """``torch.nn.functional.cross_entropy(input, target, reduction="none")`` over the last dimension
    (``logits.py:39-52``)."""
    x = require_float(lift(input), "cross_entropy")
    target = lift(target)
    if tuple(target.shape) != tuple(x.shape[:-1]):
        raise ValueError(f"cross_entropy: target of shape {target.shape} for input of shape {x.shape}")
    return _CrossEntropy.apply(x, target)
