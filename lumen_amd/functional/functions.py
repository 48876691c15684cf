"""Functional tensor operations traced into primitives (``lumen/functional/functions.py``)."""

from __future__ import annotations

import builtins
import math

from lumen_amd import dtypes as D
from lumen_amd.autograd.function import Function
from lumen_amd.graph import prims
from lumen_amd.graph.tracer import (
    TracedTensor,
    accum_dtype,
    broadcast_shapes,
    broadcast_to,
    common_dtype,
    dim_of,
    dims_of,
    dot,
    elementwise,
    ge,
    gt,
    le,
    lift,
    minimum as _min,
    ne,
    require_float,
    true_div,
)


def add(input, other):
    return elementwise(prims.add, input, other)


def sub(input, other):
    return elementwise(prims.sub, input, other)


def mul(input, other):
    return elementwise(prims.mul, input, other)


def div(input, other):
    return true_div(input, other)


def neg(input):
    return prims.neg(lift(input))


def eq(input, other):
    return elementwise(prims.eq, input, other)


def lt(input, other):
    return elementwise(prims.lt, input, other)


def maximum(input, other):
    return elementwise(prims.max, input, other)


def minimum(input, other):
    return elementwise(_min, input, other)


def where(condition, input, other):
    """``input`` where ``condition`` holds, else ``other`` (scalars take the other's dtype)."""
    cond = lift(condition)
    dtype = common_dtype("where", (input, other))
    from lumen_amd.graph.tracer import as_tensor

    x, y = as_tensor(input, dtype, "where"), as_tensor(other, dtype, "where")
    shape = broadcast_shapes(cond.shape, x.shape, y.shape)
    return prims.select(broadcast_to(cond, shape), broadcast_to(x, shape), broadcast_to(y, shape))


def exp(input):
    return prims.exp(require_float(lift(input), "exp"))


def log(input):
    return prims.log(require_float(lift(input), "log"))


def sqrt(input):
    return prims.sqrt(require_float(lift(input), "sqrt"))


def rsqrt(input):
    return prims.rsqrt(require_float(lift(input), "rsqrt"))


def tanh(input):
    return prims.tanh(require_float(lift(input), "tanh"))


def sigmoid(input):
    return prims.logistic(require_float(lift(input), "sigmoid"))


def relu(input):
    """``max(input, 0)`` (``functions.py:224``)."""
    return elementwise(prims.max, input, 0)


def gelu(input, approximate="tanh"):
    """GELU's tanh approximation written out with ``tanh`` (as ``dashboard/bench.py:246-248``): the
    primitive set has no erf, so only ``approximate="tanh"`` exists."""
    if approximate != "tanh":
        raise NotImplementedError("gelu: only approximate='tanh' (there is no erf primitive)")
    x = require_float(lift(input), "gelu")
    return 0.5 * x * (1.0 + tanh(0.7978845608 * (x + 0.044715 * x * x * x)))


def _keep(input, out, dims, keepdim):
    if not keepdim:
        return out
    return out.reshape(tuple(1 if d in dims else n for d, n in enumerate(input.shape)))


def sum(input, dim=None, keepdim=False):
    """Sum over ``dim`` accumulated in the tensor's dtype (``functions.py:265``)."""
    input = lift(input)
    dims = dims_of(dim, input.ndim)
    return _keep(input, prims.reduce_sum(input, dims, input.dtype), dims, keepdim)


def mean(input, dim=None, keepdim=False):
    input = lift(input)
    if not D.is_float(input.dtype):
        raise RuntimeError(f"mean(): input dtype must be floating point, got {input.dtype}")
    dims = dims_of(dim, input.ndim)
    count = math.prod(input.shape[d] for d in dims)
    return sum(input, dims, keepdim) / count


def amax(input, dim=(), keepdim=False):
    input = lift(input)
    dims = dims_of(dim, input.ndim)
    return _keep(input, prims.reduce_max(input, dims), dims, keepdim)


def max(input, other=None):
    if other is None:
        return amax(input)
    return maximum(input, other)


def softmax(input, dim):
    """``exp(x - max) / sum(exp(x - max))`` along ``dim`` (``functions.py:315-323``)."""
    x = require_float(lift(input), "softmax")
    e = exp(x - amax(x, dim, keepdim=True))
    return e / sum(e, dim, keepdim=True)


def log_softmax(input, dim):
    x = require_float(lift(input), "log_softmax")
    shifted = x - amax(x, dim, keepdim=True)
    return shifted - log(sum(exp(shifted), dim, keepdim=True))


class _RMSNorm(Function):
    """``rms_norm`` differentiated from each row's saved ``1 / rms`` (``functions.py:334-373``)."""

    @staticmethod
    def forward(ctx, x, weight, eps):
        h = x.to(accum_dtype(x.dtype))
        inv = prims.rsqrt(mean(h * h, -1, keepdim=True) + eps)
        ctx.save_for_backward(x, weight, inv)
        y = (h * inv).to(x.dtype)
        return y if weight is None else y * weight

    @staticmethod
    def backward(ctx, g):
        x, weight, inv = ctx.saved_tensors
        acc = accum_dtype(x.dtype)
        h = x.to(acc)
        d = (g if weight is None else g * weight).to(acc)
        dx = (d * inv - h * (((mean(d * h, -1, keepdim=True) * inv) * inv) * inv)).to(x.dtype)
        if weight is None:
            return dx, None, None
        rows = tuple(range(x.ndim - 1))
        dw = sum((g.to(acc) * inv) * h, rows).to(weight.dtype)
        return dx, dw, None


def rms_norm(input, normalized_shape, weight=None, eps=None):
    """``input * rsqrt(mean(input^2) + eps)`` over the last dimension, times ``weight`` (``functions.py:376``);
    ``eps`` defaults to the dtype's machine epsilon."""
    x = require_float(lift(input), "rms_norm")
    shape = [normalized_shape] if isinstance(normalized_shape, int) else list(normalized_shape)
    if shape != list(x.shape[-1:]):
        raise NotImplementedError(f"rms_norm normalizes the last dimension, of size {list(x.shape[-1:])}, got {shape}")
    weight = lift(weight)
    if weight is not None and (weight.dtype != x.dtype or list(weight.shape) != shape):
        raise TypeError(f"rms_norm: weight must be {x.dtype}{shape}, got {weight.dtype}{list(weight.shape)}")
    if eps is None:
        eps = {"float16": 2.0**-10, "bfloat16": 2.0**-7, "float64": 2.0**-52}.get(x.dtype, 2.0**-23)
    return _RMSNorm.apply(x, weight, eps)


def layer_norm(input, normalized_shape, weight=None, bias=None, eps=1e-5):
    """Layer norm over the last dimension, written out in primitives (as
    ``tests/graph_compiler/test_normalizations.py:103-106``): centered, divided by the root of the variance
    plus ``eps``, then scaled and shifted."""
    x = require_float(lift(input), "layer_norm")
    xc = x - mean(x, -1, keepdim=True)
    y = xc / sqrt(mean(xc * xc, -1, keepdim=True) + eps)
    if weight is not None:
        y = y * weight
    if bias is not None:
        y = y + bias
    return y


def matmul(input, other, accum_dtype, output_dtype):
    """``input @ other`` with torch's rules, accumulated in ``accum_dtype`` with result ``output_dtype``
    (``functions.py:410-448``)."""
    input, other = lift(input), lift(other)
    common_dtype("matmul", (input, other))
    accum_dtype, output_dtype = D.canonical(accum_dtype), D.canonical(output_dtype)
    if input.ndim == 0 or other.ndim == 0:
        raise RuntimeError("both arguments to matmul need to be at least 1D")
    if input.ndim > 2 and other.ndim == 2:
        k = input.shape[-1]
        rows = input.reshape(math.prod(input.shape[:-1]), k)
        out = dot(rows, other, (((1,), (0,)), ((), ())), accum_dtype, output_dtype)
        return out.reshape(*input.shape[:-1], other.shape[-1])
    x = input.unsqueeze(0) if input.ndim == 1 else input
    y = other.unsqueeze(-1) if other.ndim == 1 else other
    batch = broadcast_shapes(x.shape[:-2], y.shape[:-2])
    x, y = broadcast_to(x, batch + x.shape[-2:]), broadcast_to(y, batch + y.shape[-2:])
    b = tuple(range(len(batch)))
    out = dot(x, y, (((len(b) + 1,), (len(b),)), (b, b)), accum_dtype, output_dtype)
    if input.ndim == 1:
        out = out.squeeze(-2)
    if other.ndim == 1:
        out = out.squeeze(-1)
    return out


def square(input):
    x = lift(input)
    return x * x


def reciprocal(input):
    return true_div(1.0, lift(input))


def clamp(input, min=None, max=None):
    x = lift(input)
    if min is not None:
        x = maximum(x, min)
    if max is not None:
        x = minimum(x, max)
    return x


def cat(tensors, dim=0):
    tensors = [lift(t) for t in tensors]
    return prims.concatenate(tensors, dim_of(dim, tensors[0].ndim))


def stack(tensors, dim=0):
    tensors = [lift(t) for t in tensors]
    d = dim_of(dim, tensors[0].ndim + 1)
    return cat([t.unsqueeze(d) for t in tensors], d)


def _order_flip(x):
    """Reverses the order of ``x``'s values bijectively: negation, or bitwise not for unsigned and bool
    (whose negation would not reverse their order)."""
    if x.dtype == "bool" or x.dtype.startswith("uint"):
        return prims.not_(x)
    return prims.neg(x)


def amin(input, dim=(), keepdim=False):
    """Minimum over ``dim`` (every axis if empty), as the order-flipped maximum of the order-flipped values
    (``functions.py:581-592``; the graph has no separate minimum reduction)."""
    x = lift(input)
    return _order_flip(amax(_order_flip(x), dim, keepdim))


def _first_index(x, dim, keepdim, best):
    """Smallest position along ``dim`` at which ``x`` equals ``best`` over that axis, int32
    (``functions.py:613-626``). Positions not attaining it are replaced by the axis length, so the minimum of
    the candidates is the first hit; a NaN maximum compares unequal everywhere, giving the axis length."""
    if dim is None:
        return _first_index(x.reshape((-1,)), 0, False, best)
    d = dim_of(dim, x.ndim)
    hit = prims.eq(x, broadcast_to(best(x, d, keepdim=True), x.shape))
    pos = prims.iota("int32", x.shape, d)
    miss = prims.full(x.shape, x.shape[d], "int32")
    return amin(prims.select(hit, pos, miss), d, keepdim)


def argmax(input, dim=None, keepdim=False):
    """Index of the first maximum over ``dim`` (over every element when None), int32."""
    return _first_index(lift(input), dim, keepdim, amax)


def argmin(input, dim=None, keepdim=False):
    """Index of the first minimum over ``dim`` (over every element when None), int32."""
    return _first_index(lift(input), dim, keepdim, amin)


__all__ = [n for n in dir() if not n.startswith("_") and n not in ("builtins", "math", "D", "Function", "prims")]
_ = (builtins, ge, gt, le, ne, TracedTensor)
