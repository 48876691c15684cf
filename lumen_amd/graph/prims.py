"""Python wrappers that record each primitive into the graph being traced (``lumen/graph/prims.py``).

``bind`` checks the operands are traced values of the current trace, applies the primitive (type inference
in ``ir.infer``), records it on the autograd tapes and returns the result as a ``TracedTensor``.
"""

from __future__ import annotations

from lumen_amd import dtypes as D
from lumen_amd.graph import tracer


def bind(name, *operands, **params):
    """Records ``name(*operands, **params)`` in the graph being traced (``prims.py:103``)."""
    graph = tracer.current_graph()
    for x in operands:
        if not isinstance(x, tracer.TracedTensor) or x.graph is not graph:
            raise TypeError(f"{name}: operands must be traced tensors of the current trace, got {x!r}")
    inputs = [x.var for x in operands]
    var = graph.apply(name, inputs, params)
    tracer.record(name, inputs, params, var)
    out = tracer.TracedTensor(graph, var)
    out.weak = len(operands) == 1 and operands[0].weak and graph.type_of(var) == graph.type_of(inputs[0])
    return out


def add(x, y):
    return bind("add", x, y)


def sub(x, y):
    return bind("sub", x, y)


def mul(x, y):
    return bind("mul", x, y)


def div(x, y):
    return bind("div", x, y)


def max(x, y):
    return bind("max", x, y)


def eq(x, y):
    return bind("eq", x, y)


def lt(x, y):
    return bind("lt", x, y)


def neg(x):
    return bind("neg", x)


def exp(x):
    return bind("exp", x)


def log(x):
    return bind("log", x)


def sqrt(x):
    return bind("sqrt", x)


def tanh(x):
    return bind("tanh", x)


def logistic(x):
    return bind("logistic", x)


def cast(x, new_dtype):
    return bind("cast", x, new_dtype=D.canonical(new_dtype))


def select(pred, on_true, on_false):
    return bind("select", pred, on_true, on_false)


def reduce_sum(x, axes, accum_dtype):
    return bind("reduce_sum", x, axes=tuple(sorted(axes)), accum_dtype=D.canonical(accum_dtype))


def reduce_max(x, axes):
    return bind("reduce_max", x, axes=tuple(sorted(axes)))


def cumsum(x, axis, reverse, accum_dtype):
    return bind("cumsum", x, axis=int(axis), reverse=bool(reverse), accum_dtype=D.canonical(accum_dtype))


def dot_general(lhs, rhs, dimension_numbers, accum_dtype):
    """``((lhs_contracting, rhs_contracting), (lhs_batch, rhs_batch))``; result dims: batch, lhs free, rhs
    free; accumulates in and returns ``accum_dtype``."""
    (lc, rc), (lb, rb) = dimension_numbers
    accum_dtype = D.canonical(accum_dtype)
    return bind(
        "dot_general",
        lhs,
        rhs,
        lhs_contracting=tuple(lc),
        rhs_contracting=tuple(rc),
        lhs_batch=tuple(lb),
        rhs_batch=tuple(rb),
        accum_dtype=accum_dtype,
        output_dtype=accum_dtype,
    )


def reshape(x, new_sizes):
    return bind("reshape", x, new_sizes=tuple(int(n) for n in new_sizes))


def broadcast_in_dim(x, shape, broadcast_dimensions):
    return bind("broadcast_in_dim", x, shape=tuple(shape), broadcast_dimensions=tuple(broadcast_dimensions))


def transpose(x, permutation):
    return bind("transpose", x, permutation=tuple(permutation))


def swap_pairs(x):
    return bind("swap_pairs", x)


def slice(x, start_indices, limit_indices):
    return bind("slice", x, start_indices=tuple(start_indices), limit_indices=tuple(limit_indices))


def _start_indices(start_indices):
    traced = [i for i in start_indices if not isinstance(i, int)]
    dtype = traced[0].dtype if traced else "int32"
    return [full((), i, dtype) if isinstance(i, int) else i for i in start_indices]


def dynamic_slice(x, start_indices, slice_sizes):
    return bind("dynamic_slice", x, *_start_indices(start_indices), slice_sizes=tuple(slice_sizes))


def dynamic_update_slice(x, update, start_indices):
    return bind("dynamic_update_slice", x, update, *_start_indices(start_indices))


def gather(x, indices, axis):
    return bind("gather", x, indices, axis=int(axis))


def take_along_axis(x, indices, axis):
    return bind("take_along_axis", x, indices, axis=int(axis))


def scatter_add(x, indices, updates, axis):
    return bind("scatter_add", x, indices, updates, axis=int(axis))


def concatenate(operands, dimension):
    return bind("concatenate", *operands, dimension=int(dimension))


def full(shape, fill_value, dtype):
    dtype = D.canonical(dtype)
    if D.is_float(dtype):
        fill_value = float(fill_value)
    elif dtype == "bool":
        fill_value = bool(fill_value)
    else:
        fill_value = int(fill_value)
    return bind("full", shape=tuple(shape), fill_value=fill_value, dtype=dtype)


def iota(dtype, shape, dimension):
    return bind("iota", dtype=D.canonical(dtype), shape=tuple(shape), dimension=int(dimension))


def random_bits(seed, start, shape, offset):
    return bind("random_bits", seed, start, shape=tuple(shape), offset=int(offset))


def linear_cross_entropy(h, w, target):
    return bind("linear_cross_entropy", h, w, target)


def _unary(name):
    def f(x):
        return bind(name, x)

    f.__name__ = name
    return f


def _binary(name):
    def f(x, y):
        return bind(name, x, y)

    f.__name__ = name
    return f


sin, cos, tan, asin, acos, atan = map(_unary, ("sin", "cos", "tan", "asin", "acos", "atan"))
sinh, cosh, asinh, acosh, atanh = map(_unary, ("sinh", "cosh", "asinh", "acosh", "atanh"))
floor, ceil, round, log1p, expm1 = map(_unary, ("floor", "ceil", "round", "log1p", "expm1"))
exp2, log2, rsqrt, cbrt, erf_inv = map(_unary, ("exp2", "log2", "rsqrt", "cbrt", "erf_inv"))
is_finite, abs, sign, not_ = map(_unary, ("is_finite", "abs", "sign", "not"))
population_count, clz = map(_unary, ("population_count", "clz"))
pow, rem, min = map(_binary, ("pow", "rem", "min"))
and_, or_, xor = map(_binary, ("and", "or", "xor"))
shift_left, shift_right_logical, shift_right_arithmetic, nextafter = map(
    _binary, ("shift_left", "shift_right_logical", "shift_right_arithmetic", "nextafter")
)
and_.__name__, or_.__name__, not_.__name__ = "and_", "or_", "not_"


def reduce_precision(x, exponent_bits, mantissa_bits):
    return bind("reduce_precision", x, exponent_bits=int(exponent_bits), mantissa_bits=int(mantissa_bits))
