"""The traced dataflow IR: typed values, nodes applying primitives, and output-type inference.

Follows ``lumen/graph/mod.rs:24-252`` (``TensorType``, ``Node``, ``Graph``, ``apply``, ``prune``) and
``lumen/graph/primitive.rs:203-1077`` (the primitive set and ``infer``): a primitive is its name plus a
dict of static parameters; ``infer`` checks operands and returns the result type with the reference's
error messages.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

from lumen_amd import dtypes as D

UNARY = (
    "sin cos tan asin acos atan sinh cosh asinh acosh atanh floor ceil round log1p expm1 exp2 log2 rsqrt cbrt "
    "erf_inv is_finite reduce_precision abs sign not population_count clz"
).split()
BINARY = "pow rem min and or xor shift_left shift_right_logical shift_right_arithmetic nextafter".split()
CORE_BINARY = ("add", "sub", "mul", "div", "max", "eq", "lt")
CORE_UNARY = ("neg", "exp", "log", "sqrt", "tanh", "logistic")
ELEMENTWISE = set(CORE_BINARY + CORE_UNARY + tuple(UNARY) + tuple(BINARY) + ("cast", "select"))
TRANSCENDENTAL = {
    "exp", "log", "sqrt", "tanh", "logistic", "pow", "sin", "cos", "tan", "asin", "acos", "atan", "sinh", "cosh",
    "asinh", "acosh", "atanh", "log1p", "expm1", "exp2", "log2", "rsqrt", "cbrt", "erf_inv",
}


@dataclass(frozen=True)
class TensorType:
    """The dtype and shape of a graph value (``graph/mod.rs:24-47``)."""

    dtype: str
    shape: tuple

    def numel(self) -> int:
        return math.prod(self.shape)

    def nbytes(self) -> int:
        return self.numel() * D.size_of(self.dtype)

    def __str__(self):
        return f"{self.dtype}[{','.join(map(str, self.shape))}]"


def _freeze(v):
    if isinstance(v, list):
        return tuple(_freeze(x) for x in v)
    if isinstance(v, tuple):
        return tuple(_freeze(x) for x in v)
    return v


@dataclass
class Node:
    """One primitive application producing a single output value (``graph/mod.rs:52-70``)."""

    prim: str
    inputs: tuple
    output: int
    params: dict = field(default_factory=dict)
    backward: bool = False
    scope: tuple = ()

    def key(self):
        """Hashable (primitive, params) for CSE; fusion bodies compare by identity."""
        items = []
        for k in sorted(self.params):
            v = self.params[k]
            items.append((k, id(v) if isinstance(v, Graph) else _freeze(v)))
        return (self.prim, tuple(items))


class Graph:
    """A traced program: value types, inputs, nodes in topological order and outputs (``graph/mod.rs:72-101``)."""

    def __init__(self):
        self.types: list[TensorType] = []
        self.inputs: list[int] = []
        self.nodes: list[Node] = []
        self.outputs: list[int] = []
        self.backward = False
        self.scope: tuple = ()

    def input(self, dtype, shape) -> int:
        self.types.append(TensorType(D.canonical(dtype), tuple(int(s) for s in shape)))
        var = len(self.types) - 1
        self.inputs.append(var)
        return var

    def type_of(self, var) -> TensorType:
        return self.types[var]

    def apply(self, prim, inputs, params=None) -> int:
        """Appends ``prim(*inputs, **params)``, inferring its type (``Graph::apply``, ``graph/mod.rs:159-177``)."""
        params = dict(params or {})
        for v in inputs:
            if not 0 <= v < len(self.types):
                raise ValueError(f"%{v} is not a value of the graph")
        ty = infer(prim, [self.types[v] for v in inputs], params)
        self.types.append(ty)
        out = len(self.types) - 1
        self.nodes.append(Node(prim, tuple(inputs), out, params, self.backward, self.scope))
        return out

    def add_node(self, prim, inputs, params, ty: TensorType, backward=False) -> int:
        """Appends a node of a known type (passes rebuilding graphs)."""
        self.types.append(ty)
        out = len(self.types) - 1
        self.nodes.append(Node(prim, tuple(inputs), out, dict(params), backward))
        return out

    def set_outputs(self, outputs):
        self.outputs = list(outputs)

    def producers(self) -> dict:
        return {n.output: n for n in self.nodes}

    def users(self) -> dict:
        u: dict[int, list[Node]] = {}
        for n in self.nodes:
            for v in n.inputs:
                u.setdefault(v, []).append(n)
        return u

    def prune(self) -> dict:
        """Drops nodes no output depends on and renumbers values densely (``Graph::prune``,
        ``graph/mod.rs:203-252``); returns old var -> new var (None if dropped)."""
        live = set(self.outputs)
        keep = []
        for n in reversed(self.nodes):
            if n.output in live:
                keep.append(n)
                live.update(n.inputs)
        keep.reverse()
        mapping: dict[int, int | None] = {}
        types = []
        for v in self.inputs:
            mapping[v] = len(types)
            types.append(self.types[v])
        for n in keep:
            mapping[n.output] = len(types)
            types.append(self.types[n.output])
        for n in keep:
            n.inputs = tuple(mapping[v] for v in n.inputs)
            n.output = mapping[n.output]
        self.types = types
        self.inputs = [mapping[v] for v in self.inputs]
        self.outputs = [mapping[v] for v in self.outputs]
        self.nodes = keep
        full = {}
        for old in range(max(mapping) + 1 if mapping else 0):
            full[old] = mapping.get(old)
        return full

    def copy(self) -> "Graph":
        g = Graph()
        g.types = list(self.types)
        g.inputs = list(self.inputs)
        g.nodes = [Node(n.prim, n.inputs, n.output, dict(n.params), n.backward, n.scope) for n in self.nodes]
        g.outputs = list(self.outputs)
        return g

    def __str__(self):
        lines = [f"graph({', '.join(f'%{v}: {self.types[v]}' for v in self.inputs)}) {{"]
        for n in self.nodes:
            ps = " ".join(f"{k}={_show(v)}" for k, v in sorted(n.params.items()) if k != "body")
            body = " body=..." if "body" in n.params else ""
            lines.append(
                f"  %{n.output}: {self.types[n.output]} = {n.prim}[{ps}{body}]({', '.join(f'%{v}' for v in n.inputs)})"
            )
        lines.append(f"  return {', '.join(f'%{v}' for v in self.outputs)}")
        lines.append("}")
        return "\n".join(lines)


def _show(v):
    if isinstance(v, (tuple, list)):
        return "(" + ",".join(map(str, v)) + ("," if len(v) == 1 else "") + ")"
    return str(v)


# ---- inference ----------------------------------------------------------------------------------------


class InferError(TypeError):
    pass


def _check_dims(dims, ndim, what):
    for i, d in enumerate(dims):
        if not 0 <= d < ndim or d in dims[:i]:
            raise InferError(f"{what} {tuple(dims)} are invalid for rank {ndim}")


def _check_accum(x: TensorType, accum: str):
    narrower = D.size_of(x.dtype) < 4
    widened = narrower and ((D.is_float(x.dtype) and accum == "float32") or (D.is_int(x.dtype) and accum == "int32"))
    if not (accum == x.dtype or widened):
        raise InferError(
            f"accumulates in the operand's dtype, or float32 (int32) for narrower floats (integers): "
            f"got accum_dtype {accum} for {x}"
        )


def _gathered(x: TensorType, idx: TensorType, axis: int) -> TensorType:
    if axis >= len(x.shape):
        raise InferError(f"axis {axis} is not a dimension of {x}")
    if idx.dtype not in ("int32", "int64"):
        raise InferError(f"indices into {x} are int32 or int64, got {idx}")
    return TensorType(x.dtype, x.shape[:axis] + idx.shape + x.shape[axis + 1 :])


def free_dims(ndim, used):
    return [d for d in range(ndim) if d not in used]


_ARITY0 = {"full", "iota", "recv"}
_ARITY2 = {"add", "sub", "mul", "div", "max", "eq", "lt", "dot_general", "gather", "take_along_axis", "random_bits"} | set(
    BINARY
)
_ARITY3 = {"select", "scatter_add", "linear_cross_entropy"}


def infer(prim: str, args: list, p: dict) -> TensorType:
    """The result type of ``prim`` on operands of types ``args`` (``Primitive::infer``,
    ``graph/primitive.rs:535-1077``); ``InferError`` naming the primitive otherwise."""
    try:
        return _infer(prim, args, p)
    except InferError as e:
        raise InferError(f"{prim}: {e}") from None


def _infer(prim, args, p):
    if prim in _ARITY0:
        arity = 0
    elif prim in _ARITY2:
        arity = 2
    elif prim in _ARITY3:
        arity = 3
    elif prim == "fusion":
        arity = len(p["body"].inputs)
    elif prim in ("concatenate",):
        arity = max(1, len(args))
    elif prim == "dynamic_slice":
        arity = 1 + (len(args[0].shape) if args else 0)
    elif prim == "dynamic_update_slice":
        arity = 2 + (len(args[0].shape) if args else 0)
    elif prim in ("fusion_output",):
        arity = 1
    else:
        arity = 1
    if len(args) != arity:
        raise InferError(f"takes {arity} operands, got {len(args)}")

    if prim in CORE_BINARY:
        x, y = args
        if x != y:
            raise InferError(f"operands must have the same type, got {x} and {y}")
        if x.dtype == "bool" and prim not in ("max", "eq", "lt"):
            raise InferError("does not take bool operands")
        return TensorType("bool" if prim in ("eq", "lt") else x.dtype, x.shape)
    if prim in CORE_UNARY:
        x = args[0]
        if prim == "neg" and x.dtype == "bool":
            raise InferError("does not take bool operands")
        if prim != "neg" and not D.is_float(x.dtype):
            raise InferError(f"takes a floating-point operand, got {x}")
        return x
    if prim == "cast":
        new = p["new_dtype"]
        x = args[0]
        if D.is_int(x.dtype) and D.bits(x.dtype) > 16 and D.is_float(new) and D.bits(new) < 32:
            raise InferError(
                f"of {x.dtype} to {new} is ambiguous (rounded once, or through float32): cast to float32 first"
            )
        return TensorType(new, x.shape)
    if prim in UNARY:
        x = args[0]
        floats, ints = D.is_float(x.dtype), D.is_int(x.dtype)
        if prim in ("abs", "sign"):
            fits = floats or ints
        elif prim == "not":
            fits = ints or x.dtype == "bool"
        elif prim in ("population_count", "clz"):
            fits = ints
        else:
            fits = floats
        if not fits:
            raise InferError(f"does not take {x}")
        return TensorType("bool", x.shape) if prim == "is_finite" else x
    if prim in BINARY:
        x, y = args
        if prim == "pow" and D.is_float(x.dtype) and D.is_int(y.dtype) and x.shape == y.shape:
            return x
        if x != y:
            raise InferError(f"operands must have the same type, got {x} and {y}")
        floats, ints, bools = D.is_float(x.dtype), D.is_int(x.dtype), x.dtype == "bool"
        fits = {
            "pow": floats,
            "nextafter": floats,
            "rem": floats or ints,
            "min": True,
            "and": ints or bools,
            "or": ints or bools,
            "xor": ints or bools,
        }.get(prim, ints)
        if not fits:
            raise InferError(f"does not take {x}")
        return x
    if prim in ("host_wait", "device_wait", "to_host", "to_device"):
        return args[0]
    if prim == "select":
        pred, x, y = args
        if pred.dtype != "bool" or pred.shape != x.shape:
            raise InferError(f"pred must be bool with the shape of the cases, got {pred} for {x}")
        if x != y:
            raise InferError(f"cases must have the same type, got {x} and {y}")
        return x
    if prim == "cumsum":
        x = args[0]
        _check_dims([p["axis"]], len(x.shape), "axis")
        if x.dtype == "bool":
            raise InferError("does not take bool operands")
        _check_accum(x, p["accum_dtype"])
        return TensorType(p["accum_dtype"], x.shape)
    if prim in ("reduce_sum", "reduce_max"):
        x = args[0]
        axes = tuple(p["axes"])
        _check_dims(axes, len(x.shape), "axes")
        dtype = x.dtype
        if prim == "reduce_sum":
            if x.dtype == "bool":
                raise InferError("does not take bool operands")
            _check_accum(x, p["accum_dtype"])
            dtype = p["accum_dtype"]
        return TensorType(dtype, tuple(n for d, n in enumerate(x.shape) if d not in axes))
    if prim == "dot_general":
        lhs, rhs = args
        floats = D.is_float(lhs.dtype) and D.is_float(rhs.dtype)
        if (lhs.dtype != rhs.dtype and not floats) or lhs.dtype == "bool":
            raise InferError(f"operands must share a non-bool dtype (or be floats), got {lhs} and {rhs}")
        accum = p["accum_dtype"]
        out = p.get("output_dtype", accum)
        _check_accum(lhs, accum)
        _check_accum(rhs, accum)
        if out not in (lhs.dtype, rhs.dtype, accum):
            raise InferError(
                f"outputs the operands' dtype or accum_dtype ({accum}): got output_dtype {out} for {lhs}"
            )
        lc, rc, lb, rb = (tuple(p[k]) for k in ("lhs_contracting", "rhs_contracting", "lhs_batch", "rhs_batch"))
        ld, rd = lb + lc, rb + rc
        _check_dims(ld, len(lhs.shape), "lhs dimensions")
        _check_dims(rd, len(rhs.shape), "rhs dimensions")
        if len(lb) != len(rb) or len(lc) != len(rc) or any(lhs.shape[l] != rhs.shape[r] for l, r in zip(ld, rd)):
            raise InferError(f"batch and contracting dimensions of {lhs} and {rhs} do not match")
        shape = (
            tuple(lhs.shape[d] for d in lb)
            + tuple(lhs.shape[d] for d in free_dims(len(lhs.shape), ld))
            + tuple(rhs.shape[d] for d in free_dims(len(rhs.shape), rd))
        )
        return TensorType(out, shape)
    if prim == "reshape":
        x = args[0]
        new = tuple(p["new_sizes"])
        if math.prod(new) != x.numel():
            raise InferError(f"cannot reshape {x} to {list(new)}")
        return TensorType(x.dtype, new)
    if prim == "broadcast_in_dim":
        x = args[0]
        shape, dims = tuple(p["shape"]), tuple(p["broadcast_dimensions"])
        bad = (
            len(dims) != len(x.shape)
            or any(a >= b for a, b in zip(dims, dims[1:]))
            or (dims and dims[-1] >= len(shape))
            or any(n != 1 and n != shape[d] for d, n in zip(dims, x.shape))
        )
        if bad:
            raise InferError(f"cannot broadcast {x} to {list(shape)} along dimensions {list(dims)}")
        return TensorType(x.dtype, shape)
    if prim == "transpose":
        x = args[0]
        perm = tuple(p["permutation"])
        if len(perm) != len(x.shape):
            raise InferError(f"{list(perm)} is not a permutation for {x}")
        _check_dims(perm, len(x.shape), "permutation")
        return TensorType(x.dtype, tuple(x.shape[d] for d in perm))
    if prim == "swap_pairs":
        x = args[0]
        if not x.shape or x.shape[-1] % 2:
            raise InferError(f"needs an even-length last axis, got {x}")
        return x
    if prim == "slice":
        x = args[0]
        st, li = tuple(p["start_indices"]), tuple(p["limit_indices"])
        if len(st) != len(x.shape) or len(li) != len(x.shape):
            raise InferError(f"start_indices {list(st)} and limit_indices {list(li)} need one index per dimension")
        for d, (s, l) in enumerate(zip(st, li)):
            if s > l or l > x.shape[d]:
                raise InferError(f"dimension {d}: [{s}, {l}) is not within its size {x.shape[d]}")
        return TensorType(x.dtype, tuple(l - s for s, l in zip(st, li)))
    if prim == "dynamic_slice":
        x = args[0]
        _check_indices(x, args[1:])
        sizes = tuple(p["slice_sizes"])
        if len(sizes) != len(x.shape) or any(s > n for s, n in zip(sizes, x.shape)):
            raise InferError(f"slice_sizes {list(sizes)} are not a block of {x}")
        return TensorType(x.dtype, sizes)
    if prim == "dynamic_update_slice":
        x, u = args[0], args[1]
        _check_indices(x, args[2:])
        if u.dtype != x.dtype or len(u.shape) != len(x.shape) or any(a > b for a, b in zip(u.shape, x.shape)):
            raise InferError(f"the update {u} is not a block of {x}")
        return x
    if prim == "gather":
        return _gathered(args[0], args[1], p["axis"])
    if prim == "take_along_axis":
        x, idx = args
        axis = p["axis"]
        fits = (
            axis < len(x.shape)
            and D.is_int(idx.dtype)
            and len(idx.shape) == len(x.shape)
            and all(d == axis or idx.shape[d] <= x.shape[d] for d in range(len(x.shape)))
        )
        if not fits:
            raise InferError(
                f"indices into {x} along axis {axis} are integers of its rank, no larger but along the axis, got {idx}"
            )
        return TensorType(x.dtype, idx.shape)
    if prim == "scatter_add":
        x, idx, u = args
        want = _gathered(x, idx, p["axis"])
        if u != want:
            raise InferError(f"the updates {u} are not {want}, a gather of {x}")
        return x
    if prim == "concatenate":
        x = args[0]
        d = p["dimension"]
        if d >= len(x.shape):
            raise InferError(f"dimension {d} is not a dimension of {x}")
        total = 0
        for y in args:
            same = len(y.shape) == len(x.shape) and all(i == d or y.shape[i] == x.shape[i] for i in range(len(x.shape)))
            if y.dtype != x.dtype or not same:
                raise InferError(f"operands must share a dtype and all dimensions but {d}, got {x} and {y}")
            total += y.shape[d]
        shape = list(x.shape)
        shape[d] = total
        return TensorType(x.dtype, tuple(shape))
    if prim == "full":
        return TensorType(p["dtype"], tuple(p["shape"]))
    if prim == "iota":
        if p["dimension"] >= len(p["shape"]) or p["dtype"] == "bool":
            raise InferError(f"needs a non-bool dtype and a dimension of {list(p['shape'])}")
        return TensorType(p["dtype"], tuple(p["shape"]))
    if prim == "random_bits":
        if not all(a.dtype == "uint64" and a.shape == () for a in args):
            raise InferError(f"needs uint64 scalars (seed, start), got {args[0]} and {args[1]}")
        return TensorType("uint32", tuple(p["shape"]))
    if prim == "linear_cross_entropy":
        h, w, t = args
        if len(h.shape) != 2 or len(w.shape) != 2 or h.shape[1] != w.shape[1] or h.dtype != w.dtype:
            raise InferError(f"needs rows [B, D] and weights [V, D] of one dtype, got {h} and {w}")
        if not D.is_float(h.dtype):
            raise InferError(f"needs float rows, got {h}")
        if t.dtype not in ("int32", "int64") or t.shape != (h.shape[0],):
            raise InferError(f"needs a class a row, int32 or int64 [{h.shape[0]}], got {t}")
        return TensorType("float32", (2, h.shape[0]))
    if prim == "fusion":
        body = p["body"]
        for i, (a, v) in enumerate(zip(args, body.inputs)):
            if a != body.types[v]:
                raise InferError(f"operand {i} must be {body.types[v]}, got {a}")
        if not body.outputs:
            raise InferError("the body must have an output")
        return body.types[body.outputs[0]]
    if prim == "fusion_output":
        return p["ty"]
    raise InferError(f"unknown primitive {prim!r}")


def _check_indices(x, indices):
    dtype = indices[0].dtype if indices else None
    ok = all(i.shape == () and i.dtype == dtype and i.dtype in ("int32", "int64") for i in indices)
    if not ok:
        raise InferError(
            f"start indices into {x} are an int32 or int64 scalar a dimension, of one dtype: got "
            f"[{', '.join(map(str, indices))}]"
        )
