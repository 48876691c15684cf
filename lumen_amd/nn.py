"""``Module``: a frozen-dataclass tree of weights (``lumen/nn.py``)."""

from __future__ import annotations

import dataclasses

__all__ = ["Module"]

_KINDS = {float: "float", int: "int", bool: "bool", "float": "float", "int": "int", "bool": "bool"}


class Module:
    """A tree of weights: subclasses are frozen dataclasses whose tensor fields, recursively, are the
    weights; scalar fields (``float``, ``int``, ``bool``) stay assignable (``nn.py:10-33``)."""

    def __init_subclass__(cls, **kwargs):
        super().__init_subclass__(**kwargs)
        if "__init__" in cls.__dict__:
            # A hand-written __init__ (an optimizer's) keeps its own construction.
            init = cls.__dict__["__init__"]
            dataclasses.dataclass(frozen=True, eq=False, init=False)(cls)
            cls.__init__ = init
        else:
            dataclasses.dataclass(frozen=True, eq=False)(cls)
        frozen = cls.__setattr__

        def __setattr__(self, name, value):
            kind = _scalar_fields(type(self)).get(name)
            if kind is None:
                return frozen(self, name, value)
            object.__setattr__(self, name, value)

        cls.__setattr__ = __setattr__

    def named_parameters(self):
        """``(path, weight)`` for each weight in field order, a shared tensor listed once (``nn.py:35-42``)."""
        seen = set()
        for path, t in _leaves(self, ""):
            if id(t) not in seen:
                seen.add(id(t))
                yield path, t

    def parameters(self):
        return [t for _, t in self.named_parameters()]

    def load_state_dict(self, tensors, strict=True):
        """Copies ``{path: tensor}`` into the weights' memory (``nn.py:48-67``)."""
        params = dict(self.named_parameters())
        if strict:
            missing, unexpected = params.keys() - tensors.keys(), tensors.keys() - params.keys()
            if missing or unexpected:
                raise KeyError(f"load_state_dict: missing {sorted(missing)}, unexpected {sorted(unexpected)}")
        for path, t in tensors.items():
            if path in params:
                params[path].copy_(t)


def _scalar_fields(cls):
    fields = dataclasses.fields(cls)
    return {f.name: _KINDS[f.type] for f in fields if isinstance(f.type, (type, str)) and f.type in _KINDS}


def is_scalar(v):
    if type(v) in (float, int, bool):
        return True
    import numpy as np

    return isinstance(v, (np.bool_, np.integer, np.floating))


def _leaves(x, path):
    from lumen_amd.graph.tracer import TracedTensor
    from lumen_amd.tensor import Tensor

    prefix = f"{path}." if path else ""
    if isinstance(x, Tensor) or (isinstance(x, TracedTensor) and not x.weak):
        yield path, x
    elif isinstance(x, Module):
        for f in dataclasses.fields(x):
            yield from _leaves(getattr(x, f.name), prefix + f.name)
    elif isinstance(x, (list, tuple)):
        for i, v in enumerate(x):
            yield from _leaves(v, prefix + str(i))


def at(x, path):
    for key in path:
        x = getattr(x, key) if isinstance(x, Module) else x[key]
    return x


def assign(x, path, value):
    holder, key = at(x, path[:-1]), path[-1]
    if isinstance(holder, Module):
        object.__setattr__(holder, key, value)
    elif isinstance(holder, list):
        holder[key] = value
    else:
        raise TypeError("a scalar in a tuple cannot be assigned: hold it in a module field or a list")


def map_tensors(x, f, scalar=None, path=()):
    """``x`` with each tensor replaced by ``f(t)`` and each scalar by ``scalar(path, v)`` (``nn.py:180-192``)."""
    from lumen_amd.tensor import Tensor

    if isinstance(x, Tensor):
        return f(x)
    if scalar is not None and is_scalar(x):
        return scalar(path, x)
    if isinstance(x, Module):
        new = object.__new__(type(x))
        for fl in dataclasses.fields(x):
            object.__setattr__(new, fl.name, map_tensors(getattr(x, fl.name), f, scalar, (*path, fl.name)))
        return new
    if isinstance(x, (list, tuple)):
        return type(x)(map_tensors(v, f, scalar, (*path, i)) for i, v in enumerate(x))
    return x


def structure(x):
    """``x``'s hashable structure: classes, static values and tensor types (what a plan depends on)."""
    from lumen_amd.tensor import Tensor

    if isinstance(x, Tensor):
        return ("tensor", x.dtype, tuple(x.shape), id(x) if x._is_parameter else None)
    if isinstance(x, Module):
        return (type(x), tuple((f.name, structure(getattr(x, f.name))) for f in dataclasses.fields(x)))
    if isinstance(x, (list, tuple)):
        return (type(x), tuple(structure(v) for v in x))
    if isinstance(x, float):
        return ("float",)
    return ("static", x)


def scalar_paths(x, path=()):
    """Path of each Python float in ``x`` (the runtime scalars a module carries: a learning rate)."""
    if isinstance(x, float):
        yield path
    elif isinstance(x, Module):
        for f in dataclasses.fields(x):
            yield from scalar_paths(getattr(x, f.name), (*path, f.name))
    elif isinstance(x, (list, tuple)):
        for i, v in enumerate(x):
            yield from scalar_paths(v, (*path, i))
