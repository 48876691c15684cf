"""Dtype names, sizes and NumPy storage types (``lumen/tensor/dtype.rs:11-153``)."""

from __future__ import annotations

import numpy as np

FLOATS = ("float16", "bfloat16", "float32", "float64")
SIGNED = ("int8", "int16", "int32", "int64")
UNSIGNED = ("uint8", "uint16", "uint32", "uint64")
ALL = ("bool",) + UNSIGNED + SIGNED + FLOATS

_BITS = {
    "bool": 8,
    "uint8": 8,
    "uint16": 16,
    "uint32": 32,
    "uint64": 64,
    "int8": 8,
    "int16": 16,
    "int32": 32,
    "int64": 64,
    "float16": 16,
    "bfloat16": 16,
    "float32": 32,
    "float64": 64,
}

# NumPy arrays hold each dtype's bits; bfloat16 as uint16 bit patterns.
_STORAGE = {
    "bool": np.bool_,
    "uint8": np.uint8,
    "uint16": np.uint16,
    "uint32": np.uint32,
    "uint64": np.uint64,
    "int8": np.int8,
    "int16": np.int16,
    "int32": np.int32,
    "int64": np.int64,
    "float16": np.float16,
    "bfloat16": np.uint16,
    "float32": np.float32,
    "float64": np.float64,
}

_ALIASES = {
    "float": "float32",
    "half": "float16",
    "double": "float64",
    "bf16": "bfloat16",
    "f32": "float32",
    "f16": "float16",
    "f64": "float64",
    "long": "int64",
    "int": "int32",
}


def canonical(dtype) -> str:
    """A dtype name (``"float32"``) from a name, an alias or a NumPy dtype."""
    if isinstance(dtype, str):
        name = _ALIASES.get(dtype, dtype)
    else:
        name = np.dtype(dtype).name
        if name == "bool":
            name = "bool"
    if name not in _BITS:
        raise TypeError(f"unknown dtype {dtype!r}")
    return name


def is_float(dtype: str) -> bool:
    return dtype in FLOATS


def is_int(dtype: str) -> bool:
    return dtype in SIGNED or dtype in UNSIGNED


def is_signed(dtype: str) -> bool:
    return dtype in SIGNED


def bits(dtype: str) -> int:
    return _BITS[dtype]


def size_of(dtype: str) -> int:
    return max(1, _BITS[dtype] // 8)


def storage(dtype: str):
    """The NumPy dtype holding ``dtype``'s bits."""
    return np.dtype(_STORAGE[dtype])


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 (or float64, via float32 round to odd) values as bfloat16 bit patterns, round to nearest even."""
    x = np.asarray(x)
    if x.dtype == np.float64:
        x = _round_to_odd_f32(x)
    b = np.asarray(x, np.float32).view(np.uint32)
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((b >> 16) | 0x40).astype(np.uint16), r)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def _round_to_odd_f32(x: np.ndarray) -> np.ndarray:
    """float64 to float32 rounding to odd (an inexact result gets an odd last bit): composes with a later
    round-to-nearest to the one correct rounding (``lumen/tensor/dtype.rs:215-224``)."""
    x = np.asarray(x, np.float64)
    t = x.astype(np.float32)  # nearest
    back = t.astype(np.float64)
    inexact = (back != x) & np.isfinite(t)
    bits_ = t.view(np.uint32).copy()
    # step toward zero if rounding went away from x, then force the low bit
    away = inexact & (np.abs(back) > np.abs(x))
    bits_[away] -= 1
    bits_[inexact] |= 1
    return bits_.view(np.float32)


def to_numpy_values(raw: np.ndarray, dtype: str) -> np.ndarray:
    """Storage array as values NumPy computes with (bfloat16 widened to float32)."""
    return bf16_to_f32(raw) if dtype == "bfloat16" else raw


def from_values(values: np.ndarray, dtype: str) -> np.ndarray:
    """Values as ``dtype``'s storage (bfloat16 rounded to nearest even)."""
    if dtype == "bfloat16":
        return bf16_bits(np.asarray(values, np.float32) if np.asarray(values).dtype != np.float64 else values)
    return np.asarray(values).astype(storage(dtype))
