"""Concrete tensors: host (NumPy storage), hip (a device block from the static region) or meta (no data).

Mirrors the parts of ``lumen/tensor`` the compiled path needs: dtype-exact host conversions (bfloat16 by
round to nearest even, ``tensor/dtype.rs:215-239``), copies between host and device through the C ABI, and
weights: a meta tensor in a module is a parameter, placed on a device when the first compiled function
taking it compiles, its data written there by ``copy_`` / ``load_state_dict``.
"""

from __future__ import annotations

import math

import numpy as np

from lumen_amd import dtypes as D
from lumen_amd import native


def device_name(d) -> str:
    """``"hip:0"`` from ``"hip"``, ``"hip:0"``, ``"cpu"``, ``"meta"``. The GPU device is named ``hip``; there is
    no CUDA alias."""
    d = str(d)
    kind, _, idx = d.partition(":")
    if kind not in ("cpu", "hip", "meta"):
        raise ValueError(f"unknown device {d!r}: this backend has cpu (host data), hip and meta")
    return f"{kind}:{idx or 0}"


def device_type(d) -> str:
    return device_name(d).split(":")[0]


def device_index(d) -> int:
    return int(device_name(d).split(":")[1])


class DeviceBuffer:
    """A block of device memory from ``nhip_alloc``, freed when the last reference goes."""

    __slots__ = ("ptr", "nbytes", "device", "__weakref__")
    # devices whose static region is reserved (lumen_amd.config.static_allocator_bytes)

    _reserved: set = set()

    def __init__(self, device: int, nbytes: int):
        native.set_device(device)
        if device not in DeviceBuffer._reserved:
            from lumen_amd.config import config

            native.call("nhip_region_reserve", device, int(config.static_allocator_bytes))
            DeviceBuffer._reserved.add(device)
        self.device, self.nbytes = device, int(nbytes)
        self.ptr = native.alloc(device, max(1, self.nbytes))

    def __del__(self):
        if getattr(self, "ptr", None) and native is not None and native._lib is not None:
            try:
                native.free(self.device, self.ptr, self.nbytes)
            except Exception:
                pass
            self.ptr = None


class Tensor:
    """A tensor of ``dtype`` and ``shape`` on ``device``; hip data is ``buffer`` at byte ``offset``,
    contiguous row-major."""

    def __init__(self, dtype, shape, device="cpu", host=None, buffer=None, offset=0):
        self.dtype = D.canonical(dtype)
        self.shape = tuple(int(s) for s in shape)
        self.device = device_name(device)
        self._host = host
        self._buffer = buffer
        self._offset = offset
        self._is_parameter = False
        self._placements = {}
        self._pending = None
        self.grad = None

    # -- basics
    @property
    def ndim(self):
        return len(self.shape)

    def numel(self):
        return math.prod(self.shape)

    @property
    def nbytes(self):
        return self.numel() * D.size_of(self.dtype)

    def size(self, dim=None):
        return self.shape if dim is None else self.shape[dim]

    def data_ptr(self):
        if self._buffer is None:
            raise RuntimeError(f"a {self.device} tensor has no device pointer")
        return self._buffer.ptr + self._offset

    def __repr__(self):
        return f"Tensor(dtype={self.dtype}, shape={list(self.shape)}, device={self.device})"

    # -- data movement
    def raw(self) -> np.ndarray:
        """The storage bits as a NumPy array (bfloat16 as uint16), copied from the device if needed."""
        kind = device_type(self.device)
        if kind == "cpu":
            return self._host
        if kind == "meta":
            if self._is_parameter:
                for t in self._placements.values():
                    return t.raw()
                if self._pending is not None:
                    return self._pending
            raise RuntimeError("a meta tensor has no data")
        from lumen_amd import native

        out = np.empty(self.shape, D.storage(self.dtype))
        if out.nbytes:
            native.set_device(self._buffer.device)
            native.d2h(out.ctypes.data, self.data_ptr(), out.nbytes)
        return out

    def numpy(self):
        return to_numpy(self)

    def to(self, *args, dtype=None, device=None, **_):
        for a in args:
            if isinstance(a, str) and a.split(":")[0] in ("cpu", "hip", "meta"):
                device = a
            elif isinstance(a, Tensor):
                dtype = a.dtype
            else:
                dtype = a
        t = self
        if dtype is not None and D.canonical(dtype) != t.dtype:
            vals = D.to_numpy_values(t.raw(), t.dtype)
            t = Tensor(dtype, t.shape, "cpu", host=_convert(vals, t.dtype, D.canonical(dtype)))
            if device is None:
                device = self.device
        if device is not None and device_name(device) != t.device:
            kind = device_type(device)
            if kind == "cpu":
                t = Tensor(t.dtype, t.shape, "cpu", host=t.raw())
            elif kind == "hip":
                t = _upload(t.raw(), t.dtype, device_index(device))
            else:
                t = Tensor(t.dtype, t.shape, "meta")
        return t

    def cpu(self):
        return self.to("cpu")

    def float(self):
        return self.to(dtype="float32")

    def bfloat16(self):
        return self.to(dtype="bfloat16")

    def clone(self):
        kind = device_type(self.device)
        if kind == "hip":
            from lumen_amd import native

            out = empty(self.shape, self.dtype, self.device)
            native.d2d(out.data_ptr(), self.data_ptr(), self.nbytes)
            return out
        if kind == "cpu":
            return Tensor(self.dtype, self.shape, "cpu", host=self._host.copy())
        return Tensor(self.dtype, self.shape, "meta")

    def item(self):
        return to_numpy(self).reshape(()).item()

    def tolist(self):
        return to_numpy(self).tolist()

    def reshape(self, *shape):
        shape = tuple(shape[0]) if len(shape) == 1 and not isinstance(shape[0], int) else tuple(shape)
        if -1 in shape:
            known = math.prod(s for s in shape if s != -1)
            shape = tuple(self.numel() // known if s == -1 else s for s in shape)
        if math.prod(shape) != self.numel():
            raise RuntimeError(f"shape {list(shape)} is invalid for input of size {self.numel()}")
        kind = device_type(self.device)
        if kind == "cpu":
            return Tensor(self.dtype, shape, "cpu", host=self._host.reshape(shape))
        return Tensor(self.dtype, shape, self.device, buffer=self._buffer, offset=self._offset)

    def copy_(self, src):
        """Writes ``src``'s values (converted to this dtype) into this tensor's memory; a weight's into every
        device it is placed on (``nn.Module.load_state_dict``)."""
        if not isinstance(src, Tensor):
            src = tensor(src, dtype=self.dtype)
        if tuple(src.shape) != self.shape:
            raise RuntimeError(f"copy_: shape {list(src.shape)} does not match {list(self.shape)}")
        kind = device_type(self.device)
        if kind == "hip" and device_type(src.device) == "hip" and src.dtype == self.dtype:
            from lumen_amd import native

            native.set_device(self._buffer.device)
            native.d2d(self.data_ptr(), src.data_ptr(), self.nbytes)
            return self
        raw = src.raw() if src.dtype == self.dtype else _convert(D.to_numpy_values(src.raw(), src.dtype), src.dtype, self.dtype)
        raw = np.ascontiguousarray(raw, D.storage(self.dtype)).reshape(self.shape)
        if kind == "cpu":
            self._host[...] = raw
        elif kind == "hip":
            from lumen_amd import native

            native.set_device(self._buffer.device)
            if raw.nbytes:
                native.h2d(self.data_ptr(), raw.ctypes.data, raw.nbytes)
        elif self._is_parameter:
            self._pending = raw.copy()
            for t in self._placements.values():
                t.copy_(Tensor(self.dtype, self.shape, "cpu", host=self._pending))
        else:
            raise RuntimeError("copy_ into a meta tensor that is not a module weight")
        return self

    # -- weights
    def _placed(self, target):
        """This weight's memory on ``target`` (allocated, and given its loaded data, on first use)."""
        target = device_name(target)
        if not self._is_parameter:
            return self
        t = self._placements.get(target)
        if t is None:
            t = empty(self.shape, self.dtype, target)
            if self._pending is not None:
                t.copy_(Tensor(self.dtype, self.shape, "cpu", host=self._pending))
            self._placements[target] = t
        return t


def _convert(values, src, dst):
    """Host values of dtype ``src`` as storage of ``dst`` with the reference's cast semantics."""
    if D.is_float(dst):
        return D.from_values(np.asarray(values, np.float64) if src in ("float64",) else values, dst)
    if D.is_float(src):
        v = np.nan_to_num(np.asarray(values, np.float64), nan=0.0)
        info = np.iinfo(D.storage(dst)) if dst != "bool" else None
        if info is not None:
            v = np.clip(np.trunc(v), info.min, info.max)
        return v.astype(D.storage(dst))
    return np.asarray(values).astype(D.storage(dst))


def _upload(raw, dtype, device):
    t = empty(raw.shape, dtype, f"hip:{device}")
    if raw.nbytes:
        from lumen_amd import native

        raw = np.ascontiguousarray(raw)
        native.h2d(t.data_ptr(), raw.ctypes.data, raw.nbytes)
    return t


def empty(shape, dtype="float32", device="cpu", alignment=256):
    dtype = D.canonical(dtype)
    shape = tuple(shape)
    kind = device_type(device)
    if kind == "cpu":
        return Tensor(dtype, shape, "cpu", host=np.empty(shape, D.storage(dtype)))
    if kind == "meta":
        t = Tensor(dtype, shape, "meta")
        t._is_parameter = True
        return t
    nbytes = math.prod(shape) * D.size_of(dtype)
    return Tensor(dtype, shape, device, buffer=DeviceBuffer(device_index(device), nbytes))


def from_numpy(arr):
    arr = np.array(arr, order="C", copy=True)  # keeps 0-d arrays 0-d (ascontiguousarray makes them 1-d)
    return Tensor(D.canonical(arr.dtype), arr.shape, "cpu", host=arr)


def tensor(data, dtype=None, device="cpu"):
    arr = np.asarray(data)
    src = D.canonical(arr.dtype) if arr.dtype != np.float64 or dtype is None else "float64"
    if dtype is None:
        dtype = "float32" if arr.dtype == np.float64 else src
    dtype = D.canonical(dtype)
    host = _convert(arr, src, dtype) if src != dtype else arr.astype(D.storage(dtype))
    t = Tensor(dtype, arr.shape, "cpu", host=np.asarray(host, order="C"))
    return t.to(device=device) if device_type(device) != "cpu" else t


def full(shape, value, dtype="float32", device="cpu"):
    return tensor(np.full(tuple(shape), value, np.float64 if D.is_float(D.canonical(dtype)) else None), dtype, device)


def zeros(shape, dtype="float32", device="cpu"):
    return full(shape, 0, dtype, device)


def ones(shape, dtype="float32", device="cpu"):
    return full(shape, 1, dtype, device)


def to_numpy(t: Tensor) -> np.ndarray:
    """Values as a NumPy array; bfloat16 widened exactly to float32."""
    return D.to_numpy_values(t.raw(), t.dtype).reshape(t.shape)
