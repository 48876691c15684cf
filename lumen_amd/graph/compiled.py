"""``lumen_amd.compile`` and ``Compiled`` (``lumen/graph/tracer.py:693-1141``).

A compiled function traces its Python function once per signature (tensor dtypes and shapes, module
structure, static values; floats are runtime scalars), compiles a ``Plan`` for the device, allocates the
plan's workspace once, and on each call passes its arguments, scalars and the modules' placed weights to the
plan, returns views of the results in the workspace (the next call overwrites them) and writes weights the
function assigned back into their memory.
"""

from __future__ import annotations

import collections
import functools

import numpy as np

from lumen_amd import nn
from lumen_amd.config import config
from lumen_amd.graph.trace import trace, tree_leaves
from lumen_amd import native
from lumen_amd.tensor import DeviceBuffer, Tensor, device_name, device_type, empty


def compile(fn, device=None):
    """``fn`` compiled for ``device`` (``"hip"``; ``"meta"`` compiles without running): see ``Compiled``."""
    return Compiled(fn, device)


class Compiled:
    def __init__(self, fn, device=None):
        functools.update_wrapper(self, fn)
        self._fn = fn
        self._device = None if device is None else device_name(device)
        self._plans = {}
        self._latest = None
        self._graphs = {}  # id(plan) -> captured graphs by the addresses they read in place (empty: warm)
        self._scalars = collections.OrderedDict()  # (device, float64 bits) -> device float64 holding it

    def _target(self, args):
        if self._device is not None:
            return self._device
        tensors = [a for a in args if isinstance(a, Tensor)]
        data = [a for a in tensors if device_type(a.device) != "meta"]
        return data[0].device if data else ("meta:0" if tensors else "hip:0")

    def _key(self, args, target):
        return (tuple(nn.structure(a) for a in args), target, config.compiler.key())

    def _prepare(self, args):
        target = self._target(args)
        if device_type(target) == "cpu":
            raise RuntimeError(
                "device='cpu' is lumen's reference interpreter; this backend compiles for 'hip' (and 'meta')"
            )
        key = self._key(args, target)
        entry = self._plans.get(key)
        if entry is None:
            traced = trace(self._fn, args)
            plan, workspace = None, None
            if device_type(target) == "hip":
                from lumen_amd.compiler.plan import Plan

                weight_pos = [i for i, (kind, _) in enumerate(traced.layout) if kind == "weight"]
                # each weight the function assigns: its new value may be computed over the old one
                at = {k: i for i, (kind, k) in enumerate(traced.layout) if kind == "weight"}
                donate = {traced.n_returned + j: at[k] for j, k in enumerate(traced.written)} \
                    if config.compiler.update_in_place else {}
                plan = Plan(traced.graph, target, packable=weight_pos, donate=donate)
                workspace = DeviceBuffer(int(target.split(":")[1]), plan.workspace_bytes)
                for w in traced.weights:
                    w._placed(target)
                for pack in plan.packs:
                    _pack([traced.weights[traced.layout[i][1]] for i in pack], target)
            entry = (traced, plan, workspace)
            self._plans[key] = entry
        self._latest = key
        return target, entry

    @property
    def plan(self):
        return self._plans[self._latest][1]

    # Arguments of at least this many bytes are read by a captured graph where they lie (one graph per set of
    # such addresses, the newest GRAPHS_PER_PLAN kept) instead of being copied into its staging buffers, whose
    # copy would cost as much as a memory-bound plan itself.
    DIRECT_BYTES = 1 << 20
    GRAPHS_PER_PLAN = 8
    # runtime scalars kept on the device between calls (a learning rate is the same every step)
    SCALARS_KEPT = 64

    def _device_scalar(self, target, value):
        """A device float64 holding ``value``, uploaded once per (device, value) and kept: the upload is a
        synchronous host-to-device copy, which would otherwise make every call wait for the previous call's
        kernels before it could queue its own. Evicted entries may still be read by queued kernels; their
        memory is only reused by work queued after them on the device's one stream."""
        key = (target, np.float64(value).tobytes())
        t = self._scalars.get(key)
        if t is None:
            t = Tensor("float64", (), "cpu", host=np.array(value, np.float64)).to(device=target)
            self._scalars[key] = t
            while len(self._scalars) > self.SCALARS_KEPT:
                self._scalars.popitem(last=False)
        else:
            self._scalars.move_to_end(key)
        return t
    # Plans of fewer native steps run uncaptured: launching a graph costs the host ~40 us, launching a step
    # ~3 us, so a short plan (a fused elementwise chain is one kernel) loses time to the graph.
    GRAPH_MIN_STEPS = 16

    def _run(self, plan, workspace, traced, ptrs, keep):
        """``plan.run_in``; with ``config.compiler.hip_graphs`` (the reference's CUDA graphs,
        ``lumen/graph/tracer.py:958-1049``) a plan runs as usual on its first call (which builds and autotunes
        its kernels), is captured on its second into a HIP graph over device buffers of its own for the
        call's runtime scalars and small arguments, and from then on each call copies those in (stream-ordered)
        and launches the graph. Weights, the workspace and large arguments are read where they were captured;
        a call whose large arguments or weights lie elsewhere is captured again (the newest few graphs of a
        plan are kept, so alternating inputs replay too). Profiled runs (``plan.profile``) and plans of fewer
        than GRAPH_MIN_STEPS native steps are never captured.
        Returns the input pointers the run read."""
        short = len(getattr(plan, "native_steps", ())) < self.GRAPH_MIN_STEPS and plan._native is not None
        if not config.compiler.hip_graphs or getattr(plan, "_profiling", False) or short:
            plan.run_in(workspace.ptr, ptrs)
            return ptrs
        graphs = self._graphs.get(id(plan))
        staged = [i for i, (kind, _) in enumerate(traced.layout)
                  if kind == "scalar" or (kind == "arg" and keep[i].nbytes < self.DIRECT_BYTES)]
        fixed = (workspace.ptr,) + tuple(p for i, p in enumerate(ptrs) if i not in staged)
        if graphs is None:
            self._graphs[id(plan)] = collections.OrderedDict()  # warm: the first call runs plainly
            plan.run_in(workspace.ptr, ptrs)
            return ptrs
        entry = graphs.get(fixed)
        if entry is None:
            dev = int(plan.device.split(":")[1])
            buffers = {i: DeviceBuffer(dev, max(1, keep[i].nbytes)) for i in staged}
            gptrs = [buffers[i].ptr if i in buffers else p for i, p in enumerate(ptrs)]
            for i, b in buffers.items():
                native.d2d(b.ptr, ptrs[i], keep[i].nbytes)
            entry = (plan.capture(workspace.ptr, gptrs), buffers, gptrs)
            graphs[fixed] = entry
            if len(graphs) > self.GRAPHS_PER_PLAN:
                # launches of the evicted graph queued earlier may still read its staging buffers
                native.sync(dev)
                while len(graphs) > self.GRAPHS_PER_PLAN:
                    graphs.popitem(last=False)
        else:
            graphs.move_to_end(fixed)
            _, buffers, gptrs = entry
            for i, b in buffers.items():
                native.d2d(b.ptr, ptrs[i], keep[i].nbytes)
        entry[0].launch()
        return gptrs

    def last_buffers(self):
        """``(workspace pointer, input pointers)`` of the latest run (to replay some of its steps)."""
        return self._last_buffers

    @property
    def graph(self):
        return self._plans[self._latest][0].graph

    def __call__(self, *args):
        target, (traced, plan, workspace) = self._prepare(args)
        g = traced.graph
        ran = plan is not None and not any(isinstance(a, Tensor) and device_type(a.device) == "meta" for a in args)
        if not ran:
            outs = [Tensor(g.types[v].dtype, g.types[v].shape, "meta") for v in g.outputs]
        else:
            keep = []
            ptrs = []
            tensors = [a for a in args if isinstance(a, Tensor)]
            scalars = _scalars(args)
            for kind, k in traced.layout:
                if kind == "arg":
                    t = tensors[k]
                    if device_name(t.device) != target:
                        t = t.to(device=target)
                    keep.append(t)
                    ptrs.append(t.data_ptr())
                elif kind == "scalar":
                    t = self._device_scalar(target, scalars[k])
                    keep.append(t)
                    ptrs.append(t.data_ptr())
                else:
                    t = traced.weights[k]._placed(target)
                    keep.append(t)
                    ptrs.append(t.data_ptr())
            ptrs = self._run(plan, workspace, traced, ptrs, keep)
            self._last_buffers = (workspace.ptr, ptrs)
            outs = []
            for v, loc in zip(g.outputs, plan.output_locs):
                if loc.base[0] == "in":  # computed over the weight it replaces
                    outs.append(keep[loc.base[1]])
                    continue
                t = Tensor(loc.dtype, loc.shape, target, buffer=workspace, offset=loc.offset * _size(loc.dtype))
                outs.append(t)
            # the other weights the function assigned: written back into their memory, in stream order
            for j, k in enumerate(traced.written):
                if traced.n_returned + j not in plan.in_place_outputs:
                    traced.weights[k]._placed(target).copy_(outs[traced.n_returned + j])
            self._keep = keep
        for i, path, value in traced.static_writes:
            nn.assign(args[i], path, value)
        it = iter(outs)
        return _rebuild(traced.out, it)


def _pack(weights, target):
    """Stores ``weights`` back to back in one device block, in order (a merge_dots pack: the plan reads their
    concatenation as a view of the first), moving their current data there; a no-op when they already are."""
    placed = [w._placed(target) for w in weights]
    first = placed[0]
    if all(t._buffer is first._buffer for t in placed):
        off = first._offset
        for t in placed:
            if t._offset != off:
                break
            off += t.nbytes
        else:
            return
    dev = int(target.split(":")[1])
    block = DeviceBuffer(dev, sum(t.nbytes for t in placed))
    off = 0
    for w, t in zip(weights, placed):
        nt = Tensor(t.dtype, t.shape, target, buffer=block, offset=off)
        nt.copy_(t)
        w._placements[device_name(target)] = nt
        off += t.nbytes


def _size(dtype):
    from lumen_amd import dtypes as D

    return D.size_of(dtype)


def _scalars(args):
    out = []
    for a in args:
        if isinstance(a, float):
            out.append(a)
    # module floats follow the top-level ones in trace order
    res = []
    for a in args:
        if isinstance(a, float):
            res.append(a)
        elif isinstance(a, (nn.Module, list, tuple)):
            for path in nn.scalar_paths(a):
                res.append(nn.at(a, path))
    return res


def _rebuild(out, it):
    from lumen_amd.graph.tracer import TracedTensor

    if isinstance(out, TracedTensor):
        return next(it)
    if isinstance(out, (list, tuple)):
        return type(out)(_rebuild(v, it) for v in out)
    if isinstance(out, dict):
        return {k: _rebuild(v, it) for k, v in out.items()}
    if isinstance(out, nn.Module):
        return nn.map_tensors(out, lambda t: next(it))
    return out


_ = (tree_leaves, empty)
