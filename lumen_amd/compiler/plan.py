"""The static plan of a graph on one hip device (``lumen/plan``).

``Plan(graph, device)`` runs the hip pass pipeline, groups the graph into steps (``fusion.fuse``), places
every value a step writes in one workspace by live range at 256-byte alignment (``plan/compile.rs:49-555``,
``ALIGNMENT`` ``plan/mod.rs:26``), lowers layout ops feeding built-in kernels to strided views, generates and
compiles the loop kernels, and builds the native step list (``nhip_plan_*``). ``run_in(workspace, inputs)``
then queues every step on the device's stream with no host work per step but the launch
(``plan/run.rs:247-427``).
"""

from __future__ import annotations

import ctypes as C
import math
import struct
from dataclasses import dataclass

from lumen_amd import dtypes as D
from lumen_amd.compiler import attention as attn_pass
from lumen_amd.compiler import codegen, fusion, kcache, merge, passes, remat, schedule
from lumen_amd.config import config
from lumen_amd.graph.ir import Graph

ALIGNMENT = 256
NHIP_DT = {"float32": 0, "bfloat16": 1, "float16": 2}


@dataclass
class Loc:
    """Where a value lives: a base (``("ws", 0)`` the workspace, ``("in", i)`` plan input ``i``), an element
    offset and element strides."""

    base: tuple
    offset: int
    strides: tuple
    dtype: str
    shape: tuple

    def contiguous(self):
        return codegen.View(self.dtype, self.shape, self.offset, self.strides).contiguous()

    def view(self):
        return codegen.View(self.dtype, self.shape, self.offset, self.strides)


def _mfma_layout(d) -> bool:
    """Whether the MFMA kernels read a dot's operands (each k- or mn-contiguous with 16-byte aligned lines):
    the host-side twin of kernels.hip's mfma_ready, without the pointer alignment."""
    if d.a_k == 1 and d.k % 8 == 0 and (d.a_m % 8 == 0 or d.m == 1):
        pass
    elif not (d.a_m == 1 and d.m % 8 == 0 and d.a_k % 8 == 0):
        return False
    if d.b_k == 1 and d.k % 8 == 0 and (d.b_n % 8 == 0 or d.n == 1):
        pass
    elif not (d.b_n == 1 and d.n % 8 == 0 and d.b_k % 8 == 0):
        return False
    return all(d.a_batch[i] % 8 == 0 and d.b_batch[i] % 8 == 0 for i in range(d.nbatch))


def _contig(shape):
    return codegen._contig(shape)


def _view_of(prim, params, src: Loc, ty) -> Loc | None:
    """The layout op ``prim`` of ``src`` as a strided view, or None when strides cannot express it."""
    if prim == "transpose":
        perm = params["permutation"]
        return Loc(src.base, src.offset, tuple(src.strides[d] for d in perm), ty.dtype, ty.shape)
    if prim == "broadcast_in_dim":
        dims = params["broadcast_dimensions"]
        st = [0] * len(ty.shape)
        for i, d in enumerate(dims):
            st[d] = 0 if src.shape[i] == 1 else src.strides[i]
        return Loc(src.base, src.offset, tuple(st), ty.dtype, ty.shape)
    if prim == "slice":
        off = src.offset + sum(s * st for s, st in zip(params["start_indices"], src.strides))
        return Loc(src.base, off, src.strides, ty.dtype, ty.shape)
    if prim == "reshape":
        if src.contiguous():
            return Loc(src.base, src.offset, _contig(ty.shape), ty.dtype, ty.shape)
        st = _reshape_strides(src.shape, src.strides, ty.shape)
        return None if st is None else Loc(src.base, src.offset, st, ty.dtype, ty.shape)
    return None


class _Graph:
    """An executable HIP graph of a plan run (``Plan.capture``), destroyed with the object."""

    def __init__(self, handle):
        self.handle = handle

    def launch(self):
        from lumen_amd import native as nv

        nv.call("nhip_graph_launch", C.c_void_p(self.handle))

    def __del__(self):
        if getattr(self, "handle", None):
            try:
                from lumen_amd import native as nv

                nv.lib().nhip_graph_destroy(C.c_void_p(self.handle))
            except Exception:
                pass
            self.handle = None


def _operand_view(cat: Loc, start, operand, ty) -> Loc:
    """Where an operand of a concatenation lives inside it: the slice ``start = (dim, offset)`` of shape
    ``operand.shape``, reshaped to the producer's type ``ty``."""
    dim, off = start
    sl = Loc(cat.base, cat.offset + off * cat.strides[dim], cat.strides, operand.dtype, operand.shape)
    if operand.shape == ty.shape:
        return Loc(sl.base, sl.offset, sl.strides, ty.dtype, ty.shape)
    st = _reshape_strides(sl.shape, sl.strides, ty.shape)
    assert st is not None, "checked when the alias was chosen"
    return Loc(sl.base, sl.offset, st, ty.dtype, ty.shape)


def _reshape_strides(shape, strides, new):
    """torch's view rule: strides for ``new`` over memory laid out as ``shape``/``strides``, or None."""
    dims = [(n, s) for n, s in zip(shape, strides) if n != 1]
    out = []
    i = 0
    for n in new:
        if n == 1:
            out.append(0)
            continue
        if i >= len(dims):
            return None
        size, stride = dims[i]
        if size == n:
            out.append(stride)
            i += 1
            continue
        if size % n == 0:
            # split a dim
            dims[i] = (size // n, stride)
            out.append(stride * (size // n))
            continue
        # merge dims while contiguous
        acc, st = size, stride
        j = i + 1
        while acc < n and j < len(dims) and dims[j - 1][1] == dims[j][0] * dims[j][1]:
            acc *= dims[j][0]
            st = dims[j][1]
            j += 1
        if acc != n:
            return None
        out.append(st)
        i = j
    return tuple(out)


def compile_graph(graph: Graph, packable=()) -> tuple[Graph, list]:
    """The hip pipeline (``graph_compiler/pipeline.rs:162-320`` picks): frontend (cse, simplify), flash
    attention forward and backward matching, linear cross entropy, merge_dots over the weights at input
    positions ``packable``,
    simplify again. Returns the graph and merge_dots' packs (weight input positions stored back to back)."""
    g = passes.frontend(graph)
    if config.compiler.flash_attention:
        g = attn_pass.match(g)
        g = passes.frontend(g)
    if config.compiler.fuse and config.compiler.fused_linear_cross_entropy:
        g = passes.linear_cross_entropy(g)  # after the attention passes, as the reference orders it
    packs = []
    if config.compiler.merge_dots and packable:
        g, packs = merge.merge_dots(g, set(packable))
    # after every pattern match: the structural rewrites too (``pipeline.rs``: simplify follows the matchers)
    g = passes.frontend(g, matched=config.compiler.simplify_structural)
    return g, packs


class Plan:
    """A graph compiled for ``device`` (``"hip:0"``): steps, workspace layout and native step list."""

    def __init__(self, graph: Graph, device="hip:0", build_kernels=True, packable=(), compiled=None, donate=None):
        self.device = device
        # output position -> input position: outputs the caller writes back over that input after each run
        # (the weights a step assigns); those the placement can compute in place are written there directly
        self.donate = dict(donate or {})
        self.source_graph = graph
        self.graph, self.packs = compiled if compiled is not None else compile_graph(graph, packable)
        self._lay_out()
        limit = config.compiler.memory_limit
        if limit and compiled is None and self.workspace_bytes > limit:
            # remat.rs via plan/compile.rs:37-44: recompute values past the live-bytes peak
            def plan_of(g):
                return Plan(graph, device, build_kernels=False, compiled=(g, self.packs), donate=self.donate)

            g = remat.rematerialize(self.graph, limit, plan_of)
            if g is not self.graph:
                self.graph = g
                self._lay_out()
        self.kernels = {}
        self.sources = {}
        self.epi_alts = {}  # epilogue GEMM step -> [(k loop variant, kernel, source)] for the autotuner
        self._native = None
        if compiled is None or build_kernels:
            self._gen_kernels()
        if build_kernels:
            self.build()

    def _lay_out(self):
        """Steps, schedule and placement of ``self.graph``."""
        # concatenations of a pack's weights: views of the first weight's memory (the caller stores a pack's
        # weights back to back, in order)
        self.packed = set()
        packed_inputs = {tuple(self.graph.inputs[i] for i in pk) for pk in self.packs}
        for n in self.graph.nodes:
            if n.prim == "concatenate" and n.params["dimension"] == 0 and tuple(n.inputs) in packed_inputs:
                self.packed.add(n.output)
        self.steps = self._fuse()
        self._schedule()
        if config.compiler.fuse and config.compiler.epilogue_fusion and self._fuse_epilogues():
            self._place()

    # ---- fusion with fallback: groups the generator rejects are split
    def _fuse(self):
        steps = fusion.fuse(self.graph, fuse_loops=config.compiler.fuse, packed=self.packed)
        if config.compiler.fuse:
            steps = fusion.hoist_to_producers(self.graph, steps)
            steps = fusion.absorb_rows(self.graph, steps)
        if config.compiler.fuse and config.compiler.horizontal_fusion:
            steps = fusion.horizontal(self.graph, steps)
        return steps

    # ---- schedule (plan/compile.rs:19-47): the step order whose placement needs the least workspace
    def _schedule(self):
        """Places the steps in their fused order and in each schedule of ``schedule.SCHEDULES``, keeping the
        order with the smallest workspace (the fused order on ties); ``self.schedule`` names it."""
        fused = list(self.steps)
        self._place()
        best = (self.workspace_bytes, "fused", fused)
        self.schedule_bytes = {"fused": self.workspace_bytes}
        if config.compiler.schedules:
            for name, order_of in schedule.SCHEDULES.items():
                self.steps = order_of(self.graph, fused)
                self._place()
                self.schedule_bytes[name] = self.workspace_bytes
                if self.workspace_bytes < best[0]:
                    best = (self.workspace_bytes, name, list(self.steps))
        self.schedule = best[1]
        self.steps = best[2]
        self._place()

    # ---- outputs computed in place of an input (the reference's donated buffers)
    def _in_place_outputs(self):
        """``{output value: input position}`` for the ``donate`` pairs whose output can be written straight over
        its input: the output's step is an elementwise loop (or a GEMM epilogue) that reads the input only at
        the element it writes, through elementwise operations of the input's shape, and every other step that
        reads the input's memory (the input, its views, a pack's concatenation) runs before it. The caller's
        copy of such an output back into the input is then not needed, nor its workspace."""
        g = self.graph
        if not self.donate:
            return {}
        # the input positions whose memory each value may address
        roots = {v: {i} for i, v in enumerate(g.inputs)}
        packs = {tuple(g.inputs[i] for i in pk): set(pk) for pk in self.packs}
        for st in self.steps:
            if st.kind == "view":
                n = st.nodes[0]
                if n.output in self.packed:
                    roots[n.output] = packs.get(tuple(n.inputs), set().union(*(roots.get(u, set()) for u in n.inputs)))
                elif n.inputs[0] in roots:
                    roots[n.output] = roots[n.inputs[0]]
        # a producing step that other readers of the old value follow, none of them reading its results, moves
        # after the last of them (a weight's update after the GEMM that reads the weight for the input gradient)
        for op, ip in sorted(self.donate.items()):
            v = g.outputs[op]
            si = next((i for i, st in enumerate(self.steps) if v in st.outputs), None)
            if si is None:
                continue
            later = [sj for sj in range(si + 1, len(self.steps))
                     if any(ip in roots.get(w, ()) for w in self.steps[sj].inputs)]
            if not later:
                continue
            made = set(self.steps[si].outputs)
            if any(x in made for st in self.steps[si + 1:later[-1] + 1] for x in st.inputs):
                continue
            self.steps.insert(later[-1], self.steps.pop(si))
        producer = {v: si for si, st in enumerate(self.steps) for v in st.outputs}
        out, taken = {}, set()
        for op, ip in sorted(self.donate.items()):
            v, u = g.outputs[op], g.inputs[ip]
            tv, tu = g.types[v], g.types[u]
            if (ip in taken or g.outputs.count(v) != 1 or v in roots or u in g.outputs or tv.dtype != tu.dtype
                    or tuple(tv.shape) != tuple(tu.shape) or v not in producer):
                continue
            si = producer[v]
            st = self.steps[si]
            if st.kind == "loop":
                body, others = st.nodes, []
            elif st.kind == "hloop":
                member = next(m for m in st.members if v in m.outputs)
                body, others = member.nodes, [m for m in st.members if m is not member]
            elif st.kind == "dot" and getattr(st, "epi", None) is not None:
                body, others = st.epi.nodes, [st.nodes[0]]
            else:
                continue
            # nothing reads the input's memory after the step, nor in it but through `body` at its own element
            if any(ip in roots.get(w, ()) and (sj > si or (sj == si and w != u))
                   for sj, s2 in enumerate(self.steps) for w in s2.inputs):
                continue
            if any(ip in roots.get(w, ()) for o in others for w in o.inputs):
                continue
            reached, same = {u}, True
            for n in body:
                if any(x in reached for x in n.inputs):
                    if n.prim not in fusion.ELEMENTWISE or tuple(g.types[n.output].shape) != tuple(tu.shape):
                        same = False
                        break
                    reached.add(n.output)
            if same:
                out[v] = ip
                taken.add(ip)
        return out

    # ---- placement
    def _place(self):
        g = self.graph
        # placement may run again after a pass merges steps: start from the graph's own steps
        self.steps = [st for st in self.steps if st.kind != "copy"]
        self._copies = {}
        for st in self.steps:
            if st.kind == "alias":
                st.kind = "loop"
        self.loc: dict[int, Loc] = {}
        self.scratch: dict[int, Loc] = {}
        self.in_place = self._in_place_outputs()
        self.in_place_outputs = {g.outputs.index(v): i for v, i in self.in_place.items()}
        self.aliased = frozenset(self.in_place) | frozenset(g.inputs[i] for i in self.in_place.values())
        for i, v in enumerate(g.inputs):
            t = g.types[v]
            self.loc[v] = Loc(("in", i), 0, _contig(t.shape), t.dtype, t.shape)
        # a flash forward output read only through one transpose that keeps the head dim innermost (the
        # attention output going back to [B, S, N, H]) is written in the transposed order: the kernel takes
        # any strides, and the output projection then reads it in place instead of through a copy
        o_perm = {}
        gusers = g.users()
        for st in self.steps if self.FLASH_OUT_TRANSPOSED else ():
            if st.kind == "flash_fwd" and st.outputs[0] not in g.outputs:
                us = [u for u in gusers.get(st.outputs[0], []) if u.prim != "fusion_output"]
                if len(us) == 1 and us[0].prim == "transpose":
                    perm = tuple(us[0].params["permutation"])
                    if perm[-1] == len(perm) - 1:
                        o_perm[st.outputs[0]] = perm
        # views first: resolved lazily in step order; a view that strides cannot express becomes a copy
        last_use: dict[int, int] = {}
        base_of: dict[int, int] = {}
        for si, st in enumerate(self.steps):
            for u in st.inputs:
                last_use[u] = si
        for v in g.outputs:
            last_use[v] = len(self.steps)
        # a view keeps its base alive as long as it is used
        for si in reversed(range(len(self.steps))):
            st = self.steps[si]
            if st.kind == "view":
                v = st.outputs[0]
                src = st.nodes[0].inputs[0]
                last_use[src] = max(last_use.get(src, si), last_use.get(v, si))
        free: list[tuple[int, int]] = []  # (offset, size)
        top = 0
        live: dict[int, tuple[int, int]] = {}

        def take(size):
            nonlocal top
            size = -(-max(size, 1) // ALIGNMENT) * ALIGNMENT
            best = None
            for k, (off, sz) in enumerate(free):
                if sz >= size and (best is None or sz < free[best][1]):
                    best = k
            if best is not None:
                off, sz = free.pop(best)
                if sz > size:
                    free.append((off + size, sz - size))
                return off, size
            off = top
            top += size
            return off, size

        def release(off, size):
            free.append((off, size))
            free.sort()
            merged = []
            for o, s in free:
                if merged and merged[-1][0] + merged[-1][1] == o:
                    merged[-1] = (merged[-1][0], merged[-1][1] + s)
                else:
                    merged.append((o, s))
            free[:] = merged

        # concatenations whose operands are written straight into the result by their producers
        aliases = self._concat_aliases()
        for si, st in enumerate(self.steps):
            if st.kind == "alias":
                c = st.outputs[0]
                last_use[c] = max(last_use.get(c, si), si)

        converted = []
        for si, st in enumerate(self.steps):
            if st.kind == "alias":
                continue
            if st.kind == "view":
                n = st.nodes[0]
                src = self.loc[n.inputs[0]]
                if n.output in self.packed:
                    t = g.types[n.output]
                    loc = Loc(src.base, src.offset, _contig(t.shape), t.dtype, t.shape)
                else:
                    loc = _view_of(n.prim, n.params, src, g.types[n.output])
                if loc is not None:
                    self.loc[n.output] = loc
                    base_of[n.output] = base_of.get(n.inputs[0], n.inputs[0])
                    continue
                st.kind = "loop"
                converted.append(si)
            for v in st.outputs:
                t = g.types[v]
                if v in aliases:
                    c, start, _ = aliases[v]
                    if c not in self.loc:  # the concatenation's memory is taken at its first producer
                        ct = g.types[c]
                        off, size = take(ct.nbytes())
                        live[c] = (off, size)
                        self.loc[c] = Loc(("ws", 0), off // D.size_of(ct.dtype), _contig(ct.shape), ct.dtype, ct.shape)
                    self.loc[v] = _operand_view(self.loc[c], start, aliases[v][2], t)
                    continue
                if v in self.in_place:  # written over the input it replaces
                    self.loc[v] = Loc(("in", self.in_place[v]), 0, _contig(t.shape), t.dtype, t.shape)
                    continue
                off, size = take(t.nbytes())
                live[v] = (off, size)
                strides = _contig(t.shape)
                if v in o_perm:  # laid out as its transpose: the transpose (and a reshape of it) is then a view
                    perm = o_perm[v]
                    dense = _contig(tuple(t.shape[d] for d in perm))
                    strides = [0] * len(perm)
                    for j, d in enumerate(perm):
                        strides[d] = dense[j]
                    strides = tuple(strides)
                self.loc[v] = Loc(("ws", 0), off // D.size_of(t.dtype), strides, t.dtype, t.shape)
            if st.kind == "dot":
                st.splits, split_cfg = (1, None) if getattr(st, "epi", None) is not None else self._split_count(st.nodes[0])
                if split_cfg is not None:
                    st.config = split_cfg
                if st.splits > 1:
                    d, _ = self._gemm_desc(st.nodes[0])
                    st.scratch = st.splits * max(1, math.prod(d.batch[i] for i in range(d.nbatch))) * d.m * d.n * 4
            if st.kind == "linear_cross_entropy":
                st.scratch = self._lce_scratch(self._lce_desc(st.nodes[0]))
            if st.scratch:
                off, size = take(st.scratch)
                self.scratch[id(st)] = Loc(("ws", 0), off // 4, (1,), "float32", (st.scratch // 4,))
                release(off, size)
            for v in list(live):
                if last_use.get(v, -1) <= si and v not in g.outputs:
                    off, size = live.pop(v)
                    release(off, size)
        self.workspace_bytes = max(top, ALIGNMENT)
        self.workspace_alignment = ALIGNMENT
        # graph outputs that are plan inputs (returned unchanged) are copied into the workspace
        self.output_locs = []
        for v in g.outputs:
            loc = self.loc[v]
            if (loc.base[0] == "in" and v not in self.in_place) or not loc.contiguous():
                t = g.types[v]
                off = self.workspace_bytes
                self.workspace_bytes += -(-t.nbytes() // ALIGNMENT) * ALIGNMENT
                dst = Loc(("ws", 0), off // D.size_of(t.dtype), _contig(t.shape), t.dtype, t.shape)
                self.steps.append(fusion.Step("copy", [], [v], [v]))
                self._copies[len(self.steps) - 1] = (loc, dst)
                loc = dst
            self.output_locs.append(loc)

    # ---- GEMM epilogues (lumen/graph_compiler/passes/fusion/mod.rs:20-112, the CUDA backend's `epilogue`):
    # a loop step that reads a dot's [m, n] result element for element runs inside the dot's store
    FLASH_OUT_TRANSPOSED = True  # flash outputs laid out as the transpose that reads them (see _place)
    EPI_MIN_TILES = 256  # the streamed GEMM's own default threshold (kernels.hip: default_config)

    def _epilogue_layout(self, st):
        """``(desc, at, bt, f16)`` when dot step ``st`` can run as a streamed GEMM with a generated epilogue
        (2-D bf16/f16 operands, k a multiple of 64, one k split, operand rows 16-byte aligned), else None."""
        from lumen_amd import native as nv

        n = st.nodes[0]
        p = n.params
        if p["lhs_batch"] or p["rhs_batch"] or getattr(st, "splits", 1) > 1:
            return None
        if len(self.graph.types[n.output].shape) != 2 or self.loc[n.output].strides != _contig(self.graph.types[n.output].shape):
            return None
        try:
            d, ops = self._gemm_desc(n)
        except NotImplementedError:
            return None
        if d.a_dtype != d.b_dtype or d.a_dtype not in (nv.NHIP_BF16, nv.NHIP_F16) or d.k % 64 or d.n % 4:
            return None
        if -(-d.m // 256) * -(-d.n // 256) < self.EPI_MIN_TILES:
            return None  # too few 256 x 256 tiles to fill the CUs: a smaller tiled kernel (autotuned) is faster
        if d.a_k == 1 and d.a_m % 8 == 0:
            at = False
        elif d.a_m == 1 and d.m % 8 == 0 and d.a_k % 8 == 0:
            at = True
        else:
            return None
        if d.b_k == 1 and d.b_n % 8 == 0:
            bt = False
        elif d.b_n == 1 and d.n % 8 == 0 and d.b_k % 8 == 0:
            bt = True
        else:
            return None
        if any((loc.offset * D.size_of(loc.dtype)) % 16 for loc in ops[:2]):
            return None
        return d, at, bt, d.a_dtype == nv.NHIP_F16

    def _fuse_epilogues(self):
        """Merges each loop step that is the elementwise consumer of a dot's [m, n] result into the dot's step
        (``st.epi``); returns whether any was merged. The loop's other inputs must exist before the dot runs;
        the dot's result is still stored when other steps or the graph's outputs read it."""
        from lumen_amd.graph.ir import ELEMENTWISE

        g = self.graph
        pos = {}
        users: dict[int, list] = {}
        for si, st in enumerate(self.steps):
            for v in st.outputs:
                pos[v] = si
            for u in st.inputs:
                users.setdefault(u, []).append(si)
        outputs = set(g.outputs)
        merged = set()
        for si, st in enumerate(self.steps):
            if st.kind != "dot" or getattr(st, "epi", None) is not None:
                continue
            dv = st.nodes[0].output
            lay = self._epilogue_layout(st)
            if lay is None:
                continue
            shape = g.types[dv].shape
            for li in users.get(dv, []):
                lt = self.steps[li]
                if li in merged or lt.kind != "loop" or li <= si:
                    continue
                if any(g.types[v].shape != shape or not self.loc[v].view().contiguous() for v in lt.outputs):
                    continue
                readers = [n for n in lt.nodes if dv in n.inputs]
                if any(n.prim not in ELEMENTWISE or g.types[n.output].shape != shape for n in readers):
                    continue
                if any(u != dv and pos.get(u, -1) >= si for u in lt.inputs):
                    continue  # an operand the loop reads is made after the dot
                keep = dv in outputs or any(x != li for x in users.get(dv, []))
                st.epi = lt
                st.epi_layout = lay
                st.store_dot = keep
                st.outputs = ([dv] if keep else []) + list(lt.outputs)
                st.inputs = list(st.inputs) + [u for u in lt.inputs if u != dv and u not in st.inputs]
                st.nodes = list(st.nodes) + list(lt.nodes)
                merged.add(li)
                break
        self.steps = [st for i, st in enumerate(self.steps) if i not in merged]
        return bool(merged) | self._fuse_column_sums()

    def _fuse_column_sums(self):
        """A float32 sum over the rows of a GEMM epilogue's [m, n] output that only the sum reads (a bias or
        norm-weight gradient) moves into the epilogue: each wave adds its column sums atomically into the
        zero-filled [n] result and the [m, n] value is never stored. Returns whether any moved."""
        g = self.graph
        outputs = set(g.outputs)
        readers: dict[int, list] = {}
        for st in self.steps:
            for u in st.inputs:
                readers.setdefault(u, []).append(st)
        gone = set()
        for st in self.steps:
            if st.kind != "dot" or getattr(st, "epi", None) is None or getattr(st, "epi_colsum", None):
                continue
            shape = g.types[st.nodes[0].output].shape
            for u in st.epi.outputs:
                rs = readers.get(u, [])
                if len(rs) != 1 or u in outputs or g.types[u].dtype != "float32" or g.types[u].shape != shape:
                    continue
                r = rs[0]
                if r.kind != "reduce" or len(r.nodes) != 1 or r.nodes[0].prim != "reduce_sum":
                    continue
                n = r.nodes[0]
                if n.inputs[0] != u or tuple(n.params["axes"]) != (0,) or g.types[n.output].dtype != "float32":
                    continue
                st.epi_colsum = (u, n.output)
                st.outputs = [v for v in st.outputs if v != u] + [n.output]
                st.nodes = list(st.nodes) + [n]
                gone.add(id(r))
                break
        self.steps = [st for st in self.steps if id(st) not in gone]
        return bool(gone)

    # the producers that may write an operand of a concatenation in place, through a strided view
    ALIAS_PRODUCERS = ("flash_fwd", "flash_bwd", "dot", "loop")

    def _concat_aliases(self):
        """``{value: (concatenation, start, operand type)}`` for loop steps that only concatenate (through
        reshapes) values produced by earlier kernels that read nothing else of them: each such value is
        placed as a strided view into the concatenation at ``start`` along its dimension, and the step
        becomes an ``alias`` (no launch). A step qualifies only if every operand does."""
        g = self.graph
        users: dict[int, list] = {}
        producer: dict[int, object] = {}
        for st in self.steps:
            for u in st.inputs:
                users.setdefault(u, []).append(st)
            for v in st.outputs:
                producer[v] = st
        outputs = set(g.outputs)
        aliases = {}
        for st in self.steps:
            if st.kind != "loop" or len(st.outputs) != 1 or st.nodes[-1].prim != "concatenate":
                continue
            cat = st.nodes[-1]
            if cat.output != st.outputs[0] or any(n.prim != "reshape" for n in st.nodes[:-1]):
                continue
            made = {n.output: n.inputs[0] for n in st.nodes[:-1]}
            dim = cat.params["dimension"]
            found, start, ok = {}, 0, True
            for u in cat.inputs:
                v = u
                while v in made:
                    v = made[v]
                p_ = producer.get(v)
                if (p_ is None or p_.kind not in self.ALIAS_PRODUCERS or v in outputs or v in found
                        or v in aliases or any(x is not st for x in users.get(v, []))):
                    ok = False
                    break
                # the operand's place in the concatenation, as the producer's shape; kernels need a
                # unit-stride innermost dimension
                ct = g.types[cat.output]
                view = _operand_view(Loc(("ws", 0), 0, _contig(ct.shape), ct.dtype, ct.shape), (dim, start),
                                     g.types[u], g.types[v]) if _reshape_strides(
                    g.types[u].shape, _contig(ct.shape), g.types[v].shape) is not None else None
                if view is None or (view.strides and view.strides[-1] != 1):
                    ok = False
                    break
                found[v] = (cat.output, (dim, start), g.types[u])
                start += g.types[u].shape[dim]
            if ok and found:
                aliases.update(found)
                st.kind = "alias"
        return aliases

    # ---- kernels
    FAR_STEPS = 8  # an output whose first reader runs at least this many steps later is stored nontemporal

    def _gen_kernels(self):
        import hashlib

        g = self.graph
        first_read = {}
        for si, st in enumerate(self.steps):
            for u in st.inputs:
                first_read.setdefault(u, si)
        far = frozenset(v for si, st in enumerate(self.steps) for v in st.outputs
                        if first_read.get(v, len(self.steps)) - si >= self.FAR_STEPS)
        for si, st in enumerate(self.steps):
            if st.kind == "hloop":
                parts = []
                for m in st.members:
                    views = {v: self.loc[v].view() for v in m.inputs}
                    outs = {v: self.loc[v].view() for v in m.outputs}
                    parts.append(codegen.LoopKernel(g, m, "KNAME", views, outs, self.aliased))
                    parts[-1].far = far
                k = codegen.HorizontalKernel(parts)
                body = k.source()
                name = f"hloop_{hashlib.sha1(body.encode()).hexdigest()[:10]}"
                k.name = st.name = name
                self.kernels[si] = k
                self.sources[si] = codegen.HEADER + body.replace("KNAME", name)
                continue
            if st.kind == "dot" and getattr(st, "epi", None) is not None:
                d, at, bt, f16 = st.epi_layout
                d, _ = self._gemm_desc(st.nodes[0])
                lin = [v for v in st.epi.inputs if v != st.nodes[0].output]
                views = {v: self.loc[v].view() for v in lin}
                outs = {v: self.loc[v].view() for v in st.outputs}
                k = codegen.GemmEpilogueKernel(g, st, st.epi, d, at, bt, f16, st.store_dot, views, outs,
                                               colsum=getattr(st, "epi_colsum", None), aliased=self.aliased)
                k.far = far
                body = k.source()
                name = f"gemm_epi_{hashlib.sha1(body.encode()).hexdigest()[:10]}"
                k.name = st.name = name
                self.kernels[si] = k
                self.sources[si] = codegen.HEADER + body.replace("KNAME", name)
                # the other k loops, for the autotuner to time against this one (large dots whose operands and
                # outputs do not overlap, so a timed run changes nothing the plan reads)
                if config.compiler.autotune and d.m * d.n * d.k >= self.AUTOTUNE_MACS and not self._epi_overlaps(st):
                    for var in range(1, len(codegen.GemmEpilogueKernel.VARIANTS)):
                        if not k.variant_ok(var):
                            continue
                        kv = codegen.GemmEpilogueKernel(g, st, st.epi, d, at, bt, f16, st.store_dot, views, outs,
                                                        colsum=getattr(st, "epi_colsum", None), variant=var,
                                                        aliased=self.aliased)
                        kv.far = far
                        bv = kv.source()
                        kv.name = f"gemm_epi_{hashlib.sha1(bv.encode()).hexdigest()[:10]}"
                        self.epi_alts.setdefault(si, []).append((var, kv, codegen.HEADER + bv.replace("KNAME", kv.name)))
                continue
            if st.kind not in ("loop", "row", "reduce", "scatter_add"):
                continue
            if st.kind == "scatter_add":
                # the operand reaches the output buffer first (a fill of its constant, or a copy); the kernel
                # then reads only the indices and updates
                n = st.nodes[0]
                st.prefill = self._prefill(n)
                st.inputs = [v for v in n.inputs[1:]]
            views = {v: self.loc[v].view() for v in st.inputs}
            outs = {v: self.loc[v].view() for v in st.outputs}
            k = codegen.LoopKernel(g, st, "KNAME", views, outs, self.aliased)
            k.far = far
            body = k.source()
            name = f"{st.kind}_{hashlib.sha1(body.encode()).hexdigest()[:10]}"
            k.name = name
            st.name = name
            src = codegen.HEADER + body.replace("KNAME", name)
            self.kernels[si] = k
            self.sources[si] = src

    def _prefill(self, n):
        """How a scatter_add's output gets its operand: ``("fill", value)`` for a constant, else ``("copy", loc)``."""
        prod = self.graph.producers()
        x = prod.get(n.inputs[0])
        if x is not None and x.prim == "full":
            if float(x.params["fill_value"]) != 0.0:
                raise NotImplementedError("scatter_add into a nonzero constant: the hip backend has no kernel for it yet")
            return ("fill", 0)
        return ("copy", self.loc[n.inputs[0]])

    def build(self):
        """Compiles every generated kernel (hipcc, cached), the epilogue GEMMs' alternative k loops too."""
        keys = list(self.sources)
        alts = [(si, i) for si, lst in self.epi_alts.items() for i in range(len(lst))]
        paths = kcache.compile_many([self.sources[k] for k in keys] + [self.epi_alts[si][i][2] for si, i in alts])
        self.objects = dict(zip(keys, paths[: len(keys)]))
        self.alt_objects = {key: p for key, p in zip(alts, paths[len(keys):])}

    def _epi_overlaps(self, st):
        """Whether an epilogue GEMM step writes memory it also reads (then it is never run for timing alone).
        Outputs written over their input count as not overlapping: the autotuner writes them elsewhere."""
        ins = [self.loc[v] for v in st.nodes[0].inputs if v in self.loc] + \
              [self.loc[v] for v in st.epi.inputs if v != st.nodes[0].output and v in self.loc]
        outs = [self.loc[v] for v in st.outputs if v in self.loc and v not in self.in_place]

        def span(loc):
            lo = loc.offset * D.size_of(loc.dtype)
            hi = lo + max(1, sum((n - 1) * abs(stv) for n, stv in zip(loc.shape, loc.strides)) + 1) * D.size_of(loc.dtype)
            return loc.base, lo, hi

        for o in outs:
            bo, lo_o, hi_o = span(o)
            for i in ins:
                bi, lo_i, hi_i = span(i)
                if bi == bo and lo_i < hi_o and lo_o < hi_i:
                    return True
        return False

    # ---- native
    def _native_plan(self):
        if self._native is not None:
            return self._native
        from lumen_amd import native as nv

        if not hasattr(self, "objects"):
            self.build()
        nv.set_device(int(self.device.split(":")[1]))
        plan = C.c_void_p()
        nv.call("nhip_plan_create", C.byref(plan))
        g = self.graph
        self.native_steps = []  # python step index of each native step (fills and copies included)
        _call = nv.call

        def call(name, *args):
            if name in ("nhip_plan_add_launch", "nhip_plan_add_builtin"):
                self.native_steps.append(current[0])
            return _call(name, *args)

        current = [0]

        def reloc(slot, loc: Loc):
            r = nv.Reloc()
            r.slot = slot
            r.base = nv.NHIP_BASE_WORKSPACE if loc.base[0] == "ws" else nv.NHIP_BASE_INPUT
            r.index = loc.base[1] if loc.base[0] == "in" else 0
            r.offset = loc.offset * D.size_of(loc.dtype)
            return r

        for si, st in enumerate(self.steps):
            current[0] = si
            if st.kind == "scatter_add":
                out = self.loc[st.outputs[0]]
                nbytes = g.types[st.outputs[0]].nbytes()
                kind_, arg = st.prefill
                if kind_ == "fill":
                    desc = struct.pack("<QI", nbytes, 0) + b"\0" * 4
                    rr = (nv.Reloc * 1)(reloc(0, out))
                    call("nhip_plan_add_builtin", plan, nv.NHIP_STEP_FILL, desc, len(desc), rr, 1)
                else:
                    desc = struct.pack("<Q", nbytes)
                    rr = (nv.Reloc * 2)(reloc(0, out), reloc(1, arg))
                    call("nhip_plan_add_builtin", plan, nv.NHIP_STEP_COPY, desc, len(desc), rr, 2)
            if st.kind in ("loop", "row", "reduce", "scatter_add", "hloop") or (
                    st.kind == "dot" and getattr(st, "epi", None) is not None):
                k = self.kernels[si]
                fn = nv.module_function(self.objects[si], k.name)
                if st.kind == "dot" and getattr(st, "epi_colsum", None):  # the column sums add into zeros
                    out = self.loc[st.epi_colsum[1]]
                    desc = struct.pack("<QI", g.types[st.epi_colsum[1]].nbytes(), 0) + b"\0" * 4
                    relocs = (nv.Reloc * 1)(reloc(0, out))
                    call("nhip_plan_add_builtin", plan, nv.NHIP_STEP_FILL, desc, len(desc), relocs, 1)
                if st.kind == "reduce" and getattr(k, "atomic", False):
                    out = self.loc[st.outputs[0]]
                    desc = struct.pack("<QI", g.types[st.outputs[0]].nbytes(), 0) + b"\0" * 4
                    relocs = (nv.Reloc * 1)(reloc(0, out))
                    call("nhip_plan_add_builtin", plan, nv.NHIP_STEP_FILL, desc, len(desc), relocs, 1)
                relocs = []
                for j, (kind, v) in enumerate(k.args):
                    relocs.append(reloc(8 * j, self.loc[v]))
                args = b"\0" * (8 * len(k.args))
                grid = (C.c_uint32 * 3)(*k.grid)
                block = (C.c_uint32 * 3)(*k.block)
                rr = (nv.Reloc * max(1, len(relocs)))(*relocs)
                call("nhip_plan_add_launch", plan, fn, grid, block, k.lds, args, len(args), rr, len(relocs))
            elif st.kind == "dot":
                desc, ops = self._gemm_desc(st.nodes[0])
                desc.config = getattr(st, "config", -1)
                if getattr(st, "splits", 1) > 1:
                    desc.splits = st.splits
                    ops = ops + [self.scratch[id(st)]]
                rr = (nv.Reloc * len(ops))(*[reloc(i, l) for i, l in enumerate(ops)])
                call("nhip_plan_add_builtin", plan, nv.NHIP_STEP_GEMM, C.byref(desc), C.sizeof(desc), rr, len(ops))
            elif st.kind in ("flash_fwd", "flash_bwd"):
                kind, desc, ops = attn_pass.lower(self, st)
                rr = (nv.Reloc * len(ops))(*[reloc(i, l) for i, l in enumerate(ops)])
                call("nhip_plan_add_builtin", plan, kind, C.byref(desc), C.sizeof(desc), rr, len(ops))
            elif st.kind == "linear_cross_entropy":
                n = st.nodes[0]
                desc = self._lce_desc(n)
                ops = [self.loc[u] for u in n.inputs] + [self.loc[n.output], self.scratch[id(st)]]
                rr = (nv.Reloc * len(ops))(*[reloc(i, l) for i, l in enumerate(ops)])
                call("nhip_plan_add_builtin", plan, nv.NHIP_STEP_LCE, C.byref(desc), C.sizeof(desc), rr, len(ops))
            elif st.kind == "copy":
                src, dst = self._copies[si]
                desc = struct.pack("<Q", g.types[st.outputs[0]].nbytes())
                rr = (nv.Reloc * 2)(reloc(0, dst), reloc(1, src))
                call("nhip_plan_add_builtin", plan, nv.NHIP_STEP_COPY, desc, len(desc), rr, 2)
            elif st.kind in ("view", "alias"):
                continue
            else:
                raise NotImplementedError(f"{st.kind}: the hip backend has no kernel for it yet")
        self._native = plan
        return plan

    def _gemm_desc(self, n):
        """``nhip_gemm_desc`` of a dot_general node over its operands' strided locations."""
        from lumen_amd import native as nv

        g = self.graph
        p = n.params
        lhs, rhs = self.loc[n.inputs[0]], self.loc[n.inputs[1]]
        ot = g.types[n.output]
        # a dot whose result only feeds its fused epilogue has no location of its own: rows are n apart
        out = self.loc.get(n.output) or Loc(("ws", 0), 0, _contig(ot.shape), ot.dtype, ot.shape)
        lt, rt = g.types[n.inputs[0]], g.types[n.inputs[1]]
        lc, rc, lb, rb = p["lhs_contracting"], p["rhs_contracting"], p["lhs_batch"], p["rhs_batch"]
        lf = [d for d in range(len(lt.shape)) if d not in lc and d not in lb]
        rf = [d for d in range(len(rt.shape)) if d not in rc and d not in rb]
        if lt.dtype not in NHIP_DT or rt.dtype not in NHIP_DT or (lt.dtype == "float32") != (rt.dtype == "float32"):
            raise NotImplementedError(f"dot_general of {lt.dtype} and {rt.dtype}: the hip backend has no kernel for it yet")
        if lt.dtype != rt.dtype:
            raise NotImplementedError(f"dot_general of {lt.dtype} and {rt.dtype}: the hip backend has no kernel for it yet")
        if p["output_dtype"] not in NHIP_DT:
            raise NotImplementedError(f"dot_general to {p['output_dtype']}: the hip backend has no kernel for it yet")

        def collapse(loc, dims, what):
            """One (size, stride) for ``dims`` of ``loc``, which must be collapsible."""
            dims = [d for d in dims if loc.shape[d] != 1]
            if not dims:
                return 1, 0
            size = loc.shape[dims[-1]]
            stride = loc.strides[dims[-1]]
            for a, b in zip(reversed(dims[:-1]), reversed(dims[1:])):
                if loc.strides[a] != loc.strides[b] * loc.shape[b]:
                    raise NotImplementedError(f"dot_general: {what} dimensions are not collapsible in memory")
                size *= loc.shape[a]
            return size, stride

        m, a_m = collapse(lhs, lf, "lhs free")
        k, a_k = collapse(lhs, list(lc), "lhs contracting")
        k2, b_k = collapse(rhs, list(rc), "rhs contracting")
        nn_, b_n = collapse(rhs, rf, "rhs free")
        # output dims: batch, lhs free, rhs free
        nb = len(lb)
        od = list(range(nb))
        o_lf = list(range(nb, nb + len(lf)))
        o_rf = list(range(nb + len(lf), nb + len(lf) + len(rf)))
        m2, d_m = collapse(out, o_lf, "output rows")
        n2, d_n = collapse(out, o_rf, "output columns")
        batches = [(lt.shape[lb[i]], lhs.strides[lb[i]], rhs.strides[rb[i]], out.strides[od[i]]) for i in range(nb)]
        batches = [b for b in batches if b[0] != 1]
        if len(batches) > 3:
            raise NotImplementedError("dot_general with more than 3 batch dimensions")
        d = nv.GemmDesc()
        d.m, d.n, d.k = m, nn_, k
        d.nbatch = len(batches)
        d.a_dtype, d.b_dtype, d.d_dtype = NHIP_DT[lt.dtype], NHIP_DT[rt.dtype], NHIP_DT[p["output_dtype"]]
        for i, (size, sa, sb, sd) in enumerate(batches):
            d.batch[i], d.a_batch[i], d.b_batch[i], d.d_batch[i] = size, sa, sb, sd
        d.a_m, d.a_k, d.b_k, d.b_n, d.d_m, d.d_n = a_m, a_k, b_k, b_n, d_m, d_n
        d.config = -1
        return d, [lhs, rhs, out]

    # Linear cross entropy (Primitive::LinearCrossEntropy, lumen/reference/mod.rs:1092-1120): nhip_gemm writes the
    # float32 logits of LCE_SCRATCH bytes' worth of rows at a time into the step's scratch, a row kernel reduces
    # them; the [b, v] logits never exist whole.
    LCE_SCRATCH = 512 << 20

    def _lce_desc(self, n):
        from lumen_amd import native as nv

        g = self.graph
        h, w, t = (g.types[u] for u in n.inputs)
        for u in n.inputs:
            if not self.loc[u].contiguous():
                raise NotImplementedError("linear_cross_entropy of strided operands: the hip backend has no kernel for it yet")
        if h.dtype != w.dtype or h.dtype not in NHIP_DT or t.dtype not in ("int32", "int64"):
            raise NotImplementedError(f"linear_cross_entropy of {h.dtype}, {w.dtype}, {t.dtype}: the hip backend has no "
                                      "kernel for it yet")
        d = nv.LceDesc()
        d.b, d.d = h.shape
        d.v = w.shape[0]
        d.chunk_rows = max(1, min(d.b, self.LCE_SCRATCH // max(1, d.v * 4)))
        d.dtype = NHIP_DT[h.dtype]
        d.target_dtype = nv.NHIP_LCE_I64 if t.dtype == "int64" else nv.NHIP_LCE_I32
        return d

    @staticmethod
    def _lce_scratch(desc):
        """The step's scratch bytes: what nhip_linear_cross_entropy_workspace asks for the descriptor (the fused
        form's per-block partials, or chunk_rows rows of float32 logits)."""
        from lumen_amd import native as nv

        n = C.c_size_t()
        nv.call("nhip_linear_cross_entropy_workspace", C.byref(desc), C.byref(n))
        return n.value

    # ---- autotuning (lumen/autotune/mod.rs:20-150): bf16/f16 dots of at least 2^30 multiply-adds try every tile
    # config the kernel accepts, timed with HIP events on the step's own operands (their values do not change
    # MFMA timing), before the first run; the fastest is kept per (shape, layout, dtype) for the process.
    AUTOTUNE_MACS = 1 << 30
    AUTOTUNE_MARGIN = 0.03
    _tuned: dict = {}

    def _apply_forced(self):
        """Configs of ``lumen_amd.autotune.use`` blocks: every plain GEMM step (any size) and every flash
        forward step takes its family's forced config, untimed (``autotune/forced.rs``)."""
        from lumen_amd import autotune

        gemm, attn = autotune.forced(autotune.HipGemmConfig), autotune.forced(autotune.HipAttentionConfig)
        for st in self.steps:
            if gemm is not None and st.kind == "dot" and getattr(st, "splits", 1) == 1 \
                    and getattr(st, "epi", None) is None:
                st.config, st.forced = gemm.index, True
            if attn is not None and st.kind == "flash_fwd":
                st.config, st.forced = attn.index, True

    def _autotune(self, workspace_ptr, input_ptrs):
        self._autotune_gemms(workspace_ptr, input_ptrs)
        self._autotune_epilogues(workspace_ptr, input_ptrs)
        self._autotune_attention(workspace_ptr, input_ptrs)

    def _autotune_epilogues(self, workspace_ptr, input_ptrs):
        """Each epilogue GEMM with alternative k loops runs every one of them (a warm-up, then three timed runs
        with HIP events, on the step's own buffers); the fastest (by more than the margin) replaces the kernel
        the plan launches. Kept per generated source for the process."""
        from lumen_amd import native as nv

        from lumen_amd.tensor import DeviceBuffer

        if not self.epi_alts:
            return
        if not hasattr(self, "objects"):
            self.build()
        g = self.graph
        ev0, ev1 = nv.Event(), nv.Event()
        for si, alts in self.epi_alts.items():
            st = self.steps[si]
            key = ("epi", self.sources[si])
            if key not in Plan._tuned:
                k0 = self.kernels[si]
                ptrs = []
                spare = []  # outputs computed in place of an input go to a buffer of their own while timed
                for kind, v in k0.args:
                    loc = self.loc[v]
                    if kind == "out" and v in self.in_place:
                        spare.append(DeviceBuffer(int(self.device.split(":")[1]), g.types[v].nbytes()))
                        ptrs.append(spare[-1].ptr)
                        continue
                    base = workspace_ptr if loc.base[0] == "ws" else input_ptrs[loc.base[1]]
                    ptrs.append(base + loc.offset * D.size_of(loc.dtype))
                args = (C.c_uint64 * max(1, len(ptrs)))(*ptrs)
                cands = [(0, k0, self.objects[si])] + [(var, kv, self.alt_objects[(si, i)])
                                                       for i, (var, kv, _) in enumerate(alts)]
                best, best_ms = 0, float("inf")
                for var, kv, obj in cands:
                    fn = nv.module_function(obj, kv.name)
                    grid = (C.c_uint32 * 3)(*kv.grid)
                    block = (C.c_uint32 * 3)(*kv.block)
                    nv.call("nhip_launch", fn, grid, block, kv.lds, args, C.sizeof(args))
                    ev0.record()
                    for _ in range(3):
                        nv.call("nhip_launch", fn, grid, block, kv.lds, args, C.sizeof(args))
                    ev1.record()
                    ms = ev0.elapsed_ms(ev1) / 3
                    if ms < best_ms * (1.0 - self.AUTOTUNE_MARGIN):
                        best, best_ms = var, ms
                Plan._tuned[key] = best
            var = Plan._tuned[key]
            if var:
                i = [a[0] for a in alts].index(var)
                _, kv, _ = alts[i]
                self.kernels[si] = kv
                self.objects[si] = self.alt_objects[(si, i)]
                st.name = kv.name
            st.epi_variant = var

    ATTN_AUTOTUNE_FLOPS = 1 << 32  # flash forwards of fewer FLOPs keep the default tile

    def _autotune_attention(self, workspace_ptr, input_ptrs):
        """Times each forward tile config on a flash forward step's own operands (HIP events, 3 runs after a
        warm-up) and keeps the fastest (a later one must win by ``AUTOTUNE_MARGIN``); picks are shared by
        steps of the same shape, layout and dtype."""
        from lumen_amd import native as nv

        n_cfg = C.c_int()
        nv.call("nhip_attn_config_count", C.byref(n_cfg))
        ev0, ev1 = nv.Event(), nv.Event()
        for si, st in enumerate(self.steps):
            if st.kind != "flash_fwd" or getattr(st, "forced", False):
                continue
            flops, _ = self.cost(si)
            if flops < self.ATTN_AUTOTUNE_FLOPS:
                continue
            kind, desc, ops = attn_pass.lower(self, st)
            key = ("attn", desc.batch, desc.heads, desc.kv_heads, desc.sq, desc.sk, desc.head_dim, desc.dtype,
                   desc.causal, desc.q_s, desc.k_s, desc.v_s, desc.o_s)
            if key not in Plan._tuned:
                ptrs = []
                for loc in ops:
                    base = workspace_ptr if loc.base[0] == "ws" else input_ptrs[loc.base[1]]
                    ptrs.append(base + loc.offset * D.size_of(loc.dtype))
                best, best_ms = 0, float("inf")
                for cfg in range(n_cfg.value):
                    desc.config = cfg
                    nv.call("nhip_flash_fwd", C.byref(desc), *ptrs)  # warm-up
                    ev0.record()
                    for _ in range(3):
                        nv.call("nhip_flash_fwd", C.byref(desc), *ptrs)
                    ev1.record()
                    ms = ev0.elapsed_ms(ev1) / 3
                    if ms < best_ms * (1.0 - self.AUTOTUNE_MARGIN):
                        best, best_ms = cfg, ms
                Plan._tuned[key] = best
            st.config = Plan._tuned[key]

    def _autotune_gemms(self, workspace_ptr, input_ptrs):
        from lumen_amd import native as nv

        n_cfg = C.c_int()
        nv.call("nhip_gemm_config_count", C.byref(n_cfg))
        ev0, ev1 = nv.Event(), nv.Event()
        for st in self.steps:
            if st.kind != "dot" or getattr(st, "splits", 1) > 1 or getattr(st, "epi", None) is not None \
                    or getattr(st, "forced", False):
                continue
            try:
                d, ops = self._gemm_desc(st.nodes[0])
            except NotImplementedError:
                continue
            z = max(1, math.prod(d.batch[i] for i in range(d.nbatch)))
            if d.a_dtype == nv.NHIP_F32 or d.m * d.n * d.k * z < self.AUTOTUNE_MACS:
                continue
            key = (d.m, d.n, d.k, tuple(d.batch[i] for i in range(d.nbatch)), d.a_dtype, d.d_dtype,
                   d.a_m == 1, d.a_k == 1, d.b_k == 1, d.b_n == 1, d.d_n == 1)
            if key not in Plan._tuned:
                ptrs = []
                for loc in ops:
                    base = workspace_ptr if loc.base[0] == "ws" else input_ptrs[loc.base[1]]
                    ptrs.append(base + loc.offset * D.size_of(loc.dtype))
                best, best_ms = -1, float("inf")
                for cfg in range(n_cfg.value):
                    d.config = cfg
                    try:
                        nv.call("nhip_gemm", C.byref(d), *ptrs)  # warm-up; rejects configs the shape can't take
                    except RuntimeError:
                        continue
                    ev0.record()
                    for _ in range(3):
                        nv.call("nhip_gemm", C.byref(d), *ptrs)
                    ev1.record()
                    ms = ev0.elapsed_ms(ev1) / 3
                    # a later config must win by more than timing noise (3%), so near-ties pick the same
                    # kernel run after run
                    if ms < best_ms * (1.0 - self.AUTOTUNE_MARGIN):
                        best, best_ms = cfg, ms
                Plan._tuned[key] = best
            st.config = Plan._tuned[key]

    # Split-k policy: a bf16/f16 dot whose 256 x 256 output tiles cannot fill the 256 CUs is cut along k (in
    # powers of two, each part at least 1024 deep) until they do; its float32 partials live in the step's
    # scratch (nhip_gemm_splitk).
    SPLIT_MIN_K = 1024
    SPLIT_MAX = 8
    STREAM128 = 9  # kernels.hip's kStream128

    def _split_count(self, n):
        lhs, rhs, out = self.loc[n.inputs[0]], self.loc[n.inputs[1]], self.loc[n.output]
        if lhs.dtype not in ("bfloat16", "float16") or rhs.dtype != lhs.dtype:
            return 1, None
        try:
            d, _ = self._gemm_desc(n)
        except NotImplementedError:
            return 1, None
        if not _mfma_layout(d) or any((loc.offset * D.size_of(loc.dtype)) % 16 for loc in (lhs, rhs)):
            return 1, None
        z = max(1, math.prod(d.batch[i] for i in range(d.nbatch)))
        tiles = -(-d.m // 256) * -(-d.n // 256) * z
        if tiles >= 256:
            return 1, None
        # the 128 x 128 kernel runs two workgroups a CU: split until its tiles fill 2 x 256 of them
        tiles = -(-d.m // 128) * -(-d.n // 128) * z
        s = 1
        while (tiles * s * 2 <= 512 and s < self.SPLIT_MAX and d.k % (64 * s * 2) == 0
               and d.k // (s * 2) >= self.SPLIT_MIN_K):
            s *= 2
        return s, (self.STREAM128 if s > 1 else None)

    def run_in(self, workspace_ptr: int, input_ptrs: list):
        """Queues the plan on the stream: inputs are device pointers in graph-input order. The first run
        autotunes the plan's large GEMMs on its own buffers (when ``config.compiler.autotune``)."""
        from lumen_amd import native as nv

        if self._native is None:
            self._apply_forced()
            if config.compiler.autotune:
                self._autotune(workspace_ptr, input_ptrs)
        plan = self._native_plan()
        arr = (C.c_void_p * max(1, len(input_ptrs)))(*input_ptrs)
        nv.call("nhip_plan_run", plan, C.c_void_p(workspace_ptr), arr, len(input_ptrs))

    def capture(self, workspace_ptr: int, input_ptrs: list):
        """A HIP graph of one whole run bound to these pointers (``nhip_plan_capture``); launch it with
        ``launch_graph``. The plan must have run once (its kernels built and autotuned)."""
        from lumen_amd import native as nv

        plan = self._native_plan()
        arr = (C.c_void_p * max(1, len(input_ptrs)))(*input_ptrs)
        handle = C.c_void_p()
        nv.call("nhip_plan_capture", plan, C.c_void_p(workspace_ptr), arr, len(input_ptrs), C.byref(handle))
        return _Graph(handle.value)

    def run_steps(self, workspace_ptr: int, input_ptrs: list, si: int):
        """Queues the native steps of python step ``si`` alone (after a whole run has produced its inputs)."""
        from lumen_amd import native as nv

        plan = self._native_plan()
        idx = [i for i, s in enumerate(self.native_steps) if s == si]
        arr = (C.c_void_p * max(1, len(input_ptrs)))(*input_ptrs)
        nv.call("nhip_plan_run_steps", plan, C.c_void_p(workspace_ptr), arr, len(input_ptrs), idx[0], idx[-1] + 1)

    def __del__(self):
        if getattr(self, "_native", None) is not None:
            try:
                from lumen_amd import native as nv

                nv.lib().nhip_plan_destroy(self._native)
            except Exception:
                pass

    # ---- measurement
    def profile(self, enable=True):
        """Records a HIP event around every native step of each run (per-kernel times); profiled runs are
        never replayed from a captured graph."""
        from lumen_amd import native as nv

        nv.call("nhip_plan_profile", self._native_plan(), int(enable))
        self._profiling = bool(enable)

    def step_ms(self):
        """Milliseconds of each native step of the last profiled run, as ``(python step index, ms)``."""
        from lumen_amd import native as nv

        n = len(self.native_steps)
        arr = (C.c_float * max(1, n))()
        nv.call("nhip_plan_step_ms", self._native_plan(), arr, n)
        return [(self.native_steps[i], arr[i]) for i in range(n)]

    def cost(self, si):
        """Algorithmic ``(flops, bytes)`` of step ``si``: dots 2 m n k, flash attention 4 B N Sq Sk D (half of it
        causal; the backward 2.5x), loop kernels the bytes of their operands' distinct elements and outputs."""
        st = self.steps[si]
        g = self.graph

        def vbytes(v):
            loc = self.loc[v]
            n = 1
            for d, st_ in zip(loc.shape, loc.strides):
                if st_ != 0:
                    n *= d
            return n * D.size_of(loc.dtype)

        io = sum(vbytes(v) for v in st.inputs if v in self.loc) + sum(g.types[v].nbytes() for v in st.outputs)
        if st.kind == "dot":
            n = st.nodes[0]
            lt = g.types[n.inputs[0]]
            out = g.types[n.output]
            k = math.prod(lt.shape[d] for d in n.params["lhs_contracting"])
            return 2 * out.numel() * k, io
        if st.kind in ("flash_fwd", "flash_bwd"):
            n = st.nodes[0]
            q = g.types[n.inputs[0]]
            k = g.types[n.inputs[1]]
            if st.kind == "flash_fwd":
                qd, kd = n.params["q_dims"], n.params["k_dims"]
                b, h, sq, d = q.shape[qd[0][0]], q.shape[qd[0][1]], q.shape[qd[1]], q.shape[qd[2]]
                sk = k.shape[kd[1]]
            else:
                b, sq, h, d = q.shape
                sk = k.shape[1]
            f = 4 * b * h * sq * sk * d * (0.5 if n.params["causal"] else 1.0)
            return (f if st.kind == "flash_fwd" else 2.5 * f), io
        return 0, io

    def describe(self):
        """One line per step: its kind, name and label (``Plan.steps()``)."""
        return [
            {"kind": st.kind, "name": st.name, "label": st.label(), "outputs": list(st.outputs)} for st in self.steps
        ]


_ = math
