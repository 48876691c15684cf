"""``lumen_amd.config``: compiler flags the hip pipeline reads (``lumen/graph_compiler/config/mod.rs:82-133``)
and the static region size (``lumen/allocator/config.rs:14-25``)."""

from __future__ import annotations

import contextlib
import dataclasses


@dataclasses.dataclass
class CompilerFlags:
    fuse: bool = True                 # loop fusion of elementwise/row work
    flash_attention: bool = True      # match attention (forward and backward) into flash kernels
    merge_dots: bool = True           # one dot for dots sharing an operand (QKV)
    horizontal_fusion: bool = True    # merge small independent loop kernels into one launch
    epilogue_fusion: bool = True      # fuse elementwise consumers into GEMM stores
    autotune: bool = True             # time GEMM tile candidates before a plan's first run
    # attention backward without atomics: dQ by a kernel of its own (same bits every run); off, as in the
    # reference (graph_compiler/config/mod.rs:117), the dK/dV kernel adds dQ atomically
    deterministic: bool = True
    # deterministic attention backward: the dK/dV kernel stores dS (16-bit, B x N x Sk x Sq / 2 bytes causal) and
    # dQ = dS K reads it back, instead of a second kernel recomputing S and dP (off: no dS workspace)
    attention_store_ds: bool = True
    # above this many bytes of dS tiles for one attention the deterministic backward recomputes S and dP
    # instead (its workspace is O(Sq)), so long sequences do not need O(Sq x Sk) memory
    attention_ds_max_bytes: int = 4 << 30
    hip_graphs: bool = True           # replay a plan's calls as a captured HIP graph (from its third call)
    # a weight the compiled function assigns is computed over its old value where the step producing it reads
    # the old value only at the element it writes and nothing reads it later (off: into the workspace, then
    # copied back after the run)
    update_in_place: bool = True
    # simplify's structural rewrites after pattern matching (swapped/folded dots, ops moved across layouts)
    simplify_structural: bool = True
    # try the list and depth-first step schedules and keep the order needing the least workspace
    schedules: bool = True
    # workspace bytes a plan should fit in (0: no limit); above it values are rematerialized
    # (graph_compiler/config/mod.rs:90 memory_limit)
    memory_limit: int = 0
    # a cross entropy over h . w^T logits nothing else reads becomes one linear_cross_entropy step
    # (graph_compiler/config/mod.rs:115, on by default)
    fused_linear_cross_entropy: bool = True
    # rows a chunk of the fused linear cross entropy backward (None: off, the reference's default)
    fused_linear_cross_entropy_chunk_size: int | None = None
    _version: int = 0

    def __setattr__(self, name, value):
        object.__setattr__(self, name, value)
        if name != "_version":
            object.__setattr__(self, "_version", self._version + 1)

    @contextlib.contextmanager
    def patch(self, **flags):
        old = {k: getattr(self, k) for k in flags}
        for k, v in flags.items():
            setattr(self, k, v)
        try:
            yield self
        finally:
            for k, v in old.items():
                setattr(self, k, v)

    def key(self):
        from lumen_amd import autotune

        flags = tuple((f.name, getattr(self, f.name)) for f in dataclasses.fields(self) if f.name != "_version")
        return flags + (("forced", autotune.forced_key()),)


@dataclasses.dataclass
class Config:
    compiler: CompilerFlags = dataclasses.field(default_factory=CompilerFlags)
    # The static region weights and small tensors are carved from on each device (the reference's default is
    # 1 GiB, allocator/config.rs:14-25; an MI355X has 288 GB, and the 12-layer step's weights alone are 1.5 GB).
    # Blocks over a quarter of it (plan workspaces) get allocations of their own.
    static_allocator_bytes: int = 16 << 30


config = Config()
