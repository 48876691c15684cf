"""Compiles the generated kernels of the benchmark's training-step plans into the kernel cache ahead of time.

``python -m lumen_amd.prebuild [TINY CONFIG4 CONFIG5]``; ``__graft_entry__.build()`` runs it. Tracing and
planning need no GPU, and the cache (``lumen_amd/_kcache``) travels with the tree, so a GPU run of these
steps finds every code object already built instead of compiling them on first use.
"""

from __future__ import annotations

import sys
import time

DEFAULT = ("TINY", "CONFIG4", "CONFIG5")


def prebuild(names=DEFAULT, verbose=False):
    import lumen_amd as L
    from lumen_amd import workloads as W
    from lumen_amd.compiler.plan import Plan
    from lumen_amd.graph.trace import trace

    for name in names:
        t = time.perf_counter()
        cfg = getattr(W, name)
        model, opt = W.build(cfg, lr=1e-2)
        W.load(model, W.init_weights(model))
        ids, targets = W.batch(cfg)
        traced = trace(W.train_step, (model, opt, L.from_numpy(ids), L.from_numpy(targets)))
        packable = [i for i, (kind, _) in enumerate(traced.layout) if kind == "weight"]
        plan = Plan(traced.graph, "hip:0", packable=packable)
        plan.build()
        if verbose:
            print(f"prebuild {name}: {len(plan.sources)} generated kernels cached "
                  f"({time.perf_counter() - t:.1f} s)", flush=True)


if __name__ == "__main__":
    prebuild(sys.argv[1:] or DEFAULT, verbose=True)
