"""Writes the transformer golden fixtures (``transformer_<case>.npz``) with the CPU oracle: the loss, and for
every parameter a fixed sample of its gradient and of its SGD-updated weight, plus each gradient's norm and
largest magnitude and the sum and norm of its every row and column. Run from the repository root:
``python -m tests.golden.make_transformer_golden [case ...]``.

The oracle evaluates the same traced graph the GPU test compiles (``trace`` of ``step_with_grads``).
"""

from __future__ import annotations

import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import lumen_amd as L  # noqa: E402
from lumen_amd import dtypes as D  # noqa: E402
from lumen_amd.graph.trace import trace  # noqa: E402
from oracle import oracle  # noqa: E402
from tests.golden import transformer_cases as TC  # noqa: E402


def oracle_inputs(traced, ids, targets, weights, names, lr):
    ins = []
    args = [ids, targets]
    for kind, k in traced.layout:
        if kind == "arg":
            ins.append(args[k])
        elif kind == "scalar":
            ins.append(np.array(lr, np.float64))
        else:
            ins.append(weights[names[id(traced.weights[k])]])
    return ins


def make(case):
    cfg = TC.CASES[case]
    model, opt, weights, ids, targets = TC.setup(cfg)
    names = {id(p): n for n, p in model.named_parameters()}
    args = (model, opt, L.from_numpy(ids), L.from_numpy(targets))
    traced = trace(TC.step_with_grads, args)
    t = time.time()
    outs = oracle.run(traced.graph, oracle_inputs(traced, ids, targets, weights, names, TC.LR))
    print(f"{case}: oracle {time.time() - t:.1f} s", flush=True)
    pnames = [n for n, _ in model.named_parameters()]
    shapes = {n: tuple(p.shape) for n, p in model.named_parameters()}
    data = {"loss": np.asarray(outs[0], np.float32)}
    gdt = [traced.graph.types[v].dtype for v in traced.graph.outputs]
    for j, name in enumerate(pnames):
        g = D.to_numpy_values(outs[1 + j], gdt[1 + j]).astype(np.float64).ravel()
        idx = TC.sample_indices(name, g.size)
        data[f"idx/{name}"] = idx
        data[f"grad/{name}"] = g[idx].astype(np.float32)
        data[f"grad_norm/{name}"] = np.array(np.linalg.norm(g))
        data[f"grad_max/{name}"] = np.array(np.abs(g).max())
        # every row's and every column's sum and norm (the gradient as [leading dims, last dim]): an error
        # confined to a few rows or columns, which the sampled entries may miss, moves them
        g2 = g.reshape(TC.as_rows(shapes[name]))
        for axis, part in ((1, "row"), (0, "col")):
            data[f"{part}sum/{name}"] = g2.sum(axis=axis).astype(np.float32)
            data[f"{part}norm/{name}"] = np.sqrt((g2 * g2).sum(axis=axis)).astype(np.float32)
    written = {names[id(traced.weights[k])]: 1 + len(pnames) + j for j, k in enumerate(traced.written)}
    for name in pnames:
        w = np.asarray(outs[written[name]]).ravel()  # bf16 bits
        data[f"new/{name}"] = w[data[f"idx/{name}"]]
    meta = {"case": case, "config": cfg.__dict__, "lr": TC.LR, "digest": TC.input_digest(weights, ids),
            "grad_dtypes": dict(zip(pnames, gdt[1:])), "params": pnames}
    data["meta"] = np.array(json.dumps(meta))
    path = os.path.join(HERE, f"transformer_{case}.npz")
    np.savez_compressed(path, **data)
    print(f"wrote {path} ({os.path.getsize(path) / 1e3:.0f} KB)")


if __name__ == "__main__":
    oracle.set_threads(os.cpu_count() or 1)
    for c in sys.argv[1:] or list(TC.CASES):
        make(c)
