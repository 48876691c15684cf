"""The transformer training-step cases the golden fixtures hold (shared by the generator, which runs the CPU
oracle, and the GPU test, which runs the same program compiled for hip).

Each case is the benchmark decoder (``lumen_amd.workloads``) at a named size: ``config4_b1`` is config 4's
model at its real shapes (vocab 32000, d 512, 8 heads, FFN 2048, seq 512, 2 layers) with batch 1 of the 16;
``config5_layer`` is one config-5 layer (d 2048, 16 heads of 128, FFN 8192, vocab 32000) at batch 1 and
sequence ``CONFIG5_SEQ`` (config 5's own 4096; the oracle, threaded over rows, finishes it in about 7
minutes).
The program is one SGD training step that also returns every gradient, so one run yields the loss, each
gradient and each updated weight.
"""

from __future__ import annotations

import dataclasses

import numpy as np

from lumen_amd import workloads as W

CONFIG5_SEQ = 4096
LR = 1.0  # the SGD step's learning rate: updates of order 1e-4..1e-2, visible in bf16 weights of ~0.02
SAMPLES = 2048  # gradient / weight entries kept per parameter
CASES = {
    "config4_b1": dataclasses.replace(W.CONFIG4, batch=1),
    "config5_layer": dataclasses.replace(W.CONFIG5, batch=1, layers=1, seq=CONFIG5_SEQ),
}


def step_with_grads(model, opt, ids, targets):
    """The training step (loss, autograd backward, SGD update) returning the loss and every gradient."""
    loss = W.loss_fn(model, ids, targets)
    loss.backward()
    grads = [p.grad for p in model.parameters()]
    opt.step()
    return [loss] + grads


def setup(cfg):
    """Model, optimizer, bf16 weight bits by name and int64 ids / targets, all seeded (weights seed 0,
    ids seed 1)."""
    model, opt = W.build(cfg, lr=LR)
    weights = W.init_weights(model)
    W.load(model, weights)
    ids, targets = W.batch(cfg)
    return model, opt, weights, ids, targets


def as_rows(shape):
    """A parameter's shape as [rows, columns]: its leading dims flattened, its last dim the columns (a vector is
    one row)."""
    shape = tuple(shape)
    cols = shape[-1] if shape else 1
    return (int(np.prod(shape[:-1], dtype=np.int64)) if len(shape) > 1 else 1, cols)


def sample_indices(name, numel, k=SAMPLES):
    """Fixed flat indices of a parameter: its first and last entries and a seeded uniform sample."""
    seed = sum(ord(c) * (i + 1) for i, c in enumerate(name)) % (2**31)
    rng = np.random.default_rng(seed)
    idx = np.unique(np.concatenate([[0, numel - 1], rng.integers(0, numel, k)]))
    return idx.astype(np.int64)


def input_digest(weights, ids):
    """A checksum of the seeded inputs (so a fixture is only compared on the inputs it was made from)."""
    import hashlib

    h = hashlib.sha256()
    for name in sorted(weights):
        h.update(name.encode())
        h.update(np.ascontiguousarray(weights[name]).tobytes())
    h.update(np.ascontiguousarray(ids).tobytes())
    return h.hexdigest()[:32]
