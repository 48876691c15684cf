"""The benchmark workloads as lumen programs: the decoder-only transformer training step of configs 4 and 5
(``examples/transformer.py`` style: pre-norm blocks, causal flash attention, a GELU FFN, a cross-entropy head,
autograd backward and an SGD update inside one compiled function) and its synthetic inputs.

Weights are bfloat16 (norm scales too), every dot accumulates in float32, and the norm statistics, softmax
and loss are float32.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

import lumen_amd as L
import lumen_amd.functional as F
from lumen_amd import dtypes as D
from lumen_amd.nn import Module


@dataclass(frozen=True)
class TransformerConfig:
    vocab: int
    dim: int
    heads: int
    ffn: int
    seq: int
    batch: int
    layers: int

    @property
    def head_dim(self):
        return self.dim // self.heads

    @property
    def tokens(self):
        return self.batch * self.seq

    def step_flops(self):
        """Algorithmic FLOPs of one training step: 3x the forward's dots (forward, two gradients), causal
        attention counted at half the square."""
        t, d, f, v = self.tokens, self.dim, self.ffn, self.vocab
        per_layer = 2 * t * d * 3 * d + 2 * t * d * d + 2 * 2 * t * d * f + 2 * self.batch * self.heads * self.seq**2 * self.head_dim
        fwd = self.layers * per_layer + 2 * t * d * v
        return 3 * fwd


# The benchmark's configs 4 (2 layers, d 512) and 5 (12 layers, d 2048), and a small one for parity tests
# and the smoke check.
CONFIG4 = TransformerConfig(vocab=32000, dim=512, heads=8, ffn=2048, seq=512, batch=16, layers=2)
CONFIG5 = TransformerConfig(vocab=32000, dim=2048, heads=16, ffn=8192, seq=4096, batch=4, layers=12)
TINY = TransformerConfig(vocab=256, dim=128, heads=2, ffn=256, seq=128, batch=2, layers=2)


class Embedding(Module):
    tokens: L.Tensor
    positions: L.Tensor

    def __call__(self, ids):
        b, s = ids.shape
        return (self.tokens[ids] + self.positions).reshape(b * s, self.tokens.shape[1])


class Attention(Module):
    norm: L.Tensor
    wq: L.Tensor
    wk: L.Tensor
    wv: L.Tensor
    wo: L.Tensor

    def __call__(self, x, batch, heads):
        tokens, dim = x.shape
        q, k, v = (
            F.matmul(x, w.t(), "float32", "bfloat16").reshape(batch, tokens // batch, heads, dim // heads)
            for w in (self.wq, self.wk, self.wv)
        )
        o = F.flash_attention(q, k, v, is_causal=True)
        return F.matmul(o.reshape(tokens, dim), self.wo.t(), "float32", "bfloat16")


class MLP(Module):
    norm: L.Tensor
    w1: L.Tensor
    w2: L.Tensor

    def __call__(self, x):
        h = F.gelu(F.matmul(x, self.w1.t(), "float32", "float32")).bfloat16()
        return F.matmul(h, self.w2.t(), "float32", "bfloat16")


class Block(Module):
    attn: Attention
    mlp: MLP

    def __call__(self, x, batch, heads):
        r = x
        x = F.rms_norm(x.float(), x.size(-1), self.attn.norm.float()).bfloat16()
        x = r + self.attn(x, batch, heads)
        r = x
        x = F.rms_norm(x.float(), x.size(-1), self.mlp.norm.float()).bfloat16()
        return r + self.mlp(x)


class Transformer(Module):
    embed: Embedding
    layers: list
    norm: L.Tensor
    head: L.Tensor
    heads: int

    def __call__(self, ids):
        h = self.embed(ids)
        for layer in self.layers:
            h = layer(h, ids.shape[0], self.heads)
        return F.rms_norm(h.float(), h.size(-1), self.norm.float()).bfloat16()


class SGD(Module):
    """``p - lr * g`` for each parameter (``examples/optim.py:7-24``)."""

    params: list
    lr: float

    def step(self):
        for p in self.params:
            if p.grad is not None:
                p.copy_(p - self.lr * p.grad)


def loss_fn(model, ids, targets):
    h = model(ids)
    logits = F.matmul(h, model.head.t(), "float32", "float32")
    return F.mean(F.cross_entropy(logits, targets.reshape(-1)))


def train_step(model, opt, ids, targets):
    """One step: the loss, its gradient by autograd, and the SGD update; returns the loss."""
    loss = loss_fn(model, ids, targets)
    loss.backward()
    opt.step()
    return loss


def build(cfg: TransformerConfig, lr=1e-2):
    """The model (meta weights) and its SGD optimizer."""

    def w(*shape):
        return L.empty(list(shape), "bfloat16", "meta")

    d = cfg.dim
    model = Transformer(
        embed=Embedding(w(cfg.vocab, d), w(cfg.seq, d)),
        layers=[
            Block(Attention(w(d), w(d, d), w(d, d), w(d, d), w(d, d)), MLP(w(d), w(cfg.ffn, d), w(d, cfg.ffn)))
            for _ in range(cfg.layers)
        ],
        norm=w(d),
        head=w(cfg.vocab, d),
        heads=cfg.heads,
    )
    return model, SGD(model.parameters(), lr)


def init_weights(model, seed=0):
    """N(0, 0.02) weights, norm scales 1 (bfloat16 bits, by parameter path)."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, p in model.named_parameters():
        if len(p.shape) == 1:
            vals = np.ones(p.shape, np.float32)
        else:
            vals = (0.02 * rng.standard_normal(p.shape)).astype(np.float32)
        out[name] = D.bf16_bits(vals)
    return out


def load(model, weights):
    model.load_state_dict({k: L.Tensor("bfloat16", v.shape, "cpu", host=v) for k, v in weights.items()})


def batch(cfg: TransformerConfig, seed=1):
    """Uniform token ids and next-token targets, int64 [batch, seq]."""
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, cfg.vocab, (cfg.batch, cfg.seq)).astype(np.int64)
    return ids, np.roll(ids, -1, axis=1)


_ = math
