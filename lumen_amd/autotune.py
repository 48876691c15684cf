"""Kernel configs forced in place of the autotuner's pick (``lumen.autotune``: ``use``, the config classes;
``lumen/autotune/forced.rs:1-45``).

Inside ``with use(HipGemmConfig(9), HipAttentionConfig(waves=8)):`` every plan compiled runs each kernel of a
family given a config with that config, untimed, whether ``config.compiler.autotune`` is on or not and at any
size. An inner block's config of a family replaces an outer one's. Plans compiled inside a block are keyed on
its configs, so leaving it compiles again with the autotuner's picks.
"""

from __future__ import annotations

import contextlib

_FORCED: list = []  # the configs of each enclosing `use` block, innermost last


def _count(fn_name):
    import ctypes as C

    from lumen_amd import native

    n = C.c_int()
    native.call(fn_name, C.byref(n))
    return n.value


class HipGemmConfig:
    """A tile config of the MFMA GEMM (``nhip_gemm_desc.config``): an index into ``kernels.hip``'s table — the
    tiled register-staged kernels from 256x256 down to 64x64, then the streamed kernels (256x256 with 4 or 8
    waves, 8 waves with 32-deep k steps, 128x128, persistent 256x256). Applies to dots planned as plain GEMM
    steps (not to a GEMM with a fused epilogue, which is generated around the streamed kernel, nor to
    split-k steps)."""

    def __init__(self, index: int):
        count = _count("nhip_gemm_config_count")
        if not 0 <= int(index) < count:
            raise ValueError(f"HipGemmConfig: config {index} is not one of the {count} GEMM tile configs")
        self.index = int(index)

    @staticmethod
    def candidates() -> list:
        """Every config the autotuner times."""
        return [HipGemmConfig(i) for i in range(_count("nhip_gemm_config_count"))]

    def key(self):
        return ("gemm", self.index)

    def __eq__(self, other):
        return isinstance(other, HipGemmConfig) and other.index == self.index

    def __hash__(self):
        return hash(self.key())

    def __repr__(self):
        return f"HipGemmConfig({self.index})"


class HipAttentionConfig:
    """A tile config of the flash-attention forward kernel (``nhip_attn_desc.config``): the waves of 32 queries
    a workgroup runs over each K/V tile it streams (4: 128 queries, the default; 8: 256; 2: 64)."""

    WAVES = (4, 8, 2)  # config index -> waves

    def __init__(self, waves: int = 4):
        if waves not in self.WAVES:
            raise ValueError(f"HipAttentionConfig: waves must be one of {self.WAVES}, got {waves}")
        self.waves = int(waves)

    @property
    def index(self) -> int:
        return self.WAVES.index(self.waves)

    @staticmethod
    def candidates() -> list:
        return [HipAttentionConfig(w) for w in HipAttentionConfig.WAVES]

    def fits(self, h: int, hv: int) -> bool:
        """Whether the flash forward takes query/key head dim ``h`` and value head dim ``hv`` (each a multiple of 8
        up to 256)."""
        return all(0 < d <= 256 and d % 8 == 0 for d in (h, hv))

    def key(self):
        return ("attention", self.waves)

    def __eq__(self, other):
        return isinstance(other, HipAttentionConfig) and other.waves == self.waves

    def __hash__(self):
        return hash(self.key())

    def __repr__(self):
        return f"HipAttentionConfig(waves={self.waves})"


@contextlib.contextmanager
def use(*configs):
    """Forces ``configs`` (at most one of each family) for plans compiled inside the block."""
    kinds = [type(c) for c in configs]
    if len(set(kinds)) != len(kinds):
        raise ValueError("autotune.use: at most one config of each kernel family a block")
    for c in configs:
        if not isinstance(c, (HipGemmConfig, HipAttentionConfig)):
            raise TypeError(f"autotune.use: {c!r} is not a hip kernel config")
    _FORCED.append(list(configs))
    try:
        yield
    finally:
        _FORCED.pop()


def forced(cls):
    """The config of family ``cls`` the innermost block forcing one gives, else None."""
    for block in reversed(_FORCED):
        for c in block:
            if isinstance(c, cls):
                return c
    return None


def forced_key() -> tuple:
    """The effective forced configs, for plan cache keys."""
    return tuple(c.key() for c in (forced(HipGemmConfig), forced(HipAttentionConfig)) if c is not None)
