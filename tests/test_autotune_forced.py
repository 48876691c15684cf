"""Forced kernel configs (``lumen.autotune.use``, ``lumen/autotune/forced.rs``): the config classes, the
block stack, and plan cache keys that change with the forced configs."""

import pytest

import lumen_amd as L
from lumen_amd import autotune as A


def test_config_classes_and_candidates():
    gemms = A.HipGemmConfig.candidates()
    assert len(gemms) >= 5 and [c.index for c in gemms] == list(range(len(gemms)))
    with pytest.raises(ValueError):
        A.HipGemmConfig(len(gemms))
    attn = A.HipAttentionConfig.candidates()
    assert [c.waves for c in attn] == [4, 8, 2] and [c.index for c in attn] == [0, 1, 2]
    with pytest.raises(ValueError):
        A.HipAttentionConfig(waves=3)
    assert attn[0].fits(128, 128) and attn[0].fits(32, 32) and attn[0].fits(256, 256) and attn[0].fits(96, 96)
    assert attn[0].fits(64, 128) and not attn[0].fits(20, 20) and not attn[0].fits(264, 264)
    assert not attn[0].fits(64, 12)


def test_use_blocks_nest_and_key_plans():
    base = L.config.compiler.key()
    assert A.forced(A.HipGemmConfig) is None
    with A.use(A.HipGemmConfig(9)):
        assert A.forced(A.HipGemmConfig) == A.HipGemmConfig(9)
        outer = L.config.compiler.key()
        assert outer != base
        with A.use(A.HipGemmConfig(0), A.HipAttentionConfig(waves=8)):  # the inner block's config wins
            assert A.forced(A.HipGemmConfig) == A.HipGemmConfig(0)
            assert A.forced(A.HipAttentionConfig).waves == 8
            assert L.config.compiler.key() != outer
        assert A.forced(A.HipGemmConfig) == A.HipGemmConfig(9)
        assert A.forced(A.HipAttentionConfig) is None
    assert L.config.compiler.key() == base
    with pytest.raises(ValueError):
        with A.use(A.HipGemmConfig(0), A.HipGemmConfig(1)):
            pass
