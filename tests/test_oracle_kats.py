"""The oracle pinned by known answers: the reference's Random123 vectors, IEEE rounding closed forms
(bfloat16 and float16 as one correct rounding of the float64 value), erf_inv round trips and the
reduce_precision / nextafter special cases."""

import math

import numpy as np
import pytest

from oracle import oracle


def test_philox_random123_vectors():
    """lumen/plan/tests.rs:224-247, tests/test_random.py:37-40."""
    kat = [
        ([0, 0], [0, 0, 0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
        ([0xFFFFFFFF] * 2, [0xFFFFFFFF] * 4, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
        ([0xA4093822, 0x299F31D0], [0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344],
         [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
    ]
    for key, ctr, block in kat:
        assert oracle.philox4x32(key, ctr) == block


def test_philox_bits_are_first_words_of_a_counter_stream():
    """random_bits' element i is word 0 of the block at counter start + i, key split low/high
    (reference/mod.rs:1162-1165)."""
    lib = oracle.lib()
    seed, start = (42 << 40) | 7, 1005
    for i in range(6):
        c = start + i
        want = oracle.philox4x32([seed & 0xFFFFFFFF, seed >> 32], [c & 0xFFFFFFFF, c >> 32, 0, 0])[0]
        assert lib.oracle_philox(seed, c) == want


def _np_bf16(x32):
    """The reference test's bf16 helper (tests/test_transformer_example.py:211-216): RNE on float32 bits."""
    bits = np.asarray(x32, np.float32).view(np.uint32)
    return ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16)


def test_bf16_of_float32_values_is_round_to_nearest_even():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(2000), rng.standard_normal(500) * 1e30, rng.standard_normal(500) * 1e-35])
    x32 = x.astype(np.float32)
    got = np.array([oracle.lib().oracle_to_bf16(float(v)) for v in x32], np.uint16)
    np.testing.assert_array_equal(got, _np_bf16(x32))


def test_bf16_of_float64_is_one_correct_rounding():
    """A float64 just above a bfloat16 tie rounds up; rounding through float32 first would land on the tie
    and round to even (down): round to odd avoids that double rounding (lumen/tensor/dtype.rs:217-229)."""
    tie = 1.0 + 2.0**-8                  # exactly halfway between bf16 1.0 and 1.0 + 2^-7
    above = tie + 2.0**-40               # rounds to 1.0 in float32, then to 1.0 (even) in bf16: wrong
    assert oracle.lib().oracle_to_bf16(above) == 0x3F81
    assert oracle.lib().oracle_to_bf16(tie) == 0x3F80       # ties to even
    assert oracle.lib().oracle_to_bf16(tie + 2.0**-7) == 0x3F82  # tie between 0x3F81 and 0x3F82 -> even
    assert oracle.lib().oracle_to_bf16(float("inf")) == 0x7F80
    assert oracle.lib().oracle_to_bf16(3.5e38) == 0x7F80     # past bf16's largest -> inf
    assert oracle.lib().oracle_to_bf16(-0.0) == 0x8000
    assert (oracle.lib().oracle_to_bf16(float("nan")) & 0x7FC0) == 0x7FC0


def test_f16_of_float64_matches_ieee():
    """numpy's float64 -> float16 conversion is IEEE round to nearest even in one step."""
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(3000) * s for s in (1.0, 1e-5, 1e-7, 3e4, 7e4)])
    got = np.array([oracle.lib().oracle_to_f16(float(v)) for v in x], np.uint16)
    np.testing.assert_array_equal(got, x.astype(np.float16).view(np.uint16))


def test_round_to_odd_brackets_and_is_odd():
    rng = np.random.default_rng(2)
    for v in rng.standard_normal(500):
        f = oracle.lib().oracle_round_to_odd(float(v))
        if float(np.float32(f)) != v:
            assert np.float32(f).view(np.uint32) & 1 == 1
            lo, hi = np.nextafter(np.float32(f), np.float32(-np.inf)), np.nextafter(np.float32(f), np.float32(np.inf))
            assert float(lo) < v < float(hi)


def test_erf_inv_round_trip():
    """erf(erf_inv(x)) = x to float32 precision; +-inf at +-1 (tests/codegen/test_elementwise.py:92-97)."""
    for v in np.concatenate([np.linspace(-0.999, 0.999, 101), [0.0, 1e-6, -1e-6]]):
        y = oracle.lib().oracle_erf_inv(float(v))
        assert math.erf(y) == pytest.approx(v, rel=1e-6, abs=1e-6)
    assert oracle.lib().oracle_erf_inv(1.0) == math.inf
    assert oracle.lib().oracle_erf_inv(-1.0) == -math.inf


def test_reduce_precision_is_bf16_and_f16_rounding():
    """reduce_precision(x, 8, 7) is bfloat16's rounding and (5, 10) float16's, in their normal ranges."""
    rng = np.random.default_rng(3)
    for v in rng.standard_normal(500):
        r = oracle.lib().oracle_reduce_precision(float(v), 8, 7)
        bf = np.array([_np_bf16(np.float64(v).astype(np.float32))], np.uint16).astype(np.uint32) << 16
        if float(np.float32(v)) == v:
            assert r == float(bf.view(np.float32)[0])
        h = oracle.lib().oracle_reduce_precision(float(v), 5, 10)
        assert h == float(np.float16(v))
