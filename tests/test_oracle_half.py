"""Pins the oracle's half floats (crates/native-engine/src/half.rs) against
numpy's IEEE binary16 (round to nearest, ties to even) and the reference's
own known answers (half.rs:194-233)."""

import numpy as np


def test_every_half_widens_like_numpy(oracle):
    h = np.arange(65536, dtype=np.uint16)
    got = oracle.half_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_round_trip_every_half(oracle):
    h = np.arange(65536, dtype=np.uint16)
    back = oracle.f32_to_half(oracle.half_to_f32(h))
    nan = np.isnan(h.view(np.float16))
    assert np.array_equal(back[~nan], h[~nan])
    assert np.isnan(back[nan].view(np.float16)).all()


def test_random_float_bits_narrow_like_numpy(oracle):
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2**32, 1 << 20, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    got = oracle.f32_to_half(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.isnan(got[nan].view(np.float16)).all()


def test_reference_known_answers(oracle):
    """half.rs:204-232, verbatim cases."""
    f = lambda v: int(oracle.f32_to_half(np.float32([v]))[0])
    assert f(1.0 + 2.0**-11) == 0x3C00
    assert f(1.0 + 3.0 * 2.0**-11) == 0x3C02
    assert f(2.0**-25) == 0
    assert f(3.0 * 2.0**-25) == 2
    assert f(-(2.0**-26)) == 0x8000
    assert f(65504.0) == 0x7BFF
    assert f(65519.0) == 0x7BFF
    assert f(65520.0) == 0x7C00
    assert f(-np.inf) == 0xFC00
    cases = [(0x3C00, 1.0), (0xC000, -2.0), (0x7BFF, 65504.0), (0x3555, 0.33325195),
             (0x0001, 2.0**-24), (0x83FF, -1023.0 * 2.0**-24), (0x8000, -0.0), (0x7C00, np.inf)]
    for h, want in cases:
        got = oracle.half_to_f32(np.uint16([h]))[0]
        assert np.float32(got).view(np.uint32) == np.float32(want).view(np.uint32), hex(h)
    assert np.isnan(oracle.half_to_f32(np.uint16([0x7E00]))[0])
