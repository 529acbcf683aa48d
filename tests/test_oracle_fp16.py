"""Pins the oracle's IEEE binary16 conversions (restating nnml/include/ops.h:
276-323) bit for bit against numpy's float16 conversion (IEEE RNE)."""
import numpy as np

from oracle import oracle as O


def test_f16_to_f32_all_patterns():
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    got = O.f16_bits_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_roundtrip_of_every_f16():
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    f = h.view(np.float16).astype(np.float32)
    nan = np.isnan(f)
    got = O.f32_to_f16_bits(f)
    assert np.array_equal(got[~nan], h[~nan])
    assert np.isnan(got[nan].view(np.float16)).all()


def test_f32_to_f16_random_and_edge_patterns():
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2**32, size=4_000_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    # ties, around the subnormal boundary and the overflow threshold
    ties = (np.float32(1.0) + np.arange(1, 2049, dtype=np.float32) * np.float32(2.0 ** -11)).astype(np.float32)
    edges = np.array([0.0, -0.0, 65504.0, 65519.996, 65520.0, -65520.0, 2.0 ** -14, 2.0 ** -24,
                      2.0 ** -25, 2.0 ** -25 * 1.0000001, 2.0 ** -24 * 1.5, 6.0975552e-05, np.inf, -np.inf],
                     dtype=np.float32)
    x = np.concatenate([x, ties, edges, -ties])
    got = O.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.isnan(got[nan].view(np.float16)).all()
