"""Pins the oracle of the WO projection (Q4_0 weights x Q8_0-quantized f32
activations) without restating it:

  quantize_row_q8_0 (nnml/src/ops/arm/arm.cpp:1819-1848)
    - every value lands within half a step of x / d, never outside +-127;
    - the block's largest magnitude maps to +-127 exactly;
    - halfway cases round to even (vcvtnq), shown on a block whose step is 1;
    - an all-zero block gives d = 0 and zero values;
  nnml_vec_dot_q4_0_q8_0 / mul_mat (arm.cpp:401, common.cpp:120)
    - equals the float64 product of the dequantized rows (dequantize_row_q4_0,
      types.cpp:337-350: low nibbles are weights 0..15, high nibbles 16..31,
      both minus 8) within the float32 summation bound;
    - with unit scales, bit for bit the integer dot product;
    - a one-hot weight picks out the matching activation (nibble order);
    - y[t, n] indexes (token, row) on a non-square case.
"""
import numpy as np
import pytest

from oracle import oracle

EPS32 = 2.0 ** -24


def f16(bits):
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float64)


def dequant_q4_0(w):
    """(N, nb) Q4_0 -> (N, 32 * nb) float64 weights."""
    lo = (w["qs"] & 0x0F).astype(np.int64) - 8
    hi = (w["qs"] >> 4).astype(np.int64) - 8
    vals = np.concatenate([lo, hi], axis=-1)                     # (N, nb, 32)
    return (vals * f16(w["d"])[..., None]).reshape(w.shape[0], -1)


def dequant_q8_0(q):
    return (q["qs"].astype(np.float64) * f16(q["d"])[..., None]).reshape(q.shape[0], -1)


def abs_bound(wd, xd):
    """Sum over k of |w_k x_k|: bounds every partial sum of the product."""
    return np.abs(xd) @ np.abs(wd).T


@pytest.fixture(scope="module")
def rng():
    return np.random.default_rng(20261201)


def test_q8_0_values_within_half_step(rng):
    x = (rng.standard_normal((6, 1024)) * np.logspace(-6, 3, 6)[:, None]).astype(np.float32)
    q = oracle.quantize_q8_0(x)
    xb = x.reshape(6, -1, 32).astype(np.float64)
    amax = np.abs(xb).max(-1)
    d = (amax.astype(np.float32) / np.float32(127)).astype(np.float32)
    # the stored scale is the f16 of amax / 127
    assert np.array_equal(q["d"], d.astype(np.float16).view(np.uint16))
    v = q["qs"].astype(np.float64)
    assert np.abs(v).max() <= 127
    # q = round(x * (1 / d)): within half a step (plus the rounding of 1 / d)
    scaled = xb * (1.0 / d.astype(np.float64))[..., None]
    assert np.all(np.abs(scaled - v) <= 0.5 + 1e-5)
    # the block maximum lands on +-127
    arg = np.abs(xb).argmax(-1)
    top = np.take_along_axis(v, arg[..., None], -1)[..., 0]
    assert np.all(np.abs(top) == 127)


def test_q8_0_ties_round_to_even():
    x = np.zeros((1, 32), np.float32)
    x[0, :9] = [127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -125.5]
    q = oracle.quantize_q8_0(x)
    assert f16(q["d"])[0, 0] == 1.0
    assert q["qs"][0, 0, :9].tolist() == [127, 0, 2, 2, 0, -2, -2, 126, -126]


def test_q8_0_zero_block():
    x = np.zeros((1, 64), np.float32)
    x[0, 32:] = 1.0
    q = oracle.quantize_q8_0(x)
    assert q["d"][0, 0] == 0 and not q["qs"][0, 0].any()
    assert np.all(q["qs"][0, 1] == 127)


def test_vec_dot_against_dequantized_float64(rng):
    K = 4096
    w = oracle.random_q4_0(rng, 8, K)
    x = rng.standard_normal((1, K)).astype(np.float32)
    q = oracle.quantize_q8_0(x)
    wd, xd = dequant_q4_0(w), dequant_q8_0(q)
    bound = abs_bound(wd, xd)[0]
    for n in range(8):
        got = oracle.vec_dot_q4_0_q8_0(w[n], q[0])
        want = float(wd[n] @ xd[0])
        assert abs(got - want) <= (K // 32 + 4) * 2 * EPS32 * bound[n], (n, got, want)


def test_vec_dot_unit_scales_is_the_integer_dot(rng):
    K = 1024
    w = oracle.random_q4_0(rng, 4, K)
    w["d"] = np.float16(1.0).view(np.uint16)
    x = rng.integers(-127, 128, size=(1, K)).astype(np.float32)
    x[0, ::32] = 127.0                                          # every block's step is 1
    q = oracle.quantize_q8_0(x)
    assert np.all(f16(q["d"]) == 1.0) and np.array_equal(q["qs"].reshape(1, -1), x.astype(np.int8))
    nib = np.concatenate([(w["qs"] & 0x0F).astype(np.int64) - 8, (w["qs"] >> 4).astype(np.int64) - 8], -1)
    ints = nib.reshape(4, -1) @ x[0].astype(np.int64)
    got = [oracle.vec_dot_q4_0_q8_0(w[n], q[0]) for n in range(4)]
    assert got == [float(v) for v in ints]


@pytest.mark.parametrize("j", [0, 5, 15, 16, 21, 31])
def test_one_hot_weight_picks_its_activation(j):
    K = 64
    w = np.zeros((1, K // 32), dtype=oracle.Q4_0)
    w["qs"] = 0x88                                              # every weight 0
    w["d"] = np.float16(0.5).view(np.uint16)
    b = 1
    if j < 16:
        w["qs"][0, b, j] = 0x8B                                 # low nibble 11 -> +3
    else:
        w["qs"][0, b, j - 16] = 0xB8                            # high nibble 11 -> +3
    x = np.arange(1, K + 1, dtype=np.float32)[None, :]
    y = oracle.mul_mat_q4_0(w, x)
    q = oracle.quantize_q8_0(x)
    want = 3 * 0.5 * q["qs"][0, b, j] * f16(q["d"])[0, b]
    assert y[0, 0] == np.float32(want)


def test_mul_mat_rows_and_tokens(rng):
    N, K, T = 48, 256, 3
    w = oracle.random_q4_0(rng, N, K)
    x = rng.standard_normal((T, K)).astype(np.float32)
    y = oracle.mul_mat_q4_0(w, x)
    assert y.shape == (T, N)
    wd, xd = dequant_q4_0(w), dequant_q8_0(oracle.quantize_q8_0(x))
    want = xd @ wd.T
    assert np.all(np.abs(y - want) <= (K // 32 + 4) * 2 * EPS32 * abs_bound(wd, xd))
    q = oracle.quantize_q8_0(x)
    for t, n in [(0, 47), (2, 0), (1, 17)]:
        assert y[t, n] == np.float32(oracle.vec_dot_q4_0_q8_0(w[n], q[t]))
