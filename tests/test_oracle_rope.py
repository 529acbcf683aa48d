"""The oracle of the attention-operand producers (orc_rms_norm_rope_f32, a
restatement of nnml's rms_norm f32, mul and rope f32: nnml/src/ops/ops.cpp:
680-726, 728-777, 871-962) pinned against what the mathematics fixes:
RMSNorm of a constant row, rotation at position 0, unit vectors rotating
by (cos p, sin p) into the right partner dimension, an independent float64
evaluation of the rotation (only the float32 angle recurrence shared, as
the reference carries it), norm preservation, the relative-position
property, and the YaRN ramp from its published formula."""
import math

import numpy as np
import pytest

from arclight_amd import abi
from oracle import oracle as O

D = 128


def _rope(mode=abi.AL_ROPE_NEOX, base=1e6, freq_scale=1.0, ext=0.0, attn=1.0, n_ctx=40960, bf=32.0, bs=1.0):
    return abi.AlRopeParams(D, mode, n_ctx, base, freq_scale, ext, attn, bf, bs)


def _theta_chain(p, base):
    """Angles of the 64 pairs as the reference's cache carries them: the
    position times theta_scale, i times, in float32."""
    ts = np.float32(np.power(np.float32(base), np.float32(-2.0 / D)))
    th = np.empty(D // 2, np.float32)
    t = np.float32(p)
    for i in range(D // 2):
        th[i] = t
        t = np.float32(t * ts)
    return th


def _rms(x, w, eps):
    """float64 RMSNorm of rows (T, H, D)."""
    x64 = x.astype(np.float64)
    y = x64 / np.sqrt((x64 * x64).mean(-1, keepdims=True) + eps)
    return y * (1.0 if w is None else w.astype(np.float64))


def test_rms_norm_constant_row_closed_form():
    x = np.full((2, 3, D), 0.75, np.float32)
    w = np.linspace(-2, 2, D).astype(np.float32)
    y = O.rms_norm_rope(x, w, eps=1e-6)
    want = 0.75 / math.sqrt(0.75 ** 2 + 1e-6) * w.astype(np.float64)
    np.testing.assert_allclose(y, np.broadcast_to(want, y.shape), rtol=2e-7, atol=1e-7)


def test_rms_norm_matches_float64():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((5, 8, D)) * rng.uniform(0.01, 30, (5, 8, 1))).astype(np.float32)
    w = rng.standard_normal(D).astype(np.float32)
    y = O.rms_norm_rope(x, w, eps=1e-5)
    np.testing.assert_allclose(y, _rms(x, w, 1e-5), rtol=1e-6, atol=1e-6)


def test_position_zero_is_identity():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 4, D)).astype(np.float32)
    w = rng.standard_normal(D).astype(np.float32)
    plain = O.rms_norm_rope(x, w, eps=1e-6)
    for mode in (abi.AL_ROPE_NEOX, abi.AL_ROPE_NORMAL):
        y = O.rms_norm_rope(x, w, np.zeros(3, np.int32), eps=1e-6, rope=_rope(mode))
        assert np.array_equal(y, plain)                   # cos 0 = 1, sin 0 = 0 exactly


@pytest.mark.parametrize("mode", [abi.AL_ROPE_NEOX, abi.AL_ROPE_NORMAL])
def test_unit_vectors_rotate_into_their_partner(mode):
    # e_i at position p lands on (cos theta_i, sin theta_i) in dims (i, partner)
    p = 1234
    th = _theta_chain(p, 1e6).astype(np.float64)
    for i in (0, 1, 17, 63):
        a, b = (i, i + 64) if mode == abi.AL_ROPE_NEOX else (2 * i, 2 * i + 1)
        x = np.zeros((1, 2, D), np.float32)
        x[0, 0, a] = 1.0                                  # first element of pair i
        x[0, 1, b] = 1.0                                  # second element
        y = O.rms_norm_rope(x, None, np.array([p], np.int32), eps=0.0, rope=_rope(mode))[0] / math.sqrt(D)
        c, s = math.cos(th[i]), math.sin(th[i])
        assert y[0, a] == pytest.approx(c, abs=2e-6) and y[0, b] == pytest.approx(s, abs=2e-6)
        assert y[1, a] == pytest.approx(-s, abs=2e-6) and y[1, b] == pytest.approx(c, abs=2e-6)
        others = np.ones(D, bool)
        others[[a, b]] = False
        assert not y[:, others].any()


@pytest.mark.parametrize("mode", [abi.AL_ROPE_NEOX, abi.AL_ROPE_NORMAL])
def test_rotation_matches_float64_evaluation(mode):
    rng = np.random.default_rng(2)
    T, H = 6, 5
    x = rng.standard_normal((T, H, D)).astype(np.float32)
    w = rng.standard_normal(D).astype(np.float32)
    pos = np.array([0, 1, 77, 4095, 32767, 40959], np.int32)
    y = O.rms_norm_rope(x, w, pos, eps=1e-6, rope=_rope(mode))
    n = _rms(x, w, 1e-6)
    for t in range(T):
        th = _theta_chain(pos[t], 1e6).astype(np.float64)
        c, s = np.cos(th), np.sin(th)
        if mode == abi.AL_ROPE_NEOX:
            x0, x1 = n[t, :, :64], n[t, :, 64:]
            want = np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], -1)
        else:
            x0, x1 = n[t, :, 0::2], n[t, :, 1::2]
            want = np.empty_like(n[t])
            want[:, 0::2] = x0 * c - x1 * s
            want[:, 1::2] = x0 * s + x1 * c
        np.testing.assert_allclose(y[t], want, rtol=0, atol=5e-6)


def test_angles_follow_the_frequency_law_at_small_positions():
    # theta_i = p * base^(-2i/128): the float32 recurrence stays within 1e-5
    # rad of the closed form for p <= 100, so a wrong exponent or base fails
    for p in (1, 3, 100):
        th = _theta_chain(p, 1e6).astype(np.float64)
        want = p * 1e6 ** (-2.0 * np.arange(64) / D)
        np.testing.assert_allclose(th, want, rtol=0, atol=1e-5)
        x = np.zeros((1, 1, D), np.float32)
        x[0, 0, :64] = 1.0
        y = O.rms_norm_rope(x, None, np.array([p], np.int32), eps=0.0, rope=_rope())[0, 0] / math.sqrt(2)
        np.testing.assert_allclose(y[:64], np.cos(want), atol=2e-5)
        np.testing.assert_allclose(y[64:], np.sin(want), atol=2e-5)


def test_norm_and_relative_position_preserved():
    rng = np.random.default_rng(3)
    q = rng.standard_normal((1, 1, D)).astype(np.float32)
    k = rng.standard_normal((1, 1, D)).astype(np.float32)

    def rot(v, p):
        return O.rms_norm_rope(v, None, np.array([p], np.int32), eps=0.0, rope=_rope(base=1e4))[0, 0].astype(np.float64)

    base = O.rms_norm_rope(q, None, eps=0.0)[0, 0].astype(np.float64)
    r = rot(q, 1000)
    for i in range(64):                                   # every NEOX pair keeps its length
        assert math.hypot(r[i], r[i + 64]) == pytest.approx(math.hypot(base[i], base[i + 64]), rel=1e-5)
    d1 = rot(q, 7) @ rot(k, 3)
    d2 = rot(q, 104) @ rot(k, 100)
    d3 = rot(q, 3) @ rot(k, 7)
    assert d1 == pytest.approx(d2, abs=2e-3)              # depends on m - n only
    assert abs(d1 - d3) > 1e-2                            # and on its sign


def test_yarn_ramp_against_published_formula():
    # YaRN (Peng et al. 2023): theta = theta_interp (1 - mix) + theta_extrap mix,
    # mix = ext_factor * (1 - clamp((i - low) / (high - low), 0, 1)),
    # magnitude scaled by 1 + 0.1 ln(1 / freq_scale)
    fs, ext, attn, base, n_ctx, bf, bs = 0.25, 1.0, 1.0, 1e4, 4096, 32.0, 1.0
    rope = _rope(base=base, freq_scale=fs, ext=ext, attn=attn, n_ctx=n_ctx, bf=bf, bs=bs)

    def corr_dim(n_rot):
        return D * math.log(n_ctx / (n_rot * 2 * math.pi)) / (2 * math.log(base))

    low, high = max(0.0, math.floor(corr_dim(bf))), min(D - 1.0, math.ceil(corr_dim(bs)))
    p = 2000
    th = _theta_chain(p, base).astype(np.float64)
    i = np.arange(64)
    mix = ext * (1 - np.clip((i - low) / max(0.001, high - low), 0, 1))
    theta = fs * th * (1 - mix) + th * mix
    msc = attn * (1 + 0.1 * math.log(1 / fs))
    x = np.zeros((1, 1, D), np.float32)
    x[0, 0, :64] = 1.0
    y = O.rms_norm_rope(x, None, np.array([p], np.int32), eps=0.0, rope=rope)[0, 0] / math.sqrt(2)
    np.testing.assert_allclose(y[:64], np.cos(theta) * msc, atol=5e-5)
    np.testing.assert_allclose(y[64:], np.sin(theta) * msc, atol=5e-5)
    assert mix[0] == ext and mix[-1] == 0.0               # the ramp really spans the pairs


def test_rejects_unsupported():
    x = np.zeros((1, 1, D), np.float32)
    with pytest.raises(ValueError):
        O.rms_norm_rope(x, None, np.zeros(1, np.int32), eps=1e-6, rope=abi.AlRopeParams(64, 2, 0, 1e4, 1, 0, 1, 32, 1))
    with pytest.raises(ValueError):
        O.rms_norm_rope(x, None, np.zeros(1, np.int32), eps=1e-6, rope=abi.AlRopeParams(128, 8, 0, 1e4, 1, 0, 1, 32, 1))
