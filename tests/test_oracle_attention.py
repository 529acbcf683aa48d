"""Pins the CPU oracle of nnml_compute_forward_flash_attn_ext_f16
(nnml/src/ops/arm/arm.cpp:2196-2433) without trusting its own formula:
O1 (fp64 brute force) against scipy's softmax attention; O2 (the parity
oracle) against O1; both against closed forms and invariants chosen so that a
dropped term, a wrong sign or index or a transposed operand fails a test.
"""
import math

import numpy as np
import pytest
from scipy.special import softmax

from oracle import oracle as O

SCALE = 1.0 / math.sqrt(128)


def rel(a, b):
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def scipy_attention(q, k, v, mask=None, *, scale, kv_len=0, causal_pos0=-1, sinks=None):
    """Textbook attention in float64 from numpy/scipy primitives, with the
    reference's Q -> f16 rounding and mask semantics (-inf cells skipped)."""
    B, T, Hq, D = q.shape
    n_kv, Hkv = k.shape[1], k.shape[2]
    G = Hq // Hkv
    q16 = q.astype(np.float16).astype(np.float64)
    kf, vf = k.astype(np.float64), v.astype(np.float64)
    kv_len = n_kv if kv_len <= 0 else kv_len
    out = np.empty((B, T, Hq, v.shape[3]))
    for b in range(B):
        for t in range(T):
            for h in range(Hq):
                s = kf[b % k.shape[0], :, h // G, :] @ q16[b, t, h] * scale
                add = np.zeros(n_kv)
                if mask is not None:
                    add = mask[b % mask.shape[0], h % mask.shape[1], t].astype(np.float64)
                add[np.arange(n_kv) >= kv_len] = -np.inf
                if causal_pos0 >= 0:
                    add[np.arange(n_kv) > causal_pos0 + t] = -np.inf
                vis = add != -np.inf
                logits = s[vis] + add[vis]
                if sinks is not None:
                    w = softmax(np.append(logits, sinks[h]))[:-1]
                else:
                    w = softmax(logits) if vis.any() else np.zeros(0)
                out[b, t, h] = w @ vf[b % v.shape[0], vis, h // G, :] if vis.any() else np.nan
    return out


def test_o1_matches_scipy_softmax_attention():
    q, k, v = O.make_inputs(1, B=2, T=3, Hq=8, Hkv=2, n_kv=200)
    m = O.causal_mask(3, 200, 150, n_stream=2)
    m[1, 0, :, 30:40] = -np.inf
    want = scipy_attention(q, k, v, m, scale=SCALE)
    got = O.attention(q, k, v, m, scale=SCALE, mode="o1")
    assert rel(got, want) < 1e-6


@pytest.mark.parametrize("n_kv,kv_len", [(768, 513), (4096, 4096)])
def test_o2_matches_o1(n_kv, kv_len):
    q, k, v = O.make_inputs(n_kv, T=1, Hq=32, Hkv=8, n_kv=n_kv)
    m = O.causal_mask(1, n_kv, kv_len - 1)
    o1 = O.attention(q, k, v, m, scale=SCALE, mode="o1")
    o2 = O.attention(q, k, v, m, scale=SCALE, mode="o2")
    assert rel(o2, o1) < 1e-5
    assert float(np.abs(o2 - o1).max()) < 1e-5


def test_o2_matches_scipy_on_prefill_chunk():
    q, k, v = O.make_inputs(3, T=40, Hq=4, Hkv=1, n_kv=100)
    want = scipy_attention(q, k, v, scale=SCALE, causal_pos0=60)
    got = O.attention(q, k, v, scale=SCALE, causal_pos0=60)
    assert rel(got, want) < 1e-5


def test_single_visible_cell_returns_its_v_exactly():
    q, k, v = O.make_inputs(4, T=2, Hq=4, Hkv=2, n_kv=64)
    m = np.full((1, 1, 64, 64), -np.inf, dtype=np.float16)
    m[0, 0, 0, 9] = 0
    m[0, 0, 1, 41] = 0
    for mode in ("o1", "o2"):
        out = O.attention(q, k, v, m, scale=SCALE, mode=mode)
        vf = v.astype(np.float32)
        for h in range(4):
            assert np.array_equal(out[0, 0, h], vf[0, 9, h // 2])
            assert np.array_equal(out[0, 1, h], vf[0, 41, h // 2])


def test_equal_scores_give_the_mean_of_v():
    rng = np.random.default_rng(5)
    q = rng.standard_normal((1, 1, 2, 128), dtype=np.float32)
    k = np.broadcast_to(rng.standard_normal(128).astype(np.float16), (1, 50, 1, 128)).copy()
    v = rng.standard_normal((1, 50, 1, 128)).astype(np.float16)
    out = O.attention(q, k, v, scale=SCALE, kv_len=37)
    want = v[0, :37, 0].astype(np.float64).mean(axis=0)
    assert np.abs(out[0, 0, 0] - want).max() < 1e-6


def test_dominant_score_selects_its_cell():
    rng = np.random.default_rng(6)
    q = np.zeros((1, 1, 1, 128), dtype=np.float32)
    q[..., 0] = 8.0
    k = (rng.standard_normal((1, 64, 1, 128)) * 0.01).astype(np.float16)
    k[0, 23, 0, 0] = 60.0                 # score 8*60/sqrt(128) ~ 42 against ~0
    v = rng.standard_normal((1, 64, 1, 128)).astype(np.float16)
    out = O.attention(q, k, v, scale=SCALE)
    assert np.abs(out[0, 0, 0] - v[0, 23, 0].astype(np.float32)).max() < 1e-6


def test_masked_cells_contribute_nothing_even_if_garbage():
    q, k, v = O.make_inputs(8, T=2, Hq=8, Hkv=2, n_kv=90)
    m = O.causal_mask(2, 90, 70)
    base = O.attention(q, k, v, m, scale=SCALE)
    k2, v2 = k.copy(), v.copy()
    k2[:, 72:] = np.float16(np.nan)
    v2[:, 72:] = np.float16(np.inf)
    assert np.array_equal(O.attention(q, k2, v2, m, scale=SCALE), base)


def test_all_masked_row_is_nan_and_sink_makes_it_zero():
    q, k, v = O.make_inputs(9, T=1, Hq=2, Hkv=1, n_kv=64)
    m = np.full((1, 1, 64, 64), -np.inf, dtype=np.float16)
    for mode in ("o1", "o2"):
        assert np.isnan(O.attention(q, k, v, m, scale=SCALE, mode=mode)).all()
        out = O.attention(q, k, v, m, np.array([0.5, -2.0], dtype=np.float32), scale=SCALE, mode=mode)
        assert np.array_equal(out, np.zeros_like(out))


def test_cell_permutation_invariance():
    q, k, v = O.make_inputs(10, T=3, Hq=4, Hkv=2, n_kv=120)
    m = O.causal_mask(3, 120, 100)
    perm = np.random.default_rng(10).permutation(120)
    a = O.attention(q, k, v, m, scale=SCALE)
    b = O.attention(q, k[:, perm], v[:, perm], np.ascontiguousarray(m[..., perm]), scale=SCALE)
    assert rel(b, a) < 2e-6


def test_chunked_causal_prefill_equals_one_shot():
    q, k, v = O.make_inputs(11, T=96, Hq=4, Hkv=2, n_kv=96)
    one = O.attention(q, k, v, scale=SCALE, causal_pos0=0)
    for c in range(3):
        qc = np.ascontiguousarray(q[:, 32 * c: 32 * (c + 1)])
        part = O.attention(qc, k[:, :32 * (c + 1)], v[:, :32 * (c + 1)], scale=SCALE, causal_pos0=32 * c)
        assert np.array_equal(part, one[:, 32 * c: 32 * (c + 1)])


def test_gqa_broadcast_equals_repeated_kv_heads():
    q, k, v = O.make_inputs(12, T=2, Hq=8, Hkv=2, n_kv=80)
    a = O.attention(q, k, v, scale=SCALE)
    kr = np.repeat(k, 4, axis=2)
    vr = np.repeat(v, 4, axis=2)
    b = O.attention(q, kr, vr, scale=SCALE)
    assert np.array_equal(a, b)


def test_output_row_layout():
    # token t sees only cell t: dst row (b*T + t)*Hq + h must hold v[cell t]
    q, k, v = O.make_inputs(13, B=2, T=3, Hq=4, Hkv=1, n_kv=8)
    m = np.full((2, 1, 64, 8), -np.inf, dtype=np.float16)
    for b in range(2):
        for t in range(3):
            m[b, 0, t, 3 * b + t] = 0
    out = O.attention(q, k, v, m, scale=SCALE)
    vf = v.astype(np.float32)
    for b in range(2):
        for t in range(3):
            for h in range(4):
                assert np.array_equal(out[b, t, h], vf[b, 3 * b + t, 0])


def test_sinks_closed_form():
    q, k, v = O.make_inputs(14, T=2, Hq=6, Hkv=3, n_kv=70)
    sinks = np.array([3.0, -1.0, 0.0, 10.0, -20.0, 1.5], dtype=np.float32)
    want = scipy_attention(q, k, v, scale=SCALE, causal_pos0=50, sinks=sinks)
    for mode in ("o1", "o2"):
        got = O.attention(q, k, v, None, sinks, scale=SCALE, causal_pos0=50, mode=mode)
        assert rel(got, want) < 2e-6


def test_softcap_closed_form():
    # two visible cells: raw dots a = f16(alpha) and 0
    alpha, c, scale = 3.3, 2.0, 0.7
    q = np.zeros((1, 1, 1, 128), dtype=np.float32)
    q[..., 0] = alpha
    k = np.zeros((1, 2, 1, 128), dtype=np.float16)
    k[0, 0, 0, 0] = 1.0
    v = np.zeros((1, 2, 1, 128), dtype=np.float16)
    v[0, 0, 0, :] = 1.0
    v[0, 1, 0, :] = -2.0
    a = float(np.float16(alpha))
    s0 = c * math.tanh(a * scale / c)
    w0 = math.exp(s0) / (math.exp(s0) + 1.0)
    want = w0 * 1.0 + (1 - w0) * -2.0
    for mode in ("o1", "o2"):
        got = O.attention(q, k, v, scale=scale, logit_softcap=c, mode=mode)
        assert abs(float(got[0, 0, 0, 0]) - want) < 1e-6


def alibi_slopes_paper(n, max_bias=8.0):
    """Slopes of ALiBi (Press et al.), built as its reference get_slopes."""
    def pow2(nn):
        start = 2.0 ** (-max_bias / nn)
        return [start ** (i + 1) for i in range(nn)]
    if math.log2(n).is_integer():
        return pow2(n)
    c = 2 ** math.floor(math.log2(n))
    return pow2(c) + pow2(2 * c)[0::2][: n - c]


@pytest.mark.parametrize("Hq", [8, 12])
def test_alibi_slopes_closed_form(Hq):
    # zero scores; mask biases (0, -1) on two cells -> weights (1, e^-slope)
    q = np.zeros((1, 1, Hq, 128), dtype=np.float32)
    k = np.zeros((1, 2, 1, 128), dtype=np.float16)
    v = np.zeros((1, 2, 1, 128), dtype=np.float16)
    v[0, 0, 0, :] = 1.0
    m = np.zeros((1, 1, 64, 2), dtype=np.float16)
    m[0, 0, :, 1] = -1.0
    for mode in ("o1", "o2"):
        got = O.attention(q, k, v, m, scale=SCALE, max_bias=8.0, mode=mode)
        for h, sl in enumerate(alibi_slopes_paper(Hq)):
            want = 1.0 / (1.0 + math.exp(-sl))
            assert abs(float(got[0, 0, h, 0]) - want) < 2e-6, (h, sl)


def test_hints_equal_explicit_mask():
    q, k, v = O.make_inputs(15, T=4, Hq=8, Hkv=2, n_kv=300)
    m = O.causal_mask(4, 300, 250)
    a = O.attention(q, k, v, m, scale=SCALE)
    b = O.attention(q, k, v, scale=SCALE, kv_len=254, causal_pos0=250)
    c = O.attention(q, k, v, m, scale=SCALE, kv_len=254, causal_pos0=250)
    assert np.array_equal(a, b) and np.array_equal(a, c)


def test_arm_faithful_diagnostic_sits_outside_the_parity_bar():
    # the reference's f16 accumulator (O3) is ~3e-3 rel-L2 from exact at 512 cells
    q, k, v = O.make_inputs(16, T=1, Hq=32, Hkv=8, n_kv=768)
    m = O.causal_mask(1, 768, 512)
    o1 = O.attention(q, k, v, m, scale=SCALE, mode="o1")
    o3 = O.attention(q, k, v, m, scale=SCALE, mode="o3")
    assert 1e-3 < rel(o3, o1) < 1e-2


def _o3_exact_case(seed, equal_scores):
    """Inputs on which the ARM build's f16 arithmetic is exact: integer q, k
    and V (small enough that every f16 product and partial sum is an
    integer below 2048), and either all scores equal (q = 0: every visible
    cell weighs 1, 32 or 16 visible cells per token, so 1/S is exact) or one
    cell per kv head whose score (128, scale 1) outweighs the others (0) so
    far that exp(-128) vanishes in f16 and does not move an f32 result."""
    rng = np.random.default_rng(seed)
    T, Hq, Hkv, n_kv, D = 2, 8, 2, 64, 128
    G = Hq // Hkv
    q = np.zeros((1, T, Hq, D), np.float32)
    k = np.zeros((1, n_kv, Hkv, D), np.float16)
    v = rng.integers(-8, 9, size=(1, n_kv, Hkv, D)).astype(np.float16)
    mask = np.full((1, 1, 64, n_kv), -np.inf, np.float16)
    mask[0, 0, 0, 16:48] = 0                      # token 0: 32 visible cells
    mask[0, 0, 1, 8:24] = 0                       # token 1: 16
    dominant = {}
    if not equal_scores:
        for j in range(Hkv):
            sign = rng.choice([-1.0, 1.0], size=D).astype(np.float32)
            q[0, :, j * G:(j + 1) * G, :] = sign        # every head of group j, both tokens
            d = 20 + 3 * j                              # visible to both tokens
            k[0, d, j] = sign.astype(np.float16)        # dot 128 against 0 for every other cell
            dominant[j] = d
    return q, k, v, mask, dominant


@pytest.mark.parametrize("equal_scores", [True, False])
def test_arm_faithful_equals_exact_where_f16_is_exact(equal_scores):
    # O3 (the ARM build's f16 dot, f16 rescale and f16 V accumulator) must
    # equal O1 (float64) exactly where every f16 operation is exact (values,
    # so -0 equals +0: O1 adds the vanishing weights of the other cells); with
    # equal scores both are the mean of the visible V rows, with a dominant
    # cell both are that cell's V row (of the row's own kv head)
    q, k, v, mask, dominant = _o3_exact_case(31 + equal_scores, equal_scores)
    o1 = O.attention(q, k, v, mask, scale=1.0, mode="o1")
    o3 = O.attention(q, k, v, mask, scale=1.0, mode="o3")
    assert np.array_equal(o3, o1)
    vf = v.astype(np.float64)
    for t, (lo, hi) in enumerate(((16, 48), (8, 24))):
        for h in range(8):
            j = h // 4
            want = vf[0, lo:hi, j].mean(axis=0) if equal_scores else vf[0, dominant[j], j]
            assert np.array_equal(o1[0, t, h], want.astype(np.float32)), (t, h)


def test_rejects_what_the_reference_asserts():
    q, k, v = O.make_inputs(17, T=2, Hq=4, Hkv=2, n_kv=32)
    with pytest.raises(ValueError):
        O.attention(q, k, v, np.zeros((1, 1, 16, 32), dtype=np.float16), scale=SCALE)   # rows < PAD(T,64)
    with pytest.raises(ValueError):
        O.attention(q, k, v, scale=SCALE, max_bias=1.0)                                 # ALiBi needs a mask
    with pytest.raises(ValueError):
        O.attention(q, k, v, scale=SCALE, prec=3)


def test_set_rows_oracle_matches_numpy():
    rng = np.random.default_rng(18)
    cache = rng.standard_normal((50, 1024)).astype(np.float16).view(np.uint16)
    rows = rng.standard_normal((7, 1024)).astype(np.float32) * 100
    idx = np.array([3, 49, 0, 17, 18, 5, 33], dtype=np.int64)
    got = O.set_rows(cache, rows, idx)
    want = cache.copy()
    want[idx] = rows.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    with pytest.raises(ValueError):
        O.set_rows(cache, rows[:1], np.array([50], dtype=np.int64))
