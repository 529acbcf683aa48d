"""GPU parity of the attention-operand producers (al_rms_norm_rope_f32)
against the oracle's restatement of nnml's rms_norm, mul and rope f32
(nnml/src/ops/ops.cpp:680-726, 871-962), and a Qwen3-4B-shaped layer
prologue (Q/K norm + rope, K and V into the HBM ring) feeding the attention
operator, against the oracle chain.

Bars: f32 outputs within 1e-5 absolute + 1e-6 relative (the device's and the
host's sinf / cosf differ by an ulp or two; norm and angles are computed the
reference's way); K written to the f16 cache within one f16 ulp of the
oracle's value rounded to f16 (RNE); attention at the parity bar.
"""
import math

import numpy as np
import pytest

from arclight_amd import abi
from oracle import oracle as O
from tests.fattn_cases import assert_parity

pytestmark = pytest.mark.gpu
EPS = 1e-6


def _case(name):
    print(f"\n[case] {name}", flush=True)


def _inputs(seed, T, H, heads_total=None):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((T, heads_total or H, 128)) * rng.uniform(0.1, 20, (T, heads_total or H, 1))).astype(np.float32)
    w = rng.standard_normal(128).astype(np.float32)
    pos = rng.integers(0, 40960, T).astype(np.int32)
    return x, w, pos


def _run(x_dev, w, pos, rope, y=None, rows=None):
    from arclight_amd import device, fattn, prologue
    dw = device.DeviceTensor.from_numpy(w) if w is not None else None
    dp = device.DeviceTensor.from_numpy(pos)
    out = prologue.rms_norm_rope(x_dev, dw, dp, eps=EPS, rope=rope, y=y, rows=rows)
    device.synchronize()
    fattn.device_errors()
    return out


@pytest.mark.parametrize("T,H,mode,weighted", [(1, 32, abi.AL_ROPE_NEOX, True), (7, 8, abi.AL_ROPE_NEOX, True),
                                               (512, 32, abi.AL_ROPE_NEOX, True), (33, 5, abi.AL_ROPE_NORMAL, False),
                                               (9, 3, None, True)])
def test_q_path_matches_oracle(gpu, T, H, mode, weighted):
    from arclight_amd import device
    _case(f"norm+rope f32 T={T} H={H} mode={mode} weighted={weighted}")
    x, w, pos = _inputs(T * 100 + H, T, H)
    w = w if weighted else None
    rope = abi.AlRopeParams(128, mode, 40960, 1e6, 1.0, 0.0, 1.0, 32.0, 1.0) if mode is not None else None
    ref = O.rms_norm_rope(x, w, pos, eps=EPS, rope=rope)
    got = _run(device.DeviceTensor.from_numpy(x), w, pos, rope).numpy(np.float32)
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-5)


def test_yarn_and_strided_views(gpu):
    # Q and K as head ranges of one fused projection buffer (T, Hq + 2 Hkv, 128)
    from arclight_amd import device
    _case("yarn rope on strided head views")
    T, Hq, Hkv = 12, 16, 4
    x, w, pos = _inputs(5, T, Hq, Hq + 2 * Hkv)
    rope = abi.AlRopeParams(128, abi.AL_ROPE_NEOX, 4096, 1e4, 0.25, 1.0, 1.0, 32.0, 1.0)
    buf = device.DeviceTensor.from_numpy(x).buf
    row = (Hq + 2 * Hkv) * 512
    q = device.DeviceTensor(buf, abi.AL_TYPE_F32, (T, Hq, 128), (row, 512, 4), 0)
    k = device.DeviceTensor(buf, abi.AL_TYPE_F32, (T, Hkv, 128), (row, 512, 4), Hq * 512)
    for view, sl in ((q, slice(0, Hq)), (k, slice(Hq, Hq + Hkv))):
        ref = O.rms_norm_rope(np.ascontiguousarray(x[:, sl]), w, pos, eps=EPS, rope=rope)
        got = _run(view, w, pos, rope).numpy(np.float32)
        np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-5)


def test_k_path_into_cache(gpu):
    from arclight_amd import device
    _case("norm+rope K into the f16 cache at rows")
    T, H, n_rows = 40, 8, 300
    x, w, pos = _inputs(7, T, H)
    rope = abi.qwen3_rope()
    rows = np.random.default_rng(7).choice(n_rows, T, replace=False).astype(np.int64)
    cache = device.DeviceTensor.from_numpy(np.zeros((n_rows, H * 128), np.uint16))
    _run(device.DeviceTensor.from_numpy(x), w, pos, rope, y=cache, rows=device.DeviceTensor.from_numpy(rows))
    got = cache.numpy(np.uint16)
    ref = O.rms_norm_rope(x, w, pos, eps=EPS, rope=rope).reshape(T, H * 128).astype(np.float16).view(np.uint16)
    diff = np.abs(got[rows].astype(np.int32) - ref.astype(np.int32))
    assert diff.max() <= 1, f"max f16 ulp difference {diff.max()}"
    assert (diff != 0).mean() < 1e-3
    untouched = np.setdiff1d(np.arange(n_rows), rows)
    assert not got[untouched].any()


def test_bad_cache_row_reported(gpu):
    from arclight_amd import device, fattn, prologue
    from arclight_amd._lib import ArclightError
    _case("out-of-range cache row")
    x, w, pos = _inputs(9, 3, 2)
    cache = device.DeviceTensor.from_numpy(np.zeros((10, 256), np.uint16))
    rows = device.DeviceTensor.from_numpy(np.array([1, 10, 2], np.int64))
    prologue.rms_norm_rope(device.DeviceTensor.from_numpy(x), device.DeviceTensor.from_numpy(w),
                           device.DeviceTensor.from_numpy(pos), eps=EPS, rope=abi.qwen3_rope(), y=cache, rows=rows)
    device.synchronize()
    with pytest.raises(ArclightError, match="out of range"):
        fattn.device_errors()
    fattn.device_errors()                                  # cleared


def test_qwen3_layer_prologue_into_attention(gpu):
    """Prefill of 64 tokens, then one decode step, Qwen3-4B attention shape:
    Q/K RMSNorm + weight + rope on the device, K fused into the ring, V by
    set_rows, attention over the ring views; against the oracle chain."""
    from arclight_amd import device, fattn, kv, prologue
    Hq, Hkv, D = 32, 8, 128
    ring = kv.KvRing(1, 512, Hkv, D, 1, 256, True)
    rng = np.random.default_rng(11)
    wq = rng.standard_normal(D).astype(np.float32)
    wk = rng.standard_normal(D).astype(np.float32)
    rope = abi.qwen3_rope()
    host_k = np.zeros((512, Hkv * D), np.float16)
    host_v = np.zeros((512, Hkv * D), np.float16)
    for step, (p0, T) in enumerate(((0, 64), (64, 1))):
        _case(f"layer prologue step {step}: T={T} at {p0}")
        ub = [(p0 + i, [0]) for i in range(T)]
        rows, n_kv = ring.cells.place(ub)
        pos = np.arange(p0, p0 + T, dtype=np.int32)
        qc = rng.standard_normal((T, Hq, D)).astype(np.float32) * 3
        kc = rng.standard_normal((T, Hkv, D)).astype(np.float32) * 3
        vc = rng.standard_normal((T, Hkv, D)).astype(np.float32)
        d_rows = device.DeviceTensor.from_numpy(rows)
        d_pos = device.DeviceTensor.from_numpy(pos)
        q = prologue.rms_norm_rope(device.DeviceTensor.from_numpy(qc), device.DeviceTensor.from_numpy(wq), d_pos,
                                   eps=EPS, rope=rope)
        prologue.rms_norm_rope(device.DeviceTensor.from_numpy(kc), device.DeviceTensor.from_numpy(wk), d_pos, eps=EPS,
                               rope=rope, y=ring.cache_rows(0, "k"), rows=d_rows)
        fattn.set_rows(ring.cache_rows(0, "v"), device.DeviceTensor.from_numpy(vc.reshape(T, Hkv * D)), d_rows)
        qv = device.DeviceTensor(q.buf, abi.AL_TYPE_F32, (1, T, Hq, D), None, 0, abi.Q_AXES)
        imp = ring.cells.implicit(ub, n_kv)
        assert imp == (p0 + T, p0)
        out = fattn.flash_attn_ext(qv, ring.get_k(0, n_kv), ring.get_v(0, n_kv), scale=1 / math.sqrt(D),
                                   kv_len=imp[0], causal_pos0=imp[1])
        device.synchronize()
        fattn.device_errors()
        # the oracle chain
        q_ref = O.rms_norm_rope(qc, wq, pos, eps=EPS, rope=rope)
        host_k[rows] = O.rms_norm_rope(kc, wk, pos, eps=EPS, rope=rope).reshape(T, Hkv * D).astype(np.float16)
        host_v[rows] = vc.reshape(T, Hkv * D).astype(np.float16)
        k_ref = host_k.reshape(1, 512, Hkv, D)[:, :n_kv]
        v_ref = host_v.reshape(1, 512, Hkv, D)[:, :n_kv]
        ref = O.attention(q_ref[None], k_ref, v_ref, O.causal_mask(T, n_kv, p0, kv_len=p0 + T), scale=1 / math.sqrt(D))
        assert_parity(out.numpy(np.float32), ref, what=f"layer step {step}")
    ring.close()


@pytest.mark.parametrize("T", [1, 7])
def test_attn_inputs_one_launch_matches_the_separate_ops(gpu, T):
    """al_attn_inputs_f32 writes Q, the K cache rows and the V cache rows bit
    for bit as al_rms_norm_rope_f32 (Q; K with rows) and al_set_rows_f32_f16
    (V) do one after another; rows outside the token's cells stay untouched."""
    from arclight_amd import device, fattn, prologue
    _case(f"attention inputs in one launch, T={T}")
    Hq, Hkv, n_rows = 32, 8, 64
    rng = np.random.default_rng(70 + T)
    q, wq, pos = _inputs(71 + T, T, Hq)
    k, wk, _ = _inputs(72 + T, T, Hkv)
    v = (rng.standard_normal((T, Hkv * 128)) * 3).astype(np.float32)
    rows = rng.choice(n_rows, T, replace=False).astype(np.int64)
    rope = abi.qwen3_rope()
    d = {n: device.DeviceTensor.from_numpy(a) for n, a in
         (("q", q), ("k", k), ("v", v), ("wq", wq), ("wk", wk), ("pos", pos), ("rows", rows))}
    caches = [[device.DeviceTensor.from_numpy(np.zeros((n_rows, Hkv * 128), np.uint16)) for _ in range(2)] for _ in range(2)]
    q_outs = [device.DeviceTensor.empty((T, Hq, 128), np.float32) for _ in range(2)]
    # the separate ops
    prologue.rms_norm_rope(d["q"], d["wq"], d["pos"], eps=EPS, rope=rope, y=q_outs[0])
    prologue.rms_norm_rope(d["k"], d["wk"], d["pos"], eps=EPS, rope=rope, y=caches[0][0], rows=d["rows"])
    fattn.set_rows(caches[0][1], d["v"], d["rows"])
    # one launch
    prologue.attn_inputs(d["q"], d["wq"], d["k"], d["wk"], d["v"], d["pos"], d["rows"], q_outs[1], caches[1][0],
                         caches[1][1], eps=EPS, rope=rope)
    device.synchronize()
    fattn.device_errors()
    assert np.array_equal(q_outs[0].numpy(np.float32).view(np.uint32), q_outs[1].numpy(np.float32).view(np.uint32))
    for j, what in enumerate(("K", "V")):
        sep, one = caches[0][j].numpy(np.uint16), caches[1][j].numpy(np.uint16)
        assert np.array_equal(sep, one), f"{what} cache differs"
        assert not np.delete(one, rows, axis=0).any(), f"{what}: rows outside the tokens' cells written"
        assert one[rows].any()


def test_attn_inputs_bad_row_reported(gpu):
    from arclight_amd import device, fattn, prologue
    from arclight_amd._lib import ArclightError
    _case("attention inputs, out-of-range cache row")
    q, wq, pos = _inputs(80, 2, 4)
    k, wk, _ = _inputs(81, 2, 2)
    v = np.ones((2, 256), np.float32)
    kc = device.DeviceTensor.from_numpy(np.zeros((10, 256), np.uint16))
    vc = device.DeviceTensor.from_numpy(np.zeros((10, 256), np.uint16))
    prologue.attn_inputs(device.DeviceTensor.from_numpy(q), device.DeviceTensor.from_numpy(wq),
                         device.DeviceTensor.from_numpy(k), device.DeviceTensor.from_numpy(wk),
                         device.DeviceTensor.from_numpy(v), device.DeviceTensor.from_numpy(pos),
                         device.DeviceTensor.from_numpy(np.array([3, 10], np.int64)),
                         device.DeviceTensor.empty((2, 4, 128), np.float32), kc, vc, eps=EPS, rope=abi.qwen3_rope())
    device.synchronize()
    with pytest.raises(ArclightError, match="out of range"):
        fattn.device_errors()
    fattn.device_errors()                                  # cleared
    assert kc.numpy(np.uint16)[3].any() and vc.numpy(np.uint16)[3].any()
    assert not np.delete(kc.numpy(np.uint16), 3, axis=0).any() and not np.delete(vc.numpy(np.uint16), 3, axis=0).any()
