"""al_fattn_f16_with_inputs: the decode kernel with the layer's attention
inputs (Q and K RMSNorm + weight + rope, K and V into the f16 cache) folded
into its prologue, against the pair of calls it replaces
(al_attn_inputs_f32, then al_fattn_f16 over q_out and the caches' views):
same bits in dst, q_out and both caches, on shapes with many splits, new
cells inside and at the end of the attended range, one token (a decode
step), each rotation mode, with and without weights; one case also against
the oracle chain at the parity bar; and the calls it does not take (several
tokens, K / V views that are not the caches) rejected before anything is
enqueued.
"""
import math

import numpy as np
import pytest

from arclight_amd import abi
from oracle import oracle as O
from tests.fattn_cases import assert_parity

pytestmark = pytest.mark.gpu
EPS = 1e-6
Hq, Hkv, D = 32, 8, 128


def _case(name):
    print(f"\n[case] {name}", flush=True)


def _setup(seed, T, n_rows, rows, rope_mode=abi.AL_ROPE_NEOX, weighted=True):
    from arclight_amd import device
    rng = np.random.default_rng(seed)
    host = {
        "q": (rng.standard_normal((T, Hq, D)) * 3).astype(np.float32),
        "k": (rng.standard_normal((T, Hkv, D)) * 3).astype(np.float32),
        "v": rng.standard_normal((T, Hkv * D)).astype(np.float32),
        "wq": rng.standard_normal(D).astype(np.float32),
        "wk": rng.standard_normal(D).astype(np.float32),
        "pos": (np.asarray(rows) + 7).astype(np.int32),
        "rows": np.asarray(rows, np.int64),
        "kc": rng.standard_normal((n_rows, Hkv * D)).astype(np.float16).view(np.uint16),
        "vc": rng.standard_normal((n_rows, Hkv * D)).astype(np.float16).view(np.uint16),
    }
    dev = {n: device.DeviceTensor.from_numpy(host[n]) for n in ("q", "k", "v", "wq", "wk", "pos", "rows")}
    if not weighted:
        dev["wq"] = dev["wk"] = None
    rope = None
    if rope_mode is not None:
        rope = abi.qwen3_rope()
        rope.mode = rope_mode
    return host, dev, rope


def _pair_and_fused(host, dev, rope, T, n_kv, kv_len, causal_pos0):
    """Runs the pair and the fused call on separate copies of the caches;
    returns {what: (pair, fused)} as raw bits."""
    from arclight_amd import device, fattn, prologue
    out = {}
    res = []
    for fused in (False, True):
        kc = device.DeviceTensor.from_numpy(host["kc"])
        vc = device.DeviceTensor.from_numpy(host["vc"])
        kview = device.DeviceTensor(kc.buf, abi.AL_TYPE_F16, (1, n_kv, Hkv, D), None, 0, abi.KV_AXES)
        vview = device.DeviceTensor(vc.buf, abi.AL_TYPE_F16, (1, n_kv, Hkv, D), None, 0, abi.KV_AXES)
        q_out = device.DeviceTensor.empty((T, Hq, D), np.float32)
        dst = device.DeviceTensor.empty((1, T, Hq, D), np.float32, axes=abi.DST_AXES)
        args = (dev["q"], dev["wq"], dev["k"], dev["wk"], dev["v"], dev["pos"], dev["rows"], q_out, kc, vc)
        if fused:
            prologue.attention_with_inputs(*args, kview, vview, dst, eps=EPS, scale=1 / math.sqrt(D), rope=rope,
                                           kv_len=kv_len, causal_pos0=causal_pos0)
        else:
            prologue.attn_inputs(*args, eps=EPS, rope=rope)
            qv = device.DeviceTensor(q_out.buf, abi.AL_TYPE_F32, (1, T, Hq, D), None, 0, abi.Q_AXES)
            fattn.flash_attn_ext(qv, kview, vview, scale=1 / math.sqrt(D), dst=dst, kv_len=kv_len,
                                 causal_pos0=causal_pos0)
        device.synchronize()
        fattn.device_errors()
        res.append({"dst": dst.numpy(np.float32), "q_out": q_out.numpy(np.float32), "k cache": kc.numpy(np.uint16),
                    "v cache": vc.numpy(np.uint16)})
    for what in res[0]:
        out[what] = (res[0][what], res[1][what])
    return out


def _assert_same_bits(out, label):
    for what, (a, b) in out.items():
        assert a.shape == b.shape
        assert np.array_equal(a.view(np.uint32) if a.dtype == np.float32 else a,
                              b.view(np.uint32) if b.dtype == np.float32 else b), f"{label}: {what} differs"


@pytest.mark.parametrize("T,n_kv,rows,mode,weighted", [
    (1, 4096, [4095], abi.AL_ROPE_NEOX, True),           # decode: the new cell is the last one
    (1, 4096, [1234], abi.AL_ROPE_NEOX, True),           # a cell inside the range (another split's stage)
    (1, 32768, [32767], abi.AL_ROPE_NEOX, True),         # the benchmark's context
    (1, 512, [300], abi.AL_ROPE_NORMAL, False),
    (1, 1024, [1000], None, True),
])
def test_fused_inputs_match_the_pair(gpu, T, n_kv, rows, mode, weighted):
    _case(f"fused inputs T={T} n_kv={n_kv} rows={rows} mode={mode} weighted={weighted}")
    host, dev, rope = _setup(100 + T + n_kv % 97, T, n_kv, rows, mode, weighted)
    causal = T > 1
    out = _pair_and_fused(host, dev, rope, T, n_kv, kv_len=n_kv, causal_pos0=n_kv - T if causal else -1)
    _assert_same_bits(out, f"T={T} n_kv={n_kv}")


def test_fused_inputs_against_oracle(gpu):
    """The fused call's attention against the oracle chain (norm, rope, f16
    rounding of the new K / V rows, attention) at the parity bar."""
    _case("fused inputs vs oracle, T=1 n_kv=2048")
    T, n_kv, rows = 1, 2048, [2047]
    host, dev, rope = _setup(7, T, n_kv, rows)
    out = _pair_and_fused(host, dev, rope, T, n_kv, kv_len=n_kv, causal_pos0=-1)
    q_ref = O.rms_norm_rope(host["q"], host["wq"], host["pos"], eps=EPS, rope=rope)
    kc = host["kc"].view(np.float16).copy()
    vc = host["vc"].view(np.float16).copy()
    kc[rows] = O.rms_norm_rope(host["k"], host["wk"], host["pos"], eps=EPS, rope=rope).reshape(T, Hkv * D).astype(np.float16)
    vc[rows] = host["v"].astype(np.float16)
    ref = O.attention(q_ref[None], kc.reshape(1, n_kv, Hkv, D), vc.reshape(1, n_kv, Hkv, D), scale=1 / math.sqrt(D),
                      kv_len=n_kv)
    assert_parity(out["dst"][1], ref, what="fused inputs attention")


def test_fused_inputs_bad_row(gpu):
    """An out-of-range cache row: nothing written, reported as set_rows
    reports it."""
    from arclight_amd._lib import ArclightError
    from arclight_amd import device, fattn, prologue
    _case("fused inputs, out-of-range row")
    T, n_kv = 1, 1024
    host, dev, rope = _setup(9, T, n_kv, [n_kv + 5])
    kc = device.DeviceTensor.from_numpy(host["kc"])
    vc = device.DeviceTensor.from_numpy(host["vc"])
    kview = device.DeviceTensor(kc.buf, abi.AL_TYPE_F16, (1, n_kv, Hkv, D), None, 0, abi.KV_AXES)
    vview = device.DeviceTensor(vc.buf, abi.AL_TYPE_F16, (1, n_kv, Hkv, D), None, 0, abi.KV_AXES)
    q_out = device.DeviceTensor.empty((T, Hq, D), np.float32)
    dst = device.DeviceTensor.empty((1, T, Hq, D), np.float32, axes=abi.DST_AXES)
    prologue.attention_with_inputs(dev["q"], dev["wq"], dev["k"], dev["wk"], dev["v"], dev["pos"], dev["rows"], q_out,
                                   kc, vc, kview, vview, dst, eps=EPS, scale=1 / math.sqrt(D), rope=rope, kv_len=n_kv)
    device.synchronize()
    with pytest.raises(ArclightError, match="out of range"):
        fattn.device_errors()
    fattn.device_errors()                                  # cleared
    assert np.array_equal(kc.numpy(np.uint16), host["kc"]) and np.array_equal(vc.numpy(np.uint16), host["vc"])
    assert np.isfinite(dst.numpy(np.float32)).all()


def test_fused_inputs_rejected_shapes(gpu):
    """Several tokens, or K / V views that are not the caches the inputs
    write: AL_ERR_UNSUPPORTED, nothing enqueued (dst keeps its contents)."""
    from arclight_amd import device, prologue
    from arclight_amd._lib import ArclightError
    _case("fused inputs, rejected shapes")
    for T, n_kv, offset_cells in ((2, 1024, 0), (1, 1024, 16)):
        host, dev, rope = _setup(11, T, n_kv + 32, list(range(100, 100 + T)))
        kc = device.DeviceTensor.from_numpy(host["kc"])
        vc = device.DeviceTensor.from_numpy(host["vc"])
        off = offset_cells * Hkv * D * 2
        kview = device.DeviceTensor(kc.buf, abi.AL_TYPE_F16, (1, n_kv, Hkv, D), None, off, abi.KV_AXES)
        vview = device.DeviceTensor(vc.buf, abi.AL_TYPE_F16, (1, n_kv, Hkv, D), None, off, abi.KV_AXES)
        q_out = device.DeviceTensor.empty((T, Hq, D), np.float32)
        dst = device.DeviceTensor.from_numpy(np.full((1, T, Hq, D), 7.0, np.float32), axes=abi.DST_AXES)
        with pytest.raises(ArclightError, match="UNSUPPORTED"):
            prologue.attention_with_inputs(dev["q"], dev["wq"], dev["k"], dev["wk"], dev["v"], dev["pos"], dev["rows"],
                                           q_out, kc, vc, kview, vview, dst, eps=EPS, scale=0.1, rope=rope,
                                           kv_len=n_kv, causal_pos0=-1)
        device.synchronize()
        assert np.all(dst.numpy(np.float32) == 7.0)
        assert np.array_equal(kc.numpy(np.uint16), host["kc"])


def test_fused_inputs_in_place_query_rejected(gpu):
    """q_out over the raw query rows (an in-place Q): every split of the
    fused launch reads the raw rows while split 0 writes q_out, so the call
    is refused (AL_ERR_UNSUPPORTED, nothing enqueued); the pair of calls
    takes the in-place operand and matches the out-of-place pair."""
    from arclight_amd import device, fattn, prologue
    from arclight_amd._lib import ArclightError
    _case("fused inputs, in-place query rows (multi-split decode)")
    T, n_kv, rows = 1, 4096, [4095]
    host, dev, rope = _setup(13, T, n_kv, rows)
    out_of_place = _pair_and_fused(host, dev, rope, T, n_kv, kv_len=n_kv, causal_pos0=-1)
    kc = device.DeviceTensor.from_numpy(host["kc"])
    vc = device.DeviceTensor.from_numpy(host["vc"])
    kview = device.DeviceTensor(kc.buf, abi.AL_TYPE_F16, (1, n_kv, Hkv, D), None, 0, abi.KV_AXES)
    vview = device.DeviceTensor(vc.buf, abi.AL_TYPE_F16, (1, n_kv, Hkv, D), None, 0, abi.KV_AXES)
    q_inplace = device.DeviceTensor.from_numpy(host["q"])
    dst = device.DeviceTensor.from_numpy(np.full((1, T, Hq, D), 7.0, np.float32), axes=abi.DST_AXES)
    with pytest.raises(ArclightError, match="UNSUPPORTED"):
        prologue.attention_with_inputs(q_inplace, dev["wq"], dev["k"], dev["wk"], dev["v"], dev["pos"], dev["rows"],
                                       q_inplace, kc, vc, kview, vview, dst, eps=EPS, scale=1 / math.sqrt(D), rope=rope,
                                       kv_len=n_kv, causal_pos0=-1)
    device.synchronize()
    assert np.all(dst.numpy(np.float32) == 7.0)
    assert np.array_equal(q_inplace.numpy(np.float32), host["q"])
    # the pair in place
    prologue.attn_inputs(q_inplace, dev["wq"], dev["k"], dev["wk"], dev["v"], dev["pos"], dev["rows"], q_inplace, kc, vc,
                         eps=EPS, rope=rope)
    qv = device.DeviceTensor(q_inplace.buf, abi.AL_TYPE_F32, (1, T, Hq, D), None, 0, abi.Q_AXES)
    fattn.flash_attn_ext(qv, kview, vview, scale=1 / math.sqrt(D), dst=dst, kv_len=n_kv, causal_pos0=-1)
    device.synchronize()
    fattn.device_errors()
    assert np.array_equal(dst.numpy(np.float32).view(np.uint32), out_of_place["dst"][0].view(np.uint32))
    assert np.array_equal(q_inplace.numpy(np.float32).view(np.uint32), out_of_place["q_out"][0].view(np.uint32))
