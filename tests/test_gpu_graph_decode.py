"""A decode loop replayed from one captured HIP graph: the GPU form of the
reference's graph reuse (nnml/src/context.cpp:177-205 keeps the built graph
while the ubatch size is unchanged and n_kv stays within the graph's).

One decode step of two Qwen3-4B-shaped layers (Q/K RMSNorm + rope, K into
the HBM ring, V by set_rows, attention over the ring views, the Q4_0 WO
projection) is run once eagerly, captured once, then replayed for several
steps; between replays the host writes only the step's inputs (activations,
position, ring row, and the {kv_len, causal_pos0} pair the attention kernel
reads when it runs). Every step is checked against the oracle chain at the
parity bar (attention) and at the WO bar against the oracle WO of the
device's attention output.
"""
import math

import numpy as np
import pytest

from arclight_amd import abi
from oracle import oracle as O
from tests.fattn_cases import assert_parity
from tests.test_oracle_q4 import abs_bound, dequant_q4_0, dequant_q8_0

pytestmark = pytest.mark.gpu
EPS = 1e-6
EPS32 = 2.0 ** -24


def _case(name):
    print(f"\n[case] {name}", flush=True)


@pytest.mark.parametrize("inputs", ["separate", "one_launch", "fused"])
def test_decode_loop_graph_replay(gpu, inputs):
    """inputs: Q, K and V of a layer as three separate ops, through
    al_attn_inputs_f32 (one launch), or folded into the attention launch
    (al_fattn_f16_with_inputs)."""
    from arclight_amd import device, fattn, kv, matmul, prologue
    Hq, Hkv, D, L, N = 32, 8, 128, 2, 2560
    K = Hq * D
    KV_SIZE, NKV, P0, STEPS = 1024, 512, 300, 5
    scale = 1 / math.sqrt(D)
    rope = abi.qwen3_rope()
    rng = np.random.default_rng(2026)
    ring = kv.KvRing(L, KV_SIZE, Hkv, D, 1, 256, True)
    stream = device.Stream()
    wq = [rng.standard_normal(D).astype(np.float32) for _ in range(L)]
    wk = [rng.standard_normal(D).astype(np.float32) for _ in range(L)]
    wo = [O.random_q4_0(rng, N, K) for _ in range(L)]
    d_wq = [device.DeviceTensor.from_numpy(w) for w in wq]
    d_wk = [device.DeviceTensor.from_numpy(w) for w in wk]
    d_wo = [matmul.Q4_0Matrix(w.view(np.uint8), K, N) for w in wo]
    host_k = [np.zeros((KV_SIZE, Hkv * D), np.float16) for _ in range(L)]
    host_v = [np.zeros((KV_SIZE, Hkv * D), np.float16) for _ in range(L)]

    # the prompt's K/V, written eagerly
    _case(f"graph decode: prompt of {P0} tokens into the ring")
    rows, n_kv = ring.cells.place([(p, [0]) for p in range(P0)])
    pos = np.arange(P0, dtype=np.int32)
    d_rows_p, d_pos_p = device.DeviceTensor.from_numpy(rows), device.DeviceTensor.from_numpy(pos)
    for il in range(L):
        kc = rng.standard_normal((P0, Hkv, D)).astype(np.float32) * 3
        vc = rng.standard_normal((P0, Hkv * D)).astype(np.float32)
        prologue.rms_norm_rope(device.DeviceTensor.from_numpy(kc), d_wk[il], d_pos_p, eps=EPS, rope=rope,
                               y=ring.cache_rows(il, "k"), rows=d_rows_p)
        fattn.set_rows(ring.cache_rows(il, "v"), device.DeviceTensor.from_numpy(vc), d_rows_p)
        host_k[il][rows] = O.rms_norm_rope(kc, wk[il], pos, eps=EPS, rope=rope).reshape(P0, Hkv * D).astype(np.float16)
        host_v[il][rows] = vc.astype(np.float16)
    device.synchronize()

    # fixed device buffers of one decode step
    d_qc = device.DeviceTensor.empty((1, Hq, D), np.float32)
    d_kc = device.DeviceTensor.empty((1, Hkv, D), np.float32)
    d_vc = device.DeviceTensor.empty((1, Hkv * D), np.float32)
    d_pos = device.DeviceTensor.empty((1,), np.int32)
    d_row = device.DeviceTensor.empty((1,), np.int64)
    d_dyn = device.DeviceTensor.empty((2,), np.int32)
    d_q = [device.DeviceTensor.empty((1, Hq, D), np.float32) for _ in range(L)]
    d_att = [device.DeviceTensor.empty((1, 1, Hq, D), np.float32, axes=abi.DST_AXES) for _ in range(L)]
    d_y = [device.DeviceTensor.empty((1, N), np.float32) for _ in range(L)]

    def enqueue_step():
        for il in range(L):
            if inputs == "fused":
                prologue.attention_with_inputs(d_qc, d_wq[il], d_kc, d_wk[il], d_vc, d_pos, d_row, d_q[il],
                                               ring.cache_rows(il, "k"), ring.cache_rows(il, "v"), ring.get_k(il, NKV),
                                               ring.get_v(il, NKV), d_att[il], eps=EPS, scale=scale, rope=rope,
                                               kv_len=NKV, causal_pos0=0, dyn_len=d_dyn, stream=stream)
            else:
                if inputs == "one_launch":
                    prologue.attn_inputs(d_qc, d_wq[il], d_kc, d_wk[il], d_vc, d_pos, d_row, d_q[il],
                                         ring.cache_rows(il, "k"), ring.cache_rows(il, "v"), eps=EPS, rope=rope,
                                         stream=stream)
                else:
                    prologue.rms_norm_rope(d_qc, d_wq[il], d_pos, eps=EPS, rope=rope, y=d_q[il], stream=stream)
                    prologue.rms_norm_rope(d_kc, d_wk[il], d_pos, eps=EPS, rope=rope, y=ring.cache_rows(il, "k"),
                                           rows=d_row, stream=stream)
                    fattn.set_rows(ring.cache_rows(il, "v"), d_vc, d_row, stream=stream)
                qv = device.DeviceTensor(d_q[il].buf, abi.AL_TYPE_F32, (1, 1, Hq, D), None, 0, abi.Q_AXES)
                fattn.flash_attn_ext(qv, ring.get_k(il, NKV), ring.get_v(il, NKV), scale=scale, dst=d_att[il],
                                     kv_len=NKV, causal_pos0=0, stream=stream, dyn_len=d_dyn)
            x = device.DeviceTensor(d_att[il].buf, abi.AL_TYPE_F32, (1, K))
            matmul.mul_mat_q4_0(d_wo[il], x, d_y[il], stream)

    graph = None
    try:
        for s in range(STEPS):
            p = P0 + s
            how = ("eager" if s == 0 else "graph replay") + f", inputs {inputs}"
            _case(f"graph decode: step {s} at position {p} ({how})")
            rows, n_kv = ring.cells.place([(p, [0])])
            assert n_kv <= NKV and ring.cells.implicit([(p, [0])], n_kv) == (p + 1, p)
            qc = rng.standard_normal((1, Hq, D)).astype(np.float32) * 3
            kc = rng.standard_normal((1, Hkv, D)).astype(np.float32) * 3
            vc = rng.standard_normal((1, Hkv * D)).astype(np.float32)
            stream.synchronize()
            for t, a in ((d_qc, qc), (d_kc, kc), (d_vc, vc), (d_pos, np.array([p], np.int32)),
                         (d_row, rows.astype(np.int64)), (d_dyn, np.array([p + 1, p], np.int32))):
                t.buf.upload(np.ascontiguousarray(a))
            if s == 0:
                enqueue_step()                                        # allocates what capture must not
                stream.synchronize()
                graph = device.Graph(stream, enqueue_step)
            else:
                graph.launch(stream)
            stream.synchronize()
            fattn.device_errors()
            for il in range(L):
                q_ref = O.rms_norm_rope(qc, wq[il], np.array([p], np.int32), eps=EPS, rope=rope)
                host_k[il][rows] = O.rms_norm_rope(kc, wk[il], np.array([p], np.int32), eps=EPS,
                                                   rope=rope).reshape(1, Hkv * D).astype(np.float16)
                host_v[il][rows] = vc.astype(np.float16)
                k_ref = host_k[il].reshape(1, KV_SIZE, Hkv, D)[:, :n_kv]
                v_ref = host_v[il].reshape(1, KV_SIZE, Hkv, D)[:, :n_kv]
                ref = O.attention(q_ref[None], k_ref, v_ref, O.causal_mask(1, n_kv, p, kv_len=p + 1), scale=scale)
                att = d_att[il].numpy(np.float32)
                assert_parity(att, ref, what=f"step {s} layer {il} attention")
                # WO of the device's attention output, at the WO bar
                x = att.reshape(1, K)
                y = d_y[il].numpy(np.float32)
                y_ref = O.mul_mat_q4_0(wo[il], x)
                bound = (K // 32 + 16) * 2 * EPS32 * abs_bound(dequant_q4_0(wo[il]), dequant_q8_0(O.quantize_q8_0(x)))
                assert np.all(np.abs(y.astype(np.float64) - y_ref) <= bound), f"step {s} layer {il} WO"
    finally:
        if graph is not None:
            graph.destroy()
        stream.destroy()
        ring.close()


def test_dyn_len_rejected_off_the_decode_path(gpu):
    """dyn_len with a mask tensor, or with more than 32 query rows per kv
    head, is refused rather than run with stale lengths."""
    from arclight_amd import _lib, device, fattn
    q, k, v = O.make_inputs(3, T=16, Hq=32, Hkv=8, n_kv=256)
    dq, dk, dv = fattn.upload_q(q), fattn.upload_kv(k), fattn.upload_kv(v)
    dyn = device.DeviceTensor.from_numpy(np.array([256, 240], np.int32))
    with pytest.raises(_lib.ArclightError) as e:
        fattn.flash_attn_ext(dq, dk, dv, scale=0.1, kv_len=256, causal_pos0=0, dyn_len=dyn)
    assert e.value.status == abi.AL_ERR_UNSUPPORTED
    q1 = fattn.upload_q(q[:, :1])
    m = fattn.upload_mask(O.causal_mask(1, 256, 255))
    with pytest.raises(_lib.ArclightError) as e:
        fattn.flash_attn_ext(q1, dk, dv, m, scale=0.1, dyn_len=dyn)
    assert e.value.status == abi.AL_ERR_UNSUPPORTED


@pytest.mark.parametrize("T", [1, 4, 8])
def test_dyn_len_matches_host_lengths(gpu, T):
    """The run-time {kv_len, causal_pos0} give the same result as the same
    lengths passed on the host, for decode and for 4- and 8-draft verify
    (one and two row blocks), with the launch sized for a larger bound."""
    from arclight_amd import device, fattn
    _case(f"dyn_len T={T}")
    n_kv, C = 1024, 700
    q, k, v = O.make_inputs(40 + T, T=T, Hq=32, Hkv=8, n_kv=n_kv)
    dq, dk, dv = fattn.upload_q(q), fattn.upload_kv(k), fattn.upload_kv(v)
    dyn = device.DeviceTensor.from_numpy(np.array([C + T, C], np.int32))
    got = fattn.flash_attn_ext(dq, dk, dv, scale=0.08, kv_len=n_kv, causal_pos0=0, dyn_len=dyn)
    device.synchronize()
    fattn.device_errors()
    ref = O.attention(q, k, v, O.causal_mask(T, n_kv, C, kv_len=C + T), scale=0.08)
    assert_parity(got.numpy(np.float32), ref, what=f"dyn_len T={T}")
