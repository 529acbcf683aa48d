"""Workspace state across calls, masked many-row calls in between.

- A many-row call with a mask tensor whose prefill plan has a single split
  (Qwen3-32B shape, 1024-token chunk: 128 row tiles x 8 kv heads fill the
  device) needs no workspace; a multi-split decode call that follows on the
  library workspace matches the oracle, before and after masks the prefill
  kernel takes value by value (a hole, biases).
- Masked many-row calls on two streams, one mask a causal prefix and one
  not, overlap without touching each other's records.
- A captured masked call replayed first with a non-prefix mask and then with
  a prefix one gives the oracle's result on every replay (nothing a call
  decides about its mask outlives the call).

Bar: max-abs <= 2e-3 and rel-L2 <= 1e-3 on the fp32 output against oracle
O2, as everywhere.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O
from tests.fattn_cases import assert_parity, run_gpu

pytestmark = pytest.mark.gpu
SCALE = 1.0 / math.sqrt(128)


def _case(name):
    print(f"\n[case] {name}", flush=True)


def _decode_check(seed):
    # Qwen3-4B decode over 4096 cells: 32 splits per kv head on the library workspace
    q, k, v = O.make_inputs(seed, T=1, Hq=32, Hkv=8, n_kv=4096)
    ref = O.attention(q, k, v, scale=SCALE, kv_len=4000)
    assert_parity(run_gpu(q, k, v, scale=SCALE, kv_len=4000), ref, what=f"decode after masked prefill ({seed})")


def _dst(q):
    from arclight_amd import abi, device
    return device.DeviceTensor.empty(q.shape, np.float32, axes=abi.DST_AXES)


def _sampled(q, k, v, m, sel):
    rows = (len(sel) + 63) // 64 * 64
    ms = np.full((1, 1, rows, m.shape[3]), -np.inf, dtype=np.float16)
    ms[:, :, :len(sel)] = m[:, :, sel]
    return O.attention(np.ascontiguousarray(q[:, sel]), k, v, ms, scale=SCALE)


def test_masked_single_split_prefill_then_decode(gpu):
    from arclight_amd import fattn
    T, pos0 = 1024, 1024
    n_kv = pos0 + T
    q, k, v = O.make_inputs(77, T=T, Hq=64, Hkv=8, n_kv=n_kv)
    m = O.causal_mask(T, n_kv, pos0, kv_len=n_kv)
    # one workgroup per row tile: no merge records, no counters
    need = fattn.workspace_bytes(fattn.upload_q(q), fattn.upload_kv(k), fattn.upload_kv(v), fattn.upload_mask(m),
                                 None, _dst(q), scale=SCALE)
    assert need == 0, need
    rng = np.random.default_rng(5)
    sel = np.unique(np.concatenate([[0, 63, 64, T - 1], rng.choice(T, 20, replace=False)]))
    _case("Qwen3-32B chunk 1024, explicit causal mask (a prefix in every row)")
    got = run_gpu(q, k, v, m, scale=SCALE)
    assert_parity(got[:, sel], _sampled(q, k, v, m, sel), what="32B masked chunk")
    _case("decode after it on the library workspace")
    _decode_check(11)
    m2 = m.copy()
    m2[..., 300] = -np.inf                           # a hole: taken value by value
    _case("Qwen3-32B chunk 1024, mask with a hole")
    got = run_gpu(q, k, v, m2, scale=SCALE)
    assert_parity(got[:, sel], _sampled(q, k, v, m2, sel), what="32B masked chunk with hole")
    _case("decode after the mask with a hole")
    _decode_check(12)
    _case("prefix mask again")
    got = run_gpu(q, k, v, m, scale=SCALE)
    assert_parity(got[:, sel], _sampled(q, k, v, m, sel), what="32B masked chunk again")


def test_masked_calls_on_two_streams(gpu):
    from arclight_amd import device, fattn
    n_kv = 2048
    q, k, v = O.make_inputs(4242, T=512, Hq=32, Hkv=8, n_kv=n_kv)
    m_ok = O.causal_mask(512, n_kv, 1536, kv_len=2000)
    m_bad = m_ok.copy()
    m_bad[..., 100] = -np.inf
    m_bad[..., 200:210] = np.float16(-1.5)
    ref_ok = O.attention(q, k, v, m_ok, scale=SCALE)
    ref_bad = O.attention(q, k, v, m_bad, scale=SCALE)
    dq, dk, dv = fattn.upload_q(q), fattn.upload_kv(k), fattn.upload_kv(v)
    dm_ok, dm_bad = fattn.upload_mask(m_ok), fattn.upload_mask(m_bad)
    sa, sb = device.Stream(), device.Stream()
    try:
        outs_a = [_dst(q) for _ in range(3)]
        outs_b = [_dst(q) for _ in range(3)]
        # one eager call per stream allocates its workspace
        fattn.flash_attn_ext(dq, dk, dv, dm_bad, scale=SCALE, dst=outs_a[0], stream=sa)
        fattn.flash_attn_ext(dq, dk, dv, dm_ok, scale=SCALE, dst=outs_b[0], stream=sb)
        device.synchronize()
        _case("two streams, non-prefix and prefix masks interleaved")
        for i in range(3):
            fattn.flash_attn_ext(dq, dk, dv, dm_bad, scale=SCALE, dst=outs_a[i], stream=sa)
            fattn.flash_attn_ext(dq, dk, dv, dm_ok, scale=SCALE, dst=outs_b[i], stream=sb)
        device.synchronize()
        fattn.device_errors()
        for i in range(3):
            assert_parity(outs_a[i].numpy(np.float32), ref_bad, what=f"stream A (non-prefix mask) call {i}")
            assert_parity(outs_b[i].numpy(np.float32), ref_ok, what=f"stream B (prefix mask) call {i}")
    finally:
        device.synchronize()
        sa.destroy()
        sb.destroy()


def test_masked_call_replayed_with_nonprefix_then_prefix_mask(gpu):
    from arclight_amd import device, fattn
    n_kv = 1024
    q, k, v = O.make_inputs(99, T=512, Hq=32, Hkv=8, n_kv=n_kv)
    m_ok = O.causal_mask(512, n_kv, 512, kv_len=n_kv)
    m_bad = m_ok.copy()
    m_bad[..., 7] = -np.inf
    refs = {"ok": O.attention(q, k, v, m_ok, scale=SCALE), "bad": O.attention(q, k, v, m_bad, scale=SCALE)}
    dq, dk, dv = fattn.upload_q(q), fattn.upload_kv(k), fattn.upload_kv(v)
    dm = fattn.upload_mask(m_ok)
    dst = _dst(q)
    st = device.Stream()
    g = None
    try:
        fattn.flash_attn_ext(dq, dk, dv, dm, scale=SCALE, dst=dst, stream=st)   # workspace outside the capture
        st.synchronize()
        g = device.Graph(st, lambda: fattn.flash_attn_ext(dq, dk, dv, dm, scale=SCALE, dst=dst, stream=st))
        for i, which in enumerate(["bad", "ok", "ok", "bad", "ok"]):
            _case(f"replay {i}: {which} mask")
            dm.buf.upload(np.ascontiguousarray((m_ok if which == "ok" else m_bad).view(np.uint16)), dm.offset)
            dst.buf.zero()
            device.synchronize()
            g.launch(st)
            st.synchronize()
            fattn.device_errors()
            assert_parity(dst.numpy(np.float32), refs[which], what=f"replay {i} ({which} mask)")
    finally:
        device.synchronize()
        if g is not None:
            g.destroy()
        st.destroy()


def test_split_flags_and_counters_across_calls(gpu):
    """Split-KV merges hand records over through the workspace's counter
    region. Its lower half holds the prefill / split-KV arrival counters,
    which every call leaves at zero; its upper half the decode kernel's split
    flags, 64 words per (stream, kv head): a flag per split and the unit's
    epoch (word 32), which every multi-split decode call advances by one,
    leaving each used flag equal to it. On one caller workspace, decode (4
    rows), 4-draft verify (16 rows), 8-draft verify (32 rows, two row
    blocks), a prefill chunk whose row tiles are split across workgroups and
    decode again match the oracle, each twice, with the counter region as
    described after each."""
    from arclight_amd import device, fattn
    region = 256 << 10
    half = region // 8                                # words in each half
    ws = device.DeviceBuffer(region + (16 << 20))
    ws.zero()
    device.synchronize()
    cases = [
        ("decode, 4096 cells", dict(seed=21, T=1, n_kv=4096), dict(kv_len=4000)),
        ("verify 4 drafts, 8192 cells", dict(seed=22, T=4, n_kv=8192), dict(kv_len=8196, causal_pos0=8192)),
        ("verify 8 drafts, 8192 cells", dict(seed=23, T=8, n_kv=8448), dict(kv_len=8200, causal_pos0=8192)),
        ("256-token chunk over 512 cells (split row tiles)", dict(seed=24, T=256, n_kv=2048),
         dict(kv_len=2048, causal_pos0=1792)),
        ("decode, 1000 cells", dict(seed=25, T=1, n_kv=1024), dict(kv_len=1000)),
        ("decode, 32768 cells", dict(seed=26, T=1, n_kv=32768), dict(kv_len=32768)),
    ]
    epoch = 0
    for name, mk, kw in cases:
        _case(name)
        q, k, v = O.make_inputs(mk["seed"], T=mk["T"], Hq=32, Hkv=8, n_kv=mk["n_kv"])
        need = fattn.workspace_bytes(fattn.upload_q(q), fattn.upload_kv(k), fattn.upload_kv(v), None, None,
                                     _dst(q), scale=SCALE, **kw)
        assert 0 < need <= ws.nbytes, (name, need)
        ref = O.attention(q, k, v, scale=SCALE, **kw)
        for rep in range(2):
            got = run_gpu(q, k, v, scale=SCALE, workspace=ws, **kw)
            assert_parity(got, ref, what=f"{name}, call {rep}")
        words = ws.download(np.empty(region // 4, np.uint32))
        nz = np.flatnonzero(words[:half])
        assert nz.size == 0, f"{name}: {nz.size} nonzero arrival counters left, first at word {nz[0]}"
        if mk["T"] <= 8:                              # the decode kernel, split 32 ways here
            epoch += 2
        flags = words[half:].reshape(-1, 64)[:8]      # the 8 kv heads of stream 0
        assert (flags[:, 32] == epoch).all(), f"{name}: epochs {flags[:, 32]} != {epoch}"
        assert (flags[:, 0] == epoch).all(), f"{name}: split 0 flags {flags[:, 0]} != {epoch}"


def test_release_stream_workspace(gpu):
    """al_fattn_release_stream frees a stream's library workspace: split
    decode calls on the stream before and after the release (which
    allocates a new, zeroed workspace) match the oracle; releasing a stream
    that has none is AL_OK."""
    from arclight_amd import _lib, device, fattn
    lib = _lib.load()
    q, k, v = O.make_inputs(4343, T=1, Hq=32, Hkv=8, n_kv=8192)
    ref = O.attention(q, k, v, scale=SCALE, kv_len=8000)
    dq, dk, dv = fattn.upload_q(q), fattn.upload_kv(k), fattn.upload_kv(v)
    st = device.Stream()
    try:
        for rnd in range(3):
            _case(f"decode on a stream, workspace round {rnd}")
            for i in range(2):
                dst = _dst(q)
                fattn.flash_attn_ext(dq, dk, dv, scale=SCALE, kv_len=8000, dst=dst, stream=st)
                st.synchronize()
                fattn.device_errors()
                assert_parity(dst.numpy(np.float32), ref, what=f"round {rnd} call {i}")
            assert lib.al_fattn_release_stream(st.handle) == 0, lib.al_last_error()
        assert lib.al_fattn_release_stream(st.handle) == 0        # nothing left to free
    finally:
        device.synchronize()
        st.destroy()
