"""The HBM KV ring end to end on the GPU: cells placed by the library, K/V
rows written into the ring, the mask built on the device, and attention
read straight from the ring views.

Checks, per step of a scripted serving sequence (prefill, decode, a second
sequence, a rolled-back draft, a hole from seq_rm, reuse of freed cells):
  - ring memory == the oracle's set_rows applied to a zero cache, bit-exact;
  - device mask == host mask == oracle/kv_cells.py mask, bit-exact;
  - attention over the ring views with the device mask == oracle O2 on the
    same host operands, at the parity bar (max-abs 2e-3, rel-L2 1e-3), and
    the same with no mask whenever al_kv_cells_implicit reports the implicit
    length + causal rule.
"""
import math

import numpy as np
import pytest

from arclight_amd import abi
from oracle import kv_cells as KC
from oracle import oracle as O
from tests.fattn_cases import assert_parity

pytestmark = pytest.mark.gpu
SCALE = 1.0 / math.sqrt(128)


class Harness:
    def __init__(self, n_layer, kv_size, n_head_kv, n_head, n_seq_max, unified, n_pad=256, seed=0):
        from arclight_amd import kv
        self.ring = kv.KvRing(n_layer, kv_size, n_head_kv, 128, n_seq_max, n_pad, unified)
        self.orc = KC.KvCache(kv_size, n_seq_max=n_seq_max, n_pad=n_pad, unified=unified)
        self.n_stream = 1 if unified else n_seq_max
        self.n_layer, self.kv_size, self.hkv, self.hq = n_layer, kv_size, n_head_kv, n_head
        self.nc = n_head_kv * 128
        # host copies of every layer's K and V (f16 bits, [n_stream * kv_size, nc])
        self.host = [[np.zeros((self.n_stream * kv_size, self.nc), np.uint16) for _ in range(2)]
                     for _ in range(n_layer)]
        self.rng = np.random.default_rng(seed)

    def step(self, ub, name, n_stream_ub=1):
        from arclight_amd import device, fattn
        from arclight_amd._lib import call
        print(f"\n[case] kv ring: {name} ({len(ub)} tokens)", flush=True)
        want_rows, want_nkv = self.orc.place(ub)
        rows, n_kv, s0, ns = self.ring.cells.place_streams(ub)
        assert rows.tolist() == want_rows.tolist() and n_kv == want_nkv
        strms = sorted({self.orc.seq_to_stream[seqs[0]] for _, seqs in ub})
        assert (s0, ns) == (strms[0], strms[-1] - strms[0] + 1)
        assert ns == n_stream_ub
        d_rows = device.DeviceTensor.from_numpy(rows)
        T = len(ub) // n_stream_ub
        # the device mask, then the host and oracle masks
        rows_pad = (T + 63) // 64 * 64
        dm = device.DeviceTensor.empty((n_stream_ub, 1, rows_pad, n_kv), np.uint16, axes=abi.MASK_AXES)
        dm.type = abi.AL_TYPE_F16
        self.ring.cells.mask_device(ub, n_kv, dm, n_stream_ub)
        m_orc = self.orc.mask(ub, n_kv, n_stream_ub)
        m_host = self.ring.cells.mask_host(ub, n_kv, n_stream_ub)
        device.synchronize()
        m_dev = dm.numpy(np.uint16)
        assert np.array_equal(m_host.view(np.uint16), m_orc.view(np.uint16)), name
        assert np.array_equal(m_dev, m_orc.view(np.uint16)), name
        implicit = self.ring.cells.implicit(ub, n_kv) if n_stream_ub == 1 else None
        for il in range(self.n_layer):
            kc = self.rng.standard_normal((len(ub), self.nc), dtype=np.float32)
            vc = self.rng.standard_normal((len(ub), self.nc), dtype=np.float32)
            dk = device.DeviceTensor.from_numpy(kc)
            dv = device.DeviceTensor.from_numpy(vc)
            self.ring.cpy_kv(il, dk, dv, d_rows)
            self.host[il][0] = O.set_rows(self.host[il][0], kc, rows)
            self.host[il][1] = O.set_rows(self.host[il][1], vc, rows)
            # ring memory, all streams, bit-exact
            for view, h in ((self.ring.get_k(il, self.kv_size), self.host[il][0]),
                            (self.ring.get_v(il, self.kv_size), self.host[il][1])):
                got = np.empty_like(h)
                device.synchronize()
                fattn.device_errors()
                call("al_util_memcpy_d2h", got.ctypes.data, view.ptr, got.nbytes)
                assert np.array_equal(got, h), f"{name}: layer {il} ring contents"
            # attention from the views of the ubatch's streams
            kview = self.ring.get_k(il, n_kv, s0, ns)
            vview = self.ring.get_v(il, n_kv, s0, ns)
            q = self.rng.standard_normal((n_stream_ub, T, self.hq, 128), dtype=np.float32)
            hk = self.host[il][0].reshape(self.n_stream, self.kv_size, self.hkv, 128)[s0:s0 + ns, :n_kv]
            hv = self.host[il][1].reshape(self.n_stream, self.kv_size, self.hkv, 128)[s0:s0 + ns, :n_kv]
            ref = O.attention(q, hk.view(np.float16), hv.view(np.float16), m_orc, scale=SCALE)
            dq = fattn.upload_q(q)
            got = fattn.flash_attn_ext(dq, kview, vview, dm, scale=SCALE)
            device.synchronize()
            assert_parity(got.numpy(np.float32), ref, what=f"{name} layer {il} mask")
            if implicit is not None:
                kv_len, pos0 = implicit
                got = fattn.flash_attn_ext(dq, kview, vview, None, scale=SCALE, kv_len=kv_len, causal_pos0=pos0)
                device.synchronize()
                assert_parity(got.numpy(np.float32), ref, what=f"{name} layer {il} implicit")
        return rows, n_kv, implicit


def _seq(seq, p0, n):
    return [(p0 + i, [seq]) for i in range(n)]


def test_ring_serving_sequence_unified(gpu):
    # Qwen3-4B attention shape (8 kv heads, 32 query heads, head_dim 128), 2 layers
    h = Harness(n_layer=2, kv_size=1024, n_head_kv=8, n_head=32, n_seq_max=2, unified=True)
    _, n_kv, imp = h.step(_seq(0, 0, 300), "prefill 300")
    assert n_kv == 512 and imp == (300, 0)
    _, _, imp = h.step(_seq(0, 300, 1), "decode")
    assert imp == (301, 300)
    h.step(_seq(0, 301, 4), "verify 4 drafts")
    h.orc.seq_rm(0, 303, -1)                       # two drafts rejected
    h.ring.cells.seq_rm(0, 303, -1)
    _, _, imp = h.step(_seq(0, 303, 1), "decode after rollback")
    assert imp == (304, 303)
    h.step(_seq(1, 0, 70), "second sequence prefill")
    h.step([(304, [0]), (70, [1])], "two-sequence decode")
    h.orc.seq_rm(0, 10, 40)                        # a hole in sequence 0
    h.ring.cells.seq_rm(0, 10, 40)
    rows, _, imp = h.step(_seq(1, 71, 16), "second sequence chunk into freed cells")
    assert imp is None and rows.min() == 10      # reuses the hole first
    h.step(_seq(0, 305, 1), "decode with hole")


def test_ring_two_streams(gpu):
    h = Harness(n_layer=1, kv_size=512, n_head_kv=8, n_head=32, n_seq_max=2, unified=False, seed=1)
    h.step(_seq(0, 0, 40) + _seq(1, 0, 40), "two-stream prefill", n_stream_ub=2)
    h.step(_seq(0, 40, 1) + _seq(1, 40, 1), "two-stream decode", n_stream_ub=2)
    h.step(_seq(1, 41, 3), "one stream of two", n_stream_ub=1)


def test_ring_rejects_bad_views(gpu):
    from arclight_amd import kv
    from arclight_amd._lib import ArclightError
    r = kv.KvRing(1, 256, 8)
    with pytest.raises(ArclightError):
        r.get_k(1, 256)                             # layer out of range
    with pytest.raises(ArclightError):
        r.get_v(0, 512)                             # n_kv beyond the cache
    with pytest.raises(ArclightError):
        r.get_k(0, 256, 1, 1)                       # stream beyond the cache
    r.close()
