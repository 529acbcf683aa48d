"""The binding under nnml's threading contract, on the GPU: a worker pool in
the shape of nnml's (tests/harness/nnml_workers.cpp: nth threads walk the
nodes, each calls the op with its own (ith, nth), a global barrier after
every node, nnml/src/scheduler.cpp:122-146) runs a sequence of attention
nodes through al_fattn_f16_worker on one non-default stream.

Checks:
- every worker's status is AL_OK;
- right after each node's barrier the stream has no pending work (worker 0
  waited for it before arriving);
- workers 1..nth-1 launched nothing: their copies of each node write to a
  canary buffer, which still holds its fill pattern afterwards;
- every node's output matches oracle O2 (max-abs <= 2e-3, rel-L2 <= 1e-3).
Nodes: two decode layers, an explicitly masked decode (the call as nnml
makes it), a 4-draft verify, a masked 512-token prefill chunk, and the
masked decode and prefill nodes again carrying the library's length hints
in op_params i32[4..6] (al_fattn_apply_node_hints, as the nnml adapter
applies them: the mask is dropped and the implicit rule runs).
"""
import ctypes
import math
import os

import numpy as np
import pytest

from oracle import oracle as O
from tests.fattn_cases import assert_parity

pytestmark = pytest.mark.gpu
SCALE = 1.0 / math.sqrt(128)
HARNESS = os.path.join(os.path.dirname(os.path.abspath(__file__)), "harness", "_build", "libnnml_workers.so")
CANARY = 0x7FC0A5A5                      # a NaN pattern no kernel writes


def _case(name):
    print(f"\n[case] {name}", flush=True)


@pytest.mark.parametrize("nth", [1, 8])
def test_worker_pool_runs_nodes_like_nnml(gpu, nth):
    from arclight_amd import _lib, abi, device, fattn
    lib = _lib.load()
    assert os.path.exists(HARNESS), "harness not built (python -c 'import __graft_entry__ as g; g.build()')"
    h = ctypes.CDLL(HARNESS)
    h.al_harness_run_workers.restype = ctypes.c_int
    h.al_harness_run_workers.argtypes = [ctypes.POINTER(abi.AlFattnArgs), ctypes.POINTER(abi.AlFattnArgs),
                                         ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_int),
                                         ctypes.POINTER(ctypes.c_int)]
    st = device.Stream()
    keep = []
    nodes, others, refs, dsts, canaries = [], [], [], [], []

    def node(name, q, k, v, mask=None, hints=None, **kw):
        dq, dk, dv = fattn.upload_q(q), fattn.upload_kv(k), fattn.upload_kv(v)
        dm = fattn.upload_mask(mask) if mask is not None else None
        dst = device.DeviceTensor.empty(q.shape, np.float32, axes=abi.DST_AXES)
        can = device.DeviceTensor.from_numpy(np.full(q.shape, CANARY, np.uint32).view(np.float32),
                                             axes=abi.DST_AXES)
        keep.extend([dq, dk, dv, dm])
        a = fattn.fattn_args(dq, dk, dv, dm, None, dst, scale=SCALE, stream=st, **kw)
        b = fattn.fattn_args(dq, dk, dv, dm, None, can, scale=SCALE, stream=st, **kw)
        if hints is not None:
            op = (ctypes.c_int32 * 16)()
            op[4], op[5], op[6] = abi.AL_FATTN_HINT_TAG, hints[0], hints[1]
            assert lib.al_fattn_apply_node_hints(ctypes.byref(a), op) == 1
            assert lib.al_fattn_apply_node_hints(ctypes.byref(b), op) == 1
            assert not a.mask.data and a.kv_len == hints[0]
        nodes.append(a)
        others.append(b)
        refs.append((name, O.attention(q, k, v, mask, scale=SCALE, **kw)))
        dsts.append(dst)
        canaries.append(can)

    for l in range(2):
        q, k, v = O.make_inputs(700 + l, T=1, Hq=32, Hkv=8, n_kv=4096)
        node(f"decode layer {l}", q, k, v, kv_len=4096)
    q, k, v = O.make_inputs(710, T=1, Hq=32, Hkv=8, n_kv=4096)
    node("decode, explicit mask", q, k, v, O.causal_mask(1, 4096, 3999, kv_len=4000))
    q, k, v = O.make_inputs(711, T=4, Hq=32, Hkv=8, n_kv=4352)
    node("verify 4 drafts", q, k, v, kv_len=4100, causal_pos0=4096)
    q, k, v = O.make_inputs(712, T=512, Hq=32, Hkv=8, n_kv=2048)
    node("prefill chunk 512, explicit mask", q, k, v, O.causal_mask(512, 2048, 1536, kv_len=2048))
    q, k, v = O.make_inputs(713, T=1, Hq=32, Hkv=8, n_kv=4096)
    node("decode, explicit mask + node hints", q, k, v, O.causal_mask(1, 4096, 3999, kv_len=4000), hints=(4000, 3999))
    q, k, v = O.make_inputs(714, T=512, Hq=32, Hkv=8, n_kv=2048)
    node("prefill chunk 512, explicit mask + node hints", q, k, v, O.causal_mask(512, 2048, 1536, kv_len=2048),
         hints=(2048, 1536))

    n = len(nodes)
    arr = (abi.AlFattnArgs * n)(*nodes)
    oth = (abi.AlFattnArgs * n)(*others)
    status = (ctypes.c_int * (n * nth))()
    done = (ctypes.c_int * n)()
    try:
        _case(f"{n} nodes, {nth} workers")
        assert h.al_harness_run_workers(arr, oth, n, nth, status, done) == 0
        device.synchronize()
        fattn.device_errors()
        assert list(status) == [0] * (n * nth), list(status)
        assert list(done) == [1] * n, f"stream still busy after a node's barrier: {list(done)}"
        for (name, ref), dst, can in zip(refs, dsts, canaries):
            assert_parity(dst.numpy(np.float32), ref, what=name)
            assert (can.numpy(np.float32).view(np.uint32) == CANARY).all(), f"{name}: a worker other than 0 launched"
    finally:
        device.synchronize()
        st.destroy()
