"""al_fattn_f16_noalloc (the entry point that allocates nothing) against
al_fattn_f16 on the same inputs, through the C ABI: two calls in a row, the
second with a smaller input, each bit-identical to the allocating entry
point's result (same plan and kernels) and within the parity bar of oracle
O2 (max-abs <= 2e-3, rel-L2 <= 1e-3). Covers a multi-split decode (counters
and merge records in the device array), masked many-row calls (one whose
mask is a causal prefix, one taken value by value), and a call that needs
more scratch than the array holds (rejected with AL_ERR_WORKSPACE)."""
import ctypes
import math

import numpy as np
import pytest

from oracle import oracle as O
from tests.fattn_cases import assert_parity

pytestmark = pytest.mark.gpu
SCALE = 1.0 / math.sqrt(128)


def _case(name):
    print(f"\n[case] {name}", flush=True)


def _both(q, k, v, mask=None, **kw):
    """dst of al_fattn_f16 and of al_fattn_f16_noalloc on the same operands."""
    from arclight_amd import _lib, abi, device, fattn
    lib = _lib.load()
    dq, dk, dv = fattn.upload_q(q), fattn.upload_kv(k), fattn.upload_kv(v)
    dm = fattn.upload_mask(mask) if mask is not None else None
    outs = []
    for entry in (lib.al_fattn_f16, lib.al_fattn_f16_noalloc):
        dst = device.DeviceTensor.empty(q.shape, np.float32, axes=abi.DST_AXES)
        a = fattn.fattn_args(dq, dk, dv, dm, None, dst, scale=SCALE, **kw)
        rc = entry(ctypes.byref(a))
        assert rc == 0, lib.al_last_error().decode()
        device.synchronize()
        fattn.device_errors()
        outs.append(dst.numpy(np.float32))
    return outs


def _check(name, q, k, v, mask=None, **kw):
    _case(name)
    ref = O.attention(q, k, v, mask, scale=SCALE, **kw)
    alloc, noalloc = _both(q, k, v, mask, **kw)
    assert np.array_equal(alloc, noalloc, equal_nan=True), f"{name}: no-allocation result differs"
    assert_parity(noalloc, ref, what=name)


def test_noalloc_matches_allocating_entry(gpu):
    from arclight_amd import _lib
    assert _lib.load().al_fattn_noalloc_init() == 0
    # decode: 32 splits over 16384 cells, then a smaller call (4096 cells)
    q, k, v = O.make_inputs(501, T=1, Hq=32, Hkv=8, n_kv=16384)
    _check("decode 16384 cells", q, k, v, kv_len=16384)
    q, k, v = O.make_inputs(502, T=1, Hq=32, Hkv=8, n_kv=4096)
    _check("decode 4000 of 4096 cells (smaller)", q, k, v, kv_len=4000)
    # masked many-row calls: a causal prefix mask, then a smaller one with a hole
    q, k, v = O.make_inputs(503, T=512, Hq=32, Hkv=8, n_kv=2048)
    _check("512-token chunk, explicit causal mask", q, k, v, O.causal_mask(512, 2048, 1536, kv_len=2000))
    q, k, v = O.make_inputs(504, T=128, Hq=32, Hkv=8, n_kv=1024)
    m = O.causal_mask(128, 1024, 896, kv_len=1024)
    m[..., 5] = -np.inf
    _check("128-token chunk, mask with a hole (smaller)", q, k, v, m)


def test_noalloc_rejects_oversized_call(gpu):
    from arclight_amd import _lib, abi, device, fattn
    lib = _lib.load()
    # a masked 1008-token call whose mask rows are not 16-byte aligned (1025
    # columns), so the split-KV kernel takes it: 63 row tiles x 8 kv heads
    # in 2 splits, 504 x 2 records of 64 rows x 528 bytes (34 MB)
    T, n_kv = 1008, 1024
    dq = device.DeviceTensor.empty((1, T, 32, 128), np.float32, axes=abi.Q_AXES)
    dk = device.DeviceTensor.empty((1, n_kv, 8, 128), np.uint16, axes=abi.KV_AXES)
    dv = device.DeviceTensor.empty((1, n_kv, 8, 128), np.uint16, axes=abi.KV_AXES)
    dm = fattn.upload_mask(O.causal_mask(T, n_kv + 1, 16, kv_len=n_kv))
    dst = device.DeviceTensor.empty((1, T, 32, 128), np.float32, axes=abi.DST_AXES)
    a = fattn.fattn_args(dq, dk, dv, dm, None, dst, scale=SCALE)
    need = lib.al_fattn_workspace_bytes(ctypes.byref(a))
    assert need > (32 << 20), need
    _case(f"oversized call ({need} bytes of scratch)")
    assert lib.al_fattn_f16_noalloc(ctypes.byref(a)) == abi.AL_ERR_WORKSPACE
    assert "device array" in lib.al_last_error().decode()
