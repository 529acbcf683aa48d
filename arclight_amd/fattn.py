"""Host-side mirror of ArcLight's flash-attention operator over the HIP C ABI.

`flash_attn_ext` takes the node's operands as the reference graph builds
them (nnml_flash_attn_ext, nnml/src/tensor.cpp:1292-1320, with
nnml_flash_attn_ext_add_sinks :1322-1332 and _set_prec :1334-1338) and runs
NNML_OP_FLASH_ATTN_EXT (nnml/src/ops/ops.cpp:1432-1445) on the GPU:

    dst = flash_attn_ext(q, k, v, mask, sinks, scale=1/sqrt(128))

Operands are DeviceTensor views in HBM with the physical layouts of
arclight_amd.abi (q (B,T,Hq,D) f32, k/v (B,n_kv,Hkv,D) f16, mask
(m3,m2,rows,n_kv) f16, dst (B,T,Hq,D) f32). Errors the reference asserts on
raise ArclightError with status AL_ERR_INVALID.
"""
import ctypes

import numpy as np

from . import abi
from ._lib import call, load
from .device import DeviceTensor


def fattn_args(q, k, v, mask=None, sinks=None, dst=None, *, scale, max_bias=0.0, logit_softcap=0.0,
               prec=abi.AL_PREC_F32, kv_len=0, causal_pos0=-1, stream=None, workspace=None, dyn_len=None):
    a = abi.AlFattnArgs()
    a.q = q.desc()
    a.k = k.desc()
    a.v = v.desc()
    a.mask = mask.desc() if mask is not None else abi.empty_tensor()
    a.sinks = sinks.desc() if sinks is not None else abi.empty_tensor()
    a.dst = dst.desc()
    a.scale = scale
    a.max_bias = max_bias
    a.logit_softcap = logit_softcap
    a.prec = prec
    a.kv_len = kv_len
    a.causal_pos0 = causal_pos0
    a.stream = stream.handle if stream is not None else None
    if workspace is not None:
        a.workspace = workspace.ptr
        a.workspace_bytes = workspace.nbytes
    if dyn_len is not None:
        a.dyn_len = dyn_len.ptr
    return a


def flash_attn_ext(q, k, v, mask=None, sinks=None, *, scale, max_bias=0.0, logit_softcap=0.0,
                   prec=abi.AL_PREC_F32, dst=None, kv_len=0, causal_pos0=-1, stream=None, workspace=None,
                   dyn_len=None):
    """Enqueues the op on `stream` and returns dst (allocated when None).
    dyn_len: an int32 (2,) DeviceTensor {kv_len, causal_pos0} read when the
    kernel runs (for graphs replayed per decode step); kv_len is then the
    bound and causal_pos0 >= 0 selects causal masking."""
    if dst is None:
        B, T, Hq = q.shape[0], q.shape[1], q.shape[2]
        dst = DeviceTensor.empty((B, T, Hq, v.shape[3]), np.float32, axes=abi.DST_AXES)
    a = fattn_args(q, k, v, mask, sinks, dst, scale=scale, max_bias=max_bias, logit_softcap=logit_softcap,
                   prec=prec, kv_len=kv_len, causal_pos0=causal_pos0, stream=stream, workspace=workspace,
                   dyn_len=dyn_len)
    call("al_fattn_f16", ctypes.byref(a))
    return dst


def workspace_bytes(q, k, v, mask=None, sinks=None, dst=None, **kw):
    a = fattn_args(q, k, v, mask, sinks, dst, **kw)
    return int(load().al_fattn_workspace_bytes(ctypes.byref(a)))


def set_rows(cache, rows, idx, stream=None):
    """KV write (nnml_compute_forward_set_rows_f32, nnml/src/ops/ops.cpp:135-181):
    cache rows idx[i] <- f16(rows[i]). `cache` is an f16 DeviceTensor
    [nc, n_cells, ...], `rows` f32 [nc, n, ...], `idx` i64/i32 [n]."""
    d, s, i = cache.desc(), rows.desc(), idx.desc()
    call("al_set_rows_f32_f16", ctypes.byref(d), ctypes.byref(s), ctypes.byref(i),
         stream.handle if stream is not None else None)


def device_errors():
    call("al_device_errors")


def upload_q(arr):
    return DeviceTensor.from_numpy(np.asarray(arr, dtype=np.float32), axes=abi.Q_AXES)


def upload_kv(arr):
    arr = np.asarray(arr)
    if arr.dtype == np.float16:
        arr = arr.view(np.uint16)
    return DeviceTensor.from_numpy(arr, axes=abi.KV_AXES)


def upload_mask(arr):
    arr = np.asarray(arr)
    if arr.dtype == np.float16:
        arr = arr.view(np.uint16)
    return DeviceTensor.from_numpy(arr, axes=abi.MASK_AXES)


def upload_sinks(arr):
    return DeviceTensor.from_numpy(np.asarray(arr, dtype=np.float32))
