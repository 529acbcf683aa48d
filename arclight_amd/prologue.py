"""Host-side mirror of the attention-operand producers of ArcLight's Qwen3
layer (models/qwen3.cpp:211-224) over include/arclight_prologue.h.

    q = rms_norm_rope(qcur, q_norm_w, pos, eps=eps, rope=abi.qwen3_rope())
    rms_norm_rope(kcur, k_norm_w, pos, eps=eps, rope=..., y=k_cache, rows=rows)

is the node chain rms_norm -> mul -> rope_ext (nnml/src/ops/ops.cpp:680-726,
1248-1250, 871-962), the second form followed by cpy_k's set_rows into the
f16 cache (ops.cpp:135-181). Operands are DeviceTensors in nnml order:
qcur / kcur (T, H, 128) f32, pos (T,) int32, rows (T,) int64.

    attn_inputs(qcur, q_norm_w, kcur, k_norm_w, vcur, pos, rows, q_out, k_cache, v_cache, eps=eps, rope=...)

does both of those and the V write (cpy_v's set_rows) in one launch, and

    attention_with_inputs(qcur, q_norm_w, kcur, k_norm_w, vcur, pos, rows, q_out, k_cache, v_cache,
                          k_view, v_view, dst, eps=eps, rope=..., scale=...)

folds that launch into the decode attention kernel (al_fattn_f16_with_inputs).
"""
import ctypes

import numpy as np

from . import abi
from ._lib import call
from .device import DeviceTensor


def rms_norm_rope(x, w, pos, *, eps, rope=None, y=None, rows=None, stream=None):
    """Enqueues the op; returns y (an f32 (T, H, 128) DeviceTensor allocated
    when None and rows is None)."""
    if y is None:
        if rows is not None:
            raise ValueError("the cache form needs y (the f16 cache) and rows")
        y = DeviceTensor.empty(x.shape, np.float32)
    xd, pd, yd = x.desc(), pos.desc(), y.desc()
    wd = w.desc() if w is not None else None
    rd = rows.desc() if rows is not None else None
    call("al_rms_norm_rope_f32", ctypes.byref(xd), ctypes.byref(wd) if wd is not None else None, ctypes.byref(pd),
         eps, ctypes.byref(rope) if rope is not None else None, ctypes.byref(yd),
         ctypes.byref(rd) if rd is not None else None, stream.handle if stream is not None else None)
    return y


def _inputs_args(q, q_w, k, k_w, v, pos, rows, q_out, k_cache, v_cache, eps, rope):
    a = abi.AlAttnInputsArgs()
    a.q, a.k, a.v = q.desc(), k.desc(), v.desc()
    if q_w is not None:
        a.q_w = q_w.desc()
    if k_w is not None:
        a.k_w = k_w.desc()
    a.pos, a.rows = pos.desc(), rows.desc()
    a.q_out, a.k_cache, a.v_cache = q_out.desc(), k_cache.desc(), v_cache.desc()
    a.eps = eps
    if rope is not None:
        a.rope = ctypes.pointer(rope)
    return a


def attn_inputs(q, q_w, k, k_w, v, pos, rows, q_out, k_cache, v_cache, *, eps, rope=None, stream=None):
    """Enqueues Q into q_out, K into k_cache and V into v_cache (at cache
    rows `rows`) as one kernel; same results as rms_norm_rope for Q and K
    and set_rows for V. v is an f32 (T, n) DeviceTensor."""
    a = _inputs_args(q, q_w, k, k_w, v, pos, rows, q_out, k_cache, v_cache, eps, rope)
    call("al_attn_inputs_f32", ctypes.byref(a), stream.handle if stream is not None else None)
    return q_out


def attention_with_inputs(q, q_w, k, k_w, v, pos, rows, q_out, k_cache, v_cache, k_view, v_view, dst, *, eps,
                          scale, rope=None, kv_len=0, causal_pos0=-1, dyn_len=None, stream=None):
    """attn_inputs followed by flash_attn_ext over (q_out, k_view, v_view)
    in one decode-kernel launch, with the same results bit for bit. k_view /
    v_view are the attention's views of k_cache / v_cache (cell c = cache
    row c); q_out is (T, Hq, 128). Raises ArclightError(AL_ERR_UNSUPPORTED)
    for calls the decode kernel does not take (nothing is enqueued then)."""
    from . import fattn
    a = _inputs_args(q, q_w, k, k_w, v, pos, rows, q_out, k_cache, v_cache, eps, rope)
    T, Hq = q_out.shape[0], q_out.shape[1]
    qv = DeviceTensor(q_out.buf, abi.AL_TYPE_F32, (1, T, Hq, 128), None, q_out.offset, abi.Q_AXES)
    fa = fattn.fattn_args(qv, k_view, v_view, None, None, dst, scale=scale, kv_len=kv_len, causal_pos0=causal_pos0,
                          stream=stream, dyn_len=dyn_len)
    call("al_fattn_f16_with_inputs", ctypes.byref(a), ctypes.byref(fa))
    return dst
