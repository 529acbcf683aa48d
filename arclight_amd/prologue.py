"""Host-side mirror of the attention-operand producers of ArcLight's Qwen3
layer (models/qwen3.cpp:211-224) over include/arclight_prologue.h.

    q = rms_norm_rope(qcur, q_norm_w, pos, eps=eps, rope=abi.qwen3_rope())
    rms_norm_rope(kcur, k_norm_w, pos, eps=eps, rope=..., y=k_cache, rows=rows)

is the node chain rms_norm -> mul -> rope_ext (nnml/src/ops/ops.cpp:680-726,
1248-1250, 871-962), the second form followed by cpy_k's set_rows into the
f16 cache (ops.cpp:135-181). Operands are DeviceTensors in nnml order:
qcur / kcur (T, H, 128) f32, pos (T,) int32, rows (T,) int64.
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
