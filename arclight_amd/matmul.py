"""Host-side mirror of the attention output projection of ArcLight's Qwen3
layer over include/arclight_matmul.h.

    y = mul_mat_q4_0(wo, x)

is build_attn's build_lora_mm(WO, cur) (nnml/src/cgraph.cpp:497-500), an
nnml_mul_mat node with Q4_0 weights and the f32 attention output as src1
(nnml_compute_forward_mul_mat, nnml/src/ops/ops.cpp:1252-1274). Operands:
wo a Q4_0Matrix of N rows by K columns; x an f32 (T, K) DeviceTensor, the
flash-attention output (T, Hq, D) viewed as rows of K = Hq * D
(cgraph.cpp:294); y an f32 (T, N) DeviceTensor.
"""
import ctypes

import numpy as np

from . import abi
from ._lib import call
from .device import DeviceBuffer, DeviceTensor


class Q4_0Matrix:
    """N rows of K / 32 Q4_0 blocks in device memory, rows contiguous: the
    layout nnml keeps a Q4_0 weight tensor in (ne = [K, N], nb0 = 18,
    nb1 = K / 32 * 18)."""

    def __init__(self, blocks, K, N):
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        if K % abi.QK4_0 or blocks.size != N * (K // abi.QK4_0) * abi.Q4_0_BLOCK_BYTES:
            raise ValueError(f"Q4_0 blocks: {blocks.size} bytes for a [{K}, {N}] matrix")
        self.K, self.N = int(K), int(N)
        self.buf = DeviceBuffer(blocks.size)
        self.buf.upload(blocks)

    def desc(self):
        row = self.K // abi.QK4_0 * abi.Q4_0_BLOCK_BYTES
        return abi.make_tensor(self.buf.ptr, abi.AL_TYPE_Q4_0, [self.K, self.N, 1, 1],
                               [abi.Q4_0_BLOCK_BYTES, row, row * self.N, row * self.N])


def mul_mat_q4_0(w, x, y=None, stream=None):
    """Enqueues y = x W^T (each of the T rows of x times each of the N rows
    of W); returns y, an f32 (T, N) DeviceTensor allocated when None."""
    if y is None:
        y = DeviceTensor.empty((x.shape[0], w.N), np.float32)
    wd, xd, yd = w.desc(), x.desc(), y.desc()
    call("al_mul_mat_q4_0_f32", ctypes.byref(wd), ctypes.byref(xd), ctypes.byref(yd),
         stream.handle if stream is not None else None)
    return y


def check_inverse():
    """Floats d in [0, +inf] where the Q8_0 quantization's reciprocal of a
    block scale (hardware estimate and one Newton step on [2^-126, 2^126))
    differs from the IEEE quotient 1 / d: 0 on a correct device."""
    n = ctypes.c_ulonglong(0)
    call("al_mul_mat_q4_0_check_inverse", ctypes.byref(n))
    return n.value
