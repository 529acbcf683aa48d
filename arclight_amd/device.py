"""Device memory, streams and events through the library's C ABI.

A DeviceTensor is a device buffer described the way nnml describes a tensor
view (type, ne[4], nb[4] in bytes; nnml/include/tensor.h:78-198). Arrays
move between host numpy arrays and HBM with upload()/download().
"""
import ctypes

import numpy as np

from . import abi
from ._lib import call, load

_NP_TYPES = {np.dtype(np.float32): abi.AL_TYPE_F32, np.dtype(np.float16): abi.AL_TYPE_F16,
             np.dtype(np.uint16): abi.AL_TYPE_F16, np.dtype(np.int32): abi.AL_TYPE_I32,
             np.dtype(np.int64): abi.AL_TYPE_I64}


class DeviceBuffer:
    """An owned hipMalloc allocation."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        call("al_util_malloc", ctypes.byref(p), max(self.nbytes, 1))
        self.ptr = p.value

    def free(self):
        if self.ptr:
            call("al_util_free", self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr and load() is not None:
                load().al_util_free(self.ptr)
        except Exception:
            pass

    def upload(self, arr, offset=0):
        arr = np.ascontiguousarray(arr)
        assert offset + arr.nbytes <= self.nbytes
        call("al_util_memcpy_h2d", self.ptr + offset, arr.ctypes.data, arr.nbytes)

    def download(self, arr, offset=0):
        assert arr.flags.c_contiguous and offset + arr.nbytes <= self.nbytes
        call("al_util_memcpy_d2h", arr.ctypes.data, self.ptr + offset, arr.nbytes)
        return arr

    def zero(self):
        call("al_util_memset", self.ptr, 0, self.nbytes)


class DeviceTensor:
    """A typed view into a DeviceBuffer: nnml's (type, ne, nb, data)."""

    def __init__(self, buf, typ, shape, strides=None, offset=0, axes=None):
        """`shape`/`strides` are numpy-order (bytes); `axes[i]` names the
        numpy axis of nnml dim i (default: reversed, i.e. contiguous nnml)."""
        self.buf = buf
        self.type = typ
        self.shape = tuple(int(x) for x in shape)
        esz = abi.TYPE_SIZES[typ]
        if strides is None:
            strides = []
            acc = esz
            for d in reversed(self.shape):
                strides.insert(0, acc)
                acc *= d
        self.strides = tuple(int(x) for x in strides)
        self.offset = int(offset)
        nd = len(self.shape)
        self.axes = tuple(axes) if axes is not None else tuple(range(nd - 1, -1, -1)) + tuple(range(nd, 4))
        self._pad_shape = self.shape + (1,) * (4 - nd)
        self._pad_strides = self.strides + (self.strides[0] * self.shape[0] if nd else esz,) * (4 - nd)

    @property
    def ptr(self):
        return self.buf.ptr + self.offset

    def desc(self):
        return abi.tensor_desc(self.ptr, self.type, self._pad_shape, self._pad_strides, self.axes)

    @classmethod
    def from_numpy(cls, arr, axes=None, buf=None):
        arr = np.ascontiguousarray(arr)
        typ = _NP_TYPES[arr.dtype]
        buf = buf or DeviceBuffer(arr.nbytes)
        buf.upload(arr)
        return cls(buf, typ, arr.shape, arr.strides, 0, axes)

    @classmethod
    def empty(cls, shape, dtype, axes=None):
        dt = np.dtype(dtype)
        n = int(np.prod(shape)) * dt.itemsize
        return cls(DeviceBuffer(n), _NP_TYPES[dt], shape, None, 0, axes)

    def numpy(self, dtype):
        """Downloads a contiguous tensor into a new numpy array of `dtype`."""
        out = np.empty(self.shape, dtype=dtype)
        self.buf.download(out, self.offset)
        return out


class Stream:
    def __init__(self):
        s = ctypes.c_void_p()
        call("al_util_stream_create", ctypes.byref(s))
        self.handle = s.value

    def synchronize(self):
        call("al_util_stream_synchronize", self.handle)

    def destroy(self):
        if self.handle:
            call("al_util_stream_destroy", self.handle)
            self.handle = None


class Event:
    def __init__(self):
        e = ctypes.c_void_p()
        call("al_util_event_create", ctypes.byref(e))
        self.handle = e.value

    def record(self, stream=None):
        call("al_util_event_record", self.handle, stream.handle if stream else None)

    def synchronize(self):
        call("al_util_event_synchronize", self.handle)

    def elapsed_ms(self, end):
        ms = ctypes.c_float()
        call("al_util_event_elapsed_ms", self.handle, end.handle, ctypes.byref(ms))
        return ms.value

    def destroy(self):
        if self.handle:
            call("al_util_event_destroy", self.handle)
            self.handle = None


class Graph:
    """A HIP graph of the work enqueue() puts on `stream` (captured, not
    run): replayed by launch(). Everything the captured calls touch must
    exist before capture (device buffers, the library's workspaces, which a
    first eager call allocates)."""

    def __init__(self, stream, enqueue):
        call("al_util_graph_begin", stream.handle)
        ge = ctypes.c_void_p()
        try:
            enqueue()
        finally:
            call("al_util_graph_end", stream.handle, ctypes.byref(ge))
        self.handle = ge.value

    def launch(self, stream):
        call("al_util_graph_launch", self.handle, stream.handle)

    def destroy(self):
        if self.handle:
            call("al_util_graph_destroy", self.handle)
            self.handle = None


def synchronize():
    call("al_util_device_synchronize")


def device_count():
    n = ctypes.c_int()
    call("al_util_device_count", ctypes.byref(n))
    return n.value


def device_info():
    name = ctypes.create_string_buffer(256)
    arch = ctypes.create_string_buffer(256)
    ncu = ctypes.c_int()
    mem = ctypes.c_uint64()
    call("al_util_device_info", name, 256, ctypes.byref(ncu), ctypes.byref(mem), arch, 256)
    return {"name": name.value.decode(), "arch": arch.value.decode(), "n_cu": ncu.value, "hbm_bytes": mem.value}
