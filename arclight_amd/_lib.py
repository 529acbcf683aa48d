"""Loads libarclight_fattn.so (the HIP build of this package) through ctypes.

There is no fallback: if the library is missing or fails to load, every
entry point raises. Build it with `python -m arclight_amd.build`.
"""
import ctypes
import os

from . import abi

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libarclight_fattn.so")

# C ABI exported by the library: name -> (restype, argtypes)
_VP = ctypes.c_void_p
_U64 = ctypes.c_uint64
_I = ctypes.c_int
SIGNATURES = {
    # include/arclight_fattn.h
    "al_fattn_f16": (_I, [ctypes.POINTER(abi.AlFattnArgs)]),
    "al_fattn_workspace_bytes": (_U64, [ctypes.POINTER(abi.AlFattnArgs)]),
    "al_fattn_f16_worker": (_I, [ctypes.POINTER(abi.AlFattnArgs), _I, _I]),
    "al_fattn_apply_node_hints": (_I, [ctypes.POINTER(abi.AlFattnArgs), ctypes.POINTER(ctypes.c_int32)]),
    "al_fattn_release_stream": (_I, [_VP]),
    "al_fattn_noalloc_init": (_I, []),
    "al_fattn_f16_noalloc": (_I, [ctypes.POINTER(abi.AlFattnArgs)]),
    "al_last_error": (ctypes.c_char_p, []),
    "al_set_rows_f32_f16": (_I, [ctypes.POINTER(abi.AlTensor)] * 3 + [_VP]),
    "al_device_errors": (_I, []),
    "al_version": (ctypes.c_char_p, []),
    # include/arclight_util.h
    "al_util_device_count": (_I, [ctypes.POINTER(_I)]),
    "al_util_set_device": (_I, [_I]),
    "al_util_device_info": (_I, [ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(_I), ctypes.POINTER(_U64),
                                 ctypes.c_char_p, ctypes.c_size_t]),
    "al_util_malloc": (_I, [ctypes.POINTER(_VP), _U64]),
    "al_util_free": (_I, [_VP]),
    "al_util_memcpy_h2d": (_I, [_VP, _VP, _U64]),
    "al_util_memcpy_d2h": (_I, [_VP, _VP, _U64]),
    "al_util_memcpy_d2d": (_I, [_VP, _VP, _U64, _VP]),
    "al_util_memset": (_I, [_VP, _I, _U64]),
    "al_util_device_synchronize": (_I, []),
    "al_util_stream_create": (_I, [ctypes.POINTER(_VP)]),
    "al_util_stream_destroy": (_I, [_VP]),
    "al_util_stream_synchronize": (_I, [_VP]),
    "al_util_event_create": (_I, [ctypes.POINTER(_VP)]),
    "al_util_event_destroy": (_I, [_VP]),
    "al_util_event_record": (_I, [_VP, _VP]),
    "al_util_event_synchronize": (_I, [_VP]),
    "al_util_event_elapsed_ms": (_I, [_VP, _VP, ctypes.POINTER(ctypes.c_float)]),
    "al_util_graph_begin": (_I, [_VP]),
    "al_util_graph_end": (_I, [_VP, ctypes.POINTER(_VP)]),
    "al_util_graph_launch": (_I, [_VP, _VP]),
    "al_util_graph_destroy": (_I, [_VP]),
    "al_util_fill_randn_f32": (_I, [_VP, _U64, _U64, _U64, _VP]),
    "al_util_fill_randn_f16": (_I, [_VP, _U64, _U64, _U64, _VP]),
    "al_util_f32_to_f16": (_I, [_VP, _VP, _U64, _VP]),
    "al_util_copy_kernel": (_I, [_VP, _VP, _U64, _VP]),
    "al_util_empty_launch": (_I, [ctypes.c_int, ctypes.c_int, ctypes.c_int, _VP]),
    # include/arclight_kv.h
    "al_kv_cells_create": (_I, [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int32,
                                ctypes.POINTER(_VP)]),
    "al_kv_cells_destroy": (_I, [_VP]),
    "al_kv_cells_clear": (_I, [_VP]),
    "al_kv_cells_place": (_I, [_VP, ctypes.POINTER(abi.AlUbatch), _VP] + [ctypes.POINTER(ctypes.c_uint32)] * 3),
    "al_kv_cells_seq_rm": (_I, [_VP, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]),
    "al_kv_cells_state": (_I, [_VP, _VP, _VP]),
    "al_kv_cells_mask_host": (_I, [_VP, ctypes.POINTER(abi.AlUbatch), ctypes.c_uint32, ctypes.c_uint32, _VP]),
    "al_kv_cells_mask_device": (_I, [_VP, ctypes.POINTER(abi.AlUbatch), ctypes.c_uint32, ctypes.c_uint32,
                                     ctypes.POINTER(abi.AlTensor), _VP]),
    "al_kv_cells_implicit": (_I, [_VP, ctypes.POINTER(abi.AlUbatch), ctypes.c_uint32,
                                  ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64)]),
    "al_kv_ring_create": (_I, [ctypes.POINTER(abi.AlKvRingParams), ctypes.POINTER(_VP)]),
    "al_kv_ring_destroy": (_I, [_VP]),
    "al_kv_ring_cells": (_VP, [_VP]),
    "al_kv_ring_view_k": (_I, [_VP] + [ctypes.c_uint32] * 4 + [ctypes.POINTER(abi.AlTensor)]),
    "al_kv_ring_view_v": (_I, [_VP] + [ctypes.c_uint32] * 4 + [ctypes.POINTER(abi.AlTensor)]),
    "al_kv_ring_write": (_I, [_VP, ctypes.c_uint32] + [ctypes.POINTER(abi.AlTensor)] * 3 + [_VP]),
    # include/arclight_prologue.h
    "al_rms_norm_rope_f32": (_I, [ctypes.POINTER(abi.AlTensor)] * 3 + [ctypes.c_float, ctypes.POINTER(abi.AlRopeParams)]
                             + [ctypes.POINTER(abi.AlTensor)] * 2 + [_VP]),
    "al_attn_inputs_f32": (_I, [ctypes.POINTER(abi.AlAttnInputsArgs), _VP]),
    "al_fattn_f16_with_inputs": (_I, [ctypes.POINTER(abi.AlAttnInputsArgs), ctypes.POINTER(abi.AlFattnArgs)]),
    # include/arclight_matmul.h
    "al_mul_mat_q4_0_f32": (_I, [ctypes.POINTER(abi.AlTensor)] * 3 + [_VP]),
    "al_mul_mat_q4_0_check_inverse": (_I, [ctypes.POINTER(ctypes.c_ulonglong)]),
}

_lib = None


class ArclightError(RuntimeError):
    def __init__(self, fn, status, message):
        self.status = status
        super().__init__(f"{fn} -> {abi.STATUS_NAMES.get(status, status)}: {message}")


def load():
    """Returns the loaded library, loading it on first use. Raises if absent."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"arclight_amd HIP library not built: {LIB_PATH} "
                               "(run `python -m arclight_amd.build`)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(fn_name, status):
    if status != abi.AL_OK:
        msg = load().al_last_error().decode(errors="replace")
        raise ArclightError(fn_name, status, msg)
    return status


def call(fn_name, *args):
    """Calls a status-returning entry point and raises ArclightError on failure."""
    return check(fn_name, getattr(load(), fn_name)(*args))
