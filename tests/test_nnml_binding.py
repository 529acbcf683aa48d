"""The nnml-side binding of the operator (row a12 of the hot path: the call
site, nnml/src/scheduler.cpp:98-101,135-142, nnml/include/thread.h:153-168).

CPU checks, no GPU:
- arclight_amd/nnml/ops_fattn_hip.cpp, the code a maintainer adds to nnml,
  compiles against the reference's own headers (nnml/include/tensor.h, ops.h,
  thread.h) when the reference tree is present; only compiled, nothing of the
  reference is linked or run. ROCm's clang builds it: GCC 11 rejects the
  headers' `__fp16` declarations (ops.h:365).
- al_fattn_f16_worker returns at once for every worker but 0, without
  reading its arguments or calling the HIP runtime (here there is no GPU, so
  any runtime call would fail), and rejects (ith, nth) outside 0 <= ith < nth.
The GPU side (worker 0 launches and waits before the barrier, results match
the oracle) is tests/test_gpu_nnml_workers.py.
"""
import ctypes
import os
import shutil
import subprocess

import pytest

from arclight_amd import _lib, abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NNML_INCLUDE = "/root/reference/nnml/include"
ADAPTER = os.path.join(ROOT, "arclight_amd", "nnml", "ops_fattn_hip.cpp")
CLANG = "/opt/rocm/llvm/bin/clang++"


def test_adapter_compiles_against_nnml_headers(tmp_path):
    if not os.path.isdir(NNML_INCLUDE):
        pytest.skip("reference headers not present (they exist only in the build container)")
    if not os.path.exists(CLANG):
        pytest.skip("ROCm clang++ not present")
    obj = tmp_path / "ops_fattn_hip.o"
    r = subprocess.run([CLANG, "-std=c++17", "-D_GNU_SOURCE", "-Wall", "-Werror", "-isystem", NNML_INCLUDE,
                        "-I", os.path.join(ROOT, "include"), "-c", ADAPTER, "-o", str(obj)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    nm = shutil.which("nm")
    if nm:
        syms = subprocess.run([nm, "-C", str(obj)], capture_output=True, text=True, check=True).stdout
        assert "T nnml_compute_forward_flash_attn_ext_hip(nnml_tensor*, nnml_compute_state const*)" in syms
        assert "U al_fattn_f16_worker" in syms
        assert "U al_fattn_apply_node_hints" in syms


def _lib_cpu():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    lib.al_fattn_f16_worker.restype = ctypes.c_int
    lib.al_fattn_f16_worker.argtypes = [ctypes.POINTER(abi.AlFattnArgs), ctypes.c_int, ctypes.c_int]
    lib.al_last_error.restype = ctypes.c_char_p
    return lib


def test_other_workers_return_without_the_device():
    lib = _lib_cpu()
    a = abi.AlFattnArgs()                      # all zero: q, k, v, dst missing
    for ith in range(1, 8):
        assert lib.al_fattn_f16_worker(ctypes.byref(a), ith, 8) == abi.AL_OK
    # a null argument block is never read by those workers either
    assert lib.al_fattn_f16_worker(None, 3, 4) == abi.AL_OK


@pytest.mark.parametrize("ith,nth", [(4, 4), (-1, 4), (0, 0), (1, 1)])
def test_worker_ids_out_of_range(ith, nth):
    lib = _lib_cpu()
    a = abi.AlFattnArgs()
    assert lib.al_fattn_f16_worker(ctypes.byref(a), ith, nth) == abi.AL_ERR_INVALID
    assert b"worker" in lib.al_last_error()


def test_node_hints_applied_only_with_the_tag():
    """al_fattn_apply_node_hints (include/arclight_fattn.h): op_params
    i32[4..6] = tag, kv_len, causal_pos0 set the implicit rule and drop the
    mask; without the tag (the reference's nodes: words 4.. are zero) the
    arguments are left as they are. Host logic only, no GPU."""
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    fn = lib.al_fattn_apply_node_hints
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.POINTER(abi.AlFattnArgs), ctypes.POINTER(ctypes.c_int32)]
    a = abi.AlFattnArgs()
    a.mask.data = ctypes.c_void_p(0x1000)
    a.kv_len, a.causal_pos0 = 0, -1
    plain = (ctypes.c_int32 * 16)()                    # a reference node: words 4.. zero
    assert fn(ctypes.byref(a), plain) == 0
    assert a.mask.data == 0x1000 and a.kv_len == 0 and a.causal_pos0 == -1
    hinted = (ctypes.c_int32 * 16)()
    hinted[4], hinted[5], hinted[6] = abi.AL_FATTN_HINT_TAG, 4097, 4096
    assert fn(ctypes.byref(a), hinted) == 1
    assert not a.mask.data and a.kv_len == 4097 and a.causal_pos0 == 4096
    b = abi.AlFattnArgs()
    b.mask.data = ctypes.c_void_p(0x2000)
    hinted[6] = -5                                     # not causal
    assert fn(ctypes.byref(b), hinted) == 1 and b.causal_pos0 == -1 and b.kv_len == 4097
    assert fn(None, hinted) == 0 and fn(ctypes.byref(b), None) == 0
