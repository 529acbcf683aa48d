"""Python binding of the CPU oracle (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, as the reference results or as the timed CPU baseline. The product package
(arclight_amd) never imports it.

Arrays use the physical layouts documented in arclight_amd.abi:
q (B, T, Hq, D) f32; k, v (B, n_kv, Hkv, D) f16; mask (m3, m2, rows, n_kv)
f16; sinks (Hq,) f32; the result is (B, T, Hq, D) f32.
"""
import ctypes
import os
import subprocess

import numpy as np

from arclight_amd import abi

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liborc_fattn.so")

_lib = None


def build():
    """Compiles the oracle library with its Makefile."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library not built: {LIB_PATH} (run make -C oracle)")
        L = ctypes.CDLL(LIB_PATH)
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f32_to_f16_n.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        L.orc_f16_to_f32_n.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        for name in ("orc_fattn_o1", "orc_fattn_o2", "orc_fattn_o3"):
            f = getattr(L, name)
            f.restype = ctypes.c_int
            f.argtypes = [ctypes.POINTER(abi.AlFattnArgs), ctypes.c_int]
        L.orc_fattn_o2_pinned.restype = ctypes.c_int
        L.orc_fattn_o2_pinned.argtypes = [ctypes.POINTER(abi.AlFattnArgs), ctypes.c_int, ctypes.c_void_p]
        L.orc_set_rows_f32_f16.restype = ctypes.c_int
        L.orc_set_rows_f32_f16.argtypes = [ctypes.POINTER(abi.AlTensor)] * 3
        L.orc_rms_norm_rope_f32.restype = ctypes.c_int
        L.orc_rms_norm_rope_f32.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int64] * 3 + [
            ctypes.c_float, ctypes.POINTER(abi.AlRopeParams), ctypes.c_void_p]
        L.orc_quantize_row_q8_0.restype = None
        L.orc_quantize_row_q8_0.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        L.orc_vec_dot_q4_0_q8_0.restype = ctypes.c_float
        L.orc_vec_dot_q4_0_q8_0.argtypes = [ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
        L.orc_mul_mat_q4_0_f32.restype = ctypes.c_int
        L.orc_mul_mat_q4_0_f32.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
                                           ctypes.c_int64, ctypes.c_void_p]
        _lib = L
    return _lib


def f32_to_f16_bits(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_f16_n(x.ctypes.data, y.ctypes.data, x.size)
    return y


def f16_bits_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    y = np.empty(h.shape, dtype=np.float32)
    lib().orc_f16_to_f32_n(h.ctypes.data, y.ctypes.data, h.size)
    return y


def _bits(a):
    if a.dtype == np.float16:
        return a.view(np.uint16)
    if a.dtype != np.uint16:
        raise TypeError("f16 operand must be float16 or uint16 bits")
    return a


def default_threads():
    n = os.cpu_count() or 1
    return max(1, min(n, 16))


def _read(path):
    try:
        with open(path) as f:
            return f.read().strip()
    except OSError:
        return None


def cpu_topology():
    """The host CPUs this process may run on, one logical CPU per physical
    core: {"model", "host_physical_cores", "allowed_cpus", "cpu_quota",
    "job_share", "cpus"}. `cpus` lists one logical CPU of each physical core
    (socket, core id) in the affinity set, at most `job_share` of them: the
    CPU share the job is given (the cgroup CPU quota, or OMP_NUM_THREADS when
    the launcher sets it as the share), else every physical core."""
    allowed = sorted(os.sched_getaffinity(0))
    model = None
    txt = _read("/proc/cpuinfo") or ""
    for line in txt.splitlines():
        if line.startswith("model name"):
            model = line.split(":", 1)[1].strip()
            break
    cores, host_cores = {}, set()
    for c in range(os.cpu_count() or 0):
        base = f"/sys/devices/system/cpu/cpu{c}/topology/"
        pkg, core = _read(base + "physical_package_id"), _read(base + "core_id")
        key = (int(pkg) if pkg is not None else 0, int(core) if core is not None else c)
        host_cores.add(key)
        if c in allowed and key not in cores:
            cores[key] = c
    quota = None
    cm = _read("/sys/fs/cgroup/cpu.max")
    if cm and not cm.startswith("max"):
        q, per = cm.split()[:2]
        quota = int(q) / int(per)
    share = len(cores)
    if quota:
        share = min(share, max(1, int(quota)))
    omp = os.environ.get("OMP_NUM_THREADS")
    if omp and omp.isdigit() and int(omp) > 0:
        share = min(share, int(omp))
    cpus = [cores[k] for k in sorted(cores, key=lambda k: cores[k])][:share]
    return {"model": model, "host_physical_cores": len(host_cores), "allowed_cpus": len(allowed),
            "cpu_quota": quota, "job_share": share, "cpus": cpus}


def attention_pinned(q, k, v, mask=None, *, scale, cpus, kv_len=0, causal_pos0=-1):
    """O2 with one worker thread pinned to each logical CPU of `cpus` (the
    reference's row split over that many workers); returns dst."""
    k, v = _bits(k), _bits(v)
    if mask is not None:
        mask = _bits(mask)
    B, T, Hq, _ = q.shape
    dst = np.full((B, T, Hq, v.shape[3]), np.nan, dtype=np.float32)
    a = build_args(q, k, v, mask, None, dst, scale=scale, kv_len=kv_len, causal_pos0=causal_pos0)
    c = (ctypes.c_int * len(cpus))(*cpus)
    rc = lib().orc_fattn_o2_pinned(ctypes.byref(a), len(cpus), ctypes.cast(c, ctypes.c_void_p))
    if rc != 0:
        raise RuntimeError(f"oracle O2 failed: {rc}")
    return dst


def build_args(q, k, v, mask=None, sinks=None, dst=None, *, scale, max_bias=0.0,
               logit_softcap=0.0, kv_len=0, causal_pos0=-1, prec=abi.AL_PREC_F32):
    """al_fattn_args over host numpy arrays (kept alive by the caller)."""
    a = abi.AlFattnArgs()
    a.q = abi.tensor_desc(q.ctypes.data, abi.AL_TYPE_F32, q.shape, q.strides, abi.Q_AXES)
    a.k = abi.tensor_desc(k.ctypes.data, abi.AL_TYPE_F16, k.shape, k.strides, abi.KV_AXES)
    a.v = abi.tensor_desc(v.ctypes.data, abi.AL_TYPE_F16, v.shape, v.strides, abi.KV_AXES)
    a.mask = (abi.tensor_desc(mask.ctypes.data, abi.AL_TYPE_F16, mask.shape, mask.strides, abi.MASK_AXES)
              if mask is not None else abi.empty_tensor())
    a.sinks = (abi.make_tensor(sinks.ctypes.data, abi.AL_TYPE_F32, [sinks.shape[0]])
               if sinks is not None else abi.empty_tensor())
    a.dst = abi.tensor_desc(dst.ctypes.data, abi.AL_TYPE_F32, dst.shape, dst.strides, abi.DST_AXES)
    a.scale = scale
    a.max_bias = max_bias
    a.logit_softcap = logit_softcap
    a.prec = prec
    a.kv_len = kv_len
    a.causal_pos0 = causal_pos0
    return a


def attention(q, k, v, mask=None, sinks=None, *, scale, max_bias=0.0, logit_softcap=0.0,
              kv_len=0, causal_pos0=-1, mode="o2", threads=None, prec=abi.AL_PREC_F32):
    """Runs oracle O1 / O2 / O3 and returns dst as (B, T, Hq, D) f32."""
    assert q.dtype == np.float32 and q.ndim == 4
    k = _bits(k)
    v = _bits(v)
    if mask is not None:
        mask = _bits(mask)
    if sinks is not None:
        sinks = np.ascontiguousarray(sinks, dtype=np.float32)
    B, T, Hq, _ = q.shape
    D = v.shape[3]
    dst = np.full((B, T, Hq, D), np.nan, dtype=np.float32)
    a = build_args(q, k, v, mask, sinks, dst, scale=scale, max_bias=max_bias,
                   logit_softcap=logit_softcap, kv_len=kv_len, causal_pos0=causal_pos0, prec=prec)
    fn = {"o1": lib().orc_fattn_o1, "o2": lib().orc_fattn_o2, "o3": lib().orc_fattn_o3}[mode]
    rc = fn(ctypes.byref(a), threads or default_threads())
    if rc != 0:
        raise ValueError(f"oracle {mode} rejected the operands: {abi.STATUS_NAMES.get(rc, rc)}")
    return dst


def set_rows(cache, rows, idx):
    """Oracle of the KV write: cache (n_rows_dst, nc) f16 bits, rows (n, nc)
    f32, idx (n,) int64/int32. Returns a new cache array."""
    out = np.array(_bits(cache), copy=True)
    rows = np.ascontiguousarray(rows, dtype=np.float32)
    idx = np.ascontiguousarray(idx)
    it = abi.AL_TYPE_I64 if idx.dtype == np.int64 else abi.AL_TYPE_I32
    dst = abi.make_tensor(out.ctypes.data, abi.AL_TYPE_F16, [out.shape[1], out.shape[0]])
    src = abi.make_tensor(rows.ctypes.data, abi.AL_TYPE_F32, [rows.shape[1], rows.shape[0]])
    ix = abi.make_tensor(idx.ctypes.data, it, [idx.shape[0]])
    rc = lib().orc_set_rows_f32_f16(ctypes.byref(dst), ctypes.byref(src), ctypes.byref(ix))
    if rc != 0:
        raise ValueError(f"oracle set_rows rejected the operands: {abi.STATUS_NAMES.get(rc, rc)}")
    return out


# ---------------------------------------------------------------------------
# Seeded synthetic inputs and masks (host side).
# ---------------------------------------------------------------------------

def make_inputs(seed, *, B=1, T=1, Hq=32, Hkv=8, D=128, n_kv=512, kv_size=None):
    """q ~ N(0,1) f32 (B, T, Hq, D); k, v ~ N(0,1) rounded to f16 (RNE) in a
    cell-major cache of kv_size cells, returned as views of the first n_kv."""
    kv_size = kv_size or n_kv
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, T, Hq, D), dtype=np.float32)
    kc = rng.standard_normal((B, kv_size, Hkv, D), dtype=np.float32).astype(np.float16)
    vc = rng.standard_normal((B, kv_size, Hkv, D), dtype=np.float32).astype(np.float16)
    return q, kc[:, :n_kv], vc[:, :n_kv]


def causal_mask(T, n_kv, pos0, kv_len=None, n_stream=1):
    """f16 mask (n_stream, 1, PAD(T, 64), n_kv) of 0 / -inf, filled as
    set_inputs_attn_mask (nnml/src/cgraph.cpp:1224-1261) does for one
    contiguous sequence whose token t sits at position pos0 + t and whose
    cells hold positions 0..kv_len-1."""
    kv_len = n_kv if kv_len is None else kv_len
    rows = (T + 63) // 64 * 64
    m = np.full((n_stream, 1, rows, n_kv), -np.inf, dtype=np.float16)
    c = np.arange(n_kv)
    for t in range(T):
        vis = (c < kv_len) & (c <= pos0 + t)
        m[:, 0, t, vis] = 0.0
    return m


def rms_norm_rope(x, w=None, pos=None, *, eps=1e-6, rope=None):
    """Oracle of the Q/K producers: rope(rms_norm(x) * w) with x (T, H, D) f32,
    w (D,) or None, pos (T,) int32, rope an AlRopeParams or None."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, H, D = x.shape
    w = None if w is None else np.ascontiguousarray(w, dtype=np.float32)
    pos = np.zeros(T, np.int32) if pos is None else np.ascontiguousarray(pos, dtype=np.int32)
    y = np.empty_like(x)
    rc = lib().orc_rms_norm_rope_f32(x.ctypes.data, None if w is None else w.ctypes.data, pos.ctypes.data, T, H, D,
                                     eps, ctypes.byref(rope) if rope is not None else None, y.ctypes.data)
    if rc != 0:
        raise ValueError(f"oracle rms_norm_rope rejected the operands: {abi.STATUS_NAMES.get(rc, rc)}")
    return y


# Q4_0 / Q8_0 blocks as numpy records (nnml/include/nnml.h:646-650, 695-699).
Q4_0 = np.dtype([("d", "<u2"), ("qs", "u1", 16)])
Q8_0 = np.dtype([("d", "<u2"), ("qs", "i1", 32)])


def random_q4_0(rng, N, K, scale=0.02):
    """N rows of K / 32 Q4_0 blocks: uniform nibbles and f16 scales of both
    signs (quantize_row_q4_0_ref stores d = max / -8, types.cpp:352-377)."""
    w = np.empty((N, K // 32), dtype=Q4_0)
    w["qs"] = rng.integers(0, 256, size=(N, K // 32, 16), dtype=np.uint8)
    d = (rng.uniform(0.25, 1.0, size=(N, K // 32)) * scale * rng.choice([-1.0, 1.0], size=(N, K // 32)))
    w["d"] = d.astype(np.float16).view(np.uint16)
    return w


def quantize_q8_0(x):
    """quantize_row_q8_0 over each row of x (T, K) f32: (T, K / 32) Q8_0."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, K = x.shape
    y = np.empty((T, K // 32), dtype=Q8_0)
    for t in range(T):
        lib().orc_quantize_row_q8_0(x[t].ctypes.data, y[t].ctypes.data, K)
    return y


def vec_dot_q4_0_q8_0(wrow, qrow):
    """One Q4_0 row (K / 32 blocks) dotted with one Q8_0 row."""
    wrow = np.ascontiguousarray(wrow, dtype=Q4_0)
    qrow = np.ascontiguousarray(qrow, dtype=Q8_0)
    return float(lib().orc_vec_dot_q4_0_q8_0(32 * wrow.size, wrow.ctypes.data, qrow.ctypes.data))


def mul_mat_q4_0(w, x):
    """Oracle of the WO projection: w (N, K / 32) Q4_0, x (T, K) f32 ->
    y (T, N) f32, y[t, n] the dot product of row n with quantized row t."""
    w = np.ascontiguousarray(w, dtype=Q4_0)
    x = np.ascontiguousarray(x, dtype=np.float32)
    N, nb = w.shape
    T, K = x.shape
    if K != 32 * nb:
        raise ValueError(f"mul_mat_q4_0: w has {nb} blocks per row, x has {K} columns")
    y = np.empty((T, N), dtype=np.float32)
    rc = lib().orc_mul_mat_q4_0_f32(w.ctypes.data, K, N, x.ctypes.data, T, y.ctypes.data)
    if rc != 0:
        raise ValueError(f"oracle mul_mat_q4_0 rejected the operands: {abi.STATUS_NAMES.get(rc, rc)}")
    return y
