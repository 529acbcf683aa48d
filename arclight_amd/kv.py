"""Host-side mirror of ArcLight's KV cache for flash attention, over the C ABI
of include/arclight_kv.h.

KvCells restates llm_kv_cells / llm_kv_cache's slot bookkeeping
(nnml/include/cgraph.h:612-960, nnml/src/cgraph.cpp:1263-1590) in the
library; KvRing adds the per-layer f16 K/V tensors in HBM
(llm_kv_cache ctor, cgraph.cpp:915-986) with their attention views
(get_k / get_v, cgraph.cpp:1057-1112) and row writes (cpy_k / cpy_v,
cgraph.cpp:1114-1180).

A ubatch is a list of (pos, [seq ids]) per token; the first sequence id of a
token is its primary sequence (ubatch->seq_id[i][0]).
"""
import ctypes

import numpy as np

from . import abi
from ._lib import call, load

KQ_MASK_PAD = 64        # NNML_KQ_MASK_PAD


def _pad(x, n):
    return (x + n - 1) // n * n


class Ubatch:
    """Keeps the arrays an al_ubatch points at alive."""

    def __init__(self, tokens):
        self.n_tokens = len(tokens)
        self.pos = np.array([p for p, _ in tokens], dtype=np.int32)
        m = np.zeros(self.n_tokens, dtype=np.uint64)
        for i, (_, seqs) in enumerate(tokens):
            # the primary sequence is the lowest set bit
            if min(seqs) != seqs[0]:
                raise ValueError("the primary sequence must be the token's lowest sequence id")
            for s in seqs:
                m[i] |= np.uint64(1) << np.uint64(s)
        self.seq_mask = m
        self.c = abi.AlUbatch(self.n_tokens, self.pos.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                              self.seq_mask.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)))

    @property
    def ref(self):
        return ctypes.byref(self.c)


def _ub(tokens):
    return tokens if isinstance(tokens, Ubatch) else Ubatch(tokens)


class KvCells:
    """Cell bookkeeping of kv_size cells per stream (host only)."""

    def __init__(self, kv_size, n_seq_max=1, n_pad=256, unified=True, handle=None):
        self.kv_size = kv_size
        self.n_pad = n_pad
        self.n_stream = 1 if unified else n_seq_max
        self._owned = handle is None
        if handle is None:
            h = ctypes.c_void_p()
            call("al_kv_cells_create", kv_size, n_seq_max, n_pad, 1 if unified else 0, ctypes.byref(h))
            handle = h.value
        self.handle = handle

    def close(self):
        if self._owned and self.handle:
            call("al_kv_cells_destroy", self.handle)
        self.handle = None

    def __del__(self):
        try:
            if self._owned and self.handle:
                load().al_kv_cells_destroy(self.handle)
        except Exception:
            pass

    def clear(self):
        call("al_kv_cells_clear", self.handle)

    def place(self, tokens):
        """find_slot + apply_ubatch: returns (cache rows int64 [n_tokens], n_kv)."""
        return self.place_streams(tokens)[:2]

    def place_streams(self, tokens):
        """As place, plus the ubatch's streams s0..s0+ns-1: (rows, n_kv, s0, ns)."""
        ub = _ub(tokens)
        rows = np.empty(ub.n_tokens, dtype=np.int64)
        n_kv, s0, ns = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint32()
        call("al_kv_cells_place", self.handle, ub.ref, rows.ctypes.data, ctypes.byref(n_kv), ctypes.byref(s0),
             ctypes.byref(ns))
        return rows, n_kv.value, s0.value, ns.value

    def seq_rm(self, seq_id, p0, p1):
        call("al_kv_cells_seq_rm", self.handle, seq_id, p0, p1)

    def state(self):
        """(pos int32 [n_stream, kv_size], seq bit masks uint64 [n_stream, kv_size])."""
        pos = np.empty((self.n_stream, self.kv_size), dtype=np.int32)
        seq = np.empty((self.n_stream, self.kv_size), dtype=np.uint64)
        call("al_kv_cells_state", self.handle, pos.ctypes.data, seq.ctypes.data)
        return pos, seq

    def mask_host(self, tokens, n_kv, n_stream_ub=1):
        """f16 mask [n_stream_ub, 1, PAD(n_tokens / n_stream_ub, 64), n_kv]."""
        ub = _ub(tokens)
        rows = _pad(ub.n_tokens // n_stream_ub, KQ_MASK_PAD)
        m = np.empty((n_stream_ub, 1, rows, n_kv), dtype=np.float16)
        call("al_kv_cells_mask_host", self.handle, ub.ref, n_kv, n_stream_ub, m.ctypes.data)
        return m

    def mask_device(self, tokens, n_kv, mask, n_stream_ub=1, stream=None):
        """Builds the mask into the DeviceTensor `mask` ((n_stream_ub, 1, rows, n_kv) f16)."""
        ub = _ub(tokens)
        d = mask.desc()
        call("al_kv_cells_mask_device", self.handle, ub.ref, n_kv, n_stream_ub, ctypes.byref(d),
             stream.handle if stream is not None else None)
        return mask

    def implicit(self, tokens, n_kv):
        """(kv_len, causal_pos0) when the mask is the operator's implicit
        length + causal rule, else None."""
        ub = _ub(tokens)
        kv_len = ctypes.c_int64()
        pos0 = ctypes.c_int64()
        ok = load().al_kv_cells_implicit(self.handle, ub.ref, n_kv, ctypes.byref(kv_len), ctypes.byref(pos0))
        return (kv_len.value, pos0.value) if ok else None


class KvRing:
    """Per-layer f16 K/V in HBM plus their cell bookkeeping."""

    def __init__(self, n_layer, kv_size, n_head_kv, head_dim=128, n_seq_max=1, n_pad=256, unified=True):
        p = abi.AlKvRingParams(n_layer, kv_size, n_seq_max, n_pad, n_head_kv, head_dim, 1 if unified else 0)
        h = ctypes.c_void_p()
        call("al_kv_ring_create", ctypes.byref(p), ctypes.byref(h))
        self.handle = h.value
        self.params = p
        self.n_stream = 1 if unified else n_seq_max
        self.cells = KvCells(kv_size, n_seq_max, n_pad, unified, handle=load().al_kv_ring_cells(self.handle))

    def close(self):
        if self.handle:
            self.cells.handle = None
            call("al_kv_ring_destroy", self.handle)
            self.handle = None

    def __del__(self):
        try:
            if self.handle:
                load().al_kv_ring_destroy(self.handle)
        except Exception:
            pass

    def _view(self, fn, il, n_kv, s0, ns):
        t = abi.AlTensor()
        call(fn, self.handle, il, n_kv, s0, self.n_stream - s0 if ns is None else ns, ctypes.byref(t))
        return _RawView(t)

    def get_k(self, il, n_kv, s0=0, ns=None):
        """K of layer il over n_kv cells of streams s0..s0+ns-1 (default: all from s0)."""
        return self._view("al_kv_ring_view_k", il, n_kv, s0, ns)

    def get_v(self, il, n_kv, s0=0, ns=None):
        return self._view("al_kv_ring_view_v", il, n_kv, s0, ns)

    def cache_rows(self, il, which="k"):
        """Layer il's whole K or V cache as rows of one cell (all kv heads):
        f16 ne = [n_head_kv*head_dim, kv_size*n_stream], the destination
        the cpy_k / cpy_v set_rows write (cgraph.cpp:1114-1180)."""
        full = self.get_k(il, self.params.kv_size) if which == "k" else self.get_v(il, self.params.kv_size)
        t = abi.AlTensor()
        t.data = full.ptr
        t.type = abi.AL_TYPE_F16
        nc = self.params.n_head_kv * self.params.head_dim
        rows = self.params.kv_size * self.n_stream
        for i, (ne, nb) in enumerate(((nc, 2), (rows, nc * 2), (1, nc * 2 * rows), (1, nc * 2 * rows))):
            t.ne[i] = ne
            t.nb[i] = nb
        return _RawView(t)

    def cpy_kv(self, il, k_cur, v_cur, rows, stream=None):
        """Writes f32 rows [n_tokens, n_head_kv*head_dim] (DeviceTensors) at
        cache rows `rows` (DeviceTensor int64 [n_tokens])."""
        k, v, r = k_cur.desc(), v_cur.desc(), rows.desc()
        call("al_kv_ring_write", self.handle, il, ctypes.byref(k), ctypes.byref(v), ctypes.byref(r),
             stream.handle if stream is not None else None)


class _RawView:
    """An al_tensor the library filled in (a view of ring memory)."""

    def __init__(self, t):
        self.t = t
        self.ptr = t.data
        self.type = t.type
        # numpy order (B, n_kv, Hkv, D), as DeviceTensor views of K/V
        self.shape = (t.ne[3], t.ne[1], t.ne[2], t.ne[0])

    def desc(self):
        return self.t
