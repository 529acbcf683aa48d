#!/usr/bin/env python3
"""Benchmark of the flash-attention op on one MI355X.

Step = the decode attention of one token through all 36 layers of a
Qwen3-4B-shaped model (32 query heads, 8 KV heads, head_dim 128) at 32K
context: 36 al_fattn_f16 calls back to back on one stream, each layer with
its own f16 cache slice (128 MiB per layer, 4.5 GiB in all, so every layer
is read cold from HBM), replayed as one captured HIP graph.

    python bench.py [--steps K] [--warmup W] [--ctx 32768]

Prints one JSON line. `value` is the KV read bandwidth of the whole step:
algorithmic bytes (K+V of the visible cells, + Q + O) / step time. Extra
fields report 2048-token chunked causal prefill TFLOP/s (4 chunks of 512 over
36 layers), the roofline of the decode kernel from per-launch HIP events,
the other workloads of the family (decode at 4K / 16K, speculative verify
with 4 / 8 drafts at 8K, Qwen3-32B-shape decode at 32K and prefill of 4096
tokens in 1024-token chunks) and the CPU baseline (the f32 restatement of the
reference kernel on host cores).
"""
import argparse
import ctypes
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
F16_PEAK_TFLOPS = 2500.0       # MI355X dense f16 MFMA, TFLOP/s
DECODE_KERNEL = "fattn_decode_kernel<2, 3, 0, 1, -1, false>"   # the launch decode at q_len 1 takes


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--ctx", type=int, default=32768)
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip the 4K/16K decode, 8K verify and Qwen3-32B-shape lines")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="target CPU-baseline sample time")
    ap.add_argument("--only", choices=["decode", "decode_mask", "prefill", "wo", "copy", "step"], default=None,
                    help="run one workload only (for profiling); prints its own JSON line")
    return ap.parse_args()


class Layers:
    """Per-layer device operands of one attention call shape."""

    def __init__(self, L, T, Hq, Hkv, D, n_kv, seed):
        from arclight_amd import abi, device
        self.L, self.T, self.Hq, self.Hkv, self.D, self.n_kv = L, T, Hq, Hkv, D, n_kv
        from arclight_amd._lib import call
        self.q, self.k, self.v, self.dst = [], [], [], []
        for l in range(L):
            q = device.DeviceTensor.empty((1, T, Hq, D), np.float32, axes=abi.Q_AXES)
            k = device.DeviceTensor.empty((1, n_kv, Hkv, D), np.uint16, axes=abi.KV_AXES)
            v = device.DeviceTensor.empty((1, n_kv, Hkv, D), np.uint16, axes=abi.KV_AXES)
            d = device.DeviceTensor.empty((1, T, Hq, D), np.float32, axes=abi.DST_AXES)
            call("al_util_fill_randn_f32", q.ptr, T * Hq * D, seed, 3 * l, None)
            call("al_util_fill_randn_f16", k.ptr, n_kv * Hkv * D, seed, (3 * l + 1) << 40, None)
            call("al_util_fill_randn_f16", v.ptr, n_kv * Hkv * D, seed, (3 * l + 2) << 40, None)
            self.q.append(q); self.k.append(k); self.v.append(v); self.dst.append(d)
        device.synchronize()

    def args(self, l, stream, scale, kv_len, causal_pos0=-1, q=None, dst=None, mask=None):
        from arclight_amd import fattn
        return fattn.fattn_args(q or self.q[l], self.k[l], self.v[l], mask, None, dst or self.dst[l],
                                scale=scale, kv_len=kv_len, causal_pos0=causal_pos0, stream=stream)


def run_calls(lib, arg_list):
    f = lib.al_fattn_f16
    for a in arg_list:
        rc = f(ctypes.byref(a))
        if rc != 0:
            raise RuntimeError(lib.al_last_error().decode())


def time_graph(lib, stream, arg_list, steps, warmup, enqueue=None):
    """Captures one step (the attention calls of arg_list, or enqueue())
    into a HIP graph and replays it; returns ms per step."""
    from arclight_amd import device
    from arclight_amd._lib import call
    enqueue = enqueue or (lambda: run_calls(lib, arg_list))
    enqueue()                                     # allocates workspaces outside the capture
    stream.synchronize()
    call("al_util_graph_begin", stream.handle)
    enqueue()
    ge = ctypes.c_void_p()
    call("al_util_graph_end", stream.handle, ctypes.byref(ge))
    for _ in range(warmup):
        call("al_util_graph_launch", ge.value, stream.handle)
    stream.synchronize()
    e0, e1 = device.Event(), device.Event()
    device.synchronize()
    e0.record(stream)
    for _ in range(steps):
        call("al_util_graph_launch", ge.value, stream.handle)
    e1.record(stream)
    e1.synchronize()
    device.synchronize()
    ms = e0.elapsed_ms(e1) / steps
    call("al_util_graph_destroy", ge.value)
    return ms


def causal_mask_f16(T, n_kv, pos0, kv_len):
    """The f16 0 / -inf mask nnml builds for one sequence whose token t sits
    at position pos0 + t over cells holding positions 0 .. kv_len - 1
    (set_inputs_attn_mask, cgraph.cpp:1224-1261): PAD(T, 64) rows."""
    rows = (T + 63) // 64 * 64
    m = np.full((1, 1, rows, n_kv), -np.inf, dtype=np.float16)
    c = np.arange(n_kv)
    for t in range(T):
        m[0, 0, t, (c < kv_len) & (c <= pos0 + t)] = 0.0
    return m


def decode_bytes(ctx, Hq, Hkv, D, T=1):
    return 2 * ctx * Hkv * D * 2 + 2 * T * Hq * D * 4


def prefill_flops(T_total, chunk, Hq, D):
    pairs = 0
    for c in range(T_total // chunk):
        pairs += chunk * chunk * c + chunk * (chunk + 1) // 2
    return 4 * D * Hq * pairs


def bench_decode(lib, stream, a, ctx=None, L=None, Hq=32, T=1, steps=None, explicit_mask=False):
    """Decode (T = 1) or speculative verify (T drafts at positions ctx..ctx+T-1,
    causal among them) over L layers, each with its own cache slice of
    PAD(ctx + T, 256) cells. explicit_mask: the f16 0 / -inf mask tensor
    (PAD(T, 64) rows, as set_inputs_attn_mask builds it) instead of the
    implicit length / causal description, i.e. the call as nnml makes it."""
    Hkv, D = 8, 128
    ctx = ctx or a.ctx
    L = L or a.layers
    scale = 1.0 / math.sqrt(D)
    n_kv = (ctx + T + 255) // 256 * 256 if T > 1 else ctx
    lay = Layers(L, T, Hq, Hkv, D, n_kv, a.seed)
    if explicit_mask:
        from arclight_amd import fattn
        m = fattn.upload_mask(causal_mask_f16(T, n_kv, ctx if T > 1 else ctx - 1, ctx + (T if T > 1 else 0)))
        args = [lay.args(l, stream, scale, kv_len=0, mask=m) for l in range(L)]
        byts = decode_bytes(ctx + (T if T > 1 else 0), Hq, Hkv, D, T)
    elif T == 1:
        args = [lay.args(l, stream, scale, kv_len=ctx) for l in range(L)]
        byts = decode_bytes(ctx, Hq, Hkv, D)
    else:
        args = [lay.args(l, stream, scale, kv_len=ctx + T, causal_pos0=ctx) for l in range(L)]
        byts = 2 * (ctx + T) * Hkv * D * 2 + 2 * T * Hq * D * 4
    ms = time_graph(lib, stream, args, steps or a.steps, a.warmup)
    # the timed region is L back-to-back launches of the decode kernel on this
    # stream, so its average launch duration is ms / L
    return {
        "ms_per_step": ms,
        "bytes_per_layer": byts,
        "gbs": byts * L / (ms * 1e-3) / 1e9,
        "kernel_ms_mean": ms / L,
    }


def bench_prefill(lib, stream, a, T_total=2048, chunk=512, Hq=32, L=None, explicit_mask=False):
    """Causal chunked prefill: chunk c of every layer attends cells
    [0, chunk (c + 1)), causal within the chunk; chunks run in order, all
    layers of a chunk before the next chunk, as the model does.
    explicit_mask: each chunk's f16 0 / -inf mask over the T_total cells
    (PAD(chunk, 64) rows, as set_inputs_attn_mask builds it) and no length
    hints, i.e. the call as nnml makes it."""
    Hkv, D = 8, 128
    L = L or a.layers
    scale = 1.0 / math.sqrt(D)
    lay = Layers(L, T_total, Hq, Hkv, D, T_total, a.seed + 1)
    from arclight_amd import abi, device, fattn
    masks = [fattn.upload_mask(causal_mask_f16(chunk, T_total, chunk * c, chunk * (c + 1)))
             for c in range(T_total // chunk)] if explicit_mask else None
    args = []
    for c in range(T_total // chunk):
        for l in range(L):
            q = lay.q[l]
            qv = device.DeviceTensor(q.buf, abi.AL_TYPE_F32, (1, chunk, Hq, D), None,
                                     c * chunk * Hq * D * 4, abi.Q_AXES)
            dv = device.DeviceTensor(lay.dst[l].buf, abi.AL_TYPE_F32, (1, chunk, Hq, D), None,
                                     c * chunk * Hq * D * 4, abi.DST_AXES)
            if explicit_mask:
                args.append(lay.args(l, stream, scale, kv_len=0, causal_pos0=-1, q=qv, dst=dv, mask=masks[c]))
            else:
                args.append(lay.args(l, stream, scale, kv_len=chunk * (c + 1), causal_pos0=chunk * c, q=qv, dst=dv))
    ms = time_graph(lib, stream, args, max(1, a.steps // 2), max(1, a.warmup))
    fl = prefill_flops(T_total, chunk, Hq, D)
    return {"ms_per_step": ms, "flops_per_layer": fl, "tflops": fl * L / (ms * 1e-3) / 1e12,
            "kernel_ms_mean": ms / len(args)}


def bench_launch_floor(lib, stream, a, n=144, grid=256, block=512, lds=160 * 1024):
    """n launches of an empty kernel with the 512-token prefill chunk's launch
    shape (grid workgroups of block threads holding lds bytes of LDS), replayed
    as one graph: the dispatch cost per launch that every prefill call pays,
    and, under a tracer, the tracer's own per-dispatch overhead."""
    from arclight_amd._lib import call

    def enqueue():
        for _ in range(n):
            call("al_util_empty_launch", grid, block, lds, stream.handle)

    ms = time_graph(lib, stream, None, a.steps, a.warmup, enqueue=enqueue)
    return {"launches": n, "grid": grid, "block": block, "lds_bytes": lds, "us_per_launch": ms * 1e3 / n}


def bench_other_configs(lib, stream, a):
    """The remaining workloads of the metric's family, one line each: decode
    at 4K and 16K, speculative verify at 8K context with 4 and 8 drafts
    (Qwen3-8B attention shape = Qwen3-4B's), the 2048-token prefill in
    256-token ubatches and in 512-token chunks with the explicit mask, and
    the Qwen3-32B shape (64 query heads, 64 layers) for decode at 32K and
    4096-token prefill in 1024-token chunks; then the attention output projection (Q4_0 WO) that
    consumes the attention output, for decode and an 8-token verify; last,
    the whole attention block of a decode token (producers, K/V write,
    attention, WO) per layer, replayed as one graph."""
    out = []
    steps = max(2, a.steps // 2)

    def dec(name, **kw):
        r = bench_decode(lib, stream, a, steps=steps, **kw)
        out.append({"workload": name, "value": round(r["gbs"], 1), "unit": "GB/s",
                    "hbm_peak_frac": round(r["gbs"] / HBM_PEAK_GBS, 4),
                    "us_per_layer": round(r["kernel_ms_mean"] * 1e3, 2)})
        print(f"[bench] {out[-1]}", file=sys.stderr, flush=True)

    dec("decode, Qwen3-4B shape, context 32768, 36 layers, explicit f16 mask (the call as nnml makes it, "
        "no length hints)", ctx=32768, L=36, explicit_mask=True)
    dec("decode, Qwen3-4B shape, context 4096, 36 layers", ctx=4096, L=36)
    dec("decode, Qwen3-4B shape, context 16384, 36 layers", ctx=16384, L=36)
    dec("verify 4 drafts, Qwen3-8B shape, context 8192, 36 layers", ctx=8192, L=36, T=4)
    dec("verify 8 drafts, Qwen3-8B shape, context 8192, 36 layers", ctx=8192, L=36, T=8)
    dec("decode, Qwen3-32B shape (Hq 64), context 32768, 64 layers", ctx=32768, L=64, Hq=64)
    for name, kw in [("prefill 2048 tokens in 8 causal ubatches of 256 (ArcLight's default ubatch), Qwen3-4B shape, "
                      "36 layers", dict(chunk=256)),
                     ("prefill 2048 tokens in 4 causal chunks of 512, explicit f16 mask and no length hints (the "
                      "call as nnml makes it: the prefill kernel reads the mask), Qwen3-4B shape, 36 layers",
                      dict(chunk=512, explicit_mask=True))]:
        r = bench_prefill(lib, stream, a, **kw)
        out.append({"workload": name, "value": round(r["tflops"], 2), "unit": "TFLOP/s",
                    "mfma_peak_frac": round(r["tflops"] / F16_PEAK_TFLOPS, 4),
                    "us_per_call": round(r["kernel_ms_mean"] * 1e3, 2)})
        print(f"[bench] {out[-1]}", file=sys.stderr, flush=True)
    r = bench_prefill(lib, stream, a, T_total=4096, chunk=1024, Hq=64, L=64)
    out.append({"workload": "prefill 4096 tokens in 4 causal chunks of 1024, Qwen3-32B shape (Hq 64), 64 layers",
                "value": round(r["tflops"], 2), "unit": "TFLOP/s",
                "mfma_peak_frac": round(r["tflops"] / F16_PEAK_TFLOPS, 4),
                "us_per_call": round(r["kernel_ms_mean"] * 1e3, 2)})
    print(f"[bench] {out[-1]}", file=sys.stderr, flush=True)
    for name, K, N, T in [("WO projection Q4_0, Qwen3-4B shape (4096 -> 2560), 1 token", 4096, 2560, 1),
                          ("WO projection Q4_0, Qwen3-4B shape (4096 -> 2560), 8 tokens", 4096, 2560, 8),
                          ("WO projection Q4_0, Qwen3-32B shape (8192 -> 5120), 1 token", 8192, 5120, 1)]:
        r = bench_wo(lib, stream, a, K=K, N=N, T=T, copies=64 if K == 4096 else 16, steps=steps)
        out.append({"workload": name, "value": round(r["gbs"], 1), "unit": "GB/s",
                    "hbm_peak_frac": round(r["gbs"] / HBM_PEAK_GBS, 4),
                    "us_per_op": round(r["op_ms_mean"] * 1e3, 2)})
        print(f"[bench] {out[-1]}", file=sys.stderr, flush=True)
    ms = bench_decode_step(lib, stream, a, ctx=32768, L=36, steps=steps)
    ms1 = bench_decode_step(lib, stream, a, ctx=32768, L=36, steps=steps, inputs="one_launch")
    out.append({"workload": "decode attention block per token (Q/K RMSNorm + rope and the K/V write into the HBM "
                            "ring folded into the attention launch, attention at the run-time length, Q4_0 WO), "
                            "Qwen3-4B shape, context 32768, 36 layers, one replayed HIP graph",
                "value": round(ms * 1e3 / 36, 2), "unit": "us/layer", "higher_is_better": False,
                "tokens_per_s_attention_blocks": round(1e3 / ms, 1),
                "us_per_layer_inputs_as_own_launch": round(ms1 * 1e3 / 36, 2)})
    print(f"[bench] {out[-1]}", file=sys.stderr, flush=True)
    return out


def wo_bytes(K, N, T):
    """Algorithmic bytes of one WO projection: the Q4_0 weights (18 bytes
    per 32), the f32 activations read and the f32 outputs written."""
    return N * K // 32 * 18 + T * K * 4 + T * N * 4


def bench_wo(lib, stream, a, K=4096, N=2560, T=1, copies=64, steps=None):
    """The attention output projection with Q4_0 weights: each step runs it
    once on each of `copies` distinct weight matrices (together larger than
    the 256 MB last-level cache, so every launch streams its weights from
    HBM), as L layers would."""
    from arclight_amd import device, matmul
    rng = np.random.default_rng(a.seed + 7)
    nb = K // 32
    blocks = np.empty((N, nb, 18), np.uint8)
    blocks[:] = rng.integers(0, 256, size=(N, nb, 18), dtype=np.uint8)
    blocks[:, :, :2] = np.frombuffer(np.float16(0.01).tobytes(), np.uint8)
    ws = [matmul.Q4_0Matrix(blocks, K, N) for _ in range(copies)]
    x = device.DeviceTensor.from_numpy(rng.standard_normal((T, K)).astype(np.float32))
    y = device.DeviceTensor.empty((T, N), np.float32)

    def enqueue():
        for w in ws:
            matmul.mul_mat_q4_0(w, x, y, stream)

    ms = time_graph(lib, stream, None, steps or a.steps, a.warmup, enqueue)
    byts = wo_bytes(K, N, T)
    return {"ms_per_step": ms, "bytes_per_launch": byts, "gbs": byts * copies / (ms * 1e-3) / 1e9,
            "op_ms_mean": ms / copies}


def bench_decode_step(lib, stream, a, ctx=32768, L=36, steps=None, inputs="fused"):
    """One decode token through the attention block of every layer as the
    Qwen3 graph runs it (qwen3.cpp:215-227, cgraph.cpp:485-500), captured
    once as a HIP graph and replayed: Q and K RMSNorm + NEOX rope (K written
    into the HBM ring at the token's cell), V written by set_rows, attention
    over the ring's views at the run-time length {ctx + 1, ctx}, and the Q4_0
    WO projection of the attention output. inputs: "fused" folds the three
    producers into the attention launch (al_fattn_f16_with_inputs),
    "one_launch" runs them as one launch before it (al_attn_inputs_f32),
    "separate" as the three separate ops. Returns ms per step (L layers)."""
    from arclight_amd import abi, device, fattn, kv, matmul, prologue
    from arclight_amd._lib import call
    Hq, Hkv, D, N = 32, 8, 128, 2560
    K = Hq * D
    kv_size = (ctx + 1 + 255) // 256 * 256
    rng = np.random.default_rng(a.seed + 11)
    rope = abi.qwen3_rope()
    ring = kv.KvRing(L, kv_size, Hkv, D, 1, 256, True)
    try:
        for il in range(L):
            for j, which in enumerate("kv"):
                call("al_util_fill_randn_f16", ring.cache_rows(il, which).ptr, kv_size * Hkv * D, a.seed,
                     (2 * il + j + 7) << 40, None)
        nb = K // 32
        blocks = np.empty((N, nb, 18), np.uint8)
        blocks[:] = rng.integers(0, 256, size=(N, nb, 18), dtype=np.uint8)
        blocks[:, :, :2] = np.frombuffer(np.float16(0.01).tobytes(), np.uint8)
        wo = [matmul.Q4_0Matrix(blocks, K, N) for _ in range(L)]
        wq = [device.DeviceTensor.from_numpy(rng.standard_normal(D).astype(np.float32)) for _ in range(L)]
        wk = [device.DeviceTensor.from_numpy(rng.standard_normal(D).astype(np.float32)) for _ in range(L)]
        qc = device.DeviceTensor.from_numpy(rng.standard_normal((1, Hq, D)).astype(np.float32))
        kc = device.DeviceTensor.from_numpy(rng.standard_normal((1, Hkv, D)).astype(np.float32))
        vc = device.DeviceTensor.from_numpy(rng.standard_normal((1, Hkv * D)).astype(np.float32))
        pos = device.DeviceTensor.from_numpy(np.array([ctx], np.int32))
        row = device.DeviceTensor.from_numpy(np.array([ctx], np.int64))
        dyn = device.DeviceTensor.from_numpy(np.array([ctx + 1, ctx], np.int32))
        qs = [device.DeviceTensor.empty((1, Hq, D), np.float32) for _ in range(L)]
        att = [device.DeviceTensor.empty((1, 1, Hq, D), np.float32, axes=abi.DST_AXES) for _ in range(L)]
        ys = [device.DeviceTensor.empty((1, N), np.float32) for _ in range(L)]
        device.synchronize()

        def enqueue():
            for il in range(L):
                if inputs == "fused":
                    prologue.attention_with_inputs(qc, wq[il], kc, wk[il], vc, pos, row, qs[il], ring.cache_rows(il, "k"),
                                                   ring.cache_rows(il, "v"), ring.get_k(il, kv_size),
                                                   ring.get_v(il, kv_size), att[il], eps=1e-6, scale=1.0 / math.sqrt(D),
                                                   rope=rope, kv_len=kv_size, causal_pos0=0, dyn_len=dyn, stream=stream)
                    matmul.mul_mat_q4_0(wo[il], device.DeviceTensor(att[il].buf, abi.AL_TYPE_F32, (1, K)), ys[il], stream)
                    continue
                if inputs == "one_launch":
                    prologue.attn_inputs(qc, wq[il], kc, wk[il], vc, pos, row, qs[il], ring.cache_rows(il, "k"),
                                         ring.cache_rows(il, "v"), eps=1e-6, rope=rope, stream=stream)
                else:
                    prologue.rms_norm_rope(qc, wq[il], pos, eps=1e-6, rope=rope, y=qs[il], stream=stream)
                    prologue.rms_norm_rope(kc, wk[il], pos, eps=1e-6, rope=rope, y=ring.cache_rows(il, "k"), rows=row,
                                           stream=stream)
                    fattn.set_rows(ring.cache_rows(il, "v"), vc, row, stream=stream)
                qv = device.DeviceTensor(qs[il].buf, abi.AL_TYPE_F32, (1, 1, Hq, D), None, 0, abi.Q_AXES)
                fattn.flash_attn_ext(qv, ring.get_k(il, kv_size), ring.get_v(il, kv_size), scale=1.0 / math.sqrt(D),
                                     dst=att[il], kv_len=kv_size, causal_pos0=0, stream=stream, dyn_len=dyn)
                matmul.mul_mat_q4_0(wo[il], device.DeviceTensor(att[il].buf, abi.AL_TYPE_F32, (1, K)), ys[il], stream)

        ms = time_graph(lib, stream, None, steps or a.steps, a.warmup, enqueue)
    finally:
        device.synchronize()
        ring.close()
    return ms


def bench_copy(stream, nbytes=1 << 30):
    """Plain device copy of known size (calibrates rocprof byte counters)."""
    from arclight_amd import device
    from arclight_amd._lib import call
    a_, b_ = device.DeviceBuffer(nbytes), device.DeviceBuffer(nbytes)
    call("al_util_memset", a_.ptr, 1, nbytes)
    e0, e1 = device.Event(), device.Event()
    for _ in range(2):
        call("al_util_copy_kernel", b_.ptr, a_.ptr, nbytes, stream.handle)
    e0.record(stream)
    reps = 10
    for _ in range(reps):
        call("al_util_copy_kernel", b_.ptr, a_.ptr, nbytes, stream.handle)
    e1.record(stream)
    e1.synchronize()
    ms = e0.elapsed_ms(e1) / reps
    return {"bytes": nbytes, "ms": ms, "gbs": 2 * nbytes / (ms * 1e-3) / 1e9}


def cpu_baseline(a):
    """Oracle O2 (f32 restatement of arm.cpp:2196-2433) on the host's cores:
    one worker thread pinned to each physical core of the job's CPU share,
    rows split over the workers as arm.cpp:2250-2257 does. Two bounded
    samples of the benchmark's own workloads: 32K decode at the Qwen3-4B shape
    (single-layer calls, GB/s) and the 2048-token prefill in 4 causal chunks
    of 512 (one layer per repetition, TFLOP/s)."""
    from oracle import oracle as O
    topo = O.cpu_topology()
    cpus = topo["cpus"]
    Hq, Hkv, D, ctx = 32, 8, 128, a.ctx
    scale = 1.0 / math.sqrt(D)

    n_layers = 2
    data = [O.make_inputs(a.seed + l, T=1, Hq=Hq, Hkv=Hkv, D=D, n_kv=ctx) for l in range(n_layers)]
    O.attention_pinned(*data[0], scale=scale, kv_len=ctx, cpus=cpus)     # warm
    t0 = time.perf_counter()
    calls = 0
    while True:
        for q, k, v in data:
            O.attention_pinned(q, k, v, scale=scale, kv_len=ctx, cpus=cpus)
            calls += 1
        el = time.perf_counter() - t0
        if el >= a.cpu_seconds or calls >= 4000:
            break
    per = el / calls
    byts = decode_bytes(ctx, Hq, Hkv, D)

    T_total, chunk = 2048, 512
    q, k, v = O.make_inputs(a.seed + 1, T=T_total, Hq=Hq, Hkv=Hkv, D=D, n_kv=T_total)
    chunks = [np.ascontiguousarray(q[:, c * chunk:(c + 1) * chunk]) for c in range(T_total // chunk)]
    t0 = time.perf_counter()
    reps = 0
    while True:
        for c, qc in enumerate(chunks):
            O.attention_pinned(qc, k, v, scale=scale, kv_len=chunk * (c + 1), causal_pos0=chunk * c, cpus=cpus)
        reps += 1
        pel = time.perf_counter() - t0
        if pel >= a.cpu_seconds or reps >= 200:
            break
    fl = prefill_flops(T_total, chunk, Hq, D)
    where = (f"{len(cpus)} threads pinned one per physical core; host {topo['model']}, "
             f"{topo['host_physical_cores']} physical cores, job share {topo['job_share']} CPUs "
             f"(affinity {topo['allowed_cpus']}, cgroup quota {topo['cpu_quota']})")
    return {"value": byts / per / 1e9, "unit": "GB/s", "cores": len(cpus), "kind": "port",
            "sample": f"decode ctx {ctx}, {calls} single-layer calls over {n_layers} distinct layers, "
                      f"{el:.1f} s, {per * 1e3:.1f} ms/layer; {where}",
            "cpu_model": topo["model"], "host_physical_cores": topo["host_physical_cores"], "pinned": True,
            "prefill": {"value": fl * reps / pel / 1e12, "unit": "TFLOP/s",
                        "sample": f"2048-token causal prefill in 4 chunks of 512, one layer per repetition, "
                                  f"{reps} repetitions, {pel:.1f} s, {pel / reps * 1e3:.0f} ms/layer"}}


def load_traffic(kernel, ctx):
    """HBM bytes per decode launch from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE runs (scaled by the copy-kernel calibration), if they were
    taken for this kernel and context; else None."""
    p = os.path.join(ROOT, "profiles", "decode_traffic.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        t = json.load(f)
    if t.get("kernel") != kernel or t.get("ctx") != ctx:
        return None
    return t.get("bytes_per_launch")


def main():
    a = parse()
    if a.gpus != 1:
        print(json.dumps({"error": "bench.py runs on one GPU only; --gpus must be 1 "
                          "(attention would shard by KV head across GPUs, with no exchange before "
                          "the output projection)"}))
        sys.exit(2)
    from arclight_amd import _lib, device
    lib = _lib.load()
    info = device.device_info()
    stream = device.Stream()
    print(f"[bench] {info}", file=sys.stderr, flush=True)

    if a.only == "copy":
        print(json.dumps({"copy": bench_copy(stream)}))
        return
    if a.only == "prefill":
        print(json.dumps({"prefill": bench_prefill(lib, stream, a),
                          "prefill_explicit_mask": bench_prefill(lib, stream, a, explicit_mask=True),
                          "launch_floor": bench_launch_floor(lib, stream, a)}))
        return
    if a.only == "step":
        out = {}
        for inputs in ("fused", "one_launch", "separate"):
            ms = bench_decode_step(lib, stream, a, ctx=a.ctx, L=a.layers, inputs=inputs)
            out[f"{inputs}_inputs"] = {"ms_per_step": ms, "us_per_layer": ms * 1e3 / a.layers}
        print(json.dumps({"step": out}))
        return
    if a.only == "wo":
        print(json.dumps({"wo": [bench_wo(lib, stream, a, K=K, N=N, T=T, copies=c)
                                 for K, N, T, c in [(4096, 2560, 1, 64), (4096, 2560, 8, 64), (8192, 5120, 1, 16)]]}))
        return

    if a.only == "decode_mask":
        print(json.dumps({"decode_explicit_mask": bench_decode(lib, stream, a, explicit_mask=True)}))
        return
    dec = bench_decode(lib, stream, a)
    print(f"[bench] decode {dec}", file=sys.stderr, flush=True)
    if a.only == "decode":
        print(json.dumps({"decode": dec}))
        return
    pre = None if a.no_prefill else bench_prefill(lib, stream, a)
    if pre:
        print(f"[bench] prefill {pre}", file=sys.stderr, flush=True)
    others = None if a.no_other_configs else bench_other_configs(lib, stream, a)
    cpu = None if a.no_cpu_baseline else cpu_baseline(a)
    if cpu:
        print(f"[bench] cpu {cpu}", file=sys.stderr, flush=True)

    achieved = dec["bytes_per_layer"] / (dec["kernel_ms_mean"] * 1e-3) / 1e9
    traffic = load_traffic(DECODE_KERNEL, a.ctx)
    out = {
        "metric": "decode-attn KV GB/s (% HBM peak) + prefill-attn TFLOP/s, Qwen3-4B shape",
        "value": round(dec["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(dec["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 K/V, f32 Q/O, f32 accumulation",
        "data": "synthetic, seeded N(0,1)",
        "config": {"workload": f"decode attention, Qwen3-4B shape (Hq 32, Hkv 8, D 128), batch 1, q_len 1, "
                               f"context {a.ctx}, {a.layers} layers back to back, one cache slice per layer",
                   "parallelism": "single GPU"},
        "hbm_peak_frac": round(dec["gbs"] / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic,
                     "kernel": DECODE_KERNEL,
                     "kernel_us_mean": round(dec["kernel_ms_mean"] * 1e3, 2),
                     "algorithmic_bytes_per_launch": dec["bytes_per_layer"]},
        "prefill": None if not pre else {
            "workload": "2048-token causal prefill in 4 chunks of 512, 36 layers, Qwen3-4B shape",
            "tflops": round(pre["tflops"], 2),
            "mfma_peak_frac": round(pre["tflops"] / F16_PEAK_TFLOPS, 4),
            "ms_per_step": round(pre["ms_per_step"], 4)},
        "other_configs": others,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
