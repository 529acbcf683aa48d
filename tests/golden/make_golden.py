"""Writes tests/golden/fattn_golden.npz: known-answer vectors for the
flash-attention path (nnml/src/ops/arm/arm.cpp:2196-2433 semantics).

The reference holds no golden vectors for this operator, so the expected
outputs come from oracle O1 (float64 brute force, itself checked against
scipy's softmax attention in tests/test_oracle_attention.py). Inputs are
regenerated from their seed by oracle.make_inputs; the fixture stores a
SHA-256 of the regenerated q/k/v so that a change of the generator is
caught instead of silently comparing other data. Masks and sinks are stored
as they are (small).

    python tests/golden/make_golden.py
"""
import hashlib
import json
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402

OUT = os.path.join(HERE, "fattn_golden.npz")


def alibi_mask(T, n_kv, pos0):
    """Relative-position biases -(pos - cell) on visible cells, -inf after."""
    rows = (T + 63) // 64 * 64
    m = np.full((1, 1, rows, n_kv), -np.inf, dtype=np.float16)
    c = np.arange(n_kv)
    for t in range(T):
        vis = c <= pos0 + t
        m[0, 0, t, vis] = -(pos0 + t - c[vis])
    return m


def cases():
    s = 1.0 / math.sqrt(128)
    out = []

    def add(name, seed, shape, *, mask=None, sinks=None, **kw):
        out.append(dict(name=name, seed=seed, shape=shape, mask=mask, sinks=sinks, kw=dict(scale=s, **kw)))

    add("decode_qwen3_4b_shape", 101, dict(T=1, Hq=32, Hkv=8, n_kv=256), mask=O.causal_mask(1, 256, 200))
    add("verify_t4", 102, dict(T=4, Hq=32, Hkv=8, n_kv=192), mask=O.causal_mask(4, 192, 150))
    add("prefill_t64_implicit_causal", 103, dict(T=64, Hq=4, Hkv=1, n_kv=64), causal_pos0=0)
    add("chunk_t16_implicit_len", 104, dict(T=16, Hq=8, Hkv=2, n_kv=160), kv_len=150, causal_pos0=134)
    add("sinks_softcap", 105, dict(T=2, Hq=8, Hkv=2, n_kv=100), mask=O.causal_mask(2, 100, 90),
        sinks=np.linspace(-3, 3, 8).astype(np.float32), logit_softcap=30.0)
    add("alibi_12_heads", 106, dict(T=3, Hq=12, Hkv=4, n_kv=80), mask=alibi_mask(3, 80, 70), max_bias=8.0)
    m = O.causal_mask(2, 96, 60, n_stream=2)
    m[1, 0, 1, :] = -np.inf                                   # stream 1, token 1: nothing visible -> NaN
    add("two_streams_one_row_masked", 107, dict(B=2, T=2, Hq=8, Hkv=2, n_kv=96), mask=m)
    add("ragged_77_cells", 108, dict(T=1, Hq=16, Hkv=2, n_kv=77))
    add("gqa8_noncausal_t5", 109, dict(T=5, Hq=8, Hkv=1, n_kv=130))
    return out


def digest(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def inputs(c):
    return O.make_inputs(c["seed"], **c["shape"])


def main():
    blobs = {}
    meta = []
    for c in cases():
        q, k, v = inputs(c)
        want = O.attention(q, k, v, c["mask"], c["sinks"], mode="o1", **c["kw"])
        blobs[c["name"] + ".expected"] = want
        if c["mask"] is not None:
            blobs[c["name"] + ".mask"] = c["mask"]
        if c["sinks"] is not None:
            blobs[c["name"] + ".sinks"] = c["sinks"]
        meta.append(dict(name=c["name"], seed=c["seed"], shape=c["shape"], kw=c["kw"],
                         has_mask=c["mask"] is not None, has_sinks=c["sinks"] is not None,
                         qkv_sha256=digest(q, k, v)))
        print(f"{c['name']}: dst {want.shape}, NaN rows {int(np.isnan(want[..., 0]).sum())}")
    blobs["meta"] = np.frombuffer(json.dumps(meta).encode(), dtype=np.uint8)
    np.savez_compressed(OUT, **blobs)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
