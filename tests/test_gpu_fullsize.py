"""Parity at the benchmark shapes themselves: Qwen3-8B-shape speculative
verify over an 8192-cell context, Qwen3-32B-shape decode at 32768 cells and
prefill in 1024-token causal chunks, Qwen3-4B-shape prefill in 256-token
ubatches (implicit and explicit masks), plus a size-independent property of
the full 2048-token Qwen3-4B prefill: its four causal chunks of 512 equal
one causal call over all 2048 tokens.

Where the oracle over every row of a call would take minutes (a 1024-token
chunk at 64 query heads), the device computes the whole call and a sample of
its tokens is compared with the oracle run on those tokens alone: rows are
independent (nnml/src/ops/arm/arm.cpp:2287-2291 forms each (token, head)
row from its q row, K, V and its own mask row), so the oracle gets the
sampled q rows with their rows of the same causal mask.

Bar: max-abs <= 2e-3 and rel-L2 <= 1e-3 on the fp32 output against oracle
O2, as everywhere.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O
from tests.fattn_cases import assert_parity, run_gpu

pytestmark = pytest.mark.gpu
SCALE = 1.0 / math.sqrt(128)


def _case(name):
    print(f"\n[case] {name}", flush=True)


def _sampled_ref(q, k, v, sel, pos0, kv_len):
    """Oracle rows of tokens `sel` of a causal call whose token t sits at
    position pos0 + t over cells [0, kv_len)."""
    T, n_kv = q.shape[1], k.shape[1]
    full = O.causal_mask(T, n_kv, pos0, kv_len=kv_len)
    rows = (len(sel) + 63) // 64 * 64
    m = np.full((1, 1, rows, n_kv), -np.inf, dtype=np.float16)
    m[:, :, :len(sel)] = full[:, :, sel]
    return O.attention(np.ascontiguousarray(q[:, sel]), k, v, m, scale=SCALE)


@pytest.mark.parametrize("T", [4, 8])
def test_verify_qwen3_8b_ctx8192(gpu, T):
    # drafts at positions 8192 .. 8192 + T - 1, cells padded to 256
    C = 8192
    n_kv = (C + T + 255) // 256 * 256
    q, k, v = O.make_inputs(8192 + T, T=T, Hq=32, Hkv=8, n_kv=n_kv)
    _case(f"verify T={T} ctx {C} implicit")
    ref = O.attention(q, k, v, scale=SCALE, kv_len=C + T, causal_pos0=C)
    assert_parity(run_gpu(q, k, v, scale=SCALE, kv_len=C + T, causal_pos0=C), ref, what=f"verify T={T} implicit")
    _case(f"verify T={T} ctx {C} explicit mask")
    got = run_gpu(q, k, v, O.causal_mask(T, n_kv, C, kv_len=C + T), scale=SCALE)
    assert_parity(got, ref, what=f"verify T={T} explicit")


def test_decode_qwen3_32b_ctx32768(gpu):
    q, k, v = O.make_inputs(3232, T=1, Hq=64, Hkv=8, n_kv=32768)
    _case("decode Qwen3-32B shape ctx 32768")
    ref = O.attention(q, k, v, scale=SCALE, kv_len=32768)
    assert_parity(run_gpu(q, k, v, scale=SCALE, kv_len=32768), ref, what="decode 32B ctx 32768")


def test_decode_qwen3_4b_ctx32768_explicit_mask(gpu):
    # the benchmark's decode as nnml calls it: the new token at position
    # 32768 over 32769 valid cells of 33024 (padded to 256), with the f16 mask
    # tensor (PAD(1, 64) rows) and no length hints
    n_kv = 33024
    q, k, v = O.make_inputs(3233, T=1, Hq=32, Hkv=8, n_kv=n_kv)
    m = O.causal_mask(1, n_kv, 32768, kv_len=32769)
    _case("decode Qwen3-4B shape ctx 32768, explicit mask")
    assert_parity(run_gpu(q, k, v, m, scale=SCALE), O.attention(q, k, v, m, scale=SCALE),
                  what="decode 4B ctx 32768 explicit mask")


@pytest.mark.parametrize("pos0", [0, 1024, 2048, 3072])
def test_prefill_qwen3_32b_chunk1024(gpu, pos0):
    # the four 1024-token chunks of a 4096-token prompt at 64 query heads
    T, kv_len = 1024, pos0 + 1024
    q, k, v = O.make_inputs(1024 + pos0, T=T, Hq=64, Hkv=8, n_kv=kv_len)
    _case(f"prefill Qwen3-32B shape chunk 1024 pos0 {pos0}")
    got = run_gpu(q, k, v, scale=SCALE, kv_len=kv_len, causal_pos0=pos0)
    rng = np.random.default_rng(pos0)
    sel = np.unique(np.concatenate([[0, 1, 63, 64, T - 1], rng.choice(T, 27, replace=False)]))
    ref = _sampled_ref(q, k, v, sel, pos0, kv_len)
    assert_parity(got[:, sel], ref, what=f"prefill 32B chunk pos0 {pos0} ({len(sel)} tokens)")


def test_prefill_qwen3_32b_explicit_mask_then_split_decode(gpu):
    # the 32B 1024-token chunk as nnml calls it (the f16 mask tensor, no
    # length hints), then a split decode on the same library workspace: the
    # masked call must leave the workspace's arrival counters and split
    # flags as the decode expects them
    T, pos0 = 1024, 1024
    kv_len = pos0 + T
    q, k, v = O.make_inputs(7001, T=T, Hq=64, Hkv=8, n_kv=kv_len)
    m = O.causal_mask(T, kv_len, pos0, kv_len=kv_len)
    _case("prefill Qwen3-32B shape chunk 1024 pos0 1024, explicit mask")
    got = run_gpu(q, k, v, m, scale=SCALE)
    rng = np.random.default_rng(7)
    sel = np.unique(np.concatenate([[0, 1, 63, 64, T - 1], rng.choice(T, 27, replace=False)]))
    assert_parity(got[:, sel], _sampled_ref(q, k, v, sel, pos0, kv_len), what="prefill 32B explicit mask")
    qd, kd, vd = O.make_inputs(7002, T=1, Hq=32, Hkv=8, n_kv=16384)
    _case("decode ctx 16384 after the masked prefill")
    for rep in range(2):
        assert_parity(run_gpu(qd, kd, vd, scale=SCALE, kv_len=16384), O.attention(qd, kd, vd, scale=SCALE, kv_len=16384),
                      what=f"split decode after masked prefill, call {rep}")


def test_prefill_chunks_equal_one_causal_call(gpu):
    # 2048-token Qwen3-4B-shape prompt: 4 chunks of 512 (chunk c sees cells
    # [0, 512 (c + 1))) against one causal call over all 2048 tokens
    q, k, v = O.make_inputs(2048, T=2048, Hq=32, Hkv=8, n_kv=2048)
    _case("prefill 2048 one causal call")
    whole = run_gpu(q, k, v, scale=SCALE, kv_len=2048, causal_pos0=0)
    sel = np.array([0, 511, 512, 1000, 1535, 1536, 2047])
    assert_parity(whole[:, sel], _sampled_ref(q, k, v, sel, 0, 2048), what="one causal call, sampled rows")
    for c in range(4):
        _case(f"prefill 2048 chunk {c}")
        qc = np.ascontiguousarray(q[:, 512 * c:512 * (c + 1)])
        got = run_gpu(qc, k, v, scale=SCALE, kv_len=512 * (c + 1), causal_pos0=512 * c)
        assert_parity(got, whole[:, 512 * c:512 * (c + 1)], what=f"chunk {c} vs one call")


def test_prefill_explicit_mask_on_the_prefill_kernel(gpu):
    # a 512-token causal chunk with the f16 mask tensor and no length hints:
    # a mask of zero runs then -inf becomes per-row extents in the prefill
    # kernel; a mask with a hole and biases is taken value by value; and a
    # plain mask again after that
    n_kv = 2048
    q, k, v = O.make_inputs(4096, T=512, Hq=32, Hkv=8, n_kv=n_kv)
    m = O.causal_mask(512, n_kv, 1536, kv_len=2000)
    _case("prefill chunk 512, explicit causal + length mask")
    assert_parity(run_gpu(q, k, v, m, scale=SCALE), O.attention(q, k, v, m, scale=SCALE), what="explicit causal mask")
    m2 = m.copy()
    m2[..., 100] = -np.inf
    m2[..., 200:210] = np.float16(-1.5)
    _case("prefill chunk 512, mask with a hole and biases")
    assert_parity(run_gpu(q, k, v, m2, scale=SCALE), O.attention(q, k, v, m2, scale=SCALE), what="mask with hole")
    m3 = O.causal_mask(512, n_kv, 0, kv_len=512)
    _case("prefill first chunk, explicit causal mask")
    assert_parity(run_gpu(q, k, v, m3, scale=SCALE), O.attention(q, k, v, m3, scale=SCALE), what="first chunk mask")


@pytest.mark.parametrize("pos0", [0, 1024, 1792])
def test_prefill_qwen3_4b_ubatch256(gpu, pos0):
    # ArcLight's default 256-token ubatch (apps/al-gen.cpp:129-130) at the
    # Qwen3-4B shape: 8 ubatches make a 2048-token prompt; 1024 rows per kv
    # head take the prefill kernel's 64-row tiles, with workgroup splits.
    # Whole output against the oracle, implicit masking and the explicit f16
    # mask without length hints (the call as nnml makes it).
    T, kv_len = 256, pos0 + 256
    n_kv = 2048
    q, k, v = O.make_inputs(256 + pos0, T=T, Hq=32, Hkv=8, n_kv=n_kv)
    ref = O.attention(q, k, v, scale=SCALE, kv_len=kv_len, causal_pos0=pos0)
    _case(f"prefill Qwen3-4B ubatch 256 pos0 {pos0} implicit")
    assert_parity(run_gpu(q, k, v, scale=SCALE, kv_len=kv_len, causal_pos0=pos0), ref,
                  what=f"ubatch 256 pos0 {pos0} implicit")
    _case(f"prefill Qwen3-4B ubatch 256 pos0 {pos0} explicit mask")
    got = run_gpu(q, k, v, O.causal_mask(T, n_kv, pos0, kv_len=kv_len), scale=SCALE)
    assert_parity(got, ref, what=f"ubatch 256 pos0 {pos0} explicit")
