"""GPU parity of al_fattn_f16 against oracle O2 (the f32-accumulating
restatement of nnml_compute_forward_flash_attn_ext_f16, arm.cpp:2196-2433).

Bar: max-abs <= 2e-3 and rel-L2 <= 1e-3 on the fp32 output, identical NaN
pattern. Every case prints its name before touching the GPU.
"""
import math

import numpy as np
import pytest

from arclight_amd import abi
from oracle import oracle as O
from tests.fattn_cases import assert_parity, run_gpu

pytestmark = pytest.mark.gpu
SCALE = 1.0 / math.sqrt(128)


def _case(name):
    print(f"\n[case] {name}", flush=True)


def _check(name, q, k, v, mask=None, sinks=None, **kw):
    _case(name)
    ref = O.attention(q, k, v, mask, sinks, **kw)
    got = run_gpu(q, k, v, mask, sinks, **kw)
    assert_parity(got, ref, what=name)
    return got, ref


@pytest.mark.parametrize("explicit", [True, False])
def test_decode_qwen3_4b_c512(gpu, explicit):
    # 1 layer, q_len 1, Hq 32, Hkv 8, D 128, context 512 (+ the new token), n_kv padded to 768
    q, k, v = O.make_inputs(1234, T=1, Hq=32, Hkv=8, n_kv=768)
    if explicit:
        _check("decode c512 explicit mask", q, k, v, O.causal_mask(1, 768, 512), scale=SCALE)
    else:
        _check("decode c512 implicit", q, k, v, scale=SCALE, kv_len=513)


@pytest.mark.parametrize("ctx", [4096, 16384, 32768])
def test_decode_qwen3_4b_long(gpu, ctx):
    q, k, v = O.make_inputs(ctx, T=1, Hq=32, Hkv=8, n_kv=ctx)
    _check(f"decode ctx {ctx}", q, k, v, scale=SCALE, kv_len=ctx)


def test_decode_gqa8_qwen3_32b(gpu):
    q, k, v = O.make_inputs(7, T=1, Hq=64, Hkv=8, n_kv=4096)
    _check("decode gqa 8:1 ctx 4096", q, k, v, scale=SCALE)


@pytest.mark.parametrize("T", [2, 4, 8])
def test_verify_qwen3_8b(gpu, T):
    # speculative verify: drafts at positions C..C+T-1, causal among drafts
    C = 2048
    n_kv = 2304
    q, k, v = O.make_inputs(100 + T, T=T, Hq=32, Hkv=8, n_kv=n_kv)
    _check(f"verify T={T} explicit", q, k, v, O.causal_mask(T, n_kv, C), scale=SCALE)
    _check(f"verify T={T} implicit", q, k, v, scale=SCALE, kv_len=C + T, causal_pos0=C)


def test_verify_gqa8_t8(gpu):
    q, k, v = O.make_inputs(55, T=8, Hq=64, Hkv=8, n_kv=1024)
    _check("verify gqa8 T=8", q, k, v, scale=SCALE, kv_len=1000, causal_pos0=992)


@pytest.mark.parametrize("T,pos0", [(64, 0), (96, 160)])
def test_prefill_chunk_causal(gpu, T, pos0):
    n_kv = pos0 + T
    q, k, v = O.make_inputs(T + pos0, T=T, Hq=32, Hkv=8, n_kv=n_kv)
    _check(f"prefill T={T} pos0={pos0} explicit", q, k, v, O.causal_mask(T, n_kv, pos0), scale=SCALE)
    _check(f"prefill T={T} pos0={pos0} implicit", q, k, v, scale=SCALE, causal_pos0=pos0)


def test_streams_and_mask_broadcast(gpu):
    # two streams (nnml dim 3) with their own mask planes
    rng = np.random.default_rng(3)
    q, k, v = O.make_inputs(3, B=2, T=2, Hq=8, Hkv=2, n_kv=256)
    m = np.full((2, 1, 64, 256), -np.inf, dtype=np.float16)
    m[0, 0, :2, :100] = 0
    m[1, 0, :2, 50:230] = 0
    m[1, 0, 1, 229] = -np.inf
    _check("streams B=2", q, k, v, m, scale=SCALE)
    # per-head mask planes with finite values
    mh = rng.uniform(-3, 0, size=(1, 8, 64, 256)).astype(np.float16)
    mh[..., 200:] = -np.inf
    _check("mask per head", q, k, v, mh, scale=SCALE)


def test_sinks_softcap_alibi(gpu):
    rng = np.random.default_rng(11)
    q, k, v = O.make_inputs(11, T=3, Hq=12, Hkv=4, n_kv=320)
    sinks = rng.standard_normal(12).astype(np.float32) * 3
    m = O.causal_mask(3, 320, 300)
    _check("sinks", q, k, v, m, sinks, scale=SCALE)
    _check("softcap", q, k, v, m, scale=SCALE * 4, logit_softcap=5.0)
    alibi = m.astype(np.float32)
    alibi[0, 0, :3, :301] = -np.arange(301, dtype=np.float32)[::-1] / 64.0
    _check("alibi", q, k, v, alibi.astype(np.float16), scale=SCALE, max_bias=8.0)


def test_ragged_sizes(gpu):
    # n_kv not a multiple of 32, kv_len not a multiple of the tile, T*G = 12 rows
    q, k, v = O.make_inputs(5, T=3, Hq=8, Hkv=2, n_kv=40)
    _check("n_kv 40 kv_len 37", q, k, v, scale=SCALE, kv_len=37)
    q, k, v = O.make_inputs(6, T=5, Hq=6, Hkv=3, n_kv=33)
    _check("n_kv 33 T 5 G 2", q, k, v, O.causal_mask(5, 33, 27), scale=SCALE)


def test_all_masked_rows_are_nan_and_single_cell(gpu):
    q, k, v = O.make_inputs(9, T=2, Hq=4, Hkv=1, n_kv=64)
    m = np.full((1, 1, 64, 64), -np.inf, dtype=np.float16)
    m[0, 0, 1, 17] = 0                      # token 1 sees exactly cell 17, token 0 sees nothing
    got, ref = _check("all-masked + single cell", q, k, v, m, scale=SCALE)
    assert np.isnan(got[0, 0]).all()
    vf = v.astype(np.float32)
    np.testing.assert_allclose(got[0, 1], np.broadcast_to(vf[0, 17, 0], (4, 128)), rtol=0, atol=1e-6)


def test_garbage_in_masked_cells(gpu):
    # unwritten cache cells may hold NaN/Inf: masked cells must not leak
    q, k, v = O.make_inputs(21, T=1, Hq=32, Hkv=8, n_kv=512)
    ref = O.attention(q, k, v, scale=SCALE, kv_len=300)
    kg, vg = k.copy(), v.copy()
    kg[:, 300:] = np.float16(np.nan)
    vg[:, 300:] = np.float16(np.inf)
    _case("garbage beyond kv_len")
    got = run_gpu(q, kg, vg, scale=SCALE, kv_len=300)
    assert_parity(got, ref, what="garbage")
    m = O.causal_mask(1, 512, 299)
    _case("garbage beyond mask")
    got = run_gpu(q, kg, vg, m, scale=SCALE)
    assert_parity(got, ref, what="garbage mask")


def test_prec_default_and_determinism(gpu):
    q, k, v = O.make_inputs(31, T=1, Hq=32, Hkv=8, n_kv=2048)
    _case("determinism")
    a = run_gpu(q, k, v, scale=SCALE, prec=abi.AL_PREC_DEFAULT)
    b = run_gpu(q, k, v, scale=SCALE, prec=abi.AL_PREC_F32)
    assert np.array_equal(a, b)


def test_caller_workspace(gpu):
    from arclight_amd import device, fattn
    from arclight_amd._lib import ArclightError
    q, k, v = O.make_inputs(41, T=1, Hq=32, Hkv=8, n_kv=8192)
    ref = O.attention(q, k, v, scale=SCALE)
    dq, dk, dv = fattn.upload_q(q), fattn.upload_kv(k), fattn.upload_kv(v)
    dst = device.DeviceTensor.empty(q.shape, np.float32, axes=abi.DST_AXES)
    need = fattn.workspace_bytes(dq, dk, dv, None, None, dst, scale=SCALE)
    assert need > 0
    _case("caller workspace")
    ws = device.DeviceBuffer(need)
    ws.zero()
    for _ in range(2):
        fattn.flash_attn_ext(dq, dk, dv, scale=SCALE, dst=dst, workspace=ws)
        device.synchronize()
        assert_parity(dst.numpy(np.float32), ref, what="caller workspace")
    small = device.DeviceBuffer(need - 4)
    with pytest.raises(ArclightError) as ei:
        fattn.flash_attn_ext(dq, dk, dv, scale=SCALE, dst=dst, workspace=small)
    assert ei.value.status == abi.AL_ERR_WORKSPACE


def test_rejects_what_the_reference_asserts(gpu):
    from arclight_amd._lib import ArclightError
    q, k, v = O.make_inputs(1, T=2, Hq=8, Hkv=3 if False else 2, n_kv=64)
    short_mask = np.zeros((1, 1, 32, 64), dtype=np.float16)     # rows < PAD(T, 64)
    with pytest.raises(ArclightError) as ei:
        run_gpu(q, k, v, short_mask, scale=SCALE)
    assert ei.value.status == abi.AL_ERR_INVALID
    with pytest.raises(ArclightError) as ei:
        run_gpu(q, k, v, scale=SCALE, max_bias=1.0)              # ALiBi without mask
    assert ei.value.status == abi.AL_ERR_INVALID
    with pytest.raises(ArclightError) as ei:
        run_gpu(q, k, v, scale=SCALE, prec=3)
    assert ei.value.status == abi.AL_ERR_INVALID
    q64, k64, v64 = O.make_inputs(1, T=1, Hq=8, Hkv=2, D=64, n_kv=64)
    with pytest.raises(ArclightError) as ei:
        run_gpu(q64, k64, v64, scale=SCALE)
    assert ei.value.status == abi.AL_ERR_UNSUPPORTED


def test_split_merge_repeatable_back_to_back(gpu):
    # Multi-split calls (two merge levels) launched back to back on one stream
    # without host synchronization: every result must equal the first bit for
    # bit (the merge order is fixed) and match the oracle.
    from arclight_amd import device, fattn
    q, k, v = O.make_inputs(77, T=1, Hq=32, Hkv=8, n_kv=32768)
    ref = O.attention(q, k, v, scale=SCALE)
    dq, dk, dv = fattn.upload_q(q), fattn.upload_kv(k), fattn.upload_kv(v)
    n = 64
    dsts = [device.DeviceTensor.empty(q.shape, np.float32, axes=abi.DST_AXES) for _ in range(n)]
    _case("split merge x64 back to back")
    for rep in range(3):
        for d in dsts:
            fattn.flash_attn_ext(dq, dk, dv, scale=SCALE, dst=d)
        device.synchronize()
        outs = [d.numpy(np.float32) for d in dsts]
        if rep == 0:
            first = outs[0]
            assert_parity(first, ref, what="split merge")
        for i, o in enumerate(outs):
            assert np.array_equal(o, first), f"rep {rep} call {i} differs"


def test_shapes_alternating_on_one_workspace(gpu):
    # Calls of different shapes lay out their merge records differently; the
    # arrival counters and split flags live in a fixed region no record
    # overlaps, so alternating shapes on one workspace keeps every call
    # correct.
    from arclight_amd import device, fattn
    cases = [dict(seed=90, B=1, T=1, Hq=32, Hkv=8, n_kv=32768),
             dict(seed=91, B=2, T=2, Hq=8, Hkv=2, n_kv=2048),
             dict(seed=92, B=1, T=8, Hq=32, Hkv=8, n_kv=8192),
             dict(seed=93, B=1, T=96, Hq=32, Hkv=8, n_kv=256)]
    prepared = []
    need = 0
    for c in cases:
        seed = c.pop("seed")
        q, k, v = O.make_inputs(seed, **c)
        ref = O.attention(q, k, v, scale=SCALE)
        dq, dk, dv = fattn.upload_q(q), fattn.upload_kv(k), fattn.upload_kv(v)
        dst = device.DeviceTensor.empty(q.shape, np.float32, axes=abi.DST_AXES)
        need = max(need, fattn.workspace_bytes(dq, dk, dv, None, None, dst, scale=SCALE))
        prepared.append((dq, dk, dv, dst, ref))
    ws = device.DeviceBuffer(need)
    ws.zero()
    _case("alternating shapes, one workspace")
    for rnd in range(3):
        for order in (prepared, prepared[::-1]):
            for dq, dk, dv, dst, ref in order:
                fattn.flash_attn_ext(dq, dk, dv, scale=SCALE, dst=dst, workspace=ws)
            device.synchronize()
            for i, (dq, dk, dv, dst, ref) in enumerate(order):
                assert_parity(dst.numpy(np.float32), ref, what=f"round {rnd} call {i}")
    # the lower half of the 256 KiB counter region holds the arrival counters
    # (the upper half the decode split flags, which carry epochs)
    cnt = np.empty(32768, dtype=np.uint32)
    ws.download(cnt)
    assert not cnt.any(), "arrival counters not left at zero"


@pytest.mark.parametrize("pos0", [0, 512, 1024, 1536])
def test_prefill_kernel_chunk512_qwen3_4b(gpu, pos0):
    # each 512-token chunk of a 2048-token causal prefill (Hq 32, Hkv 8), the
    # whole output against the oracle
    n_kv = 2048
    q, k, v = O.make_inputs(500 + pos0, T=512, Hq=32, Hkv=8, n_kv=n_kv)
    _check(f"prefill chunk 512 pos0 {pos0}", q, k, v, scale=SCALE, kv_len=pos0 + 512, causal_pos0=pos0)


def test_prefill_kernel_gqa8_noncausal_sinks_softcap(gpu):
    rng = np.random.default_rng(8)
    q, k, v = O.make_inputs(600, T=256, Hq=64, Hkv=8, n_kv=1000)
    _check("prefill gqa8 chunk 256 causal", q, k, v, scale=SCALE, kv_len=1000, causal_pos0=700)
    _check("prefill gqa8 non-causal kv_len 777", q, k, v, scale=SCALE, kv_len=777)
    sinks = rng.standard_normal(64).astype(np.float32)
    _check("prefill gqa8 sinks + softcap", q, k, v, None, sinks, scale=SCALE * 3, logit_softcap=4.0,
           kv_len=1000, causal_pos0=744)


def test_prefill_kernel_explicit_masks(gpu):
    # The prefill kernel reads an explicit mask itself: prefix masks (runs
    # of zeros then -inf) as per-row extents, any other mask value by value
    # in the tiles of its rows (general mode), with ALiBi, softcap, sinks,
    # per-head mask slices and two streams.
    rng = np.random.default_rng(21)
    T, n_kv = 512, 1536
    q, k, v = O.make_inputs(2101, T=T, Hq=32, Hkv=8, n_kv=n_kv)
    m = O.causal_mask(T, n_kv, 1024, kv_len=1500)
    _check("prefill, causal prefix mask", q, k, v, m, scale=SCALE)
    mb = m.copy()
    mb[0, 0, :T, :1024] = np.where(mb[0, 0, :T, :1024] == 0, rng.uniform(-3, 0, (T, 1024)), -np.inf).astype(np.float16)
    mb[0, 0, 5:40, 100:300] = -np.inf                                 # holes inside some rows
    _check("prefill, general mask with biases and holes, ALiBi", q, k, v, mb, scale=SCALE, max_bias=8.0)
    sinks = rng.standard_normal(32).astype(np.float32)
    _check("prefill, general mask, softcap + sinks", q, k, v, mb, sinks, scale=SCALE * 4, logit_softcap=5.0)
    # one mask slice per head (mask dim 2 = Hq) and two streams (dim 3 = 2)
    q2, k2, v2 = O.make_inputs(2102, B=2, T=256, Hq=16, Hkv=4, n_kv=1024)
    mh = np.broadcast_to(O.causal_mask(256, 1024, 700, kv_len=956), (2, 16, 256, 1024)).copy()
    mh[1, 3, :, 200:220] = np.float16(-2.0)
    _check("prefill, per-head general mask, 2 streams", q2, k2, v2, mh, scale=SCALE, max_bias=4.0)


def test_prefill_kernel_explicit_masks_ragged_tiles(gpu):
    # rows per kv head not a multiple of the row tile (T=510 with G=4: 2040
    # rows; T=300 with G=8: 2400 rows), so the last tile has padding rows, with
    # a prefix mask (extents) and a mask with holes (the general mode, whose
    # padding rows must read no mask values)
    for seed, T, Hq, n_kv, pos0 in ((2111, 510, 32, 1536, 1000), (2112, 300, 64, 1024, 700)):
        q, k, v = O.make_inputs(seed, T=T, Hq=Hq, Hkv=8, n_kv=n_kv)
        m = O.causal_mask(T, n_kv, pos0, kv_len=pos0 + T)
        _check(f"prefill T={T} G={Hq // 8}, ragged last tile, prefix mask", q, k, v, m, scale=SCALE)
        mh = m.copy()
        mh[0, 0, 7:T - 3, 50:90] = -np.inf                                # holes: the general mode
        mh[0, 0, T - 1, 3] = np.float16(-1.5)
        _check(f"prefill T={T} G={Hq // 8}, ragged last tile, mask with holes", q, k, v, mh, scale=SCALE)


def test_prefill_kernel_scores_outgrow_the_reference(gpu):
    # Scores that climb by several times the lazy-rescale threshold (8
    # natural units) from tile to tile for some rows, so the reference max
    # moves inside the loop, with the scores of the next tile already
    # computed against the old one; other rows fall, keeping the first
    # tile's. Dimension 0 carries the ramp: s += a * 0.25 c (cell c), a per
    # row in {-3, -1, 0, 2, 4, 6}: 1.4 a natural units per 64-cell tile.
    rng = np.random.default_rng(2201)
    for seed, T, Hq, n_kv, pos0 in ((2202, 256, 32, 1024, 768), (2203, 512, 64, 1536, 1024)):
        q, k, v = O.make_inputs(seed, T=T, Hq=Hq, Hkv=8, n_kv=n_kv)
        q[..., 0] = rng.choice(np.array([-3.0, -1.0, 0.0, 2.0, 4.0, 6.0], dtype=np.float32), size=q.shape[:-1])
        k[..., 0] = (0.25 * np.arange(n_kv)).astype(np.float16)[None, :, None]
        name = f"prefill T={T} Hq={Hq}, growing scores"
        _check(f"{name}, length / causal rule", q, k, v, scale=SCALE, kv_len=pos0 + T, causal_pos0=pos0)
        m = O.causal_mask(T, n_kv, pos0, kv_len=pos0 + T)
        _check(f"{name}, prefix mask", q, k, v, m, scale=SCALE)
        mh = m.copy()
        mh[0, 0, 3:T - 5, 40:70] = -np.inf                                # holes: the general mode
        _check(f"{name}, mask with holes", q, k, v, mh, scale=SCALE)


def test_prefill_kernel_streams_ragged(gpu):
    # two streams, rows not a multiple of 64, cells not a multiple of 32
    q, k, v = O.make_inputs(601, B=2, T=510, Hq=16, Hkv=4, n_kv=1111)
    _check("prefill B=2 T=510 ragged", q, k, v, scale=SCALE, kv_len=1100, causal_pos0=590)


def test_decode_kernel_shapes(gpu):
    # whole-cell staged decode kernel: head groups of 4, 2 and 1, two merge
    # levels with an explicit mask over two streams, exactly 16 rows per head
    q, k, v = O.make_inputs(41, B=2, T=1, Hq=32, Hkv=8, n_kv=8192)
    m = np.full((2, 1, 64, 8192), -np.inf, dtype=np.float16)
    m[0, 0, 0, :8000] = 0
    m[1, 0, 0, :6000] = 0
    m[1, 0, 0, 3000:3100] = -np.inf
    _check("decode two streams, mask, two-level merge", q, k, v, m, scale=SCALE)
    q, k, v = O.make_inputs(42, T=1, Hq=24, Hkv=6, n_kv=3000)
    _check("decode Hkv 6 (head pairs)", q, k, v, scale=SCALE, kv_len=2999)
    q, k, v = O.make_inputs(43, T=1, Hq=16, Hkv=1, n_kv=5000)
    _check("decode 16 rows on one kv head", q, k, v, scale=SCALE, kv_len=4990)
    q, k, v = O.make_inputs(44, T=2, Hq=64, Hkv=8, n_kv=1024)
    _check("verify T=2 gqa 8:1 (16 rows)", q, k, v, scale=SCALE, kv_len=1000, causal_pos0=998)


def test_decode_kernel_two_row_blocks(gpu):
    # 17..32 query rows per kv head with implicit masks: the decode kernel's
    # two-row-block form (8-draft verify), with sinks, softcap, two streams,
    # ragged row counts and a kv_len inside the last stage
    rng = np.random.default_rng(61)
    q, k, v = O.make_inputs(61, T=8, Hq=32, Hkv=8, n_kv=2304)
    sinks = rng.standard_normal(32).astype(np.float32) * 3
    _check("two row blocks, sinks", q, k, v, None, sinks, scale=SCALE, kv_len=2056, causal_pos0=2048)
    _check("two row blocks, softcap", q, k, v, scale=SCALE * 4, logit_softcap=5.0, kv_len=2056, causal_pos0=2048)
    q, k, v = O.make_inputs(62, B=2, T=5, Hq=16, Hkv=4, n_kv=1500)
    _check("two row blocks, 2 streams, 20 rows", q, k, v, scale=SCALE, kv_len=1493, causal_pos0=1488)
    q, k, v = O.make_inputs(63, T=3, Hq=56, Hkv=7, n_kv=700)
    _check("two row blocks, 24 rows, G 8", q, k, v, scale=SCALE, kv_len=650)


def test_decode_kernel_two_row_blocks_explicit_mask(gpu):
    # 17..32 rows per kv head with the f16 mask tensor: the masked
    # two-row-block decode kernel, with the causal mask of 8 drafts, a mask
    # broadcast over two streams with ALiBi biases in it, and mask stages
    # that are all zero next to ones that are not
    q, k, v = O.make_inputs(64, T=8, Hq=32, Hkv=8, n_kv=2304)
    _check("two row blocks, explicit causal mask", q, k, v, O.causal_mask(8, 2304, 2048, kv_len=2056), scale=SCALE)
    rng = np.random.default_rng(65)
    q, k, v = O.make_inputs(65, B=2, T=6, Hq=16, Hkv=4, n_kv=1024)
    m = O.causal_mask(6, 1024, 1000, kv_len=1006)
    m[..., 200:260] = rng.uniform(-3, 0, (1, 1, m.shape[2], 60)).astype(np.float16)
    m[..., 300] = -np.inf
    _check("two row blocks, mask with biases, ALiBi, 2 streams", q, k, v, m, scale=SCALE, max_bias=8.0)


def test_decode_mask_preloaded_and_per_stage(gpu, monkeypatch):
    """A decode call with a mask tensor loads each wave's mask values into LDS
    once, before its first stage, when the workgroup's share fits
    (AL_DECODE_MASK_PRE=0: with every stage instead). Both forms apply the
    same mask values in the same order, so they give the same bits, and both
    match the oracle: one token over a mask with holes and finite values
    shared by the heads, eight drafts with the causal mask among them
    (32 rows, two row blocks), four drafts with per-head mask planes, and a
    one-token call whose share is too large to preload (131072 cells, two
    mask planes that the heads alternate between: both settings take the
    per-stage form there)."""
    rng = np.random.default_rng(77)
    cases = []
    q, k, v = O.make_inputs(771, T=1, Hq=32, Hkv=8, n_kv=4096)
    m = np.zeros((1, 1, 64, 4096), np.float16)
    m[0, 0, 0, rng.choice(4096, 700, replace=False)] = -np.inf
    m[0, 0, 0, :512] = rng.uniform(-2, 0, 512).astype(np.float16)
    m[0, 0, 0, 4000:] = -np.inf
    cases.append(("one token, holes and finite values", q, k, v, m))
    q, k, v = O.make_inputs(772, T=8, Hq=32, Hkv=8, n_kv=8448)
    cases.append(("eight drafts, causal", q, k, v, O.causal_mask(8, 8448, 8192, kv_len=8200)))
    q, k, v = O.make_inputs(773, T=4, Hq=32, Hkv=8, n_kv=2048)
    mh = rng.uniform(-1, 0, size=(1, 32, 64, 2048)).astype(np.float16)
    mh[..., 1900:] = -np.inf
    mh[0, 5, 2, :1000] = -np.inf
    cases.append(("four drafts, per-head planes", q, k, v, mh))
    q, k, v = O.make_inputs(774, T=1, Hq=8, Hkv=2, n_kv=131072)
    mb = np.zeros((1, 2, 64, 131072), np.float16)
    mb[0, 0, 0, 120000:] = -np.inf
    mb[0, 1, 0, :70000] = -np.inf
    cases.append(("one token, two mask planes, 131072 cells", q, k, v, mb))
    for name, q, k, v, m in cases:
        ref = O.attention(q, k, v, m, scale=SCALE)
        _case(f"{name}: preloaded")
        monkeypatch.delenv("AL_DECODE_MASK_PRE", raising=False)
        a = run_gpu(q, k, v, m, scale=SCALE)
        _case(f"{name}: per stage")
        monkeypatch.setenv("AL_DECODE_MASK_PRE", "0")
        b = run_gpu(q, k, v, m, scale=SCALE)
        monkeypatch.delenv("AL_DECODE_MASK_PRE", raising=False)
        assert np.array_equal(a, b, equal_nan=True), f"{name}: preloaded and per-stage masks differ"
        assert_parity(a, ref, what=name)


def test_decode_two_waves_one_pass_and_tree_merge(gpu, monkeypatch):
    """The 2-wave decode shape merges its two waves' states in one pass with
    all threads when a split covers at most AL_DECODE_ONE_PASS_CELLS cells
    (512 by default), else wave 0 folds in wave 1's state (the tree). Each
    form against the oracle, and the two against each other (the same two
    weighted terms, summed in another order: within a few ulp): one token
    over 4096 and 16384 cells (128 and 512 cells per split), the Qwen3-32B
    shape (8 rows per kv head), 2-draft verify with the causal mask among
    the drafts, 2 streams, an explicit mask with holes (preloaded and per
    stage), and one split over 40 and 10 cells (the pass writes the output
    rows; a wave with one stage or none)."""
    rng = np.random.default_rng(91)
    cases = []
    for seed, n_kv in ((911, 4096), (912, 16384)):
        q, k, v = O.make_inputs(seed, T=1, Hq=32, Hkv=8, n_kv=n_kv)
        cases.append((f"one token over {n_kv} cells", q, k, v, None, dict(kv_len=n_kv)))
    q, k, v = O.make_inputs(913, T=1, Hq=64, Hkv=8, n_kv=4096)
    cases.append(("Qwen3-32B shape, 4096 cells", q, k, v, None, dict(kv_len=4096)))
    q, k, v = O.make_inputs(914, T=2, Hq=32, Hkv=8, n_kv=8192)
    cases.append(("2 drafts over 8192 cells", q, k, v, None, dict(kv_len=8192, causal_pos0=8190)))
    q, k, v = O.make_inputs(915, B=2, T=1, Hq=32, Hkv=8, n_kv=3000)
    cases.append(("2 streams, 3000 cells", q, k, v, None, dict(kv_len=3000)))
    q, k, v = O.make_inputs(916, T=1, Hq=32, Hkv=8, n_kv=6000)
    m = np.zeros((1, 1, 64, 6000), np.float16)
    m[0, 0, 0, rng.choice(6000, 900, replace=False)] = -np.inf
    m[0, 0, 0, :300] = rng.uniform(-2, 0, 300).astype(np.float16)
    cases.append(("explicit mask with holes, 6000 cells", q, k, v, m, {}))
    for seed, n_kv in ((917, 40), (918, 10)):
        q, k, v = O.make_inputs(seed, T=1, Hq=32, Hkv=8, n_kv=n_kv)
        cases.append((f"one split over {n_kv} cells", q, k, v, None, dict(kv_len=n_kv)))
    for name, q, k, v, m, kw in cases:
        ref = O.attention(q, k, v, m, scale=SCALE, **kw)
        forms = {}
        for label, cells, pre in (("one pass", None, None), ("tree", "0", None), ("one pass, mask per stage", None, "0")):
            if pre is not None and m is None:
                continue
            _case(f"{name}: {label}")
            for var, val in (("AL_DECODE_ONE_PASS_CELLS", cells), ("AL_DECODE_MASK_PRE", pre)):
                if val is None:
                    monkeypatch.delenv(var, raising=False)
                else:
                    monkeypatch.setenv(var, val)
            forms[label] = run_gpu(q, k, v, m, scale=SCALE, **kw)
            assert_parity(forms[label], ref, what=f"{name}: {label}")
        monkeypatch.delenv("AL_DECODE_ONE_PASS_CELLS", raising=False)
        monkeypatch.delenv("AL_DECODE_MASK_PRE", raising=False)
        a, b = forms["one pass"], forms["tree"]
        assert np.array_equal(np.isnan(a), np.isnan(b)), f"{name}: forms differ in NaN rows"
        np.testing.assert_allclose(a, b, rtol=2e-6, atol=1e-6, err_msg=f"{name}: one pass against tree")
        if "one pass, mask per stage" in forms:
            assert np.array_equal(a, forms["one pass, mask per stage"], equal_nan=True), f"{name}: mask forms differ"


def test_decode_two_waves_sinks_softcap_alibi_both_merges(gpu, monkeypatch):
    """One token per stream (the 2-wave shape) with attention sinks, logit
    softcap and ALiBi over a mask with finite biases, against the oracle,
    with the one-pass and the tree merge of the waves: 4096 cells (128 per
    split: one pass by default) and 20000 cells (640 per split: the tree),
    each also with the other form forced."""
    rng = np.random.default_rng(93)
    for seed, n_kv in ((931, 4096), (932, 20000)):
        q, k, v = O.make_inputs(seed, T=1, Hq=32, Hkv=8, n_kv=n_kv)
        sinks = rng.standard_normal(32).astype(np.float32) * 3
        m = np.zeros((1, 1, 64, n_kv), np.float16)
        m[0, 0, 0, :] = (-np.arange(n_kv, dtype=np.float32)[::-1] / 4096.0).astype(np.float16)
        m[0, 0, 0, rng.choice(n_kv, n_kv // 10, replace=False)] = -np.inf
        for cells in (None, "0", "100000"):
            label = {None: "default", "0": "tree", "100000": "one pass"}[cells]
            if cells is None:
                monkeypatch.delenv("AL_DECODE_ONE_PASS_CELLS", raising=False)
            else:
                monkeypatch.setenv("AL_DECODE_ONE_PASS_CELLS", cells)
            _case(f"{n_kv} cells, sinks: {label}")
            _check(f"{n_kv} cells, sinks ({label})", q, k, v, m, sinks, scale=SCALE)
            _case(f"{n_kv} cells, softcap + ALiBi: {label}")
            _check(f"{n_kv} cells, softcap + ALiBi ({label})", q, k, v, m, scale=SCALE * 4, logit_softcap=5.0,
                   max_bias=8.0)
        monkeypatch.delenv("AL_DECODE_ONE_PASS_CELLS", raising=False)


def test_verify_waves_without_stages_and_one_pass_merge(gpu):
    """The 8-wave decode shape (17-32 query rows per kv head) merges its
    waves in one pass from their own LDS rings. Short contexts leave some of
    the 8 waves with no stage at all (they reach the merge while the others
    still work), and with one split the pass writes the output rows itself:
    8 drafts (two row blocks) over 100, 700 and 5000 cells, 5 drafts (20
    rows, one row block partly valid) over 90 cells, with the causal mask
    among the drafts, against the oracle."""
    for seed, T, n_kv in ((881, 8, 100), (882, 8, 700), (883, 8, 5000), (884, 5, 90)):
        q, k, v = O.make_inputs(seed, T=T, Hq=32, Hkv=8, n_kv=n_kv)
        kw = dict(kv_len=n_kv, causal_pos0=n_kv - T)
        _case(f"{T} drafts over {n_kv} cells")
        got = run_gpu(q, k, v, scale=SCALE, **kw)
        assert_parity(got, O.attention(q, k, v, scale=SCALE, **kw), what=f"{T} drafts over {n_kv} cells")
