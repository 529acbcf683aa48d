"""KV-cache cell bookkeeping and mask (host side, no GPU).

The oracle (oracle/kv_cells.py, a restatement of llm_kv_cells /
llm_kv_cache, nnml/include/cgraph.h:612-960 and nnml/src/cgraph.cpp:
1263-1590) is pinned first on scenarios whose outcome follows from the
reference's rules without running them: first-fit placement from the head,
n_kv = PAD(last used cell + 1, n_pad), the causal mask of one contiguous
sequence (which is oracle.causal_mask's closed form), block structure by
sequence, freed cells reused lowest-first. Then the library's C++
bookkeeping (al_kv_cells_*) must agree with the oracle bit for bit on seeded
random operation sequences: rows, n_kv, every cell's state, and the mask.
"""
import numpy as np
import pytest

from oracle import kv_cells as KC
from oracle import oracle as O

def _lib_cells(*a, **kw):
    from arclight_amd import _lib, kv
    if not __import__("os").path.exists(_lib.LIB_PATH):
        pytest.skip("library not built (run python -m arclight_amd.build)")
    return kv.KvCells(*a, **kw)


def _seq_ub(seq, p0, n):
    return [(p0 + i, [seq]) for i in range(n)]


# ---------------------------------------------------------------------------
# the oracle against what the rules fix
# ---------------------------------------------------------------------------

def test_oracle_single_sequence_prefill_then_decode():
    c = KC.KvCache(1024, n_pad=256)
    rows, n_kv = c.place(_seq_ub(0, 0, 300))
    assert rows.tolist() == list(range(300))          # first fit from head 0
    assert n_kv == 512                                # PAD(300, 256)
    m = c.mask(_seq_ub(0, 0, 300), n_kv)
    assert m.shape == (1, 1, 320, 512)                # rows padded to 64
    np.testing.assert_array_equal(m, O.causal_mask(300, 512, 0, kv_len=300))
    for p in range(300, 305):
        rows, n_kv = c.place(_seq_ub(0, p, 1))
        assert rows.tolist() == [p] and n_kv == 512
        m = c.mask(_seq_ub(0, p, 1), n_kv)
        np.testing.assert_array_equal(m, O.causal_mask(1, 512, p, kv_len=p + 1))


def test_oracle_n_kv_minimum_and_cap():
    c = KC.KvCache(512, n_pad=256)
    assert c.place(_seq_ub(0, 0, 1))[1] == 256        # at least n_pad
    c2 = KC.KvCache(512, n_pad=256)
    assert c2.place(_seq_ub(0, 0, 511))[1] == 512     # capped at the cache size


def test_oracle_two_sequences_unified_block_mask():
    c = KC.KvCache(256, n_seq_max=2, n_pad=256)
    ub = [(0, [0]), (0, [1]), (1, [0]), (1, [1]), (2, [0])]
    rows, n_kv = c.place(ub)
    assert rows.tolist() == [0, 1, 2, 3, 4]
    m = c.mask(ub, n_kv)[0, 0].astype(np.float32)
    vis = np.isfinite(m)
    # token t sees exactly the cells of its own sequence at positions <= its own
    want = np.zeros_like(vis)
    for t, (p, (s,)) in enumerate(ub):
        for j, (pj, (sj,)) in enumerate(ub):
            want[t, j] = s == sj and pj <= p
    assert np.array_equal(vis, want)


def test_oracle_shared_prompt_cells_visible_to_both():
    c = KC.KvCache(256, n_seq_max=2, n_pad=256)
    c.place([(i, [0, 1]) for i in range(4)])           # a prompt shared by sequences 0 and 1
    ub = [(4, [0]), (4, [1])]
    rows, n_kv = c.place(ub)
    assert rows.tolist() == [4, 5]
    vis = np.isfinite(c.mask(ub, n_kv)[0, 0].astype(np.float32))
    assert vis[0, :6].tolist() == [True] * 4 + [True, False]
    assert vis[1, :6].tolist() == [True] * 4 + [False, True]


def test_oracle_seq_rm_frees_and_reuses_lowest_first():
    c = KC.KvCache(256, n_seq_max=2, n_pad=256)
    c.place([(i, [i % 2]) for i in range(8)])          # cells 0..7 alternate sequences 0 and 1
    c.seq_rm(1, -1, -1)                                # sequence 1 gone: cells 1, 3, 5, 7 free
    assert [c.cells[0].is_empty(i) for i in range(8)] == [False, True] * 4
    assert c.heads[0] == 1
    rows, _ = c.place(_seq_ub(1, 0, 3))
    assert rows.tolist() == [1, 3, 5]
    c.seq_rm(0, 2, 6)                                  # sequence 0 (cells 0, 2, 4, 6) loses positions 2 and 4
    assert [c.cells[0].pos[i] for i in (0, 2, 4, 6)] == [0, -1, -1, 6]
    assert c.heads[0] == 2


def test_oracle_wraparound_and_full():
    c = KC.KvCache(256, n_pad=256)
    c.place(_seq_ub(0, 0, 256))
    assert c.place(_seq_ub(0, 256, 1)) is None         # full
    c.seq_rm(0, 0, 10)                                 # drop the 10 oldest positions
    rows, n_kv = c.place(_seq_ub(0, 256, 4))
    assert rows.tolist() == [0, 1, 2, 3] and n_kv == 256
    m = c.mask(_seq_ub(0, 256, 4), n_kv)[0, 0].astype(np.float32)
    # the new tokens see cells 10..255 (positions 10..255) and the new cells up to themselves
    for t in range(4):
        vis = np.isfinite(m[t])
        assert vis[10:].all() and vis[:t + 1].all() and not vis[t + 1:10].any()


def test_oracle_streams_map_sequences():
    c = KC.KvCache(256, n_seq_max=3, n_pad=256, unified=False)
    ub = _seq_ub(0, 0, 3) + _seq_ub(2, 0, 3)
    rows, n_kv = c.place(ub)
    assert rows.tolist() == [0, 1, 2, 512, 513, 514]  # stream * kv_size + cell
    m = c.mask(ub, n_kv, n_stream_ub=2)
    assert m.shape == (2, 1, 64, 256)
    np.testing.assert_array_equal(m[0:1], O.causal_mask(3, 256, 0, kv_len=3))
    np.testing.assert_array_equal(m[1:2], O.causal_mask(3, 256, 0, kv_len=3))


def test_oracle_head_reset_rule():
    # find_slot restarts from cell 0 when head > used + 2 * n_tokens
    c = KC.KvCache(512, n_pad=256)
    c.place(_seq_ub(0, 0, 100))
    c.seq_rm(0, -1, -1)                                # empties the cache; head stays at 0
    assert c.heads[0] == 0
    c.place(_seq_ub(0, 0, 100))
    c.seq_rm(0, 0, 50)                                 # head -> 0 (lowest freed cell)
    c.heads[0] = 300                                   # an old head far past the used cells
    rows, _ = c.place(_seq_ub(0, 100, 2))              # 300 > 50 + 4: search from 0
    assert rows.tolist() == [0, 1]


# ---------------------------------------------------------------------------
# the library against the oracle
# ---------------------------------------------------------------------------

def _check_same(lib, orc, ub=None, n_kv=None, n_stream_ub=1):
    pos, seq = lib.state()
    for s in range(orc.n_stream):
        assert pos[s].tolist() == orc.cells[s].pos
        want = [sum(1 << q for q in orc.cells[s].seq[i]) for i in range(orc.kv_size)]
        assert seq[s].tolist() == want
    if ub is not None:
        np.testing.assert_array_equal(lib.mask_host(ub, n_kv, n_stream_ub).view(np.uint16),
                                      orc.mask(ub, n_kv, n_stream_ub).view(np.uint16))


def _random_ubatch(rng, next_pos, n_seq, unified, shared_ok=True):
    seqs = sorted(rng.choice(n_seq, size=int(rng.integers(1, n_seq + 1)), replace=False).tolist())
    n_per = int(rng.integers(1, 24))
    ub = []
    for s in seqs:
        for i in range(n_per):
            extra = []
            if unified and shared_ok and rng.random() < 0.1:
                extra = [q for q in range(s + 1, n_seq) if rng.random() < 0.5]
            ub.append((next_pos[s] + i, [s] + extra))
        next_pos[s] += n_per
    return ub, len(seqs)


@pytest.mark.parametrize("unified,n_seq,seed", [(True, 1, 0), (True, 3, 1), (True, 5, 2), (False, 3, 3),
                                                (False, 2, 4)])
def test_library_matches_oracle_random_ops(unified, n_seq, seed):
    rng = np.random.default_rng(seed)
    kv_size, n_pad = 512, 128
    lib = _lib_cells(kv_size, n_seq, n_pad, unified)
    orc = KC.KvCache(kv_size, n_seq_max=n_seq, n_pad=n_pad, unified=unified)
    next_pos = [0] * n_seq
    n_place = 0
    for step in range(200):
        r = rng.random()
        if r < 0.7:
            ub, n_seqs = _random_ubatch(rng, next_pos, n_seq, unified)
            want = orc.place(ub)
            if want is None:
                with pytest.raises(Exception):
                    lib.place(ub)
                for p, seqs in ub:                     # the batch was not placed
                    next_pos[seqs[0]] = min(next_pos[seqs[0]], p)
            else:
                rows, n_kv = lib.place(ub)
                assert rows.tolist() == want[0].tolist(), f"step {step}"
                assert n_kv == want[1], f"step {step}"
                n_place += 1
                _check_same(lib, orc, ub, n_kv, 1 if unified else n_seqs)
        elif r < 0.95:
            # a rolled-back tail (speculative decoding), a hole, or an old prefix
            s = int(rng.integers(-1, n_seq)) if rng.random() < 0.15 else int(rng.integers(0, n_seq))
            top = max(next_pos[s] if s >= 0 else max(next_pos), 1)
            p0 = int(rng.integers(-1, top))
            p1 = -1 if rng.random() < 0.4 else max(p0, 0) + int(rng.integers(1, 60))
            orc.seq_rm(s, p0, p1)
            lib.seq_rm(s, p0, p1)
            if p1 == -1:
                for q in (range(n_seq) if s < 0 else [s]):
                    next_pos[q] = min(next_pos[q], max(p0, 0))
            _check_same(lib, orc)
        else:
            orc = KC.KvCache(kv_size, n_seq_max=n_seq, n_pad=n_pad, unified=unified)
            lib.clear()
            next_pos = [0] * n_seq
            _check_same(lib, orc)
    assert n_place > 40


def test_library_full_cache_leaves_state_unchanged():
    lib = _lib_cells(256, 1, 256, True)
    lib.place(_seq_ub(0, 0, 250))
    before = lib.state()
    with pytest.raises(Exception, match="no room"):
        lib.place(_seq_ub(0, 250, 10))
    after = lib.state()
    assert np.array_equal(before[0], after[0]) and np.array_equal(before[1], after[1])


def test_library_rejects_bad_input():
    from arclight_amd._lib import ArclightError
    with pytest.raises(ArclightError):
        _lib_cells(300, 1, 256, True)                  # kv_size not a multiple of n_pad
    lib = _lib_cells(256, 2, 256, False)
    with pytest.raises(ArclightError):
        lib.place(_seq_ub(0, 0, 2) + _seq_ub(1, 0, 1))   # unequal blocks per stream
    with pytest.raises(ArclightError):
        lib.mask_host(_seq_ub(0, 0, 3), 256, 2)          # 3 tokens in 2 streams


# ---------------------------------------------------------------------------
# the implicit length + causal rule
# ---------------------------------------------------------------------------

def test_implicit_rule_detected_and_exact():
    lib = _lib_cells(1024, 2, 256, True)
    ub = _seq_ub(0, 0, 300)
    _, n_kv = lib.place(ub)
    assert lib.implicit(ub, n_kv) == (300, 0)
    np.testing.assert_array_equal(lib.mask_host(ub, n_kv), O.causal_mask(300, n_kv, 0, kv_len=300))
    for p in (300, 301):
        ub = _seq_ub(0, p, 1)
        _, n_kv = lib.place(ub)
        kv_len, pos0 = lib.implicit(ub, n_kv)
        assert (kv_len, pos0) == (p + 1, p)
        np.testing.assert_array_equal(lib.mask_host(ub, n_kv), O.causal_mask(1, n_kv, pos0, kv_len=kv_len))
    # a spec-verify batch of 4 drafts
    ub = _seq_ub(0, 302, 4)
    _, n_kv = lib.place(ub)
    kv_len, pos0 = lib.implicit(ub, n_kv)
    np.testing.assert_array_equal(lib.mask_host(ub, n_kv), O.causal_mask(4, n_kv, pos0, kv_len=kv_len))


def test_implicit_rule_refused_when_it_does_not_hold():
    lib = _lib_cells(512, 2, 256, True)
    lib.place(_seq_ub(0, 0, 10))
    lib.place(_seq_ub(1, 0, 5))                         # another sequence's cells after ours
    ub = _seq_ub(0, 10, 1)
    _, n_kv = lib.place(ub)
    assert lib.implicit(ub, n_kv) is None               # cell 15 holds seq 0 position 10, not 15
    lib2 = _lib_cells(512, 1, 256, True)
    lib2.place(_seq_ub(0, 0, 20))
    lib2.seq_rm(0, 5, 8)                                # a hole
    ub = _seq_ub(0, 20, 1)
    _, n_kv = lib2.place(ub)
    assert lib2.implicit(ub, n_kv) is None
    lib3 = _lib_cells(512, 2, 256, True)
    ub = [(0, [0]), (0, [1])]
    _, n_kv = lib3.place(ub)
    assert lib3.implicit(ub, n_kv) is None              # two sequences in the batch


def test_implicit_rule_agrees_with_mask_random():
    """Whenever al_kv_cells_implicit answers yes, the host mask equals the
    implicit rule exactly."""
    rng = np.random.default_rng(9)
    hits = 0
    for trial in range(40):
        lib = _lib_cells(512, 2, 128, True)
        n0 = int(rng.integers(1, 200))
        lib.place(_seq_ub(0, 0, n0))
        if rng.random() < 0.3:
            lib.place(_seq_ub(1, 0, int(rng.integers(1, 20))))
        if rng.random() < 0.3:
            a = int(rng.integers(0, n0))
            lib.seq_rm(0, a, a + int(rng.integers(1, 5)))
        T = int(rng.integers(1, 9))
        ub = _seq_ub(0, n0, T)
        _, n_kv = lib.place(ub)
        got = lib.implicit(ub, n_kv)
        if got is not None:
            hits += 1
            np.testing.assert_array_equal(lib.mask_host(ub, n_kv), O.causal_mask(T, n_kv, got[1], kv_len=got[0]))
    assert hits >= 10
