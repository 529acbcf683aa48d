"""Oracle of the KV-cache cell bookkeeping and attention mask (test
infrastructure only: the tests compare against it, nothing ships it).

A plain-Python restatement of ArcLight's llm_kv_cells / llm_kv_cache logic
for the f16 flash-attention cache (FA on: V not transposed):
  - llm_kv_cells state and operations   nnml/include/cgraph.h:612-960
  - find_slot (non-contiguous search)   nnml/src/cgraph.cpp:1327-1418
  - apply_ubatch                        nnml/src/cgraph.cpp:1420-1466
  - get_n_kv                            nnml/src/cgraph.cpp:1472-1479
  - seq_rm                              nnml/src/cgraph.cpp:1535-1590
  - k/v row indices (set_inputs_attn_kidx)  nnml/src/cgraph.cpp:1182-1194
  - set_inputs_attn_mask + f16 cast     nnml/src/cgraph.cpp:1224-1261

A ubatch is (pos[i], seqs[i]) per token, seqs[i] a list of sequence ids
whose first entry is the token's primary sequence (ubatch->seq_id[i][0]).
"""
import numpy as np

MAX_SEQ = 64            # LLM_MAX_SEQ, nnml/include/cgraph.h:26
KQ_MASK_PAD = 64        # NNML_KQ_MASK_PAD, nnml/include/cgraph.h:28


def pad(x, n):
    return (x + n - 1) // n * n


class Cells:
    """One stream's cells (nnml/include/cgraph.h:612-960)."""

    def __init__(self, n):
        self.pos = [-1] * n
        self.seq = [set() for _ in range(n)]
        self.used = set()
        self.seq_pos = [dict() for _ in range(MAX_SEQ)]     # position -> count

    def size(self):
        return len(self.pos)

    def is_empty(self, i):
        return self.pos[i] == -1

    def used_max_p1(self):
        return max(self.used) + 1 if self.used else 0

    def _seq_pos_inc(self, s, p):
        self.seq_pos[s][p] = self.seq_pos[s].get(p, 0) + 1

    def _seq_pos_dec(self, s, p):
        self.seq_pos[s][p] -= 1
        if self.seq_pos[s][p] == 0:
            del self.seq_pos[s][p]

    def rm(self, i):
        for s in self.seq[i]:
            self._seq_pos_dec(s, self.pos[i])
        self.seq[i] = set()
        self.pos[i] = -1
        self.used.discard(i)

    def seq_rm(self, i, s):
        """Drops sequence s from cell i; True if the cell becomes empty."""
        self.seq[i].discard(s)
        self._seq_pos_dec(s, self.pos[i])
        if not self.seq[i]:
            self.pos[i] = -1
            self.used.discard(i)
            return True
        return False

    def seq_add(self, i, s):
        self.seq[i].add(s)
        self._seq_pos_inc(s, self.pos[i])

    def pos_set(self, i, p):
        self.pos[i] = p
        self.used.add(i)

    def seq_pos_min(self, s):
        return min(self.seq_pos[s]) if self.seq_pos[s] else -1


class KvCache:
    def __init__(self, kv_size, n_seq_max=1, n_pad=256, unified=True):
        assert kv_size % n_pad == 0
        self.kv_size = kv_size
        self.n_pad = n_pad
        self.n_stream = 1 if unified else n_seq_max
        self.cells = [Cells(kv_size) for _ in range(self.n_stream)]
        self.heads = [0] * self.n_stream
        self.seq_to_stream = [0] * MAX_SEQ
        if self.n_stream > 1:
            self.seq_to_stream = list(range(self.n_stream)) + [0] * (MAX_SEQ - self.n_stream)

    @staticmethod
    def _unique_seqs(ub):
        out = []
        for _, seqs in ub:
            if seqs[0] not in out:
                out.append(seqs[0])
        return out

    def find_slot(self, ub):
        """Non-contiguous first-fit search from each stream's head; returns
        [(stream, [cell idx ...])] per unique sequence, or None."""
        n_tokens = len(ub)
        seqs_unq = self._unique_seqs(ub)
        n_seqs = 1
        if self.n_stream > 1:
            assert n_tokens % len(seqs_unq) == 0
            n_seqs = len(seqs_unq)
            n_tokens //= n_seqs
        res = []
        for s in range(n_seqs):
            seq_id = seqs_unq[s]
            strm = self.seq_to_stream[seq_id]
            cells = self.cells[strm]
            head = self.heads[strm]
            if head > len(cells.used) + 2 * n_tokens:
                head = 0
            if n_tokens > cells.size():
                raise ValueError("n_tokens > cache size")
            idxs = []
            n_tested = 0
            while True:
                if head + 1 > cells.size():
                    n_tested += cells.size() - head
                    head = 0
                    continue
                idx = head
                head += 1
                n_tested += 1
                if cells.is_empty(idx):
                    idxs.append(idx)
                if len(idxs) == n_tokens:
                    break
                if n_tested >= cells.size():
                    return None
            res.append((strm, idxs))
        return res

    def apply(self, sinfo, ub):
        seq_pos_max_rm = [-1] * MAX_SEQ
        size = len(sinfo[0][1])
        for s, (strm, idxs) in enumerate(sinfo):
            cells = self.cells[strm]
            for ii, idx in enumerate(idxs):
                i = s * size + ii
                if not cells.is_empty(idx):
                    (sq,) = tuple(cells.seq[idx])
                    seq_pos_max_rm[sq] = max(seq_pos_max_rm[sq], cells.pos[idx])
                    cells.rm(idx)
                cells.pos_set(idx, ub[i][0])
                for sq in ub[i][1]:
                    cells.seq_add(idx, sq)
        for sq in range(MAX_SEQ):
            if seq_pos_max_rm[sq] == -1:
                continue
            cells = self.cells[self.seq_to_stream[sq]]
            if cells.seq_pos_min(sq) <= seq_pos_max_rm[sq]:
                self.seq_rm(sq, cells.seq_pos_min(sq), seq_pos_max_rm[sq] + 1)
        for strm, idxs in sinfo:
            self.heads[strm] = idxs[-1] + 1

    def n_kv(self, sinfo):
        r = 0
        for strm, _ in sinfo:
            cells = self.cells[strm]
            r = max(min(cells.size(), max(self.n_pad, pad(cells.used_max_p1(), self.n_pad))), r)
        return r

    def place(self, ub):
        """find_slot + apply; returns (row indices stream*kv_size + cell, n_kv)."""
        sinfo = self.find_slot(ub)
        if sinfo is None:
            return None
        self.apply(sinfo, ub)
        rows = [strm * self.kv_size + idx for strm, idxs in sinfo for idx in idxs]
        return np.array(rows, dtype=np.int64), self.n_kv(sinfo)

    def seq_rm(self, seq_id, p0, p1):
        if p0 < 0:
            p0 = 0
        if p1 < 0:
            p1 = 2 ** 31 - 1
        if seq_id >= 0:
            strm = self.seq_to_stream[seq_id]
            cells = self.cells[strm]
            new_head = cells.size()
            for i in range(cells.size()):
                if not (p0 <= cells.pos[i] < p1):
                    continue
                if seq_id in cells.seq[i] and cells.seq_rm(i, seq_id):
                    if new_head == cells.size():
                        new_head = i
            if new_head != cells.size() and new_head < self.heads[strm]:
                self.heads[strm] = new_head
        else:
            for strm in range(self.n_stream):
                cells = self.cells[strm]
                new_head = cells.size()
                for i in range(cells.size()):
                    if not (p0 <= cells.pos[i] < p1):
                        continue
                    cells.rm(i)
                    if new_head == cells.size():
                        new_head = i
                if new_head != cells.size() and new_head < self.heads[strm]:
                    self.heads[strm] = new_head
        return True

    def mask(self, ub, n_kv, n_stream_ub=1):
        """f16 mask [n_stream_ub, 1, PAD(n_tps, 64), n_kv] of 0 / -inf."""
        n_tokens = len(ub)
        assert n_tokens % n_stream_ub == 0
        n_tps = n_tokens // n_stream_ub
        rows = pad(n_tps, KQ_MASK_PAD)
        m = np.full((n_stream_ub, 1, rows, n_kv), -np.inf, dtype=np.float32)
        for s in range(n_stream_ub):
            for ii in range(n_tps):
                p1, seqs = ub[s * n_tps + ii]
                seq_id = seqs[0]
                cells = self.cells[self.seq_to_stream[seq_id]]
                for j in range(n_kv):
                    if cells.is_empty(j) or seq_id not in cells.seq[j]:
                        continue
                    if cells.pos[j] > p1:
                        continue
                    m[s, 0, ii, j] = 0.0
        return m.astype(np.float16)
