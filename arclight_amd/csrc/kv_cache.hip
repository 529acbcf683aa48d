// HBM-resident f16 KV cache ("ring") and its cell bookkeeping
// (include/arclight_kv.h).
//
// Bookkeeping restates llm_kv_cells / llm_kv_cache (nnml/include/cgraph.h:
// 612-960, nnml/src/cgraph.cpp:1263-1590) for the flash-attention cache:
// per stream, cell i holds a position (-1 = empty) and a set of sequences;
// new tokens go to the first empty cells found from the stream's head
// (non-contiguous search), overwritten cells purge their sequence's older
// positions, and attention looks at n_kv = PAD(last used cell + 1, n_pad)
// cells. The device keeps a copy of (position, sequence set) per cell,
// updated with only the cells that changed, from which a kernel builds the
// f16 attention mask of set_inputs_attn_mask (cgraph.cpp:1224-1261).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <map>
#include <set>
#include <vector>

#include "../../include/arclight_fattn.h"
#include "../../include/arclight_kv.h"
#include "runtime.hpp"

namespace {

constexpr int kMaxSeq = 64;          // LLM_MAX_SEQ
constexpr int kMaskPad = 64;         // NNML_KQ_MASK_PAD

uint32_t pad_to(uint32_t x, uint32_t n) { return (x + n - 1) / n * n; }

// One stream's cells.
struct StreamCells {
    std::vector<int32_t> pos;                      // -1 = empty
    std::vector<uint64_t> seq;                     // bit s: sequence s
    std::set<uint32_t> used;                       // non-empty cells
    std::map<int32_t, int32_t> seq_pos[kMaxSeq];   // per sequence: position -> cells

    void resize(uint32_t n) {
        pos.assign(n, -1);
        seq.assign(n, 0);
        used.clear();
        for (auto & m : seq_pos) m.clear();
    }
    uint32_t size() const { return (uint32_t) pos.size(); }
    bool empty(uint32_t i) const { return pos[i] == -1; }
    uint32_t used_max_p1() const { return used.empty() ? 0 : *used.rbegin() + 1; }
    void seq_pos_inc(int s, int32_t p) { ++seq_pos[s][p]; }
    void seq_pos_dec(int s, int32_t p) {
        auto it = seq_pos[s].find(p);
        if (--it->second == 0) seq_pos[s].erase(it);
    }
    int32_t seq_pos_min(int s) const { return seq_pos[s].empty() ? -1 : seq_pos[s].begin()->first; }
    void rm(uint32_t i) {
        for (int s = 0; s < kMaxSeq; ++s)
            if (seq[i] >> s & 1) seq_pos_dec(s, pos[i]);
        seq[i] = 0;
        pos[i] = -1;
        used.erase(i);
    }
    // drops sequence s from cell i; true when the cell becomes empty
    bool seq_rm(uint32_t i, int s) {
        seq[i] &= ~(1ull << s);
        seq_pos_dec(s, pos[i]);
        if (seq[i] == 0) {
            pos[i] = -1;
            used.erase(i);
            return true;
        }
        return false;
    }
    void seq_add(uint32_t i, int s) {
        seq[i] |= 1ull << s;
        seq_pos_inc(s, pos[i]);
    }
    void pos_set(uint32_t i, int32_t p) {
        pos[i] = p;
        used.insert(i);
    }
};

int lowest_seq(uint64_t m) { return m ? __builtin_ctzll(m) : -1; }

// (position, sequence set) of a changed cell, for the device copy
struct CellUpdate {
    uint32_t cell;
    int32_t pos;
    uint64_t seq;
};

__global__ void scatter_cells_kernel(const CellUpdate * __restrict__ upd, uint32_t n, int32_t * __restrict__ pos,
                                     uint64_t * __restrict__ seq) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const CellUpdate u = upd[i];
    pos[u.cell] = u.pos;
    seq[u.cell] = u.seq;
}

// Token data of a ubatch on the device.
struct TokenInfo {
    int32_t pos;
    int32_t seq;          // primary sequence
    uint32_t cell0;       // first cell of its stream (stream * kv_size)
    int32_t pad_;
};

// mask[s][row][j] for rows of n_tps tokens padded to `rows`, cells j < n_kv
__global__ void mask_kernel(const int32_t * __restrict__ cpos, const uint64_t * __restrict__ cseq,
                            const TokenInfo * __restrict__ tok, uint32_t n_tps, uint32_t n_kv, char * mask,
                            int64_t nb1, int64_t nb3) {
    const uint32_t j = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t row = blockIdx.y;
    const uint32_t s = blockIdx.z;
    if (j >= n_kv) return;
    bool vis = false;
    if (row < n_tps) {
        const TokenInfo t = tok[s * n_tps + row];
        const uint32_t cell = t.cell0 + j;
        const int32_t p0 = cpos[cell];
        vis = p0 != -1 && (cseq[cell] >> t.seq & 1) && p0 <= t.pos;
    }
    *(uint16_t *) (mask + (int64_t) s * nb3 + (int64_t) row * nb1 + (int64_t) j * 2) = vis ? 0x0000u : 0xfc00u;
}

// Pinned host staging plus a device copy, reused in turn (two slots), each
// slot's reuse waiting for the copy that last read it.
struct Staging {
    void * host[2] = {nullptr, nullptr};
    void * dev[2] = {nullptr, nullptr};
    size_t bytes[2] = {0, 0};
    hipEvent_t done[2] = {nullptr, nullptr};
    int next = 0;

    int get(size_t n, void ** h, void ** d, int * slot) {
        const int k = next;
        next ^= 1;
        if (done[k]) {
            const hipError_t e = hipEventSynchronize(done[k]);
            if (e != hipSuccess) return al_hip_fail(e, "hipEventSynchronize");
        } else {
            const hipError_t e = hipEventCreateWithFlags(&done[k], hipEventDisableTiming);
            if (e != hipSuccess) return al_hip_fail(e, "hipEventCreate");
        }
        if (bytes[k] < n) {
            const size_t sz = std::max<size_t>(n, 64 << 10);
            hipError_t e = hipDeviceSynchronize();                 // the old device copy may still be read
            if (e == hipSuccess && host[k]) e = hipHostFree(host[k]);
            if (e == hipSuccess && dev[k]) e = hipFree(dev[k]);
            host[k] = dev[k] = nullptr;
            bytes[k] = 0;
            if (e == hipSuccess) e = hipHostMalloc(&host[k], sz, hipHostMallocDefault);
            if (e == hipSuccess) e = hipMalloc(&dev[k], sz);
            if (e != hipSuccess) return al_hip_fail(e, "staging allocation");
            bytes[k] = sz;
        }
        *h = host[k];
        *d = dev[k];
        *slot = k;
        return AL_OK;
    }
    int send(int slot, size_t n, hipStream_t stream) {
        hipError_t e = hipMemcpyAsync(dev[slot], host[slot], n, hipMemcpyHostToDevice, stream);
        if (e == hipSuccess) e = hipEventRecord(done[slot], stream);
        return e == hipSuccess ? AL_OK : al_hip_fail(e, "staging copy");
    }
    void release() {
        for (int k = 0; k < 2; ++k) {
            if (done[k]) (void) hipEventSynchronize(done[k]);
            if (host[k]) (void) hipHostFree(host[k]);
            if (dev[k]) (void) hipFree(dev[k]);
            if (done[k]) (void) hipEventDestroy(done[k]);
            host[k] = dev[k] = nullptr;
            done[k] = nullptr;
        }
    }
};

}  // namespace

struct al_kv_cells {
    uint32_t kv_size = 0, n_stream = 1, n_pad = 1;
    std::vector<StreamCells> st;
    std::vector<uint32_t> heads;
    int32_t seq_to_stream[kMaxSeq] = {};

    // cells changed since the device copy was last updated
    std::vector<uint8_t> dirty;
    std::vector<uint32_t> dirty_list;
    // device copy of the cell state
    int32_t * d_pos = nullptr;
    uint64_t * d_seq = nullptr;
    Staging cells_stage, tok_stage;

    void touch(uint32_t strm, uint32_t i) {
        const uint32_t g = strm * kv_size + i;
        if (!dirty[g]) {
            dirty[g] = 1;
            dirty_list.push_back(g);
        }
    }
    void touch_all() {
        for (uint32_t g = 0; g < (uint32_t) dirty.size(); ++g) {
            if (!dirty[g]) {
                dirty[g] = 1;
                dirty_list.push_back(g);
            }
        }
    }
};

struct al_kv_ring {
    al_kv_ring_params prm{};
    al_kv_cells * cells = nullptr;
    std::vector<char *> k, v;          // per layer
    uint64_t row_bytes = 0;            // bytes of one cell (all kv heads)
};

namespace {

// Unique primary sequences in order of first appearance.
std::vector<int> unique_seqs(const al_ubatch * ub) {
    std::vector<int> out;
    for (int i = 0; i < ub->n_tokens; ++i) {
        const int s = lowest_seq(ub->seq_mask[i]);
        if (std::find(out.begin(), out.end(), s) == out.end()) out.push_back(s);
    }
    return out;
}

int check_ubatch(const al_kv_cells * c, const al_ubatch * ub) {
    if (!c || !ub || ub->n_tokens <= 0 || !ub->pos || !ub->seq_mask) return al_fail(AL_ERR_INVALID, "kv: ubatch required");
    for (int i = 0; i < ub->n_tokens; ++i)
        if (ub->seq_mask[i] == 0 || ub->pos[i] < 0) return al_fail(AL_ERR_INVALID, "kv: token %d has no sequence or a negative position", i);
    return AL_OK;
}

// slot_info: per unique sequence (one when unified), its stream and cells
struct Slots {
    std::vector<uint32_t> strm;
    std::vector<std::vector<uint32_t>> idxs;
};

// llm_kv_cache::find_slot with cont = false (cgraph.cpp:1327-1418)
bool find_slot(const al_kv_cells * c, const al_ubatch * ub, Slots * res) {
    uint32_t n_tokens = (uint32_t) ub->n_tokens;
    const std::vector<int> seqs = unique_seqs(ub);
    uint32_t n_seqs = 1;
    if (c->n_stream > 1) {
        if (n_tokens % seqs.size() != 0) return false;
        n_seqs = (uint32_t) seqs.size();
        n_tokens /= n_seqs;
    }
    res->strm.assign(n_seqs, 0);
    res->idxs.assign(n_seqs, {});
    for (uint32_t s = 0; s < n_seqs; ++s) {
        const int seq_id = seqs[s];
        const uint32_t strm = (uint32_t) c->seq_to_stream[seq_id];
        const StreamCells & cells = c->st[strm];
        uint32_t head = c->heads[strm];
        if (head > cells.used.size() + 2 * n_tokens) head = 0;
        if (n_tokens > cells.size()) return false;
        res->strm[s] = strm;
        std::vector<uint32_t> & idxs = res->idxs[s];
        uint32_t n_tested = 0;
        for (;;) {
            if (head + 1 > cells.size()) {
                n_tested += cells.size() - head;
                head = 0;
                continue;
            }
            const uint32_t idx = head++;
            ++n_tested;
            if (cells.empty(idx)) idxs.push_back(idx);
            if (idxs.size() == n_tokens) break;
            if (n_tested >= cells.size()) return false;
        }
    }
    return true;
}

void seq_rm_impl(al_kv_cells * c, int32_t seq_id, int32_t p0, int32_t p1);

// llm_kv_cache::apply_ubatch (cgraph.cpp:1420-1466)
void apply_ubatch(al_kv_cells * c, const Slots & si, const al_ubatch * ub) {
    int32_t seq_pos_max_rm[kMaxSeq];
    for (int s = 0; s < kMaxSeq; ++s) seq_pos_max_rm[s] = -1;
    const uint32_t size = (uint32_t) si.idxs[0].size();
    for (uint32_t s = 0; s < si.strm.size(); ++s) {
        StreamCells & cells = c->st[si.strm[s]];
        for (uint32_t ii = 0; ii < size; ++ii) {
            const uint32_t i = s * size + ii;
            const uint32_t idx = si.idxs[s][ii];
            if (!cells.empty(idx)) {
                const int sq = lowest_seq(cells.seq[idx]);
                seq_pos_max_rm[sq] = std::max(seq_pos_max_rm[sq], cells.pos[idx]);
                cells.rm(idx);
            }
            cells.pos_set(idx, ub->pos[i]);
            for (int sq = 0; sq < kMaxSeq; ++sq)
                if (ub->seq_mask[i] >> sq & 1) cells.seq_add(idx, sq);
            c->touch(si.strm[s], idx);
        }
    }
    for (int sq = 0; sq < kMaxSeq; ++sq) {
        if (seq_pos_max_rm[sq] == -1) continue;
        const StreamCells & cells = c->st[c->seq_to_stream[sq]];
        if (cells.seq_pos_min(sq) <= seq_pos_max_rm[sq]) seq_rm_impl(c, sq, cells.seq_pos_min(sq), seq_pos_max_rm[sq] + 1);
    }
    for (uint32_t s = 0; s < si.strm.size(); ++s) c->heads[si.strm[s]] = si.idxs[s].back() + 1;
}

// llm_kv_cache::seq_rm (cgraph.cpp:1535-1590)
void seq_rm_impl(al_kv_cells * c, int32_t seq_id, int32_t p0, int32_t p1) {
    if (p0 < 0) p0 = 0;
    if (p1 < 0) p1 = INT32_MAX;
    const uint32_t s_begin = seq_id >= 0 ? (uint32_t) c->seq_to_stream[seq_id] : 0;
    const uint32_t s_end = seq_id >= 0 ? s_begin + 1 : c->n_stream;
    for (uint32_t strm = s_begin; strm < s_end; ++strm) {
        StreamCells & cells = c->st[strm];
        uint32_t new_head = cells.size();
        for (uint32_t i = 0; i < cells.size(); ++i) {
            if (!(cells.pos[i] >= p0 && cells.pos[i] < p1)) continue;
            bool freed;
            if (seq_id >= 0) {
                if (!(cells.seq[i] >> seq_id & 1)) continue;
                freed = cells.seq_rm(i, seq_id);
            } else {
                cells.rm(i);
                freed = true;
            }
            c->touch(strm, i);
            if (freed && new_head == cells.size()) new_head = i;
        }
        if (new_head != cells.size() && new_head < c->heads[strm]) c->heads[strm] = new_head;
    }
}

}  // namespace

extern "C" int al_kv_cells_create(uint32_t kv_size, uint32_t n_seq_max, uint32_t n_pad, int32_t unified, al_kv_cells ** out) {
    if (!out) return al_fail(AL_ERR_INVALID, "kv: out required");
    if (kv_size == 0 || n_pad == 0 || kv_size % n_pad != 0)
        return al_fail(AL_ERR_INVALID, "kv: kv_size %u must be a positive multiple of n_pad %u (cgraph.cpp:929)", kv_size, n_pad);
    if (n_seq_max == 0 || n_seq_max > (uint32_t) kMaxSeq) return al_fail(AL_ERR_INVALID, "kv: n_seq_max %u not in 1..64", n_seq_max);
    al_kv_cells * c = new al_kv_cells;
    c->kv_size = kv_size;
    c->n_pad = n_pad;
    c->n_stream = unified ? 1 : n_seq_max;
    c->st.resize(c->n_stream);
    for (auto & s : c->st) s.resize(kv_size);
    c->heads.assign(c->n_stream, 0);
    for (int s = 0; s < kMaxSeq; ++s) c->seq_to_stream[s] = (c->n_stream > 1 && (uint32_t) s < c->n_stream) ? s : 0;
    c->dirty.assign((size_t) c->n_stream * kv_size, 0);
    c->touch_all();
    *out = c;
    return AL_OK;
}

extern "C" int al_kv_cells_destroy(al_kv_cells * c) {
    if (!c) return AL_OK;
    c->cells_stage.release();
    c->tok_stage.release();
    if (c->d_pos) (void) hipFree(c->d_pos);
    if (c->d_seq) (void) hipFree(c->d_seq);
    delete c;
    return AL_OK;
}

extern "C" int al_kv_cells_clear(al_kv_cells * c) {
    if (!c) return al_fail(AL_ERR_INVALID, "kv: cells required");
    for (auto & s : c->st) s.resize(c->kv_size);
    std::fill(c->heads.begin(), c->heads.end(), 0u);
    c->touch_all();
    return AL_OK;
}

extern "C" int al_kv_cells_place(al_kv_cells * c, const al_ubatch * ub, int64_t * rows, uint32_t * n_kv, uint32_t * s0,
                                 uint32_t * ns) {
    int rc = check_ubatch(c, ub);
    if (rc != AL_OK) return rc;
    if (!rows || !n_kv) return al_fail(AL_ERR_INVALID, "kv: rows and n_kv required");
    Slots si;
    if (!find_slot(c, ub, &si)) return al_fail(AL_ERR_INVALID, "kv: no room for %d tokens", ub->n_tokens);
    apply_ubatch(c, si, ub);
    uint32_t r = 0;
    int64_t k = 0;
    for (uint32_t s = 0; s < si.strm.size(); ++s) {
        for (uint32_t idx : si.idxs[s]) rows[k++] = (int64_t) si.strm[s] * c->kv_size + idx;
        const StreamCells & cells = c->st[si.strm[s]];
        r = std::max(std::min(cells.size(), std::max(c->n_pad, pad_to(cells.used_max_p1(), c->n_pad))), r);
    }
    *n_kv = r;
    const uint32_t lo = *std::min_element(si.strm.begin(), si.strm.end());
    const uint32_t hi = *std::max_element(si.strm.begin(), si.strm.end());
    if (s0) *s0 = lo;
    if (ns) *ns = hi - lo + 1;
    return AL_OK;
}

extern "C" int al_kv_cells_seq_rm(al_kv_cells * c, int32_t seq_id, int32_t p0, int32_t p1) {
    if (!c) return al_fail(AL_ERR_INVALID, "kv: cells required");
    if (seq_id >= kMaxSeq || seq_id < -1) return al_fail(AL_ERR_INVALID, "kv: sequence %d", seq_id);
    seq_rm_impl(c, seq_id, p0, p1);
    return AL_OK;
}

extern "C" int al_kv_cells_state(const al_kv_cells * c, int32_t * pos, uint64_t * seq_mask) {
    if (!c) return al_fail(AL_ERR_INVALID, "kv: cells required");
    for (uint32_t s = 0; s < c->n_stream; ++s) {
        if (pos) std::copy(c->st[s].pos.begin(), c->st[s].pos.end(), pos + (size_t) s * c->kv_size);
        if (seq_mask) std::copy(c->st[s].seq.begin(), c->st[s].seq.end(), seq_mask + (size_t) s * c->kv_size);
    }
    return AL_OK;
}

static int mask_shape(const al_kv_cells * c, const al_ubatch * ub, uint32_t n_kv, uint32_t n_stream_ub, uint32_t * n_tps) {
    if (n_stream_ub == 0 || ub->n_tokens % n_stream_ub != 0)
        return al_fail(AL_ERR_INVALID, "kv: %d tokens do not split into %u streams (cgraph.cpp:1231)", ub->n_tokens, n_stream_ub);
    if (n_kv == 0 || n_kv > c->kv_size) return al_fail(AL_ERR_INVALID, "kv: n_kv %u not in 1..%u", n_kv, c->kv_size);
    *n_tps = (uint32_t) ub->n_tokens / n_stream_ub;
    return AL_OK;
}

extern "C" int al_kv_cells_mask_host(const al_kv_cells * c, const al_ubatch * ub, uint32_t n_kv, uint32_t n_stream_ub,
                                     uint16_t * mask) {
    int rc = check_ubatch(c, ub);
    if (rc != AL_OK) return rc;
    uint32_t n_tps = 0;
    rc = mask_shape(c, ub, n_kv, n_stream_ub, &n_tps);
    if (rc != AL_OK) return rc;
    if (!mask) return al_fail(AL_ERR_INVALID, "kv: mask required");
    const uint32_t rows = pad_to(n_tps, kMaskPad);
    std::fill(mask, mask + (size_t) n_stream_ub * rows * n_kv, (uint16_t) 0xfc00u);
    for (uint32_t s = 0; s < n_stream_ub; ++s) {
        for (uint32_t ii = 0; ii < n_tps; ++ii) {
            const uint32_t i = s * n_tps + ii;
            const int seq_id = lowest_seq(ub->seq_mask[i]);
            const StreamCells & cells = c->st[c->seq_to_stream[seq_id]];
            uint16_t * row = mask + ((size_t) s * rows + ii) * n_kv;
            for (uint32_t j = 0; j < n_kv; ++j) {
                if (cells.empty(j) || !(cells.seq[j] >> seq_id & 1) || cells.pos[j] > ub->pos[i]) continue;
                row[j] = 0;
            }
        }
    }
    return AL_OK;
}

extern "C" int al_kv_cells_mask_device(al_kv_cells * c, const al_ubatch * ub, uint32_t n_kv, uint32_t n_stream_ub,
                                       const al_tensor * mask, void * stream_) {
    int rc = check_ubatch(c, ub);
    if (rc != AL_OK) return rc;
    uint32_t n_tps = 0;
    rc = mask_shape(c, ub, n_kv, n_stream_ub, &n_tps);
    if (rc != AL_OK) return rc;
    const uint32_t rows = pad_to(n_tps, kMaskPad);
    if (!mask || !mask->data || mask->type != AL_TYPE_F16 || mask->ne[0] != n_kv || mask->ne[1] != rows ||
        mask->ne[2] != 1 || mask->ne[3] != n_stream_ub || mask->nb[0] != 2)
        return al_fail(AL_ERR_INVALID, "kv: mask must be f16 [%u, %u, 1, %u] with contiguous rows", n_kv, rows, n_stream_ub);
    hipStream_t stream = (hipStream_t) stream_;
    const size_t n_cells = (size_t) c->n_stream * c->kv_size;
    if (!c->d_pos) {
        hipError_t e = hipMalloc(&c->d_pos, n_cells * sizeof(int32_t));
        if (e == hipSuccess) e = hipMalloc(&c->d_seq, n_cells * sizeof(uint64_t));
        if (e != hipSuccess) return al_hip_fail(e, "kv: device cell state");
    }
    // the cells that changed since the last call
    if (!c->dirty_list.empty()) {
        const size_t n = c->dirty_list.size();
        void * h = nullptr;
        void * d = nullptr;
        int slot = 0;
        rc = c->cells_stage.get(n * sizeof(CellUpdate), &h, &d, &slot);
        if (rc != AL_OK) return rc;
        CellUpdate * u = (CellUpdate *) h;
        for (size_t k = 0; k < n; ++k) {
            const uint32_t g = c->dirty_list[k];
            const StreamCells & cells = c->st[g / c->kv_size];
            u[k] = CellUpdate{g, cells.pos[g % c->kv_size], cells.seq[g % c->kv_size]};
            c->dirty[g] = 0;
        }
        c->dirty_list.clear();
        rc = c->cells_stage.send(slot, n * sizeof(CellUpdate), stream);
        if (rc != AL_OK) return rc;
        hipLaunchKernelGGL(scatter_cells_kernel, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, stream,
                           (const CellUpdate *) d, (uint32_t) n, c->d_pos, c->d_seq);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return al_hip_fail(e, "kv: cell update launch");
    }
    // the tokens
    void * h = nullptr;
    void * d = nullptr;
    int slot = 0;
    rc = c->tok_stage.get((size_t) ub->n_tokens * sizeof(TokenInfo), &h, &d, &slot);
    if (rc != AL_OK) return rc;
    TokenInfo * t = (TokenInfo *) h;
    for (int i = 0; i < ub->n_tokens; ++i) {
        const int sq = lowest_seq(ub->seq_mask[i]);
        t[i] = TokenInfo{ub->pos[i], sq, (uint32_t) c->seq_to_stream[sq] * c->kv_size, 0};
    }
    rc = c->tok_stage.send(slot, (size_t) ub->n_tokens * sizeof(TokenInfo), stream);
    if (rc != AL_OK) return rc;
    hipLaunchKernelGGL(mask_kernel, dim3((n_kv + 255) / 256, rows, n_stream_ub), dim3(256), 0, stream, c->d_pos, c->d_seq,
                       (const TokenInfo *) d, n_tps, n_kv, (char *) mask->data, (int64_t) mask->nb[1], (int64_t) mask->nb[3]);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? AL_OK : al_hip_fail(e, "kv: mask launch");
}

extern "C" int al_kv_cells_implicit(const al_kv_cells * c, const al_ubatch * ub, uint32_t n_kv, int64_t * kv_len,
                                    int64_t * causal_pos0) {
    if (check_ubatch(c, ub) != AL_OK) return 0;
    if (!kv_len || !causal_pos0 || n_kv > c->kv_size) return 0;
    const uint64_t m0 = ub->seq_mask[0];
    const int sq = lowest_seq(m0);
    for (int i = 0; i < ub->n_tokens; ++i)
        if (ub->seq_mask[i] != m0 || ub->pos[i] != ub->pos[0] + i) return 0;
    const StreamCells & cells = c->st[c->seq_to_stream[sq]];
    // cells 0..L-1: the sequence at positions 0..L-1; after that nothing of
    // the sequence that a token could see
    uint32_t L = 0;
    while (L < n_kv && !cells.empty(L) && (cells.seq[L] >> sq & 1) && cells.pos[L] == (int32_t) L) ++L;
    const int32_t last_pos = ub->pos[ub->n_tokens - 1];
    for (uint32_t j = L; j < n_kv; ++j)
        if (!cells.empty(j) && (cells.seq[j] >> sq & 1) && cells.pos[j] <= last_pos) return 0;
    *kv_len = L;
    *causal_pos0 = ub->pos[0];
    return 1;
}

// ---------------------------------------------------------------------------
// the ring
// ---------------------------------------------------------------------------

extern "C" int al_kv_ring_create(const al_kv_ring_params * prm, al_kv_ring ** out) {
    if (!prm || !out) return al_fail(AL_ERR_INVALID, "kv ring: params and out required");
    if (prm->n_layer == 0 || prm->n_head_kv == 0 || prm->head_dim == 0 || prm->head_dim % 8 != 0)
        return al_fail(AL_ERR_INVALID, "kv ring: layers, kv heads and head_dim (multiple of 8) required");
    al_kv_cells * cells = nullptr;
    int rc = al_kv_cells_create(prm->kv_size, prm->n_seq_max, prm->n_pad, prm->unified, &cells);
    if (rc != AL_OK) return rc;
    al_kv_ring * r = new al_kv_ring;
    r->prm = *prm;
    r->cells = cells;
    r->row_bytes = (uint64_t) prm->n_head_kv * prm->head_dim * 2;
    const uint64_t bytes = r->row_bytes * prm->kv_size * cells->n_stream;
    r->k.assign(prm->n_layer, nullptr);
    r->v.assign(prm->n_layer, nullptr);
    for (uint32_t il = 0; il < prm->n_layer; ++il) {
        hipError_t e = hipMalloc((void **) &r->k[il], bytes);
        if (e == hipSuccess) e = hipMalloc((void **) &r->v[il], bytes);
        if (e == hipSuccess) e = hipMemset(r->k[il], 0, bytes);
        if (e == hipSuccess) e = hipMemset(r->v[il], 0, bytes);
        if (e != hipSuccess) {
            al_kv_ring_destroy(r);
            return al_fail(AL_ERR_HIP, "kv ring: layer %u allocation of 2 x %llu bytes: %s", il, (unsigned long long) bytes,
                           hipGetErrorString(e));
        }
    }
    const hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        al_kv_ring_destroy(r);
        return al_hip_fail(e, "kv ring: zero fill");
    }
    *out = r;
    return AL_OK;
}

extern "C" int al_kv_ring_destroy(al_kv_ring * r) {
    if (!r) return AL_OK;
    (void) hipDeviceSynchronize();
    for (char * p : r->k) if (p) (void) hipFree(p);
    for (char * p : r->v) if (p) (void) hipFree(p);
    al_kv_cells_destroy(r->cells);
    delete r;
    return AL_OK;
}

extern "C" al_kv_cells * al_kv_ring_cells(al_kv_ring * r) { return r ? r->cells : nullptr; }

static int ring_view(const al_kv_ring * r, const std::vector<char *> & buf, uint32_t il, uint32_t n_kv, uint32_t s0,
                     uint32_t ns, al_tensor * t) {
    if (!r || !t || il >= r->prm.n_layer) return al_fail(AL_ERR_INVALID, "kv ring: layer %u out of range", il);
    if (n_kv == 0 || n_kv > r->prm.kv_size) return al_fail(AL_ERR_INVALID, "kv ring: n_kv %u not in 1..%u", n_kv, r->prm.kv_size);
    if (ns == 0 || s0 >= r->cells->n_stream || ns > r->cells->n_stream - s0)
        return al_fail(AL_ERR_INVALID, "kv ring: streams %u..%u of %u", s0, s0 + ns - 1, r->cells->n_stream);
    memset(t, 0, sizeof(*t));
    t->data = buf[il] + (uint64_t) s0 * r->row_bytes * r->prm.kv_size;
    t->type = AL_TYPE_F16;
    t->ne[0] = r->prm.head_dim;
    t->ne[1] = n_kv;
    t->ne[2] = r->prm.n_head_kv;
    t->ne[3] = ns;
    t->nb[0] = 2;
    t->nb[1] = r->row_bytes;
    t->nb[2] = (uint64_t) r->prm.head_dim * 2;
    t->nb[3] = r->row_bytes * r->prm.kv_size;
    return AL_OK;
}

extern "C" int al_kv_ring_view_k(const al_kv_ring * r, uint32_t il, uint32_t n_kv, uint32_t s0, uint32_t ns, al_tensor * k) {
    if (!r) return al_fail(AL_ERR_INVALID, "kv ring: ring required");
    return ring_view(r, r->k, il, n_kv, s0, ns, k);
}

extern "C" int al_kv_ring_view_v(const al_kv_ring * r, uint32_t il, uint32_t n_kv, uint32_t s0, uint32_t ns, al_tensor * v) {
    if (!r) return al_fail(AL_ERR_INVALID, "kv ring: ring required");
    return ring_view(r, r->v, il, n_kv, s0, ns, v);
}

extern "C" int al_kv_ring_write(al_kv_ring * r, uint32_t il, const al_tensor * k_cur, const al_tensor * v_cur,
                                const al_tensor * rows, void * stream) {
    if (!r || il >= r->prm.n_layer) return al_fail(AL_ERR_INVALID, "kv ring: layer %u out of range", il);
    if (!k_cur || !v_cur || !rows) return al_fail(AL_ERR_INVALID, "kv ring: k, v and rows required");
    // the whole layer cache as rows of one cell (all kv heads), streams merged
    al_tensor dst;
    memset(&dst, 0, sizeof(dst));
    dst.type = AL_TYPE_F16;
    dst.ne[0] = (int64_t) r->prm.head_dim * r->prm.n_head_kv;
    dst.ne[1] = (int64_t) r->prm.kv_size * r->cells->n_stream;
    dst.ne[2] = 1;
    dst.ne[3] = 1;
    dst.nb[0] = 2;
    dst.nb[1] = r->row_bytes;
    dst.nb[2] = dst.nb[3] = r->row_bytes * dst.ne[1];
    dst.data = r->k[il];
    int rc = al_set_rows_f32_f16(&dst, k_cur, rows, stream);
    if (rc != AL_OK) return rc;
    dst.data = r->v[il];
    return al_set_rows_f32_f16(&dst, v_cur, rows, stream);
}
