// Prefill (and long speculative-verify) attention for gfx950: many query rows
// per kv head, masking given by the length / causal rule (kv_len,
// causal_pos0) and by an explicit f16 mask tensor: a mask whose rows are
// runs of zeros followed by -inf becomes per-row extents, any other is
// added value by value.
// Semantics as nnml_compute_forward_flash_attn_ext_f16
// (nnml/src/ops/arm/arm.cpp:2196-2433), numerics as fattn_splitkv.hip.
//
// Work decomposition. One workgroup per CU: 4 computing wavefronts, one
// per SIMD, each holding 32 query rows of one kv-head group (row r ->
// token r / G, head kvh*G + r % G; one 32x32 MFMA block), and 4 producer
// wavefronts (one per SIMD too) that only move K/V tiles into LDS: an
// LDS-DMA instruction stalls the wave that issues it for tens of cycles, so
// the computing waves issue none. RG of the computing waves (the row
// groups) hold different rows and walk the same 64-cell tiles, sharing each
// tile through LDS; the other 4 / RG do the same for another cell split
// (tiles s, s + SP, ...), and the splits merge their softmax states through
// LDS at the end. RG = 4 (128 rows, one split) halves the L2 -> LDS traffic
// per MFMA; RG = 2 (64 rows, two splits) gives twice the workgroups for
// calls with few rows. When even that does not fill the device, n_split
// workgroups share a row tile and the last to arrive combines their merge
// records (the split-KV kernel's record / counter scheme).
//
// Per computing wave and tile (f16 MFMA 32x32x16, f32 accumulation):
//   S^T[64 cells x 32 rows]  = K Q^T     16 MFMA (two 32-cell blocks, 8 k-steps)
//   O^T[128 dims x 32 rows] += V^T P^T   16 MFMA (four 32-dim blocks, 4 k-steps)
// The S^T accumulator layout (lane l: row l % 32, cells (v % 4) + 8 (v / 4)
// + 4 (l / 32) of register v) is the P^T operand layout of PV when the k
// slots of each 16-cell step are ordered accordingly, so P^T is S^T in
// place; V^T operands follow the same order, read by ds_read_b64_tr_b16.
//
// Software pipeline: iteration i runs QK^T of tile i + 1 on the matrix
// cores while the vector ALU turns the scores of tile i into probabilities,
// then PV of tile i; the slots of both phases are ordered explicitly (LDS
// reads prefetched one or two slots ahead, exponentials pinned to their
// slot), so the two units overlap within each wave. Softmax: p = exp2(s c -
// b) with c = scale log2(e) and b the row's reference max in log2 units;
// without softcap the fast loop has the MFMAs produce s c - b directly (the
// query rows scaled by c before their f16 rounding, the score accumulators
// started from -b), with softcap or a general mask p = exp2(s' c - m c)
// from the scores as they are. Row sums accumulate by v_dot2 of the f16 P
// with ones, and the reference max moves lazily (only when a tile exceeds
// it by more than kTau in natural units) on a cold path outside the fast
// loop, so the O accumulators stay in the matrix cores' registers there.
//
// Memory path. K and V tiles go HBM/L2 -> LDS by LDS-DMA (buffer_load ...
// lds), each producer moving the share of its computing partner (1 / RG of
// every tile of its split), into per-split rings of NK K buffers and NV V
// buffers (RG = 2: 2 and 3; RG = 4: 4 and 6; 160 KiB in all). K(i + NK) is
// issued once iteration i starts (its buffer held K(i), read in iteration
// i - 1) and V(i + NV - 1) likewise, so every tile has one or more
// iterations to land; one workgroup barrier per iteration publishes them.
// Tiles are cell-major, 256 bytes per cell, with 16-byte granules permuted
// within a cell so that the operand reads are free of bank conflicts: K
// granule j of cell c at slot j ^ (c & 15) (a K operand read covers 32
// cells x 16 bytes), V granule j at slot j ^ 4 (c & 3) (a transposing V
// read covers 4 cells x 64 bytes). The K/V views end at the workgroup's
// last visible cell, so cells that no row sees read as zeros (unwritten
// cache cells may hold non-finite values). The query rows go straight
// into the computing waves' registers; the output rows leave through LDS,
// 16 bytes per lane over whole rows.

#include <type_traits>

#include "fattn_prefill_common.hpp"

namespace {

using namespace fattn_prefill;

constexpr int kTC = 64;                          // cells per tile
constexpr int kTileBytes = kTC * 256;            // one tile of K or of V (16 KiB)
static_assert(kLds == 10 * kTileBytes, "10 tiles fill the LDS");
static_assert(80 * 1024 + 128 * 512 + 128 * 8 <= kLds - 16 && 64 * kFattnRecordStride * 4 <= 80 * 1024,
              "output staging fits past the merge records");

// Shape of a workgroup with RG row groups: SP cell splits; per split a ring
// of NK K buffers and NV V buffers; PER LDS-DMA instructions per wave and
// tile (each wave of a split moves 1 / RG of every tile).
template <int RG>
struct Shape {
    static constexpr int SP = kWaves / RG;
    static constexpr int ROWS = 32 * RG;
    static constexpr int NK = RG == 4 ? 4 : 2;
    static constexpr int NV = RG == 4 ? 6 : 3;
    static constexpr int RING = (NK + NV) * kTileBytes;
    static constexpr int PER = kTileBytes / 1024 / RG;
    static_assert(SP * RING == kLds, "the rings fill the LDS");
    static_assert(NV > NK && PER % 4 == 0, "V runs further ahead than K; whole DMA instructions per slot");
};

// A pointer the wave holds alike in every lane, kept in SGPRs.
__device__ __forceinline__ const char * uniform_ptr(const char * q) {
    const uint64_t a = (uint64_t) q;
    const uint64_t lo = (uint32_t) __builtin_amdgcn_readfirstlane((int) (uint32_t) a);
    const uint64_t hi = (uint32_t) __builtin_amdgcn_readfirstlane((int) (uint32_t) (a >> 32));
    return (const char *) (lo | (hi << 32));
}

// raw_desc of values the wave holds alike in every lane, kept in SGPRs
__device__ __forceinline__ int4v uniform_desc(const char * base, const uint32_t bytes) {
    const uint64_t a = (uint64_t) base;
    return int4v{__builtin_amdgcn_readfirstlane((int) (uint32_t) a), __builtin_amdgcn_readfirstlane((int) (uint32_t) (a >> 32)),
                 __builtin_amdgcn_readfirstlane((int) bytes), 0x00020000};
}

template <int RG, bool SOFTCAP, bool MASK>
__global__ __launch_bounds__(2 * kWaves * 64) void fattn_prefill_kernel(const FattnParams p) {
    using S = Shape<RG>;
    constexpr int ROWS = S::ROWS, NK = S::NK, NV = S::NV, PER = S::PER;
    __shared__ __attribute__((aligned(1024))) char lds[kLds];
    prefetch_params(p);

    // Waves 0..3 compute (one per SIMD); waves 4..7 (one per SIMD too) only
    // move K/V tiles and query rows into LDS: an LDS-DMA instruction stalls
    // the wave that issues it, so the computing waves issue none. Wave w and
    // its producer w + 4 share the role w & 3: row group role % RG of cell
    // split role / RG. Every barrier below is reached by all eight waves.
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool producer = wave >= kWaves;
    const int role = wave & (kWaves - 1);
    const int rg = role % RG;                    // row group: rows 32 rg .. 32 rg + 31 of the tile
    const int si = role / RG;                    // cell split within the workgroup
    const int h = lane >> 5;                     // half of the wave (k slots 8h .. 8h + 7)
    const int lr = lane & 31;                    // this lane's row within the wave's 32

    // Grid (kv head, workgroup split, row tile + stream): kv head fastest
    // (XCD affinity: with Hkv = 8 each head's K/V stays in one XCD's L2),
    // row tiles longest first with a causal mask. No integer division on
    // the way to the first loads except for several streams.
    const int kvh = blockIdx.x;
    const int sx = blockIdx.y;                   // workgroup split of the row tile
    const int z = blockIdx.z;
    const int zt = p.B == 1 ? z : __builtin_amdgcn_readfirstlane(z % p.n_row_tiles);
    const int b = p.B == 1 ? 0 : __builtin_amdgcn_readfirstlane(z / p.n_row_tiles);
    const int rt = p.causal_pos0 >= 0 ? p.n_row_tiles - 1 - zt : zt;
    const int row0 = rt * ROWS;
    const int rows_here = min(ROWS, p.R - row0);
    // row r of the kv head: token r / G, head kvh G + r % G
    auto tok_of = [&](const int r) { return p.G == 1 ? r : (int) __umulhi((uint32_t) r, p.g_magic); };

    // An explicit mask (f16 rows of n_kv cells, 16-byte aligned) is read
    // here first: every mask row that the tile's rows use (one per token
    // when the mask is shared by the heads, else one per row) is scanned by
    // one wavefront, 16 bytes per lane and load, for its last cell that is
    // not -inf (the row's visible extent) and for whether it is a run of
    // zeros followed by -inf. When every row is, the mask is exactly the
    // extent and the tiles run as with the length rule; otherwise the whole
    // workgroup adds slope * mask to its scores tile by tile (general mode).
    // The results sit in a V buffer that no tile uses before the loop.
    constexpr bool has_mask = MASK;           // the launch picks MASK = (p.mask != nullptr)
    const int t0 = tok_of(row0);
    const int n_units = !has_mask ? 0 : p.m_ne2 == 1 ? tok_of(row0 + rows_here - 1) - t0 + 1 : rows_here;
    int * mtab = (int *) (lds + (RG == 4 ? NK + NV - 1 : NK + NV - 1) * kTileBytes);   // V buffer NV - 1 of split 0
    auto mask_row = [&](const int r) {                    // mask row of tile row r (global row row0 + r)
        const int rg_ = row0 + r, tok = tok_of(rg_);
        const int hq = kvh * p.G + (rg_ - tok * p.G);
        return p.mask + (int64_t) tok * p.m_nb1 + (int64_t) (p.m_ne2 == 1 ? 0 : hq % p.m_ne2) * p.m_nb2 +
               (int64_t) (p.m_ne3 == 1 ? 0 : b % p.m_ne3) * p.m_nb3;
    };
    if constexpr (has_mask) {
        for (int u = wave; u < n_units; u += 2 * kWaves) {
            const int r_u = p.m_ne2 == 1 ? max(0, (t0 + u) * p.G - row0) : u;   // a tile row of the unit
            const char * rowp = mask_row(r_u);
            int last_fin = -1, last0 = -1, first_inf = INT32_MAX, bad = 0;
            auto classify = [&](const uint32_t hb, const int c) {
                if (hb != 0xfc00u) last_fin = max(last_fin, c);
                if ((hb & 0x7fffu) == 0) last0 = max(last0, c);
                else if (hb == 0xfc00u) first_inf = min(first_inf, c);
                else bad = 1;
            };
            const int n8 = p.n_kv >> 3;
            for (int j0 = 0; j0 < n8; j0 += 8 * 64) {
                uint4 w[8];
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const int j = j0 + 64 * q + lane;
                    w[q] = j < n8 ? *(const uint4 *) (rowp + 16 * (int64_t) j)
                                  : uint4{0xfc00fc00u, 0xfc00fc00u, 0xfc00fc00u, 0xfc00fc00u};
                }
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const int j = j0 + 64 * q + lane;
                    if (j >= n8) continue;
                    // 8 cells at once when they are all +-0 or all -inf (the
                    // two values a causal mask holds), else value by value
                    const uint32_t x[4] = {w[q].x, w[q].y, w[q].z, w[q].w};
                    const bool zeros = ((x[0] | x[1] | x[2] | x[3]) & 0x7fff7fffu) == 0u;
                    const bool infs = x[0] == 0xfc00fc00u && x[1] == 0xfc00fc00u && x[2] == 0xfc00fc00u &&
                                      x[3] == 0xfc00fc00u;
                    if (zeros) {
                        last_fin = max(last_fin, 8 * j + 7);
                        last0 = max(last0, 8 * j + 7);
                    } else if (infs) {
                        first_inf = min(first_inf, 8 * j);
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            classify(x[e] & 0xffffu, 8 * j + 2 * e);
                            classify(x[e] >> 16, 8 * j + 2 * e + 1);
                        }
                    }
                }
            }
            for (int c = 8 * n8 + lane; c < p.n_kv; c += 64) classify(((const uint16_t *) rowp)[c], c);
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) {
                last_fin = max(last_fin, __shfl_xor(last_fin, off));
                last0 = max(last0, __shfl_xor(last0, off));
                first_inf = min(first_inf, __shfl_xor(first_inf, off));
                bad |= __shfl_xor(bad, off);
            }
            if (lane == 0) {
                const bool simple = !bad && last0 < first_inf;
                mtab[2 * u] = simple ? last0 : last_fin;
                mtab[2 * u + 1] = simple ? 0 : 1;
            }
        }
        __syncthreads();                          // (0) the mask table
    }
    auto unit_of = [&](const int r) { return p.m_ne2 == 1 ? tok_of(row0 + r) - t0 : r; };
    // general mode: some row of the tile is not a run of zeros then -inf
    int general = 0;
    if constexpr (has_mask) {
        for (int u = lane; u < n_units; u += 64) general |= mtab[2 * u + 1];
        general = __any(general) ? 1 : 0;
    }

    // Last visible cell of a row: the length / causal rule, narrowed by the
    // explicit mask's extent when a mask tensor came with the call.
    auto rule_lim = [&](const int tok) {                  // the length / causal rule for token tok
        int l = p.kv_hi - 1;
        if (p.causal_pos0 >= 0) l = (int) min((int64_t) l, p.causal_pos0 + tok);
        return l;
    };
    // this lane's row and limit; the wave's smallest limit over its valid
    // rows (a tile within it is visible to every row of the wave); hi_wg,
    // one past the last cell any row of the workgroup sees
    const int rr = 32 * rg + lr;
    const bool rvalid = rr < rows_here;
    int lim, lim_min, hi_wg;
    if constexpr (has_mask) {
        // every wave evaluates all rows of the tile, then reduces
        auto row_lim = [&](const int r_) { return min(rule_lim(tok_of(row0 + r_)), mtab[2 * unit_of(r_)]); };
        lim = rvalid ? row_lim(rr) : INT32_MAX;
        int lmin = lim, lmax = -1;
#pragma unroll
        for (int q = 0; q < RG; ++q)
            if (32 * q + lr < rows_here) lmax = max(lmax, q == rg ? lim : row_lim(32 * q + lr));
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            lmin = min(lmin, __shfl_xor(lmin, off));
            lmax = max(lmax, __shfl_xor(lmax, off));
        }
        lim_min = __builtin_amdgcn_readfirstlane(lmin);
        hi_wg = __builtin_amdgcn_readfirstlane(lmax) + 1;
    } else {
        // the rule does not decrease from row to row: the wave's first row
        // has its smallest limit, the tile's last row the largest (scalar
        // arithmetic, no cross-lane reductions on the way to the first loads)
        lim = rvalid ? rule_lim(tok_of(row0 + rr)) : INT32_MAX;
        lim_min = 32 * rg < rows_here ? rule_lim(tok_of(row0 + 32 * rg)) : INT32_MAX;
        hi_wg = rule_lim(tok_of(row0 + rows_here - 1)) + 1;
    }

    // Tiles of the whole row tile: NT of 64 cells; split s_all of n_all
    // takes tiles j n_all + s_all, visited from j = rot on. All splits run
    // NI iterations (a split with one tile fewer runs its last iteration on
    // a tile past hi_wg, which every row masks). Tiles from NI on point past
    // the end of the K/V views: they read zeros without memory traffic.
    const int n_all = p.n_split * S::SP;
    const int s_all = sx * S::SP + si;
    const int NT = (max(hi_wg, 0) + kTC - 1) / kTC;
    // NI = ceil(NT / n_all) and rot ~ rt NI / n_row_tiles by multiply-high
    // with the plan's reciprocals (0: divisor 1); rot only staggers the
    // splits' first tiles, so its rounding only needs rot < NI
    const int NI = __builtin_amdgcn_readfirstlane(
        p.split_magic ? (int) __umulhi((uint32_t) (NT + n_all - 1), p.split_magic) : NT);
    const int rot = __builtin_amdgcn_readfirstlane(
        NI > 0 ? min((int) __umulhi((uint32_t) (rt * NI), p.tiles_magic), NI - 1) : 0);
    const int n_vis = max(min(hi_wg, p.n_kv), 1);
    auto tile_c0 = [&](const int i) {                     // branch-free: selects only
        int j = i + rot;
        j = j < NI ? j : j - NI;
        const int c0 = (j * n_all + s_all) * kTC;
        return i < NI ? c0 : n_vis;
    };

    // this split's ring: K(t) in K buffer t % NK, V(t) in V buffer t % NV
    const int kring = si * S::RING, vring = kring + NK * kTileBytes;
    auto kbuf = [&](const int t) { return kring + (t % NK) * kTileBytes; };
    auto vbuf = [&](const int t) { return vring + (t % NV) * kTileBytes; };
    const uint32_t lds0 = lds_addr(lds);

    // ---- producer waves ----
    if (producer) {
        // K/V views end at the workgroup's last visible cell: loads past it read zeros
        const int bk = p.rk3 == 1 ? b : __builtin_amdgcn_readfirstlane(b / p.rk3);
        const int bv = p.rv3 == 1 ? b : __builtin_amdgcn_readfirstlane(b / p.rv3);
        const char * kbase = uniform_ptr(p.k + (int64_t) bk * p.k_nb3 + (int64_t) kvh * p.k_nb2);
        const char * vbase = uniform_ptr(p.v + (int64_t) bv * p.v_nb3 + (int64_t) kvh * p.v_nb2);
        const uint32_t k_nb1 = (uint32_t) p.k_nb1, v_nb1 = (uint32_t) p.v_nb1;
        const uint32_t k_lim = __builtin_amdgcn_readfirstlane((uint32_t) (n_vis - 1) * k_nb1 + 256);
        const uint32_t v_lim = __builtin_amdgcn_readfirstlane((uint32_t) (n_vis - 1) * v_nb1 + 256);
        // LDS-DMA instruction j of this role's 1 / RG of tile t: cells
        // cw + 4 j + (0..3) of the tile, cw = (64 / RG) rg; lane l fetches
        // granule (l & 15) ^ perm of cell 4 j + l / 16 of them (K: perm =
        // cell & 15, V: perm = 4 (cell & 3)), which lands at slot l & 15. The
        // lane offsets repeat every four instructions (K) or are all alike
        // (V); the cell offset goes into the descriptor, whose view ends at
        // the last visible cell (zero-length past it). The offsets stay below
        // 2^32 (the plan checks the K/V views).
        const int cw = (kTC / RG) * rg;
        uint32_t k_lane[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
            k_lane[q] = (uint32_t) (lane >> 4) * k_nb1 + (uint32_t) (((lane & 15) ^ ((4 * q + (lane >> 4)) & 15)) * 16);
        const uint32_t v_lane = (uint32_t) (lane >> 4) * v_nb1 + (uint32_t) (((lane & 15) ^ (4 * ((lane >> 4) & 3))) * 16);
        auto dma_k = [&](const int t) {
            const uint32_t off_t = (uint32_t) (tile_c0(t) + cw) * k_nb1;
#pragma unroll
            for (int j = 0; j < PER; ++j) {
                const uint32_t off = off_t + (uint32_t) (4 * j) * k_nb1;
                dma16(uniform_desc(kbase + off, off < k_lim ? k_lim - off : 0u), k_lane[j & 3],
                      lds0 + (uint32_t) (kbuf(t) + (cw + 4 * j) * 256));
            }
        };
        auto dma_v = [&](const int t) {
            const uint32_t off_t = (uint32_t) (tile_c0(t) + cw) * v_nb1;
#pragma unroll
            for (int j = 0; j < PER; ++j) {
                const uint32_t off = off_t + (uint32_t) (4 * j) * v_nb1;
                dma16(uniform_desc(vbase + off, off < v_lim ? v_lim - off : 0u), v_lane,
                      lds0 + (uint32_t) (vbuf(t) + (cw + 4 * j) * 256));
            }
        };
        // DMA order (the waits count on it): after barrier B_i (iteration
        // i), K(i + NK) and V(i + NV - 1); before the loop what those would
        // have been for i = 1 - NK .. -1, interleaved the same way: RG = 2:
        // K0 V0 K1 V1; RG = 4: V0 K0 V1 K1 V2 K2 V3 K3 V4. Before B_i: K(i + 1)
        // and V(i) landed (2 NK - 3 tiles issued after K(i + 1) may still fly).
        // The first tiles go out before the computing waves load the query
        // rows (barrier Q): the whole device reads its query rows at once,
        // and K0 queued behind them would hold up the first scores.
        if (NI > 0) {
            if constexpr (RG == 4) {
                dma_v(0); dma_k(0);
                __syncthreads();                  // (Q)
                dma_v(1); dma_k(1); dma_v(2); dma_k(2); dma_v(3); dma_k(3); dma_v(4);
                wait_vm<7 * PER>();               // V0, K0 landed
            } else {
                dma_k(0);
                __syncthreads();                  // (Q)
                dma_v(0); dma_k(1); dma_v(1);
                wait_vm<3 * PER>();               // K0 landed
            }
        } else {
            __syncthreads();                      // (Q)
        }
        __syncthreads();                          // (1) K0 visible
        for (int i = 0; i < NI; ++i) {
            wait_vm<(2 * NK - 3) * PER>();
            __syncthreads();                      // (B_i)
            if (i + 1 < NI) {
                dma_k(i + NK);
                dma_v(i + NV - 1);
            }
        }
        wait_vm<0>();
        __syncthreads();                          // (3) rings free
    }

    // ---- computing waves ----
    const float cexp = SOFTCAP ? kLog2e : p.scale * kLog2e;
    floatx16 o[4];
    // m_run in state units: log2 units (s c) in folded mode, else the units
    // of the scores the loop keeps (s, or the softcapped s')
    float m_run = -AL_INF, l_run = 0.0f;
    // The computing waves' work, compiled twice: GEN = the general-mask
    // mode, so that its per-value mask reads cost the fast loop nothing.
    auto compute = [&](auto gen_tag) {
        constexpr bool GEN = decltype(gen_tag)::value;
        // Folded mode (fast mode without softcap) keeps each score as t =
        // s c - b, b the row's reference max in log2 units (0 until the row
        // has one): the query rows are scaled by c before their f16 rounding
        // and the score MFMAs start from -b instead of 0, so p = exp2(t)
        // takes the scores as they are. Otherwise p = exp2(s c - m c).
        constexpr bool FOLD = !SOFTCAP && !GEN;
        const float cu = FOLD ? 1.0f : cexp;             // state units -> log2 units
        const float tau = kTau * kLog2e / cu;            // kTau in state units
        floatx16 negb = {};                               // -b in every register (folded mode)
        // the row's last visible cell less 4 h: cell c0 + 4 h + off is
        // visible when off <= limh - c0 (padding rows of a ragged last tile:
        // none in general mode, so that they read no mask values; in fast
        // mode they keep the INT32_MAX limit)
        const int limh = (GEN && !rvalid ? -1 : lim) - 4 * h;
        float thr = -AL_INF;                              // folded mode: rescale when some t exceeds it
        // general mode: this lane's mask row and the factor of its values
        // (ALiBi slope, arm.cpp:2294, over the scale the scores lack)
        const _Float16 * mrow = nullptr;
        float mslope = 0.0f;
        if constexpr (GEN) {
            mrow = (const _Float16 *) mask_row(rvalid ? rr : 0);
            const uint32_t hq = (uint32_t) (kvh * p.G + (row0 + rr) - tok_of(row0 + rr) * p.G);
            const float slope = p.max_bias > 0.0f ? (hq < p.n_head_log2 ? powf(p.m0, (float) (hq + 1))
                                                                         : powf(p.m1, (float) (2 * (hq - p.n_head_log2) + 1)))
                                                  : 1.0f;
            mslope = SOFTCAP ? slope : slope / p.scale;
        }
        // Q^T B operands: row rr (token r / G, head kvh G + r % G), dims
        // 16 ks + 8 h .. + 7, f16 (RNE), loaded straight into registers; the
        // loads go out before barrier (Q), their latency overlapping the
        // producers' first DMA
        // With two cell splits the rows of a row group are loaded once, by
        // split 0's wave, and handed to split 1's as f16 through split 1's V
        // buffer 2 (16 KiB for 64 rows; its first DMA goes out after barrier
        // B_0): every CU reads its query rows once.
        half8 qf[8];
        constexpr bool kShareQ = S::SP == 2;
        char * const qshare = lds + S::RING + NK * kTileBytes + 2 * kTileBytes;   // split 1's V buffer 2
        static_assert(!kShareQ || NV >= 3, "the shared query rows need a V buffer the prologue leaves free");
        auto qslot = [&](const int ks) { return rr * 256 + ((((2 * ks + h) ^ (rr & 15)) & 15) << 4); };
        {
            const int r = row0 + (rvalid ? rr : 0);
            const int tk = tok_of(r);
            const float * qrow = (const float *) (p.q + (int64_t) b * p.q_nb3 + (int64_t) tk * p.q_nb1 +
                                                  (int64_t) (kvh * p.G + r - tk * p.G) * p.q_nb2);
            float4 qv[16];
            if (!kShareQ || si == 0) {
#pragma unroll
                for (int ks = 0; ks < 8; ++ks) {
                    qv[2 * ks] = *(const float4 *) (qrow + 16 * ks + 8 * h);
                    qv[2 * ks + 1] = *(const float4 *) (qrow + 16 * ks + 8 * h + 4);
                }
            }
            __syncthreads();                          // (Q) the first K/V tiles are on their way
            if (!kShareQ || si == 0) {
#pragma unroll
                for (int ks = 0; ks < 8; ++ks) {
                    if constexpr (FOLD) {
                        qv[2 * ks] *= cexp;
                        qv[2 * ks + 1] *= cexp;
                    }
                    qf[ks] = rvalid ? to_half8(qv[2 * ks], qv[2 * ks + 1]) : half8{0, 0, 0, 0, 0, 0, 0, 0};
                    if (kShareQ) *(half8 *) (qshare + qslot(ks)) = qf[ks];
                }
            }
        }
        __syncthreads();                          // (1)
        if (kShareQ && si == 1) {
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) qf[ks] = *(const half8 *) (qshare + qslot(ks));
        }

        // LDS read offsets of this lane: K operand (cell 32 cb + lr, granule
        // 2 ks + h) and V^T operand (cell 16 kk + 4 h + (s16 >> 2) [+ 8],
        // granule 4 db + 2 (q16 & 1) + ((s16 & 3) >> 1), half s16 & 1, for
        // 16-lane group q16)
        int vcell, vgran, vhalf, vsw;
        auto v_offsets = [&](const int ln) {
            const int q16 = (ln >> 4) & 3, s16 = ln & 15;
            vcell = 4 * ((ln >> 5) & 1) + (s16 >> 2);
            vgran = 2 * (q16 & 1) + ((s16 & 3) >> 1);
            vhalf = (s16 & 1) * 8;
            vsw = 4 * (s16 >> 2);                         // 4 (cell & 3)
        };
        v_offsets(lane);

#pragma unroll
        for (int db = 0; db < 4; ++db) o[db] = floatx16{};

        auto lane_max = [&](const floatx16 (&sc)[2]) {
            float m0 = fmaxf(fmaxf(sc[0][0], sc[0][1]), sc[0][2]);
            float m1 = fmaxf(fmaxf(sc[1][0], sc[1][1]), sc[1][2]);
#pragma unroll
            for (int v = 3; v < 15; v += 2) {
                m0 = fmaxf(fmaxf(m0, sc[0][v]), sc[0][v + 1]);
                m1 = fmaxf(fmaxf(m1, sc[1][v]), sc[1][v + 1]);
            }
            return fmaxf(fmaxf(m0, sc[0][15]), fmaxf(m1, sc[1][15]));
        };
        auto rescale = [&](floatx16 (&sc)[2]) {         // move the reference max of outgrown rows
            const float base = FOLD ? -negb[0] : 0.0f;
            const float mt = pair_max(lane_max(sc)) + base;
            const bool g = mt > m_run + tau;
            const float mn = g ? mt : m_run;
            const float alpha = g ? __builtin_amdgcn_exp2f((m_run - mn) * cu) : 1.0f;   // 0 from -inf
#pragma unroll
            for (int db = 0; db < 4; ++db) o[db] *= alpha;
            l_run *= alpha;
            m_run = mn;
            if constexpr (FOLD) {                     // the new base: scores and MFMA start follow
                const float nb = mn == -AL_INF ? 0.0f : mn;
                const float sh = nb - base;
#pragma unroll
                for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                    for (int v = 0; v < 16; ++v) sc[cb][v] -= sh;
#pragma unroll
                for (int v = 0; v < 16; ++v) negb[v] = -nb;
                thr = mn == -AL_INF ? -AL_INF : tau;
            }
        };
        // some score of the tile above the rescale threshold (lane maximum mx)
        auto outgrows = [&](const float mx) { return FOLD ? mx > thr : mx > m_run + tau; };
        // fresh scores: softcap, -inf for cells of a tile that some row of
        // the wave does not wholly see, and the reference max moved when the
        // tile outgrows it (a rare, uniform branch; the first visible tile
        // always does)
        auto prepare = [&](floatx16 (&sc)[2], const int c0) {
            if constexpr (SOFTCAP) {
                // softcap tanh(s scale), eight values at a time (the
                // exponentials of a whole tile at once would need 32 more
                // registers than the loop has)
                const float c2 = 2.0f * kLog2e * p.scale;
#pragma unroll
                for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                    for (int v0 = 0; v0 < 16; v0 += 8) {
#pragma unroll
                        for (int v = v0; v < v0 + 8; ++v) sc[cb][v] = p.softcap * tanh_exp2(sc[cb][v], c2);
                        __builtin_amdgcn_sched_barrier(0);
                    }
            }
            if constexpr (GEN) {
                // s + slope * mask in the units the scores are kept in (raw
                // dot products: the mask term divided by the scale); cells
                // past the row's extent -inf (arm.cpp:2310-2343)
                // four cells at a time, each group's loads kept in its slot
                // (a cold path: few registers rather than latency hiding)
                // (cell c0 + 4 h + off visible when off <= d; the offsets
                // are immediates of the compares and loads; padding rows of
                // a ragged last tile load nothing)
                const int d = limh - c0;
                const _Float16 * mt = mrow + c0 + 4 * h;
#pragma unroll
                for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                    for (int w4 = 0; w4 < 4; ++w4) {
                        const int og = 32 * cb + 8 * w4;
                        float mv[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) mv[e] = og + e <= d ? (float) mt[og + e] : 0.0f;
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            sc[cb][4 * w4 + e] = og + e <= d ? sc[cb][4 * w4 + e] + mslope * mv[e] : -AL_INF;
                        __builtin_amdgcn_sched_barrier(0);
                    }
            } else if (c0 + kTC - 1 > lim_min) {
                // cell c0 + 4 h + off is visible when off <= d: one register
                // per tile, the offsets are immediates
                // (-inf from a scalar register: no vector register held for it)
                const int d = limh - c0;
                float ninf = -AL_INF;
                asm volatile("" : "+s"(ninf));
#pragma unroll
                for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const int off = 32 * cb + (v & 3) + 8 * (v >> 2);
                        sc[cb][v] = off <= d ? sc[cb][v] : ninf;
                    }
            }
        };
        // fresh scores ready: the reference max moved when the tile outgrows
        // it (a rare, uniform branch; the first visible tile always does)
        auto finish_scores = [&](floatx16 (&sc)[2], const int c0) {
            prepare(sc, c0);
            if (__any(outgrows(lane_max(sc)))) rescale(sc);
        };
        auto k_read = [&](const int kbo, const int cb, const int ks) {
            const int c = 32 * cb + lr;
            return as_half8(*(const u32x4 *) (lds + kbo + c * 256 + (((2 * ks + h) ^ (c & 15)) << 4)));
        };
        auto v_read = [&](const int vbo, const int kk, const int db) {
            const char * vt = lds + vbo;
            const int cbase = 16 * kk + vcell;
            const int g = 4 * db + vgran;
            const half4 a = lds_read_tr16(vt + cbase * 256 + ((g ^ vsw) << 4) + vhalf);
            const half4 c = lds_read_tr16(vt + (cbase + 8) * 256 + ((g ^ vsw) << 4) + vhalf);
            return half8{a[0], a[1], a[2], a[3], c[0], c[1], c[2], c[3]};
        };

        // Iteration i in eight explicitly ordered slots and a tail (each slot:
        // the LDS reads it prefetches, then its vector work and MFMAs;
        // nothing moves across slots):
        // - S(i + 1) = K(i + 1) Q^T on the matrix cores, two MFMAs per slot,
        //   K operands read two slots ahead;
        // - the vector ALU turns S(i) into unnormalised probabilities
        //   p = exp2(s c - m c), rounded to f16 (RNE) into the P^T operands,
        //   four values per lane and slot: P^T block kk (cells 16 kk ..
        //   16 kk + 15, registers 8 (kk & 1) .. + 7 of S^T block kk / 2) is
        //   complete after slot 2 kk + 1;
        // - O^T += V(i)^T P(i)^T for block kk in slots 2 kk + 2 (dims blocks
        //   0, 1) and 2 kk + 3 (2, 3), with the f16 probabilities' row sums,
        //   V operands read one slot ahead; block 3 in the tail, beside the
        //   lane maxima of S(i + 1).
        // So every slot from the third on keeps the matrix cores busy with
        // four MFMAs while the vector ALU computes its exponentials (phases
        // of exponentials and of P V products one after the other left the
        // MFMAs of the second idle behind the first's vector work). The
        // products accumulate in the same order as block by block.
        float mx;                                 // lane max of S(i + 1), from body(i) (fast mode)
        auto body = [&](const int i, const bool qk, floatx16 (&cur)[2], floatx16 (&nxt)[2]) {
            const float mc = FOLD || m_run == -AL_INF ? 0.0f : m_run * cexp;
            // the buffers' offsets as opaque values: otherwise the compiler
            // keeps every buffer's read addresses live across the loop
            int kb_ = kbuf(i + 1), vb_ = vbuf(i);
            asm volatile("" : "+s"(kb_), "+s"(vb_));
            const half2v one2 = {(_Float16) 1.0f, (_Float16) 1.0f};
            half8 pf[4];
            half8 kq[8][2];
            half8 vn[2], vc[2], v3[4];
            if (qk) {
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) {
                    kq[ks][0] = k_read(kb_, 0, ks);
                    kq[ks][1] = k_read(kb_, 1, ks);
                }
                nxt[0] = FOLD ? negb : floatx16{};
                nxt[1] = FOLD ? negb : floatx16{};
            }
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) {
                if (qk && ks + 2 < 8) {
                    kq[ks + 2][0] = k_read(kb_, 0, ks + 2);
                    kq[ks + 2][1] = k_read(kb_, 1, ks + 2);
                }
                if (ks >= 1 && ks <= 6) {             // the next slot's V operands
                    const int b = (ks - 1) >> 1, d0 = 2 * ((ks + 1) & 1);
                    vn[0] = v_read(vb_, b, d0);
                    vn[1] = v_read(vb_, b, d0 + 1);
                }
                if (ks == 7) {
#pragma unroll
                    for (int db = 0; db < 4; ++db) v3[db] = v_read(vb_, 3, db);
                }
                __builtin_amdgcn_sched_barrier(0);
                const int cb = ks >> 2, v0 = 4 * (ks & 3), kk = 2 * cb + (v0 >> 3), e0 = v0 & 4;
#pragma unroll
                for (int u = 0; u < 4; u += 2) {
                    const float2v e = FOLD ? float2v{__builtin_amdgcn_exp2f(cur[cb][v0 + u]),
                                                     __builtin_amdgcn_exp2f(cur[cb][v0 + u + 1])}
                                           : float2v{__builtin_amdgcn_exp2f(__builtin_fmaf(cur[cb][v0 + u], cexp, -mc)),
                                                     __builtin_amdgcn_exp2f(__builtin_fmaf(cur[cb][v0 + u + 1], cexp, -mc))};
                    half2v hv = __builtin_convertvector(e, half2v);
                    asm volatile("" : "+v"(hv));          // keeps the exponentials in this slot
                    pf[kk][e0 + u] = hv[0];
                    pf[kk][e0 + u + 1] = hv[1];
                }
                if (qk) {
                    nxt[0] = mfma32(kq[ks][0], qf[ks], nxt[0]);
                    nxt[1] = mfma32(kq[ks][1], qf[ks], nxt[1]);
                }
                if (ks >= 2) {                        // O^T += V^T P^T, block (ks - 2) / 2, two dims blocks
                    const int b = (ks - 2) >> 1, d0 = 2 * (ks & 1);
#pragma unroll
                    for (int w = d0; w < d0 + 2; ++w)
                        l_run = __builtin_amdgcn_fdot2(half2v{pf[b][2 * w], pf[b][2 * w + 1]}, one2, l_run, false);
                    o[d0] = mfma32(vc[0], pf[b], o[d0]);
                    o[d0 + 1] = mfma32(vc[1], pf[b], o[d0 + 1]);
                }
                vc[0] = vn[0];
                vc[1] = vn[1];
                __builtin_amdgcn_sched_barrier(0);
            }
            // tail: block 3's products and row sums; S(i + 1) prepared and its
            // lane maxima taken (fast mode; general mode prepares it after the
            // body) while they run
#pragma unroll
            for (int w = 0; w < 4; ++w)
                l_run = __builtin_amdgcn_fdot2(half2v{pf[3][2 * w], pf[3][2 * w + 1]}, one2, l_run, false);
#pragma unroll
            for (int db = 0; db < 4; ++db) o[db] = mfma32(v3[db], pf[3], o[db]);
            __builtin_amdgcn_sched_barrier(0);
            constexpr bool fold = !GEN;
            float mx0 = -AL_INF, mx1 = -AL_INF;
            if (fold && qk) {
                prepare(nxt, tile_c0(i + 1));
                float m0 = fmaxf(fmaxf(nxt[0][0], nxt[0][1]), nxt[0][2]);
                float m1 = fmaxf(fmaxf(nxt[1][0], nxt[1][1]), nxt[1][2]);
#pragma unroll
                for (int v = 3; v < 15; v += 2) {
                    m0 = fmaxf(fmaxf(m0, nxt[0][v]), nxt[0][v + 1]);
                    m1 = fmaxf(fmaxf(m1, nxt[1][v]), nxt[1][v + 1]);
                }
                mx0 = fmaxf(m0, nxt[0][15]);
                mx1 = fmaxf(m1, nxt[1][15]);
            }
            mx = fmaxf(mx0, mx1);
        };

        floatx16 s0[2], s1[2];
        if (NI > 0) {
            {
                half8 kop[2][8];
#pragma unroll
                for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                    for (int ks = 0; ks < 8; ++ks) kop[cb][ks] = k_read(kbuf(0), cb, ks);
#pragma unroll
                for (int cb = 0; cb < 2; ++cb) {
                    floatx16 acc = {};
#pragma unroll
                    for (int ks = 0; ks < 8; ++ks) acc = mfma32(kop[cb][ks], qf[ks], acc);
                    s0[cb] = acc;
                }
                finish_scores(s0, tile_c0(0));
            }
            // iteration i: S(i) in s0 for even i, s1 for odd i
            auto iteration = [&](const int i, floatx16 (&cur)[2], floatx16 (&nxt)[2]) {
                __syncthreads();                  // (B_i) K(i + 1), V(i) landed; iteration i - 1 done
                body(i, true, cur, nxt);
                if constexpr (GEN) finish_scores(nxt, tile_c0(i + 1));
                else if (__any(outgrows(mx))) rescale(nxt);
            };
            int i = 0;
            for (; i + 2 < NI; i += 2) {
                iteration(i, s0, s1);
                iteration(i + 1, s1, s0);
            }
            // the loop's last iterations with offsets derived anew from an
            // opaque lane: the loop's own are not kept live past it
            int ln = lane;
            asm volatile("" : "+v"(ln));
            v_offsets(ln);
            if (i + 1 < NI) {
                iteration(i, s0, s1);
                ++i;
            }
            __syncthreads();                      // (B_{NI - 1}) V(NI - 1) landed
            if (i & 1) body(i, false, s1, s0);
            else body(i, false, s0, s1);
        }
        __syncthreads();                          // (3) rings free
    };
    if (!producer) {
        if (MASK && general) compute(std::bool_constant<MASK>{});
        else compute(std::false_type{});
    }
    const float cu_run = !SOFTCAP && !(MASK && general) ? 1.0f : cexp;   // m_run's units -> log2 units
    float m_nat = m_run == -AL_INF ? -AL_INF : m_run * (cu_run / kLog2e);
    float l_row = pair_sum(l_run);
    // The epilogue's lane, row and half read anew: their LDS offsets are
    // computed here, not held in registers across the loop.
    const int lane_e = lane_id_fresh();
    const int he = lane_e >> 5;
    const int rre = 32 * rg + (lane_e & 31);

    // One workgroup per row tile and two cell splits in it: both splits put
    // their rows' states into LDS records [split][row][132] at once, then
    // every thread combines the two states of the 16-byte granules of the
    // rows it stores, scales them and stores whole rows, 16 bytes per lane,
    // non-temporal (one pass: no combine by split 0 alone and no staging
    // copy; the same arithmetic as the merge below).
    if (S::SP == 2 && p.n_split == 1) {
        if (!producer) {
            float * rec = (float *) lds + (si * ROWS + rre) * kRowStride;
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int bq = 0; bq < 4; ++bq)
                    *(float4 *) (rec + 32 * db + 8 * bq + 4 * he) =
                        float4{o[db][4 * bq], o[db][4 * bq + 1], o[db][4 * bq + 2], o[db][4 * bq + 3]};
            if (he == 0) *(float2 *) (rec + 128) = float2{m_nat, l_row};
        }
        __syncthreads();
        for (int item = threadIdx.x; item < rows_here * 32; item += 2 * kWaves * 64) {
            const int r = item >> 5, g = item & 31;
            const float * r0 = (const float *) lds + r * kRowStride;
            const float * r1 = (const float *) lds + (ROWS + r) * kRowStride;
            const float2 ml0 = *(const float2 *) (r0 + 128), ml1 = *(const float2 *) (r1 + 128);
            const float M = fmaxf(ml0.x, ml1.x);
            const float Mu = M == -AL_INF ? 0.0f : M;
            const float wa = exp_fast(ml0.x - Mu), wb = exp_fast(ml1.x - Mu);
            const float4 x0 = *(const float4 *) (r0 + 4 * g), x1 = *(const float4 *) (r1 + 4 * g);
            const float4 o4 = {x0.x * wa + x1.x * wb, x0.y * wa + x1.y * wb, x0.z * wa + x1.z * wb,
                               x0.w * wa + x1.w * wb};
            const float L = ml0.y * wa + ml1.y * wb;
            const int rg_ = row0 + r;
            const int tk = tok_of(rg_), hq = kvh * p.G + rg_ - tk * p.G;
            float * out = (float *) (p.dst + ((int64_t) (b * p.T + tk) * p.Hq + hq) * p.dst_nb1);
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, apply_scale(o4, row_scale(M, L, p.sinks, hq))),
                                                   make_rsrc(out, 512), 16 * g, 0, kNonTemporal);
        }
        return;
    }

    // The splits within the workgroup merge through LDS: split 1 stores its
    // rows' state as a record [row][132], split 0 combines it with its own.
    if constexpr (S::SP == 2) {
        float * rec = (float *) lds + rre * kRowStride;
        if (!producer && si == 1) {
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int bq = 0; bq < 4; ++bq)
                    *(float4 *) (rec + 32 * db + 8 * bq + 4 * he) =
                        float4{o[db][4 * bq], o[db][4 * bq + 1], o[db][4 * bq + 2], o[db][4 * bq + 3]};
            if (he == 0) *(float2 *) (rec + 128) = float2{m_nat, l_row};
        }
        __syncthreads();
    }
    const bool owner = !producer && si == 0;               // holds the workgroup's merged rows
    if (S::SP == 2 && owner) {
        const float * rec = (const float *) lds + rre * kRowStride;
        const float2 ml = *(const float2 *) (rec + 128);
        const float M = fmaxf(m_nat, ml.x);
        const float Mu = M == -AL_INF ? 0.0f : M;
        const float wa = exp_fast(m_nat - Mu), wb = exp_fast(ml.x - Mu);
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int bq = 0; bq < 4; ++bq) {
                const float4 x = *(const float4 *) (rec + 32 * db + 8 * bq + 4 * he);
                o[db][4 * bq] = o[db][4 * bq] * wa + x.x * wb;
                o[db][4 * bq + 1] = o[db][4 * bq + 1] * wa + x.y * wb;
                o[db][4 * bq + 2] = o[db][4 * bq + 2] * wa + x.z * wb;
                o[db][4 * bq + 3] = o[db][4 * bq + 3] * wa + x.w * wb;
            }
        l_row = l_row * wa + ml.y * wb;
        m_nat = M;
    }

    // O^T lane l: row lr, dims 32 db + 8 bq + 4 h .. + 3 in o[db][4 bq .. 4 bq + 3].
    // One workgroup per row tile: the owners put the finished rows into LDS
    // (past the merge records; 16-byte granule g of row r at slot g ^ (r & 31)),
    // then all threads store whole rows, 16 bytes per lane, non-temporal (the
    // rows stream to memory instead of waiting in L2 for the end of the
    // launch: 3 % on 512-token chunks).
    if (p.n_split == 1) {
        float * stage = (float *) (lds + 80 * 1024);
        if (owner && rvalid) {
            const int hq = kvh * p.G + (row0 + rre) - tok_of(row0 + rre) * p.G;
            const RowScale rs = row_scale(m_nat, l_row, p.sinks, hq);
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int bq = 0; bq < 4; ++bq) {
                    const int g = 8 * db + 2 * bq + he;
                    *(float4 *) (stage + rre * 128 + 4 * (g ^ (rre & 31))) =
                        apply_scale(float4{o[db][4 * bq], o[db][4 * bq + 1], o[db][4 * bq + 2], o[db][4 * bq + 3]}, rs);
                }
        }
        __syncthreads();
        for (int item = threadIdx.x; item < rows_here * 32; item += 2 * kWaves * 64) {
            const int r = item >> 5, g = item & 31;
            const int rg_ = row0 + r;
            const int tk = tok_of(rg_), hq = kvh * p.G + rg_ - tk * p.G;
            float * out = (float *) (p.dst + ((int64_t) (b * p.T + tk) * p.Hq + hq) * p.dst_nb1);
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, *(const float4 *) (stage + r * 128 + 4 * (g ^ (r & 31)))),
                                                   make_rsrc(out, 512), 16 * g, 0, kNonTemporal);
        }
        return;
    }

    // Workgroup splits: publish this workgroup's record [unit][sx][row][132]
    // with device-coherent stores; the last workgroup of the row tile to
    // arrive combines the records of all of them (fixed order) into dst.
    // The record goes out as whole lines: the owners put their rows into LDS
    // (as the finished rows above), then all threads store consecutive
    // 16-byte granules of the record, so every write covers whole lines
    // (a row-per-lane write of 32 bytes to each of 32 rows made every write
    // partial, and publication took ~4 us).
    const int unit = (b * p.Hkv + kvh) * p.n_row_tiles + rt;
    constexpr uint32_t RS = ROWS * kRowStride * 4;                 // record bytes
    constexpr int kGran = kRowStride / 4;                          // 16-byte granules per record row
    const rsrc_t rec = make_rsrc(p.part + (int64_t) unit * p.n_split * (ROWS * kRowStride), RS * (uint32_t) p.n_split);
    {
        float * stage = (float *) (lds + 80 * 1024);
        float2 * ml_stage = (float2 *) (lds + 80 * 1024 + 128 * 512);
        if (owner) {
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int bq = 0; bq < 4; ++bq) {
                    const int g = 8 * db + 2 * bq + he;
                    *(float4 *) (stage + rre * 128 + 4 * (g ^ (rre & 31))) =
                        float4{o[db][4 * bq], o[db][4 * bq + 1], o[db][4 * bq + 2], o[db][4 * bq + 3]};
                }
            if (he == 0) ml_stage[rre] = float2{m_nat, l_row};
        }
        __syncthreads();
        for (int i = threadIdx.x; i < rows_here * kGran; i += 2 * kWaves * 64) {
            const int r = i / kGran, j = i - r * kGran;
            const float2 ml = ml_stage[r];
            const float4 v = j < 32 ? *(const float4 *) (stage + r * 128 + 4 * (j ^ (r & 31))) : float4{ml.x, ml.y, 0.0f, 0.0f};
            buf_store16_dev(v, rec, (uint32_t) sx * RS + (uint32_t) i * 16);
        }
    }
    complete_wave_memops();
    __syncthreads();
    unsigned * cnt = p.counters + unit;
    int * s_last = (int *) (lds + kLds - 16);                       // past the staged rows
    if (threadIdx.x == 0) *s_last = (add_agent(cnt, 1u) == (unsigned) (p.n_split - 1));
    __syncthreads();
    if (!*s_last) return;
    order_after_counter();
    if (threadIdx.x == 0) st_agent_u32(cnt, 0u);                     // ready for the next call in stream order
    // Thread t takes (row, 4 dims) items t, t + 512, ..., kBatch at a time,
    // with every record's loads of the batch in flight at once (no loads for
    // splits past n_split).
    constexpr int kBatch = 4;
    for (int base = threadIdx.x; base < rows_here * 32; base += kBatch * 2 * kWaves * 64) {
        float2 ml[kBatch][kMaxPrefillSplit];
        float4 ov[kBatch][kMaxPrefillSplit];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            const int item = min(base + k * 2 * kWaves * 64, rows_here * 32 - 1);
            const int r = item >> 5, d4 = item & 31;
#pragma unroll
            for (int s2 = 0; s2 < kMaxPrefillSplit; ++s2) {
                ml[k][s2] = float2{-AL_INF, 0.0f};
                ov[k][s2] = float4{0, 0, 0, 0};
                if (s2 < p.n_split) {
                    const uint32_t row = (uint32_t) s2 * RS + (uint32_t) (r * kRowStride * 4);
                    ml[k][s2] = buf_load8_dev(rec, row + 128 * 4);
                    ov[k][s2] = buf_load16_dev(rec, row + (uint32_t) (d4 * 16));
                }
            }
        }
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            const int item = base + k * 2 * kWaves * 64;
            if (item >= rows_here * 32) break;
            const int r = item >> 5, d4 = item & 31;
            float M = ml[k][0].x;
#pragma unroll
            for (int s2 = 1; s2 < kMaxPrefillSplit; ++s2) M = fmaxf(M, ml[k][s2].x);
            const float Mu = M == -AL_INF ? 0.0f : M;
            float L = 0.0f;
            float4 acc = {0, 0, 0, 0};
#pragma unroll
            for (int s2 = 0; s2 < kMaxPrefillSplit; ++s2) {
                const float w = s2 < p.n_split ? exp_fast(ml[k][s2].x - Mu) : 0.0f;
                L += w * ml[k][s2].y;
                acc.x += w * ov[k][s2].x; acc.y += w * ov[k][s2].y; acc.z += w * ov[k][s2].z; acc.w += w * ov[k][s2].w;
            }
            const int rg_ = row0 + r;
            const int tk = tok_of(rg_), hq = kvh * p.G + rg_ - tk * p.G;
            float * out = (float *) (p.dst + ((int64_t) (b * p.T + tk) * p.Hq + hq) * p.dst_nb1);
            *(float4 *) (out + 4 * d4) = finalize4(acc, M, L, p.sinks, hq);
        }
    }
}

}  // namespace

size_t fattn_prefill_lds_bytes() { return (size_t) kLds; }

template <int RG>
static void launch_rg(const FattnParams & p, const dim3 grid, hipStream_t stream) {
    const dim3 block(2 * kWaves * 64);
    const bool sc = p.softcap != 0.0f, mk = p.mask != nullptr;
    if (sc) {
        if (mk) hipLaunchKernelGGL((fattn_prefill_kernel<RG, true, true>), grid, block, 0, stream, p);
        else    hipLaunchKernelGGL((fattn_prefill_kernel<RG, true, false>), grid, block, 0, stream, p);
    } else {
        if (mk) hipLaunchKernelGGL((fattn_prefill_kernel<RG, false, true>), grid, block, 0, stream, p);
        else    hipLaunchKernelGGL((fattn_prefill_kernel<RG, false, false>), grid, block, 0, stream, p);
    }
}

hipError_t fattn_prefill_launch(const FattnParams & p, int rows_per_tile, hipStream_t stream) {
    if (p.n_split < 1 || p.n_split > kMaxPrefillSplit || (rows_per_tile != 64 && rows_per_tile != 128))
        return hipErrorInvalidValue;
    const dim3 grid((unsigned) p.Hkv, (unsigned) p.n_split, (unsigned) ((int64_t) p.n_row_tiles * p.B));
    if (rows_per_tile == 128) launch_rg<4>(p, grid, stream);
    else launch_rg<2>(p, grid, stream);
    return hipGetLastError();
}
