// Prefill (and long speculative-verify) attention for gfx950: many query rows
// per kv head, causal / length masking given implicitly (kv_len,
// causal_pos0). Semantics as nnml_compute_forward_flash_attn_ext_f16
// (nnml/src/ops/arm/arm.cpp:2196-2433), numerics as fattn_splitkv.hip.
//
// One workgroup = one row tile of 64 query rows of one kv-head group
// (row r -> token r / G, head kvh*G + r % G) and 8 wavefronts, two per SIMD.
// Wave w takes row half w & 1 (32 rows: 2 MFMA row blocks, so each K/V
// operand read from LDS feeds 2 MFMAs) and cell split w >> 1 (every 4th
// 32-cell tile of the visible range). The two waves of a split sit on
// different SIMDs and share the split's ring of two 16 KiB LDS stages: each
// loads half of every tile, publishes "my half landed" in an LDS flag, reads
// the whole tile once the other's half has landed, publishes "stage read",
// and refills its half of the stage once the other has read it too. (With
// one wave loading whole tiles the other waited for it on every tile.)
// No workgroup barrier runs in the loop, so the splits drift apart and the
// two waves on each SIMD (different splits) overlap each other's matrix and
// vector work. A 512-token chunk of Qwen3-4B gives 32 row tiles x 8 kv heads
// = 256 workgroups, one per CU.
//
// K/V tiles travel HBM/L2 -> LDS by LDS-DMA buffer loads:
//   - K as MFMA A operands: block (mb, kb) holds, at lane l's 16-byte slot,
//     cell 16 mb + l % 16, dims 32 kb + 8 (l / 16) .. + 7, so ds_read_b128
//     at lane*16 yields the operand;
//   - V cell-major (256 bytes per cell) with the 16-byte granule j of cell c
//     at slot j ^ (c & 15), read transposed by ds_read_b64_tr_b16 into V^T
//     A operands whose k slots follow the S^T output layout (cells 4g + i
//     and 16 + 4g + i of lane group g), so P^T is S^T in place.
// The DMA is inline assembly the compiler does not count; each wave waits
// for its own half (s_waitcnt vmcnt) before publishing it. The query rows
// come the same way, once per workgroup, into a staging area that holds the
// flags afterwards.
//
// Softmax per tile: the running max is kept on the raw scores (scale > 0
// keeps their order), p = exp2(s * c - m * c) with c = scale * log2(e) is
// one FMA and one v_exp_f32 per score, P is packed to f16 two at a time,
// and the row sums l come from an extra MFMA against an all-ones operand
// (f32 accumulation of the same f16 P that weights V). The reference max
// moves lazily (only when a tile exceeds it by more than kTau in natural
// units), so O is rarely rescaled; the rescale runs outside the fast loop so
// the accumulators stay in place across iterations.
//
// The 1-D grid runs kv head fastest (XCD affinity: with Hkv = 8 each head's
// K/V stays in one XCD's L2) and, with a causal mask, row tiles longest
// first.

#include "fattn_tile.hpp"

namespace {

using namespace fattn;

constexpr int kCS = 4;                       // cell splits: tiles cs, cs + 4, ...
constexpr int kRH = 2;                       // row halves
constexpr int kPW = kCS * kRH;               // waves per workgroup
constexpr int kPRB = 2;                      // MFMA row blocks per wave
constexpr int kPRows = 16 * kPRB * kRH;      // query rows per workgroup
constexpr int kKBytes = 8 * 1024;            // K of a 32-cell tile: 8 MFMA-ordered 1 KiB blocks
constexpr int kStage = 2 * kKBytes;          // K then V (32 cells x 256 bytes)
constexpr int kNB = 2;                       // stages per split
constexpr int kStride = kCS * 32;            // cells between a split's tiles
constexpr int kRing = kCS * kNB * kStage;    // 128 KiB
constexpr int kQBytes = kPRows * 512;        // the tile's query rows, f32 (32 KiB)
constexpr int kRec = kPRows * kRowStride * 4;        // one split's merge record (64 rows)
constexpr int kLds = kCS * kRec > kRing + kQBytes ? kCS * kRec : kRing + kQBytes;   // 160 KiB
constexpr float kLog2e = 1.44269504088896341f;
constexpr int kSpinLimit = 1 << 22;          // flag polls before a wave gives up (never in a correct run)

// The operands of one tile in registers.
struct TileOps {
    u32x4 k[2][4];                           // K A operands [mb][kb]
    half8 vt[8];                             // V^T A operands, dim block d
};

// LDS-DMA of half h of tile (cells cb ..) into a stage: the 4 K blocks of
// cell block mb = h, then V blocks 4h .. 4h + 3 (cells 16h .. 16h + 15).
__device__ __forceinline__ void issue_half(const int4v kd, const int4v vd, const uint32_t base, const uint32_t cb,
                                           const uint32_t k_nb1, const uint32_t v_nb1, const int g, const int n,
                                           const int h) {
    const uint32_t kofs = (cb + (uint32_t) n) * k_nb1 + (uint32_t) (g * 16) + (uint32_t) (16 * h) * k_nb1;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
        dma16(kd, kofs + (uint32_t) (64 * kb), base + (uint32_t) ((h * 4 + kb) * 1024));
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
        const int i = 4 * h + ii;
        const int c = 4 * i + g;
        dma16(vd, (cb + (uint32_t) c) * v_nb1 + (uint32_t) (((n ^ c) & 15) * 16), base + (uint32_t) (kKBytes + i * 1024));
    }
}

// Both operands of a stage: K at lane*16 of each block; V^T from source
// cells 4g + (n >> 2) (k slots 0..3) and 16 + 4g + (n >> 2) (4..7), dims
// 16d + 4(n & 3) .. + 3 (granule 2d + ((n & 3) >> 1), half n & 1).
__device__ __forceinline__ void read_tile(TileOps & t, const char * st, const int lane, const int g, const int n) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) t.k[mb][kb] = *(const u32x4 *) (st + (mb * 4 + kb) * 1024 + lane * 16);
    const int vc0 = 4 * g + (n >> 2);
    const int vc1 = 16 + vc0;
    const int vq = (n & 3) >> 1;
    const char * r0 = st + kKBytes + vc0 * 256 + (n & 1) * 8;
    const char * r1 = st + kKBytes + vc1 * 256 + (n & 1) * 8;
#pragma unroll
    for (int d = 0; d < 8; ++d) {
        const half4 a = lds_read_tr16(r0 + (((2 * d + vq) ^ (vc0 & 15)) << 4));
        const half4 c = lds_read_tr16(r1 + (((2 * d + vq) ^ (vc1 & 15)) << 4));
        t.vt[d] = half8{a[0], a[1], a[2], a[3], c[0], c[1], c[2], c[3]};
    }
}

// LDS flag hand-off between the two waves of a split.
__device__ __forceinline__ void flag_set(int * f, int v) {
    __hip_atomic_store(f, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// Waits until *f >= v; false if it never got there (a broken hand-off),
// so the wave ends instead of hanging.
__device__ __forceinline__ bool flag_wait(const int * f, int v) {
    for (int i = 0; i < kSpinLimit; ++i) {
        if (__hip_atomic_load(const_cast<int *>(f), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= v) return true;
        __builtin_amdgcn_s_sleep(1);
    }
    return false;
}

// First cell of a split's it-th tile: the split walks its tiles starting at
// tile rot (0 <= rot < nt) and wrapping around, so the workgroups of one kv
// head (which share its K/V through one XCD's L2) are spread over the cell
// range instead of all missing the same lines at the same time.
__device__ __forceinline__ int tile_cell(const int cb0, const int it, const int rot, const int nt) {
    const int j = it + rot;
    return cb0 + (j < nt ? j : j - nt) * kStride;
}

// After the softmax of tile it, a wave refills its half of the tile's stage
// with tile it + 2 once the other wave has read the stage (its own reads are
// complete: the wave waited for them before publishing its own "read").
__device__ __forceinline__ bool refill(const int h, const int it, const int nt, const int rot, const int * done,
                                       const int4v kd, const int4v vd, const uint32_t ring_addr, const int cb0,
                                       const uint32_t k_nb1, const uint32_t v_nb1, const int g, const int n) {
    if (it + 2 >= nt) return true;
    const bool ok = flag_wait(done, it);
    if (ok) issue_half(kd, vd, ring_addr + (uint32_t) ((it & 1) * kStage), (uint32_t) tile_cell(cb0, it + 2, rot, nt),
                       k_nb1, v_nb1, g, n, h);
    return ok;
}

// P = exp2(s c - m c) in f16, then O^T += V^T P^T and l += 1 P^T.
__device__ __forceinline__ void accumulate_tile(TileOps & t, const floatx4 (&s)[kPRB][2], const bool full,
                                                const bool (&vis_any)[8], const float (&m_run)[kPRB], const float cexp,
                                                const half8 ones, const int g, floatx4 (&o)[kPRB][8],
                                                floatx4 (&lacc)[kPRB]) {
    half8 pf[kPRB];
#pragma unroll
    for (int rb = 0; rb < kPRB; ++rb) {
        const float mc = (m_run[rb] == -AL_INF) ? 0.0f : m_run[rb] * cexp;
#pragma unroll
        for (int j = 0; j < 8; ++j)
            pf[rb][j] = (_Float16) __builtin_amdgcn_exp2f(__builtin_fmaf(s[rb][j >> 2][j & 3], cexp, -mc));
    }
    if (!full) {
        // cells masked for every row contribute exact zeros, whatever their V holds
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint64_t bal = __ballot(vis_any[j]);
            if (((bal >> (16 * g)) & 0xffffull) == 0) {
#pragma unroll
                for (int d = 0; d < 8; ++d) t.vt[d][j] = (_Float16) 0.0f;
            }
        }
    }
#pragma unroll
    for (int rb = 0; rb < kPRB; ++rb) {
#pragma unroll
        for (int d = 0; d < 8; ++d) o[rb][d] = mfma_16x16x32(t.vt[d], pf[rb], o[rb][d]);
        lacc[rb] = mfma_16x16x32(ones, pf[rb], lacc[rb]);
    }
}

template <bool SOFTCAP>
__global__ __launch_bounds__(kPW * 64) void fattn_prefill_kernel(const FattnParams p) {
    __shared__ __attribute__((aligned(1024))) char lds[kLds];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rh = wave & 1;                     // row half: rows 32 rh .. 32 rh + 31 of the tile
    const int cs = wave >> 1;                    // cell split: tiles cs, cs + kCS, ...
    const int g = lane >> 4;
    const int n = lane & 15;

    int id = blockIdx.x;
    const int kvh = id % p.Hkv;
    id /= p.Hkv;
    const int rt = p.causal_pos0 >= 0 ? p.n_row_tiles - 1 - id % p.n_row_tiles : id % p.n_row_tiles;
    const int b = id / p.n_row_tiles;
    const int row0 = rt * kPRows;
    const int rows_here = min(kPRows, p.R - row0);
    const int t_last = (row0 + rows_here - 1) / p.G;
    // gated behind the mask pass: the split-KV kernel takes a rejected mask
    if (p.gate && __hip_atomic_load(p.gate, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) return;
    int hi = p.kv_hi;
    if (p.causal_pos0 >= 0) hi = (int) min((int64_t) hi, p.causal_pos0 + t_last + 1);
    // with a mask tensor, each row's last visible cell from the mask pass;
    // lane l takes row l of the tile, the workgroup's cells end after the
    // largest of them
    auto mask_lim = [&](const int rr) {
        const int r = row0 + rr;
        const int hq = kvh * p.G + r % p.G;
        return p.row_lim[((int64_t) (b % p.m_ne3) * p.m_ne2 + hq % p.m_ne2) * p.T + r / p.G];
    };
    if (p.row_lim) {
        int mx = mask_lim(min(lane, rows_here - 1));
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) mx = max(mx, __shfl_xor(mx, off));
        hi = __builtin_amdgcn_readfirstlane(min(hi, mx + 1));          // the same in every lane
    }

    const char * kbase = p.k + (int64_t) (b / p.rk3) * p.k_nb3 + (int64_t) kvh * p.k_nb2;
    const char * vbase = p.v + (int64_t) (b / p.rv3) * p.v_nb3 + (int64_t) kvh * p.v_nb2;
    const uint32_t k_nb1 = (uint32_t) p.k_nb1, v_nb1 = (uint32_t) p.v_nb1;
    const int4v kd = raw_desc(kbase, (uint32_t) (p.n_kv - 1) * k_nb1 + 256);
    const int4v vd = raw_desc(vbase, (uint32_t) (p.n_kv - 1) * v_nb1 + 256);

    // this split's tiles: cells cb0 + i * kStride, i < nt, in the order of tile_cell
    const int cb0 = cs * 32;
    const int nt = cb0 < hi ? (hi - cb0 + kStride - 1) / kStride : 0;
    const int rot = nt > 0 ? (int) (((int64_t) rt * nt) / p.n_row_tiles) : 0;
    const char * ring = &lds[cs * kNB * kStage];
    const uint32_t ring_addr = lds_addr(ring);

    // The tile's query rows travel once, by LDS-DMA into the staging area
    // behind the rings, ahead of the first K/V tiles: wave w loads rows
    // 8w .. 8w + 7 (block i = rows 2i, 2i + 1 of 512 bytes each). Granule j
    // of row r sits at slot j ^ 2(r & 15), which spreads the reads below over
    // the LDS banks.
    char * qst = &lds[kRing];
    {
        const int4v qd = raw_desc(p.q + (int64_t) b * p.q_nb3, p.q_bytes);
        const uint32_t qslot = (uint32_t) (lane & 31);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = 8 * wave + 2 * i + (lane >> 5);
            const int rq = r < rows_here ? r : 0;
            const uint32_t qofs = (uint32_t) (((row0 + rq) / p.G) * p.q_nb1 + (kvh * p.G + (row0 + rq) % p.G) * p.q_nb2);
            dma16(qd, qofs + ((qslot ^ (uint32_t) (2 * (r & 15))) & 31) * 16,
                  lds_addr(qst) + (uint32_t) ((8 * wave + 2 * i) * 512));
        }
    }
    if (nt > 0) issue_half(kd, vd, ring_addr, (uint32_t) tile_cell(cb0, 0, rot, nt), k_nb1, v_nb1, g, n, rh);
    if (nt > 1) issue_half(kd, vd, ring_addr + kStage, (uint32_t) tile_cell(cb0, 1, rot, nt), k_nb1, v_nb1, g, n, rh);
    wait_later<2, 8>(min(nt, 2));                                     // own query rows landed
    __syncthreads();                                                   // everyone's

    // query rows held by this lane (column n of its two row blocks) and their
    // Q^T B-operand fragments (k slots of block kb, group g = dims 32kb + 8g..+8)
    int tok[kPRB];
    bool rvalid[kPRB];
    half8 qf[kPRB][4];
#pragma unroll
    for (int rb = 0; rb < kPRB; ++rb) {
        const int rr = 32 * rh + 16 * rb + n;
        rvalid[rb] = rr < rows_here;
        tok[rb] = rvalid[rb] ? (row0 + rr) / p.G : 0;
        const char * qrow = qst + rr * 512;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            const int j = 2 * (4 * kb + g);                               // granules j, j + 1 of row rr
            const float4 qa = *(const float4 *) (qrow + ((j ^ (2 * n)) & 31) * 16);
            const float4 qb = *(const float4 *) (qrow + (((j + 1) ^ (2 * n)) & 31) * 16);
            qf[rb][kb] = rvalid[rb] ? to_half8(qa, qb) : half8{0, 0, 0, 0, 0, 0, 0, 0};
        }
    }
    // the staging area becomes the flags: landed[cs][rh], then done[cs][rh]
    int * flags = (int *) qst;
    __syncthreads();
    if (threadIdx.x < 4 * kCS) flags[threadIdx.x] = -1;
    __syncthreads();
    int * landed = flags + 2 * cs + rh;                               // own half landed
    const int * landed_o = flags + 2 * cs + (rh ^ 1);                 // the other wave's half
    int * done_m = flags + 2 * kCS + 2 * cs + rh;                     // own reads of the stage done
    const int * done = flags + 2 * kCS + 2 * cs + (rh ^ 1);

    int lim[kPRB];
#pragma unroll
    for (int rb = 0; rb < kPRB; ++rb) lim[rb] = row_limit(p, hi, rvalid[rb], tok[rb]);
    int lim_min = row_limit(p, hi, true, (row0 + min(32 * rh, rows_here - 1)) / p.G);   // this wave's first token
    if (p.row_lim) {
        // the mask's limits, within the length / causal ones; lim_min: the
        // smallest over the wave's valid rows
        int mn = INT32_MAX;
#pragma unroll
        for (int rb = 0; rb < kPRB; ++rb) {
            if (rvalid[rb]) lim[rb] = min(lim[rb], mask_lim(32 * rh + 16 * rb + n));
            mn = min(mn, rvalid[rb] ? lim[rb] : INT32_MAX);
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) mn = min(mn, __shfl_xor(mn, off));
        lim_min = __builtin_amdgcn_readfirstlane(mn);
    }

    // p = exp2(s * cexp - m * cexp); the max is tracked on s as computed
    // (raw dot products, or softcapped scores in natural units)
    const float cexp = SOFTCAP ? kLog2e : p.scale * kLog2e;
    const float tau = kTau * kLog2e / cexp;                           // kTau in units of s
    half8 ones;
#pragma unroll
    for (int j = 0; j < 8; ++j) ones[j] = (_Float16) 1.0f;

    floatx4 o[kPRB][8];
    floatx4 lacc[kPRB];
    float m_run[kPRB];
#pragma unroll
    for (int rb = 0; rb < kPRB; ++rb) {
        m_run[rb] = -AL_INF;
        lacc[rb] = floatx4{0, 0, 0, 0};
#pragma unroll
        for (int d = 0; d < 8; ++d) o[rb][d] = floatx4{0, 0, 0, 0};
    }

    // Tile state shared by the fast loop and the rescale path below.
    TileOps t;
    floatx4 s[kPRB][2];
    float mt[kPRB];
    bool full = true;
    bool vis_any[8];
    bool ok = true;

    // The fast loop never scales O: a tile whose max would move the
    // reference (the first tile always does) leaves it, and the scaling
    // happens outside, so the accumulators stay in MFMA registers across
    // iterations instead of being copied for a rarely taken branch.
    int it = 0;
    while (it < nt && ok) {
        for (; it < nt; ++it) {
            // tile it in its stage: own half landed (vmcnt), the other's by its flag
            wait_later<1, 8>(it + 1 < nt ? 1 : 0);
            flag_set(landed, it);
            if (!flag_wait(landed_o, it)) {
                ok = false;
                break;
            }
            read_tile(t, ring + (it & 1) * kStage, lane, g, n);
            mem_barrier();
            __builtin_amdgcn_s_waitcnt(0xC00F | (7 << 4));                 // lgkmcnt(0): the stage is read
            mem_barrier();
            flag_set(done_m, it);
            const int cb = tile_cell(cb0, it, rot, nt);

            // S^T = K Q^T: cells 4g+i (mb 0) and 16+4g+i (mb 1) of row n
#pragma unroll
            for (int rb = 0; rb < kPRB; ++rb)
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) {
                    floatx4 acc = {0, 0, 0, 0};
#pragma unroll
                    for (int kb = 0; kb < 4; ++kb) acc = mfma_16x16x32(as_half8(t.k[mb][kb]), qf[rb][kb], acc);
                    s[rb][mb] = acc;
                }
            if constexpr (SOFTCAP) {
#pragma unroll
                for (int rb = 0; rb < kPRB; ++rb)
#pragma unroll
                    for (int j = 0; j < 8; ++j) s[rb][j >> 2][j & 3] = p.softcap * tanhf(s[rb][j >> 2][j & 3] * p.scale);
            }
            full = cb + 31 <= lim_min;
#pragma unroll
            for (int j = 0; j < 8; ++j) vis_any[j] = true;
            if (!full) {
#pragma unroll
                for (int j = 0; j < 8; ++j) vis_any[j] = false;
#pragma unroll
                for (int rb = 0; rb < kPRB; ++rb)
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const bool vis = cb + cell_of_slot(g, j) <= lim[rb];
                        s[rb][j >> 2][j & 3] = vis ? s[rb][j >> 2][j & 3] : -AL_INF;
                        vis_any[j] = vis_any[j] || vis;
                    }
            }
            // lane-local maxima suffice to see that no score passes its row's
            // reference by more than tau; the row maxima (a cross-lane
            // reduction) are formed only on the rare path that moves it
            bool grow_any = false;
#pragma unroll
            for (int rb = 0; rb < kPRB; ++rb) {
                const float a = fmaxf(fmaxf(s[rb][0][0], s[rb][0][1]), s[rb][0][2]);
                const float c = fmaxf(fmaxf(s[rb][0][3], s[rb][1][0]), s[rb][1][1]);
                mt[rb] = fmaxf(fmaxf(s[rb][1][2], s[rb][1][3]), fmaxf(a, c));
                grow_any = grow_any || (mt[rb] > m_run[rb] + tau);
            }
            if (__any(grow_any)) break;
            accumulate_tile(t, s, full, vis_any, m_run, cexp, ones, g, o, lacc);
            if (!refill(rh, it, nt, rot, done, kd, vd, ring_addr, cb0, k_nb1, v_nb1, g, n)) {
                ok = false;
                break;
            }
        }
        if (it >= nt || !ok) break;
        // tile `it` moves the reference max of some rows: scale, then finish it
#pragma unroll
        for (int rb = 0; rb < kPRB; ++rb) {
            mt[rb] = colmax4(mt[rb]);                                     // the row's max, same in its 4 lanes
            const bool grow = mt[rb] > m_run[rb] + tau;
            const float mn = grow ? mt[rb] : m_run[rb];
            const float alpha = grow ? __builtin_amdgcn_exp2f((m_run[rb] - mn) * cexp) : 1.0f;   // 0 from -inf
            lacc[rb] *= alpha;
#pragma unroll
            for (int d = 0; d < 8; ++d) o[rb][d] *= alpha;
            m_run[rb] = mn;
        }
        accumulate_tile(t, s, full, vis_any, m_run, cexp, ones, g, o, lacc);
        ok = refill(rh, it, nt, rot, done, kd, vd, ring_addr, cb0, k_nb1, v_nb1, g, n);
        ++it;
    }
    if (!ok && lane == 0) atomicOr(p.err + 2, 1);                      // reported by al_device_errors
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));                          // no DMA may still target LDS

    // natural-unit max and the row sums (every element of lacc holds l)
    float m_nat[kPRB], l_run[kPRB];
#pragma unroll
    for (int rb = 0; rb < kPRB; ++rb) {
        m_nat[rb] = m_run[rb] == -AL_INF ? -AL_INF : m_run[rb] * (cexp / kLog2e);
        l_run[rb] = lacc[rb][0];
    }

    // Merge: every wave publishes its 32-row state to LDS [split][row][132]
    // (the rings are free once all waves are past their loops), then the
    // workgroup combines the 4 splits of each (row, 4 dims) and writes it.
    __syncthreads();
    float * recs = (float *) &lds[0];
    {
        float * rec = recs + cs * (kPRows * kRowStride);
#pragma unroll
        for (int rb = 0; rb < kPRB; ++rb) {
            float * row = rec + (32 * rh + 16 * rb + n) * kRowStride;
#pragma unroll
            for (int d = 0; d < 8; ++d) *(float4 *) (row + 16 * d + 4 * g) = float4{o[rb][d][0], o[rb][d][1], o[rb][d][2], o[rb][d][3]};
            if (g == 0) *(float2 *) (row + 128) = float2{m_nat[rb], l_run[rb]};
        }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kPRows * 32 / (kPW * 64); ++k) {
        const int item = k * kPW * 64 + threadIdx.x;
        const int rr = item >> 5, d4 = item & 31;
        if (rr >= rows_here) continue;
        float2 ml[kCS];
        float M = -AL_INF;
#pragma unroll
        for (int c = 0; c < kCS; ++c) {
            ml[c] = *(const float2 *) (recs + (c * kPRows + rr) * kRowStride + 128);
            M = fmaxf(M, ml[c].x);
        }
        const float Mu = (M == -AL_INF) ? 0.0f : M;
        float L = 0.0f;
        float4 acc = {0, 0, 0, 0};
#pragma unroll
        for (int c = 0; c < kCS; ++c) {
            const float w = exp_fast(ml[c].x - Mu);
            L += w * ml[c].y;
            const float4 x = *(const float4 *) (recs + (c * kPRows + rr) * kRowStride + 4 * d4);
            acc.x += w * x.x; acc.y += w * x.y; acc.z += w * x.z; acc.w += w * x.w;
        }
        const int tk = (row0 + rr) / p.G;
        const int hq = kvh * p.G + (row0 + rr) % p.G;
        float * out = (float *) (p.dst + ((int64_t) (b * p.T + tk) * p.Hq + hq) * p.dst_nb1);
        *(float4 *) (out + 4 * d4) = finalize4(acc, M, L, p.sinks, hq);
    }
}

// One workgroup per mask row (token t of mask slice (i2, i3)) over cells
// [0, n_kv): the last cell holding +-0 (-1 if none) into lims, and 1 into
// gate[0] when the row is not a run of zeros followed by -inf (another
// value, or a zero after a -inf).
__global__ __launch_bounds__(256) void mask_limits_kernel(const FattnParams p, int32_t * lims, int * gate) {
    const int t = blockIdx.x, i2 = blockIdx.y, i3 = blockIdx.z;
    const uint16_t * row = (const uint16_t *) (p.mask + (int64_t) t * p.m_nb1 + (int64_t) i2 * p.m_nb2 + (int64_t) i3 * p.m_nb3);
    int last0 = -1, first_inf = INT32_MAX, bad = 0;
    for (int c = threadIdx.x; c < p.n_kv; c += blockDim.x) {
        const uint16_t h = row[c];
        if ((h & 0x7fffu) == 0) last0 = c;
        else if (h == 0xfc00u) first_inf = min(first_inf, c);
        else bad = 1;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        last0 = max(last0, __shfl_xor(last0, off));
        first_inf = min(first_inf, __shfl_xor(first_inf, off));
        bad |= __shfl_xor(bad, off);
    }
    __shared__ int s[3][4];
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        s[0][w] = last0;
        s[1][w] = first_inf;
        s[2][w] = bad;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < (int) (blockDim.x >> 6); ++i) {
            last0 = max(last0, s[0][i]);
            first_inf = min(first_inf, s[1][i]);
            bad |= s[2][i];
        }
        lims[((int64_t) i3 * p.m_ne2 + i2) * p.T + t] = last0;
        if (bad || last0 > first_inf) __hip_atomic_store(gate, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

}  // namespace

hipError_t fattn_mask_limits_launch(const FattnParams & p, int32_t * lims, int * gate, hipStream_t stream) {
    const dim3 grid((unsigned) p.T, (unsigned) p.m_ne2, (unsigned) p.m_ne3);
    hipLaunchKernelGGL(mask_limits_kernel, grid, dim3(256), 0, stream, p, lims, gate);
    return hipGetLastError();
}

size_t fattn_prefill_lds_bytes() { return (size_t) kLds; }

hipError_t fattn_prefill_launch(const FattnParams & p, hipStream_t stream) {
    const dim3 grid((unsigned) ((int64_t) p.Hkv * p.n_row_tiles * p.B));
    if (p.softcap != 0.0f) hipLaunchKernelGGL(fattn_prefill_kernel<true>, grid, dim3(kPW * 64), 0, stream, p);
    else                   hipLaunchKernelGGL(fattn_prefill_kernel<false>, grid, dim3(kPW * 64), 0, stream, p);
    return hipGetLastError();
}
