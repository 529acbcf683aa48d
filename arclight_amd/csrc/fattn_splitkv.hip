// Split-KV GQA flash attention for gfx950: decode, speculative verify, and
// (until the dedicated prefill kernel takes over) row-tiled prefill.
//
// Semantics follow nnml_compute_forward_flash_attn_ext_f16
// (nnml/src/ops/arm/arm.cpp:2196-2433): per query row, softmax over the
// visible KV cells of scale * (f16(q) . k) [softcap] + slope * mask, times V,
// optional sinks, 1/S, stored at row (i3*T + i1)*Hq + i2 (arm.cpp:2431).
// Cells whose mask is -inf are skipped (arm.cpp:2327-2330). Accumulation is
// f32; q is rounded to f16 once (arm.cpp:2322), as the reference does.
//
// Work decomposition (one workgroup = W wavefronts):
//   blockIdx.x  split of the visible cell range (split-KV)
//   blockIdx.y  kv head + Hkv * row tile
//   blockIdx.z  stream (nnml dim 3)
// A row tile packs ROWS = 16*RB query rows of ONE kv-head group:
// row r -> token r / G, head kvh*G + r % G, so every K/V byte a wavefront
// loads serves all G heads of the group and all tokens of the tile.
// The W waves of a workgroup take interleaved 32-cell tiles of the split and
// merge their online-softmax states through LDS (a tree); the last
// workgroup of a row tile to finish merges all splits (single level, at most
// kFattnMaxSplit records, every load in flight at once) and stores dst.
//
// Per 32-cell tile a wavefront does, with no LDS:
//   S^T[32 cells x 16 rows]  = K[32 x 128] * Q^T    8 MFMA 16x16x32 per row block
//   O^T[128 dims x 16 rows] += V^T[128 x 32] * P^T  8 MFMA 16x16x32 per row block
// K goes from HBM straight into MFMA A-operand registers (16-byte buffer
// loads). V is loaded as 8 cells x 8 dims per lane (each load instruction
// reads 4 whole 256-byte rows) and transposed in registers: the A-operand
// row m of block mb' is dim 8m + mb', so no lane exchange is needed. The cell
// order of the k slots matches the MFMA output layout of S^T, so P^T is
// built from S^T in place. Each lane's O^T holds 32 consecutive dims of one
// query row. Two tile buffers alternate so one tile's loads are in flight
// while the other computes.

#include "device_common.hpp"
#include "fattn_kernels.hpp"

namespace {

constexpr int kTile = 32;                         // cells per wave iteration
constexpr int kRowStride = kFattnRecordStride;    // floats per merge-record row: O[128], m, l, pad
constexpr int kMaxSplit = kFattnMaxSplit;

typedef __amdgpu_buffer_rsrc_t rsrc_t;

// Raw buffer over [base, base + bytes): 32-bit offsets, loads past the end
// return zeros.
__device__ __forceinline__ rsrc_t make_rsrc(const void * base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int) bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 buf_load16(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int) off, 0, 0);
}
// Device-coherent (sc1) stores / loads of merge records, see st_agent.
constexpr int kCoherent = 16;
__device__ __forceinline__ void buf_store16_dev(float4 v, rsrc_t r, uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, (int) off, 0, kCoherent);
}
__device__ __forceinline__ float4 buf_load16_dev(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, (int) off, 0, kCoherent));
}
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void buf_store8_dev(float2 v, rsrc_t r, uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), r, (int) off, 0, kCoherent);
}
__device__ __forceinline__ float2 buf_load8_dev(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(r, (int) off, 0, kCoherent));
}

template <int RB>
struct Tile {
    u32x4 k[2][4];                   // [mb][kb] K A-operand chunks
    u32x4 v[8];                      // 8 cells x 8 dims (chunk n)
    uint32_t mk[RB][4];              // mask f16 pairs, cells of S^T layout (slots 2i, 2i+1)
};

__device__ __forceinline__ int cell_of_slot(int g, int j) {
    // k slot j of lane group g <-> cell offset within a 32-cell tile
    return (j < 4) ? (4 * g + j) : (16 + 4 * g + (j - 4));
}

template <int RB, bool HAS_MASK>
__device__ __forceinline__ void load_tile(Tile<RB> & t, const FattnParams & p, const rsrc_t kr, const rsrc_t vr,
                                          const uint16_t * const * mrow, const int cb, const int g, const int n) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
        const uint32_t off = (uint32_t) (cb + 16 * mb + n) * (uint32_t) p.k_nb1;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) t.k[mb][kb] = buf_load16(kr, off + (4 * kb + g) * 16);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) t.v[j] = buf_load16(vr, (uint32_t) (cb + cell_of_slot(g, j)) * (uint32_t) p.v_nb1 + n * 16);
    if constexpr (HAS_MASK) {
        // unconditional loads from clamped addresses, selected afterwards: the
        // number of loads per tile is fixed, so the next tile's loads stay in
        // flight while this one computes
        const int lastc = p.m_ne0 - 1;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const uint16_t * mp = mrow[rb] ? mrow[rb] : (const uint16_t *) p.mask;
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                const int c0 = cb + cell_of_slot(g, 2 * jj);
                uint32_t lo = mp[min(c0, lastc)];
                uint32_t hi = mp[min(c0 + 1, lastc)];
                lo = (mrow[rb] && c0 <= lastc) ? lo : 0xfc00u;             // -inf
                hi = (mrow[rb] && c0 + 1 <= lastc) ? hi : 0xfc00u;
                t.mk[rb][jj] = lo | (hi << 16);
            }
        }
    }
}

// One merge record (O[128], m, l per query row) in LDS.
template <int RB>
__device__ __forceinline__ void store_state(float * rec, const floatx4 (&o)[RB][8], const float (&m)[RB],
                                            const float (&l)[RB], int g, int n) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        float * row = rec + (16 * rb + n) * kRowStride;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            *(float4 *) (row + 32 * g + 8 * i) = float4{o[rb][0][i], o[rb][1][i], o[rb][2][i], o[rb][3][i]};
            *(float4 *) (row + 32 * g + 8 * i + 4) = float4{o[rb][4][i], o[rb][5][i], o[rb][6][i], o[rb][7][i]};
        }
        if (g == 0) *(float2 *) (row + 128) = float2{m[rb], l[rb]};
    }
}

template <int RB>
__device__ __forceinline__ void merge_state(const float * rec, floatx4 (&o)[RB][8], float (&m)[RB],
                                            float (&l)[RB], int g, int n) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const float * row = rec + (16 * rb + n) * kRowStride;
        const float2 ml = *(const float2 *) (row + 128);
        const float mn = fmaxf(m[rb], ml.x);
        const float mu = (mn == -AL_INF) ? 0.0f : mn;
        const float wa = exp_fast(m[rb] - mu);
        const float wb = exp_fast(ml.x - mu);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 lo = *(const float4 *) (row + 32 * g + 8 * i);
            const float4 hi = *(const float4 *) (row + 32 * g + 8 * i + 4);
            o[rb][0][i] = o[rb][0][i] * wa + lo.x * wb;
            o[rb][1][i] = o[rb][1][i] * wa + lo.y * wb;
            o[rb][2][i] = o[rb][2][i] * wa + lo.z * wb;
            o[rb][3][i] = o[rb][3][i] * wa + lo.w * wb;
            o[rb][4][i] = o[rb][4][i] * wa + hi.x * wb;
            o[rb][5][i] = o[rb][5][i] * wa + hi.y * wb;
            o[rb][6][i] = o[rb][6][i] * wa + hi.z * wb;
            o[rb][7][i] = o[rb][7][i] * wa + hi.w * wb;
        }
        l[rb] = l[rb] * wa + ml.y * wb;
        m[rb] = mn;
    }
}

// The workgroup's merged state as a global merge record, written with
// device-coherent stores for the merging workgroup of this launch.
template <int RB>
__device__ __forceinline__ void publish_state(const rsrc_t rr, uint32_t rec_off, const floatx4 (&o)[RB][8],
                                              const float (&m)[RB], const float (&l)[RB], int g, int n,
                                              int rows_here) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        if (16 * rb + n >= rows_here) continue;
        const uint32_t row = rec_off + (uint32_t) (16 * rb + n) * kRowStride * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            buf_store16_dev(float4{o[rb][0][i], o[rb][1][i], o[rb][2][i], o[rb][3][i]}, rr, row + (32 * g + 8 * i) * 4);
            buf_store16_dev(float4{o[rb][4][i], o[rb][5][i], o[rb][6][i], o[rb][7][i]}, rr, row + (32 * g + 8 * i + 4) * 4);
        }
        if (g == 0) buf_store8_dev(float2{m[rb], l[rb]}, rr, row + 128 * 4);
    }
}

// Sinks (arm.cpp:2402-2416) and 1/S (arm.cpp:2419-2420) on one 4-dim group.
__device__ __forceinline__ float4 finalize4(float4 o, float M, float L, const float * sinks, int head) {
    if (sinks) {
        const float s = sinks[head];
        if (s > M) {
            const float ms = expf(M - s);
            o.x *= ms; o.y *= ms; o.z *= ms; o.w *= ms;
            L = L * ms + 1.0f;
        } else {
            L = L + expf(s - M);
        }
    }
    const float inv = 1.0f / L;
    o.x *= inv; o.y *= inv; o.z *= inv; o.w *= inv;
    return o;
}

// Merges the n_split (<= kMaxSplit) records of one row tile (record stride
// ROWS*kRowStride floats) into dst. One thread per (row, 4 dims); all of a
// thread's record loads are issued before any is used; fixed merge order.
template <int ROWS>
__device__ __forceinline__ void merge_splits(const rsrc_t rr, const int n_split, const int rows_here,
                                             const FattnParams & p, const int b, const int kvh, const int row0,
                                             const int nthreads) {
    for (int idx = threadIdx.x; idx < rows_here * 32; idx += nthreads) {
        const int r = idx >> 5;
        const int d4 = idx & 31;
        float2 ml[kMaxSplit];
        float4 ov[kMaxSplit];
#pragma unroll
        for (int sp = 0; sp < kMaxSplit; ++sp) {
            if (sp < n_split) {
                const uint32_t row = (uint32_t) ((sp * ROWS + r) * kRowStride) * 4;
                ml[sp] = buf_load8_dev(rr, row + 128 * 4);
                ov[sp] = buf_load16_dev(rr, row + d4 * 16);
            } else {
                ml[sp] = float2{-AL_INF, 0.0f};
                ov[sp] = float4{0, 0, 0, 0};
            }
        }
        float M = ml[0].x;
#pragma unroll
        for (int sp = 1; sp < kMaxSplit; ++sp) M = fmaxf(M, ml[sp].x);
        const float Mu = (M == -AL_INF) ? 0.0f : M;
        float L = 0.0f;
        float4 acc = {0, 0, 0, 0};
#pragma unroll
        for (int sp = 0; sp < kMaxSplit; ++sp) {
            const float w = exp_fast(ml[sp].x - Mu);
            L += w * ml[sp].y;
            acc.x += w * ov[sp].x; acc.y += w * ov[sp].y; acc.z += w * ov[sp].z; acc.w += w * ov[sp].w;
        }
        const int rr_ = row0 + r;
        const int t = rr_ / p.G;
        const int h = kvh * p.G + rr_ % p.G;
        float * out = (float *) (p.dst + ((int64_t) (b * p.T + t) * p.Hq + h) * p.dst_nb1);
        *(float4 *) (out + 4 * d4) = finalize4(acc, M, L, p.sinks, h);
    }
}

// One 32-cell tile of one wavefront: S^T = K Q^T, scale/softcap/mask,
// online softmax update, O^T += V^T P^T.
template <int RB, bool HAS_MASK>
__device__ __forceinline__ void process_tile(Tile<RB> & cur, const int cb, const FattnParams & p, const int g, const int hi,
                                             const bool (&rvalid)[RB], const int (&tok)[RB], const float (&slope)[RB],
                                             const half8 (&qf)[RB][4], floatx4 (&o)[RB][8], float (&m_run)[RB],
                                             float (&l_run)[RB]) {
    // S^T = K Q^T
    floatx4 s[RB][2];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
            floatx4 acc = {0, 0, 0, 0};
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) acc = mfma_16x16x32(as_half8(cur.k[mb][kb]), qf[rb][kb], acc);
            s[rb][mb] = acc;
        }
    }

    // scale, softcap, mask (arm.cpp:2327-2343); invisible -> -inf
    bool vis_any[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) vis_any[j] = false;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int mb = j >> 2, i = j & 3;
            const int cell = cb + cell_of_slot(g, j);
            bool vis = rvalid[rb] && cell < hi;
            if (p.causal_pos0 >= 0) vis = vis && ((int64_t) cell <= p.causal_pos0 + tok[rb]);
            float x = s[rb][mb][i] * p.scale;
            if (p.softcap != 0.0f) x = p.softcap * tanhf(x);
            if constexpr (HAS_MASK) {
                const float mv = slope[rb] * f16_bits_to_float((uint16_t) (cur.mk[rb][j >> 1] >> (16 * (j & 1))));
                vis = vis && (mv != -AL_INF);
                x += mv;
            }
            s[rb][mb][i] = vis ? x : -AL_INF;
            vis_any[j] = vis_any[j] || vis;
        }
    }

    // online softmax; P^T operand built in place from the S^T layout
    half8 pf[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        float mt = fmaxf(fmaxf(fmaxf(s[rb][0][0], s[rb][0][1]), fmaxf(s[rb][0][2], s[rb][0][3])),
                         fmaxf(fmaxf(s[rb][1][0], s[rb][1][1]), fmaxf(s[rb][1][2], s[rb][1][3])));
        mt = colmax4(mt);
        const float mn = fmaxf(m_run[rb], mt);
        const float mu = (mn == -AL_INF) ? 0.0f : mn;
        const float alpha = exp_fast(m_run[rb] - mu);
        float ps = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float pr = exp_fast(s[rb][j >> 2][j & 3] - mu);
            ps += pr;
            pf[rb][j] = (_Float16) pr;
        }
        l_run[rb] = l_run[rb] * alpha + ps;
        m_run[rb] = mn;
#pragma unroll
        for (int d = 0; d < 8; ++d) o[rb][d] *= alpha;
    }

    // cells masked for every row of the tile contribute exact zeros
    // (their memory may hold anything, e.g. unwritten cache cells)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint64_t bal = __ballot(vis_any[j]);
        if (((bal >> (16 * g)) & 0xffffull) == 0) cur.v[j] = u32x4{0, 0, 0, 0};
    }

    // V^T A-operands: block mb' = 2*pp + h holds dim 8n + mb' of the 8 cells
    half8 vt[8];
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
        u32x4 lo16, hi16;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t a = cur.v[2 * q][pp];
            const uint32_t c = cur.v[2 * q + 1][pp];
            lo16[q] = (a & 0xffffu) | (c << 16);
            hi16[q] = (a >> 16) | (c & 0xffff0000u);
        }
        vt[2 * pp] = as_half8(lo16);
        vt[2 * pp + 1] = as_half8(hi16);
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
        for (int d = 0; d < 8; ++d) o[rb][d] = mfma_16x16x32(vt[d], pf[rb], o[rb][d]);
    }
}

template <int RB, int W, bool PREFETCH, bool HAS_MASK>
__global__ __launch_bounds__(W * 64) void fattn_splitkv_kernel(const FattnParams p) {
    constexpr int ROWS = 16 * RB;
    constexpr int NSLOT = W / 2;                   // LDS records of the wave-merge tree
    __shared__ float lds[NSLOT * ROWS * kRowStride];
    __shared__ int s_last;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int g = lane >> 4;
    const int n = lane & 15;
    const int split = blockIdx.x;
    const int kvh = blockIdx.y % p.Hkv;
    const int rt = blockIdx.y / p.Hkv;
    const int b = blockIdx.z;
    const int row0 = rt * ROWS;
    const int rows_here = min(ROWS, p.R - row0);
    const int t_last = (row0 + rows_here - 1) / p.G;

    int hi = p.kv_hi;
    if (p.causal_pos0 >= 0) hi = (int) min((int64_t) hi, p.causal_pos0 + t_last + 1);
    const int c_begin = split * p.cells_per_split;
    const int c_end = min(c_begin + p.cells_per_split, hi);

    // K/V of this (stream, kv head) as raw buffers: 32-bit offsets
    const char * kbase = p.k + (int64_t) (b / p.rk3) * p.k_nb3 + (int64_t) kvh * p.k_nb2;
    const char * vbase = p.v + (int64_t) (b / p.rv3) * p.v_nb3 + (int64_t) kvh * p.v_nb2;
    const rsrc_t kr = make_rsrc(kbase, (uint32_t) ((p.n_kv - 1) * p.k_nb1 + 256));
    const rsrc_t vr = make_rsrc(vbase, (uint32_t) ((p.n_kv - 1) * p.v_nb1 + 256));

    // query rows held by this lane (column n of every row block)
    int tok[RB];
    int head[RB];
    bool rvalid[RB];
    float slope[RB];
    const uint16_t * mrow[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int r = row0 + 16 * rb + n;
        rvalid[rb] = (16 * rb + n) < rows_here;
        tok[rb] = rvalid[rb] ? r / p.G : 0;
        head[rb] = kvh * p.G + (rvalid[rb] ? r % p.G : 0);
        mrow[rb] = nullptr;
        if (HAS_MASK && rvalid[rb]) {
            mrow[rb] = (const uint16_t *) (p.mask + (int64_t) tok[rb] * p.m_nb1 +
                                           (int64_t) (head[rb] % p.m_ne2) * p.m_nb2 +
                                           (int64_t) (b % p.m_ne3) * p.m_nb3);
        }
    }

    // the first tile's loads go out before anything else waits on memory
    constexpr int kStride = W * kTile;
    const int cb = c_begin + wave * kTile;
    const int ntiles = cb < c_end ? (c_end - cb + kStride - 1) / kStride : 0;
    const int c_last = cb + max(ntiles - 1, 0) * kStride;
    Tile<RB> ta, tb;
    if (ntiles > 0) load_tile<RB, HAS_MASK>(ta, p, kr, vr, mrow, cb, g, n);

    // Q^T B-operand fragments: k slots of block kb, group g = dims 8*(4kb+g)..+8
    half8 qf[RB][4];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const float * qrow = (const float *) (p.q + (int64_t) b * p.q_nb3 + (int64_t) tok[rb] * p.q_nb1 +
                                              (int64_t) head[rb] * p.q_nb2);
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            const float4 a = *(const float4 *) (qrow + 8 * (4 * kb + g));
            const float4 c = *(const float4 *) (qrow + 8 * (4 * kb + g) + 4);
            qf[rb][kb] = rvalid[rb] ? to_half8(a, c) : half8{0, 0, 0, 0, 0, 0, 0, 0};
        }
        slope[rb] = 1.0f;
        if (p.max_bias > 0.0f) {                                   // arm.cpp:2294
            const uint32_t h = (uint32_t) head[rb];
            slope[rb] = h < p.n_head_log2 ? powf(p.m0, (float) (h + 1))
                                          : powf(p.m1, (float) (2 * (h - p.n_head_log2) + 1));
        }
    }

    floatx4 o[RB][8];
    float m_run[RB];
    float l_run[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        m_run[rb] = -AL_INF;
        l_run[rb] = 0.0f;
#pragma unroll
        for (int d = 0; d < 8; ++d) o[rb][d] = floatx4{0, 0, 0, 0};
    }

    if constexpr (PREFETCH) {
        // Two register buffers in turn: one tile's loads are in flight while
        // the other tile computes. Every phase issues its loads
        // unconditionally (a prefetch past the range re-reads this wave's
        // last tile, an L2 hit) and the loop has one exit, so the wait before
        // each tile counts only that tile's loads.
        for (int it = 0; it < ntiles; it += 2) {
            const int c0 = cb + it * kStride;
            load_tile<RB, HAS_MASK>(tb, p, kr, vr, mrow, min(c0 + kStride, c_last), g, n);
            process_tile<RB, HAS_MASK>(ta, c0, p, g, hi, rvalid, tok, slope, qf, o, m_run, l_run);
            load_tile<RB, HAS_MASK>(ta, p, kr, vr, mrow, min(c0 + 2 * kStride, c_last), g, n);
            if (it + 1 < ntiles) process_tile<RB, HAS_MASK>(tb, c0 + kStride, p, g, hi, rvalid, tok, slope, qf, o, m_run, l_run);
        }
    } else {
        for (int it = 0; it < ntiles; ++it) {
            if (it > 0) load_tile<RB, HAS_MASK>(ta, p, kr, vr, mrow, cb + it * kStride, g, n);
            process_tile<RB, HAS_MASK>(ta, cb + it * kStride, p, g, hi, rvalid, tok, slope, qf, o, m_run, l_run);
        }
    }

#pragma unroll
    for (int rb = 0; rb < RB; ++rb) l_run[rb] = colsum4(l_run[rb]);

    // merge the W waves: a tree through NSLOT LDS records
#pragma unroll
    for (int span = W / 2; span >= 1; span /= 2) {
        if (wave >= span && wave < 2 * span) store_state<RB>(lds + (wave - span) * ROWS * kRowStride, o, m_run, l_run, g, n);
        __syncthreads();
        if (wave < span) merge_state<RB>(lds + wave * ROWS * kRowStride, o, m_run, l_run, g, n);
        __syncthreads();
    }

    if (p.n_split == 1) {
        if (wave == 0) {
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                if (!rvalid[rb]) continue;
                float * out = (float *) (p.dst + ((int64_t) (b * p.T + tok[rb]) * p.Hq + head[rb]) * p.dst_nb1);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float4 lo = {o[rb][0][i], o[rb][1][i], o[rb][2][i], o[rb][3][i]};
                    const float4 hi4 = {o[rb][4][i], o[rb][5][i], o[rb][6][i], o[rb][7][i]};
                    *(float4 *) (out + 32 * g + 8 * i) = finalize4(lo, m_run[rb], l_run[rb], p.sinks, head[rb]);
                    *(float4 *) (out + 32 * g + 8 * i + 4) = finalize4(hi4, m_run[rb], l_run[rb], p.sinks, head[rb]);
                }
            }
        }
        return;
    }

    // Split-KV: publish this split's record; the last workgroup of the row
    // tile to arrive merges all records of the tile into dst.
    const int64_t tile_id = ((int64_t) b * p.Hkv + kvh) * p.n_row_tiles + rt;
    constexpr uint32_t RS = ROWS * kRowStride * 4;                // record bytes
    const rsrc_t rr = make_rsrc(p.part + tile_id * (int64_t) p.n_split * (ROWS * kRowStride), RS * p.n_split);
    unsigned * cnt = p.counters + tile_id;
    if (wave == 0) publish_state<RB>(rr, RS * split, o, m_run, l_run, g, n, rows_here);
    complete_wave_memops();
    __syncthreads();
    if (threadIdx.x == 0) s_last = (add_agent(cnt, 1u) == (unsigned) (p.n_split - 1));
    __syncthreads();
    if (!s_last) return;
    order_after_counter();
    if (threadIdx.x == 0) st_agent_u32(cnt, 0u);              // ready for the next call in stream order
    merge_splits<ROWS>(rr, p.n_split, rows_here, p, b, kvh, row0, W * 64);
}

}  // namespace

int fattn_splitkv_rows_per_tile(int R) {
    return R <= 16 ? 16 : (R <= 32 ? 32 : 64);
}

int fattn_splitkv_waves(int rows_per_tile) {
    return rows_per_tile == 16 ? 8 : (rows_per_tile == 32 ? 4 : 2);
}

hipError_t fattn_splitkv_launch(const FattnParams & p, int rows_per_tile, hipStream_t stream) {
    const dim3 grid((unsigned) p.n_split, (unsigned) (p.Hkv * p.n_row_tiles), (unsigned) p.B);
    const bool m = p.mask != nullptr;
    switch (rows_per_tile) {
        case 16:
            if (m) hipLaunchKernelGGL((fattn_splitkv_kernel<1, 8, true, true>), grid, dim3(512), 0, stream, p);
            else   hipLaunchKernelGGL((fattn_splitkv_kernel<1, 8, true, false>), grid, dim3(512), 0, stream, p);
            break;
        case 32:
            if (m) hipLaunchKernelGGL((fattn_splitkv_kernel<2, 4, true, true>), grid, dim3(256), 0, stream, p);
            else   hipLaunchKernelGGL((fattn_splitkv_kernel<2, 4, true, false>), grid, dim3(256), 0, stream, p);
            break;
        case 64:
            if (m) hipLaunchKernelGGL((fattn_splitkv_kernel<4, 2, false, true>), grid, dim3(128), 0, stream, p);
            else   hipLaunchKernelGGL((fattn_splitkv_kernel<4, 2, false, false>), grid, dim3(128), 0, stream, p);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}
