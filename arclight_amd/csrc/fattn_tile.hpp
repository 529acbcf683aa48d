// Device building blocks of the attention kernels: tile loads, the per-tile
// MFMA + online-softmax step, wave / split merge records and finalization.
// Layouts and semantics are documented in fattn_splitkv.hip.
#pragma once

#include "device_common.hpp"
#include "fattn_kernels.hpp"
#include "kernel_args.hpp"

namespace fattn {

constexpr int kTile = 32;                         // cells per wave iteration
constexpr int kRowStride = kFattnRecordStride;    // floats per merge-record row: O[128], m, l, pad
constexpr int kMaxSplit = kFattnMaxSplit;
constexpr float kTau = 8.0f;                      // lazy-rescale threshold (natural log units)

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
// Non-temporal (nt) cache policy: output rows that no later access of the
// launch reads.
constexpr int kNonTemporal = 2;
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

// Last visible cell of a query row under the length / causal rule.
__device__ __forceinline__ int row_limit(const int64_t causal_pos0, const int hi, const bool valid, const int tok) {
    if (!valid) return -1;
    int64_t lim = hi - 1;
    if (causal_pos0 >= 0) lim = min(lim, causal_pos0 + tok);
    return (int) lim;
}
__device__ __forceinline__ int row_limit(const FattnParams & p, const int hi, const bool valid, const int tok) {
    return row_limit(p.causal_pos0, hi, valid, tok);
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
// r / G for the row index r of a kv-head group: a multiply-high by
// magic = ceil(2^32 / G) (exact for r G < 2^32, which the plan checks), or r
// itself for G = 1.
__device__ __forceinline__ int div_g(const int r, const int G, const uint32_t magic) {
    return G == 1 ? r : (int) __umulhi((uint32_t) r, magic);
}

// The same finalisation split into a per-row part (once per row) and a
// per-value part: o_out = (o * ms) * inv, ms = 1 unless a sink outweighs M.
struct RowScale {
    float ms, inv;
};
__device__ __forceinline__ RowScale row_scale(float M, float L, const float * sinks, int head) {
    float ms = 1.0f;
    if (sinks) {
        const float s = sinks[head];
        if (s > M) {
            ms = expf(M - s);
            L = L * ms + 1.0f;
        } else {
            L = L + expf(s - M);
        }
    }
    return RowScale{ms, 1.0f / L};
}
__device__ __forceinline__ float4 apply_scale(float4 o, const RowScale r) {
    o.x *= r.ms; o.y *= r.ms; o.z *= r.ms; o.w *= r.ms;
    o.x *= r.inv; o.y *= r.inv; o.z *= r.inv; o.w *= r.inv;
    return o;
}

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
// Scores of one 32-cell tile of one wavefront: S^T = K Q^T, then scale,
// softcap and mask (arm.cpp:2327-2343); invisible cells become -inf, and
// vis_any[j] tells whether slot j's cell is visible to some row of the
// lane's group. Returns through mt the tile max of each of the lane's rows.
// lim[rb]: the last visible cell of this lane's row in row block rb under the
// length / causal rule (-1 for padding rows); lim_min: the smallest lim of
// any real row of the tile (wave-uniform). A tile whose cells all lie at or
// below lim_min is fully visible and skips the masking work.
template <int RB, bool HAS_MASK>
__device__ __forceinline__ bool score_tile(const Tile<RB> & cur, const int cb, const FattnParams & p, const int g,
                                           const int (&lim)[RB], const int lim_min, const float (&slope)[RB],
                                           const half8 (&qf)[RB][4], floatx4 (&s)[RB][2], float (&mt)[RB],
                                           bool (&vis_any)[8]) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
            floatx4 acc = {0, 0, 0, 0};
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) acc = mfma_16x16x32(as_half8(cur.k[mb][kb]), qf[rb][kb], acc);
            s[rb][mb] = acc * p.scale;
        }
    }
    if (p.softcap != 0.0f) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int j = 0; j < 8; ++j) s[rb][j >> 2][j & 3] = p.softcap * tanhf(s[rb][j >> 2][j & 3]);
    }
    // the tile is taken whole when the length / causal limit passes it and,
    // with a mask, every mask value the wave holds is +0 (the masked
    // arithmetic would add zeros)
    bool full = cb + 31 <= lim_min;
    if constexpr (HAS_MASK) {
        uint32_t bits = 0;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int i = 0; i < 4; ++i) bits |= cur.mk[rb][i];
        full = full && __all(bits == 0u);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) vis_any[j] = true;
    if (!full) {
#pragma unroll
        for (int j = 0; j < 8; ++j) vis_any[j] = false;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int mb = j >> 2, i = j & 3;
                bool vis = cb + cell_of_slot(g, j) <= lim[rb];
                float x = s[rb][mb][i];
                if constexpr (HAS_MASK) {
                    const float mv = slope[rb] * f16_bits_to_float((uint16_t) (cur.mk[rb][j >> 1] >> (16 * (j & 1))));
                    vis = vis && (mv != -AL_INF);
                    x += mv;
                }
                s[rb][mb][i] = vis ? x : -AL_INF;
                vis_any[j] = vis_any[j] || vis;
            }
        }
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        float m = fmaxf(fmaxf(fmaxf(s[rb][0][0], s[rb][0][1]), fmaxf(s[rb][0][2], s[rb][0][3])),
                        fmaxf(fmaxf(s[rb][1][0], s[rb][1][1]), fmaxf(s[rb][1][2], s[rb][1][3])));
        mt[rb] = colmax4(m);
    }
    return full;
}

// Does any row's tile max exceed its reference max by more than kTau? (The
// online softmax keeps a lazily moved reference max: p = e^(s - m) stays
// below e^kTau, f16-representable, and O / l is the same for any reference.)
template <int RB>
__device__ __forceinline__ bool needs_rescale(const float (&mt)[RB], const float (&m_run)[RB]) {
    bool any = false;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) any = any || __any(mt[rb] > m_run[rb] + kTau);
    return any;
}

// Moves the reference max of the rows that outgrew it (cold path).
template <int RB>
__device__ __forceinline__ void rescale_rows(const float (&mt)[RB], floatx4 (&o)[RB][8], float (&m_run)[RB],
                                          float (&l_run)[RB]) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const bool grow = mt[rb] > m_run[rb] + kTau;
        const float mn = grow ? mt[rb] : m_run[rb];
        const float alpha = grow ? exp_fast(m_run[rb] - mn) : 1.0f;     // 0 when m was -inf
        l_run[rb] *= alpha;
#pragma unroll
        for (int d = 0; d < 8; ++d) o[rb][d] *= alpha;
        m_run[rb] = mn;
    }
}

// Second half of a tile: P = e^(S - m) (f16, in the P^T operand layout,
// built in place from the S^T layout), l += rowsum(P), O^T += V^T P^T.
template <int RB>
__device__ __forceinline__ void apply_tile(Tile<RB> & cur, const floatx4 (&s)[RB][2], const bool full,
                                           const bool (&vis_any)[8], const int g, floatx4 (&o)[RB][8],
                                           const float (&m_run)[RB], float (&l_run)[RB]) {
    half8 pf[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const float mu = (m_run[rb] == -AL_INF) ? 0.0f : m_run[rb];
        float ps = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float pr = exp_fast(s[rb][j >> 2][j & 3] - mu);
            ps += pr;
            pf[rb][j] = (_Float16) pr;
        }
        l_run[rb] += ps;
    }
    // cells masked for every row of the tile contribute exact zeros
    // (their memory may hold anything, e.g. unwritten cache cells)
    if (!full) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint64_t bal = __ballot(vis_any[j]);
            if (((bal >> (16 * g)) & 0xffffull) == 0) cur.v[j] = u32x4{0, 0, 0, 0};
        }
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

// One whole tile: scores, (rare) reference-max move, P and O update.
template <int RB, bool HAS_MASK>
__device__ __forceinline__ void process_tile(Tile<RB> & cur, const int cb, const FattnParams & p, const int g,
                                             const int (&lim)[RB], const int lim_min, const float (&slope)[RB],
                                             const half8 (&qf)[RB][4], floatx4 (&o)[RB][8], float (&m_run)[RB],
                                             float (&l_run)[RB]) {
    floatx4 s[RB][2];
    float mt[RB];
    bool vis_any[8];
    const bool full = score_tile<RB, HAS_MASK>(cur, cb, p, g, lim, lim_min, slope, qf, s, mt, vis_any);
    if (needs_rescale<RB>(mt, m_run)) rescale_rows<RB>(mt, o, m_run, l_run);
    apply_tile<RB>(cur, s, full, vis_any, g, o, m_run, l_run);
}

// ---------------------------------------------------------------------------
// LDS-DMA staging helpers
// ---------------------------------------------------------------------------

typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef short short4v __attribute__((ext_vector_type(4)));
typedef int int4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v lds_short4v;

// s_waitcnt immediates (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4,
// lgkmcnt 11:8; all-ones = no wait)
constexpr int vmcnt_imm(int v) { return (v & 15) | ((v >> 4) << 14) | (7 << 4) | (15 << 8); }

__device__ __forceinline__ floatx4 mfma_16x16x16(half4 a, half4 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// ds_read_b64_tr_b16: in each 16-lane group, lane s supplies 8 bytes (4 f16)
// that form elements 4(s%4)..4(s%4)+3 of row s/4 of a 4 x 16 matrix; lane i
// receives column i, i.e. element i%4 of the 8 bytes of lanes i/4, 4+i/4,
// 8+i/4 and 12+i/4.
__device__ __forceinline__ half4 lds_read_tr16(const char * p) {
    const short4v r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4v *) p);
    return __builtin_bit_cast(half4, r);
}

__device__ __forceinline__ void mem_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
}

// Raw buffer descriptor (the layout make_rsrc builds) for the inline DMA.
__device__ __forceinline__ int4v raw_desc(const void * base, uint32_t bytes) {
    const uint64_t a = (uint64_t) base;
    return int4v{(int) (uint32_t) a, (int) (uint32_t) (a >> 32), (int) bytes, 0x00020000};
}

// One LDS-DMA load: 16 bytes per lane from desc + voff into LDS at
// lds_base + 16 * lane. M0 carries the LDS address; nothing else in these
// kernels uses M0 (the compiler warns that a clobbered reserved register is
// not preserved, which is the intent here).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const int4v desc, uint32_t voff, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                 :
                 : "v"(voff), "s"(desc), "s"(lds_base)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ uint32_t lds_addr(const void * p) {
    return (uint32_t) (uintptr_t) (const __attribute__((address_space(3))) char *) p;
}

template <int K, int PER>
__device__ __forceinline__ void wait_vm_stages(int k) {
    if constexpr (K > 0) {
        if (k >= K) { __builtin_amdgcn_s_waitcnt(vmcnt_imm(K * PER)); return; }
        wait_vm_stages<K - 1, PER>(k);
    } else {
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    }
}

// Waits until at most k * PER memory operations are outstanding (0 <= k <=
// KMAX): the k stages issued after the data about to be read.
template <int KMAX, int PER>
__device__ __forceinline__ void wait_later(int k) {
    static_assert(KMAX >= 0 && KMAX * PER < 64, "vmcnt holds at most 63");
    mem_barrier();
    wait_vm_stages<KMAX, PER>(k);
    mem_barrier();
}

// Waits until at most `later` (<= NB - 2) stages of PER memory operations
// each are still outstanding (the stages issued after the one about to be
// read, in a ring of NB).
template <int NB, int PER>
__device__ __forceinline__ void wait_stage(int later) {
    wait_later<NB - 2, PER>(later);
}

}  // namespace fattn
