// Prefill (and long speculative-verify) attention for gfx950: many query rows
// per kv head, causal / length masking given implicitly (kv_len,
// causal_pos0). Semantics as nnml_compute_forward_flash_attn_ext_f16
// (nnml/src/ops/arm/arm.cpp:2196-2433), numerics as fattn_splitkv.hip.
//
// One workgroup = one row tile of 64 query rows of one kv-head group
// (row r -> token r / G, head kvh*G + r % G) and 8 wavefronts, two per SIMD.
// Wave w holds row half w & 1 (32 rows: 2 MFMA row blocks, so each K/V
// operand read from LDS feeds 2 MFMAs) and cell split w >> 1 (every 4th
// 32-cell tile of the visible range). The two waves of a split share its
// LDS stages, one loading K and the other V, and every wave passes two
// workgroup barriers per tile (tile landed; tile read). The 4 splits'
// online-softmax states merge through LDS at the end. A 512-token chunk of
// Qwen3-4B gives 32 row tiles x 8 kv heads = 256 workgroups.
//
// K/V tiles travel HBM/L2 -> LDS by LDS-DMA buffer loads, two 16 KiB stages
// per split in flight without costing registers:
//   - K as MFMA A operands: block (mb, kb) holds, at lane l's 16-byte slot,
//     cell 16 mb + l % 16, dims 32 kb + 8 (l / 16) .. + 7, so ds_read_b128
//     at lane*16 yields the operand;
//   - V cell-major (256 bytes per cell) with the 16-byte granule j of cell c
//     at slot j ^ (c & 15), read transposed by ds_read_b64_tr_b16 into V^T
//     A operands whose k slots follow the S^T output layout (cells 4g + i
//     and 16 + 4g + i of lane group g), so P^T is S^T in place.
// The DMA is inline assembly the compiler does not count; each wave waits
// for its own loads (s_waitcnt vmcnt), the barrier for its partner's.
//
// Softmax per tile: the running max is kept on the raw scores (scale > 0
// keeps their order), p = exp2(s * c - m * c) with c = scale * log2(e) is
// one FMA and one v_exp_f32 per score, P is packed to f16 two at a time,
// and the row sums l come from an extra MFMA against an all-ones operand
// (f32 accumulation of the same f16 P that weights V). The reference max
// moves lazily (only when a tile exceeds it by more than kTau in natural
// units), so O is rarely rescaled.
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
constexpr float kLog2e = 1.44269504088896341f;

struct PTile {
    u32x4 k[2][4];                           // [mb][kb] K A-operand chunks
    half8 vt[8];                             // V^T A operands, dim block d: rows 16d..16d+15
};

// P = exp2(s c - m c) in f16, then O^T += V^T P^T and l += 1 P^T.
__device__ __forceinline__ void accumulate_tile(PTile & t, const floatx4 (&s)[kPRB][2], const bool full,
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
    __shared__ __attribute__((aligned(1024))) char lds[kCS][2][kStage];

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
    int hi = p.kv_hi;
    if (p.causal_pos0 >= 0) hi = (int) min((int64_t) hi, p.causal_pos0 + t_last + 1);

    const char * kbase = p.k + (int64_t) (b / p.rk3) * p.k_nb3 + (int64_t) kvh * p.k_nb2;
    const char * vbase = p.v + (int64_t) (b / p.rv3) * p.v_nb3 + (int64_t) kvh * p.v_nb2;
    const uint32_t k_nb1 = (uint32_t) p.k_nb1, v_nb1 = (uint32_t) p.v_nb1;
    const int4v kd = raw_desc(kbase, (uint32_t) (p.n_kv - 1) * k_nb1 + 256);
    const int4v vd = raw_desc(vbase, (uint32_t) (p.n_kv - 1) * v_nb1 + 256);

    // this split's tiles: cells cb0 + it * 128; every wave runs the loop
    // ntiles_max times (the workgroup barriers must match), doing work only
    // while it < ntiles
    constexpr int kStride = kCS * 32;
    const int cb0 = cs * 32;
    const int ntiles = cb0 < hi ? (hi - cb0 + kStride - 1) / kStride : 0;
    const int ntiles_max = hi > 0 ? (hi + kStride - 1) / kStride : 0;

    // DMA of a tile: the row-half-0 wave of the split loads the 8 K blocks
    // (block (mb, kb) lane (g, n): cell 16 mb + n, granule 4 kb + g), the
    // row-half-1 wave the 8 V blocks (block i lane (g, n): cell c = 4i + g,
    // granule n ^ (c & 15) into slot n)
    const uint32_t ring = lds_addr(&lds[cs][0][0]);
    const uint32_t ksrc = (uint32_t) n * k_nb1 + (uint32_t) (g * 16);
    auto issue = [&](const int it, const int u) {
        const uint32_t cb = (uint32_t) (cb0 + it * kStride);
        const uint32_t base = ring + (uint32_t) (u * kStage);
        if (rh == 0) {
            const uint32_t kofs = cb * k_nb1 + ksrc;
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int kb = 0; kb < 4; ++kb)
                    dma16(kd, kofs + (uint32_t) (16 * mb) * k_nb1 + (uint32_t) (64 * kb), base + (uint32_t) ((mb * 4 + kb) * 1024));
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int c = 4 * i + g;
                dma16(vd, (cb + (uint32_t) c) * v_nb1 + (uint32_t) (((n ^ c) & 15) * 16), base + (uint32_t) (kKBytes + i * 1024));
            }
        }
    };

    // query rows held by this lane (column n of its two row blocks) and their
    // Q^T B-operand fragments (k slots of block kb, group g = dims 32kb + 8g..+8)
    int tok[kPRB];
    int head[kPRB];
    bool rvalid[kPRB];
    float4 qa[kPRB][4], qb[kPRB][4];
#pragma unroll
    for (int rb = 0; rb < kPRB; ++rb) {
        const int rr = 32 * rh + 16 * rb + n;
        rvalid[rb] = rr < rows_here;
        tok[rb] = rvalid[rb] ? (row0 + rr) / p.G : 0;
        head[rb] = kvh * p.G + (rvalid[rb] ? (row0 + rr) % p.G : 0);
        const float * qrow = (const float *) (p.q + (int64_t) b * p.q_nb3 + (int64_t) tok[rb] * p.q_nb1 +
                                              (int64_t) head[rb] * p.q_nb2);
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            qa[rb][kb] = *(const float4 *) (qrow + 8 * (4 * kb + g));
            qb[rb][kb] = *(const float4 *) (qrow + 8 * (4 * kb + g) + 4);
        }
    }
    // the first two tiles fly together with q (converting q waits for all of it)
    mem_barrier();
    if (ntiles > 0) issue(0, 0);
    if (ntiles > 1) issue(1, 1);
    half8 qf[kPRB][4];
#pragma unroll
    for (int rb = 0; rb < kPRB; ++rb)
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) qf[rb][kb] = rvalid[rb] ? to_half8(qa[rb][kb], qb[rb][kb]) : half8{0, 0, 0, 0, 0, 0, 0, 0};

    int lim[kPRB];
#pragma unroll
    for (int rb = 0; rb < kPRB; ++rb) lim[rb] = row_limit(p, hi, rvalid[rb], tok[rb]);
    const int lim_min = row_limit(p, hi, true, (row0 + min(32 * rh, rows_here - 1)) / p.G);   // this wave's first token

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

    // LDS read offsets of this lane: K at lane*16 of each block; V^T source
    // cells 4g + (n >> 2) (k slots 0..3) and 16 + 4g + (n >> 2) (4..7),
    // dims 16d + 4(n & 3) .. + 3 (granule 2d + ((n & 3) >> 1), half n & 1)
    const int vc0 = 4 * g + (n >> 2);
    const int vc1 = 16 + vc0;
    const int vr0 = kKBytes + vc0 * 256 + (n & 1) * 8;
    const int vr1 = kKBytes + vc1 * 256 + (n & 1) * 8;
    const int vq = (n & 3) >> 1;

    // Tile state shared by the fast loop and the rescale path below.
    PTile t;
    floatx4 s[kPRB][2];
    float mt[kPRB];
    bool full = true;
    bool vis_any[8];

    // The fast loop never scales O: a tile whose max would move the
    // reference (the first tile always does) leaves it, and the scaling
    // happens outside, so the accumulators stay in MFMA registers across
    // iterations instead of being copied for a rarely taken branch. Each
    // tile costs every wave exactly two workgroup barriers, on either path.
    int it = 0;
    while (it < ntiles_max) {
        for (; it < ntiles_max; ++it) {
            const bool active = it < ntiles;
            const int u = it & 1;
            // this wave's 8 loads of the tile are done once at most the next
            // tile's 8 are outstanding; the barrier makes the partner's visible
            if (active) wait_stage<3, 8>(min(1, ntiles - 1 - it));
            __syncthreads();
            if (active) {
                const char * st = &lds[cs][u][0];
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                    for (int kb = 0; kb < 4; ++kb) t.k[mb][kb] = *(const u32x4 *) (st + (mb * 4 + kb) * 1024 + lane * 16);
#pragma unroll
                for (int d = 0; d < 8; ++d) {
                    const half4 a = lds_read_tr16(st + vr0 + (((2 * d + vq) ^ (vc0 & 15)) << 4));
                    const half4 c = lds_read_tr16(st + vr1 + (((2 * d + vq) ^ (vc1 & 15)) << 4));
                    t.vt[d] = half8{a[0], a[1], a[2], a[3], c[0], c[1], c[2], c[3]};
                }
                mem_barrier();
                __builtin_amdgcn_s_waitcnt(0xC00F | (7 << 4));             // lgkmcnt(0)
                mem_barrier();
            }
            // both waves of the split have read the stage: refill it
            __syncthreads();
            if (!active) continue;
            if (it + 2 < ntiles) issue(it + 2, u);
            const int cb = cb0 + it * kStride;

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
            bool grow_any = false;
#pragma unroll
            for (int rb = 0; rb < kPRB; ++rb) {
                const float a = fmaxf(fmaxf(s[rb][0][0], s[rb][0][1]), s[rb][0][2]);
                const float c = fmaxf(fmaxf(s[rb][0][3], s[rb][1][0]), s[rb][1][1]);
                const float e = fmaxf(fmaxf(s[rb][1][2], s[rb][1][3]), fmaxf(a, c));
                mt[rb] = colmax4(e);
                grow_any = grow_any || (mt[rb] > m_run[rb] + tau);
            }
            if (__any(grow_any)) break;
            accumulate_tile(t, s, full, vis_any, m_run, cexp, ones, g, o, lacc);
        }
        if (it >= ntiles_max) break;
        // tile `it` moves the reference max of some rows: scale, then finish it
#pragma unroll
        for (int rb = 0; rb < kPRB; ++rb) {
            const bool grow = mt[rb] > m_run[rb] + tau;
            const float mn = grow ? mt[rb] : m_run[rb];
            const float alpha = grow ? __builtin_amdgcn_exp2f((m_run[rb] - mn) * cexp) : 1.0f;   // 0 from -inf
            lacc[rb] *= alpha;
#pragma unroll
            for (int d = 0; d < 8; ++d) o[rb][d] *= alpha;
            m_run[rb] = mn;
        }
        accumulate_tile(t, s, full, vis_any, m_run, cexp, ones, g, o, lacc);
        ++it;
    }

    // natural-unit max and the row sums (every element of lacc holds l)
    float m_nat[kPRB], l_run[kPRB];
#pragma unroll
    for (int rb = 0; rb < kPRB; ++rb) {
        m_nat[rb] = m_run[rb] == -AL_INF ? -AL_INF : m_run[rb] * (cexp / kLog2e);
        l_run[rb] = lacc[rb][0];
    }

    // merge the kCS splits of each row half through LDS records
    // [rh][slot][32 rows][132] in two rounds (the stages are free now)
    float * recs = (float *) &lds[0][0][0];
#pragma unroll
    for (int span = kCS / 2; span >= 1; span /= 2) {
        __syncthreads();
        if (cs >= span && cs < 2 * span) {
            float * rec = recs + (rh * (kCS / 2) + (cs - span)) * (32 * kRowStride);
#pragma unroll
            for (int rb = 0; rb < kPRB; ++rb) {
                float * row = rec + (16 * rb + n) * kRowStride;
#pragma unroll
                for (int d = 0; d < 8; ++d) *(float4 *) (row + 16 * d + 4 * g) = float4{o[rb][d][0], o[rb][d][1], o[rb][d][2], o[rb][d][3]};
                if (g == 0) *(float2 *) (row + 128) = float2{m_nat[rb], l_run[rb]};
            }
        }
        __syncthreads();
        if (cs < span) {
            const float * rec = recs + (rh * (kCS / 2) + cs) * (32 * kRowStride);
#pragma unroll
            for (int rb = 0; rb < kPRB; ++rb) {
                const float * row = rec + (16 * rb + n) * kRowStride;
                const float2 ml = *(const float2 *) (row + 128);
                const float mn = fmaxf(m_nat[rb], ml.x);
                const float mu = (mn == -AL_INF) ? 0.0f : mn;
                const float wa = exp_fast(m_nat[rb] - mu);
                const float wb = exp_fast(ml.x - mu);
#pragma unroll
                for (int d = 0; d < 8; ++d) {
                    const float4 x = *(const float4 *) (row + 16 * d + 4 * g);
                    o[rb][d][0] = o[rb][d][0] * wa + x.x * wb;
                    o[rb][d][1] = o[rb][d][1] * wa + x.y * wb;
                    o[rb][d][2] = o[rb][d][2] * wa + x.z * wb;
                    o[rb][d][3] = o[rb][d][3] * wa + x.w * wb;
                }
                l_run[rb] = l_run[rb] * wa + ml.y * wb;
                m_nat[rb] = mn;
            }
        }
    }
    if (cs != 0) return;
#pragma unroll
    for (int rb = 0; rb < kPRB; ++rb) {
        if (!rvalid[rb]) continue;
        float * out = (float *) (p.dst + ((int64_t) (b * p.T + tok[rb]) * p.Hq + head[rb]) * p.dst_nb1);
#pragma unroll
        for (int d = 0; d < 8; ++d)
            *(float4 *) (out + 16 * d + 4 * g) =
                finalize4(float4{o[rb][d][0], o[rb][d][1], o[rb][d][2], o[rb][d][3]}, m_nat[rb], l_run[rb], p.sinks, head[rb]);
    }
}

}  // namespace

size_t fattn_prefill_lds_bytes() { return sizeof(char) * kCS * 2 * kStage; }

hipError_t fattn_prefill_launch(const FattnParams & p, hipStream_t stream) {
    const dim3 grid((unsigned) ((int64_t) p.Hkv * p.n_row_tiles * p.B));
    if (p.softcap != 0.0f) hipLaunchKernelGGL(fattn_prefill_kernel<true>, grid, dim3(kPW * 64), 0, stream, p);
    else                   hipLaunchKernelGGL(fattn_prefill_kernel<false>, grid, dim3(kPW * 64), 0, stream, p);
    return hipGetLastError();
}
