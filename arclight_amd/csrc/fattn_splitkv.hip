// Split-KV GQA flash attention for gfx950 (decode, speculative verify, and
// row-tiled prefill until the dedicated prefill kernel takes over).
//
// Semantics follow nnml_compute_forward_flash_attn_ext_f16
// (nnml/src/ops/arm/arm.cpp:2196-2433): per query row, softmax over the
// visible KV cells of scale * (f16(q) . k) [softcap] + slope * mask, times V,
// optional sinks, 1/S, stored at row (i3*T + i1)*Hq + i2 (arm.cpp:2431).
// Cells whose mask is -inf are skipped (arm.cpp:2327-2330). Accumulation is
// f32; q is rounded to f16 once (arm.cpp:2322), as the reference does.
//
// Work decomposition (one workgroup = 4 wavefronts):
//   blockIdx.x  split of the visible cell range (split-KV)
//   blockIdx.y  kv head + Hkv * row tile
//   blockIdx.z  stream (nnml dim 3)
// A row tile packs ROWS = 16*RB query rows of ONE kv-head group:
// row r -> token r / G, head kvh*G + r % G, so every K/V byte a wavefront
// loads serves all G heads of the group and all tokens of the tile.
// The 4 waves of a workgroup take interleaved 32-cell tiles of the split,
// merge their online-softmax states in LDS, and the last workgroup of a row
// tile to finish merges all splits (no second kernel launch).
//
// Per 32-cell tile a wavefront does, with no LDS:
//   S^T[32 cells x 16 rows]  = K[32 x 128] * Q^T    8 MFMA 16x16x32 per row block
//   O^T[128 dims x 16 rows] += V^T[128 x 32] * P^T  8 MFMA 16x16x32 per row block
// K goes from HBM straight into MFMA A-operand registers (16-byte loads).
// V is loaded as 8 cells x 8 dims per lane (each load instruction reads 4
// whole 256-byte rows) and transposed in registers: the A-operand row m of
// block mb' is dim 8m + mb', so no lane exchange is needed. The cell order
// of the k slots matches the MFMA output layout of S^T, so P^T is built from
// S^T in place. Each lane's O^T holds 32 consecutive dims of one query row.

#include "device_common.hpp"
#include "fattn_kernels.hpp"

namespace {

constexpr int kWaves = 4;
constexpr int kTile = 32;            // cells per wave iteration
constexpr int kRowStride = 132;      // floats per row of a merge record: O[128], m, l, pad

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

template <int RB>
__device__ __forceinline__ void load_tile(Tile<RB> & t, const FattnParams & p, const char * kbase,
                                          const char * vbase, const uint16_t * const * mrow,
                                          int cb, int g, int n) {
    const int last = p.n_kv - 1;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
        const int cell = min(cb + 16 * mb + n, last);
        const char * kp = kbase + (int64_t) cell * p.k_nb1;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            t.k[mb][kb] = *(const u32x4 *) (kp + (4 * kb + g) * 16);
        }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int cell = min(cb + cell_of_slot(g, j), last);
        t.v[j] = *(const u32x4 *) (vbase + (int64_t) cell * p.v_nb1 + n * 16);
    }
    if (p.mask) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                const int c0 = cb + cell_of_slot(g, 2 * jj);
                const uint32_t lo = (mrow[rb] && c0 < p.m_ne0) ? mrow[rb][c0] : 0xfc00u;          // -inf
                const uint32_t hi = (mrow[rb] && c0 + 1 < p.m_ne0) ? mrow[rb][c0 + 1] : 0xfc00u;
                t.mk[rb][jj] = lo | (hi << 16);
            }
        }
    }
}

// One merge record (m, l, O) per query row in LDS or global memory.
template <int RB>
__device__ __forceinline__ void store_state(float * rec, const floatx4 (&o)[RB][8], const float (&m)[RB],
                                            const float (&l)[RB], int g, int n) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        float * row = rec + (16 * rb + n) * kRowStride;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float4 lo = {o[rb][0][i], o[rb][1][i], o[rb][2][i], o[rb][3][i]};
            float4 hi = {o[rb][4][i], o[rb][5][i], o[rb][6][i], o[rb][7][i]};
            *(float4 *) (row + 32 * g + 8 * i) = lo;
            *(float4 *) (row + 32 * g + 8 * i + 4) = hi;
        }
        if (g == 0) {
            row[128] = m[rb];
            row[129] = l[rb];
        }
    }
}

template <int RB>
__device__ __forceinline__ void merge_state(const float * rec, floatx4 (&o)[RB][8], float (&m)[RB],
                                            float (&l)[RB], int g, int n) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const float * row = rec + (16 * rb + n) * kRowStride;
        const float mo = row[128];
        const float lo_ = row[129];
        const float mn = fmaxf(m[rb], mo);
        const float mu = (mn == -AL_INF) ? 0.0f : mn;
        const float wa = exp_fast(m[rb] - mu);
        const float wb = exp_fast(mo - mu);
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
        l[rb] = l[rb] * wa + lo_ * wb;
        m[rb] = mn;
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

// One 32-cell tile of one wavefront: S^T = K Q^T, scale/softcap/mask,
// online softmax update, O^T += V^T P^T.
template <int RB>
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
            if (p.mask) {
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

template <int RB, bool PREFETCH>
__global__ __launch_bounds__(256) void fattn_splitkv_kernel(const FattnParams p) {
    constexpr int ROWS = 16 * RB;
    __shared__ float lds[ROWS * kRowStride];
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
        slope[rb] = 1.0f;
        if (p.max_bias > 0.0f) {                                   // arm.cpp:2294
            const uint32_t h = (uint32_t) head[rb];
            slope[rb] = h < p.n_head_log2 ? powf(p.m0, (float) (h + 1))
                                          : powf(p.m1, (float) (2 * (h - p.n_head_log2) + 1));
        }
        mrow[rb] = nullptr;
        if (p.mask && rvalid[rb]) {
            mrow[rb] = (const uint16_t *) (p.mask + (int64_t) tok[rb] * p.m_nb1 +
                                           (int64_t) (head[rb] % p.m_ne2) * p.m_nb2 +
                                           (int64_t) (b % p.m_ne3) * p.m_nb3);
        }
    }

    // Q^T B-operand fragments: k slots of block kb, group g = dims 8*(4kb+g)..+8
    half8 qf[RB][4];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const float * qrow = (const float *) (p.q + (int64_t) b * p.q_nb3 + (int64_t) tok[rb] * p.q_nb1 +
                                              (int64_t) head[rb] * p.q_nb2);
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            if (rvalid[rb]) {
                const float4 a = *(const float4 *) (qrow + 8 * (4 * kb + g));
                const float4 c = *(const float4 *) (qrow + 8 * (4 * kb + g) + 4);
                qf[rb][kb] = to_half8(a, c);
            } else {
                qf[rb][kb] = half8{0, 0, 0, 0, 0, 0, 0, 0};
            }
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

    const char * kbase = p.k + (int64_t) (b / p.rk3) * p.k_nb3 + (int64_t) kvh * p.k_nb2;
    const char * vbase = p.v + (int64_t) (b / p.rv3) * p.v_nb3 + (int64_t) kvh * p.v_nb2;

    int cb = c_begin + wave * kTile;
    if constexpr (PREFETCH) {
        // the next tile's loads are in flight while this tile computes
        Tile<RB> cur;
        if (cb < c_end) load_tile<RB>(cur, p, kbase, vbase, mrow, cb, g, n);
        for (; cb < c_end; cb += kWaves * kTile) {
            Tile<RB> nxt;
            const int cn = cb + kWaves * kTile;
            if (cn < c_end) load_tile<RB>(nxt, p, kbase, vbase, mrow, cn, g, n);
            process_tile<RB>(cur, cb, p, g, hi, rvalid, tok, slope, qf, o, m_run, l_run);
            cur = nxt;
        }
    } else {
        for (; cb < c_end; cb += kWaves * kTile) {
            Tile<RB> cur;
            load_tile<RB>(cur, p, kbase, vbase, mrow, cb, g, n);
            process_tile<RB>(cur, cb, p, g, hi, rvalid, tok, slope, qf, o, m_run, l_run);
        }
    }

#pragma unroll
    for (int rb = 0; rb < RB; ++rb) l_run[rb] = colsum4(l_run[rb]);

    // merge the 4 waves through one LDS record: 3 -> 2 -> 1 -> 0
#pragma unroll
    for (int w = kWaves - 1; w > 0; --w) {
        if (wave == w) store_state<RB>(lds, o, m_run, l_run, g, n);
        __syncthreads();
        if (wave == w - 1) merge_state<RB>(lds, o, m_run, l_run, g, n);
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
                    float4 lo = {o[rb][0][i], o[rb][1][i], o[rb][2][i], o[rb][3][i]};
                    float4 hi4 = {o[rb][4][i], o[rb][5][i], o[rb][6][i], o[rb][7][i]};
                    *(float4 *) (out + 32 * g + 8 * i) = finalize4(lo, m_run[rb], l_run[rb], p.sinks, head[rb]);
                    *(float4 *) (out + 32 * g + 8 * i + 4) = finalize4(hi4, m_run[rb], l_run[rb], p.sinks, head[rb]);
                }
            }
        }
        return;
    }

    // split-KV: publish this split, the last workgroup of the row tile merges
    const int64_t tile_id = ((int64_t) b * p.Hkv + kvh) * p.n_row_tiles + rt;
    float * part = p.part + tile_id * (int64_t) p.n_split * ROWS * kRowStride;
    if (wave == 0) store_state<RB>(part + (int64_t) split * ROWS * kRowStride, o, m_run, l_run, g, n);
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned prev = atomicAdd(p.counters + tile_id, 1u);
        s_last = (prev == (unsigned) (p.n_split - 1));
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();

    for (int idx = threadIdx.x; idx < rows_here * 32; idx += 256) {
        const int r = idx >> 5;
        const int d4 = idx & 31;
        float M = -AL_INF;
        for (int sp = 0; sp < p.n_split; ++sp) M = fmaxf(M, part[((int64_t) sp * ROWS + r) * kRowStride + 128]);
        const float Mu = (M == -AL_INF) ? 0.0f : M;
        float L = 0.0f;
        float4 acc = {0, 0, 0, 0};
        for (int sp = 0; sp < p.n_split; ++sp) {
            const float * row = part + ((int64_t) sp * ROWS + r) * kRowStride;
            const float w = exp_fast(row[128] - Mu);
            const float4 ov = *(const float4 *) (row + 4 * d4);
            L += w * row[129];
            acc.x += w * ov.x; acc.y += w * ov.y; acc.z += w * ov.z; acc.w += w * ov.w;
        }
        const int rr = row0 + r;
        const int t = rr / p.G;
        const int h = kvh * p.G + rr % p.G;
        float * out = (float *) (p.dst + ((int64_t) (b * p.T + t) * p.Hq + h) * p.dst_nb1);
        *(float4 *) (out + 4 * d4) = finalize4(acc, M, L, p.sinks, h);
    }
    if (threadIdx.x == 0) p.counters[tile_id] = 0u;   // ready for the next call in stream order
}

}  // namespace

int fattn_splitkv_rows_per_tile(int R) {
    return R <= 16 ? 16 : (R <= 32 ? 32 : 64);
}

hipError_t fattn_splitkv_launch(const FattnParams & p, int rows_per_tile, hipStream_t stream) {
    const dim3 grid((unsigned) p.n_split, (unsigned) (p.Hkv * p.n_row_tiles), (unsigned) p.B);
    const dim3 block(256);
    switch (rows_per_tile) {
        case 16: hipLaunchKernelGGL((fattn_splitkv_kernel<1, true>), grid, block, 0, stream, p); break;
        case 32: hipLaunchKernelGGL((fattn_splitkv_kernel<2, true>), grid, block, 0, stream, p); break;
        case 64: hipLaunchKernelGGL((fattn_splitkv_kernel<4, false>), grid, block, 0, stream, p); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}
