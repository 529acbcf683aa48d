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
// Work decomposition (one workgroup = W wavefronts; a 1-D grid over
// kv head (fastest), split of the visible cell range, row tile, stream).
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

#include "fattn_tile.hpp"

namespace {

using namespace fattn;

template <int RB, int W, bool PREFETCH, bool HAS_MASK>
__global__ __launch_bounds__(W * 64) void fattn_splitkv_kernel(const FattnParams p) {
    constexpr int ROWS = 16 * RB;
    // LDS records of the wave merge: a tree when W/2 records fit in 40 KiB,
    // else one record that wave 0 merges the others through in turn
    constexpr int NSLOT = ((W / 2) * ROWS * kRowStride * 4 <= 40960) ? W / 2 : 1;
    __shared__ float lds[NSLOT * ROWS * kRowStride];
    __shared__ int s_last;
    prefetch_params(p);

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int g = lane >> 4;
    const int n = lane & 15;
    // 1-D grid, kv head fastest: consecutive workgroups go to different XCDs,
    // so with Hkv = 8 every workgroup of one head shares one XCD's L2. With a
    // causal mask, row tiles are dispatched longest first.
    int id = blockIdx.x;
    const int kvh = id % p.Hkv;
    id /= p.Hkv;
    const int split = id % p.n_split;
    id /= p.n_split;
    const int rt = p.causal_pos0 >= 0 ? p.n_row_tiles - 1 - id % p.n_row_tiles : id % p.n_row_tiles;
    const int b = id / p.n_row_tiles;
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

    int lim[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) lim[rb] = row_limit(p, hi, rvalid[rb], tok[rb]);
    const int lim_min = row_limit(p, hi, true, row0 / p.G);          // the tile's first token

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
            process_tile<RB, HAS_MASK>(ta, c0, p, g, lim, lim_min, slope, qf, o, m_run, l_run);
            load_tile<RB, HAS_MASK>(ta, p, kr, vr, mrow, min(c0 + 2 * kStride, c_last), g, n);
            if (it + 1 < ntiles) process_tile<RB, HAS_MASK>(tb, c0 + kStride, p, g, lim, lim_min, slope, qf, o, m_run, l_run);
        }
    } else {
        for (int it = 0; it < ntiles; ++it) {
            if (it > 0) load_tile<RB, HAS_MASK>(ta, p, kr, vr, mrow, cb + it * kStride, g, n);
            process_tile<RB, HAS_MASK>(ta, cb + it * kStride, p, g, lim, lim_min, slope, qf, o, m_run, l_run);
        }
    }

#pragma unroll
    for (int rb = 0; rb < RB; ++rb) l_run[rb] = colsum4(l_run[rb]);

    // merge the W waves
    if constexpr (NSLOT >= W / 2) {
#pragma unroll
        for (int span = W / 2; span >= 1; span /= 2) {
            if (wave >= span && wave < 2 * span) store_state<RB>(lds + (wave - span) * ROWS * kRowStride, o, m_run, l_run, g, n);
            __syncthreads();
            if (wave < span) merge_state<RB>(lds + wave * ROWS * kRowStride, o, m_run, l_run, g, n);
            __syncthreads();
        }
    } else {
        for (int w = W - 1; w > 0; --w) {
            if (wave == w) store_state<RB>(lds, o, m_run, l_run, g, n);
            __syncthreads();
            if (wave == 0) merge_state<RB>(lds, o, m_run, l_run, g, n);
            __syncthreads();
        }
    }

    if (p.n_split == 1) {
        if (wave == 0) {
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                if (!rvalid[rb]) continue;
                float * out = (float *) (p.dst + ((int64_t) (b * p.T + tok[rb]) * p.Hq + head[rb]) * p.dst_nb1);
                const RowScale rs = row_scale(m_run[rb], l_run[rb], p.sinks, head[rb]);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float4 lo = {o[rb][0][i], o[rb][1][i], o[rb][2][i], o[rb][3][i]};
                    const float4 hi4 = {o[rb][4][i], o[rb][5][i], o[rb][6][i], o[rb][7][i]};
                    *(float4 *) (out + 32 * g + 8 * i) = apply_scale(lo, rs);
                    *(float4 *) (out + 32 * g + 8 * i + 4) = apply_scale(hi4, rs);
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
    return rows_per_tile == 16 ? 8 : 4;
}

hipError_t fattn_splitkv_launch(const FattnParams & p, int rows_per_tile, hipStream_t stream) {
    const dim3 grid((unsigned) ((int64_t) p.n_split * p.Hkv * p.n_row_tiles * p.B));
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
            if (m) hipLaunchKernelGGL((fattn_splitkv_kernel<4, 4, false, true>), grid, dim3(256), 0, stream, p);
            else   hipLaunchKernelGGL((fattn_splitkv_kernel<4, 4, false, false>), grid, dim3(256), 0, stream, p);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}
