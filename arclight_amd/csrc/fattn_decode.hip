// Decode (and short speculative-verify) attention for gfx950: up to 32 query
// rows per kv head, K/V streamed through LDS a whole cell range at a time.
// Semantics as nnml_compute_forward_flash_attn_ext_f16
// (nnml/src/ops/arm/arm.cpp:2196-2433), numerics as fattn_splitkv.hip.
//
// Work decomposition. A workgroup owns one kv head of one cell range (a
// split) of one stream and keeps up to 16 query rows of the head's group
// (row r -> token r / G, head kvh*G + r % G), or up to 32 as two MFMA row
// blocks sharing every K/V operand read (speculative verify). Its WS wavefronts take the
// range's 16-cell stages in turn (wave ws: stages ws, ws + WS, ...), each
// with a private ring of NB LDS stage buffers, so the waves never wait for
// each other until the end. The grid (split, kv head, stream) runs split
// fastest.
//
// Memory path. A stage is the head's 16 K rows and 16 V rows (4 KiB each),
// moved by LDS-DMA buffer loads of 1 KiB per instruction (4 cells x 256 B),
// 8 per stage, so a wave has NB - 1 stages (up to 24 KiB) in flight while it
// computes one. Inside a 256-byte row the 16-byte granules are XOR-swizzled
// by the cell index (granule j of cell c sits at slot j ^ c), which makes
// both operand reads below free of LDS bank conflicts. The DMA is issued by
// inline assembly, so the compiler neither counts it nor makes LDS reads of
// the current stage wait for the stages still in flight; each wave waits
// for its own stage (s_waitcnt vmcnt).
//
// Per wave and stage:
//   S^T[16 cells x 16 rows]  = K Q^T      4 MFMA 16x16x32 (K rows read as
//                                         A operands, one granule per lane)
//   O^T[128 dims x 16 rows] += V^T P^T    8 MFMA 16x16x16 (V^T operands read
//                                         by ds_read_b64_tr_b16, which
//                                         transposes 4 cells x 16 dims per
//                                         16-lane group on the way out)
// P^T comes from S^T in place: both keep cell 4g+i, row n in lane 16g+n.
// O^T lane 16g+n holds dims 16mb + 4g + i of row n (mb = 0..7).
//
// Lengths. kv_len and causal_pos0 come with the launch, or (p.dyn, for a
// graph captured once and replayed every decode step) from device memory
// when the kernel runs, bounded by the launch's kv_len; splits whose stages
// lie past the run-time length publish empty records.
//
// Merge. The WS waves merge their online-softmax states through LDS. With
// one split the workgroup then writes dst; otherwise it publishes its
// record with device-coherent stores and then its split flag, and
// min(splits, rows / merge_rows) of the (stream, kv head)'s workgroups wait
// for every flag and merge the at most 32 splits of their share of the rows
// (all loads in flight, fixed order, so results are bit-reproducible) into
// dst.

#include "fattn_tile.hpp"

namespace {

using namespace fattn;

constexpr int kSC = 16;                                   // cells per stage

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
// The largest x of each aligned group of 32 lanes, in all of them: DPP
// within rows of 16 lanes (lane ^ 1, ^ 2, then the mirrors within 8 and
// 16), then the group's two rows through a permlane swap.
__device__ __forceinline__ float max32(float x) {
    x = fmaxf(x, dpp_f<0xB1>(x));
    x = fmaxf(x, dpp_f<0x4E>(x));
    x = fmaxf(x, dpp_f<0x141>(x));
    x = fmaxf(x, dpp_f<0x140>(x));
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, x), __builtin_bit_cast(int, x), false, false);
    return fmaxf(__builtin_bit_cast(float, (int) r[0]), __builtin_bit_cast(float, (int) r[1]));
}
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// FM < 0: the query rows come ready in p.q; FM >= 0: the attention inputs
// folded in (DecodeInputs), FM the rotation mode. MASK: 0 no mask tensor, 1
// its rows loaded with every stage, 2 the mask values of all of a wave's
// stages preloaded into LDS before its first stage (p.mask_pre). OP: the
// waves' states merged and the split's record stored in one pass by all
// threads (always with four or more waves; with two, p.one_pass).
template <int WS, int NB, int MASK, int RB, int FM, bool OP>
__global__ __launch_bounds__(WS * 64) void fattn_decode_kernel(const FattnParams p, const DecodeInputs in) {
    constexpr bool FUSED = FM >= 0;
    constexpr bool HAS_MASK = MASK != 0;
    static_assert(WS == 2 || WS == 4 || WS == 8, "the wave merge is a binary tree");
    static_assert(RB == 1 || RB == 2, "16 or 32 rows");
    constexpr int PER = 8 + (MASK == 1 ? 1 : 0);          // DMA loads per stage
    constexpr int STAGE = 8192 + (MASK == 1 ? 1024 : 0);  // K rows, V rows, mask rows
    constexpr int REC = 16 * RB * kRowStride;             // floats of one state record (16 RB rows)
    static_assert(WS * NB * STAGE >= (WS / 2 > 0 ? WS / 2 : 1) * REC * 4, "LDS merge records must fit the rings");
    __shared__ __attribute__((aligned(1024))) char lds[WS][NB][STAGE];
    __shared__ __attribute__((aligned(1024))) char qlds[16 * RB * 512];  // the query rows, f32
    __shared__ __attribute__((aligned(1024))) char mpre[MASK == 2 ? kDecodeMaskPreBytes : 16];
    // fused inputs: 1 KiB slots of q_w, k_w and the new token's k and v rows
    // for this kv head (512 bytes each), then the new K (normed, rotated) and
    // V rows as f16 (256 bytes each) and the rotation pairs' (cos, sin)
    constexpr int kPieces = 4;
    __shared__ __attribute__((aligned(1024))) char fin[FUSED ? kPieces * 1024 + 1024 : 16];
    char * const kv16 = fin + kPieces * 1024;
    float2 * const rot_tab = (float2 *) (fin + kPieces * 1024 + 512);
    prefetch_params(p);

    const int lane = threadIdx.x & 63;
    const int ws = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4;
    const int n = lane & 15;

    // grid (split, kv head, stream): no integer division on the way to the
    // first loads
    const int split = blockIdx.x;
    const int kvh = blockIdx.y;
    const int b = blockIdx.z;
    const int unit = b * p.Hkv + kvh;
    const int rows_here = min(16 * RB, p.R);
    const int t_last = div_g(rows_here - 1, p.G, p.g_magic);

    // Lengths: fixed at launch, or (p.dyn: a graph replayed per decode step)
    // read when the kernel runs, within the launch's kv_len. The first
    // stages are issued against the launch's bound while the run-time
    // length is on its way (scalar loads): a stage past the run-time length
    // is then loaded and not used, and the buffer ranges keep every load
    // inside the cache.
    auto limit = [&](const int h, const int64_t c0) { return c0 >= 0 ? (int) min((int64_t) h, c0 + t_last + 1) : h; };
    // Stages of this wave: cells wbase + wstride j .. + 15 below the range's
    // end. With interleave the workgroup takes global 16-cell stages split,
    // split + n_split, ... of [0, hi) and wave ws every WS-th of them, so all
    // splits of a head sweep the cache together (measured faster than
    // contiguous ranges, and than blocks of WS adjacent stages, one per
    // wave); else the workgroup's contiguous range [c_begin, c_begin +
    // cells_per_split), wave ws taking its stages ws, ws + WS, ...
    const int c_begin = p.interleave ? 0 : split * p.cells_per_split;
    const int wbase = p.interleave ? kSC * (split + p.n_split * ws) : c_begin + kSC * ws;
    const int wstride = p.interleave ? kSC * WS * p.n_split : kSC * WS;
    auto range_end = [&](const int h) { return p.interleave ? h : min(c_begin + p.cells_per_split, h); };
    auto wave_stages = [&](const int h) {
        const int c_e = range_end(h);
        return c_e > wbase ? (c_e - wbase + wstride - 1) / wstride : 0;
    };
    const int ns_bound = wave_stages(p.dyn ? p.kv_hi : limit(p.kv_hi, p.causal_pos0));  // at the launch's bound
    const int n_pre = min(NB - 1, ns_bound);                          // issued ahead

    // K/V rows of this stream and head (loads past the end read 0)
    const uint32_t k_nb1 = (uint32_t) p.k_nb1, v_nb1 = (uint32_t) p.v_nb1;
    const int bk = p.rk3 == 1 ? b : b / p.rk3, bv = p.rv3 == 1 ? b : b / p.rv3;
    const char * kbase = p.k + (int64_t) bk * p.k_nb3 + (int64_t) kvh * p.k_nb2;
    const char * vbase = p.v + (int64_t) bv * p.v_nb3 + (int64_t) kvh * p.v_nb2;
    const int4v kd = raw_desc(kbase, (uint32_t) (p.n_kv - 1) * k_nb1 + 256);
    const int4v vd = raw_desc(vbase, (uint32_t) (p.n_kv - 1) * v_nb1 + 256);

    // DMA block i (0..3 K, 4..7 V) of a stage: LDS granule 64(i & 3) + lane
    // is cell 4(i & 3) + lane / 16, slot lane % 16, holding the global
    // granule slot ^ cell.
    const int dcell = lane >> 4;                           // + 4 (i & 3)
    const uint32_t dk = (uint32_t) dcell * k_nb1, dv = (uint32_t) dcell * v_nb1;
    uint32_t dj[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) dj[i] = (uint32_t) (((lane & 15) ^ (4 * i + dcell)) * 16);
    const uint32_t ring = lds_addr(&lds[ws][0][0]);

    // this lane's query rows: column n of each row block (row 16 rb + n)
    bool rvalid[RB];
    int tok[RB], head[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int r = 16 * rb + n;
        rvalid[rb] = r < rows_here;
        const int t = div_g(rvalid[rb] ? r : 0, p.G, p.g_magic);
        tok[rb] = t;
        head[rb] = kvh * p.G + (rvalid[rb] ? r - t * p.G : 0);
    }

    // Mask rows (f16, cells along a row) also travel by DMA, from a buffer
    // over the stream's mask slice; cells past a row read whatever follows,
    // and are past the length limit anyway. MASK 1: one 1 KiB block per
    // stage, lane l loading cells 8(l & 1)..+7 of row l >> 1 to LDS bytes 16
    // l (with one row block, lanes 32..63 repeat lanes 0..31). MASK 2: see
    // the preload below.
    int4v md = {0, 0, 0, 0};
    uint32_t msrc = 0;
    if constexpr (HAS_MASK) md = raw_desc(p.mask + (int64_t) (b % p.m_ne3) * p.m_nb3, p.m_slice_bytes);
    if constexpr (MASK == 1) {
        const int mrow = (lane >> 1) & (16 * RB - 1);
        const int mr = mrow < rows_here ? mrow : 0;
        const int mt_ = div_g(mr, p.G, p.g_magic);
        const int mh = kvh * p.G + mr - mt_ * p.G;
        msrc = (uint32_t) ((int64_t) mt_ * p.m_nb1 + (int64_t) (mh % p.m_ne2) * p.m_nb2) + (uint32_t) ((lane & 1) * 16);
    }

    // This wave's j-th stage (cells wbase + wstride j ..) into ring slot u.
    auto issue = [&](const int j, const int u) {
        const uint32_t cs = (uint32_t) (wbase + wstride * j);
        const uint32_t kofs = cs * k_nb1 + dk, vofs = cs * v_nb1 + dv;
        const uint32_t base = ring + (uint32_t) (u * STAGE);
        // the stage's V rows, then its K rows (grouped by tensor: 0.3-0.4 µs
        // per launch faster at 32K than K and V alternating, measured)
#pragma unroll
        for (int i = 0; i < 4; ++i) dma16(vd, vofs + (uint32_t) (4 * i) * v_nb1 + dj[i], base + (uint32_t) (4096 + i * 1024));
#pragma unroll
        for (int i = 0; i < 4; ++i) dma16(kd, kofs + (uint32_t) (4 * i) * k_nb1 + dj[i], base + (uint32_t) (i * 1024));
        if constexpr (MASK == 1) dma16(md, msrc + cs * 2, base + 8192u);
    };

    // The query rows travel by LDS-DMA too, ahead of the first stages, so
    // their latency overlaps the K/V loads: DMA block i holds rows 2i (lanes
    // 0..31) and 2i + 1 (lanes 32..63), 512 bytes each, and is loaded by wave
    // i % WS. Granule j of row r sits at slot j ^ 2(r & 15), which spreads
    // the 16 rows' reads below over the LDS banks.
    {
        const int rr = 2 * ws + (lane >> 5);
        const uint32_t qslot = (uint32_t) (lane & 31);
        const int4v qd = raw_desc(p.q + (int64_t) b * p.q_nb3, p.q_bytes);
        for (int i = ws, r2 = rr; i < (rows_here + 1) / 2; i += WS, r2 += 2 * WS) {
            const int rq = r2 < rows_here ? r2 : 0;
            const int tq = div_g(rq, p.G, p.g_magic);
            const uint32_t qofs = (uint32_t) (tq * p.q_nb1 + (kvh * p.G + rq - tq * p.G) * p.q_nb2);
            dma16(qd, qofs + ((qslot ^ (uint32_t) (2 * (r2 & 15))) & 31) * 16, lds_addr(qlds) + (uint32_t) (i * 1024));
        }
    }
    // fused: the weights and this kv head's new K / V rows travel the same
    // way (piece i by wave i % WS)
    if constexpr (FUSED) {
        for (int i = ws; i < kPieces; i += WS) {
            const char * src;
            if (i == 0) src = in.q_w;
            else if (i == 1) src = in.k_w;
            else if (i == 2) src = in.k + kvh * in.k_nb1;
            else src = in.v + kvh * 512;
            if (src) dma16(raw_desc(src, 512), (uint32_t) lane * 16, lds_addr(fin) + (uint32_t) (i * 1024));
        }
    }
    // Scalar loads (lgkm-counted, so the DMA waits are unaffected), issued
    // after the query rows' DMA and before the stages' (measured faster than
    // after them, where they queue behind the stages' traffic): the run-time
    // length (unconditional, from the error flags when there is no p.dyn, as
    // a branch would wait for them at once) and, fused, the token's position
    // and cache row (both words of an i64 row, or the i32 row twice).
    const int32_t * dsrc = p.dyn ? p.dyn : p.err;
    const int32_t dyn_len = ld_uniform(dsrc), dyn_pos0 = ld_uniform(dsrc + 1);
    int32_t pos_0 = 0;
    int64_t row_0 = 0;
    if constexpr (FUSED) {
        pos_0 = ld_uniform(in.pos);
        const uint32_t * rw = (const uint32_t *) in.rows;
        const uint32_t rlo = ld_uniform(rw), rhi = ld_uniform(rw + (in.rows64 ? 1 : 0));
        row_0 = in.rows64 ? (int64_t) (((uint64_t) rhi << 32) | rlo) : (int64_t) (int32_t) rlo;
    }
    // MASK 2: the mask values of this wave's stages (at the launch's bound)
    // into its LDS region, 32 bytes per (stage j, distinct mask row d) at
    // item j * D + d, before the first stages, so every wait for a stage
    // also covers them: DMA block k holds items 32 k .. 32 k + 31, lanes 2i
    // and 2i + 1 the two halves of item 32 k + i. D = p.mask_rows: the
    // workgroup's tokens when the mask rows are shared by the heads
    // (m_ne2 = 1), else its query rows. Items past the wave's last stage read
    // past the mask slice (zeros).
    if constexpr (MASK == 2) {
        const int D = p.mask_rows;
        const int items = ns_bound * D;
        const uint32_t mbase = lds_addr(mpre) + (uint32_t) (ws * p.mask_wave_bytes);
        for (int k = 0; 32 * k < items; ++k) {
            const int i = 32 * k + (lane >> 1);
            const int j = i / D, d = i - j * D;
            uint32_t off = 0xfffffff0u;
            if (i < items) {
                const int t = p.m_ne2 == 1 ? d : div_g(d, p.G, p.g_magic);
                const int hm = p.m_ne2 == 1 ? 0 : (kvh * p.G + d - t * p.G) % p.m_ne2;
                off = (uint32_t) ((int64_t) t * p.m_nb1 + (int64_t) hm * p.m_nb2) +
                      (uint32_t) (wbase + wstride * j) * 2u + (uint32_t) ((lane & 1) * 16);
            }
            dma16(md, off, mbase + (uint32_t) (k * 1024));
        }
    }
#pragma unroll
    for (int u = 0; u < NB - 1; ++u)
        if (u < n_pre) issue(u, u);
    // fused: wave 0 tabulates the rotation pairs' (cos, sin), lane i pair i
    // (while the DMA is in flight; the barrier below publishes it)
    if constexpr (FUSED) {
        if (ws == 0) {
            float c, sn;
            rope_cos_sin<FM>(in.rope, pos_0, lane, c, sn);
            rot_tab[lane] = float2{c, sn};
        }
    }

    // the run-time length (at most the launch's bound, so my_ns <= the
    // stages issued ahead + whatever the loop issues)
    int hi = p.kv_hi;
    int64_t cpos0 = p.causal_pos0;
    if (p.dyn) {
        hi = min(max(dyn_len, 0), p.kv_hi);
        if (cpos0 >= 0) cpos0 = max(dyn_pos0, 0);
    }
    hi = limit(hi, cpos0);
    const int c_end = range_end(hi);
    const int my_ns = wave_stages(hi);

    // own query rows landed (the stages were issued after them), then everyone's
    wait_later<NB - 1, PER>(n_pre);
    __syncthreads();

    // fused: the query rows through RMSNorm, weight and rotation in place,
    // and the new token's K row (normed, rotated) and V row as f16 (kv16),
    // for the wave whose stage holds the token's cell (it patches the stage)
    // and for split 0 (it writes the cache). Rows go to slots of 8 lanes:
    // slot s = 8 ws + lane / 8 (+ 8 WS per further pass) takes query row s
    // below rows_here and the K row at rows_here; lane t = lane % 8 of a slot
    // holds rotation pairs 8t..8t+7 (NEOX: dims 8t + k and 64 + 8t + k; pairs
    // (2i, 2i + 1) and no rotation: dims 16t + 2k and 16t + 2k + 1). Every
    // lane of a wave with a live slot computes (the row sums are shuffles);
    // only live slots store.
    int cell_0 = -1;                                                   // the new cell, -1 if out of range
    int j_own = -1;                                                    // this wave's stage that holds it
    if constexpr (FUSED) {
        const int t = lane & 7;
        float2 rot[8];
#pragma unroll
        for (int k = 0; k < 8; k += 2) {
            const float4 x = *(const float4 *) (rot_tab + 8 * t + k);
            rot[k] = float2{x.x, x.y};
            rot[k + 1] = float2{x.z, x.w};
        }
        const bool has_qw = in.q_w != nullptr, has_kw = in.k_w != nullptr;
        // the lane's four granules (4 dims each) of a row
        int gi[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) gi[m] = FM == 2 ? (m < 2 ? 2 * t + m : 16 + 2 * t + m - 2) : 4 * t + m;
        const int passes = (rows_here + 8 * WS) / (8 * WS);
        for (int pass = 0; pass < passes; ++pass) {
            const int s0 = pass * 8 * WS + 8 * ws;                       // the wave's first slot
            if (s0 > rows_here) continue;
            const int sl = s0 + (lane >> 3);
            const bool is_q = sl < rows_here, is_k = sl == rows_here;
            const int r = is_q ? sl : 0;
            const bool has_w = is_k ? has_kw : has_qw;
            const char * wsrc = fin + (is_k ? 1024 : 0);
            char * src[4];
            float4 a[4], w[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                // granule j of query row r sits at slot (j ^ 2(r & 15)) & 31
                src[m] = is_k ? fin + 2 * 1024 + gi[m] * 16 : qlds + r * 512 + (((gi[m] ^ (2 * (r & 15))) & 31) << 4);
                a[m] = *(const float4 *) src[m];
                w[m] = has_w ? *(const float4 *) (wsrc + gi[m] * 16) : float4{1.0f, 1.0f, 1.0f, 1.0f};
            }
            float lo[8], hi[8], wl[8], wh[8], ylo[8], yhi[8];
            if constexpr (FM == 2) {
#pragma unroll
                for (int m = 0; m < 2; ++m) {
                    lo[4 * m] = a[m].x; lo[4 * m + 1] = a[m].y; lo[4 * m + 2] = a[m].z; lo[4 * m + 3] = a[m].w;
                    hi[4 * m] = a[m + 2].x; hi[4 * m + 1] = a[m + 2].y; hi[4 * m + 2] = a[m + 2].z; hi[4 * m + 3] = a[m + 2].w;
                    wl[4 * m] = w[m].x; wl[4 * m + 1] = w[m].y; wl[4 * m + 2] = w[m].z; wl[4 * m + 3] = w[m].w;
                    wh[4 * m] = w[m + 2].x; wh[4 * m + 1] = w[m + 2].y; wh[4 * m + 2] = w[m + 2].z; wh[4 * m + 3] = w[m + 2].w;
                }
            } else {
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    lo[2 * m] = a[m].x; hi[2 * m] = a[m].y; lo[2 * m + 1] = a[m].z; hi[2 * m + 1] = a[m].w;
                    wl[2 * m] = w[m].x; wh[2 * m] = w[m].y; wl[2 * m + 1] = w[m].z; wh[2 * m + 1] = w[m].w;
                }
            }
            norm_rope_group8<FM>(lo, hi, wl, wh, in.eps, rot, ylo, yhi);
            float4 y[4];
            if constexpr (FM == 2) {
#pragma unroll
                for (int m = 0; m < 2; ++m) {
                    y[m] = float4{ylo[4 * m], ylo[4 * m + 1], ylo[4 * m + 2], ylo[4 * m + 3]};
                    y[m + 2] = float4{yhi[4 * m], yhi[4 * m + 1], yhi[4 * m + 2], yhi[4 * m + 3]};
                }
            } else {
#pragma unroll
                for (int m = 0; m < 4; ++m) y[m] = float4{ylo[2 * m], yhi[2 * m], ylo[2 * m + 1], yhi[2 * m + 1]};
            }
            if (is_q) {
#pragma unroll
                for (int m = 0; m < 4; ++m) *(float4 *) src[m] = y[m];
            }
            if (is_k) {
                // granule gi of the K row is dims 4gi..4gi+3: f16 at kv16 + 8gi;
                // the V row's dims 16t..16t+15 likewise at kv16 + 256 + 32t
#pragma unroll
                for (int m = 0; m < 4; ++m)
                    *(half4 *) (kv16 + gi[m] * 8) =
                        half4{(_Float16) y[m].x, (_Float16) y[m].y, (_Float16) y[m].z, (_Float16) y[m].w};
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const float4 v = *(const float4 *) (fin + 3 * 1024 + (4 * t + m) * 16);
                    *(half4 *) (kv16 + 256 + (4 * t + m) * 8) =
                        half4{(_Float16) v.x, (_Float16) v.y, (_Float16) v.z, (_Float16) v.w};
                }
            }
        }
        cell_0 = row_0 >= 0 && row_0 < in.n_rows ? (int) row_0 : -1;
        const int rel = cell_0 - wbase;
        if (cell_0 >= 0 && rel >= 0 && cell_0 < c_end && rel % wstride < kSC) j_own = rel / wstride;
        __syncthreads();                                               // every query row and kv16 ready
    }

    // Q^T B-operand fragments: k slots of block kb, group g = dims 32kb + 8g..+8
    half8 qf[RB][4];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const char * qrow = qlds + (16 * rb + n) * 512;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            const int j = 2 * (4 * kb + g);                               // granules j, j + 1 of the row
            const float4 qa = *(const float4 *) (qrow + ((j ^ (2 * n)) & 31) * 16);
            const float4 qb = *(const float4 *) (qrow + (((j + 1) ^ (2 * n)) & 31) * 16);
            qf[rb][kb] = rvalid[rb] ? to_half8(qa, qb) : half8{0, 0, 0, 0, 0, 0, 0, 0};
        }
    }

    float slope[RB];
    int lim[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        slope[rb] = 1.0f;
        if (p.max_bias > 0.0f) {                                       // arm.cpp:2294
            const uint32_t hq = (uint32_t) head[rb];
            slope[rb] = hq < p.n_head_log2 ? powf(p.m0, (float) (hq + 1))
                                           : powf(p.m1, (float) (2 * (hq - p.n_head_log2) + 1));
        }
        lim[rb] = row_limit(cpos0, hi, rvalid[rb], tok[rb]);
    }
    const int lim_min = row_limit(cpos0, hi, true, 0);

    floatx4 o[RB][8];
    float m_run[RB], l_run[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
        for (int mb = 0; mb < 8; ++mb) o[rb][mb] = floatx4{0, 0, 0, 0};
        m_run[rb] = -AL_INF;
        l_run[rb] = 0.0f;
    }

    // MASK 2: this lane's items in the wave's preloaded mask values (row
    // block rb: cells 4g .. 4g + 3 of its distinct mask row), per stage + 32 D
    const char * mp[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int d = p.m_ne2 == 1 ? tok[rb] : (rvalid[rb] ? 16 * rb + n : 0);
        mp[rb] = mpre + ws * p.mask_wave_bytes + d * 32 + 8 * g;
    }

    // LDS read offsets of this lane within a stage
    const int kread = n * 256;                                          // K row of cell n
    const int vcell = 4 * g + (n >> 2);                                 // V cell this lane supplies
    const int vread = 4096 + vcell * 256 + (n & 1) * 8;

    for (int j0 = 0; j0 < my_ns; j0 += NB) {
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const int j = j0 + u;
            if (j >= my_ns) break;
            // this stage landed (own DMA); slot (u + NB - 1) % NB was read
            // last iteration, so the stage NB - 1 ahead may fill it now
            wait_stage<NB, PER>(min(NB - 2, my_ns - 1 - j));
            if (j + NB - 1 < my_ns) issue(j + NB - 1, (u + NB - 1) % NB);
            mem_barrier();
            const char * st = &lds[ws][u][0];
            const int cs = wbase + wstride * j;
            if constexpr (FUSED) {
                // the new token's rows replace the cache's copy of its cell
                // (granule j of cell c at slot j ^ c): lanes 0..15 K, 16..31 V
                if (j == j_own && lane < 32) {
                    const int c = cell_0 - cs;
                    const int gj = lane & 15, part = lane >> 4;
                    *(u32x4 *) (&lds[ws][u][0] + part * 4096 + c * 256 + ((gj ^ c) << 4)) =
                        *(const u32x4 *) (kv16 + part * 256 + gj * 16);
                }
            }
            // the mask values first: LDS reads complete in order, so the
            // stage's mask test then waits for them alone, not for the K and
            // V^T operands behind them
            uint2 mk[RB];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                mk[rb] = uint2{0, 0};
                if constexpr (MASK == 1) mk[rb] = *(const uint2 *) (st + 8192 + 32 * (16 * rb + n) + 8 * g);
                if constexpr (MASK == 2) mk[rb] = *(const uint2 *) (mp[rb] + j * 32 * p.mask_rows);
            }
            u32x4 kf[4];
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) kf[kb] = *(const u32x4 *) (st + kread + (((4 * kb + g) ^ n) << 4));
            half4 vt[8];
#pragma unroll
            for (int mb = 0; mb < 8; ++mb) vt[mb] = lds_read_tr16(st + vread + (((2 * mb + ((n & 3) >> 1)) ^ vcell) << 4));

            // a stage is taken whole when the length / causal limit passes it
            // and, with a mask, every mask value of the stage is +0 (the
            // masked arithmetic would add zeros)
            bool full = cs + kSC - 1 <= lim_min;
            if constexpr (HAS_MASK) {
                uint32_t bits = 0;
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) bits |= mk[rb].x | mk[rb].y;
                full = full && __all(bits == 0u);
            }
            bool vis_any[4] = {!!full, !!full, !!full, !!full};
            half4 pf[RB];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                // S^T: cells 4g+i of row 16 rb + n
                floatx4 sc = {0, 0, 0, 0};
#pragma unroll
                for (int kb = 0; kb < 4; ++kb) sc = mfma_16x16x32(as_half8(kf[kb]), qf[rb][kb], sc);
                sc *= p.scale;
                if (p.softcap != 0.0f) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) sc[i] = p.softcap * tanhf(sc[i]);
                }
                if (!full) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        bool vis = cs + 4 * g + i <= lim[rb];
                        float x = sc[i];
                        if constexpr (HAS_MASK) {
                            const uint32_t w = i < 2 ? mk[rb].x : mk[rb].y;
                            const float mv = slope[rb] * f16_bits_to_float((uint16_t) (w >> (16 * (i & 1))));
                            vis = vis && (mv != -AL_INF);
                            x += mv;
                        }
                        sc[i] = vis ? x : -AL_INF;
                        vis_any[i] = vis_any[i] || vis;
                    }
                }
                const float mt = colmax4(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])));
                if (__any(mt > m_run[rb] + kTau)) {
                    const bool grow = mt > m_run[rb] + kTau;
                    const float mn = grow ? mt : m_run[rb];
                    const float alpha = grow ? exp_fast(m_run[rb] - mn) : 1.0f;
                    l_run[rb] *= alpha;
#pragma unroll
                    for (int mb = 0; mb < 8; ++mb) o[rb][mb] *= alpha;
                    m_run[rb] = mn;
                }
                const float mu = (m_run[rb] == -AL_INF) ? 0.0f : m_run[rb];
                float ps = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float pr = exp_fast(sc[i] - mu);
                    ps += pr;
                    pf[rb][i] = (_Float16) pr;
                }
                l_run[rb] += ps;
            }
            if (!full) {
                // cells masked for every row contribute exact zeros, whatever their V holds
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint64_t bal = __ballot(vis_any[i]);
                    if (((bal >> (16 * g)) & 0xffffull) == 0) {
#pragma unroll
                        for (int mb = 0; mb < 8; ++mb) vt[mb][i] = (_Float16) 0.0f;
                    }
                }
            }
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int mb = 0; mb < 8; ++mb) o[rb][mb] = mfma_16x16x16(vt[mb], pf[rb], o[rb][mb]);
        }
    }
    // stages issued ahead and not used (my_ns == 0 at run time) land before
    // the rings are reused (with my_ns > 0 the loop's last wait took them)
    wait_later<NB - 1, PER>(0);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) l_run[rb] = colsum4(l_run[rb]);

    // fused: split 0 stores the rotated query rows (when asked) and the new
    // token's K / V rows into the cache; a row out of range is not written
    // and is reported as set_rows reports it
    if constexpr (FUSED) {
        if (split == 0) {
            const int d0 = rope_d0<FM>(lane), d1 = rope_d1<FM>(lane);
            if (in.q_out) {
                for (int r = ws; r < rows_here; r += WS) {
                    const int t = div_g(r, p.G, p.g_magic);
                    const int hq = kvh * p.G + r - t * p.G;
                    const char * row = qlds + r * 512;
                    float * qo = (float *) (in.q_out + (int64_t) hq * in.qo_nb1 + (int64_t) t * in.qo_nb2);
                    qo[d0] = *(const float *) (row + (((d0 >> 2) ^ (2 * (r & 15))) & 31) * 16 + (d0 & 3) * 4);
                    qo[d1] = *(const float *) (row + (((d1 >> 2) ^ (2 * (r & 15))) & 31) * 16 + (d1 & 3) * 4);
                }
            }
            if (ws == 0) {
                if (cell_0 < 0) {
                    if (lane == 0 && atomicCAS(p.err, 0, 1) == 0) p.err[1] = (int) row_0;
                } else {
                    _Float16 * kc = (_Float16 *) (in.k_cache + (int64_t) cell_0 * in.kc_nb1) + kvh * 128;
                    _Float16 * vc = (_Float16 *) (in.v_cache + (int64_t) cell_0 * in.vc_nb1) + kvh * 128;
                    const _Float16 * k16 = (const _Float16 *) kv16;
                    const _Float16 * v16 = (const _Float16 *) (kv16 + 256);
                    kc[lane] = k16[lane];
                    kc[lane + 64] = k16[lane + 64];
                    vc[lane] = v16[lane];
                    vc[lane + 64] = v16[lane + 64];
                }
            }
        }
    }

    // Four or more waves, and two with short splits (OP), merge and publish
    // in one pass (kOnePass, below); otherwise the two waves merge through
    // an LDS record [row][132] (the rings are free once every wave is past
    // its loop), then wave 0 publishes. (Measured with two waves: the one
    // pass is faster up to 512 cells per split, the tree at 1024.)
    constexpr bool kOnePass = WS >= 4 || OP;
    if constexpr (WS > 1 && !kOnePass) {
        float * recs = (float *) &lds[0][0][0];
#pragma unroll
        for (int span = WS / 2; span >= 1; span /= 2) {
            __syncthreads();
            if (ws >= span && ws < 2 * span) {
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) {
                    float * rec = recs + (ws - span) * REC + (16 * rb + n) * kRowStride;
#pragma unroll
                    for (int mb = 0; mb < 8; ++mb)
                        *(float4 *) (rec + 16 * mb + 4 * g) = float4{o[rb][mb][0], o[rb][mb][1], o[rb][mb][2], o[rb][mb][3]};
                    if (g == 0) *(float2 *) (rec + 128) = float2{m_run[rb], l_run[rb]};
                }
            }
            __syncthreads();
            if (ws < span) {
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) {
                    const float * rec = recs + ws * REC + (16 * rb + n) * kRowStride;
                    const float2 ml = *(const float2 *) (rec + 128);
                    const float mn = fmaxf(m_run[rb], ml.x);
                    const float mu = (mn == -AL_INF) ? 0.0f : mn;
                    const float wa = exp_fast(m_run[rb] - mu);
                    const float wb = exp_fast(ml.x - mu);
#pragma unroll
                    for (int mb = 0; mb < 8; ++mb) {
                        const float4 x = *(const float4 *) (rec + 16 * mb + 4 * g);
                        o[rb][mb][0] = o[rb][mb][0] * wa + x.x * wb;
                        o[rb][mb][1] = o[rb][mb][1] * wa + x.y * wb;
                        o[rb][mb][2] = o[rb][mb][2] * wa + x.z * wb;
                        o[rb][mb][3] = o[rb][mb][3] * wa + x.w * wb;
                    }
                    l_run[rb] = l_run[rb] * wa + ml.y * wb;
                    m_run[rb] = mn;
                }
            }
        }
    }

    if (!kOnePass && p.n_split == 1) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            if (ws == 0 && rvalid[rb]) {
                float * out = (float *) (p.dst + ((int64_t) (b * p.T + tok[rb]) * p.Hq + head[rb]) * p.dst_nb1);
                const RowScale rs = row_scale(m_run[rb], l_run[rb], p.sinks, head[rb]);
#pragma unroll
                for (int mb = 0; mb < 8; ++mb)
                    *(float4 *) (out + 16 * mb + 4 * g) =
                        apply_scale(float4{o[rb][mb][0], o[rb][mb][1], o[rb][mb][2], o[rb][mb][3]}, rs);
            }
        }
        return;
    }

    // Publish this split's record and then, once its stores have completed,
    // the split's flag; K = min(n_split, rows) splits of the unit merge, merger
    // k taking rows k, k + K, ... (the merge is bound by the record bytes one
    // CU loads, so it is spread). A split's record holds the O rows of its 16
    // RB query rows (512 bytes each), then their (m, l) pairs, so that the
    // pairs share no line with O and every line is loaded once (re-reading a
    // line device-coherently is slow). Flags live in the upper half of the
    // counter region, 64 words per unit: a word per split and the unit's
    // epoch (word 32). A split sets its flag to epoch + 1; the mergers wait for
    // every flag to read epoch + 1; merger 0 then advances the epoch (every
    // split read it before setting its flag), so nothing needs clearing and
    // the next call in stream order waits for epoch + 2. Each split reads the
    // epoch after its loop, once its own DMA has completed (an earlier load
    // would shift the DMA counts the stage waits rely on). The mergers are
    // rotated by unit % 8 so that different units' mergers, and their
    // polling, fall on different XCDs (workgroup ids go round the XCDs, split
    // fastest). A merger waits only for workgroups of its own unit, which on
    // every XCD are dispatched ahead of any later unit's; its polls are
    // bounded anyway (kFlagPollLimit).
    constexpr uint32_t RS = 16 * RB * kDecodeRecRow;                  // bytes of one split's record
    constexpr uint32_t kPairs0 = 16 * RB * 512;                       // the pairs' offset in a record
    const rsrc_t pr = make_rsrc(p.part + (int64_t) unit * p.n_split * (RS / 4), RS * (uint32_t) p.n_split);
    unsigned * flags = p.counters + kFattnCounterWords + unit * kFattnDecodeFlagWords;
    const int K = min(p.n_split, (rows_here + p.merge_rows - 1) / p.merge_rows);
    const int kidx = ((p.n_split - 1 - split - unit % 8) % p.n_split + p.n_split) % p.n_split;
    unsigned epoch = 0;
    if constexpr (kOnePass) {
        // Every wave puts its rows' state into its own ring (its DMA has
        // landed): O rows of 32 granules, granule j of row r at slot j ^ (r &
        // 31), and the rows' (m, l) pairs after them, or in the query-row
        // buffer when the ring has no room (the query rows are in registers;
        // with the inputs folded in the ring always has room). After one
        // barrier every thread takes (row, 4 dims) items, combines the WS
        // states in wave order (the merge records' arithmetic) and writes the
        // row's output (one split) or this split's record, whose (m, l) pair
        // comes with the item of dims 0..3; once every wave's stores have
        // completed, wave 0 sets the split's flag.
        constexpr int kRecO = 16 * RB * 512;
        constexpr bool kMLinRing = NB * STAGE - kRecO >= 16 * RB * 8;
        static_assert(NB * STAGE >= kRecO, "a wave's O rows fit its ring");
        static_assert(kMLinRing || !FUSED, "the folded inputs keep the query rows until the merge");
        auto rec_o = [&](const int w) { return &lds[w][0][0]; };
        auto rec_ml = [&](const int w) {
            return kMLinRing ? (float2 *) (&lds[w][0][0] + kRecO) : (float2 *) qlds + w * 16 * RB;
        };
        // (a wave with no stages gets here while another may still be
        // reading its query fragments from qlds)
        if constexpr (!kMLinRing) __syncthreads();
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int r = 16 * rb + n;
#pragma unroll
            for (int mb = 0; mb < 8; ++mb)
                *(float4 *) (rec_o(ws) + (r * 32 + ((4 * mb + g) ^ (r & 31))) * 16) =
                    float4{o[rb][mb][0], o[rb][mb][1], o[rb][mb][2], o[rb][mb][3]};
            if (g == 0) rec_ml(ws)[r] = float2{m_run[rb], l_run[rb]};
        }
        if (ws == 0 && p.n_split > 1) epoch = ld_agent_u32(flags + 32);
        __syncthreads();
        for (int item = threadIdx.x; item < rows_here * 32; item += WS * 64) {
            const int r = item >> 5, d4 = item & 31;
            float M = -AL_INF;
#pragma unroll
            for (int w = 0; w < WS; ++w) M = fmaxf(M, rec_ml(w)[r].x);
            const float Mu = (M == -AL_INF) ? 0.0f : M;
            float L = 0.0f;
            float4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int w = 0; w < WS; ++w) {
                const float2 ml = rec_ml(w)[r];
                const float wt = exp_fast(ml.x - Mu);
                const float4 x = *(const float4 *) (rec_o(w) + (r * 32 + (d4 ^ (r & 31))) * 16);
                L += wt * ml.y;
                acc.x += wt * x.x; acc.y += wt * x.y; acc.z += wt * x.z; acc.w += wt * x.w;
            }
            if (p.n_split == 1) {
                const int t = div_g(r, p.G, p.g_magic);
                const int hq = kvh * p.G + r - t * p.G;
                float * out = (float *) (p.dst + ((int64_t) (b * p.T + t) * p.Hq + hq) * p.dst_nb1);
                *(float4 *) (out + 4 * d4) = finalize4(acc, M, L, p.sinks, hq);
            } else {
                buf_store16_dev(acc, pr, (uint32_t) split * RS + (uint32_t) (r * 512 + d4 * 16));
                if (d4 == 0) buf_store8_dev(float2{M, L}, pr, (uint32_t) split * RS + kPairs0 + (uint32_t) (r * 8));
            }
        }
        if (p.n_split == 1) return;
        complete_wave_memops();
        __syncthreads();
        if (ws == 0 && lane == 0) st_agent_u32(flags + split, epoch + 1u);
    } else if (ws == 0) {
        epoch = ld_agent_u32(flags + 32);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            if (rvalid[rb]) {
                const uint32_t row = (uint32_t) split * RS + (uint32_t) ((16 * rb + n) * 512);
#pragma unroll
                for (int mb = 0; mb < 8; ++mb)
                    buf_store16_dev(float4{o[rb][mb][0], o[rb][mb][1], o[rb][mb][2], o[rb][mb][3]}, pr,
                                    row + (16 * mb + 4 * g) * 4);
                if (g == 0)
                    buf_store8_dev(float2{m_run[rb], l_run[rb]}, pr, (uint32_t) split * RS + kPairs0 + (uint32_t) ((16 * rb + n) * 8));
            }
        }
        complete_wave_memops();
        if (lane == 0) st_agent_u32(flags + split, epoch + 1u);
    }
    if (kidx >= K) return;
    // A merger that gives up waiting (kFlagPollLimit) records the device
    // error and writes NaN rows, so that the failure shows in dst as well.
    int * const merge_failed = (int *) qlds;                           // the query rows are in registers
    if (ws == 0) {
        int gave_up = 0;
        for (int tries = 0;; ++tries) {
            const unsigned f = lane < p.n_split ? ld_agent_u32(flags + lane) : epoch + 1u;
            if (__all(f == epoch + 1u)) break;
            if (tries >= kFlagPollLimit) {
                gave_up = 1;
                if (lane == 0) atomicCAS(p.err + 2, 0, 1);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        order_after_counter();
        if (kidx == 0 && lane == 0 && !gave_up) st_agent_u32(flags + 32, epoch + 1u);
        if (lane == 0) *merge_failed = gave_up;
    }
    __syncthreads();
    const bool failed = *merge_failed != 0;

    // The merge of this merger's n_my rows. The (m, l) pair of every (row,
    // split) is loaded once (thread i takes pairs i, i + 64 WS, ...), turned
    // into the split's weight and shared through LDS; the output items are two adjacent lanes per (row,
    // 4 dims), each taking 16 of the at most 32 splits and then combining
    // with its partner (split half 0 first, on both lanes). The first
    // round's O loads are issued before the pairs go to LDS, so a merger of
    // up to 2 WS rows (WS = 2: 4 rows) makes one round trip.
    const int n_my = (rows_here - kidx + K - 1) / K;
    auto row_of = [&](const int lr) { return kidx + K * lr; };       // merger-local row -> row
    constexpr int kHalf = kMaxSplit / 2;
    constexpr int kItems = RB == 1 ? 2 : 1;                            // items per thread and round (registers)
    constexpr int kPairs = (16 * RB * kMaxSplit + WS * 64 - 1) / (WS * 64);
    float2 * ml_s = (float2 *) &lds[0][0][0];                          // [local row][kMaxSplit]; the rings are free
    float * m_row = (float *) (ml_s + 16 * RB * kMaxSplit);            // [local row]
    // (loads are unconditional, from clamped in-range addresses, and the
    // unused ones are replaced afterwards: no branch, so the O loads below
    // stay in flight while the pairs are stored)
    float2 mlv[kPairs];
#pragma unroll
    for (int i = 0; i < kPairs; ++i) {
        const int pi = i * WS * 64 + threadIdx.x;
        const int rr = row_of(min(pi / kMaxSplit, n_my - 1)), sp = min(pi % kMaxSplit, p.n_split - 1);
        mlv[i] = buf_load8_dev(pr, (uint32_t) sp * RS + kPairs0 + (uint32_t) (rr * 8));
    }
    const int n_items = n_my * 64;
    for (int base = 0; base < n_items; base += kItems * WS * 64) {
        float4 ov[kItems][kHalf];
#pragma unroll
        for (int it2 = 0; it2 < kItems; ++it2) {
            const int idx = base + it2 * WS * 64 + threadIdx.x;
            const int half = idx & 1;
            const int d4 = (idx >> 1) & 31;
            const int rr = row_of(idx < n_items ? idx >> 6 : 0);
            // an item slot of a round past the merger's items loads nothing
            // (a uniform branch: 8 waves with 8 rows fill one slot per thread)
            if (it2 > 0 && base + it2 * WS * 64 >= n_items) {
#pragma unroll
                for (int j = 0; j < kHalf; ++j) ov[it2][j] = float4{0.0f, 0.0f, 0.0f, 0.0f};
                continue;
            }
#pragma unroll
            for (int j = 0; j < kHalf; ++j) {
                const int sp = min(half * kHalf + j, p.n_split - 1);
                ov[it2][j] = buf_load16_dev(pr, (uint32_t) sp * RS + (uint32_t) (rr * 512 + d4 * 16));
            }
        }
        if (base == 0) {
            // the pairs into LDS as (weight, l), weight = e^(m - M) with M the
            // row's largest m over its splits (a row's kMaxSplit pairs are
            // adjacent lanes of one wave), and the row maxima beside them, so
            // that the items below only multiply and add; once per (row,
            // split) of this merger's rows instead of once per item (LDS and
            // lane exchanges only: no wait for the O loads in flight)
            static_assert(kMaxSplit == 32, "a row's pairs are the 32 lanes max32 reduces");
#pragma unroll
            for (int i = 0; i < kPairs; ++i) {
                if (i * WS * 64 >= n_my * kMaxSplit) break;               // past this merger's rows (uniform)
                const int pi = i * WS * 64 + threadIdx.x;
                const float2 v = (pi % kMaxSplit) < p.n_split ? mlv[i] : float2{-AL_INF, 0.0f};
                const float M = max32(v.x);
                const float Mu = (M == -AL_INF) ? 0.0f : M;
                ml_s[pi] = float2{exp_fast(v.x - Mu), v.y};
                if (pi % kMaxSplit == 0) m_row[pi / kMaxSplit] = M;
            }
            mem_barrier();
            __builtin_amdgcn_s_waitcnt(0xC07F);                        // lgkmcnt(0)
            __builtin_amdgcn_s_barrier();
            mem_barrier();
        }
#pragma unroll
        for (int it2 = 0; it2 < kItems; ++it2) {
            const int idx = base + it2 * WS * 64 + threadIdx.x;
            const int half = idx & 1;
            const int d4 = (idx >> 1) & 31;
            const int lr = idx < n_items ? idx >> 6 : 0;
            float2 wl[kHalf];                                          // (weight, l) of its splits
#pragma unroll
            for (int j = 0; j < kHalf; ++j) wl[j] = ml_s[lr * kMaxSplit + half * kHalf + j];
            const float M = m_row[lr];
            float Lh = 0.0f;
            float4 ah = {0, 0, 0, 0};
#pragma unroll
            for (int j = 0; j < kHalf; ++j) {
                const float w = wl[j].x;
                Lh += w * wl[j].y;
                ah.x += w * ov[it2][j].x; ah.y += w * ov[it2][j].y; ah.z += w * ov[it2][j].z; ah.w += w * ov[it2][j].w;
            }
            const float Lo = __shfl_xor(Lh, 1);
            const float4 ao = {__shfl_xor(ah.x, 1), __shfl_xor(ah.y, 1), __shfl_xor(ah.z, 1), __shfl_xor(ah.w, 1)};
            if (half == 0 && idx < n_items) {
                const int rr = row_of(lr);
                const float L = Lh + Lo;
                const float4 acc = {ah.x + ao.x, ah.y + ao.y, ah.z + ao.z, ah.w + ao.w};
                const int t = div_g(rr, p.G, p.g_magic);
                const int hq = kvh * p.G + rr - t * p.G;
                float * out = (float *) (p.dst + ((int64_t) (b * p.T + t) * p.Hq + hq) * p.dst_nb1);
                *(float4 *) (out + 4 * d4) =
                    failed ? float4{__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf("")}
                           : finalize4(acc, M, L, p.sinks, hq);
            }
        }
    }
}

template <int WS, int NB, bool OP>
void launch_masks(const FattnParams & p, const dim3 grid, hipStream_t stream) {
    const DecodeInputs none = {};
    if (p.mask && p.mask_pre) hipLaunchKernelGGL((fattn_decode_kernel<WS, NB, 2, 1, -1, OP>), grid, dim3(WS * 64), 0, stream, p, none);
    else if (p.mask)          hipLaunchKernelGGL((fattn_decode_kernel<WS, NB, 1, 1, -1, OP>), grid, dim3(WS * 64), 0, stream, p, none);
    else                      hipLaunchKernelGGL((fattn_decode_kernel<WS, NB, 0, 1, -1, OP>), grid, dim3(WS * 64), 0, stream, p, none);
}

// p.one_pass selects the one-pass merge for the 2 x 3 shape (the others
// have it always (four or more waves) or never).
template <int WS, int NB>
hipError_t launch_cfg(const FattnParams & p, hipStream_t stream) {
    const dim3 grid((unsigned) p.n_split, (unsigned) p.Hkv, (unsigned) p.B);
    if constexpr (WS == 2 && NB == 3) {
        if (p.one_pass) {
            launch_masks<WS, NB, true>(p, grid, stream);
            return hipGetLastError();
        }
    }
    launch_masks<WS, NB, (WS >= 4)>(p, grid, stream);
    return hipGetLastError();
}

template <int WS, int NB, bool OP>
void launch_fused_modes(const FattnParams & p, const DecodeInputs & in, const int mode, hipStream_t stream) {
    const dim3 grid((unsigned) p.n_split, (unsigned) p.Hkv, 1);
    switch (mode) {
        case 2: hipLaunchKernelGGL((fattn_decode_kernel<WS, NB, 0, 1, 2, OP>), grid, dim3(WS * 64), 0, stream, p, in); break;
        case 1: hipLaunchKernelGGL((fattn_decode_kernel<WS, NB, 0, 1, 1, OP>), grid, dim3(WS * 64), 0, stream, p, in); break;
        default: hipLaunchKernelGGL((fattn_decode_kernel<WS, NB, 0, 1, 0, OP>), grid, dim3(WS * 64), 0, stream, p, in); break;
    }
}

template <int WS, int NB>
hipError_t launch_fused(const FattnParams & p, const DecodeInputs & in, const int mode, hipStream_t stream) {
    if constexpr (WS == 2) {
        if (p.one_pass) {
            launch_fused_modes<WS, NB, true>(p, in, mode, stream);
            return hipGetLastError();
        }
    }
    launch_fused_modes<WS, NB, (WS >= 4)>(p, in, mode, stream);
    return hipGetLastError();
}

}  // namespace

bool fattn_decode_config_ok(int waves, int stages) {
    switch (waves * 10 + stages) {
        case 23: case 24: case 43: case 44: case 82: return true;
        default: return false;
    }
}

size_t fattn_decode_lds_bytes(int waves, int stages, bool mask, bool mask_pre) {
    return (size_t) waves * stages * (8192 + (mask && !mask_pre ? 1024 : 0)) + (mask && mask_pre ? kDecodeMaskPreBytes : 0);
}

hipError_t fattn_decode_launch(const FattnParams & p, int waves, int stages, hipStream_t stream) {
    if (p.R > 16) {
        // 17..32 rows: two row blocks, 8 waves x 2 stages
        if (p.R > 32 || waves != 8 || stages != 2) return hipErrorInvalidValue;
        const dim3 grid((unsigned) p.n_split, (unsigned) p.Hkv, (unsigned) p.B);
        const DecodeInputs none = {};
        if (p.mask && p.mask_pre) hipLaunchKernelGGL((fattn_decode_kernel<8, 2, 2, 2, -1, true>), grid, dim3(8 * 64), 0, stream, p, none);
        else if (p.mask)          hipLaunchKernelGGL((fattn_decode_kernel<8, 2, 1, 2, -1, true>), grid, dim3(8 * 64), 0, stream, p, none);
        else                      hipLaunchKernelGGL((fattn_decode_kernel<8, 2, 0, 2, -1, true>), grid, dim3(8 * 64), 0, stream, p, none);
        return hipGetLastError();
    }
    switch (waves * 10 + stages) {
        case 23: return launch_cfg<2, 3>(p, stream);
        case 24: return launch_cfg<2, 4>(p, stream);
        case 43: return launch_cfg<4, 3>(p, stream);
        case 44: return launch_cfg<4, 4>(p, stream);
        case 82: return launch_cfg<8, 2>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

bool fattn_decode_fused_ok(int waves, int stages) { return (waves == 2 && stages == 3) || (waves == 8 && stages == 2); }

hipError_t fattn_decode_launch_fused(const FattnParams & p, const DecodeInputs & in, int mode, int waves, int stages,
                                     hipStream_t stream) {
    if (p.R > 16 || p.B != 1 || p.mask || in.T != 1 || mode < 0 || mode > 2)
        return hipErrorInvalidValue;
    if (waves == 2 && stages == 3) return launch_fused<2, 3>(p, in, mode, stream);
    if (waves == 8 && stages == 2) return launch_fused<8, 2>(p, in, mode, stream);
    return hipErrorInvalidValue;
}
