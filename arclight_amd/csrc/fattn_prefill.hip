// Prefill (and long speculative-verify) attention for gfx950: many query rows
// per kv head, causal / length masking given implicitly (kv_len,
// causal_pos0). Semantics as nnml_compute_forward_flash_attn_ext_f16
// (nnml/src/ops/arm/arm.cpp:2196-2433), numerics as fattn_splitkv.hip.
//
// One workgroup = one row tile of 64 query rows of one kv-head group
// (row r -> token r / G, head kvh*G + r % G) and 4 wavefronts. Every wave
// holds all 64 rows (4 MFMA row blocks, so each K/V operand feeds 4 MFMAs)
// and takes every 4th 32-cell tile of the visible range; the 4 online-softmax
// states merge through LDS at the end. A 512-token chunk of Qwen3-4B gives
// 32 row tiles x 8 kv heads = 256 workgroups: one wave per SIMD of every CU.
//
// K/V tiles travel HBM/L2 -> LDS by buffer loads with the LDS-DMA path
// (buffer_load_dwordx4 ... lds): each lane's 16 bytes land at its own slot
// of a 1 KiB row, so reading them back (ds_read_b128 at lane*16) yields
// exactly the MFMA operand layout of the register path, and two tiles per
// wave are in flight without costing registers. The compiler does not track
// LDS-DMA completion, so the waits are explicit: before a tile is read, only
// the loads of the following tile may still be outstanding.
//
// The 1-D grid runs kv head fastest (XCD affinity: with Hkv = 8 each head's
// K/V stays in one XCD's L2) and, with a causal mask, row tiles longest
// first.

#include "fattn_tile.hpp"

namespace {

using namespace fattn;

constexpr int kPW = 4;                       // waves per workgroup
constexpr int kPRB = 4;                      // MFMA row blocks per wave
constexpr int kPRows = 16 * kPRB;            // query rows per workgroup
constexpr int kTileBytes = 16 * 1024;        // one 32-cell K+V tile: 16 DMA rows of 1 KiB

typedef __attribute__((address_space(3))) void lds_void_t;

// s_waitcnt immediates (gfx9 encoding: vmcnt {15:14,3:0}, expcnt 6:4,
// lgkmcnt 11:8; all-ones = no wait)
constexpr int kWaitVm16 = (1 << 14) | (7 << 4) | (15 << 8);   // vmcnt(16)
constexpr int kWaitVm0 = (7 << 4) | (15 << 8);                // vmcnt(0)
constexpr int kWaitLgkm0 = 0xC00F | (7 << 4);                  // lgkmcnt(0)

__device__ __forceinline__ void mem_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
}

// 16 DMA loads of one 32-cell tile into a wave's 16 KiB LDS stage:
// rows 0..7 the K chunks [mb][kb], rows 8..15 the V chunks [j].
__device__ __forceinline__ void dma_tile(char * stage, const FattnParams & p, const rsrc_t kr, const rsrc_t vr,
                                         const int cb, const int g, const int n) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
        const uint32_t off = (uint32_t) (cb + 16 * mb + n) * (uint32_t) p.k_nb1;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(kr, (lds_void_t *) (stage + (mb * 4 + kb) * 1024), 16,
                                                     off + (4 * kb + g) * 16, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(vr, (lds_void_t *) (stage + (8 + j) * 1024), 16,
                                                 (uint32_t) (cb + cell_of_slot(g, j)) * (uint32_t) p.v_nb1 + n * 16,
                                                 0, 0, 0);
}

__device__ __forceinline__ void read_k(Tile<kPRB> & t, const char * stage, const int lane) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) t.k[mb][kb] = *(const u32x4 *) (stage + (mb * 4 + kb) * 1024 + lane * 16);
}
__device__ __forceinline__ void read_v(Tile<kPRB> & t, const char * stage, const int lane) {
#pragma unroll
    for (int j = 0; j < 8; ++j) t.v[j] = *(const u32x4 *) (stage + (8 + j) * 1024 + lane * 16);
}

__global__ __launch_bounds__(kPW * 64) void fattn_prefill_kernel(const FattnParams p) {
    __shared__ __attribute__((aligned(16))) char lds[kPW][2][kTileBytes];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
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
    const rsrc_t kr = make_rsrc(kbase, (uint32_t) ((p.n_kv - 1) * p.k_nb1 + 256));
    const rsrc_t vr = make_rsrc(vbase, (uint32_t) ((p.n_kv - 1) * p.v_nb1 + 256));

    // this wave's tiles: cells cb0 + it * 128
    constexpr int kStride = kPW * 32;
    const int cb0 = wave * 32;
    const int ntiles = cb0 < hi ? (hi - cb0 + kStride - 1) / kStride : 0;

    int tok[kPRB];
    int head[kPRB];
    bool rvalid[kPRB];
    float slope[kPRB];
    half8 qf[kPRB][4];
#pragma unroll
    for (int rb = 0; rb < kPRB; ++rb) {
        const int r = row0 + 16 * rb + n;
        rvalid[rb] = (16 * rb + n) < rows_here;
        tok[rb] = rvalid[rb] ? r / p.G : 0;
        head[rb] = kvh * p.G + (rvalid[rb] ? r % p.G : 0);
        slope[rb] = 1.0f;
        const float * qrow = (const float *) (p.q + (int64_t) b * p.q_nb3 + (int64_t) tok[rb] * p.q_nb1 +
                                              (int64_t) head[rb] * p.q_nb2);
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            const float4 a = *(const float4 *) (qrow + 8 * (4 * kb + g));
            const float4 cc = *(const float4 *) (qrow + 8 * (4 * kb + g) + 4);
            qf[rb][kb] = rvalid[rb] ? to_half8(a, cc) : half8{0, 0, 0, 0, 0, 0, 0, 0};
        }
    }

    int lim[kPRB];
#pragma unroll
    for (int rb = 0; rb < kPRB; ++rb) lim[rb] = row_limit(p, hi, rvalid[rb], tok[rb]);
    const int lim_min = row_limit(p, hi, true, row0 / p.G);          // the tile's first token

    floatx4 o[kPRB][8];
    float m_run[kPRB];
    float l_run[kPRB];
#pragma unroll
    for (int rb = 0; rb < kPRB; ++rb) {
        m_run[rb] = -AL_INF;
        l_run[rb] = 0.0f;
#pragma unroll
        for (int d = 0; d < 8; ++d) o[rb][d] = floatx4{0, 0, 0, 0};
    }
    // (stage pointers are taken from the LDS array itself each time, so the
    // compiler keeps them in the LDS address space: ds_read, not flat loads,
    // which would count against vmcnt and wait for the DMA in flight)
    if (ntiles > 0) dma_tile(lds[wave][0], p, kr, vr, cb0, g, n);
    if (ntiles > 1) dma_tile(lds[wave][1], p, kr, vr, cb0 + kStride, g, n);
    for (int it = 0; it < ntiles; ++it) {
        // this tile's 16 DMA loads are complete once at most the next tile's
        // 16 are outstanding
        mem_barrier();
        if (it + 1 < ntiles) __builtin_amdgcn_s_waitcnt(kWaitVm16);
        else __builtin_amdgcn_s_waitcnt(kWaitVm0);
        mem_barrier();
        Tile<kPRB> t;
        read_k(t, lds[wave][it & 1], lane);
        read_v(t, lds[wave][it & 1], lane);
        mem_barrier();
        __builtin_amdgcn_s_waitcnt(kWaitLgkm0);          // stage free again
        mem_barrier();
        if (it + 2 < ntiles) dma_tile(lds[wave][it & 1], p, kr, vr, cb0 + (it + 2) * kStride, g, n);
        process_tile<kPRB, false>(t, cb0 + it * kStride, p, g, lim, lim_min, slope, qf, o, m_run, l_run);
    }

#pragma unroll
    for (int rb = 0; rb < kPRB; ++rb) l_run[rb] = colsum4(l_run[rb]);

    // merge the 4 waves through one LDS record (in the tile buffers, free now)
    __syncthreads();
    float * rec = (float *) &lds[0][0][0];
    for (int w = kPW - 1; w > 0; --w) {
        if (wave == w) store_state<kPRB>(rec, o, m_run, l_run, g, n);
        __syncthreads();
        if (wave == 0) merge_state<kPRB>(rec, o, m_run, l_run, g, n);
        __syncthreads();
    }
    if (wave != 0) return;
#pragma unroll
    for (int rb = 0; rb < kPRB; ++rb) {
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

}  // namespace

size_t fattn_prefill_lds_bytes() { return sizeof(char) * kPW * 2 * kTileBytes; }

hipError_t fattn_prefill_launch(const FattnParams & p, hipStream_t stream) {
    const dim3 grid((unsigned) ((int64_t) p.Hkv * p.n_row_tiles * p.B));
    hipLaunchKernelGGL(fattn_prefill_kernel, grid, dim3(kPW * 64), 0, stream, p);
    return hipGetLastError();
}
