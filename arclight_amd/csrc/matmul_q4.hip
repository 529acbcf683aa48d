// The attention output projection (WO) with Q4_0 weights for gfx950
// (include/arclight_matmul.h).
//
// Semantics: nnml_compute_forward_mul_mat for src0 Q4_0 / src1 f32
// (nnml/src/ops/ops.cpp:1252-1274, forward_mul_mat_generic,
// nnml/src/ops/arm/common.cpp:120-...): each activation row is quantized to
// Q8_0 (quantize_row_q8_0, arm.cpp:1819-1848: d = amax / 127, q = x / d
// rounded to nearest even), and y[t][n] = sum over blocks of
// (sumi * d_w) * d_x with sumi the integer dot product of the block's
// weights minus 8 and its Q8_0 values (nnml_vec_dot_q4_0_q8_0, arm.cpp:401).
//
// Up to 8 tokens (decode, speculative verify) take one launch,
// gemv_q4_fused_kernel: one wavefront per output row, every row resident at
// once; each workgroup issues its rows' weight loads, quantizes all T
// activation rows into LDS meanwhile (the activations are small and
// L2-resident), then lane l forms the dot products of the row's blocks
// l*BPL .. l*BPL + BPL - 1 (a contiguous 36-byte-aligned run of 18-byte
// blocks held in registers) with 8 v_dot4_i32_i8 per block on the unsigned
// nibbles, the weights' offset of 8 folded into one multiply by the block's
// value sum; lane sums meet in a DPP wave reduction.
// Longer inputs (up to 64 tokens) take two launches: quantize_q8_kernel
// (one thread per (token, block), into grow-only library scratch) and
// gemv_q4_kernel (the same dot products, activations from that scratch).
// Either way the 4-bit weights stream once: HBM-bound, 18 bytes per 32
// weights.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <mutex>

#include "../../include/arclight_matmul.h"
#include "kernel_args.hpp"
#include "runtime.hpp"

namespace {

constexpr int kMaxT = 64;

__global__ __launch_bounds__(256) void quantize_q8_kernel(const char * __restrict__ x, int64_t x_nb1, int K, int T,
                                                          int8_t * __restrict__ qs, float * __restrict__ dx,
                                                          int * __restrict__ sy) {
    const int nb = K / 32;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= T * nb) return;
    const int t = i / nb, b = i % nb;
    const float4 * xb = (const float4 *) ((const float *) (x + (int64_t) t * x_nb1) + 32 * b);
    float v[32];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float4 f = xb[j];
        v[4 * j] = f.x; v[4 * j + 1] = f.y; v[4 * j + 2] = f.z; v[4 * j + 3] = f.w;
    }
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(v[j]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    int sum = 0;
    uint32_t words[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        uint32_t wv = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int q = (int) rintf(v[4 * j + k] * id);                 // ties to even, as vcvtnq
            sum += q;
            wv |= (uint32_t) (q & 0xff) << (8 * k);
        }
        words[j] = wv;
    }
    uint4 * out = (uint4 *) (qs + (int64_t) t * K + 32 * b);
    out[0] = uint4{words[0], words[1], words[2], words[3]};
    out[1] = uint4{words[4], words[5], words[6], words[7]};
    dx[i] = (float) (_Float16) d;                                          // the block scale as stored (f16)
    sy[i] = sum;
}

// Cross-lane moves on the VALU (DPP): within rows of 16 lanes, then the
// broadcasts of a row's last lane into the next row(s).
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xf, false));
}
constexpr int kQuadXor1 = 0xB1, kQuadXor2 = 0x4E, kRowHalfMirror = 0x141, kRowMirror = 0x140, kRowBcast15 = 0x142,
              kRowBcast31 = 0x143, kRowRor8 = 0x128;

// Sum over the wavefront; the total is valid in lane 63 only.
__device__ __forceinline__ float wave_sum_to_last(float v) {
    v += dpp<kQuadXor1>(v);
    v += dpp<kQuadXor2>(v);
    v += dpp<kRowHalfMirror>(v);                                       // lane i <-> 7 - i of its 8
    v += dpp<kRowMirror>(v);                                           // lane i <-> 15 - i of its 16
    v += dpp<kRowBcast15, 0xa>(v);                                     // rows 1, 3 += last lane of rows 0, 2
    v += dpp<kRowBcast31, 0xc>(v);                                     // rows 2, 3 += lane 31
    return v;
}

// Q4_0 block j (0 .. BPL-1) of a lane's chunk of 18-byte blocks held as
// 9 * BPL / 2 dwords: its scale and its 16 bytes of nibbles as 4 dwords.
template <int BPL>
__device__ __forceinline__ void block_of(const uint32_t (&c)[9 * BPL / 2], const int j, float & d, uint32_t (&q)[4]) {
    const int byte = 18 * j;                                           // even
    const int w0 = byte >> 2;
    if ((byte & 3) == 0) {
        d = (float) __builtin_bit_cast(_Float16, (uint16_t) (c[w0] & 0xffff));
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = __builtin_amdgcn_alignbyte(c[w0 + i + 1], c[w0 + i], 2);
    } else {
        d = (float) __builtin_bit_cast(_Float16, (uint16_t) (c[w0] >> 16));
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = c[w0 + 1 + i];
    }
}

template <int BPL>
__global__ __launch_bounds__(256) void gemv_q4_kernel(const char * __restrict__ w, int64_t w_nb1, int N, int K,
                                                      const int8_t * __restrict__ qs, const float * __restrict__ dx,
                                                      const int * __restrict__ sy, int T, char * __restrict__ y,
                                                      int64_t y_nb1) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= N) return;
    const int nb = K / 32;
    const int b0 = lane * BPL;

    // the lane's blocks of this row, 36-byte aligned in global memory
    uint32_t c[9 * BPL / 2];
    const uint32_t * wr = (const uint32_t *) (w + (int64_t) row * w_nb1 + (int64_t) b0 * 18);
#pragma unroll
    for (int i = 0; i < 9 * BPL / 2; ++i) c[i] = wr[i];
    float dw[BPL];
    uint32_t lo[BPL][4], hi[BPL][4];
#pragma unroll
    for (int j = 0; j < BPL; ++j) {
        uint32_t q[4];
        block_of<BPL>(c, j, dw[j], q);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            lo[j][i] = q[i] & 0x0f0f0f0fu;                             // values 4i .. 4i + 3
            hi[j][i] = (q[i] >> 4) & 0x0f0f0f0fu;                      // values 16 + 4i ..
        }
    }

    for (int t = 0; t < T; ++t) {
        float part = 0.0f;
#pragma unroll
        for (int j = 0; j < BPL; ++j) {
            const int b = b0 + j;
            const uint4 * ab = (const uint4 *) (qs + (int64_t) t * K + 32 * b);
            const uint4 a0 = ab[0], a1 = ab[1];
            const uint32_t a[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
            int dot = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                dot = __builtin_amdgcn_sdot4((int) lo[j][i], (int) a[i], dot, false);
                dot = __builtin_amdgcn_sdot4((int) hi[j][i], (int) a[4 + i], dot, false);
            }
            const int sumi = dot - 8 * sy[t * nb + b];
            part += ((float) sumi * dw[j]) * dx[t * nb + b];
        }
        part = wave_sum_to_last(part);
        if (lane == 63) *(float *) (y + (int64_t) t * y_nb1 + (int64_t) row * 4) = part;
    }
}

// 1 / d as the IEEE division rounds it, for a Q8_0 block scale d >= 0 (0
// for d = 0, as quantize_row_q8_0 takes it): for d in [2^-126, 2^126) the
// v_rcp_f32 estimate and one Newton step give that quotient
// (al_mul_mat_q4_0_check_inverse counts the floats where they do not);
// zero, denormal d and the top two binades take the division.
__device__ __forceinline__ float q8_inverse(const float d) {
    if (d >= 0x1p-126f && d < 0x1p126f) {
        const float r = __builtin_amdgcn_rcpf(d);
        return __builtin_fmaf(__builtin_fmaf(-d, r, 1.0f), r, r);
    }
    return d != 0.0f ? 1.0f / d : 0.0f;
}

// Every non-negative float bit pattern up to +inf (grid-stride): counts the
// ones where q8_inverse differs from the division, bit for bit.
__global__ __launch_bounds__(256) void q8_inverse_check_kernel(unsigned long long * bad) {
    unsigned long long n = 0;
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t u = blockIdx.x * blockDim.x + threadIdx.x; u <= 0x7f800000u; u += stride) {
        const float d = __uint_as_float(u);
        const float ref = d != 0.0f ? 1.0f / d : 0.0f;
        n += __float_as_uint(q8_inverse(d)) != __float_as_uint(ref);
        if (u > 0x7f800000u - stride) break;
    }
    if (n) atomicAdd(bad, n);
}

// Eight values of a Q8_0 block (part 0..3 of it, the four parts in the four
// lanes of a quad) quantized into LDS.
__device__ __forceinline__ void quantize_part(const float4 f0, const float4 f1, const int part, int8_t * qdst,
                                              float2 * sdst) {
    const float v[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
    amax = fmaxf(amax, dpp<kQuadXor1>(amax));
    amax = fmaxf(amax, dpp<kQuadXor2>(amax));
    // d = amax / 127 as the IEEE division rounds it: amax r with r = RN(1/127)
    // and one FMA correction, which gives the correctly rounded quotient for
    // every finite non-negative float (all 2^31 checked against the division);
    // an infinite amax passes through as the division would give it
    constexpr float kR127 = 1.0f / 127.0f;
    const float q0 = amax * kR127;
    const float dq = __builtin_fmaf(__builtin_fmaf(-q0, 127.0f, amax), kR127, q0);
    const float d = amax <= 3.40282347e+38f ? dq : amax;
    const float id = q8_inverse(d);
    uint32_t words[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        uint32_t y[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            // rint(v * id), ties to even as vcvtnq: the product (|p| <= 127)
            // plus 1.5 * 2^23 rounds to the integer k + 1.5 * 2^23, whose
            // float holds k in its low bits (two's complement in the low byte);
            // the product is kept out of a fused multiply-add
            float pr = v[4 * j + k] * id;
            asm volatile("" : "+v"(pr));
            y[k] = __float_as_uint(pr + 12582912.0f);
        }
        // the four low bytes into one word (v_perm: bytes of y0, y1 | of y2, y3)
        words[j] = __builtin_amdgcn_perm(y[1], y[0], 0x0c0c0400u) | __builtin_amdgcn_perm(y[3], y[2], 0x04000c0cu);
    }
    // the eight values' sum: the signed bytes dotted with ones
    const int sum = __builtin_amdgcn_sdot4((int) words[1], 0x01010101, __builtin_amdgcn_sdot4((int) words[0], 0x01010101, 0, false), false);
    float fs = (float) sum;                                             // |sum| <= 1016: exact in f32
    fs += dpp<kQuadXor1>(fs);
    fs += dpp<kQuadXor2>(fs);
    *(uint2 *) qdst = uint2{words[0], words[1]};
    if (part == 0) *sdst = float2{(float) (_Float16) d, fs};           // the block scale as stored (f16), the sum
}

// Eight per-lane values (tokens 0..7) summed over the wavefront, scattered:
// token t's total ends in lanes 8t .. 8t + 7. Lanes exchange half of their
// values with lane ^ 32, then ^ 16 (permlane swaps), then ^ 8 (DPP row
// rotate), each time keeping the tokens of their side, then sum within
// their 8 lanes: 18 instructions instead of a wave sum per token.
__device__ __forceinline__ float wave_sum8_scatter(const float (&v)[8], const int lane) {
    float a[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {       // lanes 0..31 keep tokens k, lanes 32..63 tokens 4 + k
        const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, v[k]), __builtin_bit_cast(int, v[4 + k]),
                                                        false, false);
        a[k] = __builtin_bit_cast(float, (int) r[0]) + __builtin_bit_cast(float, (int) r[1]);
    }
    float b[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {       // lane bit 4 clear keeps a[k], set keeps a[k + 2]
        const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, a[k]), __builtin_bit_cast(int, a[k + 2]),
                                                        false, false);
        b[k] = __builtin_bit_cast(float, (int) r[0]) + __builtin_bit_cast(float, (int) r[1]);
    }
    const bool odd = (lane & 8) != 0;   // lane bit 3 set keeps b[1]
    const float keep = odd ? b[1] : b[0], send = odd ? b[0] : b[1];
    float c = keep + dpp<kRowRor8>(send);
    c += dpp<kQuadXor1>(c);
    c += dpp<kQuadXor2>(c);
    c += dpp<kRowHalfMirror>(c);
    return c;
}

// One launch for decode and verify (T <= TMAX): every workgroup issues its
// rows' weight loads, quantizes all T activation rows into LDS meanwhile
// (they are small and L2-resident after the first workgroup touches them;
// each thread issues the loads of all T tokens of its part of a block before
// using any), then runs the dot products of gemv_q4_kernel from LDS. One
// wavefront per row; with several tokens the rows' per-lane sums of all of
// them meet in one scattering wave reduction.
template <int BPL, int TMAX>
__global__ __launch_bounds__(1024) void gemv_q4_fused_kernel(const char * w, int64_t w_nb1, int N, int K,
                                                             const char * x, int64_t x_nb1, int T,
                                                             char * __restrict__ y, int64_t y_nb1) {
    extern __shared__ __align__(16) char lds[];
    prefetch_params(w_nb1, y_nb1, blockDim.x);
    const int nb = K / 32;
    int8_t * qs = (int8_t *) lds;                                       // [T][K]
    float2 * sc = (float2 *) (lds + T * K);                             // [T][nb]: (block scale, value sum)
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int b0 = lane * BPL;
    // LDS holds block b at slot (b % BPL) * 64 + b / BPL, so that the dot
    // products' reads (lane l, its j-th block) are lane-consecutive
    auto block_at = [](const int slot) { return (slot & 63) * BPL + (slot >> 6); };
    auto load_weights = [&](uint32_t (&c)[9 * BPL / 2]) {
        const int r = row < N ? row : N - 1;
        const uint32_t * wr = (const uint32_t *) (w + (int64_t) r * w_nb1 + (int64_t) b0 * 18);
#pragma unroll
        for (int i = 0; i < 9 * BPL / 2; ++i) c[i] = wr[i];           // (non-temporal loads measured slower)
    };
    uint32_t c[9 * BPL / 2];

    // (block, part) items of the activations, a uniform number of rounds per
    // thread; loads are unconditional (indices clamped in bounds) so that no
    // branch makes the compiler wait for outstanding loads early
    const int items = 4 * nb;
    const int rounds = (items + blockDim.x - 1) / blockDim.x;
    constexpr int PRE = TMAX == 1 ? 2 : 1;                             // rounds whose loads go out first
    float4 f[PRE][TMAX][2];
    auto load_item = [&](const int item, float4 (&g)[TMAX][2]) {
        const int it = item < items ? item : items - 1;
        const int b = block_at(it >> 2), part = it & 3;
#pragma unroll
        for (int t = 0; t < TMAX; ++t) {                                // rows past T re-read row T-1
            const int tr = t < T ? t : T - 1;
            const float4 * xb = (const float4 *) ((const float *) (x + (int64_t) tr * x_nb1) + 32 * b + 8 * part);
            g[t][0] = xb[0];
            g[t][1] = xb[1];
        }
    };
    auto quantize_item = [&](const int item, const float4 (&g)[TMAX][2]) {
        if (item < items) {
            const int sl = item >> 2, part = item & 3;
#pragma unroll
            for (int t = 0; t < TMAX; ++t)
                if (t < T) quantize_part(g[t][0], g[t][1], part, qs + t * K + 32 * sl + 8 * part, sc + t * nb + sl);
        }
    };
    // the first rounds' activations (L2) before the weights (HBM): the
    // quantization then waits only for the former
#pragma unroll
    for (int k = 0; k < PRE; ++k) load_item(threadIdx.x + k * blockDim.x, f[k]);
    asm volatile("" ::: "memory");                                     // keeps the issue order
    load_weights(c);
    asm volatile("" ::: "memory");
#pragma unroll
    for (int k = 0; k < PRE; ++k)
        if (k < rounds) quantize_item(threadIdx.x + k * blockDim.x, f[k]);
    for (int k = PRE; k < rounds; ++k) {
        load_item(threadIdx.x + k * blockDim.x, f[0]);
        quantize_item(threadIdx.x + k * blockDim.x, f[0]);
    }
    __syncthreads();
    if (row >= N) return;

    float dw[BPL];
    uint32_t lo[BPL][4], hi[BPL][4];
#pragma unroll
    for (int j = 0; j < BPL; ++j) {
        uint32_t q[4];
        block_of<BPL>(c, j, dw[j], q);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            lo[j][i] = q[i] & 0x0f0f0f0fu;
            hi[j][i] = (q[i] >> 4) & 0x0f0f0f0fu;
        }
    }
    // the row's dot product with token t's activations (this lane's blocks)
    auto dot_t = [&](const int t) {
        float part = 0.0f;
#pragma unroll
        for (int j = 0; j < BPL; ++j) {
            const int sl = j * 64 + lane;                                // block b0 + j
            const uint4 * ab = (const uint4 *) (qs + t * K + 32 * sl);
            const uint4 a0 = ab[0], a1 = ab[1];
            const float2 s2 = sc[t * nb + sl];
            const uint32_t a[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
            int dot = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                dot = __builtin_amdgcn_sdot4((int) lo[j][i], (int) a[i], dot, false);
                dot = __builtin_amdgcn_sdot4((int) hi[j][i], (int) a[4 + i], dot, false);
            }
            const int sumi = dot - 8 * (int) s2.y;
            part += ((float) sumi * dw[j]) * s2.x;
        }
        return part;
    };
    if constexpr (TMAX == 8) {
        float part[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) part[t] = t < T ? dot_t(t) : 0.0f;
        const float tot = wave_sum8_scatter(part, lane);
        const int t = lane >> 3;
        if ((lane & 7) == 0 && t < T) *(float *) (y + (int64_t) t * y_nb1 + (int64_t) row * 4) = tot;
    } else {
        for (int t = 0; t < T; ++t) {
            const float part = wave_sum_to_last(dot_t(t));
            if (lane == 63) *(float *) (y + (int64_t) t * y_nb1 + (int64_t) row * 4) = part;
        }
    }
}

constexpr int kFusedMaxT = 8;

size_t fused_lds_bytes(int64_t K, int64_t T) { return (size_t) (T * K + 8 * T * (K / 32)); }   // <= 160 KiB

template <int BPL, int TMAX>
int launch_fused(const al_tensor * w, const al_tensor * x, const al_tensor * y, int N, int K, int T, hipStream_t st) {
    int n_cu = 0;
    int rc = al_device_cu_count(&n_cu);
    if (rc != AL_OK) return rc;
    // one wavefront per row, all rows resident at once: the fewest workgroups
    // per CU that keep a workgroup at 16 waves or fewer
    const int per_cu = (N + 16 * n_cu - 1) / (16 * n_cu);
    const int waves = std::max(1, (N + per_cu * n_cu - 1) / (per_cu * n_cu));
    const size_t lds = fused_lds_bytes(K, T);
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute((const void *) gemv_q4_fused_kernel<BPL, TMAX>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int) lds);
        if (e != hipSuccess) return al_hip_fail(e, "mul_mat_q4_0: LDS attribute");
    }
    hipLaunchKernelGGL((gemv_q4_fused_kernel<BPL, TMAX>), dim3((unsigned) ((N + waves - 1) / waves)), dim3(64 * waves), lds, st,
                       (const char *) w->data, (int64_t) w->nb[1], N, K, (const char *) x->data, (int64_t) x->nb[1], T,
                       (char *) y->data, (int64_t) y->nb[1]);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? AL_OK : al_hip_fail(e, "mul_mat_q4_0: fused launch");
}

template <int BPL>
int launch_fused_t(const al_tensor * w, const al_tensor * x, const al_tensor * y, int N, int K, int T, hipStream_t st) {
    return T == 1 ? launch_fused<BPL, 1>(w, x, y, N, K, T, st) : launch_fused<BPL, kFusedMaxT>(w, x, y, N, K, T, st);
}

// Per-device scratch for the quantized activations, grown on demand.
struct Scratch {
    void * p = nullptr;
    size_t bytes = 0;
};
std::mutex g_mu;
Scratch g_scratch[64];

int scratch(size_t bytes, void ** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return al_hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= 64) return al_fail(AL_ERR_INVALID, "mul_mat_q4_0: device %d", dev);
    std::lock_guard<std::mutex> lk(g_mu);
    Scratch & s = g_scratch[dev];
    if (s.bytes < bytes) {
        if (s.p) {
            e = hipDeviceSynchronize();
            if (e == hipSuccess) e = hipFree(s.p);
            if (e != hipSuccess) return al_hip_fail(e, "mul_mat_q4_0: scratch free");
            s.p = nullptr;
            s.bytes = 0;
        }
        const size_t sz = std::max(bytes, (size_t) 1 << 20);
        e = hipMalloc(&s.p, sz);
        if (e != hipSuccess) return al_hip_fail(e, "mul_mat_q4_0: scratch");
        s.bytes = sz;
    }
    *out = s.p;
    return AL_OK;
}

}  // namespace

extern "C" int al_mul_mat_q4_0_check_inverse(unsigned long long * mismatches) {
    if (!mismatches) return al_fail(AL_ERR_INVALID, "al_mul_mat_q4_0_check_inverse: mismatches required");
    unsigned long long * dev = nullptr;
    hipError_t e = hipMalloc(&dev, sizeof(unsigned long long));
    if (e != hipSuccess) return al_hip_fail(e, "check_inverse: hipMalloc");
    e = hipMemset(dev, 0, sizeof(unsigned long long));
    if (e == hipSuccess) {
        hipLaunchKernelGGL(q8_inverse_check_kernel, dim3(4096), dim3(256), 0, (hipStream_t) 0, dev);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipMemcpy(mismatches, dev, sizeof(unsigned long long), hipMemcpyDeviceToHost);
    const hipError_t f = hipFree(dev);
    if (e != hipSuccess) return al_hip_fail(e, "check_inverse");
    if (f != hipSuccess) return al_hip_fail(f, "check_inverse: hipFree");
    return AL_OK;
}

extern "C" int al_mul_mat_q4_0_f32(const al_tensor * w, const al_tensor * x, const al_tensor * y, void * stream) {
    if (!w || !x || !y || !w->data || !x->data || !y->data) return al_fail(AL_ERR_INVALID, "mul_mat_q4_0: w, x and y required");
    if (w->type != AL_TYPE_Q4_0 || x->type != AL_TYPE_F32 || y->type != AL_TYPE_F32)
        return al_fail(AL_ERR_UNSUPPORTED, "mul_mat_q4_0: types %d x %d -> %d (Q4_0 x f32 -> f32 only)", w->type, x->type, y->type);
    const int64_t K = w->ne[0], N = w->ne[1], T = x->ne[1];
    if (x->ne[0] != K || y->ne[0] != N || y->ne[1] != T || x->ne[2] != 1 || x->ne[3] != 1 || w->ne[2] != 1 || w->ne[3] != 1)
        return al_fail(AL_ERR_INVALID, "mul_mat_q4_0: shapes w [%lld, %lld], x [%lld, %lld], y [%lld, %lld]",
                       (long long) K, (long long) N, (long long) x->ne[0], (long long) T, (long long) y->ne[0], (long long) y->ne[1]);
    if (K % 4096 != 0 || K > 16384) return al_fail(AL_ERR_UNSUPPORTED, "mul_mat_q4_0: K %lld (4096, 8192, 12288 or 16384)", (long long) K);
    if (T < 1 || T > kMaxT) return al_fail(AL_ERR_UNSUPPORTED, "mul_mat_q4_0: %lld tokens (1 .. %d)", (long long) T, kMaxT);
    if (N < 1 || N > (int64_t) 65535 * 4) return al_fail(AL_ERR_INVALID, "mul_mat_q4_0: N %lld", (long long) N);
    const int64_t nb = K / 32;
    if ((int64_t) w->nb[1] != nb * 18 || x->nb[0] != 4 || y->nb[0] != 4 || ((uintptr_t) w->data & 3) || ((uintptr_t) x->data & 15) ||
        (x->nb[1] & 15) || x->nb[1] < (uint64_t) K * 4 || y->nb[1] < (uint64_t) N * 4 || ((uintptr_t) y->data & 3))
        return al_fail(AL_ERR_INVALID, "mul_mat_q4_0: w rows must be contiguous blocks (nb1 = K/32*18, 4-byte aligned), x rows 16-byte aligned, rows not overlapping");
    hipStream_t st = (hipStream_t) stream;
    if (T <= kFusedMaxT) {
        switch (nb / 64) {
            case 2: return launch_fused_t<2>(w, x, y, (int) N, (int) K, (int) T, st);
            case 4: return launch_fused_t<4>(w, x, y, (int) N, (int) K, (int) T, st);
            case 6: return launch_fused_t<6>(w, x, y, (int) N, (int) K, (int) T, st);
            case 8: return launch_fused_t<8>(w, x, y, (int) N, (int) K, (int) T, st);
            default: return al_fail(AL_ERR_UNSUPPORTED, "mul_mat_q4_0: K %lld", (long long) K);
        }
    }
    const size_t qs_bytes = (size_t) (T * K), f_bytes = (size_t) (T * nb) * 4;
    void * s = nullptr;
    int rc = scratch(qs_bytes + 2 * f_bytes, &s);
    if (rc != AL_OK) return rc;
    int8_t * qs = (int8_t *) s;
    float * dx = (float *) ((char *) s + qs_bytes);
    int * sy = (int *) ((char *) s + qs_bytes + f_bytes);
    hipLaunchKernelGGL(quantize_q8_kernel, dim3((unsigned) ((T * nb + 255) / 256)), dim3(256), 0, st,
                       (const char *) x->data, (int64_t) x->nb[1], (int) K, (int) T, qs, dx, sy);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return al_hip_fail(e, "mul_mat_q4_0: quantize launch");
    const dim3 grid((unsigned) ((N + 3) / 4));
    switch (nb / 64) {
        case 2: hipLaunchKernelGGL(gemv_q4_kernel<2>, grid, dim3(256), 0, st, (const char *) w->data, (int64_t) w->nb[1], (int) N, (int) K, qs, dx, sy, (int) T, (char *) y->data, (int64_t) y->nb[1]); break;
        case 4: hipLaunchKernelGGL(gemv_q4_kernel<4>, grid, dim3(256), 0, st, (const char *) w->data, (int64_t) w->nb[1], (int) N, (int) K, qs, dx, sy, (int) T, (char *) y->data, (int64_t) y->nb[1]); break;
        case 6: hipLaunchKernelGGL(gemv_q4_kernel<6>, grid, dim3(256), 0, st, (const char *) w->data, (int64_t) w->nb[1], (int) N, (int) K, qs, dx, sy, (int) T, (char *) y->data, (int64_t) y->nb[1]); break;
        case 8: hipLaunchKernelGGL(gemv_q4_kernel<8>, grid, dim3(256), 0, st, (const char *) w->data, (int64_t) w->nb[1], (int) N, (int) K, qs, dx, sy, (int) T, (char *) y->data, (int64_t) y->nb[1]); break;
        default: return al_fail(AL_ERR_UNSUPPORTED, "mul_mat_q4_0: K %lld", (long long) K);
    }
    e = hipGetLastError();
    return e == hipSuccess ? AL_OK : al_hip_fail(e, "mul_mat_q4_0: launch");
}
