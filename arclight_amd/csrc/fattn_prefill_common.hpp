// Pieces of the prefill kernel (fattn_prefill.hip), whose RG = 4 (128-row
// tiles) and RG = 2 (64-row tiles, two cell splits per workgroup)
// instantiations share them.
#pragma once

#include "fattn_tile.hpp"

namespace fattn_prefill {

using namespace fattn;

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float2v __attribute__((ext_vector_type(2)));

constexpr int kWaves = 4;                        // one per SIMD, 32 rows each
constexpr int kLds = 160 * 1024;                 // the rings of all splits (all of a CU's LDS)
constexpr int kMaxPrefillSplit = kFattnPrefillMaxSplit;
constexpr float kLog2e = 1.44269504088896341f;

__device__ __forceinline__ floatx16 mfma32(half8 a, half8 b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Values of lanes l % 32 and l % 32 + 32 (the two lanes holding one row).
__device__ __forceinline__ float pair_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, x), __builtin_bit_cast(int, x), false, false);
    return fmaxf(__builtin_bit_cast(float, (int) r[0]), __builtin_bit_cast(float, (int) r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, x), __builtin_bit_cast(int, x), false, false);
    return __builtin_bit_cast(float, (int) r[0]) + __builtin_bit_cast(float, (int) r[1]);
}

// The lane's index within the wave read anew by v_mbcnt behind an opaque
// asm statement: code after a long loop derives its lane-dependent offsets
// from it instead of holding them in registers across the loop.
__device__ __forceinline__ int lane_id_fresh() {
    int l;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
    return l;
}

// tanh(x / c2 * 2 log2 e) = 1 - 2 / (2^(c2 x) + 1), with the hardware exp2
// and reciprocal: an absolute error of a few 1e-7 (and -1 / +1 exactly where
// 2^(c2 x) underflows to 0 or overflows to inf) in four instructions and no
// extra registers, so that the logit softcap keeps the slot-scheduled loop
// out of scratch. c2 = 2 log2(e) times the factor applied before tanh.
__device__ __forceinline__ float tanh_exp2(float x, float c2) {
    return 1.0f - 2.0f * __builtin_amdgcn_rcpf(__builtin_amdgcn_exp2f(x * c2) + 1.0f);
}

// Waits until at most N LDS-DMA / vector memory instructions of this wave are
// outstanding.
template <int N>
__device__ __forceinline__ void wait_vm() {
    mem_barrier();
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(N));
    mem_barrier();
}

}  // namespace fattn_prefill
