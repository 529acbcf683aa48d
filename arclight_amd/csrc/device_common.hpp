// Device-side building blocks shared by the gfx950 attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define AL_INF __builtin_inff()

// D[16x16] += A[16x32] * B[32x16], f16 inputs, f32 accumulation (gfx950).
// Lane l = 16*g + n holds A row n, B column n, k-slots 8g..8g+7 of each,
// and D rows 4g..4g+3 of column n.
__device__ __forceinline__ floatx4 mfma_16x16x32(half8 a, half8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// e^x through the hardware exp2 (v_exp_f32).
__device__ __forceinline__ float exp_fast(float x) {
    return __builtin_amdgcn_exp2f(x * 1.44269504088896341f);
}

__device__ __forceinline__ half8 as_half8(u32x4 v) { return __builtin_bit_cast(half8, v); }
__device__ __forceinline__ u32x4 as_u32x4(uint4 v) { u32x4 r = {v.x, v.y, v.z, v.w}; return r; }

// 8 f32 -> 8 f16, IEEE round-to-nearest-even (v_cvt_f16_f32 in the default mode).
__device__ __forceinline__ half8 to_half8(float4 a, float4 b) {
    half8 h;
    h[0] = (_Float16) a.x; h[1] = (_Float16) a.y; h[2] = (_Float16) a.z; h[3] = (_Float16) a.w;
    h[4] = (_Float16) b.x; h[5] = (_Float16) b.y; h[6] = (_Float16) b.z; h[7] = (_Float16) b.w;
    return h;
}

__device__ __forceinline__ float f16_bits_to_float(uint16_t b) {
    return (float) __builtin_bit_cast(_Float16, b);
}

// max / sum over the 4 lanes {n, n+16, n+32, n+48} that share column n.
__device__ __forceinline__ float colmax4(float x) {
    x = fmaxf(x, __shfl_xor(x, 16));
    x = fmaxf(x, __shfl_xor(x, 32));
    return x;
}
__device__ __forceinline__ float colsum4(float x) {
    x += __shfl_xor(x, 16);
    x += __shfl_xor(x, 32);
    return x;
}

// Hand-off of merge records between workgroups of one launch. Records are
// written and read with agent-scope (device-coherent) relaxed atomic stores
// and loads, which gfx950 performs at the device coherence point (stores
// write through the writer's L2, loads do not return stale lines of the
// reader's L2), so no L2-wide writeback or invalidate is needed. A writer
// waits for its stores to complete (s_waitcnt) before a barrier and the
// relaxed arrival-counter update; the workgroup that sees the final count
// reads the records only after that update returned. This is the ordering
// the compiler itself relies on for agent-scope atomics (a completed
// agent-scope store is visible to agent-scope loads of every CU).
__device__ __forceinline__ void st_agent(float * p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float * p) {
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned add_agent(unsigned * p, unsigned v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent_u32(unsigned * p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned ld_agent_u32(const unsigned * p) {
    return __hip_atomic_load(const_cast<unsigned *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// A wave-uniform read of memory that no kernel running alongside writes,
// as a scalar load (lgkm-counted): through the constant address space, so
// that it is scalar whatever else the kernel does to memory (an asm
// statement with side effects before it keeps the compiler from proving
// that for a global pointer, and it would then issue a vector load).
template <typename T>
__device__ __forceinline__ T ld_uniform(const T * ptr) {
    return *(const __attribute__((address_space(4))) T *) ptr;
}

// Polls of a merging workgroup for the split flags of its launch before it
// gives up and reports it (each poll a round trip to the coherence point
// after a short sleep: about a second in all).
constexpr int kFlagPollLimit = 1 << 20;
// Keeps the compiler from moving this wave's memory accesses across it and
// waits until all of them have completed (s_waitcnt 0).
__device__ __forceinline__ void complete_wave_memops() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_waitcnt(0);
}
__device__ __forceinline__ void order_after_counter() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup"); }
