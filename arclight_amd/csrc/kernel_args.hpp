// Kernel-argument access at kernel entry (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace kernel_args {

// XOR of one dword of every 64 bytes of an argument block and of its last
// dword (a scalar argument: itself).
template <typename P>
__device__ __forceinline__ uint32_t sample(const P & p) {
    if constexpr (std::is_arithmetic_v<P>) {
        return (uint32_t) p;
    } else {
        static_assert(sizeof(P) % 4 == 0, "dword-sized parameter block");
        constexpr int kWords = (int) (sizeof(P) / 4);
        const uint32_t * w = reinterpret_cast<const uint32_t *>(&p);
        uint32_t x = w[kWords - 1];
#pragma unroll
        for (int i = 0; i < kWords - 1; i += 16) x ^= w[i];
        return x;
    }
}

}  // namespace kernel_args

// Loads every 64-byte line of the given kernel arguments at kernel entry and
// waits for them once: fields are loaded through the scalar cache when first
// used, and a line first used deep in the set-up would otherwise cost the
// wave one more miss in series.
template <typename... P>
__device__ __forceinline__ void prefetch_params(const P &... p) {
    const uint32_t x = (kernel_args::sample(p) ^ ...);
    asm volatile("" ::"s"(x));
}
