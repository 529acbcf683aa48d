/* The Q8_0 activation scale d = amax / 127 as the WO kernel computes it
 * (arclight_amd/csrc/matmul_q4.hip, quantize_part): q0 = amax * r with
 * r = RN(1/127), then d = fma(fma(-q0, 127, amax), r, q0). Checks that this
 * equals the IEEE single-precision quotient amax / 127 (the reference's
 * quantize_row_q8_0, nnml/src/ops/arm/arm.cpp:1819-1848) bit for bit for
 * every float bit pattern in [lo, hi) that is finite and non-negative;
 * prints the number of mismatches. Usage: q8_scale_division lo hi (hex). */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

int main(int argc, char ** argv) {
    if (argc != 3) return 2;
    const uint64_t lo = strtoull(argv[1], NULL, 16), hi = strtoull(argv[2], NULL, 16);
    const float r = 1.0f / 127.0f;
    uint64_t bad = 0;
    for (uint64_t u = lo; u < hi && u < 0x7f800000u; ++u) {
        const float x = from_bits((uint32_t) u);
        const volatile float q = x / 127.0f;
        const float q0 = x * r;
        const float d = fmaf(fmaf(-q0, 127.0f, x), r, q0);
        if (to_bits(d) != to_bits(q)) {
            if (bad < 4) printf("x=%a: division %a, fma form %a\n", x, q, d);
            ++bad;
        }
    }
    printf("%llu\n", (unsigned long long) bad);
    return 0;
}
