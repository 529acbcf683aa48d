/*
 * arclight_matmul.h - C ABI of the attention output projection (WO) of
 * ArcLight's Qwen3 layer: the consumer of the attention output
 * (build_attn -> build_lora_mm(WO), nnml/src/cgraph.cpp:294,497-500) with
 * the model's Q4_0 weights.
 *
 * Replaces nnml_compute_forward_mul_mat (nnml/src/ops/ops.cpp:1252-1274)
 * for src0 Q4_0 and src1 f32 on the generic path (forward_mul_mat_generic,
 * nnml/src/ops/arm/common.cpp:120-...): the activations are quantized to
 * Q8_0 blocks (quantize_row_q8_0, arm.cpp:1819-1848: d = amax / 127, values
 * rounded to nearest even) and each output is the block-wise integer dot
 * product scaled by both block scales (nnml_vec_dot_q4_0_q8_0,
 * arm.cpp:401-...).
 *
 * Error convention as arclight_fattn.h.
 */
#ifndef ARCLIGHT_MATMUL_H
#define ARCLIGHT_MATMUL_H

#include <stdint.h>

#include "arclight_fattn.h"

#ifdef __cplusplus
extern "C" {
#endif

#define AL_TYPE_Q4_0 2       /* NNML_TYPE_Q4_0: blocks of 32 weights, f16 scale + 16 bytes of nibbles */

/*
 * y = W x with Q4_0 weights.
 *   w  Q4_0 ne = [K, N]: N rows of K / 32 blocks of 18 bytes (nnml.h:646-650),
 *      rows contiguous (nb1 = K / 32 * 18)
 *   x  f32 ne = [K, T], nb0 = 4
 *   y  f32 ne = [N, T], nb0 = 4
 * K must be 4096, 8192, 12288 or 16384 (the Qwen3 output projections: 4096
 * for 4B, 8192 for 32B) and T at most 64; x rows 16-byte aligned. Uses library-owned device scratch for the quantized
 * activations. Enqueues on `stream`.
 */
int al_mul_mat_q4_0_f32(const al_tensor * w, const al_tensor * x, const al_tensor * y, void * stream);

/*
 * No counterpart in the reference: a self-check of the device for callers
 * that want to confirm its arithmetic. The Q8_0 quantization above takes
 * 1 / d of a block scale d in [2^-126, 2^126) from the hardware reciprocal
 * estimate and one Newton step instead of a division; this counts, over
 * every non-negative float up to +inf, the values where that differs from
 * the IEEE quotient (0 on gfx950). Synchronous, on the default stream.
 */
int al_mul_mat_q4_0_check_inverse(unsigned long long * mismatches);

#ifdef __cplusplus
}
#endif

#endif /* ARCLIGHT_MATMUL_H */
