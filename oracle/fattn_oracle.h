/*
 * fattn_oracle.h - CPU oracle for the flash-attention path (TEST
 * INFRASTRUCTURE ONLY).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the reference results or the CPU baseline. The
 * product path (arclight_amd, libarclight_fattn.so) never calls it.
 *
 * Three restatements of ArcLight's nnml_compute_forward_flash_attn_ext_f16
 * (nnml/src/ops/arm/arm.cpp:2196-2433):
 *   O2  orc_fattn_o2  line-for-line control flow of the reference (row split
 *                     over threads, online softmax with the s > M branch,
 *                     mask skip, sinks, ALiBi, softcap, permuted store) with
 *                     Q rounded to f16 (common.cpp:19-24) and f32 accumulation
 *                     of Q.K and V. THE PARITY ORACLE.
 *   O1  orc_fattn_o1  fp64 brute force: two-pass softmax over visible cells.
 *   O3  orc_fattn_o3  ARM-faithful diagnostic: f16 FMA dot lanes
 *                     (arm.cpp:89-124, 358-376) and an f16 V accumulator
 *                     (arm.cpp:1503-1551, 1655-1755). Not a parity target.
 * All three take the product's al_fattn_args with HOST pointers, including
 * the kv_len / causal_pos0 masking rules documented in arclight_fattn.h.
 */
#ifndef ARCLIGHT_FATTN_ORACLE_H
#define ARCLIGHT_FATTN_ORACLE_H

#include <stdint.h>
#include "../include/arclight_fattn.h"
#include "../include/arclight_prologue.h"

#ifdef __cplusplus
extern "C" {
#endif

/* IEEE binary16 conversions, round-to-nearest-even
 * (restating nnml/include/ops.h:276-323). */
uint16_t orc_f32_to_f16(float f);
float    orc_f16_to_f32(uint16_t h);
void     orc_f32_to_f16_n(const float * x, uint16_t * y, int64_t n);
void     orc_f16_to_f32_n(const uint16_t * x, float * y, int64_t n);

/* Attention oracles; return 0 or a negative al status. n_threads >= 1. */
int orc_fattn_o2(const al_fattn_args * a, int n_threads);
/* O2 with thread i pinned to logical CPU cpus[i] (the timed CPU baseline). */
int orc_fattn_o2_pinned(const al_fattn_args * a, int n_threads, const int * cpus);
int orc_fattn_o1(const al_fattn_args * a, int n_threads);
int orc_fattn_o3(const al_fattn_args * a, int n_threads);

/* set_rows f32 -> f16 (nnml/src/ops/ops.cpp:135-181). */
int orc_set_rows_f32_f16(const al_tensor * dst, const al_tensor * src,
                         const al_tensor * idx);

/* The attention-operand producers of the Qwen3 layer, host memory:
 * y = rope(rms_norm(x) * w) over rows of D floats; x, y f32 [T][H][D]
 * contiguous, w [D] or NULL, pos [T], rope NULL for no rotation. Restates
 * nnml_compute_forward_rms_norm_f32 (ops.cpp:680-726), the f32 mul, and
 * nnml_compute_forward_rope_f32 (ops.cpp:871-962) with rope_yarn, the
 * rotation cache and the YaRN correction dims (ops.cpp:728-777). */
int orc_rms_norm_rope_f32(const float * x, const float * w, const int32_t * pos, int64_t T, int64_t H, int64_t D,
                          float eps, const al_rope_params * rope, float * y);

/* Q4_0 / Q8_0 blocks (nnml/include/nnml.h:646-650, 695-699). */
typedef struct { uint16_t d; uint8_t qs[16]; } orc_block_q4_0;
typedef struct { uint16_t d; int8_t qs[32]; } orc_block_q8_0;

/* quantize_row_q8_0 as the NEON build runs it (arm.cpp:1819-1848): per
 * block of 32, d = amax / 127, q = round-to-nearest-even(x / d). */
void orc_quantize_row_q8_0(const float * x, orc_block_q8_0 * y, int64_t k);
/* nnml_vec_dot_q4_0_q8_0, scalar path (arm.cpp:401-...): sum over blocks of
 * sumi * d_x * d_y in float, blocks in order. */
float orc_vec_dot_q4_0_q8_0(int64_t n, const orc_block_q4_0 * x, const orc_block_q8_0 * y);
/* mul_mat with Q4_0 weights w [N][K/32 blocks] and f32 activations
 * x [T][K]: y [T][N] (forward_mul_mat_generic, common.cpp:120-...). */
int orc_mul_mat_q4_0_f32(const void * w, int64_t K, int64_t N, const float * x, int64_t T, float * y);

#ifdef __cplusplus
}
#endif

#endif
