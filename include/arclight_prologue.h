/*
 * arclight_prologue.h - C ABI of the producers of the attention operands in
 * ArcLight's Qwen3 layer (models/qwen3.cpp:211-224): per-head RMSNorm of Q
 * and K, the multiply by the ATTN_Q_NORM / ATTN_K_NORM weights, and the
 * rotary position embedding, in one pass over f32 rows, with K optionally
 * written straight into the f16 KV cache (the cpy_k set_rows that follows,
 * nnml/src/cgraph.cpp:1114-1146).
 *
 * Replaces the node chain rms_norm -> mul -> rope_ext (-> set_rows):
 *   nnml_compute_forward_rms_norm_f32   nnml/src/ops/ops.cpp:680-726
 *   nnml_compute_forward_mul (f32)      nnml/src/ops/ops.cpp:1248-1250
 *   nnml_compute_forward_rope_f32       nnml/src/ops/ops.cpp:871-962
 *     (rope_yarn, cache init, corr dims: ops.cpp:728-777)
 *   nnml_compute_forward_set_rows_f32   nnml/src/ops/ops.cpp:135-181
 *
 * Error convention as arclight_fattn.h.
 */
#ifndef ARCLIGHT_PROLOGUE_H
#define ARCLIGHT_PROLOGUE_H

#include <stdint.h>

#include "arclight_fattn.h"

#ifdef __cplusplus
extern "C" {
#endif

#define AL_ROPE_NORMAL 0     /* pairs (2i, 2i + 1) */
#define AL_ROPE_NEOX   2     /* pairs (i, i + n_dims / 2), NNML_ROPE_TYPE_NEOX (tensor.h:28) */

/* The rope_ext op_params (nnml/src/tensor.cpp:1026-1032). Qwen3: NEOX,
 * n_dims 128, freq_base 1e6, freq_scale 1, ext_factor 0, attn_factor 1,
 * beta_fast 32, beta_slow 1 (models/qwen3.cpp:49-55). */
typedef struct al_rope_params {
    int32_t n_dims;       /* rotated dims; must equal the head dim (128) */
    int32_t mode;         /* AL_ROPE_NEOX or AL_ROPE_NORMAL */
    int32_t n_ctx_orig;
    float   freq_base;
    float   freq_scale;
    float   ext_factor;   /* YaRN ramp when != 0 */
    float   attn_factor;
    float   beta_fast;
    float   beta_slow;
} al_rope_params;

/*
 * y = rope(rms_norm(x) * w) for every (head, token) row of 128 floats.
 *   x     f32 ne = [128, H, T, 1], nb0 = 4            (Qcur / Kcur)
 *   w     f32 [128], or NULL for no weight
 *   pos   i32 [T] (device), the token positions       (inp_pos)
 *   eps   the RMSNorm epsilon (hparams f_norm_rms_eps)
 *   rope  NULL for no rotation
 * Output, one of:
 *   rows == NULL: y f32 ne = [128, H, T, 1], nb0 = 4
 *   rows != NULL: y is the f16 K cache viewed as rows of H*128 halves,
 *                 ne = [128*H, n_rows], and token t's heads go to row
 *                 rows[t] (i64 or i32 [T], device), rounded to f16 (RNE):
 *                 the fused cpy_k. Out-of-range rows are not written and are
 *                 reported by al_device_errors, as set_rows.
 * Enqueues on `stream`.
 */
int al_rms_norm_rope_f32(const al_tensor * x, const al_tensor * w, const al_tensor * pos, float eps,
                         const al_rope_params * rope, const al_tensor * y, const al_tensor * rows, void * stream);

/*
 * The three attention inputs of one layer in one launch: what
 * al_rms_norm_rope_f32 does for Q (into q_out) and for K (into the K cache
 * at rows[t]), and what al_set_rows_f32_f16 does for V (into the V cache at
 * rows[t]), with the same results bit for bit. It replaces the node run of
 * models/qwen3.cpp:211-227 up to attention (rms_norm -> mul -> rope_ext for
 * Q and K, then cpy_k / cpy_v, nnml/src/cgraph.cpp:485-488) with one kernel,
 * which saves two launch latencies per layer in a decode step. It has no
 * single counterpart in the reference, which runs those nodes one by one.
 * Operands as the two calls it replaces; v is f32 [n, T, 1, 1] with rows
 * contiguous and one row per token of q. Out-of-range rows are not written
 * and are reported by al_device_errors.
 */
typedef struct al_attn_inputs_args {
    al_tensor q;        /* f32 [128, Hq, T, 1]   (Qcur) */
    al_tensor q_w;      /* f32 [128] (ATTN_Q_NORM), or data NULL for none */
    al_tensor k;        /* f32 [128, Hkv, T, 1]  (Kcur) */
    al_tensor k_w;      /* f32 [128] (ATTN_K_NORM), or data NULL for none */
    al_tensor v;        /* f32 [n, T]            (Vcur rows) */
    al_tensor pos;      /* i32 [T], device       (inp_pos) */
    al_tensor rows;     /* i64 / i32 [T], device: the cache row of each token (k_idxs / v_idxs) */
    al_tensor q_out;    /* f32 [128, Hq, T] */
    al_tensor k_cache;  /* f16 [128 * Hkv, n_rows] */
    al_tensor v_cache;  /* f16 [n, n_rows] */
    float eps;          /* RMSNorm epsilon */
    const al_rope_params * rope;   /* NULL for no rotation */
} al_attn_inputs_args;

int al_attn_inputs_f32(const al_attn_inputs_args * a, void * stream);

/*
 * al_fattn_f16 with the layer's attention inputs folded into the decode
 * kernel: the same results, bit for bit, as al_attn_inputs_f32(in,
 * a->stream) followed by al_fattn_f16(a), in one launch (q_out and the K / V
 * cache rows are written as that pair writes them). No single counterpart
 * in the reference, which runs rms_norm -> mul -> rope_ext for Q and K,
 * cpy_k / cpy_v and flash_attn_ext as separate nodes
 * (models/qwen3.cpp:211-227, nnml/src/cgraph.cpp:485-488); it takes the
 * inputs' launch out of a decode step. a->q must view in->q_out (the query
 * rows the inputs produce), a->k and a->v the caches in->k_cache and
 * in->v_cache (cell c = cache row c, heads of 128 halves). A call that does
 * not run on the decode kernel (more than 16 query rows per kv head, a mask
 * tensor, several streams), has more than one token, or whose operands the fused
 * prologue cannot move (16-byte aligned rows and indices) returns
 * AL_ERR_UNSUPPORTED before anything is enqueued; the pair of calls then
 * does the same work.
 */
int al_fattn_f16_with_inputs(const al_attn_inputs_args * in, const al_fattn_args * a);

#ifdef __cplusplus
}
#endif

#endif /* ARCLIGHT_PROLOGUE_H */
