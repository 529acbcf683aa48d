/*
 * arclight_kv.h - C ABI of the HBM-resident f16 KV cache ("KV ring") that
 * feeds the flash-attention operator, and of its cell bookkeeping.
 *
 * The reference keeps, per layer, f16 K and V tensors [Hkv*128, kv_size,
 * n_stream] in a host bump buffer (llm_kv_cache ctor, nnml/src/cgraph.cpp:
 * 915-986) and tracks which cells hold which (sequence, position) on the
 * host (llm_kv_cells, nnml/include/cgraph.h:612-960). Each step it finds
 * cells for the batch's tokens (prepare / find_slot / apply_ubatch,
 * cgraph.cpp:1263-1466), writes the new K/V rows there (cpy_k / cpy_v ->
 * set_rows, cgraph.cpp:1114-1180) and fills the attention mask on the host
 * (set_inputs_attn_mask, cgraph.cpp:1224-1261).
 *
 * Here the K/V tensors live in HBM (hipMalloc, one allocation per layer and
 * per K / V, the reference's layout unchanged), the cell bookkeeping is the
 * same algorithm on the host, and the mask is built on the device from a
 * device copy of the cell state that is updated incrementally (only cells
 * that changed are sent). When the mask is exactly the length + causal rule
 * the flash-attention operator takes implicitly, al_kv_cells_implicit says
 * so and no mask is needed at all.
 *
 * Error convention as arclight_fattn.h (0 = AL_OK, negative status,
 * al_last_error()).
 */
#ifndef ARCLIGHT_KV_H
#define ARCLIGHT_KV_H

#include <stddef.h>
#include <stdint.h>

#include "arclight_fattn.h"

#ifdef __cplusplus
extern "C" {
#endif

/*
 * The tokens of one micro-batch (llm_ubatch): position and sequence set of
 * each token. seq_mask[i] has bit s set when token i belongs to sequence s
 * (s < 64, LLM_MAX_SEQ); its lowest set bit is the token's primary sequence
 * (ubatch->seq_id[i][0]), which picks the stream and the mask row's
 * sequence. With more than one stream, tokens come grouped by sequence in
 * equal blocks, as the reference requires (cgraph.cpp:1332-1335).
 */
typedef struct al_ubatch {
    int32_t          n_tokens;
    const int32_t *  pos;        /* host [n_tokens] */
    const uint64_t * seq_mask;   /* host [n_tokens] */
} al_ubatch;

typedef struct al_kv_cells al_kv_cells;

/* Bookkeeping of kv_size cells per stream (n_stream = 1 when unified, else
 * n_seq_max), n_kv padded to n_pad (kv_size % n_pad == 0). Host only: needs
 * no GPU until al_kv_cells_mask_device. */
int al_kv_cells_create(uint32_t kv_size, uint32_t n_seq_max, uint32_t n_pad, int32_t unified, al_kv_cells ** out);
int al_kv_cells_destroy(al_kv_cells * c);
/* Empties every cell (llm_kv_cache::clear). */
int al_kv_cells_clear(al_kv_cells * c);

/*
 * Finds cells for the ubatch and occupies them (find_slot with the
 * non-contiguous search, then apply_ubatch: cgraph.cpp:1327-1466). Writes
 * the cache row of each token, stream * kv_size + cell, to rows[n_tokens]
 * (the K/V set_rows indices, cgraph.cpp:1182-1222), the number of cells
 * attention must look at to *n_kv (get_n_kv, cgraph.cpp:1472-1479) and,
 * when not NULL, the ubatch's streams s0..s0+ns-1 (slot_info s0 / s1,
 * cgraph.cpp:1340-1345) to *s0 and *ns. AL_ERR_INVALID (nothing changed)
 * when the ubatch does not fit.
 */
int al_kv_cells_place(al_kv_cells * c, const al_ubatch * ub, int64_t * rows, uint32_t * n_kv, uint32_t * s0,
                      uint32_t * ns);

/* Removes sequence seq_id (-1: any) from positions [p0, p1) (p < 0: open),
 * llm_kv_cache::seq_rm (cgraph.cpp:1535-1590). */
int al_kv_cells_seq_rm(al_kv_cells * c, int32_t seq_id, int32_t p0, int32_t p1);

/* Cell state for inspection: pos[stream * kv_size + i] (-1 = empty) and
 * the sequence bit mask of each cell; NULL outputs are skipped. */
int al_kv_cells_state(const al_kv_cells * c, int32_t * pos, uint64_t * seq_mask);

/*
 * The attention mask of the ubatch, f16 0 / -inf, laid out as the graph
 * hands it to the operator: [n_kv, PAD(n_tokens / n_stream_ub, 64), 1,
 * n_stream_ub] (set_inputs_attn_mask + the f32 -> f16 cast, cgraph.cpp:
 * 1224-1261). The host variant writes host memory; the device variant
 * builds it on the GPU into mask->data (mask->ne / nb must describe that
 * layout, contiguous), sending only the cell state changed since its last
 * call. n_stream_ub: 1 when unified, else the ubatch's sequence count.
 */
int al_kv_cells_mask_host(const al_kv_cells * c, const al_ubatch * ub, uint32_t n_kv, uint32_t n_stream_ub,
                          uint16_t * mask);
int al_kv_cells_mask_device(al_kv_cells * c, const al_ubatch * ub, uint32_t n_kv, uint32_t n_stream_ub,
                            const al_tensor * mask, void * stream);

/*
 * Whether the ubatch's mask over n_kv cells is exactly the implicit rule of
 * al_fattn_args (cell j visible to token t iff j < kv_len and
 * j <= causal_pos0 + t): one stream, one sequence whose cells
 * 0..kv_len-1 hold positions 0..kv_len-1, consecutive token positions
 * starting at causal_pos0, no other cell of the sequence visible. Returns
 * 1 and sets *kv_len, *causal_pos0 when it is, 0 when not.
 */
int al_kv_cells_implicit(const al_kv_cells * c, const al_ubatch * ub, uint32_t n_kv, int64_t * kv_len,
                         int64_t * causal_pos0);

typedef struct al_kv_ring al_kv_ring;

typedef struct al_kv_ring_params {
    uint32_t n_layer;
    uint32_t kv_size;      /* cells per stream, multiple of n_pad */
    uint32_t n_seq_max;
    uint32_t n_pad;        /* 256 with flash attention (apps/al-gen.cpp:114) */
    uint32_t n_head_kv;
    uint32_t head_dim;     /* 128 */
    int32_t  unified;      /* 1: one stream shared by all sequences */
} al_kv_ring_params;

/* Allocates every layer's K and V, f16 [head_dim*n_head_kv, kv_size,
 * n_stream] (cgraph.cpp:969-970), zero-filled, and the cell bookkeeping. */
int al_kv_ring_create(const al_kv_ring_params * params, al_kv_ring ** out);
int al_kv_ring_destroy(al_kv_ring * r);
/* The ring's cell bookkeeping (owned by the ring). */
al_kv_cells * al_kv_ring_cells(al_kv_ring * r);

/* Attention views of layer il over the first n_kv cells of streams
 * s0..s0+ns-1: ne = [head_dim, n_kv, n_head_kv, ns], nb = [2,
 * n_head_kv*head_dim*2, head_dim*2, kv_size*n_head_kv*head_dim*2], data at
 * stream s0 (llm_kv_cache::get_k / get_v with FA, cgraph.cpp:1057-1112,
 * after the graph's permute (0, 2, 1, 3)). */
int al_kv_ring_view_k(const al_kv_ring * r, uint32_t il, uint32_t n_kv, uint32_t s0, uint32_t ns, al_tensor * k);
int al_kv_ring_view_v(const al_kv_ring * r, uint32_t il, uint32_t n_kv, uint32_t s0, uint32_t ns, al_tensor * v);

/* Writes the ubatch's K and V rows of layer il, f32 [head_dim*n_head_kv,
 * n_tokens] (token rows, nb[1] their stride), at cache rows rows->data
 * (device i64 [n_tokens], from al_kv_cells_place): cpy_k / cpy_v
 * (cgraph.cpp:1114-1180) through al_set_rows_f32_f16. */
int al_kv_ring_write(al_kv_ring * r, uint32_t il, const al_tensor * k_cur, const al_tensor * v_cur,
                     const al_tensor * rows, void * stream);

#ifdef __cplusplus
}
#endif

#endif /* ARCLIGHT_KV_H */
