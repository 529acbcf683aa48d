/*
 * arclight_fattn.h - C ABI of the MI355X (gfx950) flash-attention operator.
 *
 * This is the drop-in boundary for ArcLight's NNML_OP_FLASH_ATTN_EXT. The
 * reference executes that op as
 *     void nnml_compute_forward_flash_attn_ext(nnml_tensor * node,
 *                                              const nnml_compute_state * params)
 * (nnml/include/ops.h:433, nnml/src/ops/ops.cpp:1432-1445), which reads its
 * operands as node->get_src_tensor(0..4) = q, k, v, mask, sinks
 * (nnml/src/ops/arm/arm.cpp:2197-2202, nnml/src/tensor.cpp:1314-1318,1331),
 * its parameters from op_params f32[0..2] = {scale, max_bias, logit_softcap}
 * and i32[3] = prec (tensor.cpp:1311, 1334-1338), and writes node->data.
 *
 * Here every operand travels as an al_tensor: a data pointer plus nnml's
 * ne[4] element counts and nb[4] byte strides, with nnml's type numbering.
 * All data pointers are DEVICE pointers (HBM). No pointer is retained after
 * a call returns; the caller owns every buffer.
 *
 * Operand layouts are the ones the Qwen3 graph hands to the op
 * (nnml/src/cgraph.cpp:245-294, 1057-1112):
 *   q     f32  ne = [D,  T,    Hq,  B ]   (token, head, stream strides nb1..nb3)
 *   k     f16  ne = [D,  n_kv, Hkv, B ]   (cell-major cache view: nb1 = Hkv*D*2)
 *   v     f16  ne = [D,  n_kv, Hkv, B ]
 *   mask  f16  ne = [n_kv, >= PAD(T,64), m2, m3]   (0 / -inf, optional)
 *   sinks f32  ne = [Hq]                            (optional)
 *   dst   f32  ne = [D,  Hq,   T,   B ]   row of (i3, i1, i2) at
 *              (i3*T*Hq + i1*Hq + i2) * nb1           (arm.cpp:2431)
 *
 * Error convention: every entry point returns AL_OK (0) or a negative
 * status; al_last_error() gives the message of the calling thread's last
 * failure. The reference aborts on the same preconditions (NNML_ASSERT,
 * nnml/include/nnml.h:97-111); an nnml-side shim turns a non-zero status into
 * NNML_ABORT.
 */
#ifndef ARCLIGHT_FATTN_H
#define ARCLIGHT_FATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types, numbered as enum nnml_type (nnml/include/ops.h:140-171). */
enum {
    AL_TYPE_F32 = 0,
    AL_TYPE_F16 = 1,
    AL_TYPE_I32 = 26,
    AL_TYPE_I64 = 27
};

/* Accumulation precision, as enum nnml_prec (nnml/include/ops.h:174-177). */
enum {
    AL_PREC_DEFAULT = 0,
    AL_PREC_F32     = 10
};

/* Status codes. */
enum {
    AL_OK              = 0,
    AL_ERR_INVALID     = -1,  /* precondition the reference asserts        */
    AL_ERR_UNSUPPORTED = -2,  /* valid for the reference, not on this path */
    AL_ERR_HIP         = -3,  /* HIP runtime error                         */
    AL_ERR_WORKSPACE   = -4   /* caller workspace too small                */
};

/* One operand: nnml_tensor's data/type/ne/nb (nnml/include/tensor.h:78-198). */
typedef struct al_tensor {
    void *   data;
    int32_t  type;
    int32_t  reserved;
    int64_t  ne[4];
    uint64_t nb[4];
} al_tensor;

/*
 * Arguments of one flash-attention call.
 *
 * q, k, v, dst are required. mask.data == NULL means "no mask" and
 * sinks.data == NULL means "no sinks", as a NULL src tensor does in the
 * reference (arm.cpp:2226-2231, 2402).
 *
 * kv_len and causal_pos0 describe masking without a mask tensor, and act as
 * hints when a mask is also given:
 *   - cells c >= kv_len are masked for every query row (kv_len <= 0: n_kv);
 *   - when causal_pos0 >= 0, cell c is masked for query token t when
 *     c > causal_pos0 + t.
 * With a mask tensor present these must agree with it; the result is then
 * identical to the explicit mask alone, while wholly masked tiles are
 * skipped unread. (The nnml adapter passes the hints, without the mask,
 * when the node carries them: al_fattn_apply_node_hints below.)
 *
 * workspace: device scratch for split-KV partials. NULL lets the library use
 * its own buffer for the current device and args->stream (allocated on first
 * use, grown when needed, kept until al_fattn_release_stream; a graph
 * captured on a stream uses that stream's, so the stream needs one eager call
 * of the same shapes before the capture: allocating inside a capture fails;
 * callers that cannot make one use al_fattn_f16_noalloc).
 * A caller workspace must be zero-filled before its first use. Its first
 * 256 KiB hold arrival counters, which every call leaves at zero again, and
 * the decode kernel's split flags, which carry a per-(stream, kv head) epoch
 * from call to call (zeroing the workspace again between calls is allowed);
 * per-call merge records follow them. Calls that share one workspace must
 * be ordered on one stream.
 *
 * dyn_len: for a call captured once into a HIP graph and replayed for every
 * decode step (the GPU form of the reference's graph reuse while n_kv stays
 * within the built graph's, nnml/src/context.cpp:177-205), a device pointer
 * to two int32 {kv_len, causal_pos0} that the kernel reads when it runs.
 * The host kv_len is then the largest length the replays will use (it sizes
 * the launch) and causal_pos0 >= 0 only selects causal masking; the device
 * values must satisfy 0 < kv_len <= that bound and, when causal,
 * causal_pos0 + T <= kv_len. Needs implicit masking (no mask tensor) and up
 * to 32 query rows per kv head (the decode kernel); else AL_ERR_UNSUPPORTED.
 * Capture only after one eager call with the same shapes (workspaces are
 * allocated on first use).
 */
typedef struct al_fattn_args {
    al_tensor q;
    al_tensor k;
    al_tensor v;
    al_tensor mask;
    al_tensor sinks;
    al_tensor dst;
    float     scale;          /* op_params f32[0] */
    float     max_bias;       /* op_params f32[1] (ALiBi)   */
    float     logit_softcap;  /* op_params f32[2]           */
    int32_t   prec;           /* op_params i32[3]           */
    int64_t   kv_len;
    int64_t   causal_pos0;
    void *    stream;         /* hipStream_t; NULL = default stream */
    void *    workspace;
    uint64_t  workspace_bytes;
    const int32_t * dyn_len;  /* optional device {kv_len, causal_pos0}, see below */
} al_fattn_args;

/*
 * Flash attention, f16 K/V, f32 Q and output, f32 accumulation.
 * Replaces nnml_compute_forward_flash_attn_ext (nnml/src/ops/ops.cpp:1432-1445)
 * -> nnml_compute_forward_flash_attn_ext_f16 (nnml/src/ops/arm/arm.cpp:2196-2433).
 * Enqueues on args->stream and returns without synchronizing.
 */
int al_fattn_f16(const al_fattn_args * args);

/*
 * The op as nnml's workers run it. The reference executes a graph node on
 * every worker of the pool, each with its own (ith, nth) from its
 * nnml_compute_state (nnml/src/scheduler.cpp:98-101 inside
 * nnml_single_graph_compute_thread :122-146; nnml/include/thread.h:153-168),
 * splits the rows by ith (nnml/src/ops/arm/arm.cpp:2250-2257), and puts a
 * barrier after the node (scheduler.cpp:135-142). Here worker 0 runs
 * al_fattn_f16, waits for args->stream and returns what al_device_errors
 * then reports, so that barrier still means the output is complete (or the
 * node failed); every other worker returns AL_OK at once without reading
 * args or calling the HIP runtime. (ith, nth) outside 0 <= ith < nth gives
 * AL_ERR_INVALID.
 */
int al_fattn_f16_worker(const al_fattn_args * args, int ith, int nth);

/*
 * Length hints an nnml flash_attn_ext node carries for this library in
 * op_params i32[4..6], words the reference leaves zero (tensor_new clears
 * op_params, nnml/src/tensor.cpp:213; the node uses words 0..3,
 * tensor.cpp:1311, 1334-1338): [4] = AL_FATTN_HINT_TAG, [5] = kv_len,
 * [6] = causal_pos0 (-1: not causal). The tag states that the node's mask
 * tensor is exactly the implicit rule of al_fattn_args: the graph sets these
 * words when al_kv_cells_implicit says so for the ubatch whose mask it fills
 * (set_inputs_attn_mask, nnml/src/cgraph.cpp:1224-1261), and clears word 4
 * otherwise. No counterpart in the reference, which always reads the mask.
 * al_fattn_apply_node_hints: when op_params carries the tag, sets
 * args->kv_len and args->causal_pos0 from it and drops args->mask (the
 * implicit rule gives the same results without reading the mask) and
 * returns 1; otherwise leaves args unchanged and returns 0. NULL arguments
 * return 0.
 */
#define AL_FATTN_HINT_TAG 0x31484c41   /* "ALH1" */
int al_fattn_apply_node_hints(al_fattn_args * args, const int32_t * op_params);

/*
 * Frees the library workspace of (current device, stream) that calls with
 * workspace == NULL made, after waiting for the device (its kernels and any
 * graph replayed on the stream may still use it). No counterpart in the
 * reference (its op uses per-thread scratch of the graph's work buffer,
 * nnml/src/ops/arm/arm.cpp:2299-2302). A later call allocates again. AL_OK
 * when the stream has none.
 */
int al_fattn_release_stream(void * stream);

/* Workspace bytes al_fattn_f16 needs for these arguments (0 if none). */
uint64_t al_fattn_workspace_bytes(const al_fattn_args * args);

/*
 * al_fattn_f16 without any allocation. No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * validation, kernels and results as al_fattn_f16; args->workspace is
 * ignored. The scratch (arrival counters, decode split flags and merge
 * records) is a file-scope
 * device array of
 * AL_FATTN_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends. A
 * call that needs more (al_fattn_workspace_bytes) fails with
 * AL_ERR_WORKSPACE. Every call on one GPU shares that array: calls that
 * overlap on one GPU (two streams, or two host threads) race and may give
 * wrong results; order them on one stream.
 * al_fattn_noalloc_init sets up the current device (finds its copy of the
 * array and clears the counter region, synchronizing the default stream):
 * call it once per device before capturing a graph; otherwise the first
 * call does it.
 */
#define AL_FATTN_NOALLOC_SCRATCH_BYTES (32u << 20)
int al_fattn_noalloc_init(void);
int al_fattn_f16_noalloc(const al_fattn_args * args);

/* Message of the calling thread's most recent failure ("" if none). */
const char * al_last_error(void);

/*
 * KV write: dst[idx[i]] = f16(src[i]) row by row, IEEE round-to-nearest-even.
 * Replaces nnml_compute_forward_set_rows (nnml/src/ops/ops.cpp:1300-1320) ->
 * nnml_compute_forward_set_rows_f32 (ops.cpp:135-181) for an f16 destination,
 * the op llm_kv_cache::cpy_k / cpy_v build (nnml/src/cgraph.cpp:1114-1180).
 *   dst f16 ne = [nc, n_rows_dst, d2, d3]   (the cache, device)
 *   src f32 ne = [nc, n_rows,     d2, d3]
 *   idx i64 or i32 ne = [n_rows, i1, i2]  (broadcast over d2 % i1, d3 % i2)
 * Enqueues on `stream` without synchronizing. A row whose index lies outside
 * [0, n_rows_dst) is not written; the kernel records it, and the next
 * al_device_errors() after the stream completes returns AL_ERR_INVALID
 * (the reference asserts on it, ops.cpp:171).
 */
int al_set_rows_f32_f16(const al_tensor * dst, const al_tensor * src,
                        const al_tensor * idx, void * stream);

/*
 * Reports and clears errors that kernels recorded on the current device
 * (out-of-range set_rows indices: AL_ERR_INVALID; a decode merge that gave
 * up waiting for the other splits of its launch, about a second, which a
 * correct run never does: AL_ERR_HIP, and that call's merged rows hold
 * NaN). Call after synchronizing the stream. Returns AL_OK or the error
 * with al_last_error() set.
 */
int al_device_errors(void);

/* Library version string. */
const char * al_version(void);

#ifdef __cplusplus
}
#endif

#endif /* ARCLIGHT_FATTN_H */
