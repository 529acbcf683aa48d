// nnml-side binding of NNML_OP_FLASH_ATTN_EXT to the MI355X library.
//
// This is the code a maintainer adds to nnml next to
// nnml_compute_forward_flash_attn_ext (nnml/src/ops/ops.cpp:1432-1445),
// built with nnml's own headers:
//   nnml/include/tensor.h  nnml_tensor accessors (:98-150)
//   nnml/include/ops.h     nnml_op / nnml_type / nnml_prec, op entry points
//   nnml/include/thread.h  nnml_compute_state {ith, nth} (:153-168)
// and linked with libarclight_fattn.so. It compiles unchanged against those
// headers (tests/test_nnml_binding.py builds it from the reference tree).
//
// Every worker of the pool runs the node with its own (ith, nth)
// (nnml/src/scheduler.cpp:98-101 inside nnml_single_graph_compute_thread
// :122-146) and a barrier follows the node (scheduler.cpp:135-142).
// al_fattn_f16_worker keeps that contract: worker 0 launches and waits for
// the stream, the others return at once, so the barrier still means the
// output is complete. A non-zero status aborts, as the reference's asserts
// do (NNML_ABORT, nnml/include/nnml.h:97-111).
#include "tensor.h"
#include "ops.h"
#include "thread.h"

#include "arclight_fattn.h"

// The HIP stream the context runs device work on (a hipStream_t; nullptr is
// the default stream). Set once by the context that owns the HBM KV ring.
void * nnml_fattn_hip_stream = nullptr;

// An nnml tensor view as the library's operand descriptor: the same data
// pointer, type numbering, ne[] and nb[] (nnml/include/tensor.h:78-198).
// NULL (an absent mask or sinks operand) is the empty descriptor.
static al_tensor nnml_to_al(const nnml_tensor * t) {
    al_tensor a = {};
    if (!t) return a;
    a.data = t->tensor_data();
    a.type = (int32_t) t->get_data_type();
    for (int i = 0; i < 4; ++i) {
        a.ne[i] = t->get_elements(i);
        a.nb[i] = (uint64_t) t->get_stride_bytes(i);
    }
    return a;
}

// NNML_OP_FLASH_ATTN_EXT for a node whose K/V views point into the HBM ring:
// operands src[0..4] = q, k, v, mask, sinks (nnml/src/tensor.cpp:1314-1318,
// 1331), op_params f32[0..2] = {scale, max_bias, logit_softcap} and
// i32[3] = prec (tensor.cpp:1311, 1334-1338), output node->data.
void nnml_compute_forward_flash_attn_ext_hip(nnml_tensor * node, const nnml_compute_state * params) {
    al_fattn_args a = {};
    a.q = nnml_to_al(node->get_src_tensor(0));
    a.k = nnml_to_al(node->get_src_tensor(1));
    a.v = nnml_to_al(node->get_src_tensor(2));
    a.mask = nnml_to_al(node->get_src_tensor(3));
    a.sinks = nnml_to_al(node->get_src_tensor(4));
    a.dst = nnml_to_al(node);
    a.scale = node->get_op_params_f32(0);
    a.max_bias = node->get_op_params_f32(1);
    a.logit_softcap = node->get_op_params_f32(2);
    a.prec = node->get_op_params_i32(3);
    a.kv_len = 0;                  // the mask tensor alone decides visibility ...
    a.causal_pos0 = -1;
    // ... unless the graph marked the node: op_params i32[4..6] = tag,
    // kv_len, causal_pos0, set when the ubatch's mask is exactly that rule
    // (al_kv_cells_implicit); then the rule replaces the mask
    al_fattn_apply_node_hints(&a, node->get_operation_params());
    a.stream = nnml_fattn_hip_stream;
    const int rc = al_fattn_f16_worker(&a, params->ith, params->nth);
    if (rc != AL_OK) NNML_ABORT("flash_attn_ext (MI355X): %s", al_last_error());
}
