// KV-cache write: rows of f32 K or V converted to f16 (IEEE RNE) and stored
// at the cache cells named by an index vector. Restates
// nnml_compute_forward_set_rows_f32 (nnml/src/ops/ops.cpp:135-181), the op
// llm_kv_cache::cpy_k / cpy_v emit before attention (nnml/src/cgraph.cpp:
// 1114-1180, 485-488). One workgroup per source row; each thread converts 4
// consecutive floats (one 16-byte load, one 8-byte store).
#include <hip/hip_runtime.h>

#include "../../include/arclight_fattn.h"
#include "kv_write.hpp"
#include "runtime.hpp"

namespace {

__global__ __launch_bounds__(256) void set_rows_kernel(const SetRowsParams p) {
    prefetch_params(p);
    set_rows_row(p, blockIdx.x, blockIdx.y, blockIdx.z);
}

}  // namespace

hipError_t set_rows_launch(const SetRowsParams & p, hipStream_t stream) {
    const dim3 grid((unsigned) p.nr, (unsigned) p.ne2, (unsigned) p.ne3);
    hipLaunchKernelGGL(set_rows_kernel, grid, dim3(256), 0, stream, p);
    return hipGetLastError();
}

int set_rows_params(const al_tensor * dst, const al_tensor * src, const al_tensor * idx, SetRowsParams * out, bool * empty) {
    *empty = false;
    if (!dst || !src || !idx || !dst->data || !src->data || !idx->data)
        return al_fail(AL_ERR_INVALID, "set_rows: dst, src and idx are required");
    if (src->type != AL_TYPE_F32)
        return al_fail(AL_ERR_UNSUPPORTED, "set_rows: src type %d (f32 only, ops.cpp:1303-1315)", src->type);
    if (idx->type != AL_TYPE_I64 && idx->type != AL_TYPE_I32)
        return al_fail(AL_ERR_UNSUPPORTED, "set_rows: index type %d (i64/i32, ops.cpp:1306-1312)", idx->type);
    if (dst->type != AL_TYPE_F16) return al_fail(AL_ERR_UNSUPPORTED, "set_rows: dst type %d (f16 cache only)", dst->type);
    // ops.cpp:145-150
    if (dst->ne[0] != src->ne[0] || dst->ne[2] != src->ne[2] || dst->ne[3] != src->ne[3])
        return al_fail(AL_ERR_INVALID, "set_rows: dst and src shapes differ");
    if (idx->ne[1] <= 0 || idx->ne[2] <= 0 || src->ne[2] % idx->ne[1] != 0 || src->ne[3] % idx->ne[2] != 0)
        return al_fail(AL_ERR_INVALID, "set_rows: index tensor does not broadcast over src");
    if (idx->ne[0] < src->ne[1]) return al_fail(AL_ERR_INVALID, "set_rows: fewer indices than rows");
    if (src->nb[0] != 4 || dst->nb[0] != 2) return al_fail(AL_ERR_INVALID, "set_rows: rows must be contiguous");
    if (src->ne[1] == 0 || src->ne[2] == 0 || src->ne[3] == 0) {
        *empty = true;
        return AL_OK;
    }
    if (src->ne[1] > INT32_MAX || src->ne[2] > 65535 || src->ne[3] > 65535 || src->ne[0] > INT32_MAX)
        return al_fail(AL_ERR_UNSUPPORTED, "set_rows: sizes out of range");
    int * err = nullptr;
    int rc = al_device_error_flag(&err);
    if (rc != AL_OK) return rc;
    SetRowsParams p;
    p.src = (const char *) src->data; p.s_nb1 = src->nb[1]; p.s_nb2 = src->nb[2]; p.s_nb3 = src->nb[3];
    p.dst = (char *) dst->data; p.d_nb1 = dst->nb[1]; p.d_nb2 = dst->nb[2]; p.d_nb3 = dst->nb[3];
    p.idx = (const char *) idx->data; p.i_nb0 = idx->nb[0]; p.i_nb1 = idx->nb[1]; p.i_nb2 = idx->nb[2];
    p.idx64 = idx->type == AL_TYPE_I64;
    p.nc = (int32_t) src->ne[0]; p.nr = (int32_t) src->ne[1]; p.ne2 = (int32_t) src->ne[2]; p.ne3 = (int32_t) src->ne[3];
    p.i_ne1 = (int32_t) idx->ne[1]; p.i_ne2 = (int32_t) idx->ne[2];
    p.n_dst = dst->ne[1];
    const bool al16 = (((uintptr_t) src->data | (uintptr_t) dst->data) & 15u) == 0 &&
                      src->nb[1] % 16 == 0 && src->nb[2] % 16 == 0 && src->nb[3] % 16 == 0 &&
                      dst->nb[1] % 8 == 0 && dst->nb[2] % 8 == 0 && dst->nb[3] % 8 == 0 && (src->ne[0] % 4) == 0;
    p.vec4 = al16 ? 1 : 0;
    p.err = err;
    *out = p;
    return AL_OK;
}

extern "C" int al_set_rows_f32_f16(const al_tensor * dst, const al_tensor * src, const al_tensor * idx, void * stream) {
    SetRowsParams p;
    bool empty = false;
    const int rc = set_rows_params(dst, src, idx, &p, &empty);
    if (rc != AL_OK || empty) return rc;
    const hipError_t e = set_rows_launch(p, (hipStream_t) stream);
    if (e != hipSuccess) return al_hip_fail(e, "set_rows: kernel launch");
    return AL_OK;
}
