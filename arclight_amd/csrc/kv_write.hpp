// KV-cache write kernel (set_rows f32 -> f16).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/arclight_fattn.h"
#include "kernel_args.hpp"

struct SetRowsParams {
    const char * src;  int64_t s_nb1, s_nb2, s_nb3;   // f32 [nc, nr, ne2, ne3]
    char * dst;        int64_t d_nb1, d_nb2, d_nb3;   // f16 [nc, n_dst, ne2, ne3]
    const char * idx;  int64_t i_nb0, i_nb1, i_nb2;   // i64/i32 [nr, i_ne1, i_ne2]
    int32_t idx64;
    int32_t nc, nr, ne2, ne3, i_ne1, i_ne2;
    int64_t n_dst;
    int32_t vec4;                                     // rows 16-byte aligned, nc % 4 == 0
    int * err;
};

// Source row i of plane (i02, i03) converted to f16 (IEEE RNE) into cache
// row idx[i]; an index out of range is not written but reported through
// p.err. One workgroup of any size per row.
__device__ __forceinline__ void set_rows_row(const SetRowsParams & p, const int i, const int i02, const int i03) {
    const int i12 = i03 % p.i_ne2;
    const int i11 = i02 % p.i_ne1;
    const char * ip = p.idx + (int64_t) i * p.i_nb0 + (int64_t) i11 * p.i_nb1 + (int64_t) i12 * p.i_nb2;
    const int64_t i1 = p.idx64 ? *(const int64_t *) ip : (int64_t) *(const int32_t *) ip;
    if (i1 < 0 || i1 >= p.n_dst) {
        if (threadIdx.x == 0) {
            if (atomicCAS(p.err, 0, 1) == 0) p.err[1] = (int) i1;
        }
        return;
    }
    const float * src = (const float *) (p.src + (int64_t) i * p.s_nb1 + (int64_t) i02 * p.s_nb2 + (int64_t) i03 * p.s_nb3);
    _Float16 * dst = (_Float16 *) (p.dst + i1 * p.d_nb1 + (int64_t) i02 * p.d_nb2 + (int64_t) i03 * p.d_nb3);
    if (p.vec4) {
        for (int c = 4 * threadIdx.x; c < p.nc; c += 4 * blockDim.x) {
            const float4 x = *(const float4 *) (src + c);
            typedef _Float16 half4 __attribute__((ext_vector_type(4)));
            half4 h = {(_Float16) x.x, (_Float16) x.y, (_Float16) x.z, (_Float16) x.w};
            *(half4 *) (dst + c) = h;
        }
    } else {
        for (int c = threadIdx.x; c < p.nc; c += blockDim.x) dst[c] = (_Float16) src[c];
    }
}

// Checks dst / src / idx as al_set_rows_f32_f16 does and fills p; *empty is
// set when there is nothing to write. AL_OK or the failing status.
int set_rows_params(const al_tensor * dst, const al_tensor * src, const al_tensor * idx, SetRowsParams * p, bool * empty);

hipError_t set_rows_launch(const SetRowsParams & p, hipStream_t stream);
