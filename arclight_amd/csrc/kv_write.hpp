// KV-cache write kernel (set_rows f32 -> f16).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

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

hipError_t set_rows_launch(const SetRowsParams & p, hipStream_t stream);
