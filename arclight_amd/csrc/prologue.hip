// Producers of the attention operands for gfx950 (include/arclight_prologue.h):
// per-head RMSNorm, the norm weight and the rotary embedding of Q and K in
// one pass, K optionally straight into the f16 KV cache.
//
// Semantics: nnml_compute_forward_rms_norm_f32 (nnml/src/ops/ops.cpp:
// 680-726: squares summed in double, mean and scale in float), the f32 mul,
// and nnml_compute_forward_rope_f32 (ops.cpp:871-962) with rope_yarn and the
// rotation cache (ops.cpp:743-772): the angle of pair i is the position
// multiplied i times by theta_scale in float, exactly as the cache loop
// carries it.
//
// One wavefront per (token, head) row of 128 floats: lane l holds the two
// elements of rotation pair l (dims l and l + 64 for NEOX, 2l and 2l + 1
// otherwise), so the norm is one wave reduction and the rotation needs no
// data exchange. A workgroup takes 4 heads of one token; the pair angles and
// their cos / sin are computed once per wave.

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>

#include "../../include/arclight_prologue.h"
#include "fattn_kernels.hpp"
#include "kv_write.hpp"
#include "norm_rope.hpp"
#include "runtime.hpp"

namespace {

struct NormRopeParams {
    const char * x;     int64_t x_nb1, x_nb2;      // row (head h, token t) at x + h nb1 + t nb2
    const float * w;                               // [128] or null
    const int32_t * pos;                           // [T]
    char * y;           int64_t y_nb1, y_nb2;      // f32 rows, or the f16 cache (nb1 = row bytes)
    const char * rows;  int64_t rows_nb0;          // cache rows [T] or null
    int32_t rows64;
    int64_t n_rows_dst;
    int32_t H, T;
    float eps;
    RopeConsts rope;
    int * err;                                     // [2]: first out-of-range cache row
};

// Row (head h, token t), one wavefront. MODE: 0 no rotation, 1 pairs
// (2i, 2i + 1), 2 NEOX pairs (i, i + 64).
template <int MODE, bool CACHE>
__device__ __forceinline__ void norm_rope_row(const NormRopeParams & p, const int h, const int t, const int lane) {
    if (h >= p.H) return;
    const int d0 = rope_d0<MODE>(lane), d1 = rope_d1<MODE>(lane);
    const float w0 = p.w ? p.w[d0] : 1.0f;
    const float w1 = p.w ? p.w[d1] : 1.0f;
    const float * xr = (const float *) (p.x + (int64_t) h * p.x_nb1 + (int64_t) t * p.x_nb2);
    float y0, y1;
    norm_rope_pair<MODE>(xr[d0], xr[d1], p.w != nullptr, w0, w1, p.eps, p.rope, MODE != 0 ? p.pos[t] : 0, lane, y0, y1);
    if constexpr (CACHE) {
        const char * ip = p.rows + (int64_t) t * p.rows_nb0;
        const int64_t r = p.rows64 ? *(const int64_t *) ip : (int64_t) *(const int32_t *) ip;
        if (r < 0 || r >= p.n_rows_dst) {
            if (lane == 0 && atomicCAS(p.err, 0, 1) == 0) p.err[1] = (int) r;
            return;
        }
        _Float16 * yr = (_Float16 *) (p.y + r * p.y_nb1) + (int64_t) h * 128;
        yr[d0] = (_Float16) y0;
        yr[d1] = (_Float16) y1;
    } else {
        float * yr = (float *) (p.y + (int64_t) h * p.y_nb1 + (int64_t) t * p.y_nb2);
        yr[d0] = y0;
        yr[d1] = y1;
    }
}

template <int MODE, bool CACHE>
__global__ __launch_bounds__(256) void norm_rope_kernel(const NormRopeParams p) {
    prefetch_params(p);
    norm_rope_row<MODE, CACHE>(p, blockIdx.y * 4 + (threadIdx.x >> 6), blockIdx.x, threadIdx.x & 63);
}

// The attention inputs of one layer in one launch: blockIdx.y < yq are Q
// rows (4 heads per workgroup), then yk of K rows into the cache, then one
// workgroup per token for its V row.
template <int MODE>
__global__ __launch_bounds__(256) void attn_inputs_kernel(const NormRopeParams q, const NormRopeParams k,
                                                          const SetRowsParams v, const int yq, const int yk) {
    prefetch_params(q, k, v, yq, yk);
    const int by = blockIdx.y;
    const int hw = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (by < yq) norm_rope_row<MODE, false>(q, by * 4 + hw, blockIdx.x, lane);
    else if (by < yq + yk) norm_rope_row<MODE, true>(k, (by - yq) * 4 + hw, blockIdx.x, lane);
    else set_rows_row(v, blockIdx.x, 0, 0);
}

template <int MODE>
hipError_t launch_mode(const NormRopeParams & p, bool cache, hipStream_t stream) {
    const dim3 grid((unsigned) p.T, (unsigned) ((p.H + 3) / 4));
    if (cache) hipLaunchKernelGGL((norm_rope_kernel<MODE, true>), grid, dim3(256), 0, stream, p);
    else       hipLaunchKernelGGL((norm_rope_kernel<MODE, false>), grid, dim3(256), 0, stream, p);
    return hipGetLastError();
}

// YaRN correction dimension for a rotation count (ops.cpp:728-730).
float yarn_corr_dim(int n_dims, int n_ctx_orig, float n_rot, float base) {
    const double pi = 3.14159265358979323846;
    return n_dims * logf(n_ctx_orig / (n_rot * 2 * (float) pi)) / (2 * logf(base));
}

// Checks the operands as al_rms_norm_rope_f32 documents them and fills p
// and the rotation mode (0 none, 1 normal, 2 NEOX).
int norm_rope_params(const al_tensor * x, const al_tensor * w, const al_tensor * pos, float eps,
                     const al_rope_params * rope, const al_tensor * y, const al_tensor * rows, NormRopeParams * out,
                     int * mode_out) {
    if (!x || !pos || !y) return al_fail(AL_ERR_INVALID, "rms_norm_rope: x, pos and y required");
    if (x->type != AL_TYPE_F32 || x->ne[0] != 128 || x->nb[0] != 4 || x->ne[3] != 1)
        return al_fail(AL_ERR_UNSUPPORTED, "rms_norm_rope: x must be f32 [128, H, T, 1] with nb0 = 4");
    const int64_t H = x->ne[1], T = x->ne[2];
    if (H <= 0 || T <= 0 || T > INT32_MAX / 2 || H > 65535 * 4) return al_fail(AL_ERR_INVALID, "rms_norm_rope: bad H %lld or T %lld", (long long) H, (long long) T);
    if (!(eps >= 0.0f)) return al_fail(AL_ERR_INVALID, "rms_norm_rope: eps %g < 0 (ops.cpp:697)", (double) eps);
    if (w && (w->type != AL_TYPE_F32 || w->ne[0] < 128 || w->nb[0] != 4 || !w->data))
        return al_fail(AL_ERR_INVALID, "rms_norm_rope: w must be f32 [128]");
    if (pos->type != AL_TYPE_I32 || pos->ne[0] != T || pos->nb[0] != 4 || !pos->data)
        return al_fail(AL_ERR_INVALID, "rms_norm_rope: pos must be i32 [T] (tensor.cpp:1014-1019)");
    int mode = 0;
    NormRopeParams p;
    memset(&p, 0, sizeof(p));
    if (rope) {
        if (rope->n_dims != 128) return al_fail(AL_ERR_UNSUPPORTED, "rms_norm_rope: n_dims %d (only the full head, 128)", rope->n_dims);
        if (rope->mode == AL_ROPE_NEOX) mode = 2;
        else if (rope->mode == AL_ROPE_NORMAL) mode = 1;
        else return al_fail(AL_ERR_UNSUPPORTED, "rms_norm_rope: rope mode %d", rope->mode);
        // host-side constants exactly as the reference's rope op computes them
        p.rope.theta_scale = powf(rope->freq_base, -2.0f / rope->n_dims);
        const float start = floorf(yarn_corr_dim(rope->n_dims, rope->n_ctx_orig, rope->beta_fast, rope->freq_base));
        const float end = ceilf(yarn_corr_dim(rope->n_dims, rope->n_ctx_orig, rope->beta_slow, rope->freq_base));
        p.rope.corr0 = fmaxf(0.0f, start);
        p.rope.corr1 = fminf((float) (rope->n_dims - 1), end);
        p.rope.freq_scale = rope->freq_scale;
        p.rope.ext_factor = rope->ext_factor;
        p.rope.mscale = rope->attn_factor;
        if (rope->ext_factor != 0.0f) p.rope.mscale *= 1.0f + 0.1f * logf(1.0f / rope->freq_scale);
    }
    p.x = (const char *) x->data; p.x_nb1 = (int64_t) x->nb[1]; p.x_nb2 = (int64_t) x->nb[2];
    p.w = w ? (const float *) w->data : nullptr;
    p.pos = (const int32_t *) pos->data;
    p.H = (int32_t) H; p.T = (int32_t) T;
    p.eps = eps;
    const bool cache = rows != nullptr;
    if (cache) {
        if (y->type != AL_TYPE_F16 || y->ne[0] != 128 * H || y->nb[0] != 2 || (int64_t) y->nb[1] < 256 * H)
            return al_fail(AL_ERR_INVALID, "rms_norm_rope: cache must be f16 [128*H, n_rows] with contiguous rows");
        if ((rows->type != AL_TYPE_I64 && rows->type != AL_TYPE_I32) || rows->ne[0] != T || !rows->data)
            return al_fail(AL_ERR_INVALID, "rms_norm_rope: rows must be i64 / i32 [T]");
        p.rows = (const char *) rows->data;
        p.rows_nb0 = (int64_t) rows->nb[0];
        p.rows64 = rows->type == AL_TYPE_I64;
        p.n_rows_dst = y->ne[1];
        p.y_nb1 = (int64_t) y->nb[1];
        int rc = al_device_error_flag(&p.err);
        if (rc != AL_OK) return rc;
    } else {
        if (y->type != AL_TYPE_F32 || y->ne[0] != 128 || y->ne[1] != H || y->ne[2] != T || y->nb[0] != 4)
            return al_fail(AL_ERR_INVALID, "rms_norm_rope: y must be f32 [128, H, T] with nb0 = 4");
        p.y_nb1 = (int64_t) y->nb[1];
        p.y_nb2 = (int64_t) y->nb[2];
    }
    p.y = (char *) y->data;
    if (!p.x || !p.y) return al_fail(AL_ERR_INVALID, "rms_norm_rope: null data");
    *out = p;
    *mode_out = mode;
    return AL_OK;
}

}  // namespace

// The checks of al_attn_inputs_f32, then what the decode kernel needs to fold
// the inputs into its prologue (one token, operands it can move by 16-byte
// DMA); fills *out and the rotation mode.
int attn_inputs_decode(const al_attn_inputs_args * a, DecodeInputs * out, int * mode_out) {
    if (!a) return al_fail(AL_ERR_INVALID, "attn_inputs: null arguments");
    NormRopeParams q, k;
    int mq = 0, mk = 0;
    int rc = norm_rope_params(&a->q, a->q_w.data ? &a->q_w : nullptr, &a->pos, a->eps, a->rope, &a->q_out, nullptr, &q, &mq);
    if (rc != AL_OK) return rc;
    rc = norm_rope_params(&a->k, a->k_w.data ? &a->k_w : nullptr, &a->pos, a->eps, a->rope, &a->k_cache, &a->rows, &k, &mk);
    if (rc != AL_OK) return rc;
    if (q.T != k.T) return al_fail(AL_ERR_INVALID, "attn_inputs: q has %d tokens, k %d", q.T, k.T);
    if (a->v.ne[1] != q.T || a->v.ne[2] != 1 || a->v.ne[3] != 1)
        return al_fail(AL_ERR_INVALID, "attn_inputs: v must be f32 [n, T] with the tokens of q");
    SetRowsParams v;
    bool empty = false;
    rc = set_rows_params(&a->v_cache, &a->v, &a->rows, &v, &empty);
    if (rc != AL_OK) return rc;
    if (empty) return al_fail(AL_ERR_INVALID, "attn_inputs: empty v");
    auto al16 = [](const void * ptr) { return ((uintptr_t) ptr & 15u) == 0; };
    const int64_t esz = k.rows64 ? 8 : 4;
    if (q.T != 1 || v.nc != 128 * k.H || v.n_dst != k.n_rows_dst || k.rows_nb0 != esz ||
        !al16(k.x) || k.x_nb1 % 16 || k.x_nb2 % 16 || !al16(v.src) || v.s_nb1 % 16 || !al16(k.rows) || !al16(k.pos) ||
        (q.w && !al16(q.w)) || (k.w && !al16(k.w)))
        return al_fail(AL_ERR_UNSUPPORTED, "attn_inputs: operands the fused decode prologue cannot take");
    DecodeInputs d;
    memset(&d, 0, sizeof(d));
    d.q_w = (const char *) q.w;
    d.k = k.x; d.k_nb1 = k.x_nb1; d.k_nb2 = k.x_nb2;
    d.k_w = (const char *) k.w;
    d.v = v.src; d.v_nb1 = v.s_nb1;
    d.pos = q.pos;
    d.rows = k.rows; d.rows_nb0 = k.rows_nb0; d.rows64 = k.rows64;
    d.T = q.T;
    d.q_out = q.y; d.qo_nb1 = q.y_nb1; d.qo_nb2 = q.y_nb2;
    d.k_cache = k.y; d.kc_nb1 = k.y_nb1;
    d.v_cache = v.dst; d.vc_nb1 = v.d_nb1;
    d.n_rows = k.n_rows_dst;
    d.eps = a->eps;
    d.rope = q.rope;
    *out = d;
    *mode_out = mq;
    return AL_OK;
}

extern "C" int al_rms_norm_rope_f32(const al_tensor * x, const al_tensor * w, const al_tensor * pos, float eps,
                                    const al_rope_params * rope, const al_tensor * y, const al_tensor * rows,
                                    void * stream) {
    NormRopeParams p;
    int mode = 0;
    const int rc = norm_rope_params(x, w, pos, eps, rope, y, rows, &p, &mode);
    if (rc != AL_OK) return rc;
    const bool cache = rows != nullptr;
    hipStream_t s = (hipStream_t) stream;
    hipError_t e;
    switch (mode) {
        case 2: e = launch_mode<2>(p, cache, s); break;
        case 1: e = launch_mode<1>(p, cache, s); break;
        default: e = launch_mode<0>(p, cache, s); break;
    }
    return e == hipSuccess ? AL_OK : al_hip_fail(e, "rms_norm_rope: launch");
}

extern "C" int al_attn_inputs_f32(const al_attn_inputs_args * a, void * stream) {
    if (!a) return al_fail(AL_ERR_INVALID, "attn_inputs: null arguments");
    NormRopeParams q, k;
    int mq = 0, mk = 0;
    int rc = norm_rope_params(&a->q, a->q_w.data ? &a->q_w : nullptr, &a->pos, a->eps, a->rope, &a->q_out, nullptr, &q, &mq);
    if (rc != AL_OK) return rc;
    rc = norm_rope_params(&a->k, a->k_w.data ? &a->k_w : nullptr, &a->pos, a->eps, a->rope, &a->k_cache, &a->rows, &k, &mk);
    if (rc != AL_OK) return rc;
    if (q.T != k.T) return al_fail(AL_ERR_INVALID, "attn_inputs: q has %d tokens, k %d", q.T, k.T);
    if (a->v.ne[1] != q.T || a->v.ne[2] != 1 || a->v.ne[3] != 1)
        return al_fail(AL_ERR_INVALID, "attn_inputs: v must be f32 [n, T] with the tokens of q");
    SetRowsParams v;
    bool empty = false;
    rc = set_rows_params(&a->v_cache, &a->v, &a->rows, &v, &empty);
    if (rc != AL_OK) return rc;
    if (empty) return al_fail(AL_ERR_INVALID, "attn_inputs: empty v");
    const int yq = (q.H + 3) / 4, yk = (k.H + 3) / 4;
    const dim3 grid((unsigned) q.T, (unsigned) (yq + yk + 1));
    hipStream_t s = (hipStream_t) stream;
    switch (mq) {
        case 2: hipLaunchKernelGGL(attn_inputs_kernel<2>, grid, dim3(256), 0, s, q, k, v, yq, yk); break;
        case 1: hipLaunchKernelGGL(attn_inputs_kernel<1>, grid, dim3(256), 0, s, q, k, v, yq, yk); break;
        default: hipLaunchKernelGGL(attn_inputs_kernel<0>, grid, dim3(256), 0, s, q, k, v, yq, yk); break;
    }
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? AL_OK : al_hip_fail(e, "attn_inputs: launch");
}
