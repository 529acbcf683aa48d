// Per-head RMSNorm, weight and rotary embedding of one 128-float row by one
// wavefront (gfx950): the arithmetic of the attention-input producers,
// shared by the stand-alone kernels and the decode kernel that folds them
// into its prologue, so that both give the same bits.
//   rms_norm  nnml/src/ops/ops.cpp:680-726
//   mul       nnml/src/ops/ops.cpp:1248-1250
//   rope_ext  nnml/src/ops/ops.cpp:728-777, 871-962
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// Rotation constants of the rope_ext op, resolved on the host as the
// reference's rope op computes them (rope_yarn_corr_dims, the YaRN mscale).
struct RopeConsts {
    float theta_scale, freq_scale, ext_factor, corr0, corr1, mscale;
};

__device__ __forceinline__ double norm_rope_wave_sum(double v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// Dims of the lane's pair. MODE: 0 no rotation, 1 pairs (2i, 2i + 1),
// 2 NEOX pairs (i, i + 64).
template <int MODE> __device__ __forceinline__ int rope_d0(const int lane) { return MODE == 1 ? 2 * lane : lane; }
template <int MODE> __device__ __forceinline__ int rope_d1(const int lane) { return MODE == 1 ? 2 * lane + 1 : lane + 64; }

// cos / sin (times mscale) of the lane's pair at position pos (ops.cpp:743-772).
template <int MODE>
__device__ __forceinline__ void rope_cos_sin(const RopeConsts & r, const int32_t pos, const int lane, float & c,
                                             float & s) {
    // every product and sum rounded on its own, as the reference's C source
    // reads: at angles of thousands of radians one ulp of theta moves the
    // output by ~1e-4, so a fused multiply-add there would not match
#pragma clang fp contract(off)
    c = 1.0f;
    s = 0.0f;
    if constexpr (MODE != 0) {
        const float theta_extrap0 = (float) pos;
        float theta_extrap = theta_extrap0;
        for (int k = 0; k < 63; ++k)
            if (k < lane) theta_extrap *= r.theta_scale;
        const float theta_interp = r.freq_scale * theta_extrap;
        float theta = theta_interp;
        if (r.ext_factor != 0.0f) {
            const float yv = ((float) lane - r.corr0) / fmaxf(0.001f, r.corr1 - r.corr0);
            const float ramp = 1.0f - fminf(1.0f, fmaxf(0.0f, yv));
            const float mix = ramp * r.ext_factor;
            theta = theta_interp * (1.0f - mix) + theta_extrap * mix;
        }
        c = cosf(theta) * r.mscale;
        s = sinf(theta) * r.mscale;
    }
}

// y = rope(rms_norm(x) * w) at dims d0, d1 of the lane, given the pair's
// cos / sin (rope_cos_sin): x0, x1 and w0, w1 are those dims of the row and
// of the weight (has_w false: no weight); every lane of the wave takes part
// (the norm's sum is a wave reduction).
template <int MODE>
__device__ __forceinline__ void norm_rope_apply(const float x0, const float x1, const bool has_w, const float w0,
                                                const float w1, const float eps, const float c, const float s,
                                                float & y0, float & y1) {
#pragma clang fp contract(off)
    const float sq0 = x0 * x0, sq1 = x1 * x1;
    const double sum = norm_rope_wave_sum((double) sq0 + (double) sq1);
    const float mean = (float) (sum / 128.0);
    const float scale = 1.0f / sqrtf(mean + eps);
    float n0 = x0 * scale, n1 = x1 * scale;
    if (has_w) {
        n0 = n0 * w0;
        n1 = n1 * w1;
    }
    y0 = n0;
    y1 = n1;
    if constexpr (MODE != 0) {
        y0 = n0 * c - n1 * s;
        y1 = n0 * s + n1 * c;
    }
}

// RMSNorm, weight and rotation of rows held by groups of 8 lanes (lanes
// 8i..8i+7 of a wave hold one row), each lane with 8 rotation pairs: lo[k]
// and hi[k] are the two dims of the lane's pair k, w_lo / w_hi their
// weights (1 where there is no weight, which leaves the product bit for bit
// unchanged), rot[k] the pair's (cos, sin). Per value the arithmetic of
// norm_rope_apply; the row's sum of squares (double) is added in another
// order, so the two can differ only where the partial sums are not exact in
// double, by rounding in the double's last bits, far below the f32 mean's
// resolution. Every lane of the wave takes part (the sum's shuffles).
template <int MODE>
__device__ __forceinline__ void norm_rope_group8(const float (&lo)[8], const float (&hi)[8], const float (&w_lo)[8],
                                                 const float (&w_hi)[8], const float eps, const float2 (&rot)[8],
                                                 float (&y_lo)[8], float (&y_hi)[8]) {
#pragma clang fp contract(off)
    double part[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const float a = lo[k] * lo[k], b = hi[k] * hi[k];
        part[k] = (double) a + (double) b;
    }
#pragma unroll
    for (int h = 4; h >= 1; h /= 2)
#pragma unroll
        for (int k = 0; k < h; ++k) part[k] += part[k + h];
    double sum = part[0];
    sum += __shfl_xor(sum, 1);
    sum += __shfl_xor(sum, 2);
    sum += __shfl_xor(sum, 4);
    const float mean = (float) (sum / 128.0);
    const float scale = 1.0f / sqrtf(mean + eps);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const float n0 = (lo[k] * scale) * w_lo[k], n1 = (hi[k] * scale) * w_hi[k];
        y_lo[k] = n0;
        y_hi[k] = n1;
        if constexpr (MODE != 0) {
            y_lo[k] = n0 * rot[k].x - n1 * rot[k].y;
            y_hi[k] = n0 * rot[k].y + n1 * rot[k].x;
        }
    }
}

// Both steps for one row.
template <int MODE>
__device__ __forceinline__ void norm_rope_pair(const float x0, const float x1, const bool has_w, const float w0,
                                               const float w1, const float eps, const RopeConsts & r,
                                               const int32_t pos, const int lane, float & y0, float & y1) {
    float c, s;
    rope_cos_sin<MODE>(r, pos, lane, c, s);
    norm_rope_apply<MODE>(x0, x1, has_w, w0, w1, eps, c, s, y0, y1);
}
