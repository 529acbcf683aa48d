/*
 * fattn_oracle.c - CPU oracle for ArcLight's flash-attention op.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py, as the reference results or the timed CPU baseline.
 * Nothing in the product path links or calls this file.
 *
 * Restated from (paths relative to the ArcLight tree):
 *   nnml/src/ops/arm/arm.cpp:2196-2433  nnml_compute_forward_flash_attn_ext_f16
 *   nnml/src/ops/arm/arm.cpp:286-386    nnml_vec_dot_f16 (O3 lane structure)
 *   nnml/src/ops/arm/arm.cpp:1453-1755  vec_scale / vec_mad f16 and f32
 *   nnml/src/ops/arm/common.cpp:11-24   f32 -> f16 row conversion
 *   nnml/include/ops.h:276-323          IEEE fp16 conversions (RNE)
 *   nnml/src/ops/ops.cpp:135-181        set_rows f32 -> f16
 *   nnml/src/tensor.cpp:1292-1338       operand preconditions
 *   nnml/src/ops/ops.cpp:680-726        rms_norm f32 (squares summed in double)
 *   nnml/src/ops/ops.cpp:728-777        rope_yarn, rotation cache, YaRN corr dims
 *   nnml/src/ops/ops.cpp:871-962        rope f32 (NEOX and normal pairs)
 *   nnml/src/ops/arm/arm.cpp:1819-1848  quantize_row_q8_0 (NEON: round to nearest even)
 *   nnml/src/ops/arm/arm.cpp:401-...    vec_dot_q4_0_q8_0 (scalar path)
 *   nnml/src/ops/arm/common.cpp:120-... forward_mul_mat_generic
 *
 * Pinning (tests/test_oracle_*.py): the fp16 conversions are compared bit
 * for bit with numpy's IEEE conversions over every f16 pattern and millions
 * of f32 patterns; O1 is compared with scipy.special.softmax attention; O2
 * with O1; all three with closed forms (single visible cell, equal scores,
 * dominant score, masked cells, all-masked rows, sinks, softcap, ALiBi slopes
 * from the ALiBi paper's construction), permutation invariance and
 * chunked-equals-one-shot causal prefill.
 */
#define _GNU_SOURCE 1
#include "fattn_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* fp16 <-> fp32, IEEE binary16, round to nearest even                 */
/* ------------------------------------------------------------------ */

static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t orc_f32_to_f16(float f) {
    const uint32_t x    = f32_bits(f);
    const uint16_t sign = (uint16_t) ((x >> 16) & 0x8000u);
    const uint32_t ax   = x & 0x7fffffffu;
    if (ax > 0x7f800000u) {           /* NaN: quiet NaN, as ops.h:322 */
        return sign | 0x7e00u;
    }
    if (ax >= 0x477ff000u) {          /* >= 65520 rounds to infinity */
        return sign | 0x7c00u;
    }
    const uint32_t e = ax >> 23;      /* biased f32 exponent */
    if (e < 113) {                    /* below 2^-14: f16 subnormal or zero */
        if (e < 102) {                /* below 2^-25: rounds to zero */
            return sign;
        }
        const uint32_t m     = (ax & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126 - e;          /* 14..24 */
        uint32_t q           = m >> shift;
        const uint32_t rem   = m & ((1u << shift) - 1u);
        const uint32_t half  = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) {
            q++;
        }
        return sign | (uint16_t) q;   /* q == 0x400 is the smallest normal */
    }
    uint32_t h         = ((e - 112) << 10) | ((ax & 0x7fffffu) >> 13);
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) {
        h++;                          /* a carry rolls into the exponent */
    }
    return sign | (uint16_t) h;
}

float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t) h & 0x8000u) << 16;
    const uint32_t e    = (h >> 10) & 0x1fu;
    uint32_t m          = h & 0x3ffu;
    if (e == 0x1f) {
        return bits_f32(sign | 0x7f800000u | (m << 13));
    }
    if (e == 0) {
        if (m == 0) {
            return bits_f32(sign);
        }
        /* subnormal: m * 2^-24, exact in f32 */
        const float v = (float) m * 0x1.0p-24f;
        return sign ? -v : v;
    }
    return bits_f32(sign | ((e + 112) << 23) | (m << 13));
}

void orc_f32_to_f16_n(const float * x, uint16_t * y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_f32_to_f16(x[i]);
}

void orc_f16_to_f32_n(const uint16_t * x, float * y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_f16_to_f32(x[i]);
}

/* f16 arithmetic of the ARM build, emulated: one rounding to f16 per op. */
static inline uint16_t h_fma(uint16_t acc, uint16_t a, uint16_t b) {
    const double r = (double) orc_f16_to_f32(a) * (double) orc_f16_to_f32(b) + (double) orc_f16_to_f32(acc);
    return orc_f32_to_f16((float) r);
}
static inline uint16_t h_add(uint16_t a, uint16_t b) {
    return orc_f32_to_f16(orc_f16_to_f32(a) + orc_f16_to_f32(b));
}
static inline uint16_t h_mul(uint16_t a, uint16_t b) {
    return orc_f32_to_f16(orc_f16_to_f32(a) * orc_f16_to_f32(b));
}

/* ------------------------------------------------------------------ */
/* operand checks (tensor.cpp:1292-1320, arm.cpp:2213-2245)             */
/* ------------------------------------------------------------------ */

typedef struct {
    const al_fattn_args * a;
    int64_t D, DV, T, Hq, B, n_kv, Hkv, Bk;
    int64_t rk2, rk3, rv2, rv3;
    int64_t kv_len;
    float scale, max_bias, softcap;
    float m0, m1;
    uint32_t n_head_log2;
    int nth;
    int mode;  /* 1 = O1, 2 = O2, 3 = O3 */
} job_t;

static int prepare(job_t * j, const al_fattn_args * a, int nth, int mode) {
    memset(j, 0, sizeof(*j));
    j->a = a;
    j->nth = nth < 1 ? 1 : nth;
    j->mode = mode;
    const al_tensor *q = &a->q, *k = &a->k, *v = &a->v, *d = &a->dst;
    if (!q->data || !k->data || !v->data || !d->data) return AL_ERR_INVALID;
    if (q->type != AL_TYPE_F32 || k->type != AL_TYPE_F16 || v->type != AL_TYPE_F16 || d->type != AL_TYPE_F32) {
        return AL_ERR_UNSUPPORTED;
    }
    j->D = k->ne[0]; j->DV = v->ne[0];
    j->T = q->ne[1]; j->Hq = q->ne[2]; j->B = q->ne[3];
    j->n_kv = k->ne[1]; j->Hkv = k->ne[2]; j->Bk = k->ne[3];
    if (q->ne[0] != j->D) return AL_ERR_INVALID;
    if (v->ne[1] != j->n_kv) return AL_ERR_INVALID;
    if (q->nb[0] != 4 || k->nb[0] != 2 || v->nb[0] != 2) return AL_ERR_INVALID;
    if (d->ne[0] != j->DV || d->ne[1] != j->Hq || d->ne[2] != j->T || d->ne[3] != j->B) return AL_ERR_INVALID;
    if (d->nb[0] != 4 || d->nb[0] > d->nb[1] || d->nb[1] > d->nb[2] || d->nb[2] > d->nb[3]) return AL_ERR_INVALID;
    if (j->Hkv <= 0 || j->Hq % j->Hkv != 0 || v->ne[2] <= 0 || j->Hq % v->ne[2] != 0) return AL_ERR_INVALID;
    if (j->Bk <= 0 || j->B % j->Bk != 0 || v->ne[3] <= 0 || j->B % v->ne[3] != 0) return AL_ERR_INVALID;
    j->rk2 = j->Hq / j->Hkv; j->rk3 = j->B / j->Bk;
    j->rv2 = j->Hq / v->ne[2]; j->rv3 = j->B / v->ne[3];
    if (a->mask.data) {
        const al_tensor * m = &a->mask;
        if (m->type != AL_TYPE_F16) return AL_ERR_UNSUPPORTED;
        const int64_t tpad = (j->T + 63) / 64 * 64;
        if (m->ne[0] < j->n_kv || m->ne[1] < tpad) return AL_ERR_INVALID;
        if (m->ne[2] <= 0 || m->ne[3] <= 0 || j->Hq % m->ne[2] != 0 || j->B % m->ne[3] != 0) return AL_ERR_INVALID;
        if (m->nb[0] != 2) return AL_ERR_INVALID;
    } else if (a->max_bias > 0.0f) {
        return AL_ERR_INVALID;  /* tensor.cpp:1305-1307 */
    }
    if (a->sinks.data) {
        if (a->sinks.type != AL_TYPE_F32 || a->sinks.ne[0] != j->Hq) return AL_ERR_INVALID;
    }
    if (a->prec != AL_PREC_DEFAULT && a->prec != AL_PREC_F32) return AL_ERR_INVALID;  /* ops.cpp:1441-1443 */
    j->kv_len = (a->kv_len <= 0 || a->kv_len > j->n_kv) ? j->n_kv : a->kv_len;

    j->scale = a->scale;
    j->max_bias = a->max_bias;
    j->softcap = a->logit_softcap;
    if (j->softcap != 0.0f) j->scale /= j->softcap;                       /* arm.cpp:2267-2269 */
    j->n_head_log2 = 1u << (uint32_t) floor(log2((double) j->Hq));        /* arm.cpp:2271 */
    j->m0 = powf(2.0f, -(j->max_bias) / j->n_head_log2);                   /* arm.cpp:2273 */
    j->m1 = powf(2.0f, -(j->max_bias / 2.0f) / j->n_head_log2);            /* arm.cpp:2274 */
    return AL_OK;
}

/* effective mask value for (token iq1, head iq2, stream iq3, cell ic) */
static inline float mask_value(const job_t * j, const uint16_t * mp, float slope, int64_t iq1, int64_t ic) {
    const al_fattn_args * a = j->a;
    if (ic >= j->kv_len) return -INFINITY;
    if (a->causal_pos0 >= 0 && ic > a->causal_pos0 + iq1) return -INFINITY;
    return mp ? slope * orc_f16_to_f32(mp[ic]) : 0.0f;                     /* arm.cpp:2327 */
}

/* ------------------------------------------------------------------ */
/* one query row, three numerics                                        */
/* ------------------------------------------------------------------ */

/* f16 -> f32 of 8 values by the F16C conversion (exact, as
   orc_f16_to_f32; the oracle is built for x86-64-v3, which has F16C). */
static inline __m256 h8_to_f32(const uint16_t * x) { return _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *) x)); }

static void row_o2_o3(const job_t * j, int64_t ir, float * VKQ32, uint16_t * VKQ16, uint16_t * Q_q) {
    const al_fattn_args * a = j->a;
    const int64_t T = j->T, Hq = j->Hq, D = j->D, DV = j->DV;
    const int64_t iq3 = ir / (Hq * T);                                      /* arm.cpp:2289-2291 */
    const int64_t iq2 = (ir - iq3 * Hq * T) / T;
    const int64_t iq1 = ir - iq3 * Hq * T - iq2 * T;
    const uint32_t h = (uint32_t) iq2;
    const float slope = (j->max_bias > 0.0f)
        ? (h < j->n_head_log2 ? powf(j->m0, (float) (h + 1)) : powf(j->m1, (float) (2 * (h - j->n_head_log2) + 1)))
        : 1.0f;                                                             /* arm.cpp:2294 */
    float S = 0.0f;
    float M = -INFINITY;
    const int f16acc = (j->mode == 3);
    if (f16acc) memset(VKQ16, 0, (size_t) DV * 2); else memset(VKQ32, 0, (size_t) DV * 4);

    const uint16_t * mp = NULL;
    if (a->mask.data) {
        const al_tensor * m = &a->mask;
        mp = (const uint16_t *) ((const char *) m->data + iq1 * m->nb[1] + (iq2 % m->ne[2]) * m->nb[2] + (iq3 % m->ne[3]) * m->nb[3]);
    }
    const int64_t ik3 = iq3 / j->rk3, ik2 = iq2 / j->rk2;
    const int64_t iv3 = iq3 / j->rv3, iv2 = iq2 / j->rv2;
    const float * pq = (const float *) ((const char *) a->q.data + iq1 * a->q.nb[1] + iq2 * a->q.nb[2] + iq3 * a->q.nb[3]);
    for (int64_t d = 0; d < D; ++d) Q_q[d] = orc_f32_to_f16(pq[d]);       /* arm.cpp:2322 */
    /* the f32 loops below in 8-wide registers when D and DV are multiples of
       8: the same per-lane products and sums (separate multiply and add, as
       the scalar form compiles under ISO C) and the same lane reduction */
    const int vec = (D % 8 == 0) && (DV % 8 == 0) && D <= 1024;
    float Qf[1024];
    if (vec) for (int64_t d = 0; d < D; ++d) Qf[d] = orc_f16_to_f32(Q_q[d]);

    for (int64_t ic = 0; ic < j->n_kv; ++ic) {
        const float mv = mask_value(j, mp, slope, iq1, ic);
        if (mv == -INFINITY) continue;                                      /* arm.cpp:2328-2330 */
        const uint16_t * kd = (const uint16_t *) ((const char *) a->k.data + ic * a->k.nb[1] + ik2 * a->k.nb[2] + ik3 * a->k.nb[3]);
        float s;
        if (!f16acc) {
            /* f32 lanes of width 8, then a pairwise lane reduction */
            float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            if (vec) {
                __m256 a8 = _mm256_setzero_ps();
                for (int64_t d = 0; d < D; d += 8) a8 = _mm256_add_ps(a8, _mm256_mul_ps(h8_to_f32(kd + d), _mm256_loadu_ps(Qf + d)));
                _mm256_storeu_ps(acc, a8);
            } else {
                for (int64_t d = 0; d < D; d += 8) {
                    for (int l = 0; l < 8 && d + l < D; ++l) acc[l] += orc_f16_to_f32(kd[d + l]) * orc_f16_to_f32(Q_q[d + l]);
                }
            }
            s = ((acc[0] + acc[4]) + (acc[2] + acc[6])) + ((acc[1] + acc[5]) + (acc[3] + acc[7]));
        } else {
            /* 4 accumulators x 8 f16 lanes, f16 FMA, f16 tree add, f32 horizontal add (arm.cpp:358-376, 89-124) */
            uint16_t sum[4][8];
            memset(sum, 0, sizeof(sum));
            const int64_t np = D & ~(int64_t) 31;
            for (int64_t i = 0; i < np; i += 32)
                for (int jj = 0; jj < 4; ++jj)
                    for (int l = 0; l < 8; ++l) sum[jj][l] = h_fma(sum[jj][l], kd[i + jj * 8 + l], Q_q[i + jj * 8 + l]);
            for (int l = 0; l < 8; ++l) { sum[0][l] = h_add(sum[0][l], sum[2][l]); sum[1][l] = h_add(sum[1][l], sum[3][l]); }
            for (int l = 0; l < 8; ++l) sum[0][l] = h_add(sum[0][l], sum[1][l]);
            float t[4];
            for (int l = 0; l < 4; ++l) t[l] = orc_f16_to_f32(sum[0][l]) + orc_f16_to_f32(sum[0][l + 4]);
            double sd = (double) ((t[0] + t[1]) + (t[2] + t[3]));
            for (int64_t i = np; i < D; ++i) sd += (double) (orc_f16_to_f32(kd[i]) * orc_f16_to_f32(Q_q[i]));
            s = (float) sd;
        }
        s = s * j->scale;                                                   /* arm.cpp:2337 */
        if (j->softcap != 0.0f) s = j->softcap * tanhf(s);                  /* arm.cpp:2339-2341 */
        s += mv;                                                            /* arm.cpp:2343 */

        const float Mold = M;
        float ms = 1.0f, vs = 1.0f;
        const uint16_t * vd = (const uint16_t *) ((const char *) a->v.data + ic * a->v.nb[1] + iv2 * a->v.nb[2] + iv3 * a->v.nb[3]);
        if (s > M) {                                                        /* arm.cpp:2352-2364 */
            M = s;
            ms = expf(Mold - M);
            if (f16acc) {
                const uint16_t hs = orc_f32_to_f16(ms);
                for (int64_t d = 0; d < DV; ++d) VKQ16[d] = h_mul(VKQ16[d], hs);
            } else {
                for (int64_t d = 0; d < DV; ++d) VKQ32[d] *= ms;
            }
        } else {
            vs = expf(s - M);
        }
        if (f16acc) {
            const uint16_t hv = orc_f32_to_f16(vs);                         /* arm.cpp:1735 */
            for (int64_t d = 0; d < DV; ++d) VKQ16[d] = h_fma(VKQ16[d], vd[d], hv);
        } else if (vec) {
            const __m256 vs8 = _mm256_set1_ps(vs);
            for (int64_t d = 0; d < DV; d += 8)                             /* arm.cpp:2385-2386 */
                _mm256_storeu_ps(VKQ32 + d, _mm256_add_ps(_mm256_loadu_ps(VKQ32 + d), _mm256_mul_ps(h8_to_f32(vd + d), vs8)));
        } else {
            for (int64_t d = 0; d < DV; ++d) VKQ32[d] += orc_f16_to_f32(vd[d]) * vs;   /* arm.cpp:2385-2386 */
        }
        S = S * ms + vs;                                                    /* arm.cpp:2392 */
    }
    if (f16acc) for (int64_t d = 0; d < DV; ++d) VKQ32[d] = orc_f16_to_f32(VKQ16[d]);  /* arm.cpp:2395-2399 */

    if (a->sinks.data) {                                                    /* arm.cpp:2402-2416 */
        const float s = ((const float *) a->sinks.data)[h];
        float ms = 1.0f, vs = 1.0f;
        if (s > M) {
            ms = expf(M - s);
            for (int64_t d = 0; d < DV; ++d) VKQ32[d] *= ms;
        } else {
            vs = expf(s - M);
        }
        S = S * ms + vs;
    }
    const float S_inv = 1.0f / S;                                           /* arm.cpp:2419-2420 */
    for (int64_t d = 0; d < DV; ++d) VKQ32[d] *= S_inv;
    /* permute(0, 2, 1, 3) store (arm.cpp:2431) */
    const int64_t ne1 = Hq, ne2 = T;
    memcpy((char *) a->dst.data + (iq3 * ne2 * ne1 + iq2 + iq1 * ne1) * a->dst.nb[1], VKQ32, (size_t) DV * 4);
}

static void row_o1(const job_t * j, int64_t ir, double * sc, double * acc, uint16_t * Q_q) {
    const al_fattn_args * a = j->a;
    const int64_t T = j->T, Hq = j->Hq, D = j->D, DV = j->DV;
    const int64_t iq3 = ir / (Hq * T);
    const int64_t iq2 = (ir - iq3 * Hq * T) / T;
    const int64_t iq1 = ir - iq3 * Hq * T - iq2 * T;
    const uint32_t h = (uint32_t) iq2;
    const double slope = (j->max_bias > 0.0f)
        ? (h < j->n_head_log2 ? pow((double) j->m0, (double) (h + 1)) : pow((double) j->m1, (double) (2 * (h - j->n_head_log2) + 1)))
        : 1.0;
    const uint16_t * mp = NULL;
    if (a->mask.data) {
        const al_tensor * m = &a->mask;
        mp = (const uint16_t *) ((const char *) m->data + iq1 * m->nb[1] + (iq2 % m->ne[2]) * m->nb[2] + (iq3 % m->ne[3]) * m->nb[3]);
    }
    const int64_t ik3 = iq3 / j->rk3, ik2 = iq2 / j->rk2;
    const int64_t iv3 = iq3 / j->rv3, iv2 = iq2 / j->rv2;
    const float * pq = (const float *) ((const char *) a->q.data + iq1 * a->q.nb[1] + iq2 * a->q.nb[2] + iq3 * a->q.nb[3]);
    for (int64_t d = 0; d < D; ++d) Q_q[d] = orc_f32_to_f16(pq[d]);
    double M = -INFINITY;
    for (int64_t ic = 0; ic < j->n_kv; ++ic) {
        double mv = 0.0;
        if (ic >= j->kv_len || (a->causal_pos0 >= 0 && ic > a->causal_pos0 + iq1)) mv = -INFINITY;
        else if (mp) {
            const double mval = (double) orc_f16_to_f32(mp[ic]);
            mv = (mval == -INFINITY) ? -INFINITY : slope * mval;
        }
        if (mv == -INFINITY) { sc[ic] = -INFINITY; continue; }
        const uint16_t * kd = (const uint16_t *) ((const char *) a->k.data + ic * a->k.nb[1] + ik2 * a->k.nb[2] + ik3 * a->k.nb[3]);
        double s = 0.0;
        for (int64_t d = 0; d < D; ++d) s += (double) orc_f16_to_f32(kd[d]) * (double) orc_f16_to_f32(Q_q[d]);
        s *= (double) j->scale;
        if (j->softcap != 0.0f) s = (double) j->softcap * tanh(s);
        s += mv;
        sc[ic] = s;
        if (s > M) M = s;
    }
    double sink = -INFINITY;
    if (a->sinks.data) {
        sink = (double) ((const float *) a->sinks.data)[h];
        if (sink > M) M = sink;
    }
    double S = 0.0;
    for (int64_t d = 0; d < DV; ++d) acc[d] = 0.0;
    for (int64_t ic = 0; ic < j->n_kv; ++ic) {
        if (sc[ic] == -INFINITY) continue;
        const double p = exp(sc[ic] - M);
        const uint16_t * vd = (const uint16_t *) ((const char *) a->v.data + ic * a->v.nb[1] + iv2 * a->v.nb[2] + iv3 * a->v.nb[3]);
        for (int64_t d = 0; d < DV; ++d) acc[d] += p * (double) orc_f16_to_f32(vd[d]);
        S += p;
    }
    if (a->sinks.data) S += exp(sink - M);
    float * out = (float *) ((char *) a->dst.data + (iq3 * T * Hq + iq2 + iq1 * Hq) * a->dst.nb[1]);
    for (int64_t d = 0; d < DV; ++d) out[d] = (float) (acc[d] / S);   /* S == 0: NaN, as the reference */
}

typedef struct { const job_t * j; int ith; } worker_t;

static void * worker(void * p) {
    const worker_t * w = (const worker_t *) p;
    const job_t * j = w->j;
    const int64_t nr = j->T * j->Hq * j->B;
    const int64_t dr = (nr + j->nth - 1) / j->nth;                        /* arm.cpp:2250-2257 */
    const int64_t ir0 = dr * w->ith;
    const int64_t ir1 = ir0 + dr < nr ? ir0 + dr : nr;
    const int64_t DD = j->D > j->DV ? j->D : j->DV;
    if (j->mode == 1) {
        double * sc = (double *) malloc((size_t) j->n_kv * sizeof(double));
        double * acc = (double *) malloc((size_t) DD * sizeof(double));
        uint16_t * Q_q = (uint16_t *) malloc((size_t) DD * 2);
        for (int64_t ir = ir0; ir < ir1; ++ir) row_o1(j, ir, sc, acc, Q_q);
        free(sc); free(acc); free(Q_q);
    } else {
        float * VKQ32 = (float *) malloc((size_t) DD * 4);
        uint16_t * VKQ16 = (uint16_t *) malloc((size_t) DD * 2);
        uint16_t * Q_q = (uint16_t *) malloc((size_t) DD * 2);
        for (int64_t ir = ir0; ir < ir1; ++ir) row_o2_o3(j, ir, VKQ32, VKQ16, Q_q);
        free(VKQ32); free(VKQ16); free(Q_q);
    }
    return NULL;
}

/* The reference's worker pool (nnml/src/scheduler.cpp:122-146): nth threads,
 * each running the op with its own ith. With cpus, thread i runs pinned to
 * logical CPU cpus[i] (thread 0 is the caller, pinned for the call only). */
static int run_on(const al_fattn_args * a, int n_threads, int mode, const int * cpus) {
    job_t j;
    const int rc = prepare(&j, a, n_threads, mode);
    if (rc != AL_OK) return rc;
    pthread_t * th = (pthread_t *) malloc(sizeof(pthread_t) * (size_t) j.nth);
    worker_t * ws = (worker_t *) malloc(sizeof(worker_t) * (size_t) j.nth);
    for (int i = 0; i < j.nth; ++i) { ws[i].j = &j; ws[i].ith = i; }
    cpu_set_t saved;
    int restore = 0;
    for (int i = 1; i < j.nth; ++i) {
        pthread_attr_t at;
        pthread_attr_init(&at);
        if (cpus) {
            cpu_set_t cs;
            CPU_ZERO(&cs);
            CPU_SET(cpus[i], &cs);
            pthread_attr_setaffinity_np(&at, sizeof(cs), &cs);
        }
        pthread_create(&th[i], &at, worker, &ws[i]);
        pthread_attr_destroy(&at);
    }
    if (cpus && pthread_getaffinity_np(pthread_self(), sizeof(saved), &saved) == 0) {
        cpu_set_t cs;
        CPU_ZERO(&cs);
        CPU_SET(cpus[0], &cs);
        restore = pthread_setaffinity_np(pthread_self(), sizeof(cs), &cs) == 0;
    }
    worker(&ws[0]);
    for (int i = 1; i < j.nth; ++i) pthread_join(th[i], NULL);
    if (restore) pthread_setaffinity_np(pthread_self(), sizeof(saved), &saved);
    free(th); free(ws);
    return AL_OK;
}

static int run(const al_fattn_args * a, int n_threads, int mode) { return run_on(a, n_threads, mode, NULL); }

int orc_fattn_o2(const al_fattn_args * a, int n_threads) { return run(a, n_threads, 2); }
int orc_fattn_o2_pinned(const al_fattn_args * a, int n_threads, const int * cpus) {
    return run_on(a, n_threads, 2, cpus);
}
int orc_fattn_o1(const al_fattn_args * a, int n_threads) { return run(a, n_threads, 1); }
int orc_fattn_o3(const al_fattn_args * a, int n_threads) { return run(a, n_threads, 3); }

/* set_rows f32 -> f16 (ops.cpp:135-181), single thread */
int orc_set_rows_f32_f16(const al_tensor * dst, const al_tensor * src, const al_tensor * idx) {
    if (src->type != AL_TYPE_F32 || dst->type != AL_TYPE_F16) return AL_ERR_UNSUPPORTED;
    if (idx->type != AL_TYPE_I64 && idx->type != AL_TYPE_I32) return AL_ERR_UNSUPPORTED;
    const int64_t nc = src->ne[0], nr = src->ne[1];
    if (dst->ne[0] != nc || dst->ne[2] != src->ne[2] || dst->ne[3] != src->ne[3]) return AL_ERR_INVALID;
    if (src->ne[2] % idx->ne[1] != 0 || src->ne[3] % idx->ne[2] != 0) return AL_ERR_INVALID;
    for (int64_t i03 = 0; i03 < src->ne[3]; ++i03)
        for (int64_t i02 = 0; i02 < src->ne[2]; ++i02)
            for (int64_t i = 0; i < nr; ++i) {
                const int64_t i12 = i03 % idx->ne[2], i11 = i02 % idx->ne[1];
                const char * ip = (const char *) idx->data + i * idx->nb[0] + i11 * idx->nb[1] + i12 * idx->nb[2];
                const int64_t i1 = idx->type == AL_TYPE_I64 ? *(const int64_t *) ip : (int64_t) *(const int32_t *) ip;
                if (i1 < 0 || i1 >= dst->ne[1]) return AL_ERR_INVALID;
                const float * s = (const float *) ((const char *) src->data + i * src->nb[1] + i02 * src->nb[2] + i03 * src->nb[3]);
                uint16_t * d = (uint16_t *) ((char *) dst->data + i1 * dst->nb[1] + i02 * dst->nb[2] + i03 * dst->nb[3]);
                for (int64_t c = 0; c < nc; ++c) d[c] = orc_f32_to_f16(s[c]);
            }
    return AL_OK;
}

/* ------------------------------------------------------------------ */
/* Attention-operand producers: RMSNorm, weight, rotary embedding      */
/* ------------------------------------------------------------------ */

/* YaRN correction dimension for a rotation count (ops.cpp:728-730). */
static float yarn_corr_dim(int n_dims, int n_ctx_orig, float n_rot, float base) {
    const double pi = 3.14159265358979323846;   /* M_PI */
    return n_dims * logf(n_ctx_orig / (n_rot * 2 * (float) pi)) / (2 * logf(base));
}

/* Rotation angle of pair index i0 / 2 and its cos / sin with the YaRN
 * extrapolation mix and magnitude correction (ops.cpp:743-760). */
static void yarn_cos_sin(float theta_extrap, float freq_scale, const float corr[2], int64_t i0, float ext_factor,
                         float mscale, float * c, float * s) {
    const float theta_interp = freq_scale * theta_extrap;
    float theta = theta_interp;
    if (ext_factor != 0.0f) {
        const float y = (float) (i0 / 2 - corr[0]) / fmaxf(0.001f, corr[1] - corr[0]);
        const float ramp = 1 - fminf(1, fmaxf(0, y));
        const float mix = ramp * ext_factor;
        theta = theta_interp * (1 - mix) + theta_extrap * mix;
        mscale *= 1.0f + 0.1f * logf(1.0f / freq_scale);
    }
    *c = cosf(theta) * mscale;
    *s = sinf(theta) * mscale;
}

int orc_rms_norm_rope_f32(const float * x, const float * w, const int32_t * pos, int64_t T, int64_t H, int64_t D,
                          float eps, const al_rope_params * rope, float * y) {
    if (D <= 0 || D % 2 != 0 || eps < 0.0f) return AL_ERR_INVALID;
    if (rope && (rope->n_dims != D || (rope->mode != AL_ROPE_NEOX && rope->mode != AL_ROPE_NORMAL))) return AL_ERR_UNSUPPORTED;
    float * cs = malloc(sizeof(float) * (size_t) D);
    if (!cs) return AL_ERR_INVALID;
    float corr[2] = {0, 0};
    float theta_scale = 1.0f;
    if (rope) {
        theta_scale = powf(rope->freq_base, -2.0f / rope->n_dims);
        const float start = floorf(yarn_corr_dim(rope->n_dims, rope->n_ctx_orig, rope->beta_fast, rope->freq_base));
        const float end = ceilf(yarn_corr_dim(rope->n_dims, rope->n_ctx_orig, rope->beta_slow, rope->freq_base));
        corr[0] = fmaxf(0, start);
        corr[1] = fminf(rope->n_dims - 1, end);
    }
    for (int64_t t = 0; t < T; ++t) {
        if (rope) {
            /* the rotation cache of this position: the angle is carried from
             * pair to pair by repeated multiplication (ops.cpp:762-772) */
            float theta = (float) pos[t];
            for (int64_t i0 = 0; i0 < D; i0 += 2) {
                yarn_cos_sin(theta, rope->freq_scale, corr, i0, rope->ext_factor, rope->attn_factor, &cs[i0], &cs[i0 + 1]);
                theta *= theta_scale;
            }
        }
        for (int64_t h = 0; h < H; ++h) {
            const float * xr = x + (t * H + h) * D;
            float * yr = y + (t * H + h) * D;
            /* RMSNorm: squares summed in double, scale in float (ops.cpp:700-722) */
            double sum = 0.0;
            for (int64_t i = 0; i < D; ++i) sum += (double) (xr[i] * xr[i]);
            const float mean = (float) (sum / D);
            const float scale = 1.0f / sqrtf(mean + eps);
            float * n = malloc(sizeof(float) * (size_t) D);
            if (!n) { free(cs); return AL_ERR_INVALID; }
            for (int64_t i = 0; i < D; ++i) {
                n[i] = xr[i] * scale;
                if (w) n[i] = n[i] * w[i];
            }
            if (!rope) {
                memcpy(yr, n, sizeof(float) * (size_t) D);
            } else if (rope->mode == AL_ROPE_NEOX) {
                const int64_t half = D / 2;
                for (int64_t ic = 0; ic < half; ++ic) {
                    const float c = cs[2 * ic], s = cs[2 * ic + 1];
                    const float x0 = n[ic], x1 = n[ic + half];
                    yr[ic] = x0 * c - x1 * s;
                    yr[ic + half] = x0 * s + x1 * c;
                }
            } else {
                for (int64_t i0 = 0; i0 < D; i0 += 2) {
                    const float c = cs[i0], s = cs[i0 + 1];
                    const float x0 = n[i0], x1 = n[i0 + 1];
                    yr[i0] = x0 * c - x1 * s;
                    yr[i0 + 1] = x0 * s + x1 * c;
                }
            }
            free(n);
        }
    }
    free(cs);
    return AL_OK;
}

/* ------------------------------------------------------------------ */
/* Q4_0 x Q8_0 matrix product (the WO projection)                       */
/* ------------------------------------------------------------------ */

void orc_quantize_row_q8_0(const float * x, orc_block_q8_0 * y, int64_t k) {
    for (int64_t b = 0; b < k / 32; ++b) {
        const float * xb = x + 32 * b;
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(xb[j]));
        const float d = amax / 127;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[b].d = orc_f32_to_f16(d);
        for (int j = 0; j < 32; ++j) y[b].qs[j] = (int8_t) nearbyintf(xb[j] * id);   /* ties to even */
    }
}

float orc_vec_dot_q4_0_q8_0(int64_t n, const orc_block_q4_0 * x, const orc_block_q8_0 * y) {
    float sumf = 0.0f;
    for (int64_t b = 0; b < n / 32; ++b) {
        int lo = 0, hi = 0;
        for (int j = 0; j < 16; ++j) {
            lo += ((x[b].qs[j] & 0x0F) - 8) * y[b].qs[j];
            hi += ((x[b].qs[j] >> 4) - 8) * y[b].qs[j + 16];
        }
        const int sumi = lo + hi;
        sumf += sumi * orc_f16_to_f32(x[b].d) * orc_f16_to_f32(y[b].d);
    }
    return sumf;
}

int orc_mul_mat_q4_0_f32(const void * w, int64_t K, int64_t N, const float * x, int64_t T, float * y) {
    if (K <= 0 || K % 32 != 0 || N <= 0 || T <= 0) return AL_ERR_INVALID;
    const int64_t nb = K / 32;
    orc_block_q8_0 * q = malloc(sizeof(orc_block_q8_0) * (size_t) (nb * T));
    if (!q) return AL_ERR_INVALID;
    for (int64_t t = 0; t < T; ++t) orc_quantize_row_q8_0(x + t * K, q + t * nb, K);
    const orc_block_q4_0 * wb = (const orc_block_q4_0 *) w;
    for (int64_t t = 0; t < T; ++t)
        for (int64_t r = 0; r < N; ++r) y[t * N + r] = orc_vec_dot_q4_0_q8_0(K, wb + r * nb, q + t * nb);
    free(q);
    return AL_OK;
}
