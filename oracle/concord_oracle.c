/*
 * concord_oracle.c -- CPU restatement of Concord's packed-weight linear path.
 *
 * TEST INFRASTRUCTURE ONLY (see concord_oracle.h).  Built by oracle/Makefile
 * into oracle/_build/libconcord_oracle.so; loaded by tests/ and by bench.py's
 * cpu_baseline leg through oracle/oracle.py.  The product never links it.
 *
 * Each function cites the reference function it restates (paths relative to
 * the reference repository root).  The op order inside every expression is
 * the reference's left-to-right Triton order; the numerical conventions the
 * reference leaves to its compiler are fixed in concord_oracle.h.
 */
/* FMA contraction is disabled by the build flags (-ffp-contract=off). */
#include "concord_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- int32 helpers with Triton's wrap-around semantics ------------------ */
static inline int32_t w_add(int32_t a, int32_t b) { return (int32_t)((uint32_t)a + (uint32_t)b); }
static inline int32_t w_sub(int32_t a, int32_t b) { return (int32_t)((uint32_t)a - (uint32_t)b); }
static inline int32_t w_mul(int32_t a, int32_t b) { return (int32_t)((uint32_t)a * (uint32_t)b); }
static inline int32_t w_shl(int32_t a, int s) { return (int32_t)((uint32_t)a << s); }
static inline int32_t a_shr(int32_t a, int s) { return a >> s; } /* arithmetic (gcc) */
static inline int32_t imin(int32_t a, int32_t b) { return a < b ? a : b; }
static inline int32_t imax(int32_t a, int32_t b) { return a > b ? a : b; }
static inline int32_t clampi(int32_t v, int32_t lo, int32_t hi) { return imin(imax(v, lo), hi); }

void oracle_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* float -> int32: truncation, saturation, NaN -> 0. */
int32_t oracle_f2i(float f) {
    if (f != f) return 0;
    if (f >= 2147483648.0f) return INT32_MAX;
    if (f < -2147483648.0f) return INT32_MIN;
    return (int32_t)f;
}

/* fp32 -> bf16, round to nearest even. */
uint16_t oracle_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0;
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7FFFu + lsb;
    return (uint16_t)(u >> 16);
}

static inline float bf16_to_f32(uint16_t h) {
    uint32_t u = ((uint32_t)h) << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* 2^e for any integer e (exact; denormal/0/inf outside the normal range). */
static inline float exp2i(int32_t e) {
    if (e > 300) e = 300;
    if (e < -300) e = -300;
    return ldexpf(1.0f, e);
}

/* ---- A3: the SR hash.  concord/packed_b.py:109-117 -------------------------
 * h = x ^ salt ^ pos; h ^= h<<13; h ^= h>>17 (arithmetic); h ^= h<<5;
 * h ^= h>>7 (arithmetic); u = (h & 0xFFFFFF) * 2^-24. */
float oracle_hash_uniform(int32_t x, int32_t pos, int32_t salt) {
    int32_t h = x ^ salt ^ pos;
    h = h ^ w_shl(h, 13);
    h = h ^ a_shr(h, 17);
    h = h ^ w_shl(h, 5);
    h = h ^ a_shr(h, 7);
    return (float)(h & 0xFFFFFF) * (1.0f / 16777216.0f);
}

/* stochastic-rounding tick: int(floor(d) + (u < d - floor(d))).
 * concord/packed_b.py:596-598 (same pattern at 625-627, 640-642, ...). */
static inline int32_t sr_tick(float d, float u) {
    float fl = floorf(d);
    float fr = d - fl;
    return oracle_f2i(fl + (u < fr ? 1.0f : 0.0f));
}

/* ---- A10: Philox4x32-10 as Triton's tl.rand uses it ----------------------
 * Salmon et al., "Parallel random numbers: as easy as 1, 2, 3" (SC'11);
 * round constants, key schedule and output mapping follow
 * triton/language/random.py:13-44 (philox_impl), 127-143
 * (uint_to_uniform_float), 147-157 (rand). */
void oracle_philox4x32_10(uint32_t c[4], uint32_t k[2]) {
    uint32_t k0 = k[0], k1 = k[1];
    for (int r = 0; r < 10; ++r) {
        uint64_t p0 = (uint64_t)0xD2511F53u * c[0];
        uint64_t p1 = (uint64_t)0xCD9E8D57u * c[2];
        uint32_t n0 = (uint32_t)(p1 >> 32) ^ c[1] ^ k0;
        uint32_t n1 = (uint32_t)p1;
        uint32_t n2 = (uint32_t)(p0 >> 32) ^ c[3] ^ k1;
        uint32_t n3 = (uint32_t)p0;
        c[0] = n0; c[1] = n1; c[2] = n2; c[3] = n3;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
}

/* tl.rand(seed, offset) for an int32 seed and an int32 offset block:
 * counter (offset, 0, 0, 0), key (seed_lo, seed_hi) with the seed
 * sign-extended to 64 bits, output word 0 mapped to [0,1). */
float oracle_tl_rand(int32_t seed, int32_t offset) {
    int64_t s64 = (int64_t)seed;
    uint32_t key[2] = {(uint32_t)((uint64_t)s64 & 0xFFFFFFFFu),
                       (uint32_t)(((uint64_t)s64 >> 32) & 0xFFFFFFFFu)};
    uint32_t ctr[4] = {(uint32_t)offset, 0u, 0u, 0u};
    oracle_philox4x32_10(ctr, key);
    int32_t x = (int32_t)ctr[0];
    if (x < 0) x = w_sub(-1, x);        /* -x - 1, wrapping */
    return (float)x * 4.6566127342e-10f;
}

/* ---- deterministic (v+eps)^p for p outside {0, 0.5} ----------------------
 * Not correctly rounded; a fixed sequence of IEEE ops so that the CPU and
 * the GPU agree bit for bit.  log2 by the atanh series on a mantissa in
 * [sqrt(1/2), sqrt(2)); exp2 by a degree-8 Taylor polynomial on [-1/2,1/2). */
static float det_log2(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    int32_t e = 0;
    if ((u & 0x7F800000u) == 0) {       /* denormal: scale by 2^23 */
        x = x * 8388608.0f;
        memcpy(&u, &x, 4);
        e = -23;
    }
    e += (int32_t)((u >> 23) & 0xFF) - 127;
    uint32_t mu = (u & 0x007FFFFFu) | 0x3F800000u;   /* m in [1,2) */
    float m;
    memcpy(&m, &mu, 4);
    if (m > 1.41421356f) { m = m * 0.5f; e += 1; }
    float t = (m - 1.0f) / (m + 1.0f);
    float t2 = t * t;
    float s = 1.0f / 11.0f;
    s = s * t2 + 1.0f / 9.0f;
    s = s * t2 + 1.0f / 7.0f;
    s = s * t2 + 1.0f / 5.0f;
    s = s * t2 + 1.0f / 3.0f;
    s = s * t2 + 1.0f;
    float ln_m = 2.0f * t * s;
    return (float)e + ln_m * 1.44269504f;
}

static float det_exp2(float y) {
    if (y != y) return y;
    if (y >= 128.0f) return INFINITY;
    if (y < -150.0f) return 0.0f;
    float n = floorf(y + 0.5f);
    float f = y - n;                      /* [-0.5, 0.5] */
    float z = f * 0.693147181f;
    float p = 1.0f / 40320.0f;
    p = p * z + 1.0f / 5040.0f;
    p = p * z + 1.0f / 720.0f;
    p = p * z + 1.0f / 120.0f;
    p = p * z + 1.0f / 24.0f;
    p = p * z + 1.0f / 6.0f;
    p = p * z + 0.5f;
    p = p * z + 1.0f;
    p = p * z + 1.0f;
    int32_t ni = (int32_t)n;
    /* two-step scaling keeps the result exact into the denormal range */
    int32_t a = ni / 2, b = ni - a;
    return (p * exp2i(a)) * exp2i(b);
}

float oracle_pow_p(float x, float p) {
    if (p == 0.5f) return sqrtf(x);
    if (p == 0.0f) return 1.0f;
    return det_exp2(p * det_log2(x));
}

/* ---- A2: concord/packed_b.py:52-102 ------------------------------------- */
double oracle_drift_cancel_C(double alpha, double alpha_v_fast,
                             double alpha_v_slow, int refit_period,
                             int mass_preserve) {
    double L = (1.0 - alpha) / (alpha > 1e-12 ? alpha : 1e-12);
    double rho = alpha_v_fast + alpha_v_slow / (double)(refit_period > 1 ? refit_period : 1);
    if (mass_preserve) {
        double rho2 = 2.0 * rho;
        return L * rho2 / (1.0 - rho2);
    }
    return L * rho / (1.0 - L * alpha_v_fast);
}

/* ---- A1 unpack ----------------------------------------------------------
 * concord/packed_b.py:143-147: sf = w>>16, ss = (w<<16)>>24, vs = (w<<24)>>24 */
static inline void unpack(int32_t w, int32_t* sf, int32_t* ss, int32_t* vs) {
    *sf = a_shr(w, 16);
    *ss = a_shr(w_shl(w, 16), 24);
    *vs = a_shr(w_shl(w, 24), 24);
}

/* concord/packed_b.py:674-678 */
static inline int32_t pack(int32_t sf, int32_t ss, int32_t vs) {
    return (int32_t)((((uint32_t)sf & 0xFFFFu) << 16) | (((uint32_t)ss & 0xFFu) << 8) |
                     ((uint32_t)vs & 0xFFu));
}

/* ---- A8 / A9: materialize (concord/packed_b.py:120-155) and
 * consolidated_weight (1632-1649): bf16(float(m) * 2^(r + c - bias)),
 * m = 128 ss + sf + 128 vs (live) or 128 ss + 128 vs (consolidated). */
void oracle_materialize(const int32_t* packed, const int8_t* row_exp,
                        const int8_t* col_exp, int64_t N, int64_t K,
                        int32_t mantissa_bias, int consolidated,
                        uint16_t* out) {
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t k = 0; k < K; ++k) {
            int32_t sf, ss, vs;
            unpack(packed[n * K + k], &sf, &ss, &vs);
            int32_t m = consolidated ? w_add(w_mul(ss, 128), w_mul(vs, 128))
                                     : w_add(w_add(w_mul(ss, 128), sf), w_mul(vs, 128));
            float sc = exp2i((int32_t)row_exp[n] + (int32_t)col_exp[k] - mantissa_bias);
            out[n * K + k] = oracle_f32_to_bf16((float)m * sc);
        }
    }
}

/* concord/packed_b.py:1763-1772 (fast_gain < 1): m_gated = (ss*128 + fg*sf +
 * vs*128) * exp2(exp) in float32, left to right, then .to(bfloat16) */
void oracle_materialize_gated(const int32_t* packed, const int8_t* row_exp,
                              const int8_t* col_exp, int64_t N, int64_t K,
                              int32_t mantissa_bias, float fast_gain,
                              uint16_t* out) {
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t k = 0; k < K; ++k) {
            int32_t sf, ss, vs;
            unpack(packed[n * K + k], &sf, &ss, &vs);
            const float m = ((float)(ss * 128) + fast_gain * (float)sf) + (float)(vs * 128);
            const float sc = exp2i((int32_t)row_exp[n] + (int32_t)col_exp[k] - mantissa_bias);
            out[n * K + k] = oracle_f32_to_bf16(m * sc);
        }
    }
}

/* ---- A4: the packed optimizer update --------------------------------------
 * Canonical: concord/packed_b.py:422-703 (_apply_packed_adamw_kernel).
 * With OR_PROTO_CONSF: notebook/src/prototype_packed_b.py:454-778 (consf
 * gating, coherence-gated beta1, v-hat bias-correction factor, device floors).
 * With OR_MUON: docs/MUON_IMPLEMENTATION.md:87-119 (step = supplied drive,
 * no denominator, no clip).  The gap-feedback branch of the prototype is not
 * restated (experimental, off by default, absent from packed_b.py). */
void oracle_apply_adamw(int32_t* packed, const uint16_t* grad_bf16,
                        uint16_t* weight_bf16, const int8_t* row_exp,
                        const int8_t* col_exp, int32_t* row_max,
                        int32_t* col_max, const float* v_row,
                        const float* v_col, float sum_v_inv, float* coh_pre,
                        int64_t N, int64_t K, const oracle_update_params* P,
                        const oracle_update_scalars* S, uint32_t flags) {
    const int proto = (flags & OR_PROTO_CONSF) != 0;
    const int32_t cons = proto ? S->consolidate : 1;
    const float consf = (float)cons;
    const float lr = S->lr, eps = S->eps;
    const int32_t salt = S->salt;
    /* v-hat only feeds the trust-region denominator (not under the Muon
     * drive) and the non-fixed coherence gate; otherwise it is not read
     * (docs/MUON_IMPLEMENTATION.md:75-80) and v_row / v_col may be NULL */
    const int need_vhat = ((flags & OR_GF_TRUST_REGION) && !(flags & OR_MUON)) ||
                          (!(flags & OR_FIXED_COH) &&
                           (flags & (OR_GF_CONSOLIDATION | OR_COHPRE | OR_RATIO_COH)));
    const int need_coh = (flags & (OR_GF_CONSOLIDATION | OR_COHPRE | OR_RATIO_COH)) != 0;
    const int track = (flags & OR_TRACK_REBALANCE) != 0 && cons == 1;
    const int emit = (flags & OR_EMIT_WEIGHT) != 0 && cons == 1;

    int32_t* cmax_local = NULL;
#pragma omp parallel
    {
        int32_t* cm = (int32_t*)calloc((size_t)K, sizeof(int32_t));
#pragma omp for schedule(static)
        for (int64_t n = 0; n < N; ++n) {
            int32_t rmax = 0;
            for (int64_t k = 0; k < K; ++k) {
                const int64_t o = n * K + k;
                int32_t sf, ss, vs;
                unpack(packed[o], &sf, &ss, &vs);
                const int32_t ssf = w_mul(ss, 128), vsf = w_mul(vs, 128);
                const float g = bf16_to_f32(grad_bf16[o]);
                const int32_t te = (int32_t)row_exp[n] + (int32_t)col_exp[k] - P->mantissa_bias;
                const float scale_fwd = exp2i(te);
                const float scale_inv = exp2i(-te);

                const float d_fs = (float)sf;
                const float d_sv = (float)w_sub(ssf, vsf);
                const float noise = d_fs - P->drift_cancel_C * d_sv;
                const float nw = noise * scale_fwd;
                float v_proxy = nw * nw * P->v_scale;
                float v_hat = 0.0f, coh = 0.0f;
                if (need_vhat) {
                    v_hat = v_row[n] * v_col[k] * sum_v_inv;
                    if (proto) v_hat = v_hat * S->v_bc;
                }
                if (flags & OR_GF_TRUST_REGION) v_proxy = v_proxy + P->gf_trust_delta_sq * v_hat;
                if (need_coh) {
                    if (flags & OR_FIXED_COH) {
                        const float sig_w = P->drift_cancel_C * d_sv * scale_fwd;
                        const float sig2 = sig_w * sig_w;
                        coh = sig2 / (sig2 + nw * nw + 1e-30f);
                    } else {
                        const float mg = P->alpha_v_fast * d_sv * scale_fwd;
                        coh = mg * mg / (v_hat + 1e-12f);
                    }
                    coh = fminf(fmaxf(coh, 0.0f), 1.0f);
                }
                float step_live;
                if (flags & OR_MUON) {
                    step_live = g;
                } else {
                    const float denom = oracle_pow_p(v_proxy + eps, P->precond_p);
                    step_live = g / denom;
                    step_live = fminf(fmaxf(step_live, -P->step_cap), P->step_cap);
                }
                const float sf_in_w = d_fs * scale_fwd;
                float evap;
                if (flags & OR_GF_CONSOLIDATION) {
                    evap = lr * P->gf_consol * (1.0f - coh) * d_fs;
                } else {
                    step_live = step_live + P->weight_decay * sf_in_w;
                    evap = 0.0f;
                }
                const float delta_grad = -lr * step_live * scale_inv;
                float delta_t;
                if (proto)
                    delta_t = delta_grad + consf * (P->beta1 * coh * d_fs - evap);
                else
                    delta_t = delta_grad - P->beta1 * d_fs - evap;

                const int32_t pos = w_shl((int32_t)n, 16) ^ (int32_t)k;
                sf = w_add(sf, sr_tick(delta_t, oracle_hash_uniform(sf, pos, salt)));

                int32_t new_v = vs;
                if (flags & OR_APPLY_CHASE) {
                    float gate = 1.0f;
                    if (flags & OR_RATIO_COH) {
                        gate = S->chase_floor + (1.0f - S->chase_floor) * coh;
                    } else if (flags & OR_COHPRE) {
                        const float cp = coh_pre[o];
                        gate = coh + cp * (1.0f - coh);
                        coh_pre[o] = (1.0f - P->alpha_v_fast) * cp + P->alpha_v_fast * coh;
                    }
                    float chase = P->alpha * gate * P->gate_gain * (float)sf;
                    if (proto) chase = chase * consf;
                    const float c8 = chase / 128.0f;
                    const int32_t t2 = sr_tick(c8, oracle_hash_uniform(sf, pos, salt ^ 0x5A5A5A5A));
                    ss = w_add(ss, t2);
                    sf = w_sub(sf, w_mul(t2, 128));

                    const float gap = (float)w_sub(w_mul(ss, 128), vsf);
                    float dv8 = P->alpha_v_fast * gap / 128.0f;
                    if (proto) dv8 = dv8 * consf;
                    if (flags & OR_RATIO_COH)
                        dv8 = dv8 * (S->leak_floor + (1.0f - S->leak_floor) * coh);
                    const int32_t t3 = sr_tick(dv8, oracle_hash_uniform(sf, pos, salt ^ 0x33335555));
                    new_v = clampi(w_add(vs, t3), -128, 127);
                    if (flags & OR_MASS_PRESERVE) ss = w_sub(ss, w_sub(new_v, vs));

                    const int32_t vpost = w_mul(new_v, 128);
                    const float dsv_post = (float)w_sub(w_mul(ss, 128), vpost);
                    float wdsv = lr * P->wd_sv * dsv_post / 128.0f;
                    if (proto) wdsv = wdsv * consf;
                    const int32_t t4 = sr_tick(wdsv, oracle_hash_uniform(sf, pos, salt ^ 0x66665555));
                    ss = w_sub(ss, t4);

                    const int32_t sfl = w_add(w_mul(ss, 128), sf);
                    const float dsf = (float)w_sub(sfl, vpost);
                    float wdsf = lr * P->wd_sf * dsf;
                    if (proto) wdsf = wdsf * consf;
                    const int32_t t5 = sr_tick(wdsf, oracle_hash_uniform(sf, pos, salt ^ 0x77770000));
                    sf = w_sub(sf, t5);
                }
                const int32_t sfc = clampi(sf, -32768, 32767);
                const int32_t ssc = clampi(ss, -128, 127);
                packed[o] = pack(sfc, ssc, new_v);
                const int32_t m_new = w_add(w_add(w_mul(ssc, 128), sfc), w_mul(new_v, 128));
                if (emit) weight_bf16[o] = oracle_f32_to_bf16((float)m_new * scale_fwd);
                if (track) {
                    const int32_t a = m_new < 0 ? -m_new : m_new;
                    if (a > rmax) rmax = a;
                    if (a > cm[k]) cm[k] = a;
                }
            }
            if (track && rmax > row_max[n]) row_max[n] = rmax;
        }
        if (track) {
#pragma omp critical
            {
                for (int64_t k = 0; k < K; ++k)
                    if (cm[k] > col_max[k]) col_max[k] = cm[k];
            }
        }
        free(cm);
    }
    (void)cmax_local;
}

/* ---- SGD path: concord/packed_b.py:173-312 (_apply_packed_sgd_kernel) --- */
void oracle_apply_sgd(int32_t* packed, const uint16_t* grad_bf16,
                      uint16_t* weight_bf16, const int8_t* row_exp,
                      const int8_t* col_exp, int32_t* row_max,
                      int32_t* col_max, int64_t N, int64_t K, float lr,
                      int32_t mantissa_bias, float alpha, float beta1,
                      float alpha_v_fast, int32_t salt, uint32_t flags) {
    const int track = (flags & OR_TRACK_REBALANCE) != 0;
    const int emit = (flags & OR_EMIT_WEIGHT) != 0;
#pragma omp parallel
    {
        int32_t* cm = (int32_t*)calloc((size_t)K, sizeof(int32_t));
#pragma omp for schedule(static)
        for (int64_t n = 0; n < N; ++n) {
            int32_t rmax = 0;
            for (int64_t k = 0; k < K; ++k) {
                const int64_t o = n * K + k;
                int32_t sf, ss, vs;
                unpack(packed[o], &sf, &ss, &vs);
                const float g = bf16_to_f32(grad_bf16[o]);
                const int32_t te = (int32_t)row_exp[n] + (int32_t)col_exp[k] - mantissa_bias;
                const float scale_inv = exp2i(-te);
                const float delta_grad = -lr * g * scale_inv;
                const float delta_t = delta_grad - beta1 * (float)sf;
                const int32_t pos = w_shl((int32_t)n, 16) ^ (int32_t)k;
                sf = w_add(sf, sr_tick(delta_t, oracle_hash_uniform(sf, pos, salt)));
                const float c8 = alpha * (float)sf / 128.0f;
                const int32_t t2 = sr_tick(c8, oracle_hash_uniform(sf, pos, salt ^ 0x5A5A5A5A));
                ss = w_add(ss, t2);
                sf = w_sub(sf, w_mul(t2, 128));
                const float gap = (float)w_sub(w_mul(ss, 128), w_mul(vs, 128));
                const float dv8 = alpha_v_fast * gap / 128.0f;
                const int32_t t3 = sr_tick(dv8, oracle_hash_uniform(sf, pos, salt ^ 0x33335555));
                const int32_t new_v = clampi(w_add(vs, t3), -128, 127);
                if (flags & OR_MASS_PRESERVE) ss = w_sub(ss, w_sub(new_v, vs));
                const int32_t sfc = clampi(sf, -32768, 32767);
                const int32_t ssc = clampi(ss, -128, 127);
                packed[o] = pack(sfc, ssc, new_v);
                const int32_t m_new = w_add(w_add(w_mul(ssc, 128), sfc), w_mul(new_v, 128));
                if (emit) weight_bf16[o] = oracle_f32_to_bf16((float)m_new * exp2i(te));
                if (track) {
                    const int32_t a = m_new < 0 ? -m_new : m_new;
                    if (a > rmax) rmax = a;
                    if (a > cm[k]) cm[k] = a;
                }
            }
            if (track && rmax > row_max[n]) row_max[n] = rmax;
        }
        if (track) {
#pragma omp critical
            {
                for (int64_t k = 0; k < K; ++k)
                    if (cm[k] > col_max[k]) col_max[k] = cm[k];
            }
        }
        free(cm);
    }
}

/* ---- medians of max(|ss|, |vs|) per row / column ---------------------------
 * concord/packed_b.py:1156-1160 (torch.median: the lower middle element). */
void oracle_i8_medians(const int32_t* packed, int64_t N, int64_t K,
                       int32_t* row_med, int32_t* col_med) {
    int64_t* ch = (int64_t*)calloc((size_t)K * 129, sizeof(int64_t));
    for (int64_t n = 0; n < N; ++n) {
        int64_t rh[129];
        memset(rh, 0, sizeof(rh));
        for (int64_t k = 0; k < K; ++k) {
            int32_t sf, ss, vs;
            unpack(packed[n * K + k], &sf, &ss, &vs);
            int32_t a = imax(ss < 0 ? -ss : ss, vs < 0 ? -vs : vs);
            rh[a]++;
            ch[k * 129 + a]++;
        }
        int64_t target = (K - 1) / 2, acc = 0;
        for (int v = 0; v < 129; ++v) {
            acc += rh[v];
            if (acc > target) { row_med[n] = v; break; }
        }
    }
    for (int64_t k = 0; k < K; ++k) {
        int64_t target = (N - 1) / 2, acc = 0;
        for (int v = 0; v < 129; ++v) {
            acc += ch[k * 129 + v];
            if (acc > target) { col_med[k] = v; break; }
        }
    }
    free(ch);
}

/* ---- A10 rebalance: concord/packed_b.py:959-1095 ------------------------- */
void oracle_rebalance(int32_t* packed, int8_t* row_exp, int8_t* col_exp,
                      const int32_t* row_max, const int32_t* col_max,
                      const int32_t* row_med, const int32_t* col_med,
                      int64_t N, int64_t K, int32_t max_m, int32_t exp_max,
                      int32_t exp_min, int32_t seed, int allow_tickdown) {
    int32_t* rt = (int32_t*)malloc((size_t)N * sizeof(int32_t));
    int32_t* ct = (int32_t*)malloc((size_t)K * sizeof(int32_t));
    for (int64_t n = 0; n < N; ++n) {
        int up = row_max[n] > max_m && row_exp[n] < exp_max;
        int dn = allow_tickdown && row_max[n] <= max_m && row_med[n] <= 31 && row_exp[n] > exp_min;
        rt[n] = up - dn;
    }
    for (int64_t k = 0; k < K; ++k) {
        int up = col_max[k] > max_m && col_exp[k] < exp_max;
        int dn = allow_tickdown && col_max[k] <= max_m && col_med[k] <= 31 && col_exp[k] > exp_min;
        ct[k] = up - dn;
    }
    const int32_t nk = w_mul((int32_t)N, (int32_t)K);
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t k = 0; k < K; ++k) {
            const int32_t net = rt[n] + ct[k];
            if (net == 0) continue;   /* rsh = lsh = 0: the word is unchanged */
            const int64_t o = n * K + k;
            int32_t sf, ss, vs;
            unpack(packed[o], &sf, &ss, &vs);
            int32_t sfn, ssn, vn;
            if (net < 0) {
                const int lsh = -net;
                sfn = w_shl(sf, lsh);
                ssn = w_shl(ss, lsh);
                vn = w_shl(vs, lsh);
            } else {
                const int rsh = net;
                const float two_pos = (float)(1 << rsh);
                const int32_t off = w_add(w_mul((int32_t)n, (int32_t)K), (int32_t)k);
                int32_t q = a_shr(sf, rsh);
                float rem = (float)w_sub(sf, w_shl(q, rsh));
                int32_t sfs = q + ((oracle_tl_rand(seed, off) * two_pos < rem) ? 1 : 0);
                q = a_shr(ss, rsh);
                rem = (float)w_sub(ss, w_shl(q, rsh));
                const int32_t ssu = q + ((oracle_tl_rand(seed, w_add(off, nk)) * two_pos < rem) ? 1 : 0);
                const int32_t ssr = w_sub(w_shl(ss, 7 - rsh), w_shl(ssu, 7));
                q = a_shr(vs, rsh);
                rem = (float)w_sub(vs, w_shl(q, rsh));
                const int32_t vu = q + ((oracle_tl_rand(seed, w_add(off, w_mul(2, nk))) * two_pos < rem) ? 1 : 0);
                const int32_t vr = w_sub(w_shl(vs, 7 - rsh), w_shl(vu, 7));
                sfn = w_add(w_add(sfs, ssr), vr);
                ssn = ssu;
                vn = vu;
            }
            packed[o] = pack(clampi(sfn, -32768, 32767), clampi(ssn, -128, 127), clampi(vn, -128, 127));
        }
    }
    for (int64_t n = 0; n < N; ++n) row_exp[n] = (int8_t)(row_exp[n] + rt[n]);
    for (int64_t k = 0; k < K; ++k) col_exp[k] = (int8_t)(col_exp[k] + ct[k]);
    free(rt);
    free(ct);
}

/* ---- A5 v-hat EMA: concord/packed_b.py:1288-1303 ---------------------------
 * g2 = f32(grad)^2; v_row = b2*v_row + (1-b2)*sum_k g2; v_col likewise;
 * sum_v_inv = 1 / max(sum_n v_row, 1e-30).
 * Reduction order (this build's definition; the reference leaves it to torch).
 * The grad is cut into 64 x 64 tiles (zeros past N and K); inside a tile,
 * with g2[r][c] for tile row r and column c:
 *   row partial of row r (P_r[col tile][n]):
 *     s(y, q) = ((g2[r][16y+4q] + g2[r][16y+4q+1]) + g2[r][16y+4q+2]) + g2[r][16y+4q+3]
 *     u(q)    = ((s(0,q) + s(1,q)) + s(2,q)) + s(3,q)
 *     P       = (u(0) + u(1)) + (u(2) + u(3))
 *   column partial of column c (P_c[row tile][k]):
 *     w(p) = ((g2[p][c] + g2[16+p][c]) + g2[32+p][c]) + g2[48+p][c], p = 0..15
 *     u1(p) = w(p) + w(p+8), p < 8;  u2(p) = u1(p) + u1(p+4), p < 4;
 *     u3(p) = u2(p) + u2(p+2), p < 2;  P = u3(0) + u3(1)
 *   g2_row[n] = sum over column tiles ascending of P_r, from 0.0f; g2_col[k]
 *   likewise over row tiles;
 *   sum_v: per block of 256 rows the halving tree s_t += s_{t+h}, h = 128 ..
 *   1, over v_row (zeros past N); then the block totals ascending from 0.0f.
 * (The GPU forms these partials in the wgrad epilogue from the MFMA
 * accumulator layout: lane (p, q) of a wave holds tile rows 16x+p, columns
 * 16y+4q..16y+4q+3.) */
static float vh_row_tile(const float* g2r /* 64 values */) {
    float u[4];
    for (int q = 0; q < 4; ++q) {
        float acc = 0.0f;
        for (int y = 0; y < 4; ++y) {
            const float* v = g2r + 16 * y + 4 * q;
            const float s = ((v[0] + v[1]) + v[2]) + v[3];
            acc = y == 0 ? s : acc + s;
        }
        u[q] = acc;
    }
    return (u[0] + u[1]) + (u[2] + u[3]);
}

static float vh_col_tile(const float* g2c /* 64 values, one per tile row */) {
    float w[16], u1[8], u2[4], u3[2];
    for (int p = 0; p < 16; ++p) w[p] = ((g2c[p] + g2c[16 + p]) + g2c[32 + p]) + g2c[48 + p];
    for (int p = 0; p < 8; ++p) u1[p] = w[p] + w[p + 8];
    for (int p = 0; p < 4; ++p) u2[p] = u1[p] + u1[p + 4];
    for (int p = 0; p < 2; ++p) u3[p] = u2[p] + u2[p + 2];
    return u3[0] + u3[1];
}

void oracle_vhat_ema(const uint16_t* grad_bf16, int64_t N, int64_t K,
                     float* v_row, float* v_col, float* sum_v_inv,
                     double beta2) {
    const float b2 = (float)beta2;
    const float omb2 = (float)(1.0 - beta2);
    const int64_t nc = (K + 63) / 64, nr = (N + 63) / 64;
    float* pr = (float*)malloc((size_t)(nc * N) * sizeof(float));
    float* pc = (float*)malloc((size_t)(nr * K) * sizeof(float));
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < nr * nc; ++t) {
        const int64_t n0 = (t / nc) * 64, k0 = (t % nc) * 64;
        float g2[64][64];
        for (int r = 0; r < 64; ++r)
            for (int c = 0; c < 64; ++c) {
                const int64_t n = n0 + r, k = k0 + c;
                float g = (n < N && k < K) ? bf16_to_f32(grad_bf16[n * K + k]) : 0.0f;
                g2[r][c] = g * g;
            }
        for (int r = 0; r < 64 && n0 + r < N; ++r) pr[(k0 / 64) * N + n0 + r] = vh_row_tile(g2[r]);
        for (int c = 0; c < 64 && k0 + c < K; ++c) {
            float col[64];
            for (int r = 0; r < 64; ++r) col[r] = g2[r][c];
            pc[(n0 / 64) * K + k0 + c] = vh_col_tile(col);
        }
    }
    for (int64_t n = 0; n < N; ++n) {
        float s = 0.0f;
        for (int64_t c = 0; c < nc; ++c) s = s + pr[c * N + n];
        v_row[n] = v_row[n] * b2 + omb2 * s;
    }
    for (int64_t k = 0; k < K; ++k) {
        float s = 0.0f;
        for (int64_t r = 0; r < nr; ++r) s = s + pc[r * K + k];
        v_col[k] = v_col[k] * b2 + omb2 * s;
    }
    float total = 0.0f;
    for (int64_t b0 = 0; b0 < N; b0 += 256) {
        float part[256];
        for (int t = 0; t < 256; ++t) part[t] = (b0 + t < N) ? v_row[b0 + t] : 0.0f;
        for (int h = 128; h >= 1; h >>= 1)
            for (int t = 0; t < h; ++t) part[t] = part[t] + part[t + h];
        total = total + part[0];
    }
    const float sv = fmaxf(total, 1e-30f);
    *sum_v_inv = 1.0f / sv;
    free(pr);
    free(pc);
}

/* The block totals of the fixed-order sums below (and of the GPU's
 * wave_tree_sum): lane l (0..63) adds totals l, l+64, ... ascending from 0.0f,
 * then the halving tree over the 64 lane sums. */
static float lane_tree_sum(const float* v, int64_t n) {
    float lane[64];
    for (int l = 0; l < 64; ++l) lane[l] = 0.0f;
    for (int64_t i = 0; i < n; ++i) lane[i % 64] = lane[i % 64] + v[i];
    for (int h = 32; h >= 1; h >>= 1)
        for (int l = 0; l < h; ++l) lane[l] = lane[l] + lane[l + h];
    return lane[0];
}

/* ---- A13 Muon drive: experiments/cpu_dynamics/exp9_muon.py:44-55 (ns5),
 * 58-100 (MuonConcord.step: drive = sqrt(max(N,K)) * ns5(g / ||g||));
 * docs/MUON_IMPLEMENTATION.md:27-40 (bf16 NS, O fed to the apply as the step).
 * This build's numerics (the GPU path follows them):
 *   ||g||^2: the row-major flattening of g cut into blocks of 8192 elements;
 *     in a block, lane t (0..255) sums elements t, t+256, ... (32 of them)
 *     ascending from 0.0f, then the halving tree over the 256 lane sums.  The
 *     block totals: lane l (0..63) sums totals l, l+64, ... ascending from
 *     0.0f, then the halving tree over the 64 lane sums.  norm = sqrtf(sum).
 *   X0 = bf16(g / (n * (norm / n + 1e-7))), n = max(norm, 1e-12), transposed when N > K so
 *   X is m x n, m <= n.
 *   per iteration (a, b, c = 3.4445, -4.7750, 2.0315):
 *     A = bf16(X X^T), AA = bf16(A A), B = bf16(b A + c AA), BX = bf16(B X),
 *     X = bf16(a X + BX); the products accumulate in fp32 over ascending r.
 *   out = bf16(gamma * X), transposed back to N x K.
 * The GPU's products accumulate in MFMA order, so GPU and oracle agree to the
 * bf16 rounding of the products, not bit for bit; the norm and X0 are exact. */
float oracle_frob_sumsq(const uint16_t* g, int64_t N, int64_t K) {
    const int64_t total = N * K, nb = (total + 8191) / 8192;
    float* bt = (float*)malloc((size_t)(nb > 0 ? nb : 1) * sizeof(float));
    for (int64_t b = 0; b < nb; ++b) {
        const int64_t b0 = b * 8192;
        float part[256];
        for (int t = 0; t < 256; ++t) {
            float s = 0.0f;
            for (int i = 0; i < 32; ++i) {
                const int64_t e = b0 + t + 256 * i;
                float v = e < total ? bf16_to_f32(g[e]) : 0.0f;
                s = s + v * v;
            }
            part[t] = s;
        }
        for (int h = 128; h >= 1; h >>= 1)
            for (int t = 0; t < h; ++t) part[t] = part[t] + part[t + h];
        bt[b] = part[0];
    }
    const float r = lane_tree_sum(bt, nb);
    free(bt);
    return r;
}

/* concord/packed_b.py:2081-2091: sig = C * (s_slow - v_slow) * 128, noise =
 * s_fast - sig, coh = sig^2 / (sig^2 + noise^2 + 1e-30) (left to right);
 * summed in 8192-word blocks: lane t chains words b0 + t + 256 i, a
 * halving tree over the 256 lanes; the block totals by lane_tree_sum */
float oracle_coherence_sum(const int32_t* packed, int64_t N, int64_t K, float C) {
    const int64_t total = N * K;
    const int64_t nb = (total + 8191) / 8192;
    float* bt = (float*)malloc((size_t)(nb > 0 ? nb : 1) * sizeof(float));
    int64_t b = 0;
    for (int64_t b0 = 0; b0 < total; b0 += 8192) {
        float part[256];
        for (int t = 0; t < 256; ++t) {
            float s = 0.0f;
            for (int i = 0; i < 32; ++i) {
                const int64_t e = b0 + t + 256 * i;
                if (e >= total) continue;
                const int32_t w = packed[e];
                const int32_t sf = w >> 16, ss = (int8_t)(w >> 8), vs = (int8_t)w;
                const float sig = C * (float)((ss - vs) * 128);
                const float noise = (float)sf - sig;
                const float sig2 = sig * sig;
                s = s + sig2 / ((sig2 + noise * noise) + 1e-30f);
            }
            part[t] = s;
        }
        for (int h = 128; h >= 1; h >>= 1)
            for (int t = 0; t < h; ++t) part[t] = part[t] + part[t + h];
        bt[b++] = part[0];
    }
    const float r = lane_tree_sum(bt, nb);
    free(bt);
    return r;
}

/* cos(2 pi u) and sin(2 pi u), u in [0, 1) on a 2^-24 grid: quadrant and
 * Taylor polynomials in theta^2, the op order of the library's det_sincos2pi */
static void det_sincos2pi(float u, float* cs, float* sn2) {
    const float t = u * 4.0f;
    const float qf = floorf(t);
    const int q = (int)qf;
    const float th = (t - qf) * 1.57079632679489662f;
    const float s = th * th;
    float c = -1.0f / 3628800.0f;
    c = c * s + 1.0f / 40320.0f;
    c = c * s + -1.0f / 720.0f;
    c = c * s + 1.0f / 24.0f;
    c = c * s + -0.5f;
    c = c * s + 1.0f;
    float sn = -1.0f / 39916800.0f;
    sn = sn * s + 1.0f / 362880.0f;
    sn = sn * s + -1.0f / 5040.0f;
    sn = sn * s + 1.0f / 120.0f;
    sn = sn * s + -1.0f / 6.0f;
    sn = sn * s + 1.0f;
    sn = sn * th;
    *cs = q == 0 ? c : q == 1 ? -sn : q == 2 ? -c : sn;
    *sn2 = q == 0 ? sn : q == 1 ? c : q == 2 ? -sn : -c;
}

/* Box-Muller radius sqrt(-2 ln u1), u1 = ((w >> 8) + 1) 2^-24, and angle
 * fraction u2 = (w >> 8) 2^-24 of a Philox word */
static float bm_radius(uint32_t w) {
    const float u1 = (float)((w >> 8) + 1u) * 5.9604644775390625e-08f;
    const float ln = det_log2(u1) * 0.693147180559945309f;
    return sqrtf(-2.0f * ln);
}
static float bm_angle(uint32_t w) { return (float)(w >> 8) * 5.9604644775390625e-08f; }

float oracle_normal_draw_tag(int32_t seed, uint32_t idx, uint32_t tag) {
    uint32_t c[4] = {idx, 0u, 0u, 0u};
    uint32_t k[2] = {(uint32_t)seed, tag};
    oracle_philox4x32_10(c, k);
    float cs, sn;
    det_sincos2pi(bm_angle(c[1]), &cs, &sn);
    return bm_radius(c[0]) * cs;
}

void oracle_iso_draw4(int32_t seed, uint32_t blk, float z[4]) {
    uint32_t c[4] = {blk, 0u, 0u, 0u};
    uint32_t k[2] = {(uint32_t)seed, 0x6E6F6973u};
    oracle_philox4x32_10(c, k);
    const float r0 = bm_radius(c[0]), r2 = bm_radius(c[2]);
    float ca, sa, cb, sb;
    det_sincos2pi(bm_angle(c[1]), &ca, &sa);
    det_sincos2pi(bm_angle(c[3]), &cb, &sb);
    z[0] = r0 * ca;
    z[1] = r0 * sa;
    z[2] = r2 * cb;
    z[3] = r2 * sb;
}

float oracle_iso_draw(int32_t seed, int64_t e) {
    float z[4];
    oracle_iso_draw4(seed, (uint32_t)(e >> 2), z);
    return z[e & 3];
}

void oracle_iso_noise(uint16_t* g, int64_t N, int64_t K, float sigma, int32_t salt) {
    const int64_t total = N * K;
    const int64_t nb = (total + 8191) / 8192;
    float* btg = (float*)malloc((size_t)(nb > 0 ? nb : 1) * sizeof(float));
    float* btx = (float*)malloc((size_t)(nb > 0 ? nb : 1) * sizeof(float));
    int64_t b = 0;
    for (int64_t b0 = 0; b0 < total; b0 += 8192) {
        float pg[256], px[256];
        for (int t = 0; t < 256; ++t) {
            float ag = 0.0f, ax = 0.0f;
            for (int i = 0; i < 8; ++i) {
                const int64_t e0 = b0 + 4 * (t + 256 * i);
                if (e0 >= total) continue;
                float z[4];
                oracle_iso_draw4(salt, (uint32_t)(e0 >> 2), z);
                for (int r = 0; r < 4 && e0 + r < total; ++r) {
                    const float v = bf16_to_f32(g[e0 + r]);
                    ag = ag + v * v;
                    ax = ax + z[r] * z[r];
                }
            }
            pg[t] = ag;
            px[t] = ax;
        }
        for (int h = 128; h >= 1; h >>= 1)
            for (int t = 0; t < h; ++t) {
                pg[t] = pg[t] + pg[t + h];
                px[t] = px[t] + px[t + h];
            }
        btg[b] = pg[0];
        btx[b] = px[0];
        ++b;
    }
    const float sg = lane_tree_sum(btg, nb), sx = lane_tree_sum(btx, nb);
    free(btg);
    free(btx);
    const float ng = sqrtf(sg);
    const float nx = fmaxf(sqrtf(sx), 1e-12f);
    const float scale = (sigma * ng) / nx;
    for (int64_t e = 0; e < total; ++e)
        g[e] = oracle_f32_to_bf16(bf16_to_f32(g[e]) + oracle_iso_draw(salt, e) * scale);
}

float oracle_token_sum(int32_t seed, int64_t M) {
    const int64_t nb = (M + 8191) / 8192;
    float* bt = (float*)malloc((size_t)(nb > 0 ? nb : 1) * sizeof(float));
    int64_t b = 0;
    for (int64_t b0 = 0; b0 < M; b0 += 8192) {
        float part[256];
        for (int t = 0; t < 256; ++t) {
            float a = 0.0f;
            for (int i = 0; i < 32; ++i) {
                const int64_t m = b0 + t + 256 * i;
                if (m < M) a = a + oracle_normal_draw_tag(seed, (uint32_t)m, 0x5369676Du);
            }
            part[t] = a;
        }
        for (int h = 128; h >= 1; h >>= 1)
            for (int t = 0; t < h; ++t) part[t] = part[t] + part[t + h];
        bt[b++] = part[0];
    }
    const float r = lane_tree_sum(bt, nb);
    free(bt);
    return r;
}

void oracle_sigmag_combine(uint16_t* g, const uint16_t* P, int64_t N, int64_t K, float S, float Mf,
                           float sigma) {
    const int64_t total = N * K;
    const int64_t nb = (total + 8191) / 8192;
    float* btg = (float*)malloc((size_t)(nb > 0 ? nb : 1) * sizeof(float));
    float* btx = (float*)malloc((size_t)(nb > 0 ? nb : 1) * sizeof(float));
    int64_t b = 0;
    for (int64_t b0 = 0; b0 < total; b0 += 8192) {
        float pg[256], px[256];
        for (int t = 0; t < 256; ++t) {
            float ag = 0.0f, ax = 0.0f;
            for (int i = 0; i < 32; ++i) {
                const int64_t e = b0 + t + 256 * i;
                if (e >= total) continue;
                const float v = bf16_to_f32(g[e]);
                const float z = bf16_to_f32(P[e]) - S * (v / Mf);
                ag = ag + v * v;
                ax = ax + z * z;
            }
            pg[t] = ag;
            px[t] = ax;
        }
        for (int h = 128; h >= 1; h >>= 1)
            for (int t = 0; t < h; ++t) {
                pg[t] = pg[t] + pg[t + h];
                px[t] = px[t] + px[t + h];
            }
        btg[b] = pg[0];
        btx[b] = px[0];
        ++b;
    }
    const float sg = lane_tree_sum(btg, nb), sx = lane_tree_sum(btx, nb);
    free(btg);
    free(btx);
    const float scale = (sigma * sqrtf(sg)) / fmaxf(sqrtf(sx), 1e-12f);
    for (int64_t e = 0; e < total; ++e) {
        const float v = bf16_to_f32(g[e]);
        const float z = bf16_to_f32(P[e]) - S * (v / Mf);
        g[e] = oracle_f32_to_bf16(v + z * scale);
    }
}

static inline float rbf(float f) { return bf16_to_f32(oracle_f32_to_bf16(f)); }

/* C[I][J] = bf16(sum_r A(i,r) B(r,j)); A(i,r) = a[i*lda_i + r*lda_r], likewise B */
static void gemm_bf16(const float* a, int64_t lai, int64_t lar, const float* b, int64_t lbr, int64_t lbj,
                      float* c, int64_t I, int64_t J, int64_t R) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < I; ++i)
        for (int64_t j = 0; j < J; ++j) {
            float s = 0.0f;
            for (int64_t r = 0; r < R; ++r) s = s + a[i * lai + r * lar] * b[r * lbr + j * lbj];
            c[i * J + j] = rbf(s);
        }
}

void oracle_muon_ns5(const uint16_t* g, int64_t N, int64_t K, float gamma, uint16_t* out) {
    const float na = 3.4445f, nb = -4.7750f, nc = 2.0315f;
    const int tr = N > K;
    const int64_t m = tr ? K : N, n = tr ? N : K;
    const float norm = sqrtf(oracle_frob_sumsq(g, N, K));
    /* g / n with n = max(||g||, 1e-12), then / (||g / n|| + 1e-7):
     * exp9_muon.py:75, 82 (drive) and 47 (ns5), as one denominator
     * n * (||g|| / n + 1e-7); ||g|| / n is exactly 1 for ||g|| >= 1e-12 */
    const float nn = fmaxf(norm, 1e-12f);
    const float den = nn * (norm / nn + 1e-7f);
    float* X = (float*)malloc((size_t)(m * n) * sizeof(float));
    float* BX = (float*)malloc((size_t)(m * n) * sizeof(float));
    float* A = (float*)malloc((size_t)(m * m) * sizeof(float));
    float* AA = (float*)malloc((size_t)(m * m) * sizeof(float));
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            const float v = tr ? bf16_to_f32(g[j * K + i]) : bf16_to_f32(g[i * K + j]);
            X[i * n + j] = rbf(v / den);
        }
    for (int it = 0; it < 5; ++it) {
        gemm_bf16(X, n, 1, X, 1, n, A, m, m, n);          /* X X^T */
        gemm_bf16(A, m, 1, A, m, 1, AA, m, m, m);         /* A A */
        for (int64_t e = 0; e < m * m; ++e) A[e] = rbf(nb * A[e] + nc * AA[e]);   /* B */
        gemm_bf16(A, m, 1, X, n, 1, BX, m, n, m);         /* B X */
        for (int64_t e = 0; e < m * n; ++e) X[e] = rbf(na * X[e] + BX[e]);
    }
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            const uint16_t v = oracle_f32_to_bf16(gamma * X[i * n + j]);
            if (tr) out[j * K + i] = v; else out[i * K + j] = v;
        }
    free(X);
    free(BX);
    free(A);
    free(AA);
}

/* ---- A11 load_weights / load_weights_finetune ------------------------------
 * concord/packed_b.py:1570-1603 and 1816-1856.
 * row_exp = clamp(ceil(log2(max_k |W|) + 1), exp_min, exp_max), evaluated in
 * exact arithmetic (frexp): the reference's float log2 can differ when
 * max|W| lies within a few ulp above a power of two.  col_exp = 0.
 * Roundings are round-half-to-even (torch.round). */
void oracle_load_weights(const float* W, int64_t N, int64_t K,
                         int32_t exp_min, int32_t exp_max,
                         int32_t mantissa_bias, int finetune,
                         int32_t* packed, int8_t* row_exp, int8_t* col_exp) {
    for (int64_t k = 0; k < K; ++k) col_exp[k] = 0;
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
        float mx = 0.0f;
        for (int64_t k = 0; k < K; ++k) mx = fmaxf(mx, fabsf(W[n * K + k]));
        mx = fmaxf(mx, 1e-30f);
        int e2;
        float fr = frexpf(mx, &e2);       /* mx = fr * 2^e2, fr in [0.5, 1) */
        int32_t e = (fr == 0.5f) ? e2 : e2 + 1;
        e = clampi(e, exp_min, exp_max);
        row_exp[n] = (int8_t)e;
        const float scale = exp2i(e - mantissa_bias);
        for (int64_t k = 0; k < K; ++k) {
            const float q = rintf(W[n * K + k] / scale);
            int32_t m = oracle_f2i(q);
            int32_t sf, ss = 0, vs = 0;
            if (!finetune) {
                sf = clampi(m, -32768, 32767);
            } else {
                const int32_t tv = oracle_f2i(rintf((float)m / 2.0f));
                vs = clampi(oracle_f2i(rintf((float)tv / 128.0f)), -128, 127);
                const int32_t rem = w_sub(m, w_mul(vs, 128));
                ss = clampi(oracle_f2i(rintf((float)rem / 128.0f)), -128, 127);
                sf = clampi(w_sub(rem, w_mul(ss, 128)), -32768, 32767);
            }
            packed[n * K + k] = pack(sf, ss, vs);
        }
    }
}
