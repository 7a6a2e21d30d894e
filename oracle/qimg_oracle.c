/*
 * qimg_oracle.c — CPU restatement of qwen-image.cu's quantized-linear and
 * SageAttention hot path. TEST INFRASTRUCTURE ONLY (expected values, never
 * the product). Built with -ffp-contract=off so every fp32 operation rounds
 * exactly where the reference's source places it.
 */
#include "qimg_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ */
/* scalar conversions                                                   */
/* ------------------------------------------------------------------ */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float or_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t or_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40); /* quiet NaN */
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

float or_f16_to_f32(uint16_t h) {
    uint32_t s = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24 is exact in fp32 */
        float v = (float)m * 5.9604644775390625e-08f;
        return (s ? -v : v);
    }
    if (e == 31) return u2f(s | 0x7f800000u | (m << 13));
    return u2f(s | ((e + 112u) << 23) | (m << 13));
}

uint16_t or_f32_to_f16(float f) {
    uint32_t u = f2u(f);
    uint16_t s = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(s | 0x7e00u);
    if (a >= 0x477ff000u) return (uint16_t)(s | 0x7c00u); /* >= 65520 rounds to inf */
    if (a < 0x38800000u) {
        /* result is subnormal (or zero) in fp16: quantum 2^-24 */
        float av = u2f(a);
        float q = av * 16777216.0f; /* exact scaling by 2^24 */
        float r = rintf(q);         /* RNE */
        return (uint16_t)(s | (uint16_t)r);
    }
    uint32_t e = (a >> 23) - 112u;   /* rebias 127 -> 15 */
    uint32_t m = a & 0x7fffffu;
    uint32_t hm = m >> 13;
    uint32_t rem = m & 0x1fffu;
    uint32_t out = (e << 10) | hm;
    if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) out += 1u; /* may carry into exponent */
    return (uint16_t)(s | out);
}

uint8_t or_f32_to_e4m3(float f) {
    uint32_t u = f2u(f);
    uint8_t s = (uint8_t)((u >> 24) & 0x80u);
    float a = fabsf(f);
    if (isnan(f)) return 0x7f;
    if (a >= 448.0f) return (uint8_t)(s | 0x7e);
    if (a < 0.015625f) {
        /* subnormal range of e4m3: quantum 2^-9 */
        float r = rintf(a * 512.0f);
        return (uint8_t)(s | (uint8_t)r); /* r == 8 encodes the min normal 2^-6 */
    }
    uint32_t au = f2u(a);
    int32_t e = (int32_t)(au >> 23) - 127 + 7;
    uint32_t m = au & 0x7fffffu;
    uint32_t hm = m >> 20;
    uint32_t rem = m & 0xfffffu;
    uint32_t out = ((uint32_t)e << 3) | hm;
    if (rem > 0x80000u || (rem == 0x80000u && (hm & 1u))) out += 1u;
    if (out > 0x7eu) out = 0x7eu; /* saturate (464 <= a < 480 would round past 448) */
    return (uint8_t)(s | out);
}

float or_e4m3_to_f32(uint8_t b) {
    float sgn = (b & 0x80) ? -1.0f : 1.0f;
    int e = (b >> 3) & 0xf;
    int m = b & 7;
    if (e == 15 && m == 7) return NAN;
    if (e == 0) return sgn * (float)m * 0.001953125f; /* m * 2^-9 */
    return sgn * ldexpf(1.0f + (float)m / 8.0f, e - 7);
}

/* ------------------------------------------------------------------ */
/* threads                                                              */
/* ------------------------------------------------------------------ */
void or_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

int or_get_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------ */
/* a1, a2: Hadamard                                                     */
/* ------------------------------------------------------------------ */
int or_hadamard_block_size(int K) { return K & (-K); }

float or_fwht_norm(int hbs) { return (float)(1.0 / sqrt((double)hbs)); }

/* One row, reference stage order (cuda_kernels.cu:2226-2241): for each
 * stage half = 1, 2, 4, ... the pair (idx_a, idx_a + half) with idx_a =
 * group*2*half + within becomes (a + b, a - b). */
static void fwht_row(float* row, int K, int hbs, float norm) {
    for (int base = 0; base < K; base += hbs) {
        float* blk = row + base;
        for (int half = 1; half < hbs; half <<= 1) {
            int full = half << 1;
            for (int g = 0; g < hbs; g += full) {
                for (int w = 0; w < half; ++w) {
                    float a = blk[g + w];
                    float b = blk[g + w + half];
                    blk[g + w] = a + b;
                    blk[g + w + half] = a - b;
                }
            }
        }
        for (int i = 0; i < hbs; ++i) blk[i] = blk[i] * norm;
    }
}

void or_fwht_rows(float* x, int64_t M, int K, int hbs) {
    float norm = or_fwht_norm(hbs);
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m) fwht_row(x + m * (int64_t)K, K, hbs, norm);
}

/* ------------------------------------------------------------------ */
/* a3: per-row int8                                                     */
/* ------------------------------------------------------------------ */
static inline int8_t sat_rne_i8(float v) {
    float r = rintf(v); /* __float2int_rn: round half to even */
    if (r < -128.0f) r = -128.0f;
    if (r > 127.0f) r = 127.0f;
    return (int8_t)(int)r;
}

static void quant_row_int8(const float* row, int K, int8_t* q, float* scale) {
    float amax = 0.0f;
    for (int i = 0; i < K; ++i) amax = fmaxf(amax, fabsf(row[i]));
    *scale = amax / 127.0f;
    float inv = (amax > 0.0f) ? 127.0f / amax : 0.0f;
    for (int i = 0; i < K; ++i) q[i] = sat_rne_i8(row[i] * inv);
}

void or_quant_rows_int8(const float* x, int64_t M, int K, int8_t* q, float* scales) {
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m)
        quant_row_int8(x + m * (int64_t)K, K, q + m * (int64_t)K, scales + m);
}

/* ------------------------------------------------------------------ */
/* a4, a5                                                               */
/* ------------------------------------------------------------------ */
int or_quantize_weight_bf16(const uint16_t* w, int N, int K, int8_t* q, float* scales) {
    int hbs = or_hadamard_block_size(K);
    float norm = or_fwht_norm(hbs);
#pragma omp parallel
    {
        float* row = (float*)malloc(sizeof(float) * (size_t)K);
#pragma omp for schedule(static)
        for (int n = 0; n < N; ++n) {
            const uint16_t* src = w + (int64_t)n * K;
            for (int i = 0; i < K; ++i) row[i] = or_bf16_to_f32(src[i]);
            if (hbs > 1) fwht_row(row, K, hbs, norm);
            quant_row_int8(row, K, q + (int64_t)n * K, scales + n);
        }
        free(row);
    }
    return hbs;
}

void or_quantize_activation(const void* x, int x_is_bf16, int64_t M, int K, int hbs,
                            int8_t* q, float* scales) {
    float norm = or_fwht_norm(hbs > 0 ? hbs : 1);
#pragma omp parallel
    {
        float* row = (float*)malloc(sizeof(float) * (size_t)K);
#pragma omp for schedule(static)
        for (int64_t m = 0; m < M; ++m) {
            if (x_is_bf16) {
                const uint16_t* src = (const uint16_t*)x + m * (int64_t)K;
                for (int i = 0; i < K; ++i) row[i] = or_bf16_to_f32(src[i]);
            } else {
                memcpy(row, (const float*)x + m * (int64_t)K, sizeof(float) * (size_t)K);
            }
            if (hbs > 1) fwht_row(row, K, hbs, norm);
            quant_row_int8(row, K, q + m * (int64_t)K, scales + m);
        }
        free(row);
    }
}

/* ------------------------------------------------------------------ */
/* a7, a8                                                               */
/* ------------------------------------------------------------------ */
void or_gemm_s8s8s32(const int8_t* A, const int8_t* W, int64_t M, int N, int K,
                     int64_t m0, int64_t m1, int32_t* C) {
    (void)M;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t m = m0; m < m1; ++m) {
        const int8_t* a = A + m * (int64_t)K;
        for (int n = 0; n < N; ++n) {
            const int8_t* w = W + (int64_t)n * K;
            int32_t acc = 0;
            for (int k = 0; k < K; ++k) acc += (int32_t)a[k] * (int32_t)w[k];
            C[m * (int64_t)N + n] = acc;
        }
    }
}

static inline float gelu_tanh(float v) {
    const float c = 0.7978845608f;
    float inner = c * (v + 0.044715f * v * v * v);
    return 0.5f * v * (1.0f + tanhf(inner));
}

static inline float epilogue(int32_t acc, float as, float ws, const uint16_t* bias, int n, int gelu) {
    float v = (float)acc * as * ws;
    if (bias) v += or_bf16_to_f32(bias[n]);
    return gelu ? gelu_tanh(v) : v;
}

void or_dequant_epilogue(const int32_t* C, const float* as, const float* ws,
                         const uint16_t* bias_bf16, int64_t M, int N, int gelu, float* out) {
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n)
            out[m * (int64_t)N + n] = epilogue(C[m * (int64_t)N + n], as[m], ws[n], bias_bf16, n, gelu);
}

/* ------------------------------------------------------------------ */
/* fp8-e4m3 mode                                                        */
/* ------------------------------------------------------------------ */
void or_quant_rows_fp8(const float* x, int64_t M, int K, uint8_t* q, float* scales) {
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m) {
        const float* row = x + m * (int64_t)K;
        float amax = 0.0f;
        for (int i = 0; i < K; ++i) amax = fmaxf(amax, fabsf(row[i]));
        scales[m] = amax / 448.0f;
        float inv = (amax > 0.0f) ? 448.0f / amax : 0.0f;
        for (int i = 0; i < K; ++i) q[m * (int64_t)K + i] = or_f32_to_e4m3(row[i] * inv);
    }
}

void or_gemm_fp8_epilogue(const uint8_t* A, const uint8_t* W, const float* as, const float* ws,
                          const uint16_t* bias_bf16, int64_t M, int N, int K,
                          int64_t m0, int64_t m1, int gelu, float* out) {
    (void)M;
    float lut[256];
    for (int i = 0; i < 256; ++i) lut[i] = or_e4m3_to_f32((uint8_t)i);
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t m = m0; m < m1; ++m) {
        const uint8_t* a = A + m * (int64_t)K;
        for (int n = 0; n < N; ++n) {
            const uint8_t* w = W + (int64_t)n * K;
            double acc = 0.0;
            for (int k = 0; k < K; ++k) acc += (double)lut[a[k]] * (double)lut[w[k]];
            float v = (float)acc * as[m] * ws[n];
            if (bias_bf16) v += or_bf16_to_f32(bias_bf16[n]);
            out[m * (int64_t)N + n] = gelu ? gelu_tanh(v) : v;
        }
    }
}

/* ------------------------------------------------------------------ */
/* SageAttention                                                        */
/* ------------------------------------------------------------------ */
static inline int div_ceil(int a, int b) { return (a + b - 1) / b; }

void or_sage_k_mean(const uint16_t* k_f16, int BH, int S, int D, float* mean) {
#pragma omp parallel for schedule(static)
    for (int h = 0; h < BH; ++h) {
        for (int d = 0; d < D; ++d) {
            float sum = 0.0f;
            const uint16_t* p = k_f16 + (int64_t)h * S * D + d;
            for (int s = 0; s < S; ++s) sum += or_f16_to_f32(p[(int64_t)s * D]);
            mean[h * D + d] = sum / fmaxf((float)S, 1.0f);
        }
    }
}

static inline int8_t cvt_rni_sat_s8(float v) {
    if (isnan(v)) return 0;
    return sat_rne_i8(v);
}

void or_sage_quant_q(const uint16_t* q_f16, int BH, int S, int D, int8_t* q_out, float* q_scale) {
    int nblk = div_ceil(S, 128);
#pragma omp parallel for schedule(static)
    for (int h = 0; h < BH; ++h) {
        const uint16_t* src = q_f16 + (int64_t)h * S * D;
        int8_t* dst = q_out + (int64_t)h * S * D;
        for (int b = 0; b < nblk; ++b)
            for (int w = 0; w < 4; ++w)
                for (int g = 0; g < 8; ++g) {
                    int base = b * 128 + w * 32 + g;
                    float amax = 1e-7f;
                    for (int i = 0; i < 4; ++i) {
                        int t = base + 8 * i;
                        if (t >= S) continue;
                        for (int d = 0; d < D; ++d)
                            amax = fmaxf(amax, fabsf(or_f16_to_f32(src[(int64_t)t * D + d])));
                    }
                    float scale = amax / 127.0f + 1e-7f;
                    q_scale[(int64_t)h * (nblk * 32) + b * 32 + w * 8 + g] = scale;
                    float inv = 1.0f / scale;
                    for (int i = 0; i < 4; ++i) {
                        int t = base + 8 * i;
                        if (t >= S) continue;
                        for (int d = 0; d < D; ++d)
                            dst[(int64_t)t * D + d] = cvt_rni_sat_s8(or_f16_to_f32(src[(int64_t)t * D + d]) * inv);
                    }
                }
    }
}

void or_sage_quant_k(const uint16_t* k_f16, const float* mean, int BH, int S, int D,
                     int8_t* k_out, float* k_scale) {
    int nblk = div_ceil(S, 64);
#pragma omp parallel for schedule(static)
    for (int h = 0; h < BH; ++h) {
        const uint16_t* src = k_f16 + (int64_t)h * S * D;
        int8_t* dst = k_out + (int64_t)h * S * D;
        const float* mu = mean + (int64_t)h * D;
        for (int b = 0; b < nblk; ++b)
            for (int g = 0; g < 4; ++g) {
                int base = b * 64 + 2 * g;
                float amax = 1e-7f;
                for (int i = 0; i < 8; ++i)
                    for (int j = 0; j < 2; ++j) {
                        int t = base + 8 * i + j;
                        if (t >= S) continue;
                        for (int d = 0; d < D; ++d)
                            amax = fmaxf(amax, fabsf(or_f16_to_f32(src[(int64_t)t * D + d]) - mu[d]));
                    }
                float scale = amax / 127.0f + 1e-7f;
                k_scale[(int64_t)h * (nblk * 4) + b * 4 + g] = scale;
                float inv = 1.0f / scale;
                for (int i = 0; i < 8; ++i)
                    for (int j = 0; j < 2; ++j) {
                        int t = base + 8 * i + j;
                        if (t >= S) continue;
                        for (int d = 0; d < D; ++d)
                            dst[(int64_t)t * D + d] =
                                cvt_rni_sat_s8((or_f16_to_f32(src[(int64_t)t * D + d]) - mu[d]) * inv);
                    }
            }
    }
}

/* Per-token scale lookups used by the attention kernel (a15, the
 * q_scale_idx / k_scale_idx formulas at sageattention_sm80.cu:121-143). */
static inline float q_scale_of(const float* qs_head, int t) {
    return qs_head[(t / 128) * 32 + ((t % 128) / 32) * 8 + (t % 8)];
}
static inline float k_scale_of(const float* ks_head, int t) {
    return ks_head[(t / 64) * 4 + (t % 8) / 2];
}

void or_sage_attn(const int8_t* q, const int8_t* k, const uint16_t* v_f16,
                  const float* q_scale, const float* k_scale, int BH, int S, int D,
                  float sm_scale, int causal, int q0, int q1, uint16_t* out_f16) {
    const float LOG2E = 1.44269504088896340736f;
    const float sm = sm_scale * LOG2E;
    const int nq_scales = div_ceil(S, 128) * 32;
    const int nk_scales = div_ceil(S, 64) * 4;
    const int CTA_Q = 128, CTA_K = 64;
#pragma omp parallel
    {
        float* vf = (float*)malloc(sizeof(float) * (size_t)CTA_K * D);
        float* o = (float*)malloc(sizeof(float) * (size_t)D);
        float rs[64], mult[64], p16[64];
#pragma omp for schedule(dynamic, 1) collapse(2)
        for (int h = 0; h < BH; ++h) {
            for (int i = q0; i < q1; ++i) {
                const int8_t* qi = q + ((int64_t)h * S + i) * D;
                const int8_t* kh = k + (int64_t)h * S * D;
                const uint16_t* vh = v_f16 + (int64_t)h * S * D;
                const float qsc = q_scale_of(q_scale + (int64_t)h * nq_scales, i);
                const float* ksh = k_scale + (int64_t)h * nk_scales;
                int kv_end = S;
                if (causal) {
                    int blk_end = (i / CTA_Q + 1) * CTA_Q;
                    kv_end = S < blk_end ? S : blk_end;
                }
                int niter = div_ceil(kv_end, CTA_K);
                float m = -5000000.0f, d = 1.0f;
                for (int c = 0; c < D; ++c) o[c] = 0.0f;
                for (int it = 0; it < niter; ++it) {
                    int peeled = (it >= niter - 2); /* second-last and last iteration */
                    int last = (it == niter - 1);
                    int kb = it * CTA_K;
                    float m_tile = -5000000.0f;
                    for (int j = 0; j < CTA_K; ++j) {
                        int t = kb + j;
                        int32_t acc = 0;
                        if (t < S) {
                            const int8_t* kt = kh + (int64_t)t * D;
                            for (int c = 0; c < D; ++c) acc += (int32_t)qi[c] * (int32_t)kt[c];
                        }
                        /* keys past S inside the last tile still index
                         * that tile's 4 scale entries */
                        float ksc = k_scale_of(ksh, t);
                        float dq = qsc * ksc;
                        if (!peeled) {
                            rs[j] = (float)acc;
                            mult[j] = sm * dq;
                        } else {
                            rs[j] = (float)acc * dq;
                            mult[j] = sm;
                            if (causal && t > i) rs[j] = -5000000.0f;
                            if (last && t >= S) rs[j] = -5000000.0f;
                        }
                        float mt = rs[j] * mult[j];
                        if (mt > m_tile) m_tile = mt;
                    }
                    float m_new = fmaxf(m, m_tile);
                    float o_scale = exp2f(m - m_new);
                    m = m_new;
                    d *= o_scale;
                    for (int c = 0; c < D; ++c) o[c] *= o_scale;
                    float neg_m = -m;
                    float dsum = 0.0f;
                    for (int j = 0; j < CTA_K; ++j) {
                        float p = exp2f(fmaf(rs[j], mult[j], neg_m));
                        p16[j] = or_f16_to_f32(or_f32_to_f16(p));
                        dsum += p16[j];
                    }
                    d += dsum;
                    for (int j = 0; j < CTA_K; ++j) {
                        int t = kb + j;
                        if (t >= S || p16[j] == 0.0f) continue;
                        const uint16_t* vt = vh + (int64_t)t * D;
                        for (int c = 0; c < D; ++c) vf[c] = or_f16_to_f32(vt[c]);
                        for (int c = 0; c < D; ++c) o[c] += p16[j] * vf[c];
                    }
                }
                float rcp = 1.0f / d;
                uint16_t* dst = out_f16 + ((int64_t)h * S + i) * D;
                for (int c = 0; c < D; ++c) dst[c] = or_f32_to_f16(o[c] * rcp);
            }
        }
        free(vf);
        free(o);
    }
}

void or_sage_attention_fp16io(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                              int BH, int S, int D, float sm_scale, int causal,
                              uint16_t* out_f16) {
    size_t n = (size_t)BH * S * D;
    int8_t* qi = (int8_t*)malloc(n);
    int8_t* ki = (int8_t*)malloc(n);
    float* qs = (float*)malloc(sizeof(float) * (size_t)BH * div_ceil(S, 128) * 32);
    float* ks = (float*)malloc(sizeof(float) * (size_t)BH * div_ceil(S, 64) * 4);
    float* mean = (float*)malloc(sizeof(float) * (size_t)BH * D);
    or_sage_k_mean(k, BH, S, D, mean);
    or_sage_quant_q(q, BH, S, D, qi, qs);
    or_sage_quant_k(k, mean, BH, S, D, ki, ks);
    or_sage_attn(qi, ki, v, qs, ks, BH, S, D, sm_scale, causal, 0, S, out_f16);
    free(qi); free(ki); free(qs); free(ks); free(mean);
}
