/*
 * qimg_oracle_int4.c — CPU restatement of qwen-image.cu's INT4 paths
 * (cuda_kernels.cu:2864-4532). TEST INFRASTRUCTURE ONLY (expected values,
 * never the product). Built with -ffp-contract=off: every fp32 operation
 * rounds where the reference's source places it, and divisions are
 * correctly rounded (the reference binary's --use_fast_math approximations
 * are not modelled, as in qimg_oracle.c).
 */
#include "qimg_oracle.h"

#include <math.h>
#include <string.h>

/* cuda_kernels.cu:2869-2872 NF4_GRID (the same decimal literals). */
const float OR_NF4_GRID[16] = {
    -1.0f, -0.6962f, -0.5251f, -0.3949f, -0.2844f, -0.1848f, -0.0911f, 0.0f,
    0.0796f, 0.1609f, 0.2461f, 0.3379f, 0.4407f, 0.5626f, 0.7230f, 1.0f};

static inline int nib_signed(int n) { return n >= 8 ? n - 16 : n; }

/* cuda_kernels.cu:2876-2917 dequantize_int4_to_bf16_kernel. */
void or_dequant_int4_bf16(const uint8_t* qw, const float* scales, int N, int K, int gs, int nf4,
                          int scales_gn, int signed_int4, uint16_t* out) {
    const int G = K / gs;
    for (int64_t r = 0; r < N; ++r)
        for (int c = 0; c < K; ++c) {
            const uint8_t b = qw[r * (K / 2) + c / 2];
            const int n = (c & 1) ? (b >> 4) & 0xF : b & 0xF;
            const int g = c / gs;
            const float s = scales_gn ? scales[(int64_t)g * N + r] : scales[r * G + g];
            float v;
            if (nf4)
                v = OR_NF4_GRID[n] * s;
            else if (signed_int4)
                v = (float)nib_signed(n) * s;
            else
                v = (float)(n - 8) * s;
            out[r * K + c] = or_f32_to_bf16(v);
        }
}

static float group_amax(const float* p, int n) {
    float m = 0.0f;
    for (int i = 0; i < n; ++i) {
        const float v = fabsf(p[i]);
        if (v > m) m = v;
    }
    return m;
}

/* cuda_kernels.cu:3226-3288 quantize_linear_int4_per_group_kernel:
 * scale = amax/7, inv = amax>0 ? 7/amax : 0, q = clamp(roundf(v*inv), -7, 7) + 8. */
void or_quant_int4_linear(const float* r, int N, int K, int gs, uint8_t* qw, float* scales) {
    const int G = K / gs;
    for (int64_t row = 0; row < N; ++row)
        for (int g = 0; g < G; ++g) {
            const float* p = r + row * K + (int64_t)g * gs;
            const float amax = group_amax(p, gs);
            scales[row * G + g] = amax / 7.0f;
            const float inv = amax > 0.0f ? 7.0f / amax : 0.0f;
            for (int i = 0; i < gs; i += 2) {
                int q0 = (int)roundf(p[i] * inv), q1 = (int)roundf(p[i + 1] * inv);
                q0 = (q0 < -7 ? -7 : q0 > 7 ? 7 : q0) + 8;
                q1 = (q1 < -7 ? -7 : q1 > 7 ? 7 : q1) + 8;
                qw[row * (K / 2) + ((int64_t)g * gs + i) / 2] = (uint8_t)(q0 | (q1 << 4));
            }
        }
}

/* cuda_kernels.cu:3290-3357 quantize_int4_per_group_kernel (NF4):
 * scale = amax, inv = amax>0 ? 1/amax : 0, code = first j minimising
 * |v*inv - NF4_GRID[j]|. */
void or_quant_int4_nf4(const float* r, int N, int K, int gs, uint8_t* qw, float* scales) {
    const int G = K / gs;
    for (int64_t row = 0; row < N; ++row)
        for (int g = 0; g < G; ++g) {
            const float* p = r + row * K + (int64_t)g * gs;
            const float amax = group_amax(p, gs);
            scales[row * G + g] = amax;
            const float inv = amax > 0.0f ? 1.0f / amax : 0.0f;
            for (int i = 0; i < gs; i += 2) {
                int q[2] = {0, 0};
                for (int e = 0; e < 2; ++e) {
                    const float n = p[i + e] * inv;
                    float best = 1e9f;
                    for (int j = 0; j < 16; ++j) {
                        const float d = fabsf(n - OR_NF4_GRID[j]);
                        if (d < best) {
                            best = d;
                            q[e] = j;
                        }
                    }
                }
                qw[row * (K / 2) + ((int64_t)g * gs + i) / 2] = (uint8_t)(q[0] | (q[1] << 4));
            }
        }
}

/* cuda_kernels.cu:3575-3636 quantize_activation_int4_kernel and
 * cuda_kernels.cu:3650-3705 fused_smooth_bf16_quant_kernel (smooth may be
 * NULL; bf16_out may be NULL). v = x (/ smooth[k]); scale = amax/7 at
 * scales[g*M + m]; q = clamp(roundf(v*inv), -7, 7) as a two's complement
 * nibble, even column in the low nibble. */
void or_quant_act_int4(const float* x, const float* smooth, int M, int K, int gs, uint16_t* bf16_out,
                       uint8_t* packed, float* scales) {
    const int G = K / gs;
    float buf[1024];
    for (int64_t m = 0; m < M; ++m)
        for (int g = 0; g < G; ++g) {
            const int64_t c0 = (int64_t)g * gs;
            for (int i = 0; i < gs; ++i) {
                float v = x[m * K + c0 + i];
                if (smooth) v = v / smooth[c0 + i];
                buf[i] = v;
                if (bf16_out) bf16_out[m * K + c0 + i] = or_f32_to_bf16(v);
            }
            const float amax = group_amax(buf, gs);
            scales[(int64_t)g * M + m] = amax / 7.0f;
            const float inv = amax > 0.0f ? 7.0f / amax : 0.0f;
            for (int i = 0; i < gs; i += 2) {
                int q0 = (int)roundf(buf[i] * inv), q1 = (int)roundf(buf[i + 1] * inv);
                q0 = q0 < -7 ? -7 : q0 > 7 ? 7 : q0;
                q1 = q1 < -7 ? -7 : q1 > 7 ? 7 : q1;
                packed[m * (K / 2) + (c0 + i) / 2] = (uint8_t)((q0 & 0xF) | ((q1 & 0xF) << 4));
            }
        }
}

/* cuda_kernels.cu:4117-4255 w4a4_gemm_regdirect_kernel (and the naive
 * kernel :3732-3854, same arithmetic): per group g in order, d = exact int32
 * dot of the signed nibbles, acc = acc + ((float)d * as[g,m]) * ws[g,n];
 * then out = acc + b (accumulate: out = out + (acc + b)), b = bf16 bias or 0. */
void or_w4a4_gemm(const uint8_t* act, const uint8_t* wgt, const float* as, const float* ws, int64_t M,
                  int N, int K, int gs, int accumulate, const uint16_t* bias, int64_t m0, int64_t m1,
                  float* out) {
    const int G = K / gs;
    const int KB = K / 2;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t m = m0; m < m1; ++m) {
        const uint8_t* a = act + m * KB;
        for (int n = 0; n < N; ++n) {
            const uint8_t* w = wgt + (int64_t)n * KB;
            float acc = 0.0f;
            for (int g = 0; g < G; ++g) {
                int32_t d = 0;
                for (int j = g * gs / 2; j < (g + 1) * gs / 2; ++j) {
                    d += nib_signed(a[j] & 0xF) * nib_signed(w[j] & 0xF) +
                         nib_signed((a[j] >> 4) & 0xF) * nib_signed((w[j] >> 4) & 0xF);
                }
                const float t = (float)d * as[(int64_t)g * M + m];
                acc = acc + t * ws[(int64_t)g * N + n];
            }
            const float b = bias ? or_bf16_to_f32(bias[n]) : 0.0f;
            float* o = out + (m - m0) * N + n;
            *o = accumulate ? *o + (acc + b) : acc + b;
        }
    }
}

/* AWQ kInterleave=4 nibble address (cuda_kernels.cu:2992-3001, 3072-3085). */
static inline int awq_nibble(const int32_t* qw, int IC, int oc, int ic) {
    const int i16 = (ic >> 6 << 6) + (oc % 4) * 16 + (((ic & 63) >> 5) << 3) + (ic & 7);
    const int bit = ((i16 & 1) << 4) + (((ic >> 3) & 3) << 2);
    return (int)(((uint32_t)qw[(int64_t)(oc / 4) * (IC / 2) + (i16 >> 1)] >> bit) & 0xF);
}

/* cuda_kernels.cu:3059-3091 repack_awq_kernel: [OC/4, IC/2] -> [IC/8, OC],
 * word (ig, oc) holds the nibbles of ic = 8 ig .. 8 ig + 7, low first. */
void or_awq_repack(const int32_t* qw, int OC, int IC, int32_t* out) {
    for (int ig = 0; ig < IC / 8; ++ig)
        for (int oc = 0; oc < OC; ++oc) {
            uint32_t w = 0;
            for (int k = 0; k < 8; ++k) w |= (uint32_t)awq_nibble(qw, IC, oc, ig * 8 + k) << (4 * k);
            out[(int64_t)ig * OC + oc] = (int32_t)w;
        }
}

/* cuda_kernels.cu:3002-3038 dequantize_awq_to_bf16_kernel: out[std_oc, ic] =
 * bf16(q * scale + zero) of the interleaved channel nk_oc = feature *
 * ncomp + component. */
void or_dequant_awq_bf16(const int32_t* qw, const uint16_t* wscales, const uint16_t* wzeros, int OC, int IC,
                         int gs, int ncomp, uint16_t* out) {
    const int dim = OC / ncomp;
    for (int so = 0; so < OC; ++so) {
        const int nk = (so % dim) * ncomp + so / dim;
        for (int ic = 0; ic < IC; ++ic) {
            const int q = awq_nibble(qw, IC, nk, ic);
            const int g = ic / gs;
            const float s = or_bf16_to_f32(wscales[(int64_t)g * OC + nk]);
            const float z = or_bf16_to_f32(wzeros[(int64_t)g * OC + nk]);
            const float w = (float)q * s + z;
            out[(int64_t)so * IC + ic] = or_f32_to_bf16(w);
        }
    }
}

/* cuda_kernels.cu:3106-3153 awq_gemv_repacked_kernel (M = 1): per
 * interleaved channel, acc = acc + (q * scale + zero) * x[ic] for ic in
 * order (groups of 64: 8 words of 8 nibbles), + bias[std_oc], stored at
 * std_oc = (nk % ncomp) * dim + nk / ncomp. */
void or_awq_gemv(const float* x, const int32_t* qw_rep, const uint16_t* wscales, const uint16_t* wzeros,
                 const uint16_t* bias, int OC, int IC, int gs, int ncomp, float* out) {
    const int dim = OC / ncomp;
    const int G = IC / gs;
    const int gs8 = gs / 8;
    for (int nk = 0; nk < OC; ++nk) {
        float acc = 0.0f;
        for (int g = 0; g < G; ++g) {
            const float s = or_bf16_to_f32(wscales[(int64_t)g * OC + nk]);
            const float z = or_bf16_to_f32(wzeros[(int64_t)g * OC + nk]);
            for (int io = 0; io < 8; ++io) {
                const int ig = g * gs8 + io;
                const uint32_t p = (uint32_t)qw_rep[(int64_t)ig * OC + nk];
                for (int k = 0; k < 8; ++k) {
                    const int q = (int)((p >> (4 * k)) & 0xF);
                    const float w = (float)q * s + z;
                    acc = acc + w * x[ig * 8 + k];
                }
            }
        }
        const int so = (nk % ncomp) * dim + nk / ncomp;
        if (bias) acc = acc + or_bf16_to_f32(bias[so]);
        out[so] = acc;
    }
}

/* nunchaku MMA-swizzled nibble and scale addresses (cuda_kernels.cu:2945-2973,
 * 3446-3485). */
static inline int nk_nibble(const uint8_t* q, int K, int row, int col) {
    const int kt = K / 64, nt = row / 128, nw = row % 128;
    const int np = nw / 16, ps = (nw % 16) / 8, nl = nw % 8;
    const int ktile = col / 64, kps = (col % 64) / 32, kl = (col % 32) / 8, rk = col % 8;
    const int64_t i32 = (int64_t)nt * (kt * 1024) + ktile * 1024 + np * 128 + nl * 16 + kl * 4 + ps * 2 + kps;
    return (q[i32 * 4 + rk / 2] >> ((rk % 2) * 4)) & 0xF;
}

static inline int64_t nk_scale_off(int G, int row, int g) {
    const int nt = row / 128, nw = row % 128;
    return (int64_t)nt * G * 128 + g * 128 + (nw / 16) * 16 + ((nw % 8) / 2) * 4 + ((nw % 16) / 8) * 2 + nw % 2;
}

/* cuda_kernels.cu:3431-3487 unswizzle_nunchaku_weights_kernel: row-major
 * packed nibbles [N, K/2] and fp32 scales [G, N]. */
void or_unswizzle_nunchaku(const uint8_t* q_sw, const uint16_t* s_sw, int N, int K, int G, uint8_t* q_rm,
                           float* s_rm) {
    for (int r = 0; r < N; ++r) {
        for (int c = 0; c < K; c += 2)
            q_rm[(int64_t)r * (K / 2) + c / 2] = (uint8_t)(nk_nibble(q_sw, K, r, c) | (nk_nibble(q_sw, K, r, c + 1) << 4));
        for (int g = 0; g < G; ++g) s_rm[(int64_t)g * N + r] = or_bf16_to_f32(s_sw[nk_scale_off(G, r, g)]);
    }
}

/* cuda_kernels.cu:2932-2978 dequantize_nunchaku_to_bf16_kernel. */
void or_dequant_nunchaku_bf16(const uint8_t* q_sw, const uint16_t* s_sw, int N, int K, int G, uint16_t* out) {
    const int gs = K / G;
    for (int r = 0; r < N; ++r)
        for (int c = 0; c < K; ++c) {
            const float s = or_bf16_to_f32(s_sw[nk_scale_off(G, r, c / gs)]);
            out[(int64_t)r * K + c] = or_f32_to_bf16((float)nib_signed(nk_nibble(q_sw, K, r, c)) * s);
        }
}

/* cuda_kernels.cu:3503-3562 unswizzle_lora_weights_kernel. */
void or_unswizzle_lora(const uint16_t* packed, int rows, int cols, int is_down, uint16_t* out) {
    const int R = cols;
    for (int row = 0; row < rows; ++row)
        for (int col = 0; col < cols; ++col) {
            const int sr = is_down ? col : row, sc = is_down ? row : col;
            const int cf = is_down ? sc / 16 : sr / 16, rf = is_down ? sr / 16 : sc / 16;
            const int ln = sr % 16, lk = sc % 16;
            const int64_t f = (int64_t)cf * 16 * R + rf * 256 + (ln % 8) * 32 + ((lk % 8) / 2) * 8 + (ln / 8) * 4 +
                              (lk / 8) * 2 + lk % 2;
            out[(int64_t)row * cols + col] = packed[f];
        }
}
