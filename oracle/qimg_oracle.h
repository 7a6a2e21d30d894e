/*
 * qimg_oracle.h — CPU restatement of qwen-image.cu's quantized-linear and
 * SageAttention hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library gives the expected values: tests, the smoke
 * check and the bench's CPU-baseline leg call it to produce expected values.
 * No product code path links or calls it.
 *
 * Every function states the reference file:line it restates. Arithmetic is
 * IEEE-754 fp32 in the same operation order as the reference, except where
 * the reference relies on nvcc --use_fast_math approximations (rsqrtf, `/`,
 * tanhf, ex2.approx, rcp.approx): there the oracle uses the correctly
 * rounded operation.
 *
 * Each function is pinned by checks independent of its own code (closed
 * forms, explicit Hadamard matrices, numpy/torch conversions, brute-force
 * integer products, hand-derived known answers, float64 attention) in
 * tests/test_oracle_pins.py, and frozen by the fixtures of tests/golden/.
 * No function is left unpinned. What no check here can pin is the reference
 * binary's fast-math rounding on exact ties (see tests/test_oracle_pins.py).
 */
#ifndef QIMG_ORACLE_H
#define QIMG_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar conversions (bit-level, round-to-nearest-even) ------------ */
float    or_bf16_to_f32(uint16_t h);
uint16_t or_f32_to_bf16(float f);
float    or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);
/* OCP FP8 E4M3FN (no inf, max 448), RNE, saturating to +-448; NaN -> 0x7f. */
uint8_t  or_f32_to_e4m3(float f);
float    or_e4m3_to_f32(uint8_t b);

/* a1: cuda_kernels.cuh:253  hadamard_block_size(K) = K & -K */
int   or_hadamard_block_size(int K);
/* Normalisation factor 1/sqrt(hbs), correctly rounded to fp32.
 * Reference: rsqrtf((float)block_size), cuda_kernels.cu:2243, 2538. */
float or_fwht_norm(int hbs);

/* a2: cuda_kernels.cu:2209-2254 fwht_inplace_kernel. Row-wise block-diagonal
 * FWHT, stages half = 1,2,...,hbs/2 in that order, (a,b) <- (a+b, a-b),
 * then multiply by or_fwht_norm(hbs). In place on x[M,K]. */
void or_fwht_rows(float* x, int64_t M, int K, int hbs);

/* a3: cuda_kernels.cu:2385-2416 quantize_per_row_fp32_kernel.
 * amax = max|row|; scale = amax/127; inv = amax>0 ? 127/amax : 0;
 * q = clamp(rne(v*inv), -128, 127). */
void or_quant_rows_int8(const float* x, int64_t M, int K, int8_t* q, float* scales);

/* a4: cuda_kernels.cu:2830-2862 quantize_weight_tensor. BF16 [N,K] ->
 * FP32 -> FWHT(hbs = K & -K, if > 1) -> a3. Returns hbs. */
int or_quantize_weight_bf16(const uint16_t* w, int N, int K, int8_t* q, float* scales);

/* a5/a6: cuda_kernels.cu:2493-2619 fwht_quantize_kernel<T> and
 * quantize_activation_per_token_*: per token FWHT (hbs > 1) then a3.
 * x_is_bf16 selects the input type (else fp32). */
void or_quantize_activation(const void* x, int x_is_bf16, int64_t M, int K, int hbs,
                            int8_t* q, float* scales);

/* a7: cuda_kernels.cu:2711-2721 cublasGemmEx s8*s8->s32, C[m,n] = sum_k
 * A[m,k] * W[n,k], exact. Rows [m0, m1) only (use 0, M for all). */
void or_gemm_s8s8s32(const int8_t* A, const int8_t* W, int64_t M, int N, int K,
                     int64_t m0, int64_t m1, int32_t* C);

/* a8: cuda_kernels.cu:2623-2668 dequantize_and_bias / dequantize_bias_gelu.
 * v = ((float)acc * as[m]) * ws[n]; v += bf16 bias[n]; optional GELU-tanh
 * 0.5 v (1 + tanh(0.7978845608 (v + 0.044715 v^3))). bias may be NULL. */
void or_dequant_epilogue(const int32_t* C, const float* as, const float* ws,
                         const uint16_t* bias_bf16, int64_t M, int N, int gelu, float* out);

/* ---- fp8-e4m3 mode (no reference counterpart: new mode) -------------- */
/* Same shape as a3 with the e4m3 range: scale = amax/448,
 * inv = amax>0 ? 448/amax : 0, q = e4m3_rne_sat(v*inv). */
void or_quant_rows_fp8(const float* x, int64_t M, int K, uint8_t* q, float* scales);
/* fp8 analogue of a7 + a8: C[m,n] = sum_k e4m3(A[m,k]) e4m3(W[n,k]) in
 * double, then the a8 epilogue on the (rounded to fp32) sum. */
void or_gemm_fp8_epilogue(const uint8_t* A, const uint8_t* W, const float* as, const float* ws,
                          const uint16_t* bias_bf16, int64_t M, int N, int K,
                          int64_t m0, int64_t m1, int gelu, float* out);

/* ---- SageAttention (sageattention_sm80.cu) --------------------------- */
/* a12: :759-773 sageattention_k_mean_kernel. mean[h,d] = (sequential fp32
 * sum over s of k[h,s,d]) / max(S,1). */
void or_sage_k_mean(const uint16_t* k_f16, int BH, int S, int D, float* mean);
/* a13: :775-824. Per (head, 128-token block b, warp w, lane group g): tokens
 * b*128 + w*32 + g + 8i, i = 0..3. amax starts at 1e-7; scale = amax/127 +
 * 1e-7; q = sat_rne(v * (1/scale)). Scales [BH, ceil(S/128)*32]. */
void or_sage_quant_q(const uint16_t* q_f16, int BH, int S, int D, int8_t* q_out, float* q_scale);
/* a14: :826-886. Per (head, 64-token block b, group g in 0..3): tokens
 * b*64 + 2g + {0,1} + 8i, i = 0..7, values k - mean[h,d]. Scales
 * [BH, ceil(S/64)*4]. */
void or_sage_quant_k(const uint16_t* k_f16, const float* mean, int BH, int S, int D,
                     int8_t* k_out, float* k_scale);
/* a15/a16: :47-674 qk_int_sv_f16_attn_kernel with CTA_Q=128, CTA_K=64,
 * per-thread Q/K scales, fp32 PV accumulation, fp16 output. Online softmax in
 * base 2 over 64-key tiles, m0 = -5e6, d0 = 1, P rounded to fp16 before the
 * row sum and before PV, O/d rounded to fp16. Query rows [q0, q1) of every
 * head are computed (0, S for all); out is fp16 [BH, S, D]. */
void or_sage_attn(const int8_t* q, const int8_t* k, const uint16_t* v_f16,
                  const float* q_scale, const float* k_scale, int BH, int S, int D,
                  float sm_scale, int causal, int q0, int q1, uint16_t* out_f16);
/* Full a17 composition: fp16 q,k,v -> k-mean -> quant -> attention. */
void or_sage_attention_fp16io(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                              int BH, int S, int D, float sm_scale, int causal,
                              uint16_t* out_f16);

/* Threads used by the parallel loops (OpenMP); <= 0 leaves the default. */
void or_set_threads(int n);
int  or_get_threads(void);

/* ---- INT4 paths (cuda_kernels.cu:2864-4532; qimg_oracle_int4.c) ------ */
extern const float OR_NF4_GRID[16];
/* :2876-2917 packed nibbles [N,K/2] (even column low) -> bf16 [N,K]:
 * NF4_GRID[n]*s, (signed n)*s or (n-8)*s; scales [N,G] or [G,N]. */
void or_dequant_int4_bf16(const uint8_t* qw, const float* scales, int N, int K, int gs, int nf4,
                          int scales_gn, int signed_int4, uint16_t* out);
/* :3226-3288 linear INT4 weight quantizer (offset 8, [-7,7]). */
void or_quant_int4_linear(const float* r, int N, int K, int gs, uint8_t* qw, float* scales);
/* :3290-3357 NF4 weight quantizer (nearest grid code, first on ties). */
void or_quant_int4_nf4(const float* r, int N, int K, int gs, uint8_t* qw, float* scales);
/* :3575-3636 / :3650-3705 activation INT4 quant, optional smooth divide and
 * bf16 copy; scales [G, M]. */
void or_quant_act_int4(const float* x, const float* smooth, int M, int K, int gs, uint16_t* bf16_out,
                       uint8_t* packed, float* scales);
/* :3732-3854, :4117-4255 W4A4 GEMM, rows [m0, m1) into out[(m1-m0), N]. */
void or_w4a4_gemm(const uint8_t* act, const uint8_t* wgt, const float* as, const float* ws, int64_t M,
                  int N, int K, int gs, int accumulate, const uint16_t* bias, int64_t m0, int64_t m1,
                  float* out);
/* :3059-3091 AWQ repack, :3002-3038 AWQ dequant, :3106-3153 AWQ GEMV. */
void or_awq_repack(const int32_t* qw, int OC, int IC, int32_t* out);
void or_dequant_awq_bf16(const int32_t* qw, const uint16_t* wscales, const uint16_t* wzeros, int OC, int IC,
                         int gs, int ncomp, uint16_t* out);
void or_awq_gemv(const float* x, const int32_t* qw_rep, const uint16_t* wscales, const uint16_t* wzeros,
                 const uint16_t* bias, int OC, int IC, int gs, int ncomp, float* out);
/* :3431-3487 nunchaku weight unswizzle, :2932-2978 nunchaku dequant,
 * :3503-3562 LoRA unswizzle. */
void or_unswizzle_nunchaku(const uint8_t* q_sw, const uint16_t* s_sw, int N, int K, int G, uint8_t* q_rm,
                           float* s_rm);
void or_dequant_nunchaku_bf16(const uint8_t* q_sw, const uint16_t* s_sw, int N, int K, int G, uint16_t* out);
void or_unswizzle_lora(const uint16_t* packed, int rows, int cols, int is_down, uint16_t* out);

#ifdef __cplusplus
}
#endif
#endif
