/*
 * qimg_hot.h — C ABI of the MI355X (gfx950) quantized-linear and
 * SageAttention hot path of the qwen-image MMDiT.
 *
 * Plain pointers, sizes and a hipStream_t (passed as void*; NULL = the null
 * stream). Every entry point validates its arguments on the host before any
 * HIP call and returns a qimg_status; qimg_last_error() gives the message of
 * the last failure on the calling thread. Device pointers must be 16-byte
 * aligned. Calls are asynchronous on `stream` unless stated otherwise.
 *
 * Each function names the reference interface it replaces (file:line in the
 * qwen-image.cu tree).
 */
#ifndef QIMG_HOT_H
#define QIMG_HOT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    QIMG_OK = 0,
    QIMG_ERR_INVALID_ARG = 1,  /* null pointer, bad size, bad enum */
    QIMG_ERR_UNSUPPORTED = 2,  /* valid request this library does not implement */
    QIMG_ERR_SCRATCH = 3,      /* caller scratch smaller than required */
    QIMG_ERR_HIP = 4           /* a HIP runtime call failed */
} qimg_status;

/* Element types. Replaces DType (tensor.h:39) plus FP16 and FP8_E4M3. */
typedef enum {
    QIMG_FP32 = 0,
    QIMG_BF16 = 1,
    QIMG_FP16 = 2,
    QIMG_INT8 = 3,
    QIMG_INT32 = 4,
    QIMG_FP8_E4M3 = 5  /* OCP E4M3FN: max 448, no inf */
} qimg_dtype;

/* Quantization modes. Replaces QuantMode::INT8_HADAMARD
 * (cuda_kernels.cuh:183); FP8_HADAMARD is new (same Hadamard front end,
 * e4m3 values, scale = amax/448). */
typedef enum {
    QIMG_QM_INT8_HADAMARD = 0,
    QIMG_QM_FP8_HADAMARD = 1
} qimg_quant_mode;

const char* qimg_status_string(int status);
/* Message of the last failing call on this thread ("" if none). */
const char* qimg_last_error(void);
/* Library version string. */
const char* qimg_version(void);

/* ---- sizing helpers --------------------------------------------------- */

/* hadamard_block_size (cuda_kernels.cuh:253): K & -K. */
int qimg_hadamard_block_size(int K);

/* int8_scratch_bytes (cuda_kernels.cuh:311-319), same formula:
 * align256(max(M*K, M*N)*4) + align256(M*K) + align256(4*M).
 * qimg_linear needs only align256(M*K) + align256(4*M) of it (the int32 GEMM
 * result is never materialised), so any buffer sized by this formula works. */
int64_t qimg_int8_scratch_bytes(int M, int K, int N);

/* ---- Hadamard + quantization ----------------------------------------- */

/* fwht_inplace (cuda_kernels.cuh:250, cuda_kernels.cu:2209-2254): in-place
 * normalised block-diagonal FWHT of each row of data[M,K] (fp32),
 * hbs a power of two dividing K, hbs <= 32768. */
int qimg_fwht_inplace(float* data, int M, int K, int hbs, void* stream);

/* quantize_per_row_fp32 (cuda_kernels.cuh:260-261, cuda_kernels.cu:2385-2416):
 * per-row symmetric int8, scale = amax/127. */
int qimg_quantize_per_row_fp32(const float* x, int8_t* out, float* scales, int M, int K,
                               void* stream);

/* quantize_activation_int8_hadamard_{fp32,bf16} (cuda_kernels.cuh:277-280,
 * cuda_kernels.cu:2493-2619), fused FWHT + per-token quantization.
 *   x        [M,K], x_dtype QIMG_FP32 or QIMG_BF16
 *   hbs      Hadamard block (1 = no rotation), power of two dividing K
 *   mode     QIMG_QM_INT8_HADAMARD (int8 out, scale amax/127) or
 *            QIMG_QM_FP8_HADAMARD (e4m3 out, scale amax/448)
 *   q_out    [M,K] int8 or e4m3 bytes; scales_out [M] fp32 */
int qimg_quantize_activation(const void* x, int x_dtype, int M, int K, int hbs, int mode,
                             void* q_out, float* scales_out, void* stream);

/* quantize_weight_tensor (cuda_kernels.cuh:308, cuda_kernels.cu:2830-2862):
 * w [N,K] bf16 (or fp32) -> FWHT with hbs = K & -K -> per-row quantization.
 * Writes q_out [N,K], scales_out [N] and *hbs_out (host int, may be NULL).
 * Synchronous: returns after the device work has finished, as the
 * reference does (cudaDeviceSynchronize at :2860). */
int qimg_quantize_weight(const void* w, int w_dtype, int N, int K, int mode,
                         void* q_out, float* scales_out, int* hbs_out, void* stream);

/* ---- quantized linear ------------------------------------------------- */

/* linear_forward_int8_prequantized (cuda_kernels.cuh:297-300,
 * cuda_kernels.cu:2734-2773) with the dequant epilogue fused into the GEMM:
 *   out[m,n] = act_scale[m] * w_scale[n] * sum_k act_q[m,k] w_q[n,k]
 *              + bias[n]  (then GELU-tanh if gelu != 0)
 * act_q [M,K], w_q [N,K] in `mode`'s element type; bias bf16 [N] or NULL;
 * out [M,N] with out_dtype QIMG_FP32 (the reference's type) or QIMG_BF16.
 * No scratch is needed. */
int qimg_linear_prequantized(const void* act_q, const float* act_scales, int M, int K,
                             const void* w_q, const float* w_scales, int N, int mode,
                             const uint16_t* bias_bf16, void* out, int out_dtype, int gelu,
                             void* stream);

/* Kernel selection for qimg_linear_prequantized / qimg_linear when K is a
 * multiple of 64. No counterpart in the reference (cuBLAS picks its own
 * algorithm); it exists for tests and tuning, which compare the kernels on
 * one shape. AUTO (the default) takes the vector-ALU GEMV for M <= 4
 * (int8, and e4m3 with fp32 accumulation), 32x32 tiles for M <= 32, 64x64 tiles when fewer than 64 tiles of
 * 256x256 would cover the output (int8 of 128 rows or more: fewer than 32),
 * and the large-tile kernel otherwise: 256 rows of 256, 224 or 192 columns,
 * or int8 128x128 tiles (two per CU), whichever's rounds of tiles on the
 * device's CUs, each
 * weighted by the tile's share of a 256x256 tile's time, add up to least
 * (4096 x 3072: one full round of 256x192; int8 4352 x 3072: one round of
 * 256x224; int8 2048 x 3072: one round of 128x128). e4m3 takes 256 or 192
 * columns. LARGE_192, LARGE_224 and LARGE_128 force those tiles (e4m3 runs
 * 224 and 128 as 256x256); qimg_linear_bf16's large-tile path follows
 * LARGE_TILE and LARGE_192 too.
 * GEMV with M > 4 runs the 32x32 tiles. Process-wide; returns
 * QIMG_OK, or QIMG_ERR_INVALID_ARG for an unknown value. All choices give
 * identical int8 results. */
enum {
    QIMG_LINEAR_AUTO = 0,
    QIMG_LINEAR_LARGE_TILE = 1,
    QIMG_LINEAR_SMALL_32 = 2,
    QIMG_LINEAR_SMALL_64 = 3,
    QIMG_LINEAR_GEMV = 4,
    QIMG_LINEAR_LARGE_192 = 5,
    QIMG_LINEAR_LARGE_224 = 6,
    QIMG_LINEAR_LARGE_128 = 7
};
int qimg_set_linear_kernel(int which);
int qimg_get_linear_kernel(void);

/* dequantize_and_bias / dequantize_bias_gelu (cuda_kernels.cuh:282-291,
 * cuda_kernels.cu:2623-2668): out[m,n] = acc[m,n] * act_scale[m] * w_scale[n]
 * + bias[n] (then GELU-tanh if gelu != 0), acc int32 [M,N], out fp32 [M,N],
 * bias bf16 [N] or NULL. The same arithmetic as the fused epilogue of
 * qimg_linear_prequantized. */
int qimg_dequantize_bias(const int32_t* acc, const float* act_scales, const float* w_scales,
                         const uint16_t* bias_bf16, float* out, int M, int N, int gelu,
                         void* stream);

/* linear_forward_int8 / linear_forward_int8_bf16in (cuda_kernels.cuh:294-296,
 * 303-305; cuda_kernels.cu:2674-2732, 2776-2827): activation FWHT+quant into
 * `scratch`, then qimg_linear_prequantized. scratch_bytes must be at least
 * align256(M*K) + align256(4*M) (qimg_int8_scratch_bytes also suffices). */
int qimg_linear(const void* x, int x_dtype, int M, int K,
                const void* w_q, const float* w_scales, int N, int hbs, int mode,
                const uint16_t* bias_bf16, void* out, int out_dtype, int gelu,
                void* scratch, int64_t scratch_bytes, void* stream);

/* linear_forward_bf16 / linear_forward_bf16_bf16in (cuda_kernels.cu:4534-4596),
 * the QuantMode::BF16 path of linear_forward_quantized[_bf16in]
 * (cuda_kernels.cu:4599-4635) for layers a checkpoint keeps in bf16
 * (transformer.h:188-193: img_in, txt_in, norm_out, proj_out at
 * transformer.cu:396-419, 874-895):
 *   out[m,n] = sum_k bf16(x[m,k]) w[n,k] + bias[n]  (then GELU-tanh if gelu)
 * x [M,K] QIMG_FP32 (rounded to bf16, nearest even, as fp32_to_bf16 at
 * cuda_kernels.cu:33-42) or QIMG_BF16; w bf16 [N,K]; bias bf16 [N] or NULL;
 * out fp32 [M,N]; fp32 accumulation. No scratch is needed. */
int qimg_linear_bf16(const void* x, int x_dtype, int M, int K, const uint16_t* w_bf16, int N,
                     const uint16_t* bias_bf16, float* out, int gelu, void* stream);

/* Bytes of the static device array behind qimg_linear_noalloc (per GPU). */
#define QIMG_NOALLOC_SCRATCH_BYTES (64ll << 20)

/* qimg_linear without caller scratch and without any device allocation.
 * No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). The arguments and results are those of qimg_linear; the
 * quantized activations and their scales go to a static device array of
 * QIMG_NOALLOC_SCRATCH_BYTES that each GPU the library runs on holds until
 * the process ends. align256(M*K) + align256(4*M) must fit in it, else
 * QIMG_ERR_SCRATCH (e.g. M = 4352 rows of K = 12288 fit, 8192 rows do not).
 * Every call on one GPU shares that GPU's array and the array keeps the last
 * call's contents: calls whose kernels can overlap on one GPU (different
 * streams without ordering between them, or several host threads) race. */
int qimg_linear_noalloc(const void* x, int x_dtype, int M, int K,
                        const void* w_q, const float* w_scales, int N, int hbs, int mode,
                        const uint16_t* bias_bf16, void* out, int out_dtype, int gelu,
                        void* stream);

/* ---- SageAttention ---------------------------------------------------- */

/* Scratch needed by qimg_sage_attention for BH heads of S tokens, head dim D:
 * Q/K int8, V re-laid for the PV product, scales and the K mean. */
int64_t qimg_sage_scratch_bytes(int BH, int S, int D);

/* sageattention_k_mean_kernel (sageattention_sm80.cu:759-773): k fp16
 * [BH,S,D] -> mean fp32 [BH,D], sequential fp32 sum over s / max(S,1). */
int qimg_sage_k_mean(const uint16_t* k_f16, float* mean, int BH, int S, int D, void* stream);

/* sageattention_query_per_thread_int8_kernel (sageattention_sm80.cu:775-824):
 * q fp16 [BH,S,D] -> int8 [BH,S,D] + scales fp32 [BH, ceil(S/128)*32]. */
int qimg_sage_quant_q(const uint16_t* q_f16, int8_t* q_out, float* q_scale, int BH, int S,
                      int D, void* stream);

/* sageattention_key_per_thread_int8_kernel (sageattention_sm80.cu:826-886):
 * (k - mean) fp16 [BH,S,D] -> int8 [BH,S,D] + scales fp32 [BH, ceil(S/64)*4]. */
int qimg_sage_quant_k(const uint16_t* k_f16, const float* mean, int8_t* k_out, float* k_scale,
                      int BH, int S, int D, void* stream);

/* qk_int_sv_f16_attn_kernel via sageattention_launch_accum_f32
 * (sageattention_sm80.cu:47-674, 896-961): attention on pre-quantized
 * Q/K (scales laid out as above) and fp16 V [BH,S,D]. out [BH,S,D] in
 * out_dtype QIMG_FP16, QIMG_FP32 (fp16-rounded, as the reference) or
 * QIMG_BF16. D must be 64 or 128. `scratch` receives the re-laid V
 * (qimg_sage_scratch_bytes covers it). */
int qimg_sage_attn_quantized(const int8_t* q, const int8_t* k, const uint16_t* v_f16,
                             const float* q_scale, const float* k_scale, void* out,
                             int out_dtype, int BH, int S, int D, float sm_scale, int causal,
                             void* scratch, int64_t scratch_bytes, void* stream);

/* attention_forward_sage_sm80_fp16io (cuda_kernels.cuh:560-562,
 * sageattention_sm80.cu:965-1027): fp16 q,k,v [BH,S,D] -> out [BH,S,D]
 * (out_dtype as above; the reference writes QIMG_FP32). Uses caller scratch
 * of qimg_sage_scratch_bytes(BH,S,D) bytes instead of a hidden static
 * workspace. */
int qimg_sage_attention(const uint16_t* q_f16, const uint16_t* k_f16, const uint16_t* v_f16,
                        void* out, int out_dtype, float sm_scale, int BH, int S, int D,
                        int causal, void* scratch, int64_t scratch_bytes, void* stream);

/* ---- MMDiT joint block: the operations around the hot path ------------ */

/* silu_fp32 (cuda_kernels.cu:1881-1893): out[i] = x[i] / (1 + exp(-x[i])). */
int qimg_silu(const float* x, float* out, int64_t n, void* stream);

/* layer_norm_modulate_fp32 (cuda_kernels.cu:1799-1859), per row of `dim`:
 * (x - mean) * rsqrt(var + eps) * (1 + scale) + shift, fp32 [rows, dim];
 * dim a multiple of 4, at most 4096. */
int qimg_layernorm_modulate(const float* x, const float* shift, const float* scale, float* out,
                            int rows, int dim, float eps, void* stream);

/* qimg_layernorm_modulate followed by the FWHT + quantization of
 * qimg_quantize_activation (fwht_quantize_fp32, cuda_kernels.cu:2493-2601)
 * in one pass, for a LayerNorm whose only consumer is a quantized linear
 * (transformer.cu:526-606, 754-785): q_out int8 or e4m3 [rows, dim],
 * q_scales fp32 [rows], bit-identical to the two calls. */
int qimg_layernorm_modulate_quant(const float* x, const float* shift, const float* scale, int rows, int dim,
                                  int hbs, int mode, float eps, void* q_out, float* q_scales, void* stream);

/* rms_norm_fp32 on the per-head Q or K rows (cuda_kernels.cu:1656-1692)
 * + concat_transpose_fused_fp32 (transformer.cu:106-130, text tokens
 * first) + rope_apply_fp32_to_fp16 (cuda_kernels.cu:1935-1971), fused:
 * txt [n_txt, H*128] and img [n_img, H*128] fp32 -> out fp16
 * [H, n_txt + n_img, 128]. norm_txt / norm_img are the bf16 [128] RMSNorm
 * weights (norm_added_q / norm_q), pe is [n_txt + n_img, 64, 4] fp32
 * (cos, -sin, sin, cos) as RoPE::gen_qwen_image_pe (rope.h:154-160) lays it
 * out. With norm_txt == NULL only the concat/transpose/fp16 is applied (the
 * V path, transformer.cu:649-650). */
int qimg_joint_heads_f16(const float* txt, const float* img, const uint16_t* norm_txt,
                         const uint16_t* norm_img, const float* pe, uint16_t* out, int n_txt, int n_img,
                         int H, float eps, void* stream);

/* transpose_split_fused_fp32 (transformer.cu:84-104) on an fp16 attention
 * output [H, n_txt + n_img, 128]: -> txt [n_txt, H*128], img [n_img, H*128]
 * fp32. */
int qimg_split_heads(const uint16_t* attn_f16, float* txt, float* img, int n_txt, int n_img, int H,
                     void* stream);

/* gate_add_fp32f (cuda_kernels.cu:2181-2197): out[r,c] = x[r,c] +
 * gate[c] * y[r,c], fp32 [rows, dim], dim a multiple of 4; out may be x. */
int qimg_gate_add(const float* x, const float* gate, const float* y, float* out, int rows, int dim,
                  void* stream);

/* One quantized linear of a block: weight [N, K] (int8 or e4m3 bytes),
 * fp32 scales [N], Hadamard block size, mode, bf16 bias [N] or NULL. */
typedef struct {
    const void* w;
    const float* scales;
    int N, K, hbs, mode;
    const uint16_t* bias;
} qimg_qlinear;

/* The weights of one MMDiT joint block, field for field as
 * TransformerWeights::Block (transformer.h:89-140): hidden 3072 (24 heads
 * of 128), MLP 12288, modulation 6 x 3072 per stream. */
typedef struct {
    qimg_qlinear img_mod, txt_mod;
    qimg_qlinear to_q, to_k, to_v, add_q_proj, add_k_proj, add_v_proj;
    qimg_qlinear to_out, to_add_out;
    qimg_qlinear img_mlp_fc1, img_mlp_fc2, txt_mlp_fc1, txt_mlp_fc2;
    const uint16_t* norm_q;        /* bf16 [128] */
    const uint16_t* norm_k;
    const uint16_t* norm_added_q;
    const uint16_t* norm_added_k;
} qimg_mmdit_block;

/* Profile categories of qimg_mmdit_block_forward, in the order of the
 * reference's PROFILE_BLOCK report (transformer.cu:843-857). RMSNorm,
 * concat/transpose and RoPE of Q/K run as one fused kernel here: its time
 * is reported under QK_NORM, the V concat/transpose under
 * CONCAT_TRANSPOSE, and ROPE stays about 0. The LayerNorms write the
 * quantized input of the next linear (their time includes that
 * quantization), and the gated residuals run in the epilogues of the
 * out-projection and fc2, so GATE_ATTN and GATE_MLP stay about 0 and their
 * work is counted in OUT_GEMM and MLP_GEMM. */
enum {
    QIMG_PROF_MODULATION = 0,
    QIMG_PROF_ATTN_NORM,
    QIMG_PROF_QKV_GEMM,
    QIMG_PROF_QK_NORM,
    QIMG_PROF_CONCAT_TRANSPOSE,
    QIMG_PROF_ROPE,
    QIMG_PROF_ATTENTION,
    QIMG_PROF_TRANSPOSE_SPLIT,
    QIMG_PROF_OUT_GEMM,
    QIMG_PROF_GATE_ATTN,
    QIMG_PROF_MLP_NORM,
    QIMG_PROF_MLP_GEMM,
    QIMG_PROF_GATE_MLP,
    QIMG_PROF_COUNT
};

/* Scratch bytes for qimg_mmdit_block_forward at n_img + n_txt tokens. */
int64_t qimg_mmdit_block_scratch_bytes(int n_img, int n_txt);

/* One iteration of the MMDiT joint-block loop (transformer.cu:506-817):
 * modulation from silu(t_emb), LayerNorm + modulate, shared-quant QKV
 * linears, per-head RMSNorm + RoPE, joint SageAttention (text tokens
 * first), out-projections, gated residual, LayerNorm + modulate, GELU MLP,
 * gated residual. img [n_img, 3072] and txt [n_txt, 3072] fp32 are updated
 * in place; t_emb is fp32 [3072]; pe is [n_txt + n_img, 64, 4] fp32. With
 * prof_ms != NULL the stream is synchronised once at the end and the
 * QIMG_PROF_COUNT category times (ms) are written there. */
int qimg_mmdit_block_forward(const qimg_mmdit_block* block, float* img, float* txt, const float* t_emb,
                             const float* pe, int n_img, int n_txt, void* scratch, int64_t scratch_bytes,
                             float* prof_ms, void* stream);

/* Scratch bytes for qimg_mmdit_blocks_forward over `batch` sequences of
 * n_img + n_txt tokens. */
int64_t qimg_mmdit_blocks_scratch_bytes(int n_img, int n_txt, int batch);

/* The joint-block loop of TransformerWeights::forward
 * (transformer.cu:497-836): blocks[0 .. n_blocks) in order, each as
 * qimg_mmdit_block_forward, over `batch` sequences that share t_emb and pe
 * and have the same n_img and n_txt (batch 2 runs the two classifier-free-
 * guidance forwards of main.cu:761-773 together, each row and head
 * computing exactly what it computes alone). img is [batch, n_img, 3072],
 * txt [batch, n_txt, 3072], fp32, updated in place. With prof_ms != NULL
 * the stream is synchronised after each block and prof_ms holds the
 * category times summed over the blocks. */
int qimg_mmdit_blocks_forward(const qimg_mmdit_block* blocks, int n_blocks, float* img, float* txt,
                              const float* t_emb, const float* pe, int n_img, int n_txt, int batch, void* scratch,
                              int64_t scratch_bytes, float* prof_ms, void* stream);

/* ---- INT4 paths (cuda_kernels.cu:2864-4532) ----------------------------
 * Packed INT4 tensors hold two columns per byte, the even column in the
 * low nibble. Nibbles are NF4 codes, offset-8 linear values (value = n - 8)
 * or two's complement values, as each entry point states. The arithmetic of
 * every entry point follows the reference's source order; as for the INT8
 * path, its --use_fast_math approximations are not reproduced. */

/* dequantize_int4_to_bf16 (cuda_kernels.cu:2876-2929): qweight [N, K/2] ->
 * bf16 [N, K]; NF4_GRID[n]*s (nf4_grid), (signed n)*s (signed_int4) or
 * (n-8)*s; scales fp32 [N, K/group_size] or, with scales_gn, [K/group_size, N].
 * K % 8 == 0, K % group_size == 0. */
int qimg_dequantize_int4_bf16(const uint8_t* qweight, const float* scales, uint16_t* out, int N, int K,
                              int group_size, int nf4_grid, int scales_gn, int signed_int4, void* stream);

/* quantize_int4_per_group (NF4, cuda_kernels.cu:3290-3368) or, with
 * nf4_grid = 0, the linear quantizer (quantize_linear_int4_per_group_kernel,
 * :3226-3288: scale = amax/7, q = clamp(roundf(v*7/amax), -7, 7) + 8).
 * residual fp32 [N, K] -> qweight [N, K/2], scales fp32 [N, K/group_size]. */
int qimg_quantize_int4_per_group(const float* residual, uint8_t* qweight, float* scales, int N, int K,
                                 int group_size, int nf4_grid, void* stream);

/* quantize_activation_int4 (cuda_kernels.cu:3575-3648): x fp32 [M, K] ->
 * two's complement nibbles act_packed [M, K/2], act_scales fp32
 * [K/group_size, M] (scale amax/7). group_size 32, 64 or 128. */
int qimg_quantize_activation_int4(const float* x, uint8_t* act_packed, float* act_scales, int M, int K,
                                  int group_size, void* stream);

/* fused_smooth_bf16_quant (cuda_kernels.cu:3650-3730): v = x / smooth[k]
 * (smooth may be NULL), bf16_out = bf16(v) [M, K], then
 * qimg_quantize_activation_int4 of v. */
int qimg_fused_smooth_bf16_quant(const float* x, const float* smooth, uint16_t* bf16_out, uint8_t* act_packed,
                                 float* act_scales, int M, int K, int group_size, void* stream);

/* w4a4_gemm (cuda_kernels.cu:4257-4313; kernels :3732-3854, :4117-4255):
 * out[m,n] = sum over groups g in order of ((float)d_g[m,n] * act_scales[g,m])
 * * wgt_scales[g,n] (d_g the exact int32 dot product of the group's signed
 * nibbles), plus bias[n] (bf16, or NULL); accumulate != 0 adds the result to
 * out. act_packed [M, K/2] and wgt_packed [N, K/2] two's complement nibbles,
 * act_scales [G, M], wgt_scales [G, N] fp32, group_size % 64 == 0. The
 * reference's register-direct kernel reads an mma.sync fragment order; this
 * entry point reads the row-major packing (qweight_rowmajor). */
int qimg_w4a4_gemm(const uint8_t* act_packed, const uint8_t* wgt_packed, const float* act_scales,
                   const float* wgt_scales, float* out, int M, int N, int K, int group_size, int accumulate,
                   const uint16_t* bias_bf16, void* stream);

/* One INT4 linear layer: QuantizedWeight's INT4_SVD fields
 * (cuda_kernels.cuh:194-213). The residual is W4A4 when w4a4_qweight is set
 * (two's complement nibbles [N, K/2], w4a4_wscales fp32 [K/group_size, N]: the
 * unswizzled nunchaku form), otherwise W4A16 over qweight [N, K/2] (NF4 or
 * offset-8 codes, nf4_grid) and scales4 fp32 [N, K/group_size]. svd_up bf16
 * [N, rank] and svd_down bf16 [K, rank] are the low-rank factors; smooth fp32
 * [K] is optional; had_block_size > 1 rotates x before the W4A16 residual.
 * w4a16_nunchaku != 0 (with w4a4_qweight NULL) is the reference's W4A16
 * fallback for nunchaku weights (cuda_kernels.cu:4443-4470, taken there under
 * FORCE_W4A16 or without the MMA copy): qweight holds the unswizzled two's
 * complement nibbles, scales4 the fp32 [K/group_size, N] scales, nf4_grid and
 * had_block_size are ignored, and the residual's input is bf16(x / smooth)
 * with no rotation. */
typedef struct qimg_int4_weight {
    int N, K, rank, group_size;
    int nf4_grid, had_block_size;
    const uint8_t* qweight;
    const float* scales4;
    const uint8_t* w4a4_qweight;
    const float* w4a4_wscales;
    const uint16_t* svd_up;
    const uint16_t* svd_down;
    const float* smooth;
    int w4a16_nunchaku;
} qimg_int4_weight;

/* int4_scratch_bytes (cuda_kernels.cuh:475-487), or more where this
 * library's layout needs it (rank > K/2). */
int64_t qimg_int4_scratch_bytes(int M, int K, int N, int svd_rank);

/* linear_forward_int4 (cuda_kernels.cu:4332-4532): x fp32 [M, K] ->
 * out fp32 [M, N] = x_lr . svd_down . svd_up^T (x_lr = bf16 of x or of
 * x / smooth; the low-rank product rounded to bf16) + the residual (W4A16:
 * bf16 of the smoothed, rotated x times the dequantized weight; W4A4:
 * qimg_w4a4_gemm of the INT4-quantized smoothed x) + bias, then GELU-tanh
 * if gelu. scratch >= qimg_int4_scratch_bytes(M, K, N, rank). */
int qimg_linear_int4(const float* x, int M, const qimg_int4_weight* w, const uint16_t* bias_bf16, float* out,
                     int gelu, void* scratch, int64_t scratch_bytes, void* stream);

/* bf16_to_fp32 (cuda_kernels.cu:22-31): exact widening of n values. */
int qimg_bf16_to_fp32(const uint16_t* in, float* out, int64_t n, void* stream);

/* apply_smooth_div (cuda_kernels.cu:2257-2271) and smooth_hadamard_inplace
 * (:2273-2324): out = FWHT_hbs(x / smooth[k]) row by row, fp32 [M, K]
 * (smooth may be NULL; hbs 1: no transform). out may be x. */
int qimg_smooth_hadamard(const float* x, const float* smooth, float* out, int M, int K, int hbs, void* stream);

/* repack_awq_to_transposed (cuda_kernels.cu:3059-3102): AWQ kInterleave=4
 * qweight int32 [OC/4, IC/2] -> [IC/8, OC], word (i, oc) holding the nibbles
 * of inputs 8i .. 8i+7, low first. */
int qimg_awq_repack(const int32_t* qweight_awq, int32_t* qweight_out, int OC, int IC, void* stream);

/* dequantize_awq_to_bf16 (cuda_kernels.cu:3002-3057): bf16 [OC, IC] in the
 * de-interleaved channel order, q * wscales + wzeros (bf16 [IC/group_size, OC]). */
int qimg_dequantize_awq_bf16(const int32_t* qweight_awq, const uint16_t* wscales, const uint16_t* wzeros,
                             uint16_t* out, int OC, int IC, int group_size, int num_components, void* stream);

/* linear_forward_awq (cuda_kernels.cu:3155-3179, awq_gemv_repacked_kernel
 * :3106-3153): M = 1, x fp32 [IC], qweight from qimg_awq_repack, group_size
 * 64; out fp32 [OC] in the de-interleaved order, + bias (bf16, de-interleaved
 * order) if given. Each output is the sum over ic in order. */
int qimg_linear_awq(const float* x, const int32_t* qweight_repacked, const uint16_t* wscales,
                    const uint16_t* wzeros, const uint16_t* bias_bf16, float* out, int OC, int IC, int group_size,
                    int num_components, void* stream);

/* unswizzle_nunchaku_weights (cuda_kernels.cu:3431-3499): nunchaku's
 * MMA-swizzled qweight [N, K/2] and bf16 wscales -> row-major nibbles
 * [N, K/2] and fp32 scales [num_groups, N]. N % 128 == 0, K % 64 == 0. */
int qimg_unswizzle_nunchaku_weights(const uint8_t* qweight_swizzled, const uint16_t* wscales_swizzled,
                                    uint8_t* qweight_rowmajor, float* wscales_rowmajor, int N, int K,
                                    int num_groups, void* stream);

/* dequantize_nunchaku_to_bf16 (cuda_kernels.cu:2932-2998). */
int qimg_dequantize_nunchaku_bf16(const uint8_t* qweight_swizzled, const uint16_t* wscales_swizzled,
                                  uint16_t* out, int N, int K, int num_groups, void* stream);

/* unswizzle_lora_weights (cuda_kernels.cu:3503-3572): nunchaku's packed
 * low-rank factor -> row-major bf16 [rows, cols] (is_down: the [K, rank]
 * down factor). rows % 16 == 0, cols % 16 == 0. */
int qimg_unswizzle_lora_weights(const uint16_t* packed, uint16_t* out, int rows, int cols, int is_down,
                                void* stream);

#ifdef __cplusplus
}
#endif
#endif /* QIMG_HOT_H */
