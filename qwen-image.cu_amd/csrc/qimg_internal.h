// qimg_internal.h — host-side launcher declarations shared between the
// kernel translation units and the C ABI layer (capi.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "qimg_hot.h"

namespace qimg {

// capi.hip: the C entry points' error reporting and the quantized linear's
// checks and launch sequence, for entry points defined in other files.
// api_fail sets the calling thread's qimg_last_error message and returns
// `status`; api_hip_status maps a HIP error to QIMG_ERR_HIP (or QIMG_OK).
int api_fail(int status, const char* fmt, ...);
int api_hip_status(hipError_t e, const char* where);
// Arguments of qimg_linear (without its scratch); on success *need holds the
// scratch bytes: align256(M*K) quantized activations, then align256(4*M)
// scales.
int check_linear(const char* fn, const void* x, int x_dtype, int M, int K, const void* w_q, const float* w_scales,
                 int N, int hbs, int mode, void* out, int out_dtype, int64_t* need);
// Activation FWHT + quantization into `scratch` (laid out as above), then
// the fused GEMM, on stream s.
int run_linear(const char* fn, const void* x, int x_dtype, int M, int K, const void* w_q, const float* w_scales,
               int N, int hbs, int mode, const uint16_t* bias_bf16, void* out, int out_dtype, int gelu, void* scratch,
               hipStream_t s);

// hadamard_quant.hip
size_t rows_lds_bytes(int K);
hipError_t launch_fwht_quant(const void* x, int x_dtype, int M, int K, int hbs, int mode,
                             void* q_out, float* scales, hipStream_t stream);
// launch_fwht_quant of gelu_tanh_fast(x) for fp32 rows of 2-4 Hadamard blocks
// of 4096 (the fc2 input, with fc1 run without its GELU: the same values as
// the GELU in fc1's epilogue); hipErrorNotSupported for other shapes.
bool fwht_quant_gelu_supported(int K, int hbs);
hipError_t launch_fwht_quant_gelu(const float* x, int M, int K, int hbs, int mode, void* q_out, float* scales,
                                  hipStream_t stream);
// LayerNorm + modulate of fp32 rows [M, K] (K <= 4096) straight into the
// FWHT + int8/e4m3 quantization of launch_fwht_quant (same values).
hipError_t launch_ln_fwht_quant(const float* x, const float* shift, const float* scale, int M, int K, int hbs,
                                int mode, float eps, void* q_out, float* scales, hipStream_t stream);
// launch_ln_fwht_quant on the rows of two matrices with the same K, hbs
// and mode (a joint block's image and text streams) in one launch where
// the wave-per-row kernel takes them; the same values as two calls.
hipError_t launch_ln_fwht_quant_pair(const float* xa, const float* shift_a, const float* scale_a, int Ma, void* qa,
                                     float* sa, const float* xb, const float* shift_b, const float* scale_b, int Mb,
                                     void* qb, float* sb, int K, int hbs, int mode, float eps, hipStream_t stream);
// launch_heads_fwht_quant of the image rows (s0 = n_txt) and the text rows
// (s0 = 0) of the joint sequences in one launch where the wave-per-row
// kernel takes them; the same values as the two calls.
hipError_t launch_heads_fwht_quant_pair(const uint16_t* attn, int batch, int H, int S, int n_txt, int n_img, int hbs,
                                        int mode, void* q_img, float* s_img, void* q_txt, float* s_txt,
                                        hipStream_t stream);
// Rows s0 .. s0+n of each of `batch` sequences of the fp16 attention
// output [batch][H][S][128] (K = H * 128, hbs >= 16) quantized as
// launch_fwht_quant quantizes their fp32 split copy.
hipError_t launch_heads_fwht_quant(const uint16_t* attn, int batch, int H, int S, int s0, int n, int hbs, int mode,
                                   void* q_out, float* scales, hipStream_t stream);
hipError_t launch_fwht_inplace(float* data, int M, int K, int hbs, hipStream_t stream);

// gemm_w8a8.hip
// One linear of launch_linear_pair.
// A linear whose output goes straight into the attention's operand layouts.
// Row r of its [M, N] product is token off + r % n of sequence b0 + r / n
// (S tokens per sequence), column c is dim c % 128 of head c / 128
// (N = 128 * heads):
//   HEADS_V: fp16 in the V^T tile layout [seq * heads + head][ceil(S/64)]
//     [128][64] (positions of keys past S are not written);
//   HEADS_K: RMSNorm with the bf16 [128] weight `norm` and eps, RoPE with
//     `pe` [S][64][4], fp16 [seq * heads + head][S][128], as
//     launch_joint_heads_f16 computes it;
//   HEADS_Q: the same, then the Sage int8 quantization of
//     launch_heads_quant_q: int8 [seq * heads + head][S][128] and `q_scale`
//     for the 32-token slices that hold tokens. Each slice must lie inside
//     the linear: off a multiple of 32, and n too unless M = n.
// fp32-out launch_linear_multi only, without GELU.
constexpr int HEADS_V = 1, HEADS_K = 2, HEADS_Q = 3;
struct HeadsOut {
    int kind, heads, S, off, n, b0;
    const uint16_t* norm;
    const float* pe;
    float* q_scale;
    float eps;
};

struct LinearArgs {
    const void* act_q;
    const float* act_scales;
    int M, K;
    const void* w_q;
    const float* w_scales;
    int N;
    const uint16_t* bias;
    void* out;
    // non-null: gated residual out = out + gate[n] * value (fp32 out), fused
    // into the large-tile epilogue; rows another kernel computes go through
    // tmp [M, N] and the gate-add kernel
    const float* gate;
    float* tmp;
    // non-null (launch_linear_multi): this linear's output goes to `out`
    // in an attention operand layout instead
    const HeadsOut* heads = nullptr;
};
hipError_t launch_linear_pair(const LinearArgs& a, const LinearArgs& b, int mode, int out_dtype, int gelu,
                              hipStream_t stream);
// Up to kMaxLinearMulti linears (same mode, output type and epilogue) in one
// launch of the large tiles; hipErrorNotSupported (nothing launched) when
// they do not all fit it, the launch is too small for the large tiles or the
// kernel choice is forced. check_linear_multi answers the same question
// without launching, so a caller can validate several launches before it
// starts the first.
constexpr int kMaxLinearMulti = 8;
hipError_t check_linear_multi(const LinearArgs* list, int n, int out_dtype, int gelu);
hipError_t launch_linear_multi(const LinearArgs* list, int n, int mode, int out_dtype, int gelu,
                               hipStream_t stream);
hipError_t launch_linear_prequantized(const void* act_q, const float* act_scales, int M, int K,
                                      const void* w_q, const float* w_scales, int N, int mode,
                                      const uint16_t* bias, void* out, int out_dtype, int gelu,
                                      hipStream_t stream,
                                      const float* gate = nullptr, float* tmp = nullptr);
hipError_t launch_dequant_bias(const int32_t* acc, const float* as, const float* ws, const uint16_t* bias,
                              float* out, int M, int N, int gelu, hipStream_t stream);

// gemm_bf16.hip: out fp32 [M, N] = bf16(x) . w^T + bias (GELU), x fp32
// (rounded to bf16) or bf16 [M, K], w bf16 [N, K].
// accumulate != 0: out = out + x . w^T, then the bias and GELU
hipError_t launch_linear_bf16(const void* x, int x_dtype, int M, int K, const uint16_t* w, int N,
                              const uint16_t* bias, float* out, int gelu, hipStream_t stream, int accumulate = 0);

// gemm_w8a8.hip: the same product for bf16 x with the 256x256 tiles of the
// quantized linear (K % 64 == 0); launch_linear_bf16 takes it when the
// problem has at least 128 such tiles.
hipError_t launch_gemm_bf16_large(const uint16_t* x, int M, int K, const uint16_t* w, int N, const uint16_t* bias,
                                  float* out, int gelu, int accumulate, hipStream_t stream);

// ---- INT4 paths (int4.hip, hadamard_quant.hip) ----
hipError_t launch_dequant_int4_bf16(const uint8_t* qw, const float* scales, uint16_t* out, int N, int K, int gs,
                                    int nf4, int scales_gn, int signed_int4, hipStream_t stream);
hipError_t launch_quant_int4_weight(const float* r, uint8_t* qw, float* scales, int N, int K, int gs, int nf4,
                                    hipStream_t stream);
hipError_t launch_quant_act_int4(const float* x, const float* smooth, uint16_t* bf16_out, uint8_t* packed,
                                 float* scales, int M, int K, int gs, hipStream_t stream);
hipError_t launch_w4a4_gemm(const uint8_t* act, const uint8_t* wgt, const float* as, const float* ws, float* out,
                            int M, int N, int K, int gs, int accumulate, const uint16_t* bias, int gelu,
                            hipStream_t stream);
hipError_t launch_awq_repack(const int32_t* qw, int32_t* out, int OC, int IC, hipStream_t stream);
hipError_t launch_awq_dequant(const int32_t* qw, const uint16_t* wscales, const uint16_t* wzeros, uint16_t* out,
                              int OC, int IC, int gs, int ncomp, hipStream_t stream);
hipError_t launch_awq_gemv(const float* x, const int32_t* qw_rep, const uint16_t* wscales, const uint16_t* wzeros,
                           const uint16_t* bias, float* out, int OC, int IC, int gs, int ncomp, hipStream_t stream);
hipError_t launch_nk_unswizzle(const uint8_t* q_sw, const uint16_t* s_sw, uint8_t* q_rm, float* s_rm, int N, int K,
                               int G, hipStream_t stream);
hipError_t launch_nk_dequant(const uint8_t* q_sw, const uint16_t* s_sw, uint16_t* out, int N, int K, int G,
                             hipStream_t stream);
hipError_t launch_lora_unswizzle(const uint16_t* packed, uint16_t* out, int rows, int cols, int is_down,
                                 hipStream_t stream);
hipError_t launch_transpose_u16(const uint16_t* in, uint16_t* out, int R, int C, hipStream_t stream);
hipError_t launch_f32_to_bf16(const float* in, uint16_t* out, int64_t n, hipStream_t stream);
hipError_t launch_bf16_to_f32(const uint16_t* in, float* out, int64_t n, hipStream_t stream);
// Rows of x fp32 [M, K]: v = x (/ smooth[k]); xs_bf16 = bf16(v) (if
// non-null); xr_bf16 = bf16(FWHT_hbs(v)) (hbs > 1; hbs <= 1: bf16(v)).
hipError_t launch_int4_prep(const float* x, const float* smooth, uint16_t* xs_bf16, uint16_t* xr_bf16, int M, int K,
                            int hbs, hipStream_t stream);
// out = FWHT_hbs(x / smooth[k]) fp32 (smooth may be null, hbs <= 1: no
// transform); out may be x.
hipError_t launch_smooth_fwht_f32(const float* x, const float* smooth, float* out, int M, int K, int hbs,
                                  hipStream_t stream);

// Kernel selection override for the quantized linear (QIMG_LINEAR_*);
// returns the previous setting.
int set_linear_kernel(int which);
int get_linear_kernel();

// gemm_small_m.hip: 0 = use the large-tile kernel, 1 = 32x32 tiles
// (M <= 32), 2 = 64x64 tiles (fewer than kSmallMTileLimit large tiles),
// 3 = vector-ALU GEMV (int8, M <= 4; e4m3 falls back to 1)
// (64: at 48 tiles of 256x256 or fewer the 64x64 tiles measured faster, at
// 72 or more the large tiles, for int8 and e4m3, K = 3072 and 12288)
constexpr int kSmallMTileLimit = 64;
// int8 linears of at least 128 rows and this many tiles of 256x256 leave
// the 64x64 tiles for the large-tile kernel's plan, whose 128x128 tiles
// serve them
// (1024 x 3072 x 3072: 19.2 against 23.4 us; 512 x 3072 x 3072, 24 tiles:
// 16.4 against 15.2 us, kept on 64x64)
constexpr int kMidTileMin = 32;
int small_m_variant(int M, int N, int K);
// Two int8 or two e4m3 (mode) linears of one M <= 4 activation (act_q,
// act_scales, K) as one GEMV launch into a.out and b.out (a.act_q / b.act_q
// are not read). Returns false, launching nothing, when the pair is not
// that case (or a kernel choice other than AUTO is set); otherwise true with
// the launch status in *err.
bool launch_gemv_pair(const void* act_q, const float* act_scales, int M, int K, const LinearArgs& a,
                      const LinearArgs& b, int mode, int out_dtype, hipStream_t stream, hipError_t* err);
bool small_m_fits(int M, int N, int K);  // sizes the small-tile kernels can address
hipError_t launch_linear_small_m(const void* act_q, const float* act_scales, int M, int K, const void* w_q,
                                 const float* w_scales, int N, int mode, const uint16_t* bias, void* out,
                                 int out_dtype, int gelu, int variant, hipStream_t stream);

// sage_attention.hip
struct SageScratch {
    int8_t* q_i8;
    int8_t* k_i8;
    uint16_t* v_t;  // V re-laid for the PV product
    float* q_scale;
    float* k_scale;
    float* k_mean;
};
int64_t sage_scratch_layout(int BH, int S, int D, void* base, SageScratch* out);
int64_t sage_vt_bytes(int BH, int S, int D);
hipError_t launch_sage_k_mean(const uint16_t* k, float* mean, int BH, int S, int D,
                              hipStream_t stream);
hipError_t launch_sage_quant_q(const uint16_t* q, int8_t* q_out, float* q_scale, int BH, int S,
                               int D, hipStream_t stream);
hipError_t launch_sage_quant_k(const uint16_t* k, const float* mean, int8_t* k_out,
                               float* k_scale, int BH, int S, int D, hipStream_t stream);
hipError_t launch_sage_attn(const int8_t* q, const int8_t* k, const uint16_t* v,
                            const float* q_scale, const float* k_scale, void* out, int out_dtype,
                            int BH, int S, int D, float sm_scale, int causal, uint16_t* v_t,
                            hipStream_t stream);
// Workgroups of one launch_sage_attn_vt call.
int64_t sage_attn_workgroups(int BH, int S);
// launch_sage_attn with V already in the Vt layout (no re-layout pass).
hipError_t launch_sage_attn_vt(const int8_t* q, const int8_t* k, const uint16_t* v_t, const float* q_scale,
                               const float* k_scale, void* out, int out_dtype, int BH, int S, int D, float sm_scale,
                               int causal, hipStream_t stream);
// The joint block's V (fp32 text and image linear outputs, H heads of 128)
// -> fp16 in the Vt layout of launch_sage_attn_vt.
// What the attention's operand passes write and linears writing those
// operands (HeadsOut) do not: zeros at the Vt positions of the keys past S
// in each last key tile, and (q_scale non-null) the Q scales of the 32-token
// slices without tokens in the last 128-token block.
hipError_t launch_sage_tail_fill(uint16_t* v_t, float* q_scale, int BH, int S, hipStream_t stream);
hipError_t launch_heads_v_relayout(const float* txt, const float* img, uint16_t* v_t, int n_txt, int n_img,
                                   int batch, int H, hipStream_t stream);
// The joint block's Q (fp32 text and image linear outputs) -> RMSNorm +
// RoPE + fp16 rounding -> the int8 Q and scales of launch_sage_quant_q.
hipError_t launch_heads_quant_q(const float* txt, const float* img, const uint16_t* w_txt, const uint16_t* w_img,
                                const float* pe, int8_t* q_out, float* q_scale, int n_txt, int n_img, int batch, int H,
                                float eps, hipStream_t stream);


// block_ops.hip
hipError_t launch_silu(const float* x, float* out, int64_t n, hipStream_t stream);
hipError_t launch_layernorm_modulate(const float* x, const float* shift, const float* scale, float* out, int rows,
                                     int dim, float eps, hipStream_t stream);
hipError_t launch_joint_heads_f16(const float* txt, const float* img, const uint16_t* w_txt, const uint16_t* w_img,
                                  const float* pe, uint16_t* out, int n_txt, int n_img, int batch, int H, float eps,
                                  hipStream_t stream);
hipError_t launch_split_heads(const uint16_t* in, float* txt, float* img, int n_txt, int n_img, int batch, int H,
                              hipStream_t stream);
hipError_t launch_gate_add(const float* x, const float* gate, const float* y, float* out, int rows, int dim,
                           hipStream_t stream);

// Compute units of the current device (0 if the query fails).
int device_cu_count();

// mmdit_block.hip
struct BlockScratch {
    float* t_silu;
    uint8_t* mod_q;    // quantized silu(t_emb), the modulation linears' input,
    float* mod_scale;  // kept across the blocks of one call
    // two sets of modulation chunks: a block reads its own set while the
    // next block's are computed into the other
    float* img_mods[2];
    float* txt_mods[2];
    float* img_norm;
    float* txt_norm;
    uint8_t* act_q;  // image stream (and the modulation input)
    float* act_scales;
    uint8_t* act_q_txt;  // text stream
    float* act_scales_txt;
    float* img_qkv[3];
    float* txt_qkv[3];
    uint16_t* k16;  // fp16 K
    uint16_t* attn16;
    float* img_mlp;
    float* txt_mlp;
    uint8_t* sage;
    int64_t sage_bytes;
};
// `batch` sequences of n_img + n_txt tokens (same lengths, shared t_emb
// and pe): img [batch, n_img, 3072], txt [batch, n_txt, 3072].
int64_t mmdit_block_scratch_layout(int n_img, int n_txt, int batch, void* base, BlockScratch* out);
// prof_ms != nullptr: the stream is synchronised at the end and each
// category's time is ADDED to prof_ms[c].
// t_ready: silu(t_emb) and its quantization for b.img_mod are already in
// w.t_silu / w.mod_q (left by the previous block of the same call, whose
// img_mod has the same K, Hadamard block and mode).
// mods_set: the modulation chunk set (w.img_mods / w.txt_mods index) the
// block reads; mods_ready: the previous block has already computed it.
// next != nullptr: the next block of the call, whose modulation chunks this
// block may compute into the other set (beside its attention); *next_ready
// says whether it did.
hipError_t run_mmdit_block(const qimg_mmdit_block& b, float* img, float* txt, const float* t_emb, const float* pe,
                           int n_img, int n_txt, int batch, const BlockScratch& w, float* prof_ms, hipStream_t s,
                           bool t_ready = false, int mods_set = 0, bool mods_ready = false,
                           const qimg_mmdit_block* next = nullptr, bool* next_ready = nullptr);

}  // namespace qimg
