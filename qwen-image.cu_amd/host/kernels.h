// kernels.h — the quantized-linear and SageAttention operators of the
// qwen-image MMDiT forward pass, with the reference's C++ call surface
// (qwen-image.cu cuda_kernels.cuh:177-320, 415-424, 555-562) on the HIP
// runtime. Every operator runs the gfx950 kernels of libqimg_hot.so through
// its C ABI (include/qimg_hot.h); there is no host fallback.
//
// Differences from the reference surface, all additive:
//   * QuantMode::FP8_HADAMARD: the same Hadamard front end with OCP e4m3
//     weights/activations (scale = amax/448); QuantizedWeight::data is then
//     DType::FP8_E4M3.
//   * `out` may be FP32 (the reference's type) or BF16.
//   * QuantMode::BF16 weights (layers kept unquantized) run the library's
//     BF16 kernel behind linear_forward_quantized[_bf16in], as the
//     reference's linear_forward_bf16[_bf16in].
//   * INT4_SVD and INT4_AWQ run the library's INT4 kernels. The W4A4
//     residual reads the row-major packing: swizzle_w4a4_weights_mma
//     copies the row-major nibbles into qweight_mma (the buffer the
//     reference's loader allocates has room for them), so
//     TransformerWeights::load runs unchanged and w4a4_gemm /
//     linear_forward_int4 read qweight_mma as [N, K/2] row-major.
//
// Error behaviour follows the reference (assert / CUDA_CHECK -> exit(1)): a
// rejected argument or failed HIP call prints "qimg: <function>: <reason>"
// to stderr and exits with status 1.
#pragma once

#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>

#include <algorithm>
#include <cstdint>
#include <vector>

#include "qimg_hot.h"
#include "tensor.h"

enum class QuantMode { INT8_HADAMARD, INT4_SVD, BF16, INT4_AWQ, FP8_HADAMARD };

// cuda_kernels.cuh:187-245 (plus the e4m3 mode). Unused fields stay null.
struct QuantizedWeight {
    QuantMode mode = QuantMode::INT8_HADAMARD;

    // INT8 / FP8 / BF16
    Tensor data;             // [N, K] INT8, FP8_E4M3 for FP8_HADAMARD, BF16 for BF16
    Tensor scales;           // [N] FP32
    int had_block_size = 0;  // Hadamard block size (power of 2)

    // INT4 + SVD
    Tensor qweight;          // [N, K/2] UINT8 packed INT4 (NF4 or offset-8 codes)
    Tensor scales4;          // [N, K/group_size] FP32
    Tensor svd_up;           // [N, r] BF16
    Tensor svd_down;         // [K, r] BF16
    Tensor smooth;           // [K] FP32, optional
    int group_size = 128;
    int svd_rank = 0;
    bool nf4_grid = true;

    // nunchaku INT4 (two's complement nibbles)
    bool nunchaku_swizzle = false;
    Tensor wscales_bf16;      // [num_groups, N] BF16, swizzled
    Tensor qweight_rowmajor;  // [N, K/2] UINT8
    Tensor wscales_rowmajor;  // [num_groups, N] FP32
    Tensor qweight_mma;       // row-major [N, K/2] nibbles here (see above)

    // AWQ INT4 (modulation layers)
    Tensor awq_qweight;   // [IC/8, OC] INT32 after repack_awq_to_transposed
    Tensor awq_wscales;   // [num_groups, OC] BF16
    Tensor awq_wzeros;    // [num_groups, OC] BF16
    int awq_OC = 0;
    int awq_IC = 0;
    int awq_group_size = 64;
    int awq_num_components = 6;

    QuantizedWeight() = default;
    QuantizedWeight(QuantizedWeight&&) = default;
    QuantizedWeight& operator=(QuantizedWeight&&) = default;

    void free_data() {
        for (Tensor* t : {&data, &scales, &qweight, &scales4, &svd_up, &svd_down, &smooth, &wscales_bf16,
                          &qweight_rowmajor, &wscales_rowmajor, &qweight_mma, &awq_qweight, &awq_wscales, &awq_wzeros})
            t->free_data();
    }
};

// ---- Hadamard + quantization (cuda_kernels.cuh:247-280) ----------------
void fwht_inplace(float* data, int M, int K, int had_block_size, hipStream_t stream = 0);
inline int hadamard_block_size(int K) { return K & (-K); }
void quantize_per_row_fp32(const float* x, int8_t* out, float* scales, int M, int K,
                           hipStream_t stream = 0);
void quantize_activation_per_token_fp32(const float* x, int8_t* out, float* scales, int M, int K,
                                        hipStream_t stream = 0);
void quantize_activation_per_token_bf16(const __hip_bfloat16* x, int8_t* out, float* scales, int M,
                                        int K, hipStream_t stream = 0);
void fwht_quantize_fp32(const float* input, int8_t* output, float* scales, int M, int K,
                        int had_block_size, hipStream_t stream = 0);
void fwht_quantize_bf16(const __hip_bfloat16* input, int8_t* output, float* scales, int M, int K,
                        int had_block_size, hipStream_t stream = 0);
void quantize_activation_int8_hadamard_fp32(const float* input, int8_t* output, float* scales, int M,
                                            int K, int had_block_size, hipStream_t stream = 0);
void quantize_activation_int8_hadamard_bf16(const __hip_bfloat16* input, int8_t* output,
                                            float* scales, int M, int K, int had_block_size,
                                            hipStream_t stream = 0);

// ---- dequant epilogue as a separate pass (cuda_kernels.cuh:282-291) ----
void dequantize_and_bias(const int32_t* gemm_out, const float* act_scales, const float* w_scales,
                         const __hip_bfloat16* bias, float* out, int M, int N, hipStream_t stream = 0);
void dequantize_bias_gelu(const int32_t* gemm_out, const float* act_scales, const float* w_scales,
                          const __hip_bfloat16* bias, float* out, int M, int N, hipStream_t stream = 0);

// ---- quantized linears (cuda_kernels.cuh:293-319, 420-424) -------------
// out[M,N] = dequant(quant(FWHT(x)) * W^T) + bias, optional GELU-tanh.
void linear_forward_int8(const Tensor& x, const QuantizedWeight& weight, const Tensor* bias, Tensor& out,
                         Tensor& scratch, bool apply_gelu = false);
void linear_forward_int8_prequantized(const int8_t* act_int8, const float* act_scales, int M, int K,
                                      const QuantizedWeight& weight, const Tensor* bias, Tensor& out,
                                      Tensor& scratch, bool apply_gelu = false);
void linear_forward_int8_bf16in(const Tensor& x, const QuantizedWeight& weight, const Tensor* bias,
                                Tensor& out, Tensor& scratch, bool apply_gelu = false);

// BF16 [N,K] -> FWHT(K & -K) -> per-row quantization; synchronous, as the
// reference (cuda_kernels.cu:2830-2862). quantize_weight_tensor_fp8 is the
// e4m3 twin (mode FP8_HADAMARD).
QuantizedWeight quantize_weight_tensor(const Tensor& bf16_weight);
QuantizedWeight quantize_weight_tensor_fp8(const Tensor& bf16_weight);

inline int64_t int8_scratch_bytes(int M, int K, int N) {
    const int64_t regionA = ((std::max(static_cast<int64_t>(M) * K, static_cast<int64_t>(M) * N) * 4 + 255) & ~255LL);
    const int64_t act = ((static_cast<int64_t>(M) * K + 255) & ~255LL);
    const int64_t scales = ((static_cast<int64_t>(M) * 4 + 255) & ~255LL);
    return regionA + act + scales;
}

// Dispatch on weight.mode (cuda_kernels.cu:4599-4635): x FP32 resp. BF16.
// QuantMode::BF16: weight.data BF16 [N, K], no scales, out FP32, scratch
// unused (the fp32 -> bf16 rounding of x happens inside the kernel).
// INT4_SVD: linear_forward_int4 (a BF16 x is widened to FP32 first, as the
// reference does); INT4_AWQ: linear_forward_awq (M = 1).
void linear_forward_quantized(const Tensor& x, const QuantizedWeight& weight, const Tensor* bias,
                              Tensor& out, Tensor& scratch, bool apply_gelu = false);
void linear_forward_quantized_bf16in(const Tensor& x, const QuantizedWeight& weight, const Tensor* bias,
                                     Tensor& out, Tensor& scratch);

// ---- INT4 paths (cuda_kernels.cuh:322-470) -----------------------------
void dequantize_int4_to_bf16(const uint8_t* qweight, const float* scales, __hip_bfloat16* out, int N, int K,
                             int group_size, hipStream_t stream = 0, bool nf4_grid = true, bool scales_gn = false,
                             bool signed_int4 = false);
void dequantize_nunchaku_to_bf16(const uint8_t* qweight, const __hip_bfloat16* wscales, __hip_bfloat16* out, int N,
                                 int K, int num_groups, hipStream_t stream = 0);
void quantize_int4_per_group(const float* residual, uint8_t* qweight, float* scales, int N, int K, int group_size,
                             hipStream_t stream = 0);
void linear_forward_awq(const Tensor& x, const QuantizedWeight& weight, const Tensor* bias, Tensor& out);
void repack_awq_to_transposed(const int32_t* qweight_awq, int32_t* qweight_out, int OC, int IC,
                              hipStream_t stream = 0);
void dequantize_awq_to_bf16(const int32_t* qweight, const __hip_bfloat16* wscales, const __hip_bfloat16* wzeros,
                            __hip_bfloat16* out, int OC, int IC, int group_size, int num_components,
                            hipStream_t stream = 0);
void unswizzle_nunchaku_weights(const uint8_t* qweight_swizzled, const __hip_bfloat16* wscales_swizzled,
                                uint8_t* qweight_rowmajor, float* wscales_rowmajor, int N, int K, int num_groups,
                                hipStream_t stream = 0);
void unswizzle_lora_weights(const __hip_bfloat16* packed, __hip_bfloat16* standard, int rows, int cols, bool is_down,
                            hipStream_t stream = 0);
void quantize_activation_int4(const float* x, uint8_t* act_packed, float* act_scales, int M, int K, int group_size,
                              hipStream_t stream = 0);
// Keeps the row-major packing (copied into wgt_mma), which this library's
// W4A4 GEMM reads.
void swizzle_w4a4_weights_mma(const uint8_t* wgt_rowmajor, uint32_t* wgt_mma, int N, int K, int group_size,
                              hipStream_t stream = 0);
// wgt_packed, or wgt_mma when wgt_packed is null, is [N, K/2] row-major.
void w4a4_gemm(const uint8_t* act_packed, const uint8_t* wgt_packed, const float* act_scales, const float* wgt_scales,
               float* output, int M, int N, int K, int group_size, const uint32_t* wgt_mma = nullptr,
               bool accumulate = false, const __hip_bfloat16* bias = nullptr, hipStream_t stream = 0);
void fused_smooth_bf16_quant(const float* x, const float* smooth, __hip_bfloat16* bf16_out, uint8_t* act_packed,
                             float* act_scales, int M, int K, int group_size, hipStream_t stream = 0);
void apply_smooth_div(const float* x, const float* smooth, float* out, int M, int K, hipStream_t stream = 0);
void smooth_hadamard_inplace(float* data, const float* smooth, int M, int K, int had_block_size,
                             hipStream_t stream = 0);
// x FP32 [M, K], out FP32 [M, N]; scratch >= int4_scratch_bytes(M, K, N, r).
void linear_forward_int4(const Tensor& x, const QuantizedWeight& weight, const Tensor* bias, Tensor& out,
                         Tensor& scratch, bool apply_gelu = false);
inline int64_t int4_scratch_bytes(int M, int K, int N, int svd_rank) {
    return qimg_int4_scratch_bytes(M, K, N, svd_rank);
}

// ---- SageAttention (cuda_kernels.cuh:558-562) --------------------------
// FP16 q, k, v [BH, S, D] -> FP32 out [BH, S, D] (values rounded through
// FP16, as the reference). D in {64, 128}. Uses a per-device workspace the
// library grows on demand (the reference's SageAttentionWorkspace). Like the
// reference's static workspace, one buffer serves every stream: calls whose
// kernels could overlap (different streams, no ordering between them) race.
// Growing synchronises the device, so a call that grows the workspace must
// not be captured into a graph (make the largest call once before capture).
void attention_forward_sage_sm80_fp16io(const __half* q, const __half* k, const __half* v, float* out,
                                        float scale, int BH, int S, int D, bool causal = false,
                                        hipStream_t stream = 0);

// ---- the joint-block loop (transformer.cu:497-836) ---------------------
// View of one quantized linear and its BF16 bias (or nullptr) for the
// library's block loop. The tensors must outlive the view.
qimg_qlinear qlinear_view(const QuantizedWeight& w, const Tensor* bias);

// View of one TransformerWeights::Block (transformer.h:94-140). `Block` is
// any struct with the reference's field names (img_mod_weight,
// img_mod_bias, ..., norm_added_k_weight), so the reference's own type can
// be passed as is.
template <class Block>
qimg_mmdit_block mmdit_block_view(const Block& b) {
    qimg_mmdit_block v{};
    v.img_mod = qlinear_view(b.img_mod_weight, &b.img_mod_bias);
    v.txt_mod = qlinear_view(b.txt_mod_weight, &b.txt_mod_bias);
    v.to_q = qlinear_view(b.to_q_weight, &b.to_q_bias);
    v.to_k = qlinear_view(b.to_k_weight, &b.to_k_bias);
    v.to_v = qlinear_view(b.to_v_weight, &b.to_v_bias);
    v.add_q_proj = qlinear_view(b.add_q_proj_weight, &b.add_q_proj_bias);
    v.add_k_proj = qlinear_view(b.add_k_proj_weight, &b.add_k_proj_bias);
    v.add_v_proj = qlinear_view(b.add_v_proj_weight, &b.add_v_proj_bias);
    v.to_out = qlinear_view(b.to_out_weight, &b.to_out_bias);
    v.to_add_out = qlinear_view(b.to_add_out_weight, &b.to_add_out_bias);
    v.img_mlp_fc1 = qlinear_view(b.img_mlp_fc1_weight, &b.img_mlp_fc1_bias);
    v.img_mlp_fc2 = qlinear_view(b.img_mlp_fc2_weight, &b.img_mlp_fc2_bias);
    v.txt_mlp_fc1 = qlinear_view(b.txt_mlp_fc1_weight, &b.txt_mlp_fc1_bias);
    v.txt_mlp_fc2 = qlinear_view(b.txt_mlp_fc2_weight, &b.txt_mlp_fc2_bias);
    v.norm_q = static_cast<const uint16_t*>(b.norm_q_weight.data);
    v.norm_k = static_cast<const uint16_t*>(b.norm_k_weight.data);
    v.norm_added_q = static_cast<const uint16_t*>(b.norm_added_q_weight.data);
    v.norm_added_k = static_cast<const uint16_t*>(b.norm_added_k_weight.data);
    return v;
}

// The blocks of `table` in order over `batch` sequences that share temb
// and pe (batch 2 runs the two CFG forwards of main.cu:761-773 as one):
// img FP32 [batch * n_img, 3072], txt FP32 [batch * n_txt, 3072], both
// updated in place; temb FP32 [3072]; pe FP32 [n_txt + n_img, 64, 4], text
// first (rope.h:154-160). The library grows a per-device workspace, with
// the same sharing and graph-capture rules as the SageAttention wrapper.
// prof_ms, if given, receives the QIMG_PROF_COUNT PROFILE_BLOCK categories
// (transformer.cu:486-495) summed over the blocks.
void mmdit_blocks_forward(const std::vector<qimg_mmdit_block>& table, Tensor& img, Tensor& txt, const Tensor& temb,
                          const Tensor& pe, int batch = 1, float* prof_ms = nullptr, hipStream_t stream = 0);
