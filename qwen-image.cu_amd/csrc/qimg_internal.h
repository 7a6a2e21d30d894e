// qimg_internal.h — host-side launcher declarations shared between the
// kernel translation units and the C ABI layer (capi.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "qimg_hot.h"

namespace qimg {

// hadamard_quant.hip
size_t rows_lds_bytes(int K);
hipError_t launch_fwht_quant(const void* x, int x_dtype, int M, int K, int hbs, int mode,
                             void* q_out, float* scales, hipStream_t stream);
hipError_t launch_fwht_inplace(float* data, int M, int K, int hbs, hipStream_t stream);

// gemm_w8a8.hip
hipError_t launch_linear_prequantized(const void* act_q, const float* act_scales, int M, int K,
                                      const void* w_q, const float* w_scales, int N, int mode,
                                      const uint16_t* bias, void* out, int out_dtype, int gelu,
                                      hipStream_t stream);
hipError_t launch_dequant_bias(const int32_t* acc, const float* as, const float* ws, const uint16_t* bias,
                              float* out, int M, int N, int gelu, hipStream_t stream);

// Kernel selection override for the quantized linear (QIMG_LINEAR_*);
// returns the previous setting.
int set_linear_kernel(int which);
int get_linear_kernel();

// gemm_small_m.hip: 0 = use the large-tile kernel, 1 = 32x32 tiles
// (M <= 32), 2 = 64x64 tiles (few large tiles), 3 = vector-ALU GEMV (int8,
// M <= 4; e4m3 falls back to 1)
int small_m_variant(int M, int N, int K);
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

}  // namespace qimg
