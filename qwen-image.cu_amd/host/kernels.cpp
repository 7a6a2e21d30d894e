// kernels.cpp — the reference-signature C++ operators (kernels.h) on top of
// the C ABI of libqimg_hot.so. Shape/dtype checks mirror the reference's
// asserts (cuda_kernels.cu:2681-2686, 2744-2748, 2783-2785, 2831-2832); the
// C ABI repeats the numeric checks and its message is reported on failure.
#include "kernels.h"

#include <cstdarg>
#include <cstdlib>
#include <mutex>
#include <vector>

#include "qimg_hot.h"

namespace {

[[noreturn]] void die(const char* fn, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    fprintf(stderr, "qimg: %s: ", fn);
    vfprintf(stderr, fmt, ap);
    fprintf(stderr, "\n");
    va_end(ap);
    exit(1);
}

void check(int status, const char* fn) {
    if (status != QIMG_OK) die(fn, "%s (%s)", qimg_last_error(), qimg_status_string(status));
}

#define REQUIRE(cond, fn, ...) \
    do {                       \
        if (!(cond)) die(fn, __VA_ARGS__); \
    } while (0)

int qmode(QuantMode m, const char* fn) {
    switch (m) {
        case QuantMode::INT8_HADAMARD: return QIMG_QM_INT8_HADAMARD;
        case QuantMode::FP8_HADAMARD: return QIMG_QM_FP8_HADAMARD;
        case QuantMode::INT4_SVD: die(fn, "QuantMode::INT4_SVD weights take linear_forward_int4");
        case QuantMode::INT4_AWQ: die(fn, "QuantMode::INT4_AWQ weights take linear_forward_awq");
        case QuantMode::BF16:
            die(fn, "QuantMode::BF16 weights are not quantized (linear_forward_quantized[_bf16in] take them)");
    }
    die(fn, "unknown QuantMode");
}

DType qdtype(QuantMode m) { return m == QuantMode::FP8_HADAMARD ? DType::FP8_E4M3 : DType::INT8; }

int out_code(const Tensor& out, const char* fn) {
    if (out.dtype == DType::FP32) return QIMG_FP32;
    if (out.dtype == DType::BF16) return QIMG_BF16;
    die(fn, "out must be FP32 or BF16 (got %s)", dtype_name(out.dtype));
}

const uint16_t* bias_ptr(const Tensor* bias, int N, const char* fn) {
    if (!bias) return nullptr;
    REQUIRE(bias->dtype == DType::BF16, fn, "bias must be BF16 (got %s)", dtype_name(bias->dtype));
    REQUIRE(bias->numel() == N, fn, "bias has %lld elements, expected N=%d", (long long)bias->numel(), N);
    return static_cast<const uint16_t*>(bias->data);
}

void check_weight(const QuantizedWeight& w, int K, const char* fn) {
    REQUIRE(w.data.ndim == 2, fn, "weight.data must be 2-D [N, K]");
    REQUIRE(w.data.dtype == qdtype(w.mode), fn, "weight.data is %s, mode expects %s", dtype_name(w.data.dtype),
            dtype_name(qdtype(w.mode)));
    REQUIRE(w.scales.dtype == DType::FP32 && w.scales.numel() == w.data.shape[0], fn,
            "weight.scales must be FP32 [N]");
    REQUIRE(w.data.shape[1] == K, fn, "weight K=%lld != input K=%d", (long long)w.data.shape[1], K);
}

void check_out(const Tensor& out, int M, int N, const char* fn) {
    REQUIRE(out.ndim == 2 && out.shape[0] == M && out.shape[1] == N, fn, "out is %s, expected [%d, %d]",
            out.shape_str().c_str(), M, N);
}

// QuantMode::BF16 (linear_forward_bf16 / _bf16in, cuda_kernels.cu:4534-4596):
// x FP32 (rounded to BF16 by the kernel) or BF16, weight.data BF16 [N, K],
// out FP32 (asserted by the reference, :4539, :4581).
void linear_bf16(const Tensor& x, DType want, const QuantizedWeight& weight, const Tensor* bias, Tensor& out,
                 bool apply_gelu, const char* fn) {
    REQUIRE(x.ndim == 2, fn, "x must be 2-D [M, K] (got %s)", x.shape_str().c_str());
    REQUIRE(x.dtype == want, fn, "x must be %s (got %s)", dtype_name(want), dtype_name(x.dtype));
    REQUIRE(weight.data.ndim == 2 && weight.data.dtype == DType::BF16, fn,
            "a QuantMode::BF16 weight must be BF16 [N, K] (got %s %s)", dtype_name(weight.data.dtype),
            weight.data.shape_str().c_str());
    const int M = static_cast<int>(x.shape[0]);
    const int K = static_cast<int>(x.shape[1]);
    REQUIRE(weight.data.shape[1] == K, fn, "weight K=%lld != input K=%d", (long long)weight.data.shape[1], K);
    const int N = static_cast<int>(weight.data.shape[0]);
    REQUIRE(out.dtype == DType::FP32, fn, "out must be FP32 (got %s)", dtype_name(out.dtype));
    check_out(out, M, N, fn);
    check(qimg_linear_bf16(x.data, want == DType::BF16 ? QIMG_BF16 : QIMG_FP32, M, K,
                           static_cast<const uint16_t*>(weight.data.data), N, bias_ptr(bias, N, fn),
                           static_cast<float*>(out.data), apply_gelu ? 1 : 0, nullptr),
          fn);
}

void linear_common(const Tensor& x, DType want, const QuantizedWeight& weight, const Tensor* bias, Tensor& out,
                   Tensor& scratch, bool apply_gelu, const char* fn) {
    REQUIRE(x.ndim == 2, fn, "x must be 2-D [M, K] (got %s)", x.shape_str().c_str());
    REQUIRE(x.dtype == want, fn, "x must be %s (got %s)", dtype_name(want), dtype_name(x.dtype));
    const int M = static_cast<int>(x.shape[0]);
    const int K = static_cast<int>(x.shape[1]);
    const int mode = qmode(weight.mode, fn);
    check_weight(weight, K, fn);
    const int N = static_cast<int>(weight.data.shape[0]);
    check_out(out, M, N, fn);
    check(qimg_linear(x.data, want == DType::BF16 ? QIMG_BF16 : QIMG_FP32, M, K, weight.data.data,
                      static_cast<const float*>(weight.scales.data), N, weight.had_block_size, mode,
                      bias_ptr(bias, N, fn), out.data, out_code(out, fn), apply_gelu ? 1 : 0, scratch.data,
                      static_cast<int64_t>(scratch.nbytes()), nullptr),
          fn);
}

QuantizedWeight quantize_weight_common(const Tensor& w, QuantMode mode, const char* fn) {
    REQUIRE(w.dtype == DType::BF16, fn, "weight must be BF16 (got %s)", dtype_name(w.dtype));
    REQUIRE(w.ndim == 2, fn, "weight must be 2-D [N, K]");
    const int N = static_cast<int>(w.shape[0]);
    const int K = static_cast<int>(w.shape[1]);
    QuantizedWeight qw;
    qw.mode = mode;
    qw.data = Tensor::alloc({static_cast<int64_t>(N), static_cast<int64_t>(K)}, qdtype(mode));
    qw.scales = Tensor::alloc({static_cast<int64_t>(N)}, DType::FP32);
    int hbs = 0;
    check(qimg_quantize_weight(w.data, QIMG_BF16, N, K, qmode(mode, fn), qw.data.data,
                               static_cast<float*>(qw.scales.data), &hbs, nullptr),
          fn);
    qw.had_block_size = hbs;
    return qw;
}

// Per-device SageAttention workspace, grown on demand (the reference keeps
// a static SageAttentionWorkspace, sageattention_sm80.cu:679-757).
//
// A caller holds the workspace's lock from the size check until its kernels
// are queued, so a second thread cannot free the buffer in between. Growing
// synchronises the device before the old buffer is freed (work queued
// earlier may still read it), so a call that grows the workspace must not be
// made while a stream is being captured into a graph: make the first call at
// the largest size before capturing. As with the reference's static
// workspace, calls queued on different streams share one buffer, so their
// kernels must not overlap in time.
struct SageWorkspace {
    std::mutex mu;
    std::vector<void*> buf;
    std::vector<int64_t> bytes;
};

SageWorkspace& sage_ws() {
    static SageWorkspace ws;
    return ws;
}

// The same for the block loop's workspace.
SageWorkspace& block_ws() {
    static SageWorkspace ws;
    return ws;
}

// The workspace buffer of the current device, at least `need` bytes, with
// its lock held for as long as the lease lives.
struct WorkspaceLease {
    std::unique_lock<std::mutex> lock;
    void* ptr = nullptr;
};

WorkspaceLease grown(SageWorkspace& w, int64_t need) {
    int dev = 0;
    HIP_CHECK(hipGetDevice(&dev));
    WorkspaceLease lease{std::unique_lock<std::mutex>(w.mu), nullptr};
    if (static_cast<int>(w.buf.size()) <= dev) {
        w.buf.resize(dev + 1, nullptr);
        w.bytes.resize(dev + 1, 0);
    }
    if (w.bytes[dev] < need) {
        // the previous buffer may still be read by work queued earlier
        HIP_CHECK(hipDeviceSynchronize());
        if (w.buf[dev]) HIP_CHECK(hipFree(w.buf[dev]));
        w.buf[dev] = nullptr;
        w.bytes[dev] = 0;
        HIP_CHECK(hipMalloc(&w.buf[dev], need));
        w.bytes[dev] = need;
    }
    lease.ptr = w.buf[dev];
    return lease;
}

}  // namespace

void fwht_inplace(float* data, int M, int K, int had_block_size, hipStream_t stream) {
    check(qimg_fwht_inplace(data, M, K, had_block_size, stream), "fwht_inplace");
}

void quantize_per_row_fp32(const float* x, int8_t* out, float* scales, int M, int K, hipStream_t stream) {
    check(qimg_quantize_per_row_fp32(x, out, scales, M, K, stream), "quantize_per_row_fp32");
}

void quantize_activation_per_token_fp32(const float* x, int8_t* out, float* scales, int M, int K,
                                        hipStream_t stream) {
    check(qimg_quantize_activation(x, QIMG_FP32, M, K, 1, QIMG_QM_INT8_HADAMARD, out, scales, stream),
          "quantize_activation_per_token_fp32");
}

void quantize_activation_per_token_bf16(const __hip_bfloat16* x, int8_t* out, float* scales, int M, int K,
                                        hipStream_t stream) {
    check(qimg_quantize_activation(x, QIMG_BF16, M, K, 1, QIMG_QM_INT8_HADAMARD, out, scales, stream),
          "quantize_activation_per_token_bf16");
}

void fwht_quantize_fp32(const float* input, int8_t* output, float* scales, int M, int K, int had_block_size,
                        hipStream_t stream) {
    check(qimg_quantize_activation(input, QIMG_FP32, M, K, had_block_size, QIMG_QM_INT8_HADAMARD, output,
                                   scales, stream),
          "fwht_quantize_fp32");
}

void fwht_quantize_bf16(const __hip_bfloat16* input, int8_t* output, float* scales, int M, int K,
                        int had_block_size, hipStream_t stream) {
    check(qimg_quantize_activation(input, QIMG_BF16, M, K, had_block_size, QIMG_QM_INT8_HADAMARD, output,
                                   scales, stream),
          "fwht_quantize_bf16");
}

void quantize_activation_int8_hadamard_fp32(const float* input, int8_t* output, float* scales, int M, int K,
                                            int had_block_size, hipStream_t stream) {
    check(qimg_quantize_activation(input, QIMG_FP32, M, K, had_block_size, QIMG_QM_INT8_HADAMARD, output,
                                   scales, stream),
          "quantize_activation_int8_hadamard_fp32");
}

void quantize_activation_int8_hadamard_bf16(const __hip_bfloat16* input, int8_t* output, float* scales, int M,
                                            int K, int had_block_size, hipStream_t stream) {
    check(qimg_quantize_activation(input, QIMG_BF16, M, K, had_block_size, QIMG_QM_INT8_HADAMARD, output,
                                   scales, stream),
          "quantize_activation_int8_hadamard_bf16");
}

void dequantize_and_bias(const int32_t* gemm_out, const float* act_scales, const float* w_scales,
                         const __hip_bfloat16* bias, float* out, int M, int N, hipStream_t stream) {
    check(qimg_dequantize_bias(gemm_out, act_scales, w_scales, reinterpret_cast<const uint16_t*>(bias), out, M, N,
                               0, stream),
          "dequantize_and_bias");
}

void dequantize_bias_gelu(const int32_t* gemm_out, const float* act_scales, const float* w_scales,
                          const __hip_bfloat16* bias, float* out, int M, int N, hipStream_t stream) {
    check(qimg_dequantize_bias(gemm_out, act_scales, w_scales, reinterpret_cast<const uint16_t*>(bias), out, M, N,
                               1, stream),
          "dequantize_bias_gelu");
}

void linear_forward_int8(const Tensor& x, const QuantizedWeight& weight, const Tensor* bias, Tensor& out,
                         Tensor& scratch, bool apply_gelu) {
    REQUIRE(weight.mode == QuantMode::INT8_HADAMARD, "linear_forward_int8", "weight.mode must be INT8_HADAMARD");
    linear_common(x, DType::FP32, weight, bias, out, scratch, apply_gelu, "linear_forward_int8");
}

void linear_forward_int8_bf16in(const Tensor& x, const QuantizedWeight& weight, const Tensor* bias, Tensor& out,
                                Tensor& scratch, bool apply_gelu) {
    REQUIRE(weight.mode == QuantMode::INT8_HADAMARD, "linear_forward_int8_bf16in",
            "weight.mode must be INT8_HADAMARD");
    linear_common(x, DType::BF16, weight, bias, out, scratch, apply_gelu, "linear_forward_int8_bf16in");
}

void linear_forward_int8_prequantized(const int8_t* act_int8, const float* act_scales, int M, int K,
                                      const QuantizedWeight& weight, const Tensor* bias, Tensor& out,
                                      Tensor& /*scratch: the fused kernel needs none*/, bool apply_gelu) {
    const char* fn = "linear_forward_int8_prequantized";
    const int mode = qmode(weight.mode, fn);
    check_weight(weight, K, fn);
    const int N = static_cast<int>(weight.data.shape[0]);
    check_out(out, M, N, fn);
    check(qimg_linear_prequantized(act_int8, act_scales, M, K, weight.data.data,
                                   static_cast<const float*>(weight.scales.data), N, mode, bias_ptr(bias, N, fn),
                                   out.data, out_code(out, fn), apply_gelu ? 1 : 0, nullptr),
          fn);
}

QuantizedWeight quantize_weight_tensor(const Tensor& bf16_weight) {
    return quantize_weight_common(bf16_weight, QuantMode::INT8_HADAMARD, "quantize_weight_tensor");
}

QuantizedWeight quantize_weight_tensor_fp8(const Tensor& bf16_weight) {
    return quantize_weight_common(bf16_weight, QuantMode::FP8_HADAMARD, "quantize_weight_tensor_fp8");
}

// ---- INT4 paths ---------------------------------------------------------
void dequantize_int4_to_bf16(const uint8_t* qweight, const float* scales, __hip_bfloat16* out, int N, int K,
                             int group_size, hipStream_t stream, bool nf4_grid, bool scales_gn, bool signed_int4) {
    check(qimg_dequantize_int4_bf16(qweight, scales, reinterpret_cast<uint16_t*>(out), N, K, group_size, nf4_grid,
                                    scales_gn, signed_int4, stream),
          "dequantize_int4_to_bf16");
}

void dequantize_nunchaku_to_bf16(const uint8_t* qweight, const __hip_bfloat16* wscales, __hip_bfloat16* out, int N,
                                 int K, int num_groups, hipStream_t stream) {
    check(qimg_dequantize_nunchaku_bf16(qweight, reinterpret_cast<const uint16_t*>(wscales),
                                        reinterpret_cast<uint16_t*>(out), N, K, num_groups, stream),
          "dequantize_nunchaku_to_bf16");
}

void quantize_int4_per_group(const float* residual, uint8_t* qweight, float* scales, int N, int K, int group_size,
                             hipStream_t stream) {
    check(qimg_quantize_int4_per_group(residual, qweight, scales, N, K, group_size, 1, stream),
          "quantize_int4_per_group");
}

void repack_awq_to_transposed(const int32_t* qweight_awq, int32_t* qweight_out, int OC, int IC, hipStream_t stream) {
    check(qimg_awq_repack(qweight_awq, qweight_out, OC, IC, stream), "repack_awq_to_transposed");
}

void dequantize_awq_to_bf16(const int32_t* qweight, const __hip_bfloat16* wscales, const __hip_bfloat16* wzeros,
                            __hip_bfloat16* out, int OC, int IC, int group_size, int num_components,
                            hipStream_t stream) {
    check(qimg_dequantize_awq_bf16(qweight, reinterpret_cast<const uint16_t*>(wscales),
                                   reinterpret_cast<const uint16_t*>(wzeros), reinterpret_cast<uint16_t*>(out), OC, IC,
                                   group_size, num_components, stream),
          "dequantize_awq_to_bf16");
}

void unswizzle_nunchaku_weights(const uint8_t* qweight_swizzled, const __hip_bfloat16* wscales_swizzled,
                                uint8_t* qweight_rowmajor, float* wscales_rowmajor, int N, int K, int num_groups,
                                hipStream_t stream) {
    check(qimg_unswizzle_nunchaku_weights(qweight_swizzled, reinterpret_cast<const uint16_t*>(wscales_swizzled),
                                          qweight_rowmajor, wscales_rowmajor, N, K, num_groups, stream),
          "unswizzle_nunchaku_weights");
}

void unswizzle_lora_weights(const __hip_bfloat16* packed, __hip_bfloat16* standard, int rows, int cols, bool is_down,
                            hipStream_t stream) {
    check(qimg_unswizzle_lora_weights(reinterpret_cast<const uint16_t*>(packed), reinterpret_cast<uint16_t*>(standard),
                                      rows, cols, is_down, stream),
          "unswizzle_lora_weights");
}

void quantize_activation_int4(const float* x, uint8_t* act_packed, float* act_scales, int M, int K, int group_size,
                              hipStream_t stream) {
    check(qimg_quantize_activation_int4(x, act_packed, act_scales, M, K, group_size, stream),
          "quantize_activation_int4");
}

void swizzle_w4a4_weights_mma(const uint8_t* wgt_rowmajor, uint32_t* wgt_mma, int N, int K, int group_size,
                              hipStream_t stream) {
    const char* fn = "swizzle_w4a4_weights_mma";
    REQUIRE(N > 0 && K > 0 && group_size > 0 && K % group_size == 0, fn, "bad sizes N=%d K=%d group_size=%d", N, K,
            group_size);
    // [num_groups, ceil(N/8), 256 B] holds the N * K/2 row-major bytes
    const size_t bytes = static_cast<size_t>(N) * (K / 2);
    const hipError_t e = hipMemcpyAsync(wgt_mma, wgt_rowmajor, bytes, hipMemcpyDeviceToDevice, stream);
    REQUIRE(e == hipSuccess, fn, "%s", hipGetErrorString(e));
}

void w4a4_gemm(const uint8_t* act_packed, const uint8_t* wgt_packed, const float* act_scales, const float* wgt_scales,
               float* output, int M, int N, int K, int group_size, const uint32_t* wgt_mma, bool accumulate,
               const __hip_bfloat16* bias, hipStream_t stream) {
    const uint8_t* w = wgt_packed ? wgt_packed : reinterpret_cast<const uint8_t*>(wgt_mma);
    check(qimg_w4a4_gemm(act_packed, w, act_scales, wgt_scales, output, M, N, K, group_size, accumulate,
                         reinterpret_cast<const uint16_t*>(bias), stream),
          "w4a4_gemm");
}

void fused_smooth_bf16_quant(const float* x, const float* smooth, __hip_bfloat16* bf16_out, uint8_t* act_packed,
                             float* act_scales, int M, int K, int group_size, hipStream_t stream) {
    check(qimg_fused_smooth_bf16_quant(x, smooth, reinterpret_cast<uint16_t*>(bf16_out), act_packed, act_scales, M, K,
                                       group_size, stream),
          "fused_smooth_bf16_quant");
}

void apply_smooth_div(const float* x, const float* smooth, float* out, int M, int K, hipStream_t stream) {
    check(qimg_smooth_hadamard(x, smooth, out, M, K, 1, stream), "apply_smooth_div");
}

void smooth_hadamard_inplace(float* data, const float* smooth, int M, int K, int had_block_size, hipStream_t stream) {
    check(qimg_smooth_hadamard(data, smooth, data, M, K, had_block_size, stream), "smooth_hadamard_inplace");
}

void linear_forward_int4(const Tensor& x, const QuantizedWeight& weight, const Tensor* bias, Tensor& out,
                         Tensor& scratch, bool apply_gelu) {
    const char* fn = "linear_forward_int4";
    REQUIRE(x.dtype == DType::FP32 && x.ndim == 2, fn, "x must be FP32 [M, K] (got %s %s)", dtype_name(x.dtype),
            x.shape_str().c_str());
    REQUIRE(out.dtype == DType::FP32, fn, "out must be FP32 (got %s)", dtype_name(out.dtype));
    REQUIRE(weight.mode == QuantMode::INT4_SVD, fn, "weight.mode must be INT4_SVD");
    REQUIRE(weight.svd_up.ndim == 2 && weight.svd_down.ndim == 2 && weight.svd_up.dtype == DType::BF16 &&
                weight.svd_down.dtype == DType::BF16,
            fn, "svd_up [N, r] and svd_down [K, r] must be BF16");
    // N and K from the low-rank factors (cuda_kernels.cu:4340-4342)
    const int M = static_cast<int>(x.shape[0]);
    const int N = static_cast<int>(weight.svd_up.shape[0]);
    const int K = static_cast<int>(weight.svd_down.shape[0]);
    const int r = static_cast<int>(weight.svd_up.shape[1]);
    REQUIRE(x.shape[1] == K, fn, "x K=%lld != weight K=%d", (long long)x.shape[1], K);
    REQUIRE(weight.svd_down.shape[1] == r, fn, "svd_down rank %lld != svd_up rank %d",
            (long long)weight.svd_down.shape[1], r);
    check_out(out, M, N, fn);
    qimg_int4_weight w{};
    w.N = N;
    w.K = K;
    w.rank = r;
    w.group_size = weight.group_size;
    w.nf4_grid = weight.nf4_grid ? 1 : 0;
    w.had_block_size = weight.had_block_size;
    w.svd_up = static_cast<const uint16_t*>(weight.svd_up.data);
    w.svd_down = static_cast<const uint16_t*>(weight.svd_down.data);
    w.smooth = static_cast<const float*>(weight.smooth.data);
    // The reference takes W4A4 only for nunchaku weights with the MMA copy
    // and without FORCE_W4A16 (cuda_kernels.cu:4362); other nunchaku weights
    // go through its W4A16 fallback on the row-major nibbles (:4443-4470).
    const bool use_w4a4 = weight.nunchaku_swizzle && weight.qweight_mma.data && !getenv("FORCE_W4A16");
    if (use_w4a4) {
        REQUIRE(weight.wscales_rowmajor.dtype == DType::FP32 && weight.wscales_rowmajor.data, fn,
                "W4A4 needs wscales_rowmajor FP32 [num_groups, N]");
        w.w4a4_qweight = static_cast<const uint8_t*>(weight.qweight_mma.data);
        w.w4a4_wscales = static_cast<const float*>(weight.wscales_rowmajor.data);
    } else if (weight.nunchaku_swizzle && weight.qweight_rowmajor.data) {
        REQUIRE(weight.wscales_rowmajor.dtype == DType::FP32 && weight.wscales_rowmajor.data, fn,
                "W4A16 (nunchaku) needs wscales_rowmajor FP32 [num_groups, N]");
        w.qweight = static_cast<const uint8_t*>(weight.qweight_rowmajor.data);
        w.scales4 = static_cast<const float*>(weight.wscales_rowmajor.data);
        w.w4a16_nunchaku = 1;
    } else {
        REQUIRE(weight.qweight.data && weight.scales4.dtype == DType::FP32, fn,
                "W4A16 needs qweight [N, K/2] and scales4 FP32 [N, K/group_size]");
        w.qweight = static_cast<const uint8_t*>(weight.qweight.data);
        w.scales4 = static_cast<const float*>(weight.scales4.data);
    }
    check(qimg_linear_int4(static_cast<const float*>(x.data), M, &w, bias_ptr(bias, N, fn),
                           static_cast<float*>(out.data), apply_gelu ? 1 : 0, scratch.data,
                           static_cast<int64_t>(scratch.nbytes()), nullptr),
          fn);
}

void linear_forward_awq(const Tensor& x, const QuantizedWeight& weight, const Tensor* bias, Tensor& out) {
    const char* fn = "linear_forward_awq";
    REQUIRE(x.dtype == DType::FP32 && out.dtype == DType::FP32, fn, "x and out must be FP32");
    REQUIRE(weight.mode == QuantMode::INT4_AWQ, fn, "weight.mode must be INT4_AWQ");
    REQUIRE(x.shape[0] == 1, fn, "AWQ GEMV only supports M=1 (got %lld)", (long long)x.shape[0]);
    const int OC = weight.awq_OC, IC = weight.awq_IC;
    REQUIRE(x.numel() == IC && out.numel() == OC, fn, "x must hold IC=%d values and out OC=%d", IC, OC);
    check(qimg_linear_awq(static_cast<const float*>(x.data), static_cast<const int32_t*>(weight.awq_qweight.data),
                          static_cast<const uint16_t*>(weight.awq_wscales.data),
                          static_cast<const uint16_t*>(weight.awq_wzeros.data), bias_ptr(bias, OC, fn),
                          static_cast<float*>(out.data), OC, IC, weight.awq_group_size, weight.awq_num_components,
                          nullptr),
          fn);
}

namespace {

// A BF16 input widened to FP32 in a temporary (the reference's bf16in
// dispatch, cuda_kernels.cu:4616-4631).
Tensor widen_bf16(const Tensor& x, const char* fn) {
    REQUIRE(x.dtype == DType::BF16, fn, "x must be BF16 (got %s)", dtype_name(x.dtype));
    Tensor f = Tensor::alloc(std::vector<int64_t>(x.shape, x.shape + x.ndim), DType::FP32);
    check(qimg_bf16_to_fp32(static_cast<const uint16_t*>(x.data), static_cast<float*>(f.data), x.numel(), nullptr),
          fn);
    return f;
}

}  // namespace

void linear_forward_quantized(const Tensor& x, const QuantizedWeight& weight, const Tensor* bias, Tensor& out,
                              Tensor& scratch, bool apply_gelu) {
    const char* fn = "linear_forward_quantized";
    if (weight.mode == QuantMode::BF16) return linear_bf16(x, DType::FP32, weight, bias, out, apply_gelu, fn);
    if (weight.mode == QuantMode::INT4_AWQ) return linear_forward_awq(x, weight, bias, out);
    if (weight.mode == QuantMode::INT4_SVD) return linear_forward_int4(x, weight, bias, out, scratch, apply_gelu);
    linear_common(x, DType::FP32, weight, bias, out, scratch, apply_gelu, fn);
}

void linear_forward_quantized_bf16in(const Tensor& x, const QuantizedWeight& weight, const Tensor* bias,
                                     Tensor& out, Tensor& scratch) {
    const char* fn = "linear_forward_quantized_bf16in";
    if (weight.mode == QuantMode::BF16) return linear_bf16(x, DType::BF16, weight, bias, out, false, fn);
    if (weight.mode == QuantMode::INT4_AWQ || weight.mode == QuantMode::INT4_SVD) {
        Tensor xf = widen_bf16(x, fn);
        if (weight.mode == QuantMode::INT4_AWQ)
            linear_forward_awq(xf, weight, bias, out);
        else
            linear_forward_int4(xf, weight, bias, out, scratch);
        REQUIRE(hipDeviceSynchronize() == hipSuccess, fn, "device synchronisation failed");
        return;
    }
    linear_common(x, DType::BF16, weight, bias, out, scratch, false, fn);
}

void attention_forward_sage_sm80_fp16io(const __half* q, const __half* k, const __half* v, float* out,
                                        float scale, int BH, int S, int D, bool causal, hipStream_t stream) {
    const char* fn = "attention_forward_sage_sm80_fp16io";
    // sageattention_sm80.cu:975-978 rejects other head dims; checked here
    // before the workspace is touched
    REQUIRE(D == 64 || D == 128, fn, "head_dim %d not supported (64 or 128)", D);
    REQUIRE(BH > 0 && S > 0, fn, "need BH > 0 and S > 0 (BH=%d S=%d)", BH, S);
    const int64_t need = qimg_sage_scratch_bytes(BH, S, D);
    const WorkspaceLease ws = grown(sage_ws(), need);  // held until the kernels are queued
    check(qimg_sage_attention(reinterpret_cast<const uint16_t*>(q), reinterpret_cast<const uint16_t*>(k),
                              reinterpret_cast<const uint16_t*>(v), out, QIMG_FP32, scale, BH, S, D, causal ? 1 : 0,
                              ws.ptr, need, stream),
          fn);
}

qimg_qlinear qlinear_view(const QuantizedWeight& w, const Tensor* bias) {
    const char* fn = "qlinear_view";
    REQUIRE(w.data.ndim == 2 && w.scales.data, fn, "weight must be a quantized [N, K] tensor");
    REQUIRE(!bias || !bias->data || bias->dtype == DType::BF16, fn, "bias must be BF16");
    return {w.data.data, static_cast<const float*>(w.scales.data), static_cast<int>(w.data.shape[0]),
            static_cast<int>(w.data.shape[1]), w.had_block_size, qmode(w.mode, fn),
            bias && bias->data ? static_cast<const uint16_t*>(bias->data) : nullptr};
}

void mmdit_blocks_forward(const std::vector<qimg_mmdit_block>& table, Tensor& img, Tensor& txt, const Tensor& temb,
                          const Tensor& pe, int batch, float* prof_ms, hipStream_t stream) {
    const char* fn = "mmdit_blocks_forward";
    REQUIRE(!table.empty(), fn, "no blocks");
    REQUIRE(batch >= 1, fn, "batch must be >= 1 (got %d)", batch);
    REQUIRE(img.dtype == DType::FP32 && txt.dtype == DType::FP32 && temb.dtype == DType::FP32 &&
                pe.dtype == DType::FP32,
            fn, "img, txt, temb and pe must be FP32");
    REQUIRE(img.numel() % (int64_t{batch} * 3072) == 0 && txt.numel() % (int64_t{batch} * 3072) == 0, fn,
            "img/txt must hold batch x n x 3072 values");
    const int n_img = static_cast<int>(img.numel() / (int64_t{batch} * 3072));
    const int n_txt = static_cast<int>(txt.numel() / (int64_t{batch} * 3072));
    REQUIRE(temb.numel() == 3072, fn, "temb must be [3072]");
    REQUIRE(pe.numel() == static_cast<int64_t>(n_img + n_txt) * 256, fn, "pe must be [%d, 64, 4]", n_img + n_txt);
    const int64_t need = qimg_mmdit_blocks_scratch_bytes(n_img, n_txt, batch);
    REQUIRE(need > 0, fn, "bad token counts n_img=%d n_txt=%d", n_img, n_txt);
    const WorkspaceLease ws = grown(block_ws(), need);  // held until the kernels are queued
    check(qimg_mmdit_blocks_forward(table.data(), static_cast<int>(table.size()), static_cast<float*>(img.data),
                                    static_cast<float*>(txt.data), static_cast<const float*>(temb.data),
                                    static_cast<const float*>(pe.data), n_img, n_txt, batch, ws.ptr, need, prof_ms,
                                    stream),
          fn);
}
