// kernels.cpp — the reference-signature C++ operators (kernels.h) on top of
// the C ABI of libqimg_hot.so. Shape/dtype checks mirror the reference's
// asserts (cuda_kernels.cu:2681-2686, 2744-2748, 2783-2785, 2831-2832); the
// C ABI repeats the numeric checks and its message is reported on failure.
#include "kernels.h"

#include <cstdarg>
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
        case QuantMode::INT4_SVD: die(fn, "QuantMode::INT4_SVD is not part of this library");
        case QuantMode::INT4_AWQ: die(fn, "QuantMode::INT4_AWQ is not part of this library");
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

void linear_forward_quantized(const Tensor& x, const QuantizedWeight& weight, const Tensor* bias, Tensor& out,
                              Tensor& scratch, bool apply_gelu) {
    const char* fn = "linear_forward_quantized";
    if (weight.mode == QuantMode::BF16) return linear_bf16(x, DType::FP32, weight, bias, out, apply_gelu, fn);
    qmode(weight.mode, fn);  // INT4 modes are reported here
    linear_common(x, DType::FP32, weight, bias, out, scratch, apply_gelu, fn);
}

void linear_forward_quantized_bf16in(const Tensor& x, const QuantizedWeight& weight, const Tensor* bias,
                                     Tensor& out, Tensor& scratch) {
    const char* fn = "linear_forward_quantized_bf16in";
    if (weight.mode == QuantMode::BF16) return linear_bf16(x, DType::BF16, weight, bias, out, false, fn);
    qmode(weight.mode, fn);
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
