// capi.hip — the extern "C" boundary (include/qimg_hot.h).
//
// Every entry point validates its arguments on the host before any HIP call
// (the reference aborts via assert/exit instead, cuda_kernels.cu:2681-2686,
// sageattention_sm80.cu:975-978) and returns a qimg_status. The message of the
// last failure is kept per thread for qimg_last_error().
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "qimg_internal.h"

namespace {

thread_local char g_err[512] = "";

int vfail(int status, const char* fmt, va_list ap) {
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    return status;
}

int fail(int status, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vfail(status, fmt, ap);
    va_end(ap);
    return status;
}

int hip_status(hipError_t e, const char* where) {
    if (e == hipSuccess) return QIMG_OK;
    return fail(QIMG_ERR_HIP, "%s: %s", where, hipGetErrorString(e));
}

bool is_pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Every device pointer an entry point takes must be 16-byte aligned (the
// kernels use 16-byte vector and DMA accesses from the base); null pointers
// (optional arguments) pass.
template <typename... P>
bool all_aligned16(const P*... p) {
    return (aligned16(p) && ...);
}

int64_t align256(int64_t v) { return (v + 255) & ~static_cast<int64_t>(255); }

constexpr int kMaxRowK = 32768;  // the fused row kernels keep one row in LDS

#define QIMG_REQUIRE(cond, ...)                                  \
    do {                                                         \
        if (!(cond)) return fail(QIMG_ERR_INVALID_ARG, __VA_ARGS__); \
    } while (0)

int check_rows(const char* fn, int M, int K, int hbs) {
    QIMG_REQUIRE(M >= 0 && K > 0, "%s: need M >= 0 and K > 0 (M=%d K=%d)", fn, M, K);
    QIMG_REQUIRE(is_pow2(hbs), "%s: hbs=%d is not a power of two", fn, hbs);
    QIMG_REQUIRE(K % hbs == 0, "%s: K=%d is not a multiple of hbs=%d", fn, K, hbs);
    if (K > kMaxRowK)
        return fail(QIMG_ERR_UNSUPPORTED, "%s: K=%d exceeds the fused row limit %d", fn, K, kMaxRowK);
    return QIMG_OK;
}

}  // namespace

namespace qimg {

int api_fail(int status, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vfail(status, fmt, ap);
    va_end(ap);
    return status;
}

int api_hip_status(hipError_t e, const char* where) { return hip_status(e, where); }

int check_linear(const char* fn, const void* x, int x_dtype, int M, int K, const void* w_q, const float* w_scales,
                 int N, int hbs, int mode, void* out, int out_dtype, int64_t* need) {
    QIMG_REQUIRE(x_dtype == QIMG_FP32 || x_dtype == QIMG_BF16, "%s: x_dtype %d must be FP32 or BF16", fn,
                 x_dtype);
    QIMG_REQUIRE(mode == QIMG_QM_INT8_HADAMARD || mode == QIMG_QM_FP8_HADAMARD, "%s: bad mode %d", fn, mode);
    QIMG_REQUIRE(out_dtype == QIMG_FP32 || out_dtype == QIMG_BF16, "%s: out_dtype %d must be FP32 or BF16",
                 fn, out_dtype);
    int st = check_rows(fn, M, K, hbs);
    if (st) return st;
    QIMG_REQUIRE(N >= 0, "%s: bad N=%d", fn, N);
    *need = align256(static_cast<int64_t>(M) * K) + align256(static_cast<int64_t>(M) * 4);
    if (M == 0 || N == 0) return QIMG_OK;
    QIMG_REQUIRE(x && w_q && w_scales && out, "%s: null pointer", fn);
    QIMG_REQUIRE(all_aligned16(x, w_q, out), "%s: x, w_q and out must be 16-byte aligned", fn);
    if (mode == QIMG_QM_FP8_HADAMARD && K % 64 != 0)
        return fail(QIMG_ERR_UNSUPPORTED, "%s: e4m3 mode needs K %% 64 == 0 (K=%d)", fn, K);
    return QIMG_OK;
}

int run_linear(const char* fn, const void* x, int x_dtype, int M, int K, const void* w_q, const float* w_scales,
               int N, int hbs, int mode, const uint16_t* bias_bf16, void* out, int out_dtype, int gelu, void* scratch,
               hipStream_t s) {
    uint8_t* qa = static_cast<uint8_t*>(scratch);
    float* sa = reinterpret_cast<float*>(qa + align256(static_cast<int64_t>(M) * K));
    int st = hip_status(qimg::launch_fwht_quant(x, x_dtype, M, K, hbs, mode, qa, sa, s), fn);
    if (st) return st;
    return hip_status(qimg::launch_linear_prequantized(qa, sa, M, K, w_q, w_scales, N, mode, bias_bf16, out,
                                                       out_dtype, gelu, s),
                      fn);
}

}  // namespace qimg

extern "C" {

const char* qimg_status_string(int status) {
    switch (status) {
        case QIMG_OK: return "ok";
        case QIMG_ERR_INVALID_ARG: return "invalid argument";
        case QIMG_ERR_UNSUPPORTED: return "unsupported";
        case QIMG_ERR_SCRATCH: return "scratch too small";
        case QIMG_ERR_HIP: return "HIP error";
        default: return "unknown status";
    }
}

const char* qimg_last_error(void) { return g_err; }

const char* qimg_version(void) { return "qimg-hot 0.1 gfx950"; }

int qimg_hadamard_block_size(int K) { return K & (-K); }

int64_t qimg_int8_scratch_bytes(int M, int K, int N) {
    const int64_t mk = static_cast<int64_t>(M) * K;
    const int64_t mn = static_cast<int64_t>(M) * N;
    return align256((mk > mn ? mk : mn) * 4) + align256(mk) + align256(static_cast<int64_t>(M) * 4);
}

int qimg_fwht_inplace(float* data, int M, int K, int hbs, void* stream) {
    int st = check_rows("qimg_fwht_inplace", M, K, hbs);
    if (st) return st;
    QIMG_REQUIRE(data || M == 0, "qimg_fwht_inplace: data is null");
    QIMG_REQUIRE(aligned16(data), "qimg_fwht_inplace: data must be 16-byte aligned");
    return hip_status(qimg::launch_fwht_inplace(data, M, K, hbs, static_cast<hipStream_t>(stream)),
                      "qimg_fwht_inplace");
}

int qimg_quantize_per_row_fp32(const float* x, int8_t* out, float* scales, int M, int K,
                               void* stream) {
    int st = check_rows("qimg_quantize_per_row_fp32", M, K, 1);
    if (st) return st;
    QIMG_REQUIRE(M == 0 || (x && out && scales), "qimg_quantize_per_row_fp32: null pointer");
    QIMG_REQUIRE(all_aligned16(x, out), "qimg_quantize_per_row_fp32: x and out must be 16-byte aligned");
    return hip_status(qimg::launch_fwht_quant(x, QIMG_FP32, M, K, 1, QIMG_QM_INT8_HADAMARD, out, scales,
                                              static_cast<hipStream_t>(stream)),
                      "qimg_quantize_per_row_fp32");
}

int qimg_quantize_activation(const void* x, int x_dtype, int M, int K, int hbs, int mode,
                             void* q_out, float* scales_out, void* stream) {
    const char* fn = "qimg_quantize_activation";
    QIMG_REQUIRE(x_dtype == QIMG_FP32 || x_dtype == QIMG_BF16, "%s: x_dtype %d must be FP32 or BF16", fn,
                 x_dtype);
    QIMG_REQUIRE(mode == QIMG_QM_INT8_HADAMARD || mode == QIMG_QM_FP8_HADAMARD, "%s: bad mode %d", fn, mode);
    int st = check_rows(fn, M, K, hbs);
    if (st) return st;
    QIMG_REQUIRE(M == 0 || (x && q_out && scales_out), "%s: null pointer", fn);
    QIMG_REQUIRE(all_aligned16(x, q_out), "%s: x and q_out must be 16-byte aligned", fn);
    return hip_status(qimg::launch_fwht_quant(x, x_dtype, M, K, hbs, mode, q_out, scales_out,
                                              static_cast<hipStream_t>(stream)),
                      fn);
}

int qimg_quantize_weight(const void* w, int w_dtype, int N, int K, int mode, void* q_out,
                         float* scales_out, int* hbs_out, void* stream) {
    const char* fn = "qimg_quantize_weight";
    QIMG_REQUIRE(w_dtype == QIMG_FP32 || w_dtype == QIMG_BF16, "%s: w_dtype %d must be BF16 or FP32", fn,
                 w_dtype);
    QIMG_REQUIRE(mode == QIMG_QM_INT8_HADAMARD || mode == QIMG_QM_FP8_HADAMARD, "%s: bad mode %d", fn, mode);
    QIMG_REQUIRE(N > 0 && K > 0, "%s: need N > 0 and K > 0 (N=%d K=%d)", fn, N, K);
    const int hbs = K & (-K);
    int st = check_rows(fn, N, K, hbs);
    if (st) return st;
    QIMG_REQUIRE(w && q_out && scales_out, "%s: null pointer", fn);
    QIMG_REQUIRE(all_aligned16(w, q_out), "%s: w and q_out must be 16-byte aligned", fn);
    hipStream_t s = static_cast<hipStream_t>(stream);
    st = hip_status(qimg::launch_fwht_quant(w, w_dtype, N, K, hbs, mode, q_out, scales_out, s), fn);
    if (st) return st;
    st = hip_status(hipStreamSynchronize(s), fn);
    if (st) return st;
    if (hbs_out) *hbs_out = hbs;
    return QIMG_OK;
}

int qimg_linear_prequantized(const void* act_q, const float* act_scales, int M, int K,
                             const void* w_q, const float* w_scales, int N, int mode,
                             const uint16_t* bias_bf16, void* out, int out_dtype, int gelu,
                             void* stream) {
    const char* fn = "qimg_linear_prequantized";
    QIMG_REQUIRE(mode == QIMG_QM_INT8_HADAMARD || mode == QIMG_QM_FP8_HADAMARD, "%s: bad mode %d", fn, mode);
    QIMG_REQUIRE(out_dtype == QIMG_FP32 || out_dtype == QIMG_BF16, "%s: out_dtype %d must be FP32 or BF16",
                 fn, out_dtype);
    QIMG_REQUIRE(M >= 0 && N >= 0 && K > 0, "%s: bad sizes M=%d N=%d K=%d", fn, M, N, K);
    if (M == 0 || N == 0) return QIMG_OK;
    QIMG_REQUIRE(act_q && act_scales && w_q && w_scales && out, "%s: null pointer", fn);
    if (K % 64 != 0) {
        if (mode == QIMG_QM_FP8_HADAMARD)
            return fail(QIMG_ERR_UNSUPPORTED, "%s: e4m3 mode needs K %% 64 == 0 (K=%d)", fn, K);
    }
    QIMG_REQUIRE(all_aligned16(act_q, w_q, out), "%s: act_q, w_q and out must be 16-byte aligned", fn);
    return hip_status(qimg::launch_linear_prequantized(act_q, act_scales, M, K, w_q, w_scales, N, mode,
                                                       bias_bf16, out, out_dtype, gelu,
                                                       static_cast<hipStream_t>(stream)),
                      fn);
}

int qimg_dequantize_bias(const int32_t* acc, const float* act_scales, const float* w_scales,
                         const uint16_t* bias_bf16, float* out, int M, int N, int gelu, void* stream) {
    const char* fn = "qimg_dequantize_bias";
    QIMG_REQUIRE(M >= 0 && N >= 0, "%s: bad sizes M=%d N=%d", fn, M, N);
    if (M == 0 || N == 0) return QIMG_OK;
    QIMG_REQUIRE(acc && act_scales && w_scales && out, "%s: null pointer", fn);
    return hip_status(qimg::launch_dequant_bias(acc, act_scales, w_scales, bias_bf16, out, M, N, gelu,
                                                static_cast<hipStream_t>(stream)),
                      fn);
}

int qimg_set_linear_kernel(int which) {
    QIMG_REQUIRE(which >= QIMG_LINEAR_AUTO && which <= QIMG_LINEAR_LARGE_128,
                 "qimg_set_linear_kernel: unknown kernel choice %d", which);
    qimg::set_linear_kernel(which);
    return QIMG_OK;
}

int qimg_get_linear_kernel(void) {
    return qimg::get_linear_kernel();
}

int qimg_linear(const void* x, int x_dtype, int M, int K, const void* w_q, const float* w_scales, int N,
                int hbs, int mode, const uint16_t* bias_bf16, void* out, int out_dtype, int gelu,
                void* scratch, int64_t scratch_bytes, void* stream) {
    const char* fn = "qimg_linear";
    int64_t need = 0;
    int st = qimg::check_linear(fn, x, x_dtype, M, K, w_q, w_scales, N, hbs, mode, out, out_dtype, &need);
    if (st || M == 0 || N == 0) return st;
    if (!scratch || scratch_bytes < need)
        return fail(QIMG_ERR_SCRATCH, "%s: scratch %lld bytes < required %lld", fn,
                    static_cast<long long>(scratch_bytes), static_cast<long long>(need));
    QIMG_REQUIRE(aligned16(scratch), "%s: scratch must be 16-byte aligned", fn);
    return qimg::run_linear(fn, x, x_dtype, M, K, w_q, w_scales, N, hbs, mode, bias_bf16, out, out_dtype, gelu, scratch,
                      static_cast<hipStream_t>(stream));
}

int qimg_linear_bf16(const void* x, int x_dtype, int M, int K, const uint16_t* w_bf16, int N,
                     const uint16_t* bias_bf16, float* out, int gelu, void* stream) {
    const char* fn = "qimg_linear_bf16";
    QIMG_REQUIRE(x_dtype == QIMG_FP32 || x_dtype == QIMG_BF16, "%s: x_dtype %d must be FP32 or BF16", fn,
                 x_dtype);
    QIMG_REQUIRE(M >= 0 && N >= 0 && K > 0, "%s: bad sizes M=%d N=%d K=%d", fn, M, N, K);
    if (M == 0 || N == 0) return QIMG_OK;
    QIMG_REQUIRE(x && w_bf16 && out, "%s: null pointer", fn);
    QIMG_REQUIRE(all_aligned16(x, w_bf16, out), "%s: x, w and out must be 16-byte aligned", fn);
    return hip_status(qimg::launch_linear_bf16(x, x_dtype, M, K, w_bf16, N, bias_bf16, out, gelu,
                                               static_cast<hipStream_t>(stream)),
                      fn);
}

int64_t qimg_sage_scratch_bytes(int BH, int S, int D) {
    if (BH <= 0 || S <= 0 || D <= 0) return 0;
    return qimg::sage_scratch_layout(BH, S, D, nullptr, nullptr);
}

static int check_sage(const char* fn, int BH, int S, int D) {
    QIMG_REQUIRE(BH > 0 && S > 0, "%s: need BH > 0 and S > 0 (BH=%d S=%d)", fn, BH, S);
    if (D != 64 && D != 128)
        return fail(QIMG_ERR_UNSUPPORTED, "%s: head_dim %d not supported (64 or 128)", fn, D);
    QIMG_REQUIRE(static_cast<int64_t>(BH) * S * D < (static_cast<int64_t>(1) << 31),
                 "%s: BH*S*D must be < 2^31", fn);
    return QIMG_OK;
}

int qimg_sage_k_mean(const uint16_t* k_f16, float* mean, int BH, int S, int D, void* stream) {
    const char* fn = "qimg_sage_k_mean";
    int st = check_sage(fn, BH, S, D);
    if (st) return st;
    QIMG_REQUIRE(k_f16 && mean, "%s: null pointer", fn);
    QIMG_REQUIRE(aligned16(k_f16), "%s: k must be 16-byte aligned", fn);
    return hip_status(qimg::launch_sage_k_mean(k_f16, mean, BH, S, D, static_cast<hipStream_t>(stream)), fn);
}

int qimg_sage_quant_q(const uint16_t* q_f16, int8_t* q_out, float* q_scale, int BH, int S, int D,
                      void* stream) {
    const char* fn = "qimg_sage_quant_q";
    int st = check_sage(fn, BH, S, D);
    if (st) return st;
    QIMG_REQUIRE(q_f16 && q_out && q_scale, "%s: null pointer", fn);
    QIMG_REQUIRE(aligned16(q_f16) && aligned16(q_out), "%s: q and q_out must be 16-byte aligned", fn);
    return hip_status(qimg::launch_sage_quant_q(q_f16, q_out, q_scale, BH, S, D, static_cast<hipStream_t>(stream)),
                      fn);
}

int qimg_sage_quant_k(const uint16_t* k_f16, const float* mean, int8_t* k_out, float* k_scale, int BH, int S,
                      int D, void* stream) {
    const char* fn = "qimg_sage_quant_k";
    int st = check_sage(fn, BH, S, D);
    if (st) return st;
    QIMG_REQUIRE(k_f16 && mean && k_out && k_scale, "%s: null pointer", fn);
    QIMG_REQUIRE(aligned16(k_f16) && aligned16(k_out), "%s: k and k_out must be 16-byte aligned", fn);
    return hip_status(
        qimg::launch_sage_quant_k(k_f16, mean, k_out, k_scale, BH, S, D, static_cast<hipStream_t>(stream)), fn);
}

int qimg_sage_attn_quantized(const int8_t* q, const int8_t* k, const uint16_t* v_f16, const float* q_scale,
                             const float* k_scale, void* out, int out_dtype, int BH, int S, int D,
                             float sm_scale, int causal, void* scratch, int64_t scratch_bytes,
                             void* stream) {
    const char* fn = "qimg_sage_attn_quantized";
    int st = check_sage(fn, BH, S, D);
    if (st) return st;
    QIMG_REQUIRE(out_dtype == QIMG_FP16 || out_dtype == QIMG_FP32 || out_dtype == QIMG_BF16,
                 "%s: out_dtype %d must be FP16, FP32 or BF16", fn, out_dtype);
    QIMG_REQUIRE(q && k && v_f16 && q_scale && k_scale && out, "%s: null pointer", fn);
    QIMG_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v_f16) && aligned16(out) && aligned16(k_scale),
                 "%s: buffers must be 16-byte aligned", fn);
    const int64_t need = qimg::sage_vt_bytes(BH, S, D);
    if (!scratch || scratch_bytes < need)
        return fail(QIMG_ERR_SCRATCH, "%s: scratch %lld bytes < required %lld", fn,
                    static_cast<long long>(scratch_bytes), static_cast<long long>(need));
    QIMG_REQUIRE(aligned16(scratch), "%s: scratch must be 16-byte aligned", fn);
    return hip_status(qimg::launch_sage_attn(q, k, v_f16, q_scale, k_scale, out, out_dtype, BH, S, D, sm_scale,
                                             causal, static_cast<uint16_t*>(scratch),
                                             static_cast<hipStream_t>(stream)),
                      fn);
}

int qimg_sage_attention(const uint16_t* q_f16, const uint16_t* k_f16, const uint16_t* v_f16, void* out,
                        int out_dtype, float sm_scale, int BH, int S, int D, int causal, void* scratch,
                        int64_t scratch_bytes, void* stream) {
    const char* fn = "qimg_sage_attention";
    int st = check_sage(fn, BH, S, D);
    if (st) return st;
    QIMG_REQUIRE(out_dtype == QIMG_FP16 || out_dtype == QIMG_FP32 || out_dtype == QIMG_BF16,
                 "%s: out_dtype %d must be FP16, FP32 or BF16", fn, out_dtype);
    QIMG_REQUIRE(q_f16 && k_f16 && v_f16 && out, "%s: null pointer", fn);
    QIMG_REQUIRE(aligned16(q_f16) && aligned16(k_f16) && aligned16(v_f16) && aligned16(out),
                 "%s: buffers must be 16-byte aligned", fn);
    const int64_t need = qimg::sage_scratch_layout(BH, S, D, nullptr, nullptr);
    if (!scratch || scratch_bytes < need)
        return fail(QIMG_ERR_SCRATCH, "%s: scratch %lld bytes < required %lld", fn,
                    static_cast<long long>(scratch_bytes), static_cast<long long>(need));
    QIMG_REQUIRE(aligned16(scratch), "%s: scratch must be 16-byte aligned", fn);
    qimg::SageScratch ws;
    qimg::sage_scratch_layout(BH, S, D, scratch, &ws);
    hipStream_t s = static_cast<hipStream_t>(stream);
    st = hip_status(qimg::launch_sage_k_mean(k_f16, ws.k_mean, BH, S, D, s), fn);
    if (st) return st;
    st = hip_status(qimg::launch_sage_quant_q(q_f16, ws.q_i8, ws.q_scale, BH, S, D, s), fn);
    if (st) return st;
    st = hip_status(qimg::launch_sage_quant_k(k_f16, ws.k_mean, ws.k_i8, ws.k_scale, BH, S, D, s), fn);
    if (st) return st;
    return hip_status(qimg::launch_sage_attn(ws.q_i8, ws.k_i8, v_f16, ws.q_scale, ws.k_scale, out, out_dtype,
                                             BH, S, D, sm_scale, causal, ws.v_t, s),
                      fn);
}


/* ---- MMDiT joint block ------------------------------------------------ */

int qimg_silu(const float* x, float* out, int64_t n, void* stream) {
    const char* fn = "qimg_silu";
    QIMG_REQUIRE(n >= 0, "%s: bad n=%lld", fn, static_cast<long long>(n));
    if (n == 0) return QIMG_OK;
    QIMG_REQUIRE(x && out, "%s: null pointer", fn);
    QIMG_REQUIRE(all_aligned16(x, out), "%s: x and out must be 16-byte aligned", fn);
    return hip_status(qimg::launch_silu(x, out, n, static_cast<hipStream_t>(stream)), fn);
}

int qimg_layernorm_modulate(const float* x, const float* shift, const float* scale, float* out, int rows, int dim,
                            float eps, void* stream) {
    const char* fn = "qimg_layernorm_modulate";
    QIMG_REQUIRE(rows >= 0 && dim > 0 && dim % 4 == 0 && dim <= 4096,
                 "%s: need rows >= 0 and dim a multiple of 4 in (0, 4096] (rows=%d dim=%d)", fn, rows, dim);
    if (rows == 0) return QIMG_OK;
    QIMG_REQUIRE(x && shift && scale && out, "%s: null pointer", fn);
    QIMG_REQUIRE(aligned16(x) && aligned16(shift) && aligned16(scale) && aligned16(out),
                 "%s: buffers must be 16-byte aligned", fn);
    return hip_status(qimg::launch_layernorm_modulate(x, shift, scale, out, rows, dim, eps,
                                                      static_cast<hipStream_t>(stream)),
                      fn);
}

int qimg_layernorm_modulate_quant(const float* x, const float* shift, const float* scale, int rows, int dim, int hbs,
                                  int mode, float eps, void* q_out, float* q_scales, void* stream) {
    const char* fn = "qimg_layernorm_modulate_quant";
    QIMG_REQUIRE(rows >= 0 && dim > 0 && dim % 4 == 0 && dim <= 4096,
                 "%s: need rows >= 0 and dim a multiple of 4 in (0, 4096] (rows=%d dim=%d)", fn, rows, dim);
    QIMG_REQUIRE(mode == QIMG_QM_INT8_HADAMARD || mode == QIMG_QM_FP8_HADAMARD, "%s: bad mode %d", fn, mode);
    QIMG_REQUIRE(hbs >= 1 && (hbs & (hbs - 1)) == 0 && dim % hbs == 0,
                 "%s: hbs=%d must be a power of two dividing dim=%d", fn, hbs, dim);
    if (rows == 0) return QIMG_OK;
    QIMG_REQUIRE(x && shift && scale && q_out && q_scales, "%s: null pointer", fn);
    QIMG_REQUIRE(aligned16(x) && aligned16(shift) && aligned16(scale) && aligned16(q_out),
                 "%s: buffers must be 16-byte aligned", fn);
    return hip_status(qimg::launch_ln_fwht_quant(x, shift, scale, rows, dim, hbs, mode, eps, q_out, q_scales,
                                                 static_cast<hipStream_t>(stream)),
                      fn);
}

static int check_heads(const char* fn, int n_txt, int n_img, int H) {
    QIMG_REQUIRE(n_txt >= 0 && n_img >= 0 && H > 0, "%s: bad sizes n_txt=%d n_img=%d H=%d", fn, n_txt, n_img, H);
    QIMG_REQUIRE(static_cast<int64_t>(n_txt + n_img) * H * 128 < (int64_t{1} << 31), "%s: too many elements", fn);
    return QIMG_OK;
}

int qimg_joint_heads_f16(const float* txt, const float* img, const uint16_t* norm_txt, const uint16_t* norm_img,
                         const float* pe, uint16_t* out, int n_txt, int n_img, int H, float eps, void* stream) {
    const char* fn = "qimg_joint_heads_f16";
    int st = check_heads(fn, n_txt, n_img, H);
    if (st) return st;
    if (n_txt + n_img == 0) return QIMG_OK;
    QIMG_REQUIRE(out && (txt || n_txt == 0) && (img || n_img == 0), "%s: null pointer", fn);
    QIMG_REQUIRE((norm_txt == nullptr) == (norm_img == nullptr), "%s: give both RMSNorm weights or neither", fn);
    QIMG_REQUIRE(norm_txt == nullptr || pe != nullptr, "%s: RMSNorm + RoPE needs pe", fn);
    QIMG_REQUIRE(all_aligned16(txt, img, pe, out), "%s: txt, img, pe and out must be 16-byte aligned", fn);
    return hip_status(qimg::launch_joint_heads_f16(txt, img, norm_txt, norm_img, pe, out, n_txt, n_img, 1, H, eps,
                                                   static_cast<hipStream_t>(stream)),
                      fn);
}

int qimg_split_heads(const uint16_t* attn_f16, float* txt, float* img, int n_txt, int n_img, int H, void* stream) {
    const char* fn = "qimg_split_heads";
    int st = check_heads(fn, n_txt, n_img, H);
    if (st) return st;
    if (n_txt + n_img == 0) return QIMG_OK;
    QIMG_REQUIRE(attn_f16 && (txt || n_txt == 0) && (img || n_img == 0), "%s: null pointer", fn);
    QIMG_REQUIRE(all_aligned16(attn_f16, txt, img), "%s: attn, txt and img must be 16-byte aligned", fn);
    return hip_status(
        qimg::launch_split_heads(attn_f16, txt, img, n_txt, n_img, 1, H, static_cast<hipStream_t>(stream)), fn);
}

int qimg_gate_add(const float* x, const float* gate, const float* y, float* out, int rows, int dim, void* stream) {
    const char* fn = "qimg_gate_add";
    QIMG_REQUIRE(rows >= 0 && dim > 0 && dim % 4 == 0, "%s: need dim a multiple of 4 (rows=%d dim=%d)", fn, rows,
                 dim);
    if (rows == 0) return QIMG_OK;
    QIMG_REQUIRE(x && gate && y && out, "%s: null pointer", fn);
    QIMG_REQUIRE(aligned16(x) && aligned16(gate) && aligned16(y) && aligned16(out),
                 "%s: buffers must be 16-byte aligned", fn);
    return hip_status(qimg::launch_gate_add(x, gate, y, out, rows, dim, static_cast<hipStream_t>(stream)), fn);
}

int64_t qimg_mmdit_blocks_scratch_bytes(int n_img, int n_txt, int batch) {
    if (n_img < 0 || n_txt < 0 || n_img + n_txt == 0 || batch < 1) return 0;
    return qimg::mmdit_block_scratch_layout(n_img, n_txt, batch, nullptr, nullptr);
}

int64_t qimg_mmdit_block_scratch_bytes(int n_img, int n_txt) { return qimg_mmdit_blocks_scratch_bytes(n_img, n_txt, 1); }

static int check_qlinear(const char* fn, const char* name, const qimg_qlinear& l, int N, int K) {
    QIMG_REQUIRE(l.w && l.scales, "%s: %s: null weight", fn, name);
    QIMG_REQUIRE(l.N == N && l.K == K, "%s: %s is [%d, %d], expected [%d, %d]", fn, name, l.N, l.K, N, K);
    QIMG_REQUIRE(l.mode == QIMG_QM_INT8_HADAMARD || l.mode == QIMG_QM_FP8_HADAMARD, "%s: %s: bad mode %d", fn, name,
                 l.mode);
    QIMG_REQUIRE(l.hbs == (K & -K), "%s: %s: hbs %d must be K & -K = %d", fn, name, l.hbs, K & -K);
    QIMG_REQUIRE(aligned16(l.w) && aligned16(l.scales), "%s: %s: weights must be 16-byte aligned", fn, name);
    return QIMG_OK;
}

static int check_block(const char* fn, int index, const qimg_mmdit_block* b) {
    QIMG_REQUIRE(b->norm_q && b->norm_k && b->norm_added_q && b->norm_added_k, "%s: block %d: null RMSNorm weight",
                 fn, index);
    const int D = 3072, F = 12288;
    struct {
        const char* name;
        const qimg_qlinear* l;
        int N, K;
    } lin[] = {{"img_mod", &b->img_mod, 6 * D, D},      {"txt_mod", &b->txt_mod, 6 * D, D},
               {"to_q", &b->to_q, D, D},                {"to_k", &b->to_k, D, D},
               {"to_v", &b->to_v, D, D},                {"add_q_proj", &b->add_q_proj, D, D},
               {"add_k_proj", &b->add_k_proj, D, D},    {"add_v_proj", &b->add_v_proj, D, D},
               {"to_out", &b->to_out, D, D},            {"to_add_out", &b->to_add_out, D, D},
               {"img_mlp_fc1", &b->img_mlp_fc1, F, D},  {"img_mlp_fc2", &b->img_mlp_fc2, D, F},
               {"txt_mlp_fc1", &b->txt_mlp_fc1, F, D},  {"txt_mlp_fc2", &b->txt_mlp_fc2, D, F}};
    for (const auto& e : lin) {
        int st = check_qlinear(fn, e.name, *e.l, e.N, e.K);
        if (st) return st;
    }
    return QIMG_OK;
}

int qimg_mmdit_blocks_forward(const qimg_mmdit_block* blocks, int n_blocks, float* img, float* txt,
                              const float* t_emb, const float* pe, int n_img, int n_txt, int batch, void* scratch,
                              int64_t scratch_bytes, float* prof_ms, void* stream) {
    const char* fn = "qimg_mmdit_blocks_forward";
    QIMG_REQUIRE(blocks != nullptr && n_blocks >= 1, "%s: need at least one block (n_blocks=%d)", fn, n_blocks);
    QIMG_REQUIRE(batch >= 1, "%s: batch must be >= 1 (got %d)", fn, batch);
    QIMG_REQUIRE(n_img >= 0 && n_txt >= 0 && n_img + n_txt > 0, "%s: bad token counts n_img=%d n_txt=%d", fn,
                 n_img, n_txt);
    const int64_t rows = static_cast<int64_t>(batch) * (n_img > n_txt ? n_img : n_txt);
    QIMG_REQUIRE(static_cast<int64_t>(batch) * (n_img + n_txt) * 3072 < (int64_t{1} << 31) &&
                     rows * 12288 < (int64_t{1} << 31),
                 "%s: too many tokens", fn);
    QIMG_REQUIRE((img || n_img == 0) && (txt || n_txt == 0) && t_emb && pe, "%s: null pointer", fn);
    QIMG_REQUIRE((n_img == 0 || aligned16(img)) && (n_txt == 0 || aligned16(txt)),
                 "%s: img/txt must be 16-byte aligned", fn);
    for (int i = 0; i < n_blocks; ++i) {
        int st = check_block(fn, i, blocks + i);
        if (st) return st;
    }
    const int64_t need = qimg::mmdit_block_scratch_layout(n_img, n_txt, batch, nullptr, nullptr);
    if (!scratch || scratch_bytes < need)
        return fail(QIMG_ERR_SCRATCH, "%s: scratch %lld bytes < required %lld", fn,
                    static_cast<long long>(scratch_bytes), static_cast<long long>(need));
    QIMG_REQUIRE(aligned16(scratch), "%s: scratch must be 16-byte aligned", fn);
    qimg::BlockScratch ws;
    qimg::mmdit_block_scratch_layout(n_img, n_txt, batch, scratch, &ws);
    if (prof_ms)
        for (int c = 0; c < QIMG_PROF_COUNT; ++c) prof_ms[c] = 0.0f;
    // (a block's modulation chunks may have been computed by the block
    // before it, into the chunk set the block reads)
    bool mods_ready = false;
    for (int i = 0; i < n_blocks; ++i) {
        // silu(t_emb) and its quantization carry over from the previous block
        // when its img_mod quantizes the same way
        const qimg_qlinear& m = blocks[i].img_mod;
        const bool t_ready = i > 0 && blocks[i - 1].img_mod.K == m.K && blocks[i - 1].img_mod.hbs == m.hbs &&
                             blocks[i - 1].img_mod.mode == m.mode;
        bool next_ready = false;
        const int st = hip_status(
            qimg::run_mmdit_block(blocks[i], img, txt, t_emb, pe, n_img, n_txt, batch, ws, prof_ms,
                                  static_cast<hipStream_t>(stream), t_ready, i & 1, mods_ready,
                                  i + 1 < n_blocks ? blocks + i + 1 : nullptr, &next_ready),
            fn);
        if (st) return st;
        mods_ready = next_ready;
    }
    return QIMG_OK;
}

int qimg_mmdit_block_forward(const qimg_mmdit_block* b, float* img, float* txt, const float* t_emb, const float* pe,
                             int n_img, int n_txt, void* scratch, int64_t scratch_bytes, float* prof_ms,
                             void* stream) {
    return qimg_mmdit_blocks_forward(b, 1, img, txt, t_emb, pe, n_img, n_txt, 1, scratch, scratch_bytes, prof_ms,
                                     stream);
}

}  // extern "C"
