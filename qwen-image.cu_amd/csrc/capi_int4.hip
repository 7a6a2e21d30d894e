// capi_int4.hip — the extern "C" boundary of the INT4 paths
// (include/qimg_hot.h, cuda_kernels.cu:2864-4532). Arguments are checked on
// the host before any HIP call; failures return a qimg_status with the
// message in qimg_last_error().
#include <algorithm>

#include "qimg_internal.h"

namespace {

using qimg::api_fail;
using qimg::api_hip_status;

#define QIMG_REQUIRE(cond, ...)                                           \
    do {                                                                  \
        if (!(cond)) return api_fail(QIMG_ERR_INVALID_ARG, __VA_ARGS__); \
    } while (0)

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <typename... P>
bool all_aligned16(const P*... p) {
    return (aligned16(p) && ...);
}

int64_t align256(int64_t v) { return (v + 255) & ~static_cast<int64_t>(255); }

hipStream_t hs(void* s) { return static_cast<hipStream_t>(s); }

// Scratch layout of qimg_linear_int4 (offsets into the caller's buffer).
struct Int4Layout {
    int64_t a, xr, xs, lr32, lr16, svd_t, act_scales, total;
};

Int4Layout int4_layout(int M, int K, int N, int r, int group_size, bool w4a4) {
    Int4Layout L{};
    int64_t off = 0;
    auto take = [&](int64_t bytes) {
        const int64_t at = off;
        off += align256(bytes);
        return at;
    };
    if (w4a4) {
        L.a = take(static_cast<int64_t>(M) * (K / 2));  // packed activations
        L.act_scales = take(static_cast<int64_t>(K / group_size) * M * 4);
        L.svd_t = take(static_cast<int64_t>(r) * K * 2);
        L.xr = -1;
    } else {
        // dequantized residual weight; first the transposed down factor
        L.a = take(std::max(static_cast<int64_t>(N) * K * 2, static_cast<int64_t>(r) * K * 2));
        L.svd_t = L.a;
        L.act_scales = -1;
        L.xr = take(static_cast<int64_t>(M) * K * 2);
    }
    L.xs = take(static_cast<int64_t>(M) * K * 2);
    L.lr32 = take(static_cast<int64_t>(M) * r * 4);
    L.lr16 = take(static_cast<int64_t>(M) * r * 2);
    L.total = off;
    return L;
}

// int4_scratch_bytes, cuda_kernels.cuh:475-487 (group size 64 assumed there)
int64_t reference_int4_scratch(int M, int K, int N, int r) {
    const int64_t a16 = static_cast<int64_t>(N) * K * 2;
    const int64_t a4 = align256(static_cast<int64_t>(M) * (K / 2)) + align256(static_cast<int64_t>(K / 64) * M * 4) +
                       static_cast<int64_t>(M) * N * 4;
    return align256(std::max(a16, a4)) + align256(static_cast<int64_t>(M) * K * 4) +
           align256(static_cast<int64_t>(M) * K * 2) + align256(static_cast<int64_t>(M) * r * 2);
}

}  // namespace

extern "C" {

int qimg_dequantize_int4_bf16(const uint8_t* qweight, const float* scales, uint16_t* out, int N, int K,
                              int group_size, int nf4_grid, int scales_gn, int signed_int4, void* stream) {
    const char* fn = "qimg_dequantize_int4_bf16";
    QIMG_REQUIRE(N >= 0 && K > 0 && group_size > 0, "%s: bad sizes N=%d K=%d group_size=%d", fn, N, K, group_size);
    QIMG_REQUIRE(K % 8 == 0 && K % group_size == 0, "%s: K=%d must be a multiple of 8 and of group_size=%d", fn, K,
                 group_size);
    if (N == 0) return QIMG_OK;
    QIMG_REQUIRE(qweight && scales && out, "%s: null pointer", fn);
    QIMG_REQUIRE(all_aligned16(qweight, scales, out), "%s: pointers must be 16-byte aligned", fn);
    return api_hip_status(qimg::launch_dequant_int4_bf16(qweight, scales, out, N, K, group_size, nf4_grid != 0,
                                                         scales_gn != 0, signed_int4 != 0, hs(stream)),
                          fn);
}

int qimg_quantize_int4_per_group(const float* residual, uint8_t* qweight, float* scales, int N, int K,
                                 int group_size, int nf4_grid, void* stream) {
    const char* fn = "qimg_quantize_int4_per_group";
    QIMG_REQUIRE(N >= 0 && K > 0 && group_size > 0 && group_size % 2 == 0 && K % group_size == 0,
                 "%s: bad sizes N=%d K=%d group_size=%d", fn, N, K, group_size);
    if (N == 0) return QIMG_OK;
    QIMG_REQUIRE(residual && qweight && scales, "%s: null pointer", fn);
    QIMG_REQUIRE(all_aligned16(residual, qweight, scales), "%s: pointers must be 16-byte aligned", fn);
    return api_hip_status(
        qimg::launch_quant_int4_weight(residual, qweight, scales, N, K, group_size, nf4_grid != 0, hs(stream)), fn);
}

static int act_int4(const char* fn, const float* x, const float* smooth, uint16_t* bf16_out, uint8_t* packed,
                    float* scales, int M, int K, int group_size, void* stream) {
    QIMG_REQUIRE(M >= 0 && K > 0, "%s: bad sizes M=%d K=%d", fn, M, K);
    if (group_size != 32 && group_size != 64 && group_size != 128)
        return api_fail(QIMG_ERR_UNSUPPORTED, "%s: group_size %d not supported (32, 64 or 128)", fn, group_size);
    QIMG_REQUIRE(K % group_size == 0, "%s: K=%d is not a multiple of group_size=%d", fn, K, group_size);
    if (M == 0) return QIMG_OK;
    QIMG_REQUIRE(x && packed && scales, "%s: null pointer", fn);
    QIMG_REQUIRE(all_aligned16(x, smooth, bf16_out, packed, scales), "%s: pointers must be 16-byte aligned", fn);
    return api_hip_status(
        qimg::launch_quant_act_int4(x, smooth, bf16_out, packed, scales, M, K, group_size, hs(stream)), fn);
}

int qimg_quantize_activation_int4(const float* x, uint8_t* act_packed, float* act_scales, int M, int K,
                                  int group_size, void* stream) {
    return act_int4("qimg_quantize_activation_int4", x, nullptr, nullptr, act_packed, act_scales, M, K, group_size,
                    stream);
}

int qimg_fused_smooth_bf16_quant(const float* x, const float* smooth, uint16_t* bf16_out, uint8_t* act_packed,
                                 float* act_scales, int M, int K, int group_size, void* stream) {
    const char* fn = "qimg_fused_smooth_bf16_quant";
    QIMG_REQUIRE(bf16_out != nullptr || M == 0, "%s: bf16_out is null", fn);
    return act_int4(fn, x, smooth, bf16_out, act_packed, act_scales, M, K, group_size, stream);
}

int qimg_w4a4_gemm(const uint8_t* act_packed, const uint8_t* wgt_packed, const float* act_scales,
                   const float* wgt_scales, float* out, int M, int N, int K, int group_size, int accumulate,
                   const uint16_t* bias_bf16, void* stream) {
    const char* fn = "qimg_w4a4_gemm";
    QIMG_REQUIRE(M >= 0 && N >= 0 && K > 0, "%s: bad sizes M=%d N=%d K=%d", fn, M, N, K);
    if (group_size <= 0 || group_size % 64 != 0 || K % group_size != 0)
        return api_fail(QIMG_ERR_UNSUPPORTED, "%s: group_size %d must be a multiple of 64 dividing K=%d", fn,
                        group_size, K);
    if (M == 0 || N == 0) return QIMG_OK;
    QIMG_REQUIRE(act_packed && wgt_packed && act_scales && wgt_scales && out, "%s: null pointer", fn);
    QIMG_REQUIRE(all_aligned16(act_packed, wgt_packed, act_scales, wgt_scales, out),
                 "%s: pointers must be 16-byte aligned", fn);
    return api_hip_status(qimg::launch_w4a4_gemm(act_packed, wgt_packed, act_scales, wgt_scales, out, M, N, K,
                                                 group_size, accumulate != 0, bias_bf16, 0, hs(stream)),
                          fn);
}

int64_t qimg_int4_scratch_bytes(int M, int K, int N, int svd_rank) {
    if (M <= 0 || K <= 0 || N <= 0 || svd_rank < 0) return 0;
    const int64_t mine = std::max(int4_layout(M, K, N, svd_rank, 64, false).total,
                                  int4_layout(M, K, N, svd_rank, 32, true).total);
    return std::max(mine, reference_int4_scratch(M, K, N, svd_rank));
}

int qimg_linear_int4(const float* x, int M, const qimg_int4_weight* w, const uint16_t* bias_bf16, float* out,
                     int gelu, void* scratch, int64_t scratch_bytes, void* stream) {
    const char* fn = "qimg_linear_int4";
    QIMG_REQUIRE(w != nullptr, "%s: null weight", fn);
    const int N = w->N, K = w->K, r = w->rank, gs = w->group_size;
    QIMG_REQUIRE(M >= 0 && N > 0 && K > 0 && r >= 0 && gs > 0, "%s: bad sizes M=%d N=%d K=%d rank=%d group_size=%d",
                 fn, M, N, K, r, gs);
    QIMG_REQUIRE(K % gs == 0 && K % 8 == 0, "%s: K=%d must be a multiple of 8 and of group_size=%d", fn, K, gs);
    const bool w4a4 = w->w4a4_qweight != nullptr;
    if (w4a4 && gs != 64 && gs != 128)
        return api_fail(QIMG_ERR_UNSUPPORTED, "%s: W4A4 group_size %d not supported (64 or 128)", fn, gs);
    // nunchaku weights through the W4A16 residual: signed nibbles, scales
    // [K/gs, N], no rotation (cuda_kernels.cu:4443-4470)
    const bool nk16 = !w4a4 && w->w4a16_nunchaku != 0;
    const int hbs = (w4a4 || nk16) ? 1 : (w->had_block_size > 1 ? w->had_block_size : 1);
    QIMG_REQUIRE((hbs & (hbs - 1)) == 0 && K % hbs == 0, "%s: had_block_size %d must be a power of two dividing K", fn,
                 w->had_block_size);
    if (K > 32768) return api_fail(QIMG_ERR_UNSUPPORTED, "%s: K=%d exceeds the row limit 32768", fn, K);
    if (M == 0) return QIMG_OK;
    QIMG_REQUIRE(x && out, "%s: null x or out", fn);
    QIMG_REQUIRE(r == 0 || (w->svd_up && w->svd_down), "%s: rank %d needs svd_up and svd_down", fn, r);
    QIMG_REQUIRE(w4a4 ? w->w4a4_wscales != nullptr : (w->qweight && w->scales4), "%s: missing residual weight", fn);
    QIMG_REQUIRE(all_aligned16(x, out, w->qweight, w->scales4, w->w4a4_qweight, w->w4a4_wscales, w->svd_up,
                               w->svd_down, w->smooth, scratch),
                 "%s: pointers must be 16-byte aligned", fn);
    const Int4Layout L = int4_layout(M, K, N, r, gs, w4a4);
    if (scratch == nullptr || scratch_bytes < L.total)
        return api_fail(QIMG_ERR_SCRATCH, "%s: scratch %lld bytes < %lld needed", fn,
                        static_cast<long long>(scratch_bytes), static_cast<long long>(L.total));
    hipStream_t s = hs(stream);
    uint8_t* base = static_cast<uint8_t*>(scratch);
    uint16_t* xs = reinterpret_cast<uint16_t*>(base + L.xs);
    hipError_t e;
    // 1. the inputs of both branches in one pass over x
    if (w4a4)
        e = qimg::launch_quant_act_int4(x, w->smooth, xs, base + L.a, reinterpret_cast<float*>(base + L.act_scales), M,
                                        K, gs, s);
    else
        e = qimg::launch_int4_prep(x, w->smooth, xs, reinterpret_cast<uint16_t*>(base + L.xr), M, K, hbs, s);
    if (e != hipSuccess) return api_hip_status(e, fn);
    // 2. low-rank branch: lr = bf16(x_lr . svd_down), out = lr . svd_up^T
    if (r > 0) {
        uint16_t* svd_t = reinterpret_cast<uint16_t*>(base + L.svd_t);
        float* lr32 = reinterpret_cast<float*>(base + L.lr32);
        uint16_t* lr16 = reinterpret_cast<uint16_t*>(base + L.lr16);
        if ((e = qimg::launch_transpose_u16(w->svd_down, svd_t, K, r, s)) != hipSuccess ||
            (e = qimg::launch_linear_bf16(xs, QIMG_BF16, M, K, svd_t, r, nullptr, lr32, 0, s)) != hipSuccess ||
            (e = qimg::launch_f32_to_bf16(lr32, lr16, static_cast<int64_t>(M) * r, s)) != hipSuccess ||
            (e = qimg::launch_linear_bf16(lr16, QIMG_BF16, M, r, w->svd_up, N, nullptr, out, 0, s)) != hipSuccess)
            return api_hip_status(e, fn);
    }
    // 3. residual onto it, then the bias and GELU
    if (w4a4) {
        e = qimg::launch_w4a4_gemm(base + L.a, w->w4a4_qweight, reinterpret_cast<const float*>(base + L.act_scales),
                                   w->w4a4_wscales, out, M, N, K, gs, r > 0, bias_bf16, gelu != 0, s);
    } else {
        uint16_t* deq = reinterpret_cast<uint16_t*>(base + L.a);
        e = nk16 ? qimg::launch_dequant_int4_bf16(w->qweight, w->scales4, deq, N, K, gs, 0, 1, 1, s)
                 : qimg::launch_dequant_int4_bf16(w->qweight, w->scales4, deq, N, K, gs, w->nf4_grid != 0, 0, 0, s);
        if (e == hipSuccess)
            e = qimg::launch_linear_bf16(reinterpret_cast<const uint16_t*>(base + L.xr), QIMG_BF16, M, K, deq, N,
                                         bias_bf16, out, gelu != 0, s, r > 0);
    }
    return api_hip_status(e, fn);
}

int qimg_bf16_to_fp32(const uint16_t* in, float* out, int64_t n, void* stream) {
    const char* fn = "qimg_bf16_to_fp32";
    QIMG_REQUIRE(n >= 0, "%s: bad n=%lld", fn, static_cast<long long>(n));
    if (n == 0) return QIMG_OK;
    QIMG_REQUIRE(in && out, "%s: null pointer", fn);
    return api_hip_status(qimg::launch_bf16_to_f32(in, out, n, hs(stream)), fn);
}

int qimg_smooth_hadamard(const float* x, const float* smooth, float* out, int M, int K, int hbs, void* stream) {
    const char* fn = "qimg_smooth_hadamard";
    QIMG_REQUIRE(M >= 0 && K > 0, "%s: bad sizes M=%d K=%d", fn, M, K);
    QIMG_REQUIRE(hbs >= 1 && (hbs & (hbs - 1)) == 0 && K % hbs == 0, "%s: hbs=%d must be a power of two dividing K=%d",
                 fn, hbs, K);
    if (K > 32768) return api_fail(QIMG_ERR_UNSUPPORTED, "%s: K=%d exceeds the row limit 32768", fn, K);
    if (M == 0) return QIMG_OK;
    QIMG_REQUIRE(x && out, "%s: null pointer", fn);
    QIMG_REQUIRE(all_aligned16(x, smooth, out), "%s: pointers must be 16-byte aligned", fn);
    return api_hip_status(qimg::launch_smooth_fwht_f32(x, smooth, out, M, K, hbs, hs(stream)), fn);
}

int qimg_awq_repack(const int32_t* qweight_awq, int32_t* qweight_out, int OC, int IC, void* stream) {
    const char* fn = "qimg_awq_repack";
    QIMG_REQUIRE(OC >= 0 && IC > 0 && OC % 4 == 0 && IC % 64 == 0, "%s: bad sizes OC=%d IC=%d", fn, OC, IC);
    if (OC == 0) return QIMG_OK;
    QIMG_REQUIRE(qweight_awq && qweight_out, "%s: null pointer", fn);
    QIMG_REQUIRE(all_aligned16(qweight_awq, qweight_out), "%s: pointers must be 16-byte aligned", fn);
    return api_hip_status(qimg::launch_awq_repack(qweight_awq, qweight_out, OC, IC, hs(stream)), fn);
}

int qimg_dequantize_awq_bf16(const int32_t* qweight_awq, const uint16_t* wscales, const uint16_t* wzeros,
                             uint16_t* out, int OC, int IC, int group_size, int num_components, void* stream) {
    const char* fn = "qimg_dequantize_awq_bf16";
    QIMG_REQUIRE(OC >= 0 && IC > 0 && OC % 4 == 0 && IC % 64 == 0 && group_size > 0 && IC % group_size == 0 &&
                     num_components > 0 && OC % num_components == 0,
                 "%s: bad sizes OC=%d IC=%d group_size=%d num_components=%d", fn, OC, IC, group_size,
                 num_components);
    if (OC == 0) return QIMG_OK;
    QIMG_REQUIRE(qweight_awq && wscales && wzeros && out, "%s: null pointer", fn);
    QIMG_REQUIRE(all_aligned16(qweight_awq, wscales, wzeros, out), "%s: pointers must be 16-byte aligned", fn);
    return api_hip_status(
        qimg::launch_awq_dequant(qweight_awq, wscales, wzeros, out, OC, IC, group_size, num_components, hs(stream)),
        fn);
}

int qimg_linear_awq(const float* x, const int32_t* qweight_repacked, const uint16_t* wscales,
                    const uint16_t* wzeros, const uint16_t* bias_bf16, float* out, int OC, int IC, int group_size,
                    int num_components, void* stream) {
    const char* fn = "qimg_linear_awq";
    QIMG_REQUIRE(OC >= 0 && IC > 0 && IC % 64 == 0 && num_components > 0 && OC % num_components == 0,
                 "%s: bad sizes OC=%d IC=%d num_components=%d", fn, OC, IC, num_components);
    if (group_size != 64)
        return api_fail(QIMG_ERR_UNSUPPORTED, "%s: group_size %d not supported (the GEMV reads groups of 64)", fn,
                        group_size);
    if (IC > 16384) return api_fail(QIMG_ERR_UNSUPPORTED, "%s: IC=%d exceeds 16384", fn, IC);
    if (OC == 0) return QIMG_OK;
    QIMG_REQUIRE(x && qweight_repacked && wscales && wzeros && out, "%s: null pointer", fn);
    QIMG_REQUIRE(all_aligned16(x, qweight_repacked, wscales, wzeros, out), "%s: pointers must be 16-byte aligned", fn);
    return api_hip_status(qimg::launch_awq_gemv(x, qweight_repacked, wscales, wzeros, bias_bf16, out, OC, IC,
                                                group_size, num_components, hs(stream)),
                          fn);
}

int qimg_unswizzle_nunchaku_weights(const uint8_t* qweight_swizzled, const uint16_t* wscales_swizzled,
                                    uint8_t* qweight_rowmajor, float* wscales_rowmajor, int N, int K,
                                    int num_groups, void* stream) {
    const char* fn = "qimg_unswizzle_nunchaku_weights";
    QIMG_REQUIRE(N >= 0 && K > 0 && N % 128 == 0 && K % 64 == 0 && num_groups > 0 && K % num_groups == 0 &&
                     (K / num_groups) % 2 == 0,
                 "%s: bad sizes N=%d K=%d num_groups=%d", fn, N, K, num_groups);
    if (N == 0) return QIMG_OK;
    QIMG_REQUIRE(qweight_swizzled && wscales_swizzled && qweight_rowmajor && wscales_rowmajor, "%s: null pointer", fn);
    QIMG_REQUIRE(all_aligned16(qweight_swizzled, wscales_swizzled, qweight_rowmajor, wscales_rowmajor),
                 "%s: pointers must be 16-byte aligned", fn);
    return api_hip_status(qimg::launch_nk_unswizzle(qweight_swizzled, wscales_swizzled, qweight_rowmajor,
                                                    wscales_rowmajor, N, K, num_groups, hs(stream)),
                          fn);
}

int qimg_dequantize_nunchaku_bf16(const uint8_t* qweight_swizzled, const uint16_t* wscales_swizzled,
                                  uint16_t* out, int N, int K, int num_groups, void* stream) {
    const char* fn = "qimg_dequantize_nunchaku_bf16";
    QIMG_REQUIRE(N >= 0 && K > 0 && N % 128 == 0 && K % 64 == 0 && num_groups > 0 && K % num_groups == 0,
                 "%s: bad sizes N=%d K=%d num_groups=%d", fn, N, K, num_groups);
    if (N == 0) return QIMG_OK;
    QIMG_REQUIRE(qweight_swizzled && wscales_swizzled && out, "%s: null pointer", fn);
    QIMG_REQUIRE(all_aligned16(qweight_swizzled, wscales_swizzled, out), "%s: pointers must be 16-byte aligned", fn);
    return api_hip_status(
        qimg::launch_nk_dequant(qweight_swizzled, wscales_swizzled, out, N, K, num_groups, hs(stream)), fn);
}

int qimg_unswizzle_lora_weights(const uint16_t* packed, uint16_t* out, int rows, int cols, int is_down,
                                void* stream) {
    const char* fn = "qimg_unswizzle_lora_weights";
    QIMG_REQUIRE(rows >= 0 && cols > 0 && rows % 16 == 0 && cols % 16 == 0, "%s: bad sizes rows=%d cols=%d", fn, rows,
                 cols);
    if (rows == 0) return QIMG_OK;
    QIMG_REQUIRE(packed && out, "%s: null pointer", fn);
    QIMG_REQUIRE(all_aligned16(packed, out), "%s: pointers must be 16-byte aligned", fn);
    return api_hip_status(qimg::launch_lora_unswizzle(packed, out, rows, cols, is_down != 0, hs(stream)), fn);
}

}  // extern "C"
