// block_ops.hip — the element-wise and per-row operations of an MMDiT joint
// block around the quantized linears and the attention (transformer.cu:
// 497-836): SiLU, LayerNorm + modulate, per-head RMSNorm + RoPE on Q/K
// (fused with the txt-first concat and the [S,H,D] -> [H,S,D] transpose),
// the V concat/transpose, the attention-output transpose/split, and the
// gated residual add.
//
// The reference runs RMSNorm, concat/transpose and RoPE as three kernels
// with two fp32 round trips (cuda_kernels.cu:1656-1687,
// transformer.cu:106-130, cuda_kernels.cu:1935-1971); here one wave per
// (token, head) does all three from registers and writes fp16 once. The
// attention output is read as fp16 directly by the split (the reference
// converts it to fp32 first, sageattention_sm80.cu:1026; fp16 -> fp32 is
// exact, so the values are the same).
//
// Head dim is 128 (one lane per RoPE pair), hidden = H * 128.
#include "qimg_device.h"
#include "qimg_internal.h"

namespace qimg {

namespace {

constexpr int HD = 128;  // head dim

// silu_fp32_kernel (cuda_kernels.cu:1881-1887)
__global__ __launch_bounds__(256) void silu_kernel(const float* __restrict__ x, float* __restrict__ out, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) {
        const float v = x[i];
        out[i] = v / (1.0f + expf(-v));
    }
}

// layer_norm_modulate_fp32_kernel (cuda_kernels.cu:1799-1853), one
// workgroup per row (ln_modulate_row).
__global__ __launch_bounds__(LN_THR) void layernorm_modulate_kernel(const float* __restrict__ x,
                                                                    const float* __restrict__ shift,
                                                                    const float* __restrict__ scale,
                                                                    float* __restrict__ out, int dim, float eps) {
    __shared__ float red[LN_THR / 64];
    const int64_t row = blockIdx.x;
    v4f* o = reinterpret_cast<v4f*>(out + row * dim);
    ln_modulate_row(x + row * dim, shift, scale, dim, eps, red, [&](int c, v4f v) { o[c] = v; });
}

// One workgroup of four waves per (sequence b, token s) of the joint
// sequences (txt tokens first; the pe table is shared by the sequences);
// wave w takes heads w, w + 4, ..., with the loads of up to JH_BATCH heads
// in flight at once and the token's RoPE row read once. Per head:
// optional RMSNorm over its 128 values with a bf16 weight
// (rms_norm_fp32_kernel, cuda_kernels.cu:1656-1687), optional RoPE on the
// pair (2l, 2l+1) held by lane l with pe[s][l] = (cos, -sin, sin, cos)
// (rope_apply_fp32_to_fp16_kernel, :1935-1962), fp16 out at [b][h][s][:]
// (concat_transpose_fused_fp32, transformer.cu:106-130).
constexpr int JH_BATCH = 6;

template <bool NORM_ROPE>
__global__ __launch_bounds__(256) void joint_heads_f16_kernel(const float* __restrict__ txt,
                                                              const float* __restrict__ img,
                                                              const uint16_t* __restrict__ w_txt,
                                                              const uint16_t* __restrict__ w_img,
                                                              const float* __restrict__ pe,
                                                              uint16_t* __restrict__ out, int n_txt, int n_img,
                                                              int batch, int H, float eps) {
    const int S = n_txt + n_img;
    const int b = blockIdx.x / S;
    const int s = blockIdx.x - b * S;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const bool is_txt = s < n_txt;
    const float* src = is_txt ? txt + (static_cast<int64_t>(b) * n_txt + s) * H * HD
                              : img + (static_cast<int64_t>(b) * n_img + s - n_txt) * H * HD;
    v4f p = {0.0f, 0.0f, 0.0f, 0.0f};
    float w0 = 0.0f, w1 = 0.0f;
    if constexpr (NORM_ROPE) {
        p = reinterpret_cast<const v4f*>(pe)[static_cast<int64_t>(s) * (HD / 2) + lane];
        const uint32_t wp = reinterpret_cast<const uint32_t*>(is_txt ? w_txt : w_img)[lane];
        w0 = bf16_to_f32(static_cast<uint16_t>(wp & 0xffffu));
        w1 = bf16_to_f32(static_cast<uint16_t>(wp >> 16));
    }
    for (int h0 = wave; h0 < H; h0 += 4 * JH_BATCH) {
        float2 x[JH_BATCH];
#pragma unroll
        for (int k = 0; k < JH_BATCH; ++k) {
            const int h = h0 + 4 * k;
            x[k] = h < H ? reinterpret_cast<const float2*>(src + h * HD)[lane] : make_float2(0.0f, 0.0f);
        }
#pragma unroll
        for (int k = 0; k < JH_BATCH; ++k) {
            const int h = h0 + 4 * k;
            if (h >= H) break;  // wave-uniform
            float2 y = x[k];
            if constexpr (NORM_ROPE) {
                // (explicit fused multiply-adds: the fused Q quantization in
                // sage_attention.hip repeats this arithmetic bit for bit)
                const float ss = wave_sum_dpp(__builtin_fmaf(y.x, y.x, y.y * y.y));
                const float rms = rsqrtf(ss / HD + eps);
                y.x = y.x * rms * w0;
                y.y = y.y * rms * w1;
                const float o0 = __builtin_fmaf(y.x, p.x, y.y * p.y);
                const float o1 = __builtin_fmaf(y.x, p.z, y.y * p.w);
                y = make_float2(o0, o1);
            }
            const uint32_t packed =
                static_cast<uint32_t>(f32_to_f16(y.x)) | (static_cast<uint32_t>(f32_to_f16(y.y)) << 16);
            reinterpret_cast<uint32_t*>(out + ((static_cast<int64_t>(b) * H + h) * S + s) * HD)[lane] = packed;
        }
    }
}

// transpose_split_fused_fp32 (transformer.cu:84-104) on the fp16
// attention output [batch][H][S][128]: token s < n_txt of sequence b goes
// to txt[b][s][h*128..], the rest to img[b][s - n_txt][h*128..], as fp32.
__global__ __launch_bounds__(256) void split_heads_kernel(const uint16_t* __restrict__ in, float* __restrict__ txt,
                                                          float* __restrict__ img, int n_txt, int n_img, int batch,
                                                          int H) {
    const int S = n_txt + n_img;
    const int64_t gw = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
    if (gw >= static_cast<int64_t>(batch) * S * H) return;
    const int lane = threadIdx.x & 63;
    const int b = static_cast<int>(gw / (static_cast<int64_t>(S) * H));
    const int sh = static_cast<int>(gw - static_cast<int64_t>(b) * S * H);
    const int s = sh / H;
    const int h = sh - s * H;
    const uint32_t v =
        reinterpret_cast<const uint32_t*>(in + ((static_cast<int64_t>(b) * H + h) * S + s) * HD)[lane];
    const float2 f = make_float2(f16_to_f32(static_cast<uint16_t>(v & 0xffffu)), f16_to_f32(static_cast<uint16_t>(v >> 16)));
    float* dst = s < n_txt ? txt + ((static_cast<int64_t>(b) * n_txt + s) * H + h) * HD
                           : img + ((static_cast<int64_t>(b) * n_img + s - n_txt) * H + h) * HD;
    reinterpret_cast<float2*>(dst)[lane] = f;
}

// gate_add_fp32f_kernel (cuda_kernels.cu:2181-2189): out = x + gate[c] * y
// as one fused multiply-add per element, the operation the large-tile GEMM
// epilogue applies when it takes the gate itself (out may alias x).
__global__ __launch_bounds__(256) void gate_add_kernel(const float* x, const float* __restrict__ gate,
                                                       const float* __restrict__ y, float* out, int64_t n4,
                                                       int dim4) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n4) return;
    const int c = static_cast<int>(i % dim4);
    const v4f g = reinterpret_cast<const v4f*>(gate)[c];
    const v4f a = reinterpret_cast<const v4f*>(x)[i];
    const v4f b = reinterpret_cast<const v4f*>(y)[i];
    reinterpret_cast<v4f*>(out)[i] = (v4f){__builtin_fmaf(g.x, b.x, a.x), __builtin_fmaf(g.y, b.y, a.y),
                                           __builtin_fmaf(g.z, b.z, a.z), __builtin_fmaf(g.w, b.w, a.w)};
}

inline int div_up_i(int64_t a, int64_t b) { return static_cast<int>((a + b - 1) / b); }

}  // namespace

hipError_t launch_silu(const float* x, float* out, int64_t n, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(silu_kernel, dim3(div_up_i(n, 256)), dim3(256), 0, stream, x, out, n);
    return hipGetLastError();
}

hipError_t launch_layernorm_modulate(const float* x, const float* shift, const float* scale, float* out, int rows,
                                     int dim, float eps, hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    if ((dim & 3) != 0 || dim > LN_MAX_DIM) return hipErrorInvalidValue;
    hipLaunchKernelGGL(layernorm_modulate_kernel, dim3(rows), dim3(LN_THR), 0, stream, x, shift, scale, out, dim, eps);
    return hipGetLastError();
}

hipError_t launch_joint_heads_f16(const float* txt, const float* img, const uint16_t* w_txt, const uint16_t* w_img,
                                  const float* pe, uint16_t* out, int n_txt, int n_img, int batch, int H, float eps,
                                  hipStream_t stream) {
    const int64_t tokens = static_cast<int64_t>(n_txt + n_img) * batch;
    if (tokens == 0 || H == 0) return hipSuccess;
    const int blocks = static_cast<int>(tokens);
    if (w_txt != nullptr)
        hipLaunchKernelGGL(joint_heads_f16_kernel<true>, dim3(blocks), dim3(256), 0, stream, txt, img, w_txt, w_img,
                           pe, out, n_txt, n_img, batch, H, eps);
    else
        hipLaunchKernelGGL(joint_heads_f16_kernel<false>, dim3(blocks), dim3(256), 0, stream, txt, img, w_txt, w_img,
                           pe, out, n_txt, n_img, batch, H, eps);
    return hipGetLastError();
}

hipError_t launch_split_heads(const uint16_t* in, float* txt, float* img, int n_txt, int n_img, int batch, int H,
                              hipStream_t stream) {
    const int64_t waves = static_cast<int64_t>(n_txt + n_img) * H * batch;
    if (waves == 0) return hipSuccess;
    hipLaunchKernelGGL(split_heads_kernel, dim3(div_up_i(waves, 4)), dim3(256), 0, stream, in, txt, img, n_txt, n_img,
                       batch, H);
    return hipGetLastError();
}

hipError_t launch_gate_add(const float* x, const float* gate, const float* y, float* out, int rows, int dim,
                           hipStream_t stream) {
    if ((dim & 3) != 0) return hipErrorInvalidValue;
    const int64_t n4 = static_cast<int64_t>(rows) * (dim / 4);
    if (n4 == 0) return hipSuccess;
    hipLaunchKernelGGL(gate_add_kernel, dim3(div_up_i(n4, 256)), dim3(256), 0, stream, x, gate, y, out, n4, dim / 4);
    return hipGetLastError();
}

}  // namespace qimg
