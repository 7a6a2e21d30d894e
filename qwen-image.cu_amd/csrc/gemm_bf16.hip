// gemm_bf16.hip — the BF16-mode linear layer for gfx950 (the layers a
// quantized checkpoint keeps unquantized: img_in, txt_in, norm_out and
// proj_out, transformer.cu:396-419, 874-895):
//   out[m,n] = sum_k bf16(x[m,k]) * w[n,k] + bias[n]   (then GELU-tanh)
// with x fp32 (rounded to bf16, round to nearest even, as the reference's
// fp32_to_bf16 pass) or bf16, w bf16 [N, K], fp32 accumulation and an fp32
// output. Replaces linear_forward_bf16 / linear_forward_bf16_bf16in
// (cuda_kernels.cu:4534-4596: fp32_to_bf16, cublasGemmEx bf16 x bf16 -> fp32,
// bias_add_fp32, gelu_fp32) with one kernel: the fp32 -> bf16 rounding
// happens on the operand registers and the bias / GELU on the accumulators.
// With `accumulate`, the product is added to the fp32 values already in out
// before the bias (the INT4 linear's residual GEMM onto its low-rank term,
// cublasGemmEx with beta = 1, cuda_kernels.cu:4488-4497).
//
// Shapes (M = tokens): img_in 3072 x 64, txt_in 3072 x 3584, norm_out
// 6144 x 3072 at M = 1 (or 2), proj_out 64 x 3072. They are bound by reading
// the weights (norm_out, txt_in) or the activations (proj_out) or by writing
// the output (img_in), so the kernel is built like the small-M quantized
// linear: a workgroup owns a 32x32 or 64x64 output tile, its four waves
// split K in 32-element blocks dealt round-robin (every operand byte is
// read by one wave), and the partial tiles are summed through LDS in wave
// order. Operands go straight from global memory into MFMA fragment
// registers with buffer loads (rows past M or N and blocks past K read as
// zero), DEPTH blocks in flight per wave. v_mfma_f32_32x32x16_bf16: lane
// (row r = lane%32, half h = lane/32) of a 32-row block holds, for k-step s
// of K block kb, the 8 elements kb*32 + 16h + 8s .. +7; both operands use
// the same assignment, so each dot product covers every k once.
#include <utility>

#include "qimg_device.h"
#include "qimg_internal.h"

namespace qimg {

namespace {

constexpr int BF_THR = 256;  // four waves, one K quarter each
constexpr int BF_KB = 32;    // elements of K per block
constexpr int kRsrcWord3 = 0x00020000;  // raw unswizzled buffer (gfx9 family)
constexpr uint32_t kOob = 0x80000000u;  // offset >= num_records: reads zero

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

template <int TMW, int TNW>
struct BfEpi {
    float b[TMW * TNW][4];
};

// 16 fp32 -> 8 + 8 bf16 (round to nearest even, the reference's
// __float2bfloat16) as two MFMA fragments.
__device__ __forceinline__ void f32x16_to_frags(const v4f (&x)[4], v8bf& lo, v8bf& hi) {
    uint32_t p[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        p[2 * i] = pack_bf16x2(x[i][0], x[i][1]);
        p[2 * i + 1] = pack_bf16x2(x[i][2], x[i][3]);
    }
    lo = __builtin_bit_cast(v8bf, (v4i){static_cast<int>(p[0]), static_cast<int>(p[1]), static_cast<int>(p[2]),
                                        static_cast<int>(p[3])});
    hi = __builtin_bit_cast(v8bf, (v4i){static_cast<int>(p[4]), static_cast<int>(p[5]), static_cast<int>(p[6]),
                                        static_cast<int>(p[7])});
}

template <bool XF32, int TMW, int TNW, int DEPTH, bool GELU>
__global__ __launch_bounds__(BF_THR) void gemm_bf16_kernel(const void* __restrict__ X,
                                                           const uint16_t* __restrict__ Wt,
                                                           const uint16_t* __restrict__ bias,
                                                           float* out, int M, int N, int K, int accumulate) {
    constexpr int MB = 32 * TMW;
    constexpr int NB = 32 * TNW;
    constexpr int NBLK = TMW * TNW;
    constexpr int NW = BF_THR / 64;
    constexpr int XE = XF32 ? 4 : 2;  // bytes per x element
    // partial tiles [wave][block][run g][lane], 16 bytes each
    __shared__ v4f red[NW * NBLK * 4 * 64];

    const int tiles_m = (M + MB - 1) / MB;
    const int tiles_n = (N + NB - 1) / NB;
    const int logical = xcd_remap(blockIdx.x, tiles_m * tiles_n);
    const int m0 = (logical % tiles_m) * MB;
    const int n0 = (logical / tiles_m) * NB;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 31;
    const int h = lane >> 5;

    // bias of the (row, 4-column run) groups this thread stores (the
    // mapping of the epilogue below), loaded now
    BfEpi<TMW, TNW> epi;
#pragma unroll
    for (int q = 0; q < NBLK; ++q) {
        const int idx = threadIdx.x + BF_THR * q;
        const int blk = idx >> 8;
        const int nb = n0 + 32 * (blk % TNW) + 8 * ((idx >> 6) & 3) + 4 * ((idx >> 5) & 1);
#pragma unroll
        for (int c = 0; c < 4; ++c)
            epi.b[q][c] = bias != nullptr ? bf16_to_f32(bias[nb + c < N ? nb + c : N - 1]) : 0.0f;
    }

    const int nkb = K / BF_KB;
    const int T = (nkb + NW - 1) / NW;
    const int Tp = ((T + DEPTH - 1) / DEPTH) * DEPTH;
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void*>(X), 0, static_cast<int>(static_cast<int64_t>(M) * K * XE), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(Wt), 0, static_cast<int>(static_cast<int64_t>(N) * K * 2), kRsrcWord3);
    uint32_t ox[TMW], ow[TNW];
#pragma unroll
    for (int i = 0; i < TMW; ++i) {
        const int gm = m0 + 32 * i + r;
        ox[i] = (static_cast<uint32_t>(gm) * K + 16 * h) * XE | (gm < M ? 0u : kOob);
    }
#pragma unroll
    for (int j = 0; j < TNW; ++j) {
        const int gn = n0 + 32 * j + r;
        ow[j] = (static_cast<uint32_t>(gn) * K + 16 * h) * 2 | (gn < N ? 0u : kOob);
    }

    v16f acc[TMW][TNW];
#pragma unroll
    for (int i = 0; i < TMW; ++i)
#pragma unroll
        for (int j = 0; j < TNW; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    // one K block's operands of this lane: x 16 elements per row block,
    // w 16 elements per column block
    v4f bx[DEPTH][TMW][XF32 ? 4 : 1];
    v4i bxh[DEPTH][TMW][2];
    v4i bw[DEPTH][TNW][2];
    auto load = [&](int d, int t) {
        const int kb = NW * t + wave;
        const uint32_t kbad = kb < nkb ? 0u : kOob;
#pragma unroll
        for (int i = 0; i < TMW; ++i) {
            const uint32_t o = (ox[i] + static_cast<uint32_t>(kb) * BF_KB * XE) | (ox[i] & kOob) | kbad;
            if constexpr (XF32) {
#pragma unroll
                for (int s = 0; s < 4; ++s)
                    bx[d][i][s] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(rx, o + 16 * s, 0, 0));
            } else {
#pragma unroll
                for (int s = 0; s < 2; ++s)
                    bxh[d][i][s] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rx, o + 16 * s, 0, 0));
            }
        }
#pragma unroll
        for (int j = 0; j < TNW; ++j) {
            const uint32_t o = (ow[j] + static_cast<uint32_t>(kb) * BF_KB * 2) | (ow[j] & kOob) | kbad;
#pragma unroll
            for (int s = 0; s < 2; ++s)
                bw[d][j][s] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rw, o + 16 * s, 0, 0));
        }
    };
    auto compute = [&](int d) {
        v8bf fx[TMW][2];
#pragma unroll
        for (int i = 0; i < TMW; ++i) {
            if constexpr (XF32) {
                f32x16_to_frags(bx[d][i], fx[i][0], fx[i][1]);
            } else {
                fx[i][0] = __builtin_bit_cast(v8bf, bxh[d][i][0]);
                fx[i][1] = __builtin_bit_cast(v8bf, bxh[d][i][1]);
            }
        }
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int i = 0; i < TMW; ++i)
#pragma unroll
                for (int j = 0; j < TNW; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, bw[d][j][s]),
                                                                        fx[i][s], acc[i][j], 0, 0, 0);
    };
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
        load(d, d);
        __builtin_amdgcn_sched_barrier(0);
    }
    for (int t0 = 0; t0 < Tp; t0 += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            compute(d);
            load(d, t0 + d + DEPTH);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // partial tiles -> LDS; the first wave's lanes own whole runs below
#pragma unroll
    for (int i = 0; i < TMW; ++i)
#pragma unroll
        for (int j = 0; j < TNW; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g)
                red[((wave * NBLK + i * TNW + j) * 4 + g) * 64 + lane] =
                    (v4f){acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
    __syncthreads();

    // Epilogue: thread idx owns (block, run g, lane) groups of 4 columns:
    // row m = 32 i + lane%32, columns 8 g + 4 (lane/32) + c (the MFMA D
    // layout, D = W x X^T indexed [n][m]). Partials are added in wave order,
    // then the bias (bias_add_fp32), then GELU (gelu_fp32).
    const bool vec_ok = (N & 3) == 0;
#pragma unroll
    for (int q = 0; q < NBLK; ++q) {
        const int idx = threadIdx.x + BF_THR * q;
        const int blk = idx >> 8;
        const int g = (idx >> 6) & 3;
        const int ln = idx & 63;
        const int i = blk / TNW;
        const int j = blk % TNW;
        const int m = m0 + 32 * i + (ln & 31);
        const int nb = n0 + 32 * j + 8 * g + 4 * (ln >> 5);
        if (m >= M || nb >= N) continue;
        v4f sum = red[(blk * 4 + g) * 64 + ln];
#pragma unroll
        for (int w = 1; w < NW; ++w) sum += red[((w * NBLK + blk) * 4 + g) * 64 + ln];
        float* o = out + static_cast<int64_t>(m) * N + nb;
        float prev[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (accumulate) {
            if (vec_ok) {
                const v4f p4 = *reinterpret_cast<const v4f*>(o);
                prev[0] = p4[0]; prev[1] = p4[1]; prev[2] = p4[2]; prev[3] = p4[3];
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    if (nb + c < N) prev[c] = o[c];
            }
        }
        float v[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            float t = sum[c];
            if (accumulate) t = t + prev[c];
            if (bias != nullptr) t = t + epi.b[q][c];
            if (GELU) t = gelu_tanh(t);
            v[c] = t;
        }
        if (vec_ok) {
            *reinterpret_cast<v4f*>(o) = (v4f){v[0], v[1], v[2], v[3]};
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c)
                if (nb + c < N) o[c] = v[c];
        }
    }
}

// Short K (img_in: K = 64): the four waves of a workgroup own the four
// 32x32 blocks of a 64x64 tile and each runs the whole of K, so no partial
// tiles are reduced and no LDS is used; the operand loads and the fragment
// layout are those of gemm_bf16_kernel, the products are summed in K-block
// order, and each lane stores its 16 outputs (row m = lane%32, columns
// 8g + 4(lane/32) + c) as four 16-byte runs.
template <bool XF32, bool GELU>
__global__ __launch_bounds__(BF_THR) void gemm_bf16_shortk_kernel(const void* __restrict__ X,
                                                                  const uint16_t* __restrict__ Wt,
                                                                  const uint16_t* __restrict__ bias,
                                                                  float* out, int M, int N, int K, int accumulate) {
    constexpr int XE = XF32 ? 4 : 2;
    const int tiles_m = (M + 63) / 64;
    const int tiles_n = (N + 63) / 64;
    const int logical = xcd_remap(blockIdx.x, tiles_m * tiles_n);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int m0 = (logical % tiles_m) * 64 + 32 * (wave >> 1);
    const int n0 = (logical / tiles_m) * 64 + 32 * (wave & 1);
    const int r = lane & 31;
    const int h = lane >> 5;
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void*>(X), 0, static_cast<int>(static_cast<int64_t>(M) * K * XE), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(Wt), 0, static_cast<int>(static_cast<int64_t>(N) * K * 2), kRsrcWord3);
    const uint32_t ox = (static_cast<uint32_t>(m0 + r) * K + 16 * h) * XE | (m0 + r < M ? 0u : kOob);
    const uint32_t ow = (static_cast<uint32_t>(n0 + r) * K + 16 * h) * 2 | (n0 + r < N ? 0u : kOob);
    float bv[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int n = n0 + 8 * (e >> 2) + 4 * h + (e & 3);
        bv[e] = bias != nullptr ? bf16_to_f32(bias[n < N ? n : N - 1]) : 0.0f;
    }
    v16f acc;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
    const int nkb = K / BF_KB;
    for (int kb = 0; kb < nkb; ++kb) {
        const uint32_t dx = static_cast<uint32_t>(kb) * BF_KB * XE;
        const uint32_t dw = static_cast<uint32_t>(kb) * BF_KB * 2;
        v8bf fx[2], fw[2];
        if constexpr (XF32) {
            v4f xv[4];
#pragma unroll
            for (int s = 0; s < 4; ++s)
                xv[s] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(rx, ((ox + dx) | (ox & kOob)) + 16 * s, 0, 0));
            f32x16_to_frags(xv, fx[0], fx[1]);
        } else {
#pragma unroll
            for (int s = 0; s < 2; ++s)
                fx[s] = __builtin_bit_cast(v8bf, __builtin_amdgcn_raw_buffer_load_b128(rx, ((ox + dx) | (ox & kOob)) + 16 * s, 0, 0));
        }
#pragma unroll
        for (int s = 0; s < 2; ++s)
            fw[s] = __builtin_bit_cast(v8bf, __builtin_amdgcn_raw_buffer_load_b128(rw, ((ow + dw) | (ow & kOob)) + 16 * s, 0, 0));
#pragma unroll
        for (int s = 0; s < 2; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fw[s], fx[s], acc, 0, 0, 0);
    }
    const int m = m0 + r;
    if (m >= M) return;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int nb = n0 + 8 * g + 4 * h;
        if (nb >= N) continue;
        float* o = out + static_cast<int64_t>(m) * N + nb;
        float prev[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (accumulate) {
#pragma unroll
            for (int c = 0; c < 4; ++c)
                if (nb + c < N) prev[c] = o[c];
        }
        float v[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            float t = acc[4 * g + c];
            if (accumulate) t = t + prev[c];
            if (bias != nullptr) t = t + bv[4 * g + c];
            if (GELU) t = gelu_tanh(t);
            v[c] = t;
        }
        if ((N & 3) == 0) {
            *reinterpret_cast<v4f*>(o) = (v4f){v[0], v[1], v[2], v[3]};
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c)
                if (nb + c < N) o[c] = v[c];
        }
    }
}

// Shapes the tiled kernel does not take (K not a multiple of 32, or byte
// sizes past the 32-bit buffer range): one thread per output, products
// summed in k order.
template <bool XF32>
__global__ __launch_bounds__(256) void gemm_bf16_simple_kernel(const void* __restrict__ X,
                                                               const uint16_t* __restrict__ Wt,
                                                               const uint16_t* __restrict__ bias,
                                                               float* out, int M, int N, int K, int gelu,
                                                               int accumulate) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= static_cast<int64_t>(M) * N) return;
    const int m = static_cast<int>(idx / N);
    const int n = static_cast<int>(idx % N);
    const uint16_t* w = Wt + static_cast<int64_t>(n) * K;
    float s = 0.0f;
    for (int k = 0; k < K; ++k) {
        float xv;
        if constexpr (XF32)
            xv = bf16_to_f32(f32_to_bf16(static_cast<const float*>(X)[static_cast<int64_t>(m) * K + k]));
        else
            xv = bf16_to_f32(static_cast<const uint16_t*>(X)[static_cast<int64_t>(m) * K + k]);
        s = __builtin_fmaf(xv, bf16_to_f32(w[k]), s);
    }
    if (accumulate) s = s + out[idx];
    if (bias != nullptr) s = s + bf16_to_f32(bias[n]);
    if (gelu) s = gelu_tanh(s);
    out[idx] = s;
}

template <bool XF32, int TMW, int TNW>
hipError_t launch_tiled_bf16(const void* x, int M, int K, const uint16_t* w, int N, const uint16_t* bias, float* out,
                             int gelu, int accumulate, hipStream_t stream) {
    constexpr int DEPTH = 4;
    const int tiles = ((M + 32 * TMW - 1) / (32 * TMW)) * ((N + 32 * TNW - 1) / (32 * TNW));
    if (gelu)
        hipLaunchKernelGGL((gemm_bf16_kernel<XF32, TMW, TNW, DEPTH, true>), dim3(tiles), dim3(BF_THR), 0, stream, x,
                           w, bias, out, M, N, K, accumulate);
    else
        hipLaunchKernelGGL((gemm_bf16_kernel<XF32, TMW, TNW, DEPTH, false>), dim3(tiles), dim3(BF_THR), 0, stream, x,
                           w, bias, out, M, N, K, accumulate);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_linear_bf16(const void* x, int x_dtype, int M, int K, const uint16_t* w, int N,
                              const uint16_t* bias, float* out, int gelu, hipStream_t stream, int accumulate) {
    if (M == 0 || N == 0) return hipSuccess;
    const bool xf32 = x_dtype == QIMG_FP32;
    const int64_t xbytes = static_cast<int64_t>(M) * K * (xf32 ? 4 : 2);
    const int64_t wbytes = static_cast<int64_t>(N) * K * 2;
    // Large problems with bf16 x (the INT4 linear's residual GEMM at 4096
    // tokens): the quantized linear's 256x256 tiles with bf16 MFMA.
    const int64_t tiles256 = static_cast<int64_t>((M + 255) / 256) * ((N + 255) / 256);
    if (!xf32 && (K % 64) == 0 && tiles256 >= 128)
        return launch_gemm_bf16_large(static_cast<const uint16_t*>(x), M, K, w, N, bias, out, gelu, accumulate,
                                      stream);
    const bool tiled = (K % BF_KB) == 0 && xbytes < (int64_t{1} << 31) && wbytes < (int64_t{1} << 31);
    if (!tiled) {
        const int64_t total = static_cast<int64_t>(M) * N;
        const int blocks = static_cast<int>((total + 255) / 256);
        if (xf32)
            hipLaunchKernelGGL(gemm_bf16_simple_kernel<true>, dim3(blocks), dim3(256), 0, stream, x, w, bias, out, M,
                               N, K, gelu, accumulate);
        else
            hipLaunchKernelGGL(gemm_bf16_simple_kernel<false>, dim3(blocks), dim3(256), 0, stream, x, w, bias, out, M,
                               N, K, gelu, accumulate);
        return hipGetLastError();
    }
    // 64x64 tiles when they give at least 256 workgroups, otherwise 32x32
    // (M <= 32: norm_out's 6144 columns; proj_out's 64 columns); K of at
    // most 256 (img_in) without the split of K over the waves
    const int64_t big = static_cast<int64_t>((M + 63) / 64) * ((N + 63) / 64);
    if (K <= 256 && big >= 256) {
        const int tiles = static_cast<int>(big);
#define QIMG_SHORTK(XF, GL)                                                                                    \
    hipLaunchKernelGGL((gemm_bf16_shortk_kernel<XF, GL>), dim3(tiles), dim3(BF_THR), 0, stream, x, w, bias, out, M, \
                       N, K, accumulate)
        if (xf32) {
            if (gelu)
                QIMG_SHORTK(true, true);
            else
                QIMG_SHORTK(true, false);
        } else {
            if (gelu)
                QIMG_SHORTK(false, true);
            else
                QIMG_SHORTK(false, false);
        }
#undef QIMG_SHORTK
        return hipGetLastError();
    }
    if (M > 32 && big >= 256)
        return xf32 ? launch_tiled_bf16<true, 2, 2>(x, M, K, w, N, bias, out, gelu, accumulate, stream)
                    : launch_tiled_bf16<false, 2, 2>(x, M, K, w, N, bias, out, gelu, accumulate, stream);
    return xf32 ? launch_tiled_bf16<true, 1, 1>(x, M, K, w, N, bias, out, gelu, accumulate, stream)
                : launch_tiled_bf16<false, 1, 1>(x, M, K, w, N, bias, out, gelu, accumulate, stream);
}

}  // namespace qimg
