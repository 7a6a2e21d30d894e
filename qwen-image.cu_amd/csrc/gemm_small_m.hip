// gemm_small_m.hip — quantized linear for problems with few output tiles:
//   out[m,n] = act_scale[m] * w_scale[n] * sum_k a[m,k] w[n,k] + bias[n]
//
// Small M is where the 256x256-tile kernel idles the chip: the modulation
// linears run at M = 1 (N = 18432, K = 3072, 56.6 MB of int8 weights per
// call, transformer.cu:506-515), the timestep MLP at M = 1
// (transformer.cu:329-349), the text-stream linears at M = 256 (12 tiles of
// 256x256 for N = 3072). These shapes are bound by reading the weights once
// from HBM (M = 1) or close to the ridge (M = 256), so the kernel here is
// built around streaming W:
//
//  - A workgroup owns a small output tile, 32x32 (M <= 32) or 64x64, and its
//    four waves split K four ways, so every operand byte the tile needs is
//    read by exactly one wave (the same L2 traffic as an LDS-shared tile)
//    and the chip gets N/32 (or M/64 * N/64) workgroups.
//  - Operands go straight from global memory into MFMA fragment registers:
//    lane (row r = lane%32, half h = lane/32) of a 32-row block reads the 32
//    contiguous bytes [64*kb + 32*h, +32) of its row for 64-byte K block kb.
//    No LDS staging and no barriers in the main loop; each wave keeps DEPTH
//    K blocks of loads in flight.
//  - int8: two v_mfma_i32_32x32x32_i8 per K block (16 bytes each); e4m3: one
//    v_mfma_scale_f32_32x32x64_f8f6f4 with unit scales (32 bytes). Both
//    operands use the same K assignment, so each dot product covers every k
//    once and the int8 result is exact.
//  - The four waves' partial tiles are summed through LDS (int32 sums are
//    exact; e4m3 partials are added in wave order), then the dequant epilogue
//    is applied as the tile is stored, with the arithmetic of the large-tile
//    kernel, so both give identical outputs.
//
// Rows past M and columns past N are clamped on load and never stored.
#include "qimg_device.h"
#include "qimg_internal.h"

namespace qimg {

namespace {

constexpr int SM_THR = 256;  // four waves, one K quarter each
constexpr int SM_KB = 64;    // bytes of K per block

template <bool FP8>
struct SmAcc;
template <>
struct SmAcc<false> {
    typedef v16i type;
};
template <>
struct SmAcc<true> {
    typedef v16f type;
};

template <bool FP8, int TMW, int TNW, int DEPTH, int OUT_DT, bool GELU>
__global__ __launch_bounds__(SM_THR) void gemm_small_m_kernel(
    const uint8_t* __restrict__ A, const uint8_t* __restrict__ W, const float* __restrict__ as,
    const float* __restrict__ ws, const uint16_t* __restrict__ bias, void* __restrict__ out, int M,
    int N, int K) {
    constexpr int MB = 32 * TMW;
    constexpr int NB = 32 * TNW;
    constexpr int NBLK = TMW * TNW;
    __shared__ v4i red[4 * NBLK * 4 * 64];

    const int tiles_m = (M + MB - 1) / MB;
    const int tiles_n = (N + NB - 1) / NB;
    // consecutive logical tiles share a weight slice (m fastest) and land on
    // one XCD
    const int logical = xcd_remap(blockIdx.x, tiles_m * tiles_n);
    const int m0 = (logical % tiles_m) * MB;
    const int n0 = (logical / tiles_m) * NB;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 31;
    const int h = lane >> 5;

    const int nkb = K / SM_KB;
    const int kb0 = (nkb * wave) >> 2;
    const int kb1 = (nkb * (wave + 1)) >> 2;

    const uint8_t* pa[TMW];
    const uint8_t* pw[TNW];
#pragma unroll
    for (int i = 0; i < TMW; ++i) {
        int gm = m0 + 32 * i + r;
        gm = gm < M ? gm : M - 1;
        pa[i] = A + static_cast<int64_t>(gm) * K + 32 * h;
    }
#pragma unroll
    for (int j = 0; j < TNW; ++j) {
        int gn = n0 + 32 * j + r;
        gn = gn < N ? gn : N - 1;
        pw[j] = W + static_cast<int64_t>(gn) * K + 32 * h;
    }

    typedef typename SmAcc<FP8>::type acc_t;
    acc_t acc[TMW][TNW];
#pragma unroll
    for (int i = 0; i < TMW; ++i)
#pragma unroll
        for (int j = 0; j < TNW; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;

    v4i ba[DEPTH][TMW][2];
    v4i bw[DEPTH][TNW][2];
    auto load = [&](int d, int kb) {
        const int off = kb * SM_KB;
#pragma unroll
        for (int i = 0; i < TMW; ++i)
#pragma unroll
            for (int s = 0; s < 2; ++s) ba[d][i][s] = *reinterpret_cast<const v4i*>(pa[i] + off + 16 * s);
#pragma unroll
        for (int j = 0; j < TNW; ++j)
#pragma unroll
            for (int s = 0; s < 2; ++s) bw[d][j][s] = *reinterpret_cast<const v4i*>(pw[j] + off + 16 * s);
    };
    auto compute = [&](int d) {
#pragma unroll
        for (int i = 0; i < TMW; ++i)
#pragma unroll
            for (int j = 0; j < TNW; ++j) {
                if constexpr (!FP8) {
#pragma unroll
                    for (int s = 0; s < 2; ++s)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bw[d][j][s], ba[d][i][s], acc[i][j],
                                                                           0, 0, 0);
                } else {
                    const v4i a0 = ba[d][i][0], a1 = ba[d][i][1];
                    const v4i w0 = bw[d][j][0], w1 = bw[d][j][1];
                    const v8i fa = (v8i){a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
                    const v8i fw = (v8i){w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fw, fa, acc[i][j], 0, 0, 0,
                                                                                127, 0, 127);
                }
            }
    };

    // Software pipeline over this wave's K blocks: block kb+d is consumed
    // from register set d, which is then refilled with block kb+d+DEPTH.
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
        if (kb0 + d < kb1) load(d, kb0 + d);
    for (int kb = kb0; kb < kb1; kb += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            if (kb + d < kb1) {
                compute(d);
                if (kb + d + DEPTH < kb1) load(d, kb + d + DEPTH);
            }
        }
    }

    // Partial tiles -> LDS as [wave][block][run g][lane] of 16 bytes: lane
    // holds 4 consecutive n per run (MFMA 32x32 layout, D = W x A, so lane
    // has m = lane%32 and n = 8g + 4h + c for accumulator element 4g + c).
#pragma unroll
    for (int i = 0; i < TMW; ++i)
#pragma unroll
        for (int j = 0; j < TNW; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                // (each element is copied to a scalar first: a bit cast of a
                // vector-element lvalue reads element 0)
                int b[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const auto e = acc[i][j][4 * g + c];
                    b[c] = __builtin_bit_cast(int, e);
                }
                red[((wave * NBLK + i * TNW + j) * 4 + g) * 64 + lane] = (v4i){b[0], b[1], b[2], b[3]};
            }
    __syncthreads();

    const bool has_bias = bias != nullptr;
    const bool vec_ok = (N & 3) == 0;
#pragma unroll
    for (int q = 0; q < NBLK; ++q) {
        const int idx = threadIdx.x + SM_THR * q;
        const int blk = idx >> 8;
        const int g = (idx >> 6) & 3;
        const int ln = idx & 63;
        const int i = blk / TNW;
        const int j = blk % TNW;
        const int m = m0 + 32 * i + (ln & 31);
        const int nb = n0 + 32 * j + 8 * g + 4 * (ln >> 5);
        if (m >= M || nb >= N) continue;
        float v[4];
        if constexpr (!FP8) {
            v4i s = red[(blk * 4 + g) * 64 + ln];
#pragma unroll
            for (int w = 1; w < 4; ++w) s += red[((w * NBLK + blk) * 4 + g) * 64 + ln];
#pragma unroll
            for (int c = 0; c < 4; ++c) v[c] = static_cast<float>(s[c]);
        } else {
            v4f s = __builtin_bit_cast(v4f, red[(blk * 4 + g) * 64 + ln]);
#pragma unroll
            for (int w = 1; w < 4; ++w) s += __builtin_bit_cast(v4f, red[((w * NBLK + blk) * 4 + g) * 64 + ln]);
#pragma unroll
            for (int c = 0; c < 4; ++c) v[c] = s[c];
        }
        const float sa = as[m];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int n = nb + c < N ? nb + c : N - 1;
            v[c] = dequant_elem<GELU>(v[c], sa, ws[n], has_bias, has_bias ? bf16_to_f32(bias[n]) : 0.0f);
        }
        if (OUT_DT == QIMG_FP32) {
            float* o = reinterpret_cast<float*>(out) + static_cast<int64_t>(m) * N + nb;
            if (vec_ok) {
                *reinterpret_cast<v4f*>(o) = (v4f){v[0], v[1], v[2], v[3]};
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    if (nb + c < N) o[c] = v[c];
            }
        } else {
            uint16_t* o = reinterpret_cast<uint16_t*>(out) + static_cast<int64_t>(m) * N + nb;
            if (vec_ok) {
                *reinterpret_cast<uint2*>(o) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    if (nb + c < N) o[c] = f32_to_bf16(v[c]);
            }
        }
    }
}

template <bool FP8, int TMW, int TNW, int DEPTH>
hipError_t launch_small(const void* a, const float* as, int M, int K, const void* w, const float* ws,
                        int N, const uint16_t* bias, void* out, int out_dt, int gelu, hipStream_t stream) {
    const int tiles = ((M + 32 * TMW - 1) / (32 * TMW)) * ((N + 32 * TNW - 1) / (32 * TNW));
    const uint8_t* A = static_cast<const uint8_t*>(a);
    const uint8_t* Wq = static_cast<const uint8_t*>(w);
#define QIMG_SMALL_LAUNCH(ODT, GL)                                                                      \
    hipLaunchKernelGGL((gemm_small_m_kernel<FP8, TMW, TNW, DEPTH, ODT, GL>), dim3(tiles), dim3(SM_THR), 0, \
                       stream, A, Wq, as, ws, bias, out, M, N, K)
    if (out_dt == QIMG_FP32) {
        if (gelu)
            QIMG_SMALL_LAUNCH(QIMG_FP32, true);
        else
            QIMG_SMALL_LAUNCH(QIMG_FP32, false);
    } else {
        if (gelu)
            QIMG_SMALL_LAUNCH(QIMG_BF16, true);
        else
            QIMG_SMALL_LAUNCH(QIMG_BF16, false);
    }
#undef QIMG_SMALL_LAUNCH
    return hipGetLastError();
}

}  // namespace

int small_m_variant(int M, int N, int K) {
    if (M <= 0 || N <= 0 || (K % SM_KB) != 0) return 0;
    if (M <= 32) return 1;
    const int64_t big_tiles = static_cast<int64_t>((M + 255) / 256) * ((N + 255) / 256);
    return big_tiles < 128 ? 2 : 0;
}

hipError_t launch_linear_small_m(const void* act_q, const float* act_scales, int M, int K, const void* w_q,
                                 const float* w_scales, int N, int mode, const uint16_t* bias, void* out,
                                 int out_dtype, int gelu, int variant, hipStream_t stream) {
    const bool fp8 = (mode == QIMG_QM_FP8_HADAMARD);
    if ((K % SM_KB) != 0 || M <= 0 || N <= 0) return hipErrorInvalidValue;
    if (variant == 1)
        return fp8 ? launch_small<true, 1, 1, 8>(act_q, act_scales, M, K, w_q, w_scales, N, bias, out, out_dtype,
                                                 gelu, stream)
                   : launch_small<false, 1, 1, 8>(act_q, act_scales, M, K, w_q, w_scales, N, bias, out,
                                                  out_dtype, gelu, stream);
    if (variant == 2)
        return fp8 ? launch_small<true, 2, 2, 4>(act_q, act_scales, M, K, w_q, w_scales, N, bias, out, out_dtype,
                                                 gelu, stream)
                   : launch_small<false, 2, 2, 4>(act_q, act_scales, M, K, w_q, w_scales, N, bias, out,
                                                  out_dtype, gelu, stream);
    return hipErrorInvalidValue;
}

}  // namespace qimg
