// gemm_w8a8.hip — quantized linear layer for gfx950:
//   out[m,n] = act_scale[m] * w_scale[n] * sum_k a[m,k] w[n,k] + bias[n]
//              (optionally GELU-tanh), fp32 or bf16 out.
//
// Replaces the reference's three-kernel chain (cublasGemmEx s8s8s32 into a
// scratch int32 [M,N], then dequantize_and_bias / dequantize_bias_gelu;
// cuda_kernels.cu:2709-2731, 2623-2668) with one kernel: the int32 (or fp32
// for e4m3) accumulator never leaves registers, and the dequant epilogue is
// applied as it is stored.
//
// Tiling (CDNA4, wave64): a 256-thread workgroup owns a 256x256 output tile,
// four waves in a 2x2 arrangement each own 128x128 = 4x4 MFMA 32x32 blocks
// (v_mfma_i32_32x32x32_i8 for int8, v_mfma_scale_f32_32x32x64_f8f6f4 with
// unit scales for e4m3). Both operands are K-major [rows, K] as the
// reference stores them (TN GEMM). K advances 64 bytes per stage through a
// double-buffered LDS ring (2 x 32 KB); the next stage's global loads are
// issued before the current stage's MFMAs so HBM/L2 latency hides behind
// matrix work. LDS rows are 64 bytes with the 16-byte chunk index XOR-
// swizzled by ((row>>1) ^ (row>>3)) & 3, so MFMA fragment reads of 8 or 16
// consecutive rows touch distinct banks.
//
// The k ordering inside a 64-byte stage is the same for both operands, so
// the dot product is exact for int8 regardless of how the instruction
// consumes bytes within a lane.
#include "qimg_device.h"
#include "qimg_internal.h"

namespace qimg {

namespace {

constexpr int BM = 256;
constexpr int BN = 256;
constexpr int BK = 64;  // bytes of K per stage
constexpr int NTHR = 256;
constexpr int WTM = 128;  // wave tile
constexpr int WTN = 128;
constexpr int TM = WTM / 32;  // 32x32 blocks per wave
constexpr int TN = WTN / 32;
constexpr int STAGE_BYTES = (BM + BN) * BK;

__device__ __forceinline__ int swz(int row, int chunk) {
    return row * BK + ((chunk ^ (((row >> 1) ^ (row >> 3)) & 3)) << 4);
}

// Map the hardware workgroup id so that each XCD (workgroups are dispatched
// round-robin over 8 XCDs) receives a contiguous range of logical tiles,
// which keeps the tiles that share operand rows in one L2.
__device__ __forceinline__ int xcd_remap(int bid, int nwg) {
    const int xcd = bid & 7;
    const int local = bid >> 3;
    const int per = nwg >> 3;
    const int extra = nwg & 7;
    return (xcd < extra) ? xcd * (per + 1) + local : extra * (per + 1) + (xcd - extra) * per + local;
}

template <bool FP8>
struct Acc;
template <>
struct Acc<false> {
    typedef v16i type;
};
template <>
struct Acc<true> {
    typedef v16f type;
};

template <bool FP8, int OUT_DT, bool GELU>
__global__ __launch_bounds__(NTHR, 1) void gemm_w8a8_kernel(
    const uint8_t* __restrict__ A, const uint8_t* __restrict__ W, const float* __restrict__ as,
    const float* __restrict__ ws, const uint16_t* __restrict__ bias, void* __restrict__ out, int M,
    int N, int K) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * STAGE_BYTES];

    const int tiles_m = (M + BM - 1) / BM;
    const int tiles_n = (N + BN - 1) / BN;
    const int logical = xcd_remap(blockIdx.x, tiles_m * tiles_n);
    // Column-major over tiles: consecutive logical tiles share the weight
    // slice and walk down the activation rows.
    const int tm_idx = logical % tiles_m;
    const int tn_idx = logical / tiles_m;
    const int m0 = tm_idx * BM;
    const int n0 = tn_idx * BN;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1;
    const int wn = wave & 1;

    // Global->LDS copy assignment: thread t moves rows t/4 + 64 i, chunk t%4.
    const int ld_row = tid >> 2;
    const int ld_chunk = tid & 3;
    const uint8_t* a_src[4];
    const uint8_t* w_src[4];
    int lds_off[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = ld_row + 64 * i;
        int gm = m0 + r;
        gm = gm < M ? gm : M - 1;  // clamp: rows past M are computed, never stored
        int gn = n0 + r;
        gn = gn < N ? gn : N - 1;
        a_src[i] = A + static_cast<int64_t>(gm) * K + ld_chunk * 16;
        w_src[i] = W + static_cast<int64_t>(gn) * K + ld_chunk * 16;
        lds_off[i] = swz(r, ld_chunk);
    }

    typedef typename Acc<FP8>::type acc_t;
    acc_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

    v4i ga[4], gw[4];
    const int KT = K / BK;

    // prologue: stage 0
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        ga[i] = *reinterpret_cast<const v4i*>(a_src[i]);
        gw[i] = *reinterpret_cast<const v4i*>(w_src[i]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        *reinterpret_cast<v4i*>(lds + lds_off[i]) = ga[i];
        *reinterpret_cast<v4i*>(lds + BM * BK + lds_off[i]) = gw[i];
    }
    __syncthreads();

    const int frag_row = lane & 31;
    const int half = lane >> 5;

    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        const bool more = (kt + 1) < KT;
        if (more) {
            const int koff = (kt + 1) * BK;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                ga[i] = *reinterpret_cast<const v4i*>(a_src[i] + koff);
                gw[i] = *reinterpret_cast<const v4i*>(w_src[i] + koff);
            }
        }
        const uint8_t* la = lds + cur * STAGE_BYTES;
        const uint8_t* lw = la + BM * BK;
        if constexpr (!FP8) {
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const int chunk = 2 * ks + half;
                v4i fa[TM], fw[TN];
#pragma unroll
                for (int i = 0; i < TM; ++i)
                    fa[i] = *reinterpret_cast<const v4i*>(la + swz(wm * WTM + i * 32 + frag_row, chunk));
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    fw[j] = *reinterpret_cast<const v4i*>(lw + swz(wn * WTN + j * 32 + frag_row, chunk));
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fw[j], fa[i], acc[i][j], 0, 0, 0);
            }
        } else {
            v8i fa[TM], fw[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int r = wm * WTM + i * 32 + frag_row;
                v4i lo4 = *reinterpret_cast<const v4i*>(la + swz(r, 2 * half));
                v4i hi4 = *reinterpret_cast<const v4i*>(la + swz(r, 2 * half + 1));
                fa[i] = (v8i){lo4.x, lo4.y, lo4.z, lo4.w, hi4.x, hi4.y, hi4.z, hi4.w};
            }
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int r = wn * WTN + j * 32 + frag_row;
                v4i lo4 = *reinterpret_cast<const v4i*>(lw + swz(r, 2 * half));
                v4i hi4 = *reinterpret_cast<const v4i*>(lw + swz(r, 2 * half + 1));
                fw[j] = (v8i){lo4.x, lo4.y, lo4.z, lo4.w, hi4.x, hi4.y, hi4.z, hi4.w};
            }
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                        fw[j], fa[i], acc[i][j], 0, 0, 0, 127, 0, 127);
        }
        if (more) {
            uint8_t* nxt = lds + (cur ^ 1) * STAGE_BYTES;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                *reinterpret_cast<v4i*>(nxt + lds_off[i]) = ga[i];
                *reinterpret_cast<v4i*>(nxt + BM * BK + lds_off[i]) = gw[i];
            }
        }
        __syncthreads();
    }

    // Epilogue. The MFMA was issued as D = W_frag x A_frag, so the 32x32
    // block is indexed [n][m]: lane holds m = lane%32 and n rows
    // 8*(r/4) + 4*(lane/32) + r%4. Each lane therefore owns one output row
    // per block and 16 columns in four runs of 4 consecutive n, stored as
    // one 16-byte (fp32) or 8-byte (bf16) write per run.
    const bool has_bias = bias != nullptr;
    const bool vec_ok = (N & 3) == 0;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int nj = n0 + wn * WTN + j * 32 + 4 * half;
        float wsv[16], bv[16];
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                int n = nj + 8 * g + c;
                n = n < N ? n : N - 1;
                wsv[4 * g + c] = ws[n];
                bv[4 * g + c] = has_bias ? bf16_to_f32(bias[n]) : 0.0f;
            }
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int m = m0 + wm * WTM + i * 32 + (lane & 31);
            if (m >= M) continue;
            const float sa = as[m];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int nb = nj + 8 * g;
                float v[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    float t;
                    {
#pragma clang fp contract(off)
                        t = static_cast<float>(acc[i][j][4 * g + c]) * sa * wsv[4 * g + c];
                        if (has_bias) t = t + bv[4 * g + c];
                    }
                    if (GELU) t = gelu_tanh(t);
                    v[c] = t;
                }
                if (OUT_DT == QIMG_FP32) {
                    float* o = reinterpret_cast<float*>(out) + static_cast<int64_t>(m) * N + nb;
                    if (vec_ok && nb + 3 < N) {
                        *reinterpret_cast<v4f*>(o) = (v4f){v[0], v[1], v[2], v[3]};
                    } else {
#pragma unroll
                        for (int c = 0; c < 4; ++c)
                            if (nb + c < N) o[c] = v[c];
                    }
                } else {
                    uint16_t* o = reinterpret_cast<uint16_t*>(out) + static_cast<int64_t>(m) * N + nb;
                    if (vec_ok && nb + 3 < N) {
                        uint32_t lo = f32_to_bf16(v[0]) | (static_cast<uint32_t>(f32_to_bf16(v[1])) << 16);
                        uint32_t hi = f32_to_bf16(v[2]) | (static_cast<uint32_t>(f32_to_bf16(v[3])) << 16);
                        *reinterpret_cast<uint2*>(o) = make_uint2(lo, hi);
                    } else {
#pragma unroll
                        for (int c = 0; c < 4; ++c)
                            if (nb + c < N) o[c] = f32_to_bf16(v[c]);
                    }
                }
            }
        }
    }
}

// Fallback for int8 shapes the tiled kernel does not take (K not a
// multiple of 64): one thread per output element, same epilogue order.
__global__ void gemm_i8_simple_kernel(const int8_t* __restrict__ A, const int8_t* __restrict__ W,
                                      const float* __restrict__ as, const float* __restrict__ ws,
                                      const uint16_t* __restrict__ bias, void* __restrict__ out,
                                      int M, int N, int K, int out_dt, int gelu) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= static_cast<int64_t>(M) * N) return;
    const int m = static_cast<int>(idx / N);
    const int n = static_cast<int>(idx % N);
    const int8_t* a = A + static_cast<int64_t>(m) * K;
    const int8_t* w = W + static_cast<int64_t>(n) * K;
    int32_t s = 0;
    for (int k = 0; k < K; ++k) s += static_cast<int32_t>(a[k]) * static_cast<int32_t>(w[k]);
    float t;
    {
#pragma clang fp contract(off)
        t = static_cast<float>(s) * as[m] * ws[n];
        if (bias) t = t + bf16_to_f32(bias[n]);
    }
    if (gelu) t = gelu_tanh(t);
    if (out_dt == QIMG_FP32)
        reinterpret_cast<float*>(out)[idx] = t;
    else
        reinterpret_cast<uint16_t*>(out)[idx] = f32_to_bf16(t);
}

template <bool FP8, int OUT_DT, bool GELU>
hipError_t launch_tiled(const void* a, const float* as, int M, int K, const void* w,
                        const float* ws, int N, const uint16_t* bias, void* out,
                        hipStream_t stream) {
    const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    hipLaunchKernelGGL((gemm_w8a8_kernel<FP8, OUT_DT, GELU>), dim3(tiles), dim3(NTHR), 0, stream,
                       static_cast<const uint8_t*>(a), static_cast<const uint8_t*>(w), as, ws, bias,
                       out, M, N, K);
    return hipGetLastError();
}

template <bool FP8>
hipError_t dispatch_tiled(const void* a, const float* as, int M, int K, const void* w,
                          const float* ws, int N, const uint16_t* bias, void* out, int out_dt,
                          int gelu, hipStream_t stream) {
    if (out_dt == QIMG_FP32)
        return gelu ? launch_tiled<FP8, QIMG_FP32, true>(a, as, M, K, w, ws, N, bias, out, stream)
                    : launch_tiled<FP8, QIMG_FP32, false>(a, as, M, K, w, ws, N, bias, out, stream);
    return gelu ? launch_tiled<FP8, QIMG_BF16, true>(a, as, M, K, w, ws, N, bias, out, stream)
                : launch_tiled<FP8, QIMG_BF16, false>(a, as, M, K, w, ws, N, bias, out, stream);
}

}  // namespace

hipError_t launch_linear_prequantized(const void* act_q, const float* act_scales, int M, int K,
                                      const void* w_q, const float* w_scales, int N, int mode,
                                      const uint16_t* bias, void* out, int out_dtype, int gelu,
                                      hipStream_t stream) {
    if (M == 0 || N == 0) return hipSuccess;
    const bool fp8 = (mode == QIMG_QM_FP8_HADAMARD);
    if ((K % BK) == 0) {
        return fp8 ? dispatch_tiled<true>(act_q, act_scales, M, K, w_q, w_scales, N, bias, out,
                                          out_dtype, gelu, stream)
                   : dispatch_tiled<false>(act_q, act_scales, M, K, w_q, w_scales, N, bias, out,
                                           out_dtype, gelu, stream);
    }
    const int64_t total = static_cast<int64_t>(M) * N;
    const int blocks = static_cast<int>((total + 255) / 256);
    if (fp8) return hipErrorInvalidValue;  // e4m3 needs K % 64 == 0 (checked by the caller)
    hipLaunchKernelGGL(gemm_i8_simple_kernel, dim3(blocks), dim3(256), 0, stream,
                       static_cast<const int8_t*>(act_q), static_cast<const int8_t*>(w_q),
                       act_scales, w_scales, bias, out, M, N, K, out_dtype, gelu);
    return hipGetLastError();
}

}  // namespace qimg
