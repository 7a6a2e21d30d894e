// int4.hip — the INT4 weight paths of qwen-image.cu (cuda_kernels.cu:
// 2864-4532) for gfx950: INT4 dequantization (NF4 grid, offset-8 linear and
// two's complement nibbles), the INT4 weight and activation quantizers, the
// W4A4 GEMM, the AWQ GEMV with its repacking, and the nunchaku layout
// conversions. Packed nibbles hold the even column in the low nibble.
//
// W4A4 GEMM. gfx950 has no 4-bit integer MFMA, so INT4 x INT4 runs on
// v_mfma_i32_32x32x32_i8: a 32-bit word of eight nibbles becomes two words of
// int8 lanes with one AND each, (w << 4) & 0xF0F0F0F0 and w & 0xF0F0F0F0: each
// byte is 16 x the signed nibble (two's complement in the high half of the
// byte), so the MFMA returns 256 x the exact dot product, and an arithmetic
// shift by 8 recovers it. The element order inside a fragment is a
// permutation of k that is the same for both operands, so every dot product
// is the exact int32 sum of the reference's group. Each group's sum is then
// rescaled and accumulated in fp32 in the reference's operation order,
// acc = acc + ((float)d * as[g,m]) * ws[g,n] (w4a4_gemm_regdirect_kernel,
// cuda_kernels.cu:4206-4212), so the result is the same for every tiling.
#include "qimg_device.h"
#include "qimg_internal.h"

namespace qimg {

namespace {

__constant__ float kNf4Grid[16] = {-1.0f,   -0.6962f, -0.5251f, -0.3949f, -0.2844f, -0.1848f,
                                   -0.0911f, 0.0f,    0.0796f,  0.1609f,  0.2461f,  0.3379f,
                                   0.4407f,  0.5626f, 0.7230f,  1.0f};

__device__ __forceinline__ int nib_signed(int n) { return n >= 8 ? n - 16 : n; }

__device__ __forceinline__ float dequant_nibble(int n, float s, int nf4, int signed_int4) {
    if (nf4) return kNf4Grid[n] * s;
    if (signed_int4) return static_cast<float>(nib_signed(n)) * s;
    return static_cast<float>(n - 8) * s;
}

// dequantize_int4_to_bf16_kernel (cuda_kernels.cu:2876-2917): one thread per
// 4 packed bytes (8 columns, one 16-byte bf16 store). K % 8 == 0.
__global__ __launch_bounds__(256) void dequant_int4_bf16_kernel(const uint8_t* __restrict__ qw,
                                                                const float* __restrict__ scales,
                                                                uint16_t* __restrict__ out, int N, int K, int gs,
                                                                int nf4, int scales_gn, int signed_int4) {
    const int64_t words = static_cast<int64_t>(N) * (K / 8);
    const int G = K / gs;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < words;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int row = static_cast<int>(i / (K / 8));
        const int c0 = static_cast<int>(i % (K / 8)) * 8;
        const uint32_t w = reinterpret_cast<const uint32_t*>(qw)[i];
        u32x4 o;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            float v[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int c = c0 + 2 * p + e;
                const int g = c / gs;
                const float s = scales_gn ? scales[static_cast<int64_t>(g) * N + row]
                                          : scales[static_cast<int64_t>(row) * G + g];
                v[e] = dequant_nibble((w >> (8 * p + 4 * e)) & 0xF, s, nf4, signed_int4);
            }
            o[p] = static_cast<uint32_t>(f32_to_bf16(v[0])) | (static_cast<uint32_t>(f32_to_bf16(v[1])) << 16);
        }
        reinterpret_cast<u32x4*>(out)[i] = o;
    }
}

// INT4 weight quantizers, one wave per (row, group): the linear form
// (quantize_linear_int4_per_group_kernel, cuda_kernels.cu:3226-3288) and NF4
// (quantize_int4_per_group_kernel, :3290-3357).
template <bool NF4>
__global__ __launch_bounds__(256) void quant_int4_weight_kernel(const float* __restrict__ r,
                                                                uint8_t* __restrict__ qw,
                                                                float* __restrict__ scales, int N, int K, int gs) {
    const int G = K / gs;
    const int64_t task = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (task >= static_cast<int64_t>(N) * G) return;
    const int lane = threadIdx.x & 63;
    const int64_t row = task / G;
    const int g = static_cast<int>(task % G);
    const float* p = r + row * K + static_cast<int64_t>(g) * gs;
    float amax = 0.0f;
    for (int i = lane; i < gs; i += 64) amax = fmaxf(amax, fabsf(p[i]));
    amax = wave_max(amax);
    const float scale = NF4 ? amax : amax / 7.0f;
    if (lane == 0) scales[row * G + g] = scale;
    const float inv = NF4 ? (scale > 0.0f ? 1.0f / scale : 0.0f) : (amax > 0.0f ? 7.0f / amax : 0.0f);
    for (int i = lane; i < gs / 2; i += 64) {
        int q[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const float v = p[2 * i + e] * inv;
            if (NF4) {
                int best_j = 0;
                float best = 1e9f;
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const float d = fabsf(v - kNf4Grid[j]);
                    if (d < best) {
                        best = d;
                        best_j = j;
                    }
                }
                q[e] = best_j;
            } else {
                const int t = static_cast<int>(roundf(v));
                q[e] = (t < -7 ? -7 : (t > 7 ? 7 : t)) + 8;
            }
        }
        qw[row * (K / 2) + (static_cast<int64_t>(g) * gs) / 2 + i] = static_cast<uint8_t>(q[0] | (q[1] << 4));
    }
}

// Activation INT4 quant (quantize_activation_int4_kernel, cuda_kernels.cu:
// 3575-3636; with a smooth divide and a bf16 copy, fused_smooth_bf16_quant_
// kernel, :3650-3705). A thread owns one column pair; a group of gs columns
// is gs/2 consecutive lanes of one wave (gs = 32, 64 or 128), reduced with
// lane exchanges. scales [G, M].
template <int GS>
__global__ __launch_bounds__(256) void quant_act_int4_kernel(const float* __restrict__ x,
                                                             const float* __restrict__ smooth,
                                                             uint16_t* __restrict__ bf16_out,
                                                             uint8_t* __restrict__ packed,
                                                             float* __restrict__ scales, int M, int K) {
    constexpr int L = GS / 2;  // lanes per group
    const int64_t pairs = static_cast<int64_t>(M) * (K / 2);
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    // every lane takes part in the exchanges; lanes past the end hold zeros
    const bool live = t < pairs;
    const int64_t tt = live ? t : 0;
    const int64_t m = tt / (K / 2);
    const int c = static_cast<int>(tt % (K / 2)) * 2;
    float v0 = 0.0f, v1 = 0.0f;
    if (live) {
        const float2 xv = *reinterpret_cast<const float2*>(x + m * K + c);
        v0 = xv.x;
        v1 = xv.y;
        if (smooth != nullptr) {
            v0 = v0 / smooth[c];
            v1 = v1 / smooth[c + 1];
        }
        if (bf16_out != nullptr)
            *reinterpret_cast<uint32_t*>(bf16_out + m * K + c) =
                static_cast<uint32_t>(f32_to_bf16(v0)) | (static_cast<uint32_t>(f32_to_bf16(v1)) << 16);
    }
    float amax = fmaxf(fabsf(v0), fabsf(v1));
#pragma unroll
    for (int off = 1; off < L; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off, kWave));
    if (!live) return;
    const int g = c / GS;
    if ((c % GS) == 0) scales[static_cast<int64_t>(g) * M + m] = amax / 7.0f;
    const float inv = amax > 0.0f ? 7.0f / amax : 0.0f;
    int q0 = static_cast<int>(roundf(v0 * inv));
    int q1 = static_cast<int>(roundf(v1 * inv));
    q0 = q0 < -7 ? -7 : (q0 > 7 ? 7 : q0);
    q1 = q1 < -7 ? -7 : (q1 > 7 ? 7 : q1);
    packed[m * (K / 2) + c / 2] = static_cast<uint8_t>((q0 & 0xF) | ((q1 & 0xF) << 4));
}

// ---- W4A4 GEMM ---------------------------------------------------------
// A 512-thread workgroup owns a 128 x 128 output tile: eight waves in a 4 x 2
// arrangement, each a 32 x 64 wave tile (two 32 x 32 blocks), two waves per
// SIMD so that one wave's rescale (VALU work on every accumulator, each
// group) runs beside the other's MFMAs. Operand chunks are loaded two chunks
// ahead of their use, and the tile's scales of up to 64 groups at a time sit
// in LDS: loading them from global memory inside each rescale left the
// kernel waiting on their latency every group (290 -> 495 TOP/s at
// 4096 x 3072 x 3072, group 64, bit-identical). Capping the registers at
// 128 for four waves per SIMD spilled and ran at half the speed.
constexpr int W4_THR = 512;
constexpr int W4_BM = 128;
constexpr int W4_BN = 128;

// Eight packed bytes (16 nibbles) -> one i8 MFMA fragment of 16 bytes, each
// 16 x its signed nibble.
__device__ __forceinline__ v4i unpack16(uint2 p) {
    return (v4i){static_cast<int>((p.x << 4) & 0xF0F0F0F0u), static_cast<int>(p.x & 0xF0F0F0F0u),
                 static_cast<int>((p.y << 4) & 0xF0F0F0F0u), static_cast<int>(p.y & 0xF0F0F0F0u)};
}

// out[m,n] (+)= sum_g ((float)d_g * as[g,m]) * ws[g,n] + bias[n] (then GELU,
// gelu_fp32 after the reference's GEMM, cuda_kernels.cu:4529-4531). The MFMA
// is issued as D = W x A^T, so lane l holds m = l % 32 and n rows
// 8 (r/4) + 4 (l/32) + r%4 of each 32 x 32 block. gs % 64 == 0.
__global__ __launch_bounds__(W4_THR) void w4a4_gemm_kernel(const uint8_t* __restrict__ act,
                                                           const uint8_t* __restrict__ wgt,
                                                           const float* __restrict__ as,
                                                           const float* __restrict__ ws, float* out, int M, int N,
                                                           int K, int gs, int accumulate,
                                                           const uint16_t* __restrict__ bias, int gelu) {
    const int tiles_m = (M + W4_BM - 1) / W4_BM;
    const int tiles_n = (N + W4_BN - 1) / W4_BN;
    const int logical = xcd_remap(blockIdx.x, tiles_m * tiles_n);
    // M-tile fastest: consecutive workgroups share a weight slice
    const int m0 = (logical % tiles_m) * W4_BM;
    const int n0 = (logical / tiles_m) * W4_BN;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int h = lane >> 5;
    const int KB = K / 2;
    const int G = K / gs;

    const int m = m0 + wm * 32 + (lane & 31);
    const int mrow = m < M ? m : M - 1;  // rows past the end are computed, never stored
    // Lane half h takes packed bytes [16h, 16h + 16) of each 32-byte
    // (64-column) chunk of its row, one 16-byte load for two MFMA steps:
    // bytes 16h + 8s .. +8 feed step s (a k order that both operands share).
    const uint8_t* ap = act + static_cast<int64_t>(mrow) * KB + 16 * h;
    const uint8_t* wp[2];
    int ncol[2][4];  // the 16 output columns of block j held by this lane, as 4 runs of 4
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = n0 + wn * 64 + 32 * j + (lane & 31);
        wp[j] = wgt + static_cast<int64_t>(n < N ? n : N - 1) * KB + 16 * h;
#pragma unroll
        for (int q = 0; q < 4; ++q) ncol[j][q] = n0 + wn * 64 + 32 * j + 8 * q + 4 * h;
    }

    float acc[2][16];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;

    const int chunks = gs / 64;  // 64-column chunks (two MFMA steps) per group
    const int nch = K / 64;
    // Chunk loads run PF chunks ahead of their use (the loads of a chunk
    // are three 16-byte loads per lane straight from global memory).
    constexpr int PF = 2;
    uint4 ra[PF + 1], rw[PF + 1][2];
    auto load = [&](int c, int slot) {
        const int off = 32 * c;
        ra[slot] = *reinterpret_cast<const uint4*>(ap + off);
#pragma unroll
        for (int j = 0; j < 2; ++j) rw[slot][j] = *reinterpret_cast<const uint4*>(wp[j] + off);
    };
#pragma unroll
    for (int p = 0; p < PF; ++p)
        if (p < nch) load(p, p);
    v16i d[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) d[j][r] = 0;
    // The tile's activation and weight scales of up to SG groups at a time
    // in LDS (loaded together between two barriers at a group boundary), so
    // a group's rescale reads them without global latency.
    constexpr int SG = 64;
    __shared__ __attribute__((aligned(16))) float s_as[SG][W4_BM];
    __shared__ __attribute__((aligned(16))) float s_ws[SG][W4_BN];
    auto stage_scales = [&](int g0) {
        const int ng = G - g0 < SG ? G - g0 : SG;
        __syncthreads();  // every wave is done with the previous groups' scales
        for (int i = threadIdx.x; i < ng * W4_BM; i += W4_THR) {
            const int gi = i / W4_BM, r = i % W4_BM;
            const int mm = m0 + r < M ? m0 + r : M - 1;
            const int nn = n0 + r < N ? n0 + r : N - 1;
            s_as[gi][r] = as[static_cast<int64_t>(g0 + gi) * M + mm] * 0.00390625f;
            s_ws[gi][r] = ws[static_cast<int64_t>(g0 + gi) * N + nn];
        }
        __syncthreads();
    };
    const int mloc = wm * 32 + (lane & 31);
    int g = 0, cg = 0;
    stage_scales(0);
    for (int c0 = 0; c0 < nch; c0 += PF + 1) {
#pragma unroll
        for (int u = 0; u < PF + 1; ++u) {
            const int c = c0 + u;
            if (c >= nch) break;
            // slot of chunk c is u; chunk c + PF goes to slot (u + PF) % (PF + 1)
            if (c + PF < nch) load(c + PF, (u + PF) % (PF + 1));
            const uint4 pa = ra[u];
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const v4i fa = unpack16(s ? make_uint2(pa.z, pa.w) : make_uint2(pa.x, pa.y));
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const v4i fw = unpack16(s ? make_uint2(rw[u][j].z, rw[u][j].w) : make_uint2(rw[u][j].x, rw[u][j].y));
                    // a group's first step starts from zero (no reset of d)
                    const v16i zero = {};
                    d[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fw, fa, (s == 0 && cg == 0) ? zero : d[j], 0, 0, 0);
                }
            }
            if (++cg == chunks) {
                cg = 0;
                // (float)(d >> 8) * sa == (float)d * (sa * 2^-8): d = 256 x an
                // exact sum below 2^12 in magnitude, and the power-of-two
                // scaling is exact, so the product rounds identically.
                const int gi = g % SG;
                const float sa = s_as[gi][mloc];
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const v4f sw = *reinterpret_cast<const v4f*>(&s_ws[gi][ncol[j][q] - n0]);
#pragma unroll
                        for (int cc = 0; cc < 4; ++cc) {
#pragma clang fp contract(off)
                            const float t = static_cast<float>(d[j][4 * q + cc]) * sa;
                            acc[j][4 * q + cc] = acc[j][4 * q + cc] + t * sw[cc];
                        }
                    }
                ++g;
                if (g % SG == 0 && g < G) stage_scales(g);
            }
        }
    }

    if (m >= M) return;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int n = ncol[j][q] + c;
                if (n >= N) continue;
                const float b = bias != nullptr ? bf16_to_f32(bias[n]) : 0.0f;
                float* o = out + static_cast<int64_t>(m) * N + n;
                float v;
                {
#pragma clang fp contract(off)
                    v = acc[j][4 * q + c] + b;
                    if (accumulate) v = *o + v;
                }
                if (gelu) v = gelu_tanh(v);
                *o = v;
            }
}

// ---- AWQ ----------------------------------------------------------------
// AWQ kInterleave=4 nibble address (cuda_kernels.cu:3072-3085).
__device__ __forceinline__ int awq_nibble(const int32_t* qw, int IC, int oc, int ic) {
    const int i16 = ((ic >> 6) << 6) + (oc & 3) * 16 + (((ic & 63) >> 5) << 3) + (ic & 7);
    const int bit = ((i16 & 1) << 4) + (((ic >> 3) & 3) << 2);
    return static_cast<int>((static_cast<uint32_t>(qw[static_cast<int64_t>(oc >> 2) * (IC / 2) + (i16 >> 1)]) >> bit) &
                            0xF);
}

// repack_awq_kernel (cuda_kernels.cu:3059-3091): [OC/4, IC/2] -> [IC/8, OC].
__global__ __launch_bounds__(256) void awq_repack_kernel(const int32_t* __restrict__ qw, int32_t* __restrict__ out,
                                                         int OC, int IC) {
    const int oc = blockIdx.x * blockDim.x + threadIdx.x;
    const int ig = blockIdx.y;
    if (oc >= OC) return;
    uint32_t w = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) w |= static_cast<uint32_t>(awq_nibble(qw, IC, oc, ig * 8 + k)) << (4 * k);
    out[static_cast<int64_t>(ig) * OC + oc] = static_cast<int32_t>(w);
}

// dequantize_awq_to_bf16_kernel (cuda_kernels.cu:3002-3038).
__global__ __launch_bounds__(256) void awq_dequant_kernel(const int32_t* __restrict__ qw,
                                                          const uint16_t* __restrict__ wscales,
                                                          const uint16_t* __restrict__ wzeros,
                                                          uint16_t* __restrict__ out, int OC, int IC, int gs,
                                                          int ncomp) {
    const int64_t total = static_cast<int64_t>(OC) * IC;
    const int dim = OC / ncomp;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int so = static_cast<int>(i / IC);
        const int ic = static_cast<int>(i % IC);
        const int nk = (so % dim) * ncomp + so / dim;
        const int g = ic / gs;
        const float s = bf16_to_f32(wscales[static_cast<int64_t>(g) * OC + nk]);
        const float z = bf16_to_f32(wzeros[static_cast<int64_t>(g) * OC + nk]);
        float w;
        {
#pragma clang fp contract(off)
            w = static_cast<float>(awq_nibble(qw, IC, nk, ic)) * s + z;
        }
        out[i] = f32_to_bf16(w);
    }
}

// awq_gemv_repacked_kernel (cuda_kernels.cu:3106-3153), M = 1, gs = 64: one
// lane per interleaved output channel, the input row in LDS, the sum over
// ic in order (a dependent chain per lane). The next group's eight weight
// words and its scale and zero are loaded while the current group is
// summed, so the chain waits on the memory latency once, not per group;
// 64-lane workgroups spread the channels over the CUs.
__global__ __launch_bounds__(64) void awq_gemv_kernel(const float* __restrict__ x, const int32_t* __restrict__ qw,
                                                      const uint16_t* __restrict__ wscales,
                                                      const uint16_t* __restrict__ wzeros,
                                                      const uint16_t* __restrict__ bias, float* __restrict__ out,
                                                      int OC, int IC, int ncomp) {
    extern __shared__ float s_x[];
    for (int i = threadIdx.x; i < IC; i += blockDim.x) s_x[i] = x[i];
    __syncthreads();
    const int nk_raw = blockIdx.x * blockDim.x + threadIdx.x;
    const bool live = nk_raw < OC;
    const int nk = live ? nk_raw : OC - 1;
    const int G = IC / 64;
    auto load = [&](int g, uint32_t* p, uint16_t& s, uint16_t& z) {
#pragma unroll
        for (int io = 0; io < 8; ++io) p[io] = static_cast<uint32_t>(qw[static_cast<int64_t>(g * 8 + io) * OC + nk]);
        s = wscales[static_cast<int64_t>(g) * OC + nk];
        z = wzeros[static_cast<int64_t>(g) * OC + nk];
    };
    uint32_t p[8], pn[8];
    uint16_t s16, z16, sn16 = 0, zn16 = 0;
    load(0, p, s16, z16);
    float acc = 0.0f;
    for (int g = 0; g < G; ++g) {
        if (g + 1 < G) load(g + 1, pn, sn16, zn16);
        const float s = bf16_to_f32(s16);
        const float z = bf16_to_f32(z16);
        const v4f* xv = reinterpret_cast<const v4f*>(s_x + g * 64);
#pragma unroll
        for (int io = 0; io < 8; ++io) {
            const v4f x0 = xv[2 * io], x1 = xv[2 * io + 1];
            const float xs[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
#pragma unroll
            for (int k = 0; k < 8; ++k) {
#pragma clang fp contract(off)
                const float w = static_cast<float>((p[io] >> (4 * k)) & 0xF) * s + z;
                acc = acc + w * xs[k];
            }
        }
#pragma unroll
        for (int io = 0; io < 8; ++io) p[io] = pn[io];
        s16 = sn16;
        z16 = zn16;
    }
    if (!live) return;
    const int dim = OC / ncomp;
    const int so = (nk % ncomp) * dim + nk / ncomp;
    if (bias != nullptr) acc = acc + bf16_to_f32(bias[so]);
    out[so] = acc;
}

// ---- nunchaku layouts ----------------------------------------------------
// MMA-swizzled nibble and scale addresses (cuda_kernels.cu:2945-2973).
__device__ __forceinline__ int nk_nibble(const uint8_t* q, int K, int row, int col) {
    const int kt = K / 64, nt = row / 128, nw = row % 128;
    const int np = nw / 16, ps = (nw % 16) / 8, nl = nw % 8;
    const int ktile = col / 64, kps = (col % 64) / 32, kl = (col % 32) / 8, rk = col % 8;
    const int64_t i32 = static_cast<int64_t>(nt) * (kt * 1024) + ktile * 1024 + np * 128 + nl * 16 + kl * 4 + ps * 2 + kps;
    return (q[i32 * 4 + rk / 2] >> ((rk % 2) * 4)) & 0xF;
}

__device__ __forceinline__ int64_t nk_scale_off(int G, int row, int g) {
    const int nt = row / 128, nw = row % 128;
    return static_cast<int64_t>(nt) * G * 128 + g * 128 + (nw / 16) * 16 + ((nw % 8) / 2) * 4 + ((nw % 16) / 8) * 2 +
           nw % 2;
}

// unswizzle_nunchaku_weights_kernel (cuda_kernels.cu:3431-3487).
__global__ __launch_bounds__(256) void nk_unswizzle_kernel(const uint8_t* __restrict__ q_sw,
                                                           const uint16_t* __restrict__ s_sw,
                                                           uint8_t* __restrict__ q_rm, float* __restrict__ s_rm,
                                                           int N, int K, int G) {
    const int64_t total = static_cast<int64_t>(N) * (K / 2);
    const int gs = K / G;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int row = static_cast<int>(i / (K / 2));
        const int c0 = static_cast<int>(i % (K / 2)) * 2;
        q_rm[i] = static_cast<uint8_t>(nk_nibble(q_sw, K, row, c0) | (nk_nibble(q_sw, K, row, c0 + 1) << 4));
        if (c0 % gs == 0) s_rm[static_cast<int64_t>(c0 / gs) * N + row] = bf16_to_f32(s_sw[nk_scale_off(G, row, c0 / gs)]);
    }
}

// dequantize_nunchaku_to_bf16_kernel (cuda_kernels.cu:2932-2978).
__global__ __launch_bounds__(256) void nk_dequant_kernel(const uint8_t* __restrict__ q_sw,
                                                         const uint16_t* __restrict__ s_sw,
                                                         uint16_t* __restrict__ out, int N, int K, int G) {
    const int64_t total = static_cast<int64_t>(N) * K;
    const int gs = K / G;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int row = static_cast<int>(i / K);
        const int col = static_cast<int>(i % K);
        const float s = bf16_to_f32(s_sw[nk_scale_off(G, row, col / gs)]);
        out[i] = f32_to_bf16(static_cast<float>(nib_signed(nk_nibble(q_sw, K, row, col))) * s);
    }
}

// unswizzle_lora_weights_kernel (cuda_kernels.cu:3503-3562).
__global__ __launch_bounds__(256) void lora_unswizzle_kernel(const uint16_t* __restrict__ packed,
                                                             uint16_t* __restrict__ out, int rows, int cols,
                                                             int is_down) {
    const int64_t total = static_cast<int64_t>(rows) * cols;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int row = static_cast<int>(i / cols);
        const int col = static_cast<int>(i % cols);
        const int sr = is_down ? col : row, sc = is_down ? row : col;
        const int cf = is_down ? sc / 16 : sr / 16, rf = is_down ? sr / 16 : sc / 16;
        const int ln = sr % 16, lk = sc % 16;
        const int64_t f = static_cast<int64_t>(cf) * 16 * cols + rf * 256 + (ln % 8) * 32 + ((lk % 8) / 2) * 8 +
                          (ln / 8) * 4 + (lk / 8) * 2 + lk % 2;
        out[i] = packed[f];
    }
}

// bf16 transpose [R, C] -> [C, R] (the low-rank down projection is stored
// [K, r]; the GEMM takes its weight as [r, K]).
__global__ __launch_bounds__(256) void transpose_u16_kernel(const uint16_t* __restrict__ in,
                                                            uint16_t* __restrict__ out, int R, int C) {
    const int64_t total = static_cast<int64_t>(R) * C;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int c = static_cast<int>(i / R);
        const int r = static_cast<int>(i % R);
        out[i] = in[static_cast<int64_t>(r) * C + c];
    }
}

// fp32 -> bf16, round to nearest even (fp32_to_bf16, cuda_kernels.cu:33-42).
__global__ __launch_bounds__(256) void f32_to_bf16_kernel(const float* __restrict__ in, uint16_t* __restrict__ out,
                                                          int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x)
        out[i] = f32_to_bf16(in[i]);
}

// bf16 -> fp32 (bf16_to_fp32, cuda_kernels.cu:22-31): exact widening.
__global__ __launch_bounds__(256) void bf16_to_f32_kernel(const uint16_t* __restrict__ in, float* __restrict__ out,
                                                          int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x)
        out[i] = bf16_to_f32(in[i]);
}

int grid_for(int64_t n, int per_block = 256) {
    const int64_t b = (n + per_block - 1) / per_block;
    return static_cast<int>(b < 65536 ? (b > 0 ? b : 1) : 65536);
}

}  // namespace

hipError_t launch_dequant_int4_bf16(const uint8_t* qw, const float* scales, uint16_t* out, int N, int K, int gs,
                                    int nf4, int scales_gn, int signed_int4, hipStream_t stream) {
    if (N == 0 || K == 0) return hipSuccess;
    if (K % 8 != 0 || gs <= 0 || K % gs != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(dequant_int4_bf16_kernel, dim3(grid_for(static_cast<int64_t>(N) * (K / 8))), dim3(256), 0,
                       stream, qw, scales, out, N, K, gs, nf4, scales_gn, signed_int4);
    return hipGetLastError();
}

hipError_t launch_quant_int4_weight(const float* r, uint8_t* qw, float* scales, int N, int K, int gs, int nf4,
                                    hipStream_t stream) {
    if (N == 0 || K == 0) return hipSuccess;
    if (gs <= 0 || gs % 2 != 0 || K % gs != 0) return hipErrorInvalidValue;
    const int64_t tasks = static_cast<int64_t>(N) * (K / gs);
    const int blocks = static_cast<int>((tasks + 3) / 4);
    if (nf4)
        hipLaunchKernelGGL(quant_int4_weight_kernel<true>, dim3(blocks), dim3(256), 0, stream, r, qw, scales, N, K, gs);
    else
        hipLaunchKernelGGL(quant_int4_weight_kernel<false>, dim3(blocks), dim3(256), 0, stream, r, qw, scales, N, K,
                           gs);
    return hipGetLastError();
}

hipError_t launch_quant_act_int4(const float* x, const float* smooth, uint16_t* bf16_out, uint8_t* packed,
                                 float* scales, int M, int K, int gs, hipStream_t stream) {
    if (M == 0 || K == 0) return hipSuccess;
    if (K % gs != 0) return hipErrorInvalidValue;
    const int64_t pairs = static_cast<int64_t>(M) * (K / 2);
    const int64_t blocks64 = (pairs + 255) / 256;
    if (blocks64 > 0x7fffffff) return hipErrorInvalidValue;
    const int blocks = static_cast<int>(blocks64);
    switch (gs) {
        case 32:
            hipLaunchKernelGGL(quant_act_int4_kernel<32>, dim3(blocks), dim3(256), 0, stream, x, smooth, bf16_out,
                               packed, scales, M, K);
            break;
        case 64:
            hipLaunchKernelGGL(quant_act_int4_kernel<64>, dim3(blocks), dim3(256), 0, stream, x, smooth, bf16_out,
                               packed, scales, M, K);
            break;
        case 128:
            hipLaunchKernelGGL(quant_act_int4_kernel<128>, dim3(blocks), dim3(256), 0, stream, x, smooth, bf16_out,
                               packed, scales, M, K);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_w4a4_gemm(const uint8_t* act, const uint8_t* wgt, const float* as, const float* ws, float* out,
                            int M, int N, int K, int gs, int accumulate, const uint16_t* bias, int gelu,
                            hipStream_t stream) {
    if (M == 0 || N == 0) return hipSuccess;
    if (gs <= 0 || gs % 64 != 0 || K % gs != 0) return hipErrorInvalidValue;
    const int64_t tiles = static_cast<int64_t>((M + W4_BM - 1) / W4_BM) * ((N + W4_BN - 1) / W4_BN);
    if (tiles > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL(w4a4_gemm_kernel, dim3(static_cast<unsigned>(tiles)), dim3(W4_THR), 0, stream, act, wgt, as, ws,
                       out, M, N, K, gs, accumulate, bias, gelu);
    return hipGetLastError();
}

hipError_t launch_awq_repack(const int32_t* qw, int32_t* out, int OC, int IC, hipStream_t stream) {
    if (OC == 0 || IC == 0) return hipSuccess;
    if (OC % 4 != 0 || IC % 64 != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(awq_repack_kernel, dim3((OC + 255) / 256, IC / 8), dim3(256), 0, stream, qw, out, OC, IC);
    return hipGetLastError();
}

hipError_t launch_awq_dequant(const int32_t* qw, const uint16_t* wscales, const uint16_t* wzeros, uint16_t* out,
                              int OC, int IC, int gs, int ncomp, hipStream_t stream) {
    if (OC == 0 || IC == 0) return hipSuccess;
    if (OC % 4 != 0 || IC % 64 != 0 || gs <= 0 || IC % gs != 0 || ncomp <= 0 || OC % ncomp != 0)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(awq_dequant_kernel, dim3(grid_for(static_cast<int64_t>(OC) * IC)), dim3(256), 0, stream, qw,
                       wscales, wzeros, out, OC, IC, gs, ncomp);
    return hipGetLastError();
}

hipError_t launch_awq_gemv(const float* x, const int32_t* qw_rep, const uint16_t* wscales, const uint16_t* wzeros,
                           const uint16_t* bias, float* out, int OC, int IC, int gs, int ncomp, hipStream_t stream) {
    if (OC == 0) return hipSuccess;
    // the reference's GEMV reads 8 words (64 inputs) per group
    if (gs != 64 || IC % 64 != 0 || ncomp <= 0 || OC % ncomp != 0 || IC > 16384) return hipErrorInvalidValue;
    hipLaunchKernelGGL(awq_gemv_kernel, dim3((OC + 63) / 64), dim3(64), IC * sizeof(float), stream, x, qw_rep, wscales,
                       wzeros, bias, out, OC, IC, ncomp);
    return hipGetLastError();
}

hipError_t launch_nk_unswizzle(const uint8_t* q_sw, const uint16_t* s_sw, uint8_t* q_rm, float* s_rm, int N, int K,
                               int G, hipStream_t stream) {
    if (N == 0 || K == 0) return hipSuccess;
    if (K % 64 != 0 || G <= 0 || K % G != 0 || N % 128 != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(nk_unswizzle_kernel, dim3(grid_for(static_cast<int64_t>(N) * (K / 2))), dim3(256), 0, stream,
                       q_sw, s_sw, q_rm, s_rm, N, K, G);
    return hipGetLastError();
}

hipError_t launch_nk_dequant(const uint8_t* q_sw, const uint16_t* s_sw, uint16_t* out, int N, int K, int G,
                             hipStream_t stream) {
    if (N == 0 || K == 0) return hipSuccess;
    if (K % 64 != 0 || G <= 0 || K % G != 0 || N % 128 != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(nk_dequant_kernel, dim3(grid_for(static_cast<int64_t>(N) * K)), dim3(256), 0, stream, q_sw,
                       s_sw, out, N, K, G);
    return hipGetLastError();
}

hipError_t launch_lora_unswizzle(const uint16_t* packed, uint16_t* out, int rows, int cols, int is_down,
                                 hipStream_t stream) {
    if (rows == 0 || cols == 0) return hipSuccess;
    if (rows % 16 != 0 || cols % 16 != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(lora_unswizzle_kernel, dim3(grid_for(static_cast<int64_t>(rows) * cols)), dim3(256), 0, stream,
                       packed, out, rows, cols, is_down);
    return hipGetLastError();
}

hipError_t launch_transpose_u16(const uint16_t* in, uint16_t* out, int R, int C, hipStream_t stream) {
    if (R == 0 || C == 0) return hipSuccess;
    hipLaunchKernelGGL(transpose_u16_kernel, dim3(grid_for(static_cast<int64_t>(R) * C)), dim3(256), 0, stream, in,
                       out, R, C);
    return hipGetLastError();
}

hipError_t launch_f32_to_bf16(const float* in, uint16_t* out, int64_t n, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(f32_to_bf16_kernel, dim3(grid_for(n)), dim3(256), 0, stream, in, out, n);
    return hipGetLastError();
}

hipError_t launch_bf16_to_f32(const uint16_t* in, float* out, int64_t n, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(bf16_to_f32_kernel, dim3(grid_for(n)), dim3(256), 0, stream, in, out, n);
    return hipGetLastError();
}

}  // namespace qimg
