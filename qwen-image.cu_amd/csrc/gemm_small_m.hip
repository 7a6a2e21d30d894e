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
//    K blocks of loads in flight. Buffer loads with out-of-range offsets
//    stand in for every bounds check (rows past M or N, blocks past K).
//  - int8: two v_mfma_i32_32x32x32_i8 per K block (16 bytes each); e4m3: one
//    v_mfma_scale_f32_32x32x64_f8f6f4 with unit scales (32 bytes). Both
//    operands use the same K assignment, so each dot product covers every k
//    once and the int8 result is exact.
//  - The four waves' partial tiles are summed through LDS (int32 sums are
//    exact; e4m3 partials are added in wave order), then the dequant epilogue
//    is applied as the tile is stored, with the arithmetic of the large-tile
//    kernel, so both give identical outputs.
//
// Rows past M and columns past N read as zero and are never stored. The
// byte sizes M*K and N*K must be below 2^31 (buffer offsets are 32-bit).
#include <type_traits>
#include <utility>

#include "qimg_device.h"
#include "qimg_internal.h"

namespace qimg {

namespace {

constexpr int SM_THR = 256;  // four waves, one K quarter each
constexpr int SM_KB = 64;    // bytes of K per block
// Buffer resource word 3 for gfx9-family raw (unswizzled, unformatted) buffers.
constexpr int kBufferRsrcWord3 = 0x00020000;

// f(integral_constant<int, 0>), ..., f(integral_constant<int, N-1>)
template <typename F, int... Is>
__device__ __forceinline__ void sm_static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
    (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void sm_static_for(F&& f) {
    sm_static_for_impl(f, std::make_integer_sequence<int, N>{});
}

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

// Epilogue operands of the (row, 4-column run) groups a thread of the first
// four waves stores (the mapping of sm_finish), loaded at kernel start so
// their latency hides behind the operand stream: clamped indices, and a
// branch-free bias load (from ws when there is no bias) so the loads issue
// together.
template <int NBLK>
struct SmEpi {
    float as[NBLK];
    float ws[NBLK][4];
    uint16_t b[NBLK][4];
};

template <int TMW, int TNW>
__device__ __forceinline__ void sm_prefetch(SmEpi<TMW * TNW>& e, const float* as, const float* ws,
                                            const uint16_t* bias, int m0, int n0, int M, int N) {
    const uint16_t* bsrc = bias != nullptr ? bias : reinterpret_cast<const uint16_t*>(ws);
#pragma unroll
    for (int q = 0; q < TMW * TNW; ++q) {
        const int idx = (threadIdx.x & (SM_THR - 1)) + SM_THR * q;
        const int blk = idx >> 8;
        const int m = m0 + 32 * (blk / TNW) + (idx & 31);
        const int nb = n0 + 32 * (blk % TNW) + 8 * ((idx >> 6) & 3) + 4 * ((idx >> 5) & 1);
        e.as[q] = as[m < M ? m : M - 1];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int n = nb + c < N ? nb + c : N - 1;
            e.ws[q][c] = ws[n];
            e.b[q][c] = bsrc[n];
        }
    }
}

// Sum the waves' partial tiles through LDS and store the dequantized tile.
// Partial tiles go to LDS as [wave][block][run g][lane] of 16 bytes: lane
// holds 4 consecutive n per run (MFMA 32x32 layout, D = W x A, so lane has
// m = lane%32 and n = 8g + 4h + c for accumulator element 4g + c). With
// eight waves, waves 4-7 store first and waves 0-3 add them in. The first
// four waves then each own a quarter of the runs. `red` needs
// 4 * TMW * TNW * 4 KB; callers synchronise before reusing other LDS for it.
template <bool FP8, int TMW, int TNW, int NW, int OUT_DT, bool GELU, typename AccT>
__device__ __forceinline__ void sm_finish(AccT (&acc)[TMW][TNW], v4i* red, int wave, int lane,
                                          const SmEpi<TMW * TNW>& e, bool has_bias, void* out, int m0, int n0,
                                          int M, int N) {
    constexpr int NBLK = TMW * TNW;
    auto store_partial = [&](int slot, bool add) {
#pragma unroll
        for (int i = 0; i < TMW; ++i)
#pragma unroll
            for (int j = 0; j < TNW; ++j)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    v4i* dst = &red[((slot * NBLK + i * TNW + j) * 4 + g) * 64 + lane];
                    // (each element is copied to a scalar first: a bit cast of a
                    // vector-element lvalue reads element 0)
                    int b[4];
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        const auto x = acc[i][j][4 * g + c];
                        b[c] = __builtin_bit_cast(int, x);
                    }
                    v4i v = (v4i){b[0], b[1], b[2], b[3]};
                    if (add) {
                        const v4i o = *dst;
                        if constexpr (FP8)
                            v = __builtin_bit_cast(v4i, __builtin_bit_cast(v4f, v) + __builtin_bit_cast(v4f, o));
                        else
                            v += o;
                    }
                    *dst = v;
                }
    };
    if constexpr (NW == 8) {
        if (wave >= 4) store_partial(wave - 4, false);
        __syncthreads();
        if (wave < 4) store_partial(wave, true);
    } else {
        store_partial(wave, false);
    }
    __syncthreads();
    if (wave >= 4) return;

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
            v4i sum = red[(blk * 4 + g) * 64 + ln];
#pragma unroll
            for (int w = 1; w < 4; ++w) sum += red[((w * NBLK + blk) * 4 + g) * 64 + ln];
#pragma unroll
            for (int c = 0; c < 4; ++c) v[c] = static_cast<float>(sum[c]);
        } else {
            v4f sum = __builtin_bit_cast(v4f, red[(blk * 4 + g) * 64 + ln]);
#pragma unroll
            for (int w = 1; w < 4; ++w)
                sum += __builtin_bit_cast(v4f, red[((w * NBLK + blk) * 4 + g) * 64 + ln]);
#pragma unroll
            for (int c = 0; c < 4; ++c) v[c] = sum[c];
        }
#pragma unroll
        for (int c = 0; c < 4; ++c)
            v[c] = dequant_elem<GELU>(v[c], e.as[q], e.ws[q][c], has_bias, bf16_to_f32(e.b[q][c]));
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

// NW waves per workgroup (4 or 8) split K; the epilogue runs on the first
// four waves.
template <bool FP8, int TMW, int TNW, int DEPTH, int NW, int OUT_DT, bool GELU>
__global__ __launch_bounds__(64 * NW) void gemm_small_m_kernel(
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

    const bool has_bias = bias != nullptr;
    SmEpi<NBLK> epi;
    sm_prefetch<TMW, TNW>(epi, as, ws, bias, m0, n0, M, N);

    // K blocks are dealt round-robin to the waves (block 4t + wave), so the
    // four waves read adjacent 64-byte pieces of the same rows at the same
    // time. Operands are read with buffer loads: a lane whose row is past
    // M or N, or a block past K, gets an offset outside the buffer, which
    // returns zeros without touching memory. The main loop therefore has no
    // branches, every wave runs the same number of blocks, and the loads of
    // DEPTH blocks stay in flight while older blocks are consumed.
    const int nkb = K / SM_KB;
    const int T = (nkb + NW - 1) / NW;
    const int Tp = ((T + DEPTH - 1) / DEPTH) * DEPTH;
    constexpr uint32_t kOob = 0x80000000u;  // >= num_records: reads as zero
    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(A), 0, M * K, kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(W), 0, N * K, kBufferRsrcWord3);
    // Row offsets with the out-of-range bit or-ed in for rows past the end
    // (valid offsets are below 2^31, so the bit alone decides).
    uint32_t oa[TMW], ow[TNW];
#pragma unroll
    for (int i = 0; i < TMW; ++i) {
        const int gm = m0 + 32 * i + r;
        oa[i] = (static_cast<uint32_t>(gm) * K + 32 * h) | (gm < M ? 0u : kOob);
    }
#pragma unroll
    for (int j = 0; j < TNW; ++j) {
        const int gn = n0 + 32 * j + r;
        ow[j] = (static_cast<uint32_t>(gn) * K + 32 * h) | (gn < N ? 0u : kOob);
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
    auto load = [&](int d, int t) {
        const int kb = NW * t + wave;
        // block past K: the out-of-range bit (branch-free, wave-uniform)
        const uint32_t koff = (static_cast<uint32_t>(kb) * SM_KB) | (kb < nkb ? 0u : kOob);
#pragma unroll
        for (int i = 0; i < TMW; ++i) {
            const uint32_t o = (oa[i] + koff) | (oa[i] & kOob) | (koff & kOob);
#pragma unroll
            for (int s = 0; s < 2; ++s)
                ba[d][i][s] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(ra, o + 16 * s, 0, 0));
        }
#pragma unroll
        for (int j = 0; j < TNW; ++j) {
            const uint32_t o = (ow[j] + koff) | (ow[j] & kOob) | (koff & kOob);
#pragma unroll
            for (int s = 0; s < 2; ++s)
                bw[d][j][s] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rw, o + 16 * s, 0, 0));
        }
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

    // Block t is consumed from register set t % DEPTH, which is then refilled
    // with block t + DEPTH (past the end: zero-returning loads).
    // (sched_barrier keeps the prologue in block order: the scheduler would
    // otherwise issue block 0 last, next to its first use, and the first
    // wait would then drain every load.)
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

    sm_finish<FP8, TMW, TNW, NW, OUT_DT, GELU>(acc, red, wave, lane, epi, has_bias, out, m0, n0, M, N);
}

template <bool FP8, int TMW, int TNW, int DEPTH, int NW>
hipError_t launch_small(const void* a, const float* as, int M, int K, const void* w, const float* ws,
                        int N, const uint16_t* bias, void* out, int out_dt, int gelu, hipStream_t stream) {
    const int tiles = ((M + 32 * TMW - 1) / (32 * TMW)) * ((N + 32 * TNW - 1) / (32 * TNW));
    const uint8_t* A = static_cast<const uint8_t*>(a);
    const uint8_t* Wq = static_cast<const uint8_t*>(w);
#define QIMG_SMALL_LAUNCH(ODT, GL)                                                                      \
    hipLaunchKernelGGL((gemm_small_m_kernel<FP8, TMW, TNW, DEPTH, NW, ODT, GL>), dim3(tiles), dim3(64 * NW), \
                       0, stream, A, Wq, as, ws, bias, out, M, N, K)
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


// LDS-staged variant for K a multiple of 4 * BKB. A load instruction whose 64
// lanes touch 32 different rows (the direct fragment loads above) costs the
// address unit several times more than one whose lanes read whole rows of
// contiguous bytes, so here each wave copies its K blocks into its own LDS
// ring with global -> LDS DMA and reads MFMA fragments from LDS. BKB = 128
// (K blocks of one whole 128-byte line per row, 8 rows per DMA instruction,
// the large-tile kernel's swizzle) moves about twice the bytes per unit
// time of BKB = 64 (half lines, 16 rows per instruction). The rings are
// private to their waves, so the main loop needs no barrier: a wave waits
// only for its own DMA (vmcnt) and its own reads (lgkmcnt). Rows past M or
// N are clamped (computed, never stored); K is split exactly.
template <int BKB>
__device__ __forceinline__ int sm_swz(int row) {
    if constexpr (BKB == 128)
        return (row >> 1) & 7;
    else
        return swz_row(row);
}

template <bool FP8, int TMW, int TNW, int D, int OUT_DT, bool GELU, int BKB>
__global__ __launch_bounds__(SM_THR) void gemm_small_dma_kernel(
    const uint8_t* __restrict__ A, const uint8_t* __restrict__ W, const float* __restrict__ as,
    const float* __restrict__ ws, const uint16_t* __restrict__ bias, void* __restrict__ out, int M,
    int N, int K) {
    constexpr int NW = SM_THR / 64;
    constexpr int MB = 32 * TMW;
    constexpr int NB = 32 * TNW;
    constexpr int NBLK = TMW * TNW;
    constexpr int ROWS = MB + NB;
    constexpr int CPR = BKB / 16;       // 16-byte chunks per row of a block
    constexpr int RPI = 1024 / BKB;     // rows per DMA instruction
    constexpr int SLOT = ROWS * BKB;    // one K block of the tile's rows
    constexpr int NDMA = ROWS / RPI;    // DMA instructions per block
    constexpr int RING = D * SLOT;      // per wave
    constexpr int LDS_RING = NW * RING;
    constexpr int LDS_RED = 4 * NBLK * 4 * 64 * 16;
    constexpr int LDS_BYTES = LDS_RING > LDS_RED ? LDS_RING : LDS_RED;
    static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
    static_assert(MB % RPI == 0, "A rows fill whole DMA instructions");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[LDS_BYTES];

    const int tiles_m = (M + MB - 1) / MB;
    const int tiles_n = (N + NB - 1) / NB;
    const int logical = xcd_remap(blockIdx.x, tiles_m * tiles_n);
    const int m0 = (logical % tiles_m) * MB;
    const int n0 = (logical / tiles_m) * NB;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 31;
    const int h = lane >> 5;

    const bool has_bias = bias != nullptr;
    SmEpi<NBLK> epi;
    sm_prefetch<TMW, TNW>(epi, as, ws, bias, m0, n0, M, N);

    // Block t of this wave is K block NW*t + wave. DMA instruction i fills
    // slot rows RPI*i .. RPI*i + RPI-1 (A rows first, then W rows); lane ->
    // row RPI*i + lane/CPR at physical chunk lane%CPR.
    const int T = K / (BKB * NW);
    const uint8_t* src[NDMA];
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
        const int row = RPI * i + lane / CPR;
        const int c = (lane % CPR) ^ sm_swz<BKB>(row);
        const uint8_t* base;
        if (RPI * i < MB) {
            const int gm = m0 + row < M ? m0 + row : M - 1;
            base = A + static_cast<int64_t>(gm) * K;
        } else {
            const int gn = n0 + row - MB < N ? n0 + row - MB : N - 1;
            base = W + static_cast<int64_t>(gn) * K;
        }
        src[i] = base + wave * BKB + c * 16;
    }
    uint8_t* ring = lds + wave * RING;
    auto issue = [&](int t, int slot) {
        const int64_t koff = static_cast<int64_t>(t) * (NW * BKB);
        uint8_t* dst = ring + slot * SLOT;
#pragma unroll
        for (int i = 0; i < NDMA; ++i)
            __builtin_amdgcn_global_load_lds((gbl_ptr_t)(src[i] + koff), (lds_ptr_t)(dst + i * 1024), 16, 0, 1);
    };

    typedef typename SmAcc<FP8>::type acc_t;
    acc_t acc[TMW][TNW];
#pragma unroll
    for (int i = 0; i < TMW; ++i)
#pragma unroll
        for (int j = 0; j < TNW; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;

    auto frag = [&](const uint8_t* base, int row, int chunk) {
        return *reinterpret_cast<const v4i*>(base + row * BKB + ((chunk ^ sm_swz<BKB>(row)) << 4));
    };
    // Lane half h takes chunks [h*CPR/2, (h+1)*CPR/2) of every row: int8
    // steps of one chunk each, e4m3 steps of two (both operands alike, so
    // each dot product covers every k of the block once).
    auto compute = [&](int slot) {
        const uint8_t* base = ring + slot * SLOT;
        if constexpr (!FP8) {
#pragma unroll
            for (int s = 0; s < CPR / 2; ++s) {
                v4i fa[TMW], fw[TNW];
#pragma unroll
                for (int i = 0; i < TMW; ++i) fa[i] = frag(base, 32 * i + r, (CPR / 2) * h + s);
#pragma unroll
                for (int j = 0; j < TNW; ++j) fw[j] = frag(base, MB + 32 * j + r, (CPR / 2) * h + s);
#pragma unroll
                for (int i = 0; i < TMW; ++i)
#pragma unroll
                    for (int j = 0; j < TNW; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fw[j], fa[i], acc[i][j], 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int s = 0; s < CPR / 4; ++s) {
                const int c0 = (CPR / 2) * h + 2 * s;
                v8i fa[TMW], fw[TNW];
#pragma unroll
                for (int i = 0; i < TMW; ++i) {
                    const v4i lo = frag(base, 32 * i + r, c0), hi = frag(base, 32 * i + r, c0 + 1);
                    fa[i] = (v8i){lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
                }
#pragma unroll
                for (int j = 0; j < TNW; ++j) {
                    const v4i lo = frag(base, MB + 32 * j + r, c0), hi = frag(base, MB + 32 * j + r, c0 + 1);
                    fw[j] = (v8i){lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
                }
#pragma unroll
                for (int i = 0; i < TMW; ++i)
#pragma unroll
                    for (int j = 0; j < TNW; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fw[j], fa[i], acc[i][j], 0, 0,
                                                                                    0, 127, 0, 127);
            }
        }
    };

    // Prologue: the first min(T, D) blocks. Steady state: block t lands
    // (all but the D-1 younger blocks' DMA done), is consumed, and its slot
    // is refilled with block t + D once this wave's reads of it returned.
    // Tail: the last D blocks, with the wait shrinking as no younger blocks
    // are issued.
#pragma unroll
    for (int d = 0; d < D; ++d)
        if (d < T) issue(d, d);
    int t = 0;
    for (; t + D < T; ++t) {
        const int slot = t % D;
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt<(D - 1) * NDMA>();
        compute(slot);
        __builtin_amdgcn_sched_barrier(0);
        wait_lgkmcnt0();
        issue(t + D, slot);
    }
    sm_static_for<D>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        const int tt = T - D + j;
        if (tt >= 0) {
            __builtin_amdgcn_sched_barrier(0);
            wait_vmcnt<(D - 1 - j) * NDMA>();
            compute(tt % D);
        }
    });
    __syncthreads();  // every wave is done with its ring: reuse LDS for the reduction
    sm_finish<FP8, TMW, TNW, NW, OUT_DT, GELU>(acc, reinterpret_cast<v4i*>(lds), wave, lane, epi, has_bias, out,
                                               m0, n0, M, N);
}

template <bool FP8, int TMW, int TNW, int D, int BKB = SM_KB>
hipError_t launch_small_dma(const void* a, const float* as, int M, int K, const void* w, const float* ws, int N,
                            const uint16_t* bias, void* out, int out_dt, int gelu, hipStream_t stream) {
    const int tiles = ((M + 32 * TMW - 1) / (32 * TMW)) * ((N + 32 * TNW - 1) / (32 * TNW));
    const uint8_t* A = static_cast<const uint8_t*>(a);
    const uint8_t* Wq = static_cast<const uint8_t*>(w);
#define QIMG_SMALL_DMA_LAUNCH(ODT, GL)                                                                            \
    hipLaunchKernelGGL((gemm_small_dma_kernel<FP8, TMW, TNW, D, ODT, GL, BKB>), dim3(tiles), dim3(SM_THR), 0, stream, A, \
                       Wq, as, ws, bias, out, M, N, K)
    if (out_dt == QIMG_FP32) {
        if (gelu)
            QIMG_SMALL_DMA_LAUNCH(QIMG_FP32, true);
        else
            QIMG_SMALL_DMA_LAUNCH(QIMG_FP32, false);
    } else {
        if (gelu)
            QIMG_SMALL_DMA_LAUNCH(QIMG_BF16, true);
        else
            QIMG_SMALL_DMA_LAUNCH(QIMG_BF16, false);
    }
#undef QIMG_SMALL_DMA_LAUNCH
    return hipGetLastError();
}

typedef float v2f __attribute__((ext_vector_type(2)));

// Rows of A at most GV_MAXM: a weight-streaming GEMV on the vector ALU.
// Each wave owns RW consecutive weight rows and reads them front to back,
// 1 KB per load instruction (lane i takes bytes 16i.. of each 1 KB piece),
// so the wave streams one contiguous RW*K-byte range of W; every lane also
// loads the matching 16 bytes of the MR activation rows (cache hits after
// the first wave). int8: v_dot4_i32_i8 accumulates per lane, a wave
// reduction gives each (m, n) dot product, exact in int32. e4m3 (FP8): the
// bytes are converted to fp32 (v_cvt_pk_f32_fp8; each product of two e4m3
// values is exact in fp32) and accumulated with fp32 FMAs per lane, then
// summed over the wave. Out-of-range rows and chunks read as zero through
// buffer loads, as in the MFMA kernel.
constexpr int GV_MAXM = 4;

// The weight-side operands of one GEMV of a launch.
struct GemvOut {
    const uint8_t* W;
    const float* ws;
    const uint16_t* bias;
    void* out;
    int N;
};

// Workgroups [0, split) compute GEMV g0, the rest g1 (two linears of the
// same activation in one launch, e.g. a block's image and text modulation).
// ONE: the whole row fits in IU chunks per lane (K <= IU*1024): all loads
// are issued at once and nothing is loaded past K; otherwise steps of IU
// chunks alternate between two register sets.
template <int MR, int RW, int IU, bool ONE, int OUT_DT, bool GELU, bool FP8 = false>
__global__ __launch_bounds__(SM_THR) void gemv_i8_kernel(const uint8_t* __restrict__ A, const float* __restrict__ as,
                                                         int M, int K, GemvOut g0, GemvOut g1, int split) {
    const bool second = static_cast<int>(blockIdx.x) >= split;
    const uint8_t* __restrict__ W = second ? g1.W : g0.W;
    const float* __restrict__ ws = second ? g1.ws : g0.ws;
    const uint16_t* __restrict__ bias = second ? g1.bias : g0.bias;
    void* __restrict__ out = second ? g1.out : g0.out;
    const int N = second ? g1.N : g0.N;
    const int bid = second ? static_cast<int>(blockIdx.x) - split : static_cast<int>(blockIdx.x);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n0 = (bid * (SM_THR / 64) + wave) * RW;
    if (n0 >= N) return;  // wave-uniform; no barriers below
    constexpr uint32_t kOob = 0x80000000u;
    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(A), 0, M * K, kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(W), 0, N * K, kBufferRsrcWord3);
    const int KC = K >> 4;              // 16-byte chunks per row
    const int I = (KC + 63) >> 6;       // chunks per lane
    const int S = (I + 2 * IU - 1) / (2 * IU) * 2;  // steps of IU chunks, even
    uint32_t arow[MR], wrow[RW];
#pragma unroll
    for (int m = 0; m < MR; ++m) arow[m] = m < M ? static_cast<uint32_t>(m) * K : kOob;
#pragma unroll
    for (int q = 0; q < RW; ++q) wrow[q] = n0 + q < N ? static_cast<uint32_t>(n0 + q) * K : kOob;

    // Lane l < MR*RW stores output (m = l / RW, n = n0 + l % RW); its scales
    // and bias are loaded now (clamped, branch-free) so their latency hides
    // behind the weight stream.
    const bool has_bias = bias != nullptr;
    const int e_m = lane / RW;
    const int e_n = n0 + lane % RW;
    const int e_nc = e_n < N ? e_n : N - 1;
    const float e_as = as[e_m < M ? e_m : M - 1];
    const float e_ws = ws[e_nc];
    const uint16_t e_b = (has_bias ? bias : reinterpret_cast<const uint16_t*>(ws))[e_nc];

    typedef typename std::conditional<FP8, float, int>::type acc_t;
    acc_t acc[MR][RW];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int q = 0; q < RW; ++q) acc[m][q] = 0;

    v4i fa[ONE ? 1 : 2][IU][MR], fw[ONE ? 1 : 2][IU][RW];
    auto load = [&](int set, int step) {
#pragma unroll
        for (int u = 0; u < IU; ++u) {
            const int c = (step * IU + u) * 64 + lane;
            const uint32_t col = c < KC ? static_cast<uint32_t>(c) * 16 : kOob;
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const uint32_t o = (arow[m] + col) | ((arow[m] | col) & kOob);
                fa[set][u][m] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(ra, o, 0, 0));
            }
#pragma unroll
            for (int q = 0; q < RW; ++q) {
                const uint32_t o = (wrow[q] + col) | ((wrow[q] | col) & kOob);
                fw[set][u][q] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rw, o, 0, 0));
            }
        }
    };
    auto compute = [&](int set) {
#pragma unroll
        for (int u = 0; u < IU; ++u) {
            if constexpr (FP8) {
                // 16 e4m3 bytes -> 16 fp32, in byte order
                auto widen = [](const v4i& c, float (&f)[16]) {
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        const v2f lo = __builtin_amdgcn_cvt_pk_f32_fp8(c[d], false);
                        const v2f hi = __builtin_amdgcn_cvt_pk_f32_fp8(c[d], true);
                        f[4 * d] = lo.x;
                        f[4 * d + 1] = lo.y;
                        f[4 * d + 2] = hi.x;
                        f[4 * d + 3] = hi.y;
                    }
                };
                float af[MR][16];
#pragma unroll
                for (int m = 0; m < MR; ++m) widen(fa[set][u][m], af[m]);
#pragma unroll
                for (int q = 0; q < RW; ++q) {
                    float wf[16];
                    widen(fw[set][u][q], wf);
#pragma unroll
                    for (int m = 0; m < MR; ++m) {
                        float t = acc[m][q];
#pragma unroll
                        for (int e = 0; e < 16; ++e) t = __builtin_fmaf(af[m][e], wf[e], t);
                        acc[m][q] = t;
                    }
                }
            } else {
#pragma unroll
                for (int m = 0; m < MR; ++m)
#pragma unroll
                    for (int q = 0; q < RW; ++q) {
                        const v4i a = fa[set][u][m];
                        const v4i w = fw[set][u][q];
                        int t = acc[m][q];
                        t = __builtin_amdgcn_sdot4(a.x, w.x, t, false);
                        t = __builtin_amdgcn_sdot4(a.y, w.y, t, false);
                        t = __builtin_amdgcn_sdot4(a.z, w.z, t, false);
                        t = __builtin_amdgcn_sdot4(a.w, w.w, t, false);
                        acc[m][q] = t;
                    }
            }
        }
    };
    load(0, 0);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (ONE) {
        compute(0);
    } else {
    for (int st = 0; st < S; st += 2) {
        load(1, st + 1);
        __builtin_amdgcn_sched_barrier(0);
        compute(0);
        load(0, st + 2);  // past the end: zero-returning loads
        __builtin_amdgcn_sched_barrier(0);
        compute(1);
    }
    }

    // wave reductions; lane m*RW + q keeps the (m, q) total
    acc_t mine = 0;
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int q = 0; q < RW; ++q) {
            const acc_t tot = wave_sum_dpp(acc[m][q]);
            mine = lane == m * RW + q ? tot : mine;
        }
    if (lane < MR * RW && e_m < M && e_n < N) {
        const float v = dequant_elem<GELU>(static_cast<float>(mine), e_as, e_ws, has_bias, bf16_to_f32(e_b));
        if (OUT_DT == QIMG_FP32)
            reinterpret_cast<float*>(out)[static_cast<int64_t>(e_m) * N + e_n] = v;
        else
            reinterpret_cast<uint16_t*>(out)[static_cast<int64_t>(e_m) * N + e_n] = f32_to_bf16(v);
    }
}

template <int MR, int RW, int IU, bool ONE, bool FP8>
hipError_t launch_gemv(const void* a, const float* as, int M, int K, const GemvOut& g0, const GemvOut& g1,
                       int out_dt, int gelu, hipStream_t stream) {
    auto blocks_of = [](int N) {
        const int waves = (N + RW - 1) / RW;
        return (waves + SM_THR / 64 - 1) / (SM_THR / 64);
    };
    const int split = blocks_of(g0.N);
    const int blocks = split + (g1.N > 0 ? blocks_of(g1.N) : 0);
    const uint8_t* A = static_cast<const uint8_t*>(a);
#define QIMG_GEMV_LAUNCH(ODT, GL)                                                                              \
    hipLaunchKernelGGL((gemv_i8_kernel<MR, RW, IU, ONE, ODT, GL, FP8>), dim3(blocks), dim3(SM_THR), 0, stream, A, as, M, \
                       K, g0, g1, split)
    if (out_dt == QIMG_FP32) {
        if (gelu)
            QIMG_GEMV_LAUNCH(QIMG_FP32, true);
        else
            QIMG_GEMV_LAUNCH(QIMG_FP32, false);
    } else {
        if (gelu)
            QIMG_GEMV_LAUNCH(QIMG_BF16, true);
        else
            QIMG_GEMV_LAUNCH(QIMG_BF16, false);
    }
#undef QIMG_GEMV_LAUNCH
    return hipGetLastError();
}

template <bool FP8>
hipError_t dispatch_gemv(const void* a, const float* as, int M, int K, const GemvOut& g0, const GemvOut& g1,
                         int out_dt, int gelu, hipStream_t stream) {
    const int chunks = ((K >> 4) + 63) >> 6;  // 16-byte chunks per lane
#define QIMG_GEMV(MR_, RW_, IU_, ONE_) \
    return launch_gemv<MR_, RW_, IU_, ONE_, FP8>(a, as, M, K, g0, g1, out_dt, gelu, stream)
    if (M <= 2 && chunks <= 4) {
        if (M == 1) {
            if (chunks == 1) QIMG_GEMV(1, 8, 1, true);
            if (chunks == 2) QIMG_GEMV(1, 8, 2, true);
            if (chunks == 3) QIMG_GEMV(1, 8, 3, true);
            QIMG_GEMV(1, 8, 4, true);
        }
        if (chunks == 1) QIMG_GEMV(2, 8, 1, true);
        if (chunks == 2) QIMG_GEMV(2, 8, 2, true);
        if (chunks == 3) QIMG_GEMV(2, 8, 3, true);
        QIMG_GEMV(2, 8, 4, true);
    }
    if (M == 1) QIMG_GEMV(1, 8, 2, false);
    if (M == 2) QIMG_GEMV(2, 8, 2, false);
    QIMG_GEMV(4, 4, 2, false);
#undef QIMG_GEMV
}
}  // namespace

bool small_m_fits(int M, int N, int K) {
    return M > 0 && N > 0 && (K % SM_KB) == 0 && static_cast<int64_t>(M) * K < (int64_t{1} << 31) &&
           static_cast<int64_t>(N) * K < (int64_t{1} << 31);
}

// Two linears of the same M <= GV_MAXM activation and mode in one GEMV
// launch (false: not that case; the caller then runs them one at a time).
bool launch_gemv_pair(const void* act_q, const float* act_scales, int M, int K, const LinearArgs& a,
                      const LinearArgs& b, int mode, int out_dtype, hipStream_t stream, hipError_t* err) {
    if (!(get_linear_kernel() == QIMG_LINEAR_AUTO && M >= 1 && M <= GV_MAXM && small_m_fits(M, a.N, K) &&
          small_m_fits(M, b.N, K) && a.K == K && b.K == K &&
          small_m_variant(M, a.N, K) == 3 && small_m_variant(M, b.N, K) == 3))
        return false;
    const GemvOut ga{static_cast<const uint8_t*>(a.w_q), a.w_scales, a.bias, a.out, a.N};
    const GemvOut gb{static_cast<const uint8_t*>(b.w_q), b.w_scales, b.bias, b.out, b.N};
    *err = mode == QIMG_QM_FP8_HADAMARD
               ? dispatch_gemv<true>(act_q, act_scales, M, K, ga, gb, out_dtype, 0, stream)
               : dispatch_gemv<false>(act_q, act_scales, M, K, ga, gb, out_dtype, 0, stream);
    return true;
}

int small_m_variant(int M, int N, int K) {
    if (!small_m_fits(M, N, K)) return 0;
    if (M <= GV_MAXM) return 3;
    if (M <= 32) return 1;
    const int64_t big_tiles = static_cast<int64_t>((M + 255) / 256) * ((N + 255) / 256);
    return big_tiles < kSmallMTileLimit ? 2 : 0;
}

hipError_t launch_linear_small_m(const void* act_q, const float* act_scales, int M, int K, const void* w_q,
                                 const float* w_scales, int N, int mode, const uint16_t* bias, void* out,
                                 int out_dtype, int gelu, int variant, hipStream_t stream) {
    const bool fp8 = (mode == QIMG_QM_FP8_HADAMARD);
    if (!small_m_fits(M, N, K)) return hipErrorInvalidValue;
    // The LDS-staged kernels split K exactly over four waves.
    const bool lds_staged = (K % (SM_KB * (SM_THR / 64))) == 0;
    // Whole-line K blocks where K is long (text fc2, K = 12288: 25.8 -> 20.7
    // us at M = 256, in-process A/B, output identical); at K = 3072 they
    // measured equal.
    const bool whole_lines = (K % (128 * (SM_THR / 64))) == 0 && K >= 8192;
    if (variant == 3 && M <= GV_MAXM) {
        const GemvOut g{static_cast<const uint8_t*>(w_q), w_scales, bias, out, N};
        return fp8 ? dispatch_gemv<true>(act_q, act_scales, M, K, g, GemvOut{}, out_dtype, gelu, stream)
                   : dispatch_gemv<false>(act_q, act_scales, M, K, g, GemvOut{}, out_dtype, gelu, stream);
    }
    if (variant == 3) variant = 1;  // more rows than the GEMV takes
    if (variant == 1 && lds_staged)
        return fp8 ? launch_small_dma<true, 1, 1, 4>(act_q, act_scales, M, K, w_q, w_scales, N, bias, out,
                                                     out_dtype, gelu, stream)
                   : launch_small_dma<false, 1, 1, 4>(act_q, act_scales, M, K, w_q, w_scales, N, bias, out,
                                                      out_dtype, gelu, stream);
    if (variant == 2 && whole_lines)
        return fp8 ? launch_small_dma<true, 2, 2, 2, 128>(act_q, act_scales, M, K, w_q, w_scales, N, bias, out,
                                                          out_dtype, gelu, stream)
                   : launch_small_dma<false, 2, 2, 2, 128>(act_q, act_scales, M, K, w_q, w_scales, N, bias, out,
                                                           out_dtype, gelu, stream);
    if (variant == 2 && lds_staged) {
        // two slots per wave (64 KB) leave room for two workgroups per CU
        // when there are enough tiles to use them
        const int64_t tiles = static_cast<int64_t>((M + 63) / 64) * ((N + 63) / 64);
        if (tiles > 256)
            return fp8 ? launch_small_dma<true, 2, 2, 2>(act_q, act_scales, M, K, w_q, w_scales, N, bias, out,
                                                         out_dtype, gelu, stream)
                       : launch_small_dma<false, 2, 2, 2>(act_q, act_scales, M, K, w_q, w_scales, N, bias, out,
                                                          out_dtype, gelu, stream);
        return fp8 ? launch_small_dma<true, 2, 2, 3>(act_q, act_scales, M, K, w_q, w_scales, N, bias, out,
                                                     out_dtype, gelu, stream)
                   : launch_small_dma<false, 2, 2, 3>(act_q, act_scales, M, K, w_q, w_scales, N, bias, out,
                                                      out_dtype, gelu, stream);
    }
    if (variant == 1)
        return fp8 ? launch_small<true, 1, 1, 8, 4>(act_q, act_scales, M, K, w_q, w_scales, N, bias, out, out_dtype,
                                                 gelu, stream)
                   : launch_small<false, 1, 1, 8, 4>(act_q, act_scales, M, K, w_q, w_scales, N, bias, out,
                                                  out_dtype, gelu, stream);
    if (variant == 2)
        return fp8 ? launch_small<true, 2, 2, 4, 8>(act_q, act_scales, M, K, w_q, w_scales, N, bias, out, out_dtype,
                                                 gelu, stream)
                   : launch_small<false, 2, 2, 4, 8>(act_q, act_scales, M, K, w_q, w_scales, N, bias, out,
                                                  out_dtype, gelu, stream);
    return hipErrorInvalidValue;
}

}  // namespace qimg
