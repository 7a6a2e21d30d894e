// mfma_probe.hip — the sustained matrix-core rate of this GPU, measured: a
// register-only loop of one MFMA form per launch (no memory traffic in the
// loop), each wave recording the shader-clock counter (s_memtime) and the
// constant 100 MHz counter (s_memrealtime) around its loop, so the host gets
// both the achieved op rate and the clock it ran at. It is the ceiling the
// GEMM and attention kernels of this library are compared against beside the
// spec-sheet peak (the spec figures assume the 2.4 GHz peak clock, which the
// chip does not hold under a full matrix-core load).
//
// Built into its own library (lib/libqimg_probe.so); no product code calls it.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

// Probe kinds (qimg_probe_mfma's `kind`) and ops per instruction.
constexpr int KIND_I8_32 = 0;   // v_mfma_i32_32x32x32_i8            65536 ops
constexpr int KIND_I8_16 = 1;   // v_mfma_i32_16x16x64_i8            32768 ops
constexpr int KIND_F8_32 = 2;   // v_mfma_scale_f32_32x32x64_f8f6f4 131072 flops (e4m3, unit scales)
constexpr int KIND_F16_32 = 3;  // v_mfma_f32_32x32x16_f16           32768 flops
constexpr int KIND_BF16_32 = 4; // v_mfma_f32_32x32x16_bf16          32768 flops
constexpr int KIND_F8_16 = 5;   // v_mfma_scale_f32_16x16x128_f8f6f4 65536 flops (e4m3, unit scales)
constexpr int KIND_F16_16 = 6;  // v_mfma_f32_16x16x32_f16           16384 flops

constexpr int NCH = 4;     // independent accumulator chains
constexpr int UNROLL = 4;  // MFMAs per chain per loop iteration

// Operand bits that change from lane to lane and register to register (a
// 32-bit integer hash), masked per kind so no value is an fp Inf or NaN.
__device__ __forceinline__ uint32_t mix(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

template <int KIND>
__device__ __forceinline__ uint32_t operand_bits(uint32_t seed) {
    const uint32_t r = mix(seed);
    if constexpr (KIND == KIND_F8_32 || KIND == KIND_F8_16) return r & 0xf7f7f7f7u;  // e4m3: exponent <= 14
    if constexpr (KIND == KIND_F16_32 || KIND == KIND_BF16_32 || KIND == KIND_F16_16)
        return r & 0xbfffbfffu;  // |x| < 2
    return r;
}

template <int KIND, int LDS_KB>
__global__ __launch_bounds__(256) void mfma_probe_kernel(int iters, uint64_t* __restrict__ clocks,
                                                         int* __restrict__ sink) {
    // (occupancy: the LDS each workgroup holds caps the workgroups per CU)
    __shared__ int pad[LDS_KB * 256];
    const int lane = threadIdx.x & 63;
    const int gw = blockIdx.x * 4 + (threadIdx.x >> 6);  // global wave index
    uint32_t a[8], b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        a[i] = operand_bits<KIND>(static_cast<uint32_t>((gw * 64 + lane) * 16 + i));
        b[i] = operand_bits<KIND>(static_cast<uint32_t>((gw * 64 + lane) * 16 + 8 + i));
    }
    if (threadIdx.x == 0) pad[blockIdx.x & 255] = static_cast<int>(a[0]);
    __syncthreads();

    const uint64_t t0 = __builtin_amdgcn_s_memtime();
    const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
    int result = 0;
    if constexpr (KIND == KIND_I8_32) {
        const v4i va = {static_cast<int>(a[0]), static_cast<int>(a[1]), static_cast<int>(a[2]), static_cast<int>(a[3])};
        const v4i vb = {static_cast<int>(b[0]), static_cast<int>(b[1]), static_cast<int>(b[2]), static_cast<int>(b[3])};
        v16i acc[NCH] = {};
        for (int it = 0; it < iters; ++it) {
#pragma unroll
            for (int u = 0; u < UNROLL; ++u)
#pragma unroll
                for (int c = 0; c < NCH; ++c) acc[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(va, vb, acc[c], 0, 0, 0);
        }
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
            for (int r = 0; r < 16; ++r) result += acc[c][r];
    } else if constexpr (KIND == KIND_I8_16) {
        const v4i va = {static_cast<int>(a[0]), static_cast<int>(a[1]), static_cast<int>(a[2]), static_cast<int>(a[3])};
        const v4i vb = {static_cast<int>(b[0]), static_cast<int>(b[1]), static_cast<int>(b[2]), static_cast<int>(b[3])};
        v4i acc[2 * NCH] = {};
        for (int it = 0; it < iters; ++it) {
#pragma unroll
            for (int u = 0; u < 2 * UNROLL; ++u)
#pragma unroll
                for (int c = 0; c < 2 * NCH; ++c)
                    acc[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(va, vb, acc[c], 0, 0, 0);
        }
#pragma unroll
        for (int c = 0; c < 2 * NCH; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) result += acc[c][r];
    } else if constexpr (KIND == KIND_F8_32) {
        v8i va, vb;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            va[i] = static_cast<int>(a[i]);
            vb[i] = static_cast<int>(b[i]);
        }
        v16f acc[NCH] = {};
        for (int it = 0; it < iters; ++it) {
#pragma unroll
            for (int u = 0; u < UNROLL; ++u)
#pragma unroll
                for (int c = 0; c < NCH; ++c)
                    acc[c] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(va, vb, acc[c], 0, 0, 0, 127, 0, 127);
        }
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
            for (int r = 0; r < 16; ++r) result ^= __float_as_int(acc[c][r]);
    } else if constexpr (KIND == KIND_F8_16) {
        v8i va, vb;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            va[i] = static_cast<int>(a[i]);
            vb[i] = static_cast<int>(b[i]);
        }
        v4f acc[2 * NCH] = {};
        for (int it = 0; it < iters; ++it) {
#pragma unroll
            for (int u = 0; u < 2 * UNROLL; ++u)
#pragma unroll
                for (int c = 0; c < 2 * NCH; ++c)
                    acc[c] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(va, vb, acc[c], 0, 0, 0, 127, 0, 127);
        }
#pragma unroll
        for (int c = 0; c < 2 * NCH; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) result ^= __float_as_int(acc[c][r]);
    } else if constexpr (KIND == KIND_F16_16) {
        const v4i wa = {static_cast<int>(a[0]), static_cast<int>(a[1]), static_cast<int>(a[2]), static_cast<int>(a[3])};
        const v4i wb = {static_cast<int>(b[0]), static_cast<int>(b[1]), static_cast<int>(b[2]), static_cast<int>(b[3])};
        v4f acc[2 * NCH] = {};
        for (int it = 0; it < iters; ++it) {
#pragma unroll
            for (int u = 0; u < 2 * UNROLL; ++u)
#pragma unroll
                for (int c = 0; c < 2 * NCH; ++c)
                    acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, wa),
                                                                    __builtin_bit_cast(v8h, wb), acc[c], 0, 0, 0);
        }
#pragma unroll
        for (int c = 0; c < 2 * NCH; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) result ^= __float_as_int(acc[c][r]);
    } else {
        v4i wa = {static_cast<int>(a[0]), static_cast<int>(a[1]), static_cast<int>(a[2]), static_cast<int>(a[3])};
        v4i wb = {static_cast<int>(b[0]), static_cast<int>(b[1]), static_cast<int>(b[2]), static_cast<int>(b[3])};
        v16f acc[NCH] = {};
        for (int it = 0; it < iters; ++it) {
#pragma unroll
            for (int u = 0; u < UNROLL; ++u)
#pragma unroll
                for (int c = 0; c < NCH; ++c) {
                    if constexpr (KIND == KIND_F16_32)
                        acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, wa),
                                                                        __builtin_bit_cast(v8h, wb), acc[c], 0, 0, 0);
                    else
                        acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, wa),
                                                                         __builtin_bit_cast(v8bf, wb), acc[c], 0, 0,
                                                                         0);
                }
        }
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
            for (int r = 0; r < 16; ++r) result ^= __float_as_int(acc[c][r]);
    }
    const uint64_t t1 = __builtin_amdgcn_s_memtime();
    const uint64_t r1 = __builtin_amdgcn_s_memrealtime();
    if (lane == 0) {
        clocks[4 * gw + 0] = t0;
        clocks[4 * gw + 1] = t1;
        clocks[4 * gw + 2] = r0;
        clocks[4 * gw + 3] = r1;
    }
    sink[blockIdx.x * 256 + threadIdx.x] = result + pad[blockIdx.x & 255];
}

template <int KIND>
hipError_t launch(int wps, int cus, int iters, uint64_t* clocks, int* sink, hipStream_t s) {
    const dim3 grid(cus * wps), block(256);
    if (wps == 1)
        hipLaunchKernelGGL((mfma_probe_kernel<KIND, 96>), grid, block, 0, s, iters, clocks, sink);
    else
        hipLaunchKernelGGL((mfma_probe_kernel<KIND, 64>), grid, block, 0, s, iters, clocks, sink);
    return hipGetLastError();
}

}  // namespace

extern "C" {

// MFMAs one wave issues per loop iteration of `kind`.
int qimg_probe_mfma_per_iter(int kind) {
    return (kind == KIND_I8_16 || kind == KIND_F8_16 || kind == KIND_F16_16) ? 4 * NCH * UNROLL : NCH * UNROLL;
}

// One launch of the probe: `cus` x `wps` workgroups of four waves (one per
// SIMD; the LDS each holds lets at most wps of them share a CU: wps 1 or 2),
// each wave running `iters` loop iterations. clocks: uint64 [4 * waves]
// (s_memtime start, end, s_memrealtime start, end per wave); sink: int
// [cus * wps * 256]. Returns 0, or 1 for bad arguments, or 2 for a HIP error.
int qimg_probe_mfma(int kind, int wps, int cus, int iters, uint64_t* clocks, int* sink, void* stream) {
    if (kind < KIND_I8_32 || kind > KIND_F16_16 || (wps != 1 && wps != 2) || cus < 1 || iters < 1 ||
        clocks == nullptr || sink == nullptr)
        return 1;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e;
    switch (kind) {
        case KIND_I8_32: e = launch<KIND_I8_32>(wps, cus, iters, clocks, sink, s); break;
        case KIND_I8_16: e = launch<KIND_I8_16>(wps, cus, iters, clocks, sink, s); break;
        case KIND_F8_32: e = launch<KIND_F8_32>(wps, cus, iters, clocks, sink, s); break;
        case KIND_F16_32: e = launch<KIND_F16_32>(wps, cus, iters, clocks, sink, s); break;
        case KIND_F8_16: e = launch<KIND_F8_16>(wps, cus, iters, clocks, sink, s); break;
        case KIND_F16_16: e = launch<KIND_F16_16>(wps, cus, iters, clocks, sink, s); break;
        case KIND_BF16_32: e = launch<KIND_BF16_32>(wps, cus, iters, clocks, sink, s); break;
        default: return 1;
    }
    return e == hipSuccess ? 0 : 2;
}

}  // extern "C"
