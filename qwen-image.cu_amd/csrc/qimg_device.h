// qimg_device.h — device-side helpers shared by the gfx950 kernels:
// element conversions with explicit rounding, wave-64 reductions, and
// small vector types for 16-byte memory traffic.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qimg {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round-to-nearest-even fp32 -> bf16 bits (NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
    _Float16 x;
    __builtin_memcpy(&x, &h, 2);
    return static_cast<float>(x);
}

// fp32 -> fp16 bits with the IEEE default rounding (nearest even).
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
    _Float16 x = static_cast<_Float16>(f);
    uint16_t h;
    __builtin_memcpy(&h, &x, 2);
    return h;
}

// Saturating round-half-to-even to int8 (the reference's
// __float2int_rn + clamp and cvt.rni.sat.s8.f32). NaN maps to 0.
__device__ __forceinline__ int8_t sat_rne_i8(float v) {
    float r = __builtin_rintf(v);
    r = fminf(fmaxf(r, -128.0f), 127.0f);
    return static_cast<int8_t>(static_cast<int>(r));
}

// Four fp32 values -> saturating round-half-to-even int8 bytes (a in the
// low byte), the same values as sat_rne_i8 on each: clamp to [-128, 127]
// (v_med3_f32; clamping first gives the same integer as rounding first),
// add 1.5 * 2^23 so the addition rounds to an integer (ulp 1) and the low
// mantissa byte is its two's-complement byte, then gather the four low
// bytes with v_perm_b32. NaN gives 0.
__device__ __forceinline__ uint32_t i8x4_rne_sat(float a, float b, float c, float d) {
    constexpr float kRound = 12582912.0f;  // 1.5 * 2^23
    const uint32_t ra = __float_as_uint(__builtin_amdgcn_fmed3f(a, -128.0f, 127.0f) + kRound);
    const uint32_t rb = __float_as_uint(__builtin_amdgcn_fmed3f(b, -128.0f, 127.0f) + kRound);
    const uint32_t rc = __float_as_uint(__builtin_amdgcn_fmed3f(c, -128.0f, 127.0f) + kRound);
    const uint32_t rd = __float_as_uint(__builtin_amdgcn_fmed3f(d, -128.0f, 127.0f) + kRound);
    // v_perm_b32(s0, s1, sel): byte i = byte sel_i of {s1 (0-3), s0 (4-7)}, 0x0c -> 0
    const uint32_t ab = __builtin_amdgcn_perm(rb, ra, 0x0c0c0400u);
    const uint32_t cd = __builtin_amdgcn_perm(rd, rc, 0x0c0c0400u);
    return __builtin_amdgcn_perm(cd, ab, 0x05040100u);
}

// Four fp32 values -> OCP E4M3FN bytes (a in the low byte) with
// v_cvt_pk_fp8_f32: round to nearest even, subnormals kept (quantum 2^-9).
// The quantizers call it on values already scaled to |v| <= 448 (plus one
// rounding, which still rounds to 448), so no input reaches the NaN code.
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
    return static_cast<uint32_t>(w);
}

// Address-space pointer types of the global -> LDS DMA builtin
// (global_load_lds_dwordx4: each lane's 16 bytes land at the LDS base
// + 16 * lane).
typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef const __attribute__((address_space(1))) void* gbl_ptr_t;

// XOR swizzle of the four 16-byte chunks of a 64-byte LDS row: chunk c of
// row r is stored at physical chunk c ^ swz_row(r), so 16-byte fragment reads
// of 8 consecutive rows at one logical chunk hit distinct banks.
__device__ __forceinline__ int swz_row(int row) { return ((row >> 1) ^ (row >> 3)) & 3; }

// s_waitcnt lgkmcnt(0), the other counters left alone.
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xc07f); }

// s_waitcnt with vmcnt = n (0..63) and the other counters left alone.
template <int n>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(n >= 0 && n < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((0x0f70 & ~0xc00f) | (n & 15) | ((n >> 4) << 14));
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

template <typename T>
__device__ __forceinline__ T wave_max(T v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
    return v;
}

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// Wave64 all-reduce without LDS round trips: DPP quad_perm [1,0,3,2] and
// [2,3,0,1] (pairs, quads), row_half_mirror (lane i with 7-i: 8 lanes),
// row_mirror (i with 15-i: a row of 16), v_permlane16_swap (rows 0+1, 2+3)
// and v_permlane32_swap (the two halves). Every lane ends with the same
// value (each step combines two partial results in either order).
template <int CTRL, typename T>
__device__ __forceinline__ T dpp32(T v) {
    static_assert(sizeof(T) == 4, "32-bit lanes");
    return __builtin_bit_cast(T, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
template <typename T, typename Op>
__device__ __forceinline__ T wave_reduce_dpp(T v, Op op) {
    v = op(v, dpp32<0xB1>(v));   // quad_perm:[1,0,3,2]
    v = op(v, dpp32<0x4E>(v));   // quad_perm:[2,3,0,1]
    v = op(v, dpp32<0x141>(v));  // row_half_mirror
    v = op(v, dpp32<0x140>(v));  // row_mirror
    {
        const unsigned u = __builtin_bit_cast(unsigned, v);
        const auto sw = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        v = op(__builtin_bit_cast(T, static_cast<unsigned>(sw[0])), __builtin_bit_cast(T, static_cast<unsigned>(sw[1])));
    }
    {
        const unsigned u = __builtin_bit_cast(unsigned, v);
        const auto sw = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        v = op(__builtin_bit_cast(T, static_cast<unsigned>(sw[0])), __builtin_bit_cast(T, static_cast<unsigned>(sw[1])));
    }
    return v;
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
    return wave_reduce_dpp(v, [](float a, float b) { return a + b; });
}
__device__ __forceinline__ int wave_sum_dpp(int v) {
    return wave_reduce_dpp(v, [](int a, int b) { return a + b; });
}
__device__ __forceinline__ float wave_max_dpp(float v) {
    return wave_reduce_dpp(v, [](float a, float b) { return fmaxf(a, b); });
}

// Two fp32 values -> packed bf16x2 bits with the hardware RNE conversion
// (v_cvt_pk_bf16_f32); same result as f32_to_bf16 on each.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    typedef float f2 __attribute__((ext_vector_type(2)));
    const f2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf2));
}

// GELU-tanh, 0.5 v (1 + tanh(u)) with u = sqrt(2/pi) (v + 0.044715 v^3),
// written as v - v / (exp(2u) + 1) (since 0.5 (1 + tanh u) = 1 - 1/(e^2u + 1))
// with 2u log2(e) = v (C1 + C2 v^2): five full-rate operations and the
// hardware exp2 / rcp (about 2e-7 absolute error in tanh; the reference
// evaluates tanhf under fast-math approximation as well).
__device__ __forceinline__ float gelu_tanh_fast(float v) {
    constexpr float C1 = 2.3022082f;    // 2 sqrt(2/pi) log2(e)
    constexpr float C2 = 0.10294324f;   // C1 * 0.044715
    const float x = v * __builtin_fmaf(C2, v * v, C1);
    const float r = __builtin_amdgcn_rcpf(__builtin_amdgcn_exp2f(x) + 1.0f);
    return __builtin_fmaf(-v, r, v);
}

__device__ __forceinline__ float gelu_tanh(float v) {
    const float c = 0.7978845608f;
    float inner = c * (v + 0.044715f * v * v * v);
    return 0.5f * v * (1.0f + tanhf(inner));
}

// Dequant epilogue of one output element, in the reference's order
// (cuda_kernels.cu:2623-2668): acc * act_scale * w_scale, then + bias, each
// step rounded (no contraction), then GELU-tanh.
template <bool GELU>
__device__ __forceinline__ float dequant_elem(float acc, float sa, float sw, bool has_bias, float b) {
    float t;
    {
#pragma clang fp contract(off)
        t = acc * sa * sw;
        if (has_bias) t = t + b;
    }
    if (GELU) t = gelu_tanh_fast(t);
    return t;
}


// ---- LayerNorm + modulate of one row (layer_norm_modulate_fp32_kernel,
// cuda_kernels.cu:1799-1853): mean, then the variance about it,
// inv_std = rsqrt(var/dim + eps), out = (x - mean) * inv_std * (1 + scale)
// + shift. A workgroup of LN_THR threads owns the row, held in registers
// between the passes (float4 chunk c = tid + j * LN_THR); emit(c, v) receives
// each modulated chunk. Every kernel that normalizes a row calls this, so
// the reduction order, and the result, is the same in all of them.
constexpr int LN_THR = 256;
constexpr int LN_MAXV = 4;  // float4 chunks per thread
constexpr int LN_MAX_DIM = LN_THR * 4 * LN_MAXV;

__device__ __forceinline__ float ln_block_sum(float v, float* red) {
    v = wave_sum_dpp(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();  // red may still be read by a previous call
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < LN_THR / 64; ++w) t += red[w];
    return t;
}

template <class Emit>
__device__ __forceinline__ void ln_modulate_row(const float* __restrict__ xrow, const float* __restrict__ shift,
                                                const float* __restrict__ scale, int dim, float eps, float* red,
                                                Emit emit) {
#pragma clang fp contract(off)
    const v4f* xr = reinterpret_cast<const v4f*>(xrow);
    const int nv = dim >> 2;
    v4f v[LN_MAXV];
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < LN_MAXV; ++j) {
        const int c = threadIdx.x + j * LN_THR;
        v[j] = c < nv ? xr[c] : (v4f){0.0f, 0.0f, 0.0f, 0.0f};
        s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
    }
    const float mean = ln_block_sum(s, red) / dim;
    float q = 0.0f;
#pragma unroll
    for (int j = 0; j < LN_MAXV; ++j) {
        const int c = threadIdx.x + j * LN_THR;
        if (c < nv) {
            const v4f d = v[j] - mean;
            q += (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w);
        }
    }
    const float inv_std = rsqrtf(ln_block_sum(q, red) / dim + eps);
    const v4f* sh = reinterpret_cast<const v4f*>(shift);
    const v4f* sc = reinterpret_cast<const v4f*>(scale);
#pragma unroll
    for (int j = 0; j < LN_MAXV; ++j) {
        const int c = threadIdx.x + j * LN_THR;
        if (c < nv) emit(c, (v[j] - mean) * inv_std * (1.0f + sc[c]) + sh[c]);
    }
}

}  // namespace qimg
