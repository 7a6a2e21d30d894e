// hadamard_quant.hip — fused block-diagonal Walsh-Hadamard transform +
// per-row quantization for gfx950.
//
// Semantics follow qwen-image.cu:
//   fwht_inplace_kernel        cuda_kernels.cu:2209-2254   (weights, in place)
//   quantize_per_row_fp32      cuda_kernels.cu:2385-2416
//   fwht_quantize_kernel<T>    cuda_kernels.cu:2493-2577   (activations)
//   quantize_weight_tensor     cuda_kernels.cu:2830-2862
// Every output element sees the same fp32 operation sequence as the
// reference: butterfly stages half = 1, 2, ..., hbs/2 in that order with
// (a, b) <- (a + b, a - b), then one multiply by 1/sqrt(hbs). The
// reference runs each stage as a separate shared-memory sweep; here a
// thread applies up to four consecutive stages to 16 elements held in
// registers (a radix-16 pass), so a 1024-point transform takes three LDS
// sweeps instead of ten, and the first sweep comes straight from the
// global load. The per-element arithmetic, and therefore the result, is
// unchanged.
//
// One workgroup owns one row: the row lives in LDS (K fp32 plus one pad
// word per 16, which makes the strided radix passes bank-conflict free).
#include "qimg_device.h"
#include "qimg_internal.h"

namespace qimg {

enum class RowOut { Int8 = 0, Fp8 = 1, Fp32 = 2, Bf16 = 3 };

__device__ __forceinline__ int lds_pad(int i) { return i + (i >> 4); }

// Butterfly stages on a register array: stage s pairs v[i], v[i + 2^s].
template <int RB>
__device__ __forceinline__ void butterfly(float* v) {
    constexpr int R = 1 << RB;
#pragma unroll
    for (int s = 0; s < RB; ++s) {
        const int h = 1 << s;
#pragma unroll
        for (int i = 0; i < R; ++i) {
            if ((i & h) == 0) {
                float a = v[i];
                float b = v[i + h];
                v[i] = a + b;
                v[i + h] = a - b;
            }
        }
    }
}

// One radix-2^RB sweep over the row in LDS covering bits [lo, lo + RB) of
// the index inside each Hadamard block.
template <int RB>
__device__ __forceinline__ void lds_pass(float* lds, int K, int lo, bool last, float norm,
                                         float& amax) {
    constexpr int R = 1 << RB;
    const int ngroups = K >> RB;
    const int lomask = (1 << lo) - 1;
    for (int g = threadIdx.x; g < ngroups; g += blockDim.x) {
        const int base = (g & lomask) + ((g >> lo) << (lo + RB));
        float v[R];
#pragma unroll
        for (int i = 0; i < R; ++i) v[i] = lds[lds_pad(base + (i << lo))];
        butterfly<RB>(v);
        if (last) {
#pragma unroll
            for (int i = 0; i < R; ++i) {
                v[i] = v[i] * norm;
                amax = fmaxf(amax, fabsf(v[i]));
            }
        }
#pragma unroll
        for (int i = 0; i < R; ++i) lds[lds_pad(base + (i << lo))] = v[i];
    }
}

__device__ __forceinline__ void lds_pass_dispatch(int rb, float* lds, int K, int lo, bool last,
                                                  float norm, float& amax) {
    switch (rb) {
        case 1: lds_pass<1>(lds, K, lo, last, norm, amax); break;
        case 2: lds_pass<2>(lds, K, lo, last, norm, amax); break;
        case 3: lds_pass<3>(lds, K, lo, last, norm, amax); break;
        default: lds_pass<4>(lds, K, lo, last, norm, amax); break;
    }
}

template <typename InT>
__device__ __forceinline__ void load16(const InT* p, float* v);

template <>
__device__ __forceinline__ void load16<float>(const float* p, float* v) {
    const v4f* q = reinterpret_cast<const v4f*>(p);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        v4f t = q[j];
        v[4 * j + 0] = t.x; v[4 * j + 1] = t.y; v[4 * j + 2] = t.z; v[4 * j + 3] = t.w;
    }
}

template <>
__device__ __forceinline__ void load16<uint16_t>(const uint16_t* p, float* v) {
    const u32x4* q = reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        u32x4 t = q[j];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            v[8 * j + 2 * c + 0] = __uint_as_float(t[c] << 16);
            v[8 * j + 2 * c + 1] = __uint_as_float(t[c] & 0xffff0000u);
        }
    }
}

template <typename InT>
__device__ __forceinline__ float load1(const InT* p);
template <>
__device__ __forceinline__ float load1<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float load1<uint16_t>(const uint16_t* p) { return bf16_to_f32(*p); }

// The remaining butterfly stages (from bit `lo`) on the row in LDS, then the
// row's output: fp32 as is, or per-row scale amax/QMAX and int8/e4m3 values.
template <RowOut OUT>
__device__ __forceinline__ void fwht_quant_tail(float* lds, float* red, int K, int hbs_log2, float norm, int lo,
                                                float amax, void* out, float* __restrict__ scales, int row) {
    const int tid = threadIdx.x;
    const int nthr = blockDim.x;
    while (lo < hbs_log2) {
        const int rem = hbs_log2 - lo;
        const int rb = rem >= 8 ? 4 : (rem > 4 ? (rem + 1) / 2 : rem);
        const bool last = (lo + rb == hbs_log2);
        lds_pass_dispatch(rb, lds, K, lo, last, norm, amax);
        lo += rb;
        __syncthreads();
    }

    if constexpr (OUT == RowOut::Fp32) {
        float* o = reinterpret_cast<float*>(out) + static_cast<int64_t>(row) * K;
        for (int i = tid; i < K; i += nthr) o[i] = lds[lds_pad(i)];
        return;
    } else if constexpr (OUT == RowOut::Bf16) {
        uint16_t* o = reinterpret_cast<uint16_t*>(out) + static_cast<int64_t>(row) * K;
        for (int i = tid; i < K; i += nthr) o[i] = f32_to_bf16(lds[lds_pad(i)]);
        return;
    } else {
        amax = wave_max_dpp(amax);
        if ((tid & (kWave - 1)) == 0) red[tid / kWave] = amax;
        __syncthreads();
        amax = red[0];
        for (int w = 1; w < nthr / kWave; ++w) amax = fmaxf(amax, red[w]);
        constexpr float QMAX = (OUT == RowOut::Int8) ? 127.0f : 448.0f;
        if (tid == 0) scales[row] = amax / QMAX;
        const float inv = (amax > 0.0f) ? QMAX / amax : 0.0f;

        uint8_t* o = reinterpret_cast<uint8_t*>(out) + static_cast<int64_t>(row) * K;
        if ((K & 15) == 0) {
            for (int c = tid; c < (K >> 4); c += nthr) {
                u32x4 pk;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    float v[4];
#pragma unroll
                    for (int b = 0; b < 4; ++b) v[b] = lds[lds_pad(16 * c + 4 * w + b)] * inv;
                    uint32_t word = 0;
                    if constexpr (OUT == RowOut::Int8) {
                        word = i8x4_rne_sat(v[0], v[1], v[2], v[3]);
                    } else {
                        word = e4m3x4(v[0], v[1], v[2], v[3]);
                    }
                    pk[w] = word;
                }
                *reinterpret_cast<u32x4*>(o + 16 * c) = pk;
            }
        } else {
            for (int i = tid; i < K; i += nthr) {
                float v = lds[lds_pad(i)] * inv;
                if constexpr (OUT == RowOut::Int8)
                    o[i] = static_cast<uint8_t>(sat_rne_i8(v));
                else
                    o[i] = static_cast<uint8_t>(e4m3x4(v, 0.0f, 0.0f, 0.0f) & 0xffu);
            }
        }
    }
}

// grid.x = rows, blockDim.x = 64..256 (multiple of 64).
// hbs_log2 = log2(hbs) (0 = no transform). K % 16 == 0 and hbs >= 16 take
// the vector path (first 4 stages in registers straight from global).
// RPT: chunks a thread loads before transforming them (4 when a row has
// more 16-value chunks than the workgroup has threads, else 1).
template <typename InT, RowOut OUT, int RPT>
__global__ __launch_bounds__(256) void fwht_quant_rows_kernel(
    const InT* x, void* out, float* __restrict__ scales, int M, int K,
    int hbs_log2, float norm) {
    extern __shared__ float lds[];
    float* red = lds + lds_pad(K) + 1;  // 4 floats for the cross-wave max
    const int row = blockIdx.x;
    if (row >= M) return;
    const InT* xin = x + static_cast<int64_t>(row) * K;
    const int tid = threadIdx.x;
    const int nthr = blockDim.x;

    const bool vec = (hbs_log2 >= 4) && ((K & 15) == 0);
    float amax = 0.0f;
    int lo;  // first stage bit still to do

    if (vec) {
        const bool only = (hbs_log2 == 4);
        // up to RPT chunks per thread per pass, all loads issued before the
        // first transform (a K = 12288 row is 3 chunks per thread)
        const int nch = K >> 4;
        for (int c0 = tid; c0 < nch; c0 += RPT * nthr) {
            float v[RPT][16];
#pragma unroll
            for (int j = 0; j < RPT; ++j)
                if (c0 + j * nthr < nch) load16<InT>(xin + 16 * (c0 + j * nthr), v[j]);
#pragma unroll
            for (int j = 0; j < RPT; ++j) {
                const int c = c0 + j * nthr;
                if (c < nch) {
                    butterfly<4>(v[j]);
                    if (only) {
#pragma unroll
                        for (int i = 0; i < 16; ++i) {
                            v[j][i] = v[j][i] * norm;
                            amax = fmaxf(amax, fabsf(v[j][i]));
                        }
                    }
#pragma unroll
                    for (int i = 0; i < 16; ++i) lds[lds_pad(16 * c + i)] = v[j][i];
                }
            }
        }
        lo = 4;
    } else {
        for (int i = tid; i < K; i += nthr) {
            float v = load1<InT>(xin + i);
            if (hbs_log2 == 0) amax = fmaxf(amax, fabsf(v));
            lds[lds_pad(i)] = v;
        }
        lo = 0;
    }
    __syncthreads();

    fwht_quant_tail<OUT>(lds, red, K, hbs_log2, norm, lo, amax, out, scales, row);
}

// Rows of NB Hadamard blocks of 4096 values (e.g. the fc2 input, K = 12288
// = 3 x 4096), 256 threads. The blocks go through one block-sized LDS
// buffer in turn (17 KB instead of the whole row's 52 KB, so twice as many
// rows are in flight per CU). Per block: thread t transforms its chunk t
// (16 consecutive values, stages 1-8) in registers straight from the load,
// one LDS sweep does stages 16-128, and the last sweep (stages 256-2048)
// leaves thread t holding values t + 256 i, i < 16, in registers until the
// row's absmax is known; the quantized bytes are stored from there (each
// store instruction writes 64 consecutive bytes per wave). Each value sees
// the same butterfly stages in the same order as in fwht_quant_rows_kernel.
// GELU_IN: each loaded value v is first replaced by gelu_tanh_fast(v), the
// GELU of the linear epilogue (the fc1 -> fc2 hop with the GELU applied by
// the consumer: the same function of the same fp32 value, so the same bits).
template <typename InT, RowOut OUT, int NB, bool GELU_IN = false>
__global__ __launch_bounds__(256) void fwht_quant_blocks_kernel(const InT* x, void* out, float* __restrict__ scales,
                                                                int M, int K, float norm) {
    constexpr int HBS = 4096;
    extern __shared__ float lds[];
    float* red = lds + lds_pad(HBS) + 1;
    const int row = blockIdx.x;
    if (row >= M) return;
    const InT* xin = x + static_cast<int64_t>(row) * K;
    const int tid = threadIdx.x;

    float v[NB][16];
#pragma unroll
    for (int b = 0; b < NB; ++b) load16<InT>(xin + b * HBS + 16 * tid, v[b]);
    if constexpr (GELU_IN) {
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int i = 0; i < 16; ++i) v[b][i] = gelu_tanh_fast(v[b][i]);
    }
    float amax = 0.0f;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        butterfly<4>(v[b]);
#pragma unroll
        for (int i = 0; i < 16; ++i) lds[lds_pad(16 * tid + i)] = v[b][i];
        __syncthreads();
        lds_pass<4>(lds, HBS, 4, false, norm, amax);
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 16; ++i) v[b][i] = lds[lds_pad(tid + (i << 8))];
        butterfly<4>(v[b]);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            v[b][i] = v[b][i] * norm;
            amax = fmaxf(amax, fabsf(v[b][i]));
        }
        __syncthreads();  // the next block's chunks overwrite the buffer
    }

    amax = wave_max_dpp(amax);
    if ((tid & (kWave - 1)) == 0) red[tid / kWave] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    constexpr float QMAX = (OUT == RowOut::Int8) ? 127.0f : 448.0f;
    if (tid == 0) scales[row] = amax / QMAX;
    const float inv = (amax > 0.0f) ? QMAX / amax : 0.0f;
    uint8_t* o = reinterpret_cast<uint8_t*>(out) + static_cast<int64_t>(row) * K + tid;
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < 16; i += 4) {
            // four values 256 apart converted together, stored byte by byte
            const float q0 = v[b][i] * inv, q1 = v[b][i + 1] * inv;
            const float q2 = v[b][i + 2] * inv, q3 = v[b][i + 3] * inv;
            uint32_t w;
            if constexpr (OUT == RowOut::Int8)
                w = i8x4_rne_sat(q0, q1, q2, q3);
            else
                w = e4m3x4(q0, q1, q2, q3);
#pragma unroll
            for (int c = 0; c < 4; ++c) o[b * HBS + ((i + c) << 8)] = static_cast<uint8_t>(w >> (8 * c));
        }
}

// LDS operations of one wave complete in order; this keeps the compiler
// from moving a read of another lane's value above the write.
__device__ __forceinline__ void wave_lds_order() {
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
}

// Rows of NB Hadamard blocks of 1024 values (K = 3072 linear inputs), one
// wave per row and four rows per workgroup: with 4352 rows the whole
// problem is about one round of rows, so the time is one row's latency, and
// a wave-private row needs no workgroup barrier. Lane l transforms chunk l
// (16 consecutive values) of each block in registers straight from the load
// (stages 1-8), one radix-16 sweep through the wave's LDS buffer does
// stages 16-128, and the last radix-4 sweep (stages 256, 512) leaves lane l
// holding values l + 64 q + 256 i (q, i < 4) in registers until the row's
// absmax is known. Each value sees the same butterfly stages in the same
// order as in fwht_quant_rows_kernel.
// Where a row's 16-value chunk c comes from. fetch() issues the loads into
// raw registers, unpack() turns them into fp32 once they are needed, so that
// a wave can have its next row in flight while it transforms this one.
// A row-major [M, K] matrix ...
template <typename InT>
struct RowsLoader;
template <>
struct RowsLoader<float> {
    static constexpr bool kWholeRow = false;
    typedef v4f Raw[4];
    const float* x;
    int K;
    __device__ __forceinline__ void fetch(int row, int c, Raw& r) const {
        const v4f* q = reinterpret_cast<const v4f*>(x + static_cast<int64_t>(row) * K + 16 * c);
#pragma unroll
        for (int j = 0; j < 4; ++j) r[j] = q[j];
    }
    __device__ __forceinline__ static void unpack(const Raw& r, float* v) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[4 * j + 0] = r[j].x; v[4 * j + 1] = r[j].y; v[4 * j + 2] = r[j].z; v[4 * j + 3] = r[j].w;
        }
    }
};
template <>
struct RowsLoader<uint16_t> {  // bf16
    static constexpr bool kWholeRow = false;
    typedef u32x4 Raw[2];
    const uint16_t* x;
    int K;
    __device__ __forceinline__ void fetch(int row, int c, Raw& r) const {
        const u32x4* q = reinterpret_cast<const u32x4*>(x + static_cast<int64_t>(row) * K + 16 * c);
        r[0] = q[0];
        r[1] = q[1];
    }
    __device__ __forceinline__ static void unpack(const Raw& r, float* v) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                v[8 * j + 2 * c + 0] = __uint_as_float(r[j][c] << 16);
                v[8 * j + 2 * c + 1] = __uint_as_float(r[j][c] & 0xffff0000u);
            }
    }
};
// ... or the fp16 attention output [batch][H][S][128], read as the rows of
// the out-projection's input (token s of sequence b: head h = c / 8, dims
// 16 (c % 8) .. +16; the rows are tokens s0 .. s0 + n - 1 of each sequence).
struct HeadsLoader {
    static constexpr bool kWholeRow = false;
    typedef u32x4 Raw[2];
    const uint16_t* attn;
    int S, H, s0, n;
    __device__ __forceinline__ void fetch(int row, int c, Raw& r) const {
        const int b = row / n;
        const int s = s0 + row - b * n;
        const uint16_t* src = attn + ((static_cast<int64_t>(b) * H + (c >> 3)) * S + s) * 128 + 16 * (c & 7);
        const u32x4* q = reinterpret_cast<const u32x4*>(src);
        r[0] = q[0];
        r[1] = q[1];
    }
    __device__ __forceinline__ static void unpack(const Raw& r, float* v) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[8 * j + 2 * e] = f16_to_f32(static_cast<uint16_t>(r[j][e] & 0xffffu));
                v[8 * j + 2 * e + 1] = f16_to_f32(static_cast<uint16_t>(r[j][e] >> 16));
            }
    }
};

// The 16-lane rows of a wave reduced with the first four levels of
// wave_reduce_dpp (pairs, quads, eights, sixteens of lanes).
__device__ __forceinline__ float row16_sum_dpp(float v) {
    v = v + dpp32<0xB1>(v);
    v = v + dpp32<0x4E>(v);
    v = v + dpp32<0x141>(v);
    v = v + dpp32<0x140>(v);
    return v;
}

// ... or the LayerNorm + modulate of a row-major fp32 [M, K] matrix
// (K = 1024 NB), normalized as a whole row (finish_row) before the
// transform. The arithmetic is ln_modulate_row's, in its order: its thread
// t = 4 lane + e holds float4 chunks t + 256 j, which are quarter e of this
// lane's 16-value chunk j, so each lane keeps that thread's partial sums for
// e = 0..3 (the same loop, including the zero chunks up to LN_MAXV). Its
// reduction tree over 64 lanes is, level by level, the two lowest levels
// inside this lane and the next four across this wave's 16-lane row w
// (which stands for its wave w); the four row totals are then added in
// order from zero, as its wave totals are.
struct LnLoader : RowsLoader<float> {
    static constexpr bool kWholeRow = true;
    const float* shift;
    const float* scale;
    float eps;
    __device__ __forceinline__ static float total(float part) {
        const float r = row16_sum_dpp(part);
        float t = 0.0f;
#pragma unroll
        for (int w = 0; w < LN_THR / 64; ++w)
            t += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, r), 16 * w));
        return t;
    }
    template <int NB>
    __device__ __forceinline__ void finish_row(int /*row*/, int lane, float (&v)[NB][16]) const {
        finish_row_get<NB>(lane, v, [&](int j, int e, v4f& sh, v4f& sc) {
            sh = reinterpret_cast<const v4f*>(shift + j * 1024 + 16 * lane)[e];
            sc = reinterpret_cast<const v4f*>(scale + j * 1024 + 16 * lane)[e];
        });
    }
    // (get(j, e, sh, sc) gives float4 e of the lane's chunk j of shift and
    // scale)
    template <int NB, typename Get>
    __device__ __forceinline__ void finish_row_get(int lane, float (&v)[NB][16], Get get) const {
#pragma clang fp contract(off)
        static_assert(NB <= LN_MAXV && LN_THR == 256, "ln_modulate_row's thread layout");
        float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < LN_MAXV; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (j < NB)
                    s[e] += (v[j][4 * e] + v[j][4 * e + 1]) + (v[j][4 * e + 2] + v[j][4 * e + 3]);
                else
                    s[e] += 0.0f;  // a chunk past the row reads as zeros there
            }
        const float mean = total((s[0] + s[1]) + (s[2] + s[3])) / K;
        float q[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const v4f d = (v4f){v[j][4 * e], v[j][4 * e + 1], v[j][4 * e + 2], v[j][4 * e + 3]} - mean;
                q[e] += (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w);
            }
        const float inv_std = rsqrtf(total((q[0] + q[1]) + (q[2] + q[3])) / K + eps);
#pragma unroll
        for (int j = 0; j < NB; ++j) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v4f sh, sc;
                get(j, e, sh, sc);
                const v4f xv = (v4f){v[j][4 * e], v[j][4 * e + 1], v[j][4 * e + 2], v[j][4 * e + 3]};
                const v4f o = (xv - mean) * inv_std * (1.0f + sc) + sh;
                v[j][4 * e] = o.x;
                v[j][4 * e + 1] = o.y;
                v[j][4 * e + 2] = o.z;
                v[j][4 * e + 3] = o.w;
            }
        }
    }
};

// Where row r's quantized values and scale go: a row-major [M, K] output ...
struct RowDest {
    void* out;
    float* scales;
    __device__ __forceinline__ uint8_t* row_out(int r, int K) const {
        return reinterpret_cast<uint8_t*>(out) + static_cast<int64_t>(r) * K;
    }
    __device__ __forceinline__ float* scale(int r) const { return scales + r; }
};

// ... or two of them, rows [0, Ma) to the first and the rest to the second
// (with PairLoader: the image and text rows of a joint block in one launch,
// so that the few text rows' latency hides behind the image rows).
struct PairDest {
    RowDest a, b;
    int Ma;
    __device__ __forceinline__ uint8_t* row_out(int r, int K) const {
        return r < Ma ? a.row_out(r, K) : b.row_out(r - Ma, K);
    }
    __device__ __forceinline__ float* scale(int r) const { return r < Ma ? a.scale(r) : b.scale(r - Ma); }
};
template <typename L>
struct PairLoader {
    static constexpr bool kWholeRow = L::kWholeRow;
    typedef typename L::Raw Raw;
    L a, b;
    int Ma;
    // (one copy of the segment's code, on the selected operands)
    __device__ __forceinline__ void fetch(int row, int c, Raw& r) const {
        const L& l = row < Ma ? a : b;
        l.fetch(row < Ma ? row : row - Ma, c, r);
    }
    __device__ __forceinline__ static void unpack(const Raw& r, float* v) { L::unpack(r, v); }
    template <int NB>
    __device__ __forceinline__ void finish_row(int row, int lane, float (&v)[NB][16]) const {
        const L& l = row < Ma ? a : b;
        l.template finish_row<NB>(row < Ma ? row : row - Ma, lane, v);
    }
};

// The transform, absmax and quantized store of one row held as lane l's
// 16-value chunk l of each of the NB blocks (v), through the wave's LDS
// buffer (lds, HBS + HBS / 16 floats).
template <RowOut OUT, int NB, typename Dest>
__device__ __forceinline__ void wave_row_fwht_quant_store(float (&v)[NB][16], float* lds, int lane, int row, int K,
                                                          float norm, const Dest& dst) {
    constexpr int HBS = 1024;
    float amax = 0.0f;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        butterfly<4>(v[b]);
#pragma unroll
        for (int i = 0; i < 16; ++i) lds[lds_pad(16 * lane + i)] = v[b][i];
        wave_lds_order();
        // stages 16-128: group lane = elements base + 16 i
        {
            const int base = (lane & 15) + ((lane >> 4) << 8);
            float t[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) t[i] = lds[lds_pad(base + (i << 4))];
            butterfly<4>(t);
#pragma unroll
            for (int i = 0; i < 16; ++i) lds[lds_pad(base + (i << 4))] = t[i];
        }
        wave_lds_order();
        // stages 256, 512: groups lane + 64 q = elements (lane + 64 q) + 256 i
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float t[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) t[i] = lds[lds_pad(lane + 64 * q + 256 * i)];
            butterfly<2>(t);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[b][4 * q + i] = t[i] * norm;
                amax = fmaxf(amax, fabsf(v[b][4 * q + i]));
            }
        }
        wave_lds_order();  // the next block's chunks overwrite the buffer
    }
    amax = wave_max_dpp(amax);
    constexpr float QMAX = (OUT == RowOut::Int8) ? 127.0f : 448.0f;
    if (lane == 0) *dst.scale(row) = amax / QMAX;
    const float inv = (amax > 0.0f) ? QMAX / amax : 0.0f;
    uint8_t* o = dst.row_out(row, K) + lane;
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // four values 64 apart (q = 0..3) converted together
            const float q0 = v[b][i] * inv, q1 = v[b][4 + i] * inv, q2 = v[b][8 + i] * inv,
                        q3 = v[b][12 + i] * inv;
            uint32_t w;
            if constexpr (OUT == RowOut::Int8)
                w = i8x4_rne_sat(q0, q1, q2, q3);
            else
                w = e4m3x4(q0, q1, q2, q3);
#pragma unroll
            for (int c = 0; c < 4; ++c) o[b * HBS + 64 * c + 256 * i] = static_cast<uint8_t>(w >> (8 * c));
        }
}

template <typename Loader, RowOut OUT, int NB, typename Dest>
__global__ __launch_bounds__(256) void fwht_quant_wave_rows_kernel(Loader ld, Dest dst, int M, int K, float norm) {
    constexpr int HBS = 1024;
    constexpr int PADDED = HBS + HBS / 16;
    __shared__ float lds_all[4 * PADDED];
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + wave;
    if (row >= M) return;  // whole waves: no barrier below
    float* lds = lds_all + wave * PADDED;

    typename Loader::Raw raw[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) ld.fetch(row, b * (HBS / 16) + lane, raw[b]);
    float v[NB][16];
#pragma unroll
    for (int b = 0; b < NB; ++b) Loader::unpack(raw[b], v[b]);
    if constexpr (Loader::kWholeRow) ld.template finish_row<NB>(row, lane, v);
    wave_row_fwht_quant_store<OUT, NB>(v, lds, lane, row, K, norm, dst);
}

// LayerNorm + modulate + FWHT quant rows as above, eight rows (waves) per
// workgroup sharing the modulation vectors: the workgroup stages the shift
// and scale of its first row's stream in LDS once, instead of every wave
// reading its 2 K floats from L2 (at 4352 rows those reads were twice the
// activation bytes, and replacing them by constants made the kernel 22%
// faster). A wave whose row belongs to the other stream (only in the
// workgroup that straddles the two) reads them from global memory. Every
// wave reaches the one barrier before a wave past M leaves.
// (LDS chunk c of the staged vectors is stored at c ^ ((c >> 4) & 3): the
// 16 lanes of a ds_read_b128 read chunks 4 l + e, which lands them on 16
// different bank groups; the staging writes stay conflict-free too.)
__device__ __forceinline__ int ln_vec_swz(int c) { return c ^ ((c >> 4) & 3); }

template <RowOut OUT, int NB>
__global__ __launch_bounds__(512) void ln_fwht_quant_rows8_kernel(PairLoader<LnLoader> ld, PairDest dst, int M,
                                                                  float norm) {
    constexpr int HBS = 1024;
    constexpr int PADDED = HBS + HBS / 16;
    constexpr int K = NB * HBS;
    constexpr int NCH = 2 * K / 4;               // 16-byte chunks of shift, then scale
    constexpr int PER = (NCH + 511) / 512;       // chunks staged by each thread
    __shared__ float lds_all[8 * PADDED];
    __shared__ __attribute__((aligned(16))) float lds_vec[2 * K];
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int row0 = blockIdx.x * 8;  // < M
    const int row = row0 + wave;
    const bool active = row < M;
    const bool staged_a = row0 < ld.Ma;
    const LnLoader& ls = staged_a ? ld.a : ld.b;

    // the staged vectors' loads first, then the row's (a wave past M loads
    // row M - 1 and drops it)
    v4f stg[PER];
#pragma unroll
    for (int t = 0; t < PER; ++t) {
        const int ci = threadIdx.x + 512 * t;
        if (ci < NCH)
            stg[t] = ci < K / 4 ? reinterpret_cast<const v4f*>(ls.shift)[ci]
                                : reinterpret_cast<const v4f*>(ls.scale)[ci - K / 4];
    }
    const int rr = active ? row : M - 1;
    typename LnLoader::Raw raw[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) ld.fetch(rr, b * (HBS / 16) + lane, raw[b]);
#pragma unroll
    for (int t = 0; t < PER; ++t) {
        const int ci = threadIdx.x + 512 * t;
        if (ci < NCH) *reinterpret_cast<v4f*>(lds_vec + 4 * ln_vec_swz(ci)) = stg[t];
    }
    __syncthreads();
    if (!active) return;

    float v[NB][16];
#pragma unroll
    for (int b = 0; b < NB; ++b) LnLoader::unpack(raw[b], v[b]);
    const bool in_a = row < ld.Ma;
    if (in_a == staged_a) {
        const LnLoader& l = in_a ? ld.a : ld.b;
        l.finish_row_get<NB>(lane, v, [&](int j, int e, v4f& sh, v4f& sc) {
            const int c = 256 * j + 4 * lane + e;
            sh = *reinterpret_cast<const v4f*>(lds_vec + 4 * ln_vec_swz(c));
            sc = *reinterpret_cast<const v4f*>(lds_vec + 4 * ln_vec_swz(K / 4 + c));
        });
    } else {
        ld.finish_row<NB>(row, lane, v);
    }
    wave_row_fwht_quant_store<OUT, NB>(v, lds_all + wave * PADDED, lane, row, K, norm, dst);
}

template <RowOut OUT>
static hipError_t launch_ln_rows8(const PairLoader<LnLoader>& ld, const PairDest& dst, int M, int K, float norm,
                                  hipStream_t stream) {
    const int blocks = (M + 7) / 8;
    switch (K / 1024) {
        case 1:
            hipLaunchKernelGGL((ln_fwht_quant_rows8_kernel<OUT, 1>), dim3(blocks), dim3(512), 0, stream, ld, dst, M,
                               norm);
            break;
        case 2:
            hipLaunchKernelGGL((ln_fwht_quant_rows8_kernel<OUT, 2>), dim3(blocks), dim3(512), 0, stream, ld, dst, M,
                               norm);
            break;
        case 3:
            hipLaunchKernelGGL((ln_fwht_quant_rows8_kernel<OUT, 3>), dim3(blocks), dim3(512), 0, stream, ld, dst, M,
                               norm);
            break;
        default:
            hipLaunchKernelGGL((ln_fwht_quant_rows8_kernel<OUT, 4>), dim3(blocks), dim3(512), 0, stream, ld, dst, M,
                               norm);
            break;
    }
    return hipGetLastError();
}

// The INT4 linear's input preparation (linear_forward_int4, cuda_kernels.cu:
// 4378-4395 and 4452-4470): v = x / smooth[k] (apply_smooth_div, :2258-2264),
// its bf16 copy for the low-rank branch, and the block FWHT of v for the
// residual (fwht_inplace / smooth_hadamard_inplace, :2209-2254, :2275-2317),
// as bf16 (fp32_to_bf16) or fp32, one row per workgroup in one pass. The row
// is in LDS before anything is written, so xr may be x.
template <RowOut OUT>
__global__ __launch_bounds__(256) void smooth_fwht_rows_kernel(const float* x, const float* __restrict__ smooth,
                                                               uint16_t* __restrict__ xs, void* xr, int K,
                                                               int hbs_log2, float norm) {
    extern __shared__ float lds[];
    float* red = lds + lds_pad(K) + 1;
    const int row = blockIdx.x;
    const int64_t base = static_cast<int64_t>(row) * K;
    for (int i = threadIdx.x; i < K; i += blockDim.x) {
        float v = x[base + i];
        if (smooth != nullptr) v = v / smooth[i];
        if (xs != nullptr) xs[base + i] = f32_to_bf16(v);
        lds[lds_pad(i)] = v;
    }
    __syncthreads();
    fwht_quant_tail<OUT>(lds, red, K, hbs_log2, norm, 0, 0.0f, xr, nullptr, row);
}

template <RowOut OUT>
static hipError_t launch_smooth_fwht(const float* x, const float* smooth, uint16_t* xs, void* xr, int M, int K,
                                     int hbs, hipStream_t stream) {
    if (M == 0 || K == 0) return hipSuccess;
    if (hbs < 1) hbs = 1;
    if ((hbs & (hbs - 1)) != 0 || K % hbs != 0) return hipErrorInvalidValue;
    const size_t lds = sizeof(float) * (static_cast<size_t>(K) + K / 16 + 1 + 8);
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(smooth_fwht_rows_kernel<OUT>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        if (e != hipSuccess) return e;
    }
    int threads = ((K / 4 + kWave - 1) / kWave) * kWave;
    threads = threads < 64 ? 64 : (threads > 256 ? 256 : threads);
    int lg = 0;
    while ((1 << lg) < hbs) ++lg;
    const float norm = static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(hbs)));
    hipLaunchKernelGGL(smooth_fwht_rows_kernel<OUT>, dim3(M), dim3(threads), lds, stream, x, smooth, xs, xr, K, lg,
                       norm);
    return hipGetLastError();
}

hipError_t launch_int4_prep(const float* x, const float* smooth, uint16_t* xs_bf16, uint16_t* xr_bf16, int M, int K,
                            int hbs, hipStream_t stream) {
    return launch_smooth_fwht<RowOut::Bf16>(x, smooth, xs_bf16, xr_bf16, M, K, hbs, stream);
}

hipError_t launch_smooth_fwht_f32(const float* x, const float* smooth, float* out, int M, int K, int hbs,
                                  hipStream_t stream) {
    return launch_smooth_fwht<RowOut::Fp32>(x, smooth, nullptr, out, M, K, hbs, stream);
}

// LayerNorm + modulate (ln_modulate_row) feeding the FWHT + row quant of
// the next linear's input in one pass: the normalized row goes to LDS
// instead of HBM. One LN_THR-thread workgroup per row, K <= LN_MAX_DIM.
// Each element sees the same operations as layernorm_modulate followed by
// fwht_quant_rows_kernel, so the int8/e4m3 values and scales are the same.
template <RowOut OUT>
__global__ __launch_bounds__(LN_THR) void ln_fwht_quant_kernel(const float* __restrict__ x,
                                                               const float* __restrict__ shift,
                                                               const float* __restrict__ scale, float eps,
                                                               void* out, float* __restrict__ scales, int K,
                                                               int hbs_log2, float norm) {
    extern __shared__ float lds[];
    float* red = lds + lds_pad(K) + 1;
    const int row = blockIdx.x;
    const int tid = threadIdx.x;
    ln_modulate_row(x + static_cast<int64_t>(row) * K, shift, scale, K, eps, red, [&](int c, v4f v) {
        lds[lds_pad(4 * c + 0)] = v.x;
        lds[lds_pad(4 * c + 1)] = v.y;
        lds[lds_pad(4 * c + 2)] = v.z;
        lds[lds_pad(4 * c + 3)] = v.w;
    });
    __syncthreads();
    float amax = 0.0f;
    int lo = 0;
    if (hbs_log2 >= 4 && (K & 15) == 0) {
        const bool only = (hbs_log2 == 4);
        for (int c = tid; c < (K >> 4); c += LN_THR) {
            float v[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) v[e] = lds[lds_pad(16 * c + e)];
            butterfly<4>(v);
            if (only) {
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    v[e] = v[e] * norm;
                    amax = fmaxf(amax, fabsf(v[e]));
                }
            }
#pragma unroll
            for (int e = 0; e < 16; ++e) lds[lds_pad(16 * c + e)] = v[e];
        }
        lo = 4;
        __syncthreads();
    } else if (hbs_log2 == 0) {
        for (int e = tid; e < K; e += LN_THR) amax = fmaxf(amax, fabsf(lds[lds_pad(e)]));
    }
    fwht_quant_tail<OUT>(lds, red, K, hbs_log2, norm, lo, amax, out, scales, row);
}

// The attention output fp16 [batch][H][S][128] read as the token rows of
// one stream (transpose_split_fused_fp32, transformer.cu:84-104: sequence b,
// token s0 + r of the joint sequence is row b * n + r), straight into the
// FWHT + row quant of the out-projection input. fp16 -> fp32 is exact, so
// the values are those of the split followed by fwht_quant_rows_kernel.
// K = H * 128, hbs >= 16 (the first four stages run on the 16 values a
// thread loads, as in fwht_quant_rows_kernel).
template <RowOut OUT>
__global__ __launch_bounds__(256) void heads_fwht_quant_kernel(const uint16_t* __restrict__ attn, int S, int H,
                                                               int s0, int n, void* out,
                                                               float* __restrict__ scales, int hbs_log2,
                                                               float norm) {
    extern __shared__ float lds[];
    const int K = H * 128;
    float* red = lds + lds_pad(K) + 1;
    const int row = blockIdx.x;
    const int b = row / n;
    const int s = s0 + row - b * n;
    const int tid = threadIdx.x;
    const bool only = (hbs_log2 == 4);
    float amax = 0.0f;
    for (int c = tid; c < (K >> 4); c += blockDim.x) {
        const int h = c >> 3;
        const uint16_t* src = attn + ((static_cast<int64_t>(b) * H + h) * S + s) * 128 + 16 * (c & 7);
        float v[16];
        const u32x4* q = reinterpret_cast<const u32x4*>(src);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const u32x4 t = q[j];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[8 * j + 2 * e] = f16_to_f32(static_cast<uint16_t>(t[e] & 0xffffu));
                v[8 * j + 2 * e + 1] = f16_to_f32(static_cast<uint16_t>(t[e] >> 16));
            }
        }
        butterfly<4>(v);
        if (only) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                v[e] = v[e] * norm;
                amax = fmaxf(amax, fabsf(v[e]));
            }
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) lds[lds_pad(16 * c + e)] = v[e];
    }
    __syncthreads();
    fwht_quant_tail<OUT>(lds, red, K, hbs_log2, norm, 4, amax, out, scales, row);
}

static int ilog2(int v) {
    int r = 0;
    while ((1 << r) < v) ++r;
    return r;
}

size_t rows_lds_bytes(int K) { return sizeof(float) * (static_cast<size_t>(K) + K / 16 + 1 + 8); }

// Rows of 1-4 Hadamard blocks of 1024 (K / 1024 of them), one wave per row.
template <RowOut OUT, typename Loader, typename Dest>
static hipError_t launch_wave_rows(const Loader& ld, const Dest& dst, int M, int K, float norm, hipStream_t stream) {
    const int blocks = (M + 3) / 4;
    switch (K / 1024) {
        case 1:
            hipLaunchKernelGGL((fwht_quant_wave_rows_kernel<Loader, OUT, 1, Dest>), dim3(blocks), dim3(256), 0, stream,
                               ld, dst, M, K, norm);
            break;
        case 2:
            hipLaunchKernelGGL((fwht_quant_wave_rows_kernel<Loader, OUT, 2, Dest>), dim3(blocks), dim3(256), 0, stream,
                               ld, dst, M, K, norm);
            break;
        case 3:
            hipLaunchKernelGGL((fwht_quant_wave_rows_kernel<Loader, OUT, 3, Dest>), dim3(blocks), dim3(256), 0, stream,
                               ld, dst, M, K, norm);
            break;
        default:
            hipLaunchKernelGGL((fwht_quant_wave_rows_kernel<Loader, OUT, 4, Dest>), dim3(blocks), dim3(256), 0, stream,
                               ld, dst, M, K, norm);
            break;
    }
    return hipGetLastError();
}
template <RowOut OUT, typename Loader>
static hipError_t launch_wave_rows(const Loader& ld, void* out, float* scales, int M, int K, float norm,
                                   hipStream_t stream) {
    return launch_wave_rows<OUT>(ld, RowDest{out, scales}, M, K, norm, stream);
}

template <typename InT, RowOut OUT>
static hipError_t launch_rows(const InT* x, void* out, float* scales, int M, int K, int hbs,
                              hipStream_t stream) {
    if (M == 0) return hipSuccess;
    const float norm = static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(hbs)));
    if constexpr (OUT == RowOut::Int8 || OUT == RowOut::Fp8) {
        // rows of 1-4 Hadamard blocks of 1024 values: one wave per row
        if (hbs == 1024 && K % 1024 == 0 && K / 1024 <= 4) {
            return launch_wave_rows<OUT>(RowsLoader<InT>{x, K}, out, scales, M, K, norm, stream);
        }
        // rows of 2-4 Hadamard blocks of 4096 values: block by block
        const int nb = K / 4096;
        if (hbs == 4096 && nb >= 2 && nb <= 4 && nb * 4096 == K) {
            const size_t lds = sizeof(float) * (4096 + 4096 / 16 + 1 + 8);
            auto kern = nb == 2 ? fwht_quant_blocks_kernel<InT, OUT, 2>
                      : nb == 3 ? fwht_quant_blocks_kernel<InT, OUT, 3>
                                : fwht_quant_blocks_kernel<InT, OUT, 4>;
            hipLaunchKernelGGL(kern, dim3(M), dim3(256), lds, stream, x, out, scales, M, K, norm);
            return hipGetLastError();
        }
    }
    int chunks = (K + 15) / 16;
    int threads = ((chunks + kWave - 1) / kWave) * kWave;
    threads = threads < 64 ? 64 : (threads > 256 ? 256 : threads);
    const size_t lds = rows_lds_bytes(K);
    auto kern = chunks > threads ? fwht_quant_rows_kernel<InT, OUT, 4> : fwht_quant_rows_kernel<InT, OUT, 1>;
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           static_cast<int>(lds));
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kern, dim3(M), dim3(threads), lds, stream, x, out, scales, M, K, ilog2(hbs),
                       norm);
    return hipGetLastError();
}

hipError_t launch_fwht_quant(const void* x, int x_dtype, int M, int K, int hbs, int mode,
                             void* q_out, float* scales, hipStream_t stream) {
    const bool fp8 = (mode == QIMG_QM_FP8_HADAMARD);
    if (x_dtype == QIMG_BF16) {
        const uint16_t* xi = static_cast<const uint16_t*>(x);
        return fp8 ? launch_rows<uint16_t, RowOut::Fp8>(xi, q_out, scales, M, K, hbs, stream)
                   : launch_rows<uint16_t, RowOut::Int8>(xi, q_out, scales, M, K, hbs, stream);
    }
    const float* xf = static_cast<const float*>(x);
    return fp8 ? launch_rows<float, RowOut::Fp8>(xf, q_out, scales, M, K, hbs, stream)
               : launch_rows<float, RowOut::Int8>(xf, q_out, scales, M, K, hbs, stream);
}

bool fwht_quant_gelu_supported(int K, int hbs) {
    const int nb = K / 4096;
    return hbs == 4096 && nb >= 2 && nb <= 4 && nb * 4096 == K;
}

hipError_t launch_fwht_quant_gelu(const float* x, int M, int K, int hbs, int mode, void* q_out, float* scales,
                                  hipStream_t stream) {
    if (!fwht_quant_gelu_supported(K, hbs)) return hipErrorNotSupported;
    if (M == 0) return hipSuccess;
    const float norm = static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(hbs)));
    const size_t lds = sizeof(float) * (4096 + 4096 / 16 + 1 + 8);
    const int nb = K / 4096;
    const bool fp8 = mode == QIMG_QM_FP8_HADAMARD;
    auto kern = fp8 ? (nb == 2   ? fwht_quant_blocks_kernel<float, RowOut::Fp8, 2, true>
                       : nb == 3 ? fwht_quant_blocks_kernel<float, RowOut::Fp8, 3, true>
                                 : fwht_quant_blocks_kernel<float, RowOut::Fp8, 4, true>)
                    : (nb == 2   ? fwht_quant_blocks_kernel<float, RowOut::Int8, 2, true>
                       : nb == 3 ? fwht_quant_blocks_kernel<float, RowOut::Int8, 3, true>
                                 : fwht_quant_blocks_kernel<float, RowOut::Int8, 4, true>);
    hipLaunchKernelGGL(kern, dim3(M), dim3(256), lds, stream, x, q_out, scales, M, K, norm);
    return hipGetLastError();
}

hipError_t launch_ln_fwht_quant(const float* x, const float* shift, const float* scale, int M, int K, int hbs,
                                int mode, float eps, void* q_out, float* scales, hipStream_t stream) {
    if (M == 0) return hipSuccess;
    if ((K & 3) != 0 || K > LN_MAX_DIM || hbs < 1 || (hbs & (hbs - 1)) != 0 || K % hbs != 0)
        return hipErrorInvalidValue;
    const size_t lds = rows_lds_bytes(K);
    const float norm = static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(hbs)));
    // rows of 1-4 Hadamard blocks of 1024 values (the block's K = 3072
    // linear inputs), at least 1024 of them: one wave per row, the row
    // normalized in registers (4096 x 3072: 21.3 -> 18.9 us, 13778 x 3072
    // e4m3: 53.1 -> 45.4 us; with 256 or 300 rows one workgroup per row is
    // faster, 6.4 against 7.2 us)
    if (hbs == 1024 && K % 1024 == 0 && M >= 1024) {
        const LnLoader l{{x, K}, shift, scale, eps};
        const PairLoader<LnLoader> ld{l, l, M};
        const PairDest dst{RowDest{q_out, scales}, RowDest{q_out, scales}, M};
        return mode == QIMG_QM_FP8_HADAMARD ? launch_ln_rows8<RowOut::Fp8>(ld, dst, M, K, norm, stream)
                                            : launch_ln_rows8<RowOut::Int8>(ld, dst, M, K, norm, stream);
    }
    if (mode == QIMG_QM_FP8_HADAMARD)
        hipLaunchKernelGGL(ln_fwht_quant_kernel<RowOut::Fp8>, dim3(M), dim3(LN_THR), lds, stream, x, shift, scale,
                           eps, q_out, scales, K, ilog2(hbs), norm);
    else
        hipLaunchKernelGGL(ln_fwht_quant_kernel<RowOut::Int8>, dim3(M), dim3(LN_THR), lds, stream, x, shift, scale,
                           eps, q_out, scales, K, ilog2(hbs), norm);
    return hipGetLastError();
}

hipError_t launch_heads_fwht_quant(const uint16_t* attn, int batch, int H, int S, int s0, int n, int hbs, int mode,
                                   void* q_out, float* scales, hipStream_t stream) {
    const int M = batch * n;
    if (M == 0) return hipSuccess;
    const int K = H * 128;
    if (hbs < 16 || (hbs & (hbs - 1)) != 0 || K % hbs != 0 || s0 < 0 || s0 + n > S) return hipErrorInvalidValue;
    int threads = ((K / 16 + kWave - 1) / kWave) * kWave;
    threads = threads > 256 ? 256 : threads;
    const size_t lds = rows_lds_bytes(K);
    const float norm = static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(hbs)));
    // rows of 1-4 blocks of 1024 (the out-projection input, K = 3072): one
    // wave per row, as for the activations in row-major layout
    if (hbs == 1024 && K % 1024 == 0 && K / 1024 <= 4) {
        const HeadsLoader ld{attn, S, H, s0, n};
        return mode == QIMG_QM_FP8_HADAMARD ? launch_wave_rows<RowOut::Fp8>(ld, q_out, scales, M, K, norm, stream)
                                            : launch_wave_rows<RowOut::Int8>(ld, q_out, scales, M, K, norm, stream);
    }
    if (mode == QIMG_QM_FP8_HADAMARD)
        hipLaunchKernelGGL(heads_fwht_quant_kernel<RowOut::Fp8>, dim3(M), dim3(threads), lds, stream, attn, S, H, s0,
                           n, q_out, scales, ilog2(hbs), norm);
    else
        hipLaunchKernelGGL(heads_fwht_quant_kernel<RowOut::Int8>, dim3(M), dim3(threads), lds, stream, attn, S, H, s0,
                           n, q_out, scales, ilog2(hbs), norm);
    return hipGetLastError();
}

hipError_t launch_ln_fwht_quant_pair(const float* xa, const float* shift_a, const float* scale_a, int Ma, void* qa,
                                     float* sa, const float* xb, const float* shift_b, const float* scale_b, int Mb,
                                     void* qb, float* sb, int K, int hbs, int mode, float eps, hipStream_t stream) {
    if (!(hbs == 1024 && K % 1024 == 0 && K <= LN_MAX_DIM && Ma > 0 && Mb > 0 && Ma + Mb >= 1024)) {
        const hipError_t e = launch_ln_fwht_quant(xa, shift_a, scale_a, Ma, K, hbs, mode, eps, qa, sa, stream);
        return e != hipSuccess ? e : launch_ln_fwht_quant(xb, shift_b, scale_b, Mb, K, hbs, mode, eps, qb, sb, stream);
    }
    const float norm = static_cast<float>(1.0 / __builtin_sqrt(1024.0));
    const PairLoader<LnLoader> ld{LnLoader{{xa, K}, shift_a, scale_a, eps}, LnLoader{{xb, K}, shift_b, scale_b, eps},
                                  Ma};
    const PairDest dst{RowDest{qa, sa}, RowDest{qb, sb}, Ma};
    return mode == QIMG_QM_FP8_HADAMARD ? launch_ln_rows8<RowOut::Fp8>(ld, dst, Ma + Mb, K, norm, stream)
                                        : launch_ln_rows8<RowOut::Int8>(ld, dst, Ma + Mb, K, norm, stream);
}

hipError_t launch_heads_fwht_quant_pair(const uint16_t* attn, int batch, int H, int S, int n_txt, int n_img, int hbs,
                                        int mode, void* q_img, float* s_img, void* q_txt, float* s_txt,
                                        hipStream_t stream) {
    const int K = H * 128;
    const int Ma = batch * n_img, Mb = batch * n_txt;
    if (!(hbs == 1024 && K % 1024 == 0 && K / 1024 <= 4 && Ma > 0 && Mb > 0 && n_txt + n_img == S)) {
        const hipError_t e =
            launch_heads_fwht_quant(attn, batch, H, S, n_txt, n_img, hbs, mode, q_img, s_img, stream);
        return e != hipSuccess ? e : launch_heads_fwht_quant(attn, batch, H, S, 0, n_txt, hbs, mode, q_txt, s_txt, stream);
    }
    const float norm = static_cast<float>(1.0 / __builtin_sqrt(1024.0));
    const PairLoader<HeadsLoader> ld{HeadsLoader{attn, S, H, n_txt, n_img}, HeadsLoader{attn, S, H, 0, n_txt}, Ma};
    const PairDest dst{RowDest{q_img, s_img}, RowDest{q_txt, s_txt}, Ma};
    return mode == QIMG_QM_FP8_HADAMARD ? launch_wave_rows<RowOut::Fp8>(ld, dst, Ma + Mb, K, norm, stream)
                                        : launch_wave_rows<RowOut::Int8>(ld, dst, Ma + Mb, K, norm, stream);
}

hipError_t launch_fwht_inplace(float* data, int M, int K, int hbs, hipStream_t stream) {
    // Rows are transformed through LDS, so in place is safe: each workgroup
    // reads its whole row before writing it back.
    return launch_rows<float, RowOut::Fp32>(data, data, nullptr, M, K, hbs, stream);
}

}  // namespace qimg
