// sage_attention.hip — SageAttention-style joint attention for gfx950.
//
// Semantics follow the kernels qwen-image.cu vendors from SageAttention
// (sageattention_sm80.cu):
//   k mean                 :759-773  sequential fp32 sum over tokens / max(S,1)
//   Q int8, per 4 tokens   :775-824  tokens b*128 + w*32 + g + 8i, i < 4
//   K int8, per 16 tokens  :826-886  tokens b*64 + 2g + {0,1} + 8i, i < 8,
//                                    values k - mean
//   attention              :47-674   int8 QK^T, base-2 online softmax over
//                                    64-key tiles, P rounded to fp16, fp16 PV
//                                    with fp32 accumulation, O/d -> fp16
//                                    (the running max here moves lazily; see
//                                    kRescaleSlack)
// The quantized values and scales are bit-identical to the reference's
// formulas (scale = amax/127 + 1e-7, q = rne_sat(v * (1/scale))).
//
// MI355X design of the attention kernel:
//  * Each wave owns 32 queries, exactly one of the reference's per-thread Q
//    scale groups' 32-token windows.
//  * Scores are computed transposed, S^T = K Q^T, with
//    v_mfma_i32_32x32x32_i8: lane l then holds ONE query (l % 32) and 32 of
//    the tile's 64 keys, so the softmax row max / row sum are lane-local
//    plus one exchange with lane l ^ 32. No 4-lane shuffles per row.
//  * O is accumulated transposed too, O^T = V^T P^T with
//    v_mfma_f32_32x32x16_f16: the P^T registers produced by the score MFMA
//    are already the B operand, and the output keeps one query per lane, so
//    the online-softmax rescale is a per-lane scalar.
//  * V is re-laid once per call into [head][64-key tile][d][64 keys] with a
//    fixed permutation of each 16-key group that makes a lane's 8 keys of a
//    PV fragment contiguous (one ds_read_b128).
//  * A workgroup is 8 waves over 256 queries; K (int8) and V (fp16) tiles
//    stream through a 4-slot LDS ring filled by direct global->LDS DMA, with
//    an XOR swizzle for bank-conflict-free 16-byte fragment reads; Q stays in
//    registers for the whole kernel.
#include <type_traits>

#include "qimg_device.h"
#include "qimg_internal.h"

namespace qimg {

namespace {

constexpr int KTILE = 64;
constexpr int QBLK = 128;

__host__ __device__ constexpr int div_up(int a, int b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------- k mean
// mean[h,d] = (sum over s of k[h,s,d], left to right in fp32) / max(S,1),
// bit-equal to the reference's one-thread-per-(h,d) loop. The sum must stay
// sequential, so the work is arranged to keep everything else off that
// chain: a 256-thread workgroup owns KM_DIMS (h,d) chains (one head, 32
// dims), so that BH * D / 32 workgroups stream K from HBM together (the
// chain, 4352 dependent adds at S = 4352, is the same length whatever the
// slice width; a narrow slice spreads the loads over more CUs, and 32 dims
// measured faster than 16, whose loads touch 32 rows for 32 bytes each,
// and than 64). Wave 0 only
// sums, one chain per lane (lanes past KM_DIMS repeat a chain and store
// nothing), one fp32 add per token (the fp16 -> fp32 conversions stay off
// the dependent chain), with the LDS reads of each group of 32 tokens
// issued two groups ahead. Waves 1-3
// stream KM_CHUNK-token chunks of k[h, :, d0:d0+32] (each lane 16 bytes =
// 8 dims of 4 consecutive tokens), transpose 4 tokens x 8 dims in registers
// and store them to LDS as [d][s] with 8-byte writes; rows are padded to a
// pitch of 4 banks mod 64. Chunks are double-buffered in LDS,
// and the loads run one chunk ahead of the LDS writes.
constexpr int KM_DIMS = 32;                        // chains per workgroup
constexpr int KM_G = KM_DIMS / 8;                  // 16-byte dim groups per token row
constexpr int KM_CHUNK = 1024;                     // tokens per chunk
constexpr int KM_PITCH = KM_CHUNK / 2 + 4;         // dwords per LDS row
constexpr int KM_QPR = 64 / KM_G;                  // token quads per loader round
constexpr int KM_ROUNDS = KM_CHUNK / 4 / KM_QPR;   // loader rounds per chunk
constexpr int KM_MAXR = (KM_ROUNDS + 2) / 3;       // rounds per loader wave (at most)

// acc + (fp16 token in the low / high half of v): the fp16 -> fp32
// conversion is exact, so the sum is rounded once per token, as the
// reference's float add of the converted value.
__device__ __forceinline__ float km_add_lo(float acc, uint32_t v) {
    return acc + f16_to_f32(static_cast<uint16_t>(v & 0xffffu));
}
__device__ __forceinline__ float km_add_hi(float acc, uint32_t v) {
    return acc + f16_to_f32(static_cast<uint16_t>(v >> 16));
}

__global__ __launch_bounds__(256) void k_mean_kernel(const uint16_t* __restrict__ k, float* __restrict__ mean,
                                                     int S, int D) {
    __shared__ __attribute__((aligned(16))) uint32_t tile[2][KM_DIMS * KM_PITCH];
    const int slices = D / KM_DIMS;
    const int h = blockIdx.x / slices;
    const int d0 = (blockIdx.x % slices) * KM_DIMS;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const uint16_t* src = k + static_cast<int64_t>(h) * S * D + d0;
    const int nchunk = div_up(S, KM_CHUNK);

    // loader lane: dim group g = lane % KM_G, token quad KM_QPR * round +
    // lane / KM_G. issue() starts the loads of a chunk into registers,
    // commit() writes them transposed to an LDS buffer; chunk c+2 is issued
    // right after chunk c+1 is committed, so its memory latency overlaps a
    // whole chunk of the sum. (A second register set, two chunks in flight,
    // measured slower: the compiler's in-order vmcnt waits drain both.)
    const int g = lane % KM_G;
    u32x4 v[1][KM_MAXR][4];
    auto issue = [&](int c, int set) {
#pragma unroll
        for (int r = 0; r < KM_MAXR; ++r) {
            const int round = (wave - 1) + 3 * r;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int s = c * KM_CHUNK + 4 * (KM_QPR * round + lane / KM_G) + i;
                v[set][r][i] = (u32x4){0u, 0u, 0u, 0u};
                if (round < KM_ROUNDS && s < S)
                    v[set][r][i] = *reinterpret_cast<const u32x4*>(src + static_cast<int64_t>(s) * D + 8 * g);
            }
        }
    };
    auto commit = [&](int buf, int set) {
#pragma unroll
        for (int r = 0; r < KM_MAXR; ++r) {
            const int round = (wave - 1) + 3 * r;
            if (round >= KM_ROUNDS) continue;
            const int tq = KM_QPR * round + lane / KM_G;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                // dim 8g + e of tokens 4tq .. 4tq+3: fp16 e of each 16-byte row piece
                const int w = e >> 1;
                const int sh = (e & 1) * 16;
                const uint32_t t0 = (v[set][r][0][w] >> sh) & 0xffffu, t1 = (v[set][r][1][w] >> sh) & 0xffffu;
                const uint32_t t2 = (v[set][r][2][w] >> sh) & 0xffffu, t3 = (v[set][r][3][w] >> sh) & 0xffffu;
                const int d = 8 * g + e;
                uint32_t* dst = &tile[buf][d * KM_PITCH + 2 * tq];
                *reinterpret_cast<uint2*>(dst) = make_uint2(t0 | (t1 << 16), t2 | (t3 << 16));
            }
        }
    };

    float sum = 0.0f;
    if (wave > 0) {
        issue(0, 0);
        commit(0, 0);
        if (nchunk > 1) issue(1, 0);
    }
    __syncthreads();
    for (int c = 0; c < nchunk; ++c) {
        const int buf = c & 1;
        if (wave > 0) {
            if (c + 1 < nchunk) {
                commit(buf ^ 1, 0);              // chunk c+1, issued one chunk ago
                if (c + 2 < nchunk) issue(c + 2, 0);
            }
        } else {
            const int n = min(KM_CHUNK, S - c * KM_CHUNK);
            const uint32_t* row = &tile[buf][(lane % KM_DIMS) * KM_PITCH];
            auto rd = [&](int t8) { return *reinterpret_cast<const u32x4*>(row + 4 * t8); };
            // groups of 32 tokens, read two groups ahead in two register
            // sets; a read past the chunk's last full group re-reads group
            // 0 (in bounds, unused)
            const int full = n >> 5;
            auto group = [&](int gi, u32x4 (&cur)[4]) {
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        sum = km_add_lo(sum, cur[r][e]);
                        sum = km_add_hi(sum, cur[r][e]);
                    }
                const int nx = gi + 2 < full ? gi + 2 : 0;
#pragma unroll
                for (int r = 0; r < 4; ++r) cur[r] = rd(4 * nx + r);
            };
            u32x4 ga[4], gb[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                ga[r] = rd(r);
                gb[r] = rd(4 + r);
            }
            int gi = 0;
            for (; gi + 1 < full; gi += 2) {
                group(gi, ga);
                group(gi + 1, gb);
            }
            if (gi < full) group(gi, ga);
            for (int t = full << 5; t < n; ++t) {
                const uint32_t wv = row[t >> 1];
                sum = (t & 1) ? km_add_hi(sum, wv) : km_add_lo(sum, wv);
            }
        }
        __syncthreads();
    }
    if (tid < KM_DIMS) mean[static_cast<int64_t>(h) * D + d0 + tid] = sum / fmaxf(static_cast<float>(S), 1.0f);
}

// ---------------------------------------------------------------- Q quant
// Block = 256 threads for one (head, 128-token block). Thread t holds token
// t/2, half t%2 of the head dim (D/2 values).
template <int D>
__global__ __launch_bounds__(256) void quant_q_kernel(const uint16_t* __restrict__ q,
                                                      int8_t* __restrict__ q_out,
                                                      float* __restrict__ q_scale, int S) {
    constexpr int HD = D / 2;
    __shared__ float red[QBLK][2];
    __shared__ float inv_s[32];
    const int b = blockIdx.x;
    const int h = blockIdx.y;
    const int tid = threadIdx.x;
    const int tok = b * QBLK + (tid >> 1);
    const int part = tid & 1;
    const bool valid = tok < S;
    const uint16_t* src = q + (static_cast<int64_t>(h) * S + tok) * D + part * HD;
    uint32_t raw[HD / 2];
    float amax = 0.0f;
    if (valid) {
#pragma unroll
        for (int c = 0; c < HD / 8; ++c) {
            u32x4 t = reinterpret_cast<const u32x4*>(src)[c];
            raw[4 * c + 0] = t.x; raw[4 * c + 1] = t.y; raw[4 * c + 2] = t.z; raw[4 * c + 3] = t.w;
        }
#pragma unroll
        for (int i = 0; i < HD / 2; ++i) {
            amax = fmaxf(amax, fabsf(f16_to_f32(static_cast<uint16_t>(raw[i] & 0xffffu))));
            amax = fmaxf(amax, fabsf(f16_to_f32(static_cast<uint16_t>(raw[i] >> 16))));
        }
    }
    red[tid >> 1][part] = amax;
    __syncthreads();
    if (tid < 32) {
        const int w = tid >> 3, g = tid & 7;
        float a = 1e-7f;  // the reference starts its max at 1e-7
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int lt = w * 32 + g + 8 * i;
            a = fmaxf(a, fmaxf(red[lt][0], red[lt][1]));
        }
        const float scale = a / 127.0f + 1e-7f;
        const int nq = div_up(S, QBLK) * 32;
        q_scale[static_cast<int64_t>(h) * nq + b * 32 + w * 8 + g] = scale;
        inv_s[tid] = 1.0f / scale;
    }
    __syncthreads();
    if (!valid) return;
    const int lt = tid >> 1;
    const float inv = inv_s[((lt % QBLK) / 32) * 8 + (lt & 7)];
    int8_t* dst = q_out + (static_cast<int64_t>(h) * S + tok) * D + part * HD;
#pragma unroll
    for (int c = 0; c < HD / 16; ++c) {
        u32x4 pk;
#pragma unroll
        for (int wd = 0; wd < 4; ++wd) {
            const uint32_t r0 = raw[8 * c + 2 * wd], r1 = raw[8 * c + 2 * wd + 1];
            pk[wd] = i8x4_rne_sat(f16_to_f32(static_cast<uint16_t>(r0 & 0xffffu)) * inv,
                                  f16_to_f32(static_cast<uint16_t>(r0 >> 16)) * inv,
                                  f16_to_f32(static_cast<uint16_t>(r1 & 0xffffu)) * inv,
                                  f16_to_f32(static_cast<uint16_t>(r1 >> 16)) * inv);
        }
        reinterpret_cast<u32x4*>(dst)[c] = pk;
    }
}

// ---------------------------------------------------------------- K quant
// Block = 128 threads for one (head, 64-token block); thread t holds token
// t/2, half t%2 of the head dim, values k - mean.
template <int D>
__global__ __launch_bounds__(128) void quant_k_kernel(const uint16_t* __restrict__ k,
                                                      const float* __restrict__ mean,
                                                      int8_t* __restrict__ k_out,
                                                      float* __restrict__ k_scale, int S) {
    constexpr int HD = D / 2;
    __shared__ float red[KTILE][2];
    __shared__ float inv_s[4];
    const int b = blockIdx.x;
    const int h = blockIdx.y;
    const int tid = threadIdx.x;
    const int tok = b * KTILE + (tid >> 1);
    const int part = tid & 1;
    const bool valid = tok < S;
    const uint16_t* src = k + (static_cast<int64_t>(h) * S + tok) * D + part * HD;
    const float* mu = mean + static_cast<int64_t>(h) * D + part * HD;
    float v[HD];
    float amax = 0.0f;
    if (valid) {
#pragma unroll
        for (int c = 0; c < HD / 8; ++c) {
            u32x4 t = reinterpret_cast<const u32x4*>(src)[c];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[8 * c + 2 * e + 0] = f16_to_f32(static_cast<uint16_t>(t[e] & 0xffffu)) - mu[8 * c + 2 * e + 0];
                v[8 * c + 2 * e + 1] = f16_to_f32(static_cast<uint16_t>(t[e] >> 16)) - mu[8 * c + 2 * e + 1];
            }
        }
#pragma unroll
        for (int i = 0; i < HD; ++i) amax = fmaxf(amax, fabsf(v[i]));
    }
    red[tid >> 1][part] = amax;
    __syncthreads();
    if (tid < 4) {
        float a = 1e-7f;
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int lt = 2 * tid + j + 8 * i;
                a = fmaxf(a, fmaxf(red[lt][0], red[lt][1]));
            }
        const float scale = a / 127.0f + 1e-7f;
        const int nk = div_up(S, KTILE) * 4;
        k_scale[static_cast<int64_t>(h) * nk + b * 4 + tid] = scale;
        inv_s[tid] = 1.0f / scale;
    }
    __syncthreads();
    if (!valid) return;
    const float inv = inv_s[((tid >> 1) & 7) >> 1];
    int8_t* dst = k_out + (static_cast<int64_t>(h) * S + tok) * D + part * HD;
#pragma unroll
    for (int c = 0; c < HD / 16; ++c) {
        u32x4 pk;
#pragma unroll
        for (int wd = 0; wd < 4; ++wd) {
            const int e = 16 * c + 4 * wd;
            pk[wd] = i8x4_rne_sat(v[e] * inv, v[e + 1] * inv, v[e + 2] * inv, v[e + 3] * inv);
        }
        reinterpret_cast<u32x4*>(dst)[c] = pk;
    }
}

// K quant for head dim 128 with contiguous accesses: the 128 threads of a
// (head, 64-token block) read the block's 16 KB in eight 2 KB steps, thread
// t taking dims 8 (t % 16) .. +8 of tokens 8 c + t / 16 (c = 0..7). A
// token's scale group (token % 8) / 2 is then t / 32: each group is one
// half-wave, whose max needs lane exchanges only. Same per-element
// arithmetic as quant_k_kernel (k - mean, max |.| from 1e-7, scale =
// max / 127 + 1e-7, q = rne_sat(v * (1 / scale))).
__global__ __launch_bounds__(128) void quant_k128_kernel(const uint16_t* __restrict__ k,
                                                         const float* __restrict__ mean,
                                                         int8_t* __restrict__ k_out,
                                                         float* __restrict__ k_scale, int S) {
    constexpr int D = 128;
    const int b = blockIdx.x;
    const int h = blockIdx.y;
    const int t = threadIdx.x;
    const int d0 = 8 * (t & 15);
    const float* mu = mean + static_cast<int64_t>(h) * D + d0;
    float m8[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) m8[e] = mu[e];  // (the mean need not be 16-byte aligned)
    const int64_t base = (static_cast<int64_t>(h) * S + b * KTILE) * D;
    float v[8][8];
    float amax = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const int tok = b * KTILE + 8 * c + (t >> 4);
        if (tok < S) {
            const u32x4 r = *reinterpret_cast<const u32x4*>(k + base + (8 * c + (t >> 4)) * D + d0);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[c][2 * e] = f16_to_f32(static_cast<uint16_t>(r[e] & 0xffffu)) - m8[2 * e];
                v[c][2 * e + 1] = f16_to_f32(static_cast<uint16_t>(r[e] >> 16)) - m8[2 * e + 1];
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[c][e]));
        }
    }
    // max over the half-wave (the 16 tokens of scale group t / 32)
#pragma unroll
    for (int off = 1; off < 32; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 32));
    const float a = fmaxf(1e-7f, amax);
    const float scale = a / 127.0f + 1e-7f;
    const int g = t >> 5;
    if ((t & 31) == 0) k_scale[static_cast<int64_t>(h) * (div_up(S, KTILE) * 4) + b * 4 + g] = scale;
    const float inv = 1.0f / scale;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const int tok = b * KTILE + 8 * c + (t >> 4);
        if (tok >= S) continue;
        uint2 pk;
        pk.x = i8x4_rne_sat(v[c][0] * inv, v[c][1] * inv, v[c][2] * inv, v[c][3] * inv);
        pk.y = i8x4_rne_sat(v[c][4] * inv, v[c][5] * inv, v[c][6] * inv, v[c][7] * inv);
        *reinterpret_cast<uint2*>(k_out + base + (8 * c + (t >> 4)) * D + d0) = pk;
    }
}

constexpr int HQ_BATCH = 8;  // tokens whose loads a wave keeps in flight

// ------------------------------------------------------------ V re-layout
// V fp16 [BH][S][D] -> Vt [BH][ceil(S/64)][D][64]: for each 64-key tile the
// head dim becomes rows, and inside each 16-key group position p holds key
// 8*((p%8)/4) + 4*(p/8) + p%4. Keys past S are zero.
__device__ __forceinline__ int vt_key_of_pos(int p) {
    const int g = p >> 4, r = p & 15;
    return g * 16 + 8 * ((r & 7) >> 2) + 4 * (r >> 3) + (r & 3);
}

template <int D>
__global__ __launch_bounds__(256) void v_relayout_kernel(const uint16_t* __restrict__ v,
                                                         uint16_t* __restrict__ vt, int S) {
    __shared__ uint16_t tile[KTILE][D + 2];
    const int kt = blockIdx.x;
    const int h = blockIdx.y;
    const int tid = threadIdx.x;
    const uint16_t* src = v + static_cast<int64_t>(h) * S * D;
    // load 64 x D, 16 bytes per piece
    constexpr int PIECES = KTILE * D / 8;
    for (int pc = tid; pc < PIECES; pc += 256) {
        const int key = pc / (D / 8);
        const int c = pc % (D / 8);
        const int tok = kt * KTILE + key;
        u32x4 val = {0u, 0u, 0u, 0u};
        if (tok < S) val = reinterpret_cast<const u32x4*>(src + static_cast<int64_t>(tok) * D)[c];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            tile[key][8 * c + 2 * e + 0] = static_cast<uint16_t>(val[e] & 0xffffu);
            tile[key][8 * c + 2 * e + 1] = static_cast<uint16_t>(val[e] >> 16);
        }
    }
    __syncthreads();
    uint16_t* dst = vt + (static_cast<int64_t>(h) * div_up(S, KTILE) + kt) * D * KTILE;
    for (int pc = tid; pc < PIECES; pc += 256) {
        const int d = pc / 8;
        const int c = pc % 8;
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t lo = tile[vt_key_of_pos(8 * c + 2 * e)][d];
            const uint32_t hi = tile[vt_key_of_pos(8 * c + 2 * e + 1)][d];
            o[e] = lo | (hi << 16);
        }
        reinterpret_cast<u32x4*>(dst + d * KTILE)[c] = o;
    }
}

// Zeros at the positions of keys S .. 64 ceil(S/64) - 1 of the last key
// tile of every (sequence, head) of Vt [BH][ceil(S/64)][D][64], which the
// relayout kernels write and a linear writing Vt directly does not (the
// attention reads whole tiles and gives those keys zero weight); with
// q_scale, also the scales heads_quant_q_wave_kernel writes for the 32-token
// slices of the last 128-token block that hold no token (its group maximum
// of zeros). Grid BH, one thread per dim.
template <int D>
__global__ __launch_bounds__(D) void sage_tail_fill_kernel(uint16_t* __restrict__ vt, float* __restrict__ q_scale,
                                                           int S) {
    const int nt = div_up(S, KTILE);
    const int rem = S - (nt - 1) * KTILE;
    if (rem < KTILE) {
        uint16_t* row = vt + ((static_cast<int64_t>(blockIdx.x) * nt + nt - 1) * D + threadIdx.x) * KTILE;
        for (int p = 0; p < KTILE; ++p)
            if (vt_key_of_pos(p) >= rem) row[p] = 0;
    }
    const int nslice = div_up(S, QBLK) * 4;
    const int first_empty = div_up(S, 32);
    const int idx = first_empty * 8 + static_cast<int>(threadIdx.x);  // (slice, group g) pairs
    if (q_scale != nullptr && idx < nslice * 8) {
        const int slice = idx >> 3, g = idx & 7;
        const float a = fmaxf(1e-7f, 0.0f);
        const int nq = div_up(S, QBLK) * 32;
        q_scale[static_cast<int64_t>(blockIdx.x) * nq + (slice >> 2) * 32 + (slice & 3) * 8 + g] = a / 127.0f + 1e-7f;
    }
}

// The V of the joint block straight from the text and image linears' fp32
// outputs (token s < n_txt of sequence b is txt[b][s], the rest img[b][s -
// n_txt], head hh at columns hh*D..): the fp16 values of the V concat +
// transpose (concat_transpose_fused_fp32, transformer.cu:106-130) laid out
// as v_relayout_kernel lays them out, in one pass. Grid (ceil(S/64),
// batch * H); Vt is [batch * H][ceil(S/64)][D][64].
template <int D>
__global__ __launch_bounds__(256) void heads_v_relayout_kernel(const float* __restrict__ txt,
                                                               const float* __restrict__ img,
                                                               uint16_t* __restrict__ vt, int n_txt, int n_img,
                                                               int H) {
    __shared__ uint16_t tile[KTILE][D + 2];
    const int S = n_txt + n_img;
    const int kt = blockIdx.x;
    const int bh = blockIdx.y;
    const int b = bh / H, hh = bh - b * H;
    const int tid = threadIdx.x;
    constexpr int PIECES = KTILE * D / 4;  // 4 fp32 per piece
#pragma unroll 4
    for (int pc = tid; pc < PIECES; pc += 256) {
        const int key = pc / (D / 4);
        const int c = pc % (D / 4);
        const int tok = kt * KTILE + key;
        v4f val = {0.0f, 0.0f, 0.0f, 0.0f};
        if (tok < S) {
            const float* row = tok < n_txt ? txt + (static_cast<int64_t>(b) * n_txt + tok) * H * D
                                           : img + (static_cast<int64_t>(b) * n_img + tok - n_txt) * H * D;
            val = reinterpret_cast<const v4f*>(row + hh * D)[c];
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) tile[key][4 * c + e] = f32_to_f16(val[e]);
    }
    __syncthreads();
    uint16_t* dst = vt + (static_cast<int64_t>(bh) * div_up(S, KTILE) + kt) * D * KTILE;
    constexpr int OPIECES = KTILE * D / 8;
    for (int pc = tid; pc < OPIECES; pc += 256) {
        const int d = pc / 8;
        const int c = pc % 8;
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t lo = tile[vt_key_of_pos(8 * c + 2 * e)][d];
            const uint32_t hi = tile[vt_key_of_pos(8 * c + 2 * e + 1)][d];
            o[e] = lo | (hi << 16);
        }
        reinterpret_cast<u32x4*>(dst + d * KTILE)[c] = o;
    }
}

// ------------------------------------------------------------ attention
// A workgroup is 8 waves (two per SIMD) over AQ = 256 queries; wave w owns
// queries 32w .. 32w+31 of the block. K (int8 [64][D]) and V^T (fp16
// [D][64]) tiles stream through a 5-slot LDS ring filled by direct
// global->LDS DMA (global_load_lds_dwordx4), three tiles ahead of the
// compute, so each 64-key tile is fetched once for 256 queries. Rows are
// unpadded; a per-row XOR swizzle of the 16-byte chunks keeps the fragment
// reads of 8 consecutive rows on distinct LDS banks (the DMA source address
// of each lane applies the same swizzle).
// max(v, v of lane ^ 32): v_permlane32_swap gives every lane the values of
// both lane halves at its position (no LDS round trip)
__device__ __forceinline__ float max_lane_halves(float v) {
    const unsigned u = __float_as_uint(v);
    const auto sw = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
}

constexpr int AQ = 256;          // queries per workgroup
constexpr float kRescaleSlack = 8.0f;  // lazy-rescale threshold of the running max (log2 units)
constexpr int AWAVES = AQ / 32;  // 8
constexpr int ANSLOT = 5;        // LDS ring depth (tiles)
constexpr int AHEAD = 3;         // tiles in the ring ahead of the current one
// step kt reads tiles kt-1 (V), kt and kt+1 (K); kt+2 is in flight and the
// DMA issued at its start fills the slot of tile kt-2
static_assert(ANSLOT == AHEAD + 2, "ring depth");

template <int D>
struct AttnCfg {
    static constexpr int K_BYTES = KTILE * D;             // int8 K tile
    static constexpr int V_BYTES = D * KTILE * 2;         // fp16 V^T tile (rows of 128 B)
    static constexpr int STAGE = K_BYTES + V_BYTES;
    static constexpr int KSTEPS = D / 32;                 // int8 MFMA k-steps
    static constexpr int DT = D / 32;                     // 32-row d tiles of O^T
    static constexpr int K_CPR = D / 16;                  // 16-byte chunks per K row
    static constexpr int K_INSTR = K_BYTES / 1024;        // 1 KB DMA instructions per tile
    static constexpr int V_INSTR = V_BYTES / 1024;
    static constexpr int NI = K_INSTR + V_INSTR;
    static constexpr int PER_WAVE = (NI + AWAVES - 1) / AWAVES;
    // DMA instructions left in flight at a hand-off: tiles are issued three
    // steps ahead and step kt reads the K of tile kt+1, so at the end of step
    // kt-1 only tile kt+2 may be missing
    static constexpr int KEEP = PER_WAVE;
};

// physical 16-byte chunk of logical chunk c in row `row` (involution).
// ds_read_b128 serves 16 lanes per cycle from 64 banks (256 bytes); a
// fragment read has 16 consecutive rows at one logical chunk, so the 16
// physical (row, chunk) bank groups must differ: for 128-byte rows the rows
// of each parity need distinct chunks, for 64-byte rows each residue mod 4.
template <int CPR>
__device__ __forceinline__ int swz_chunk(int row, int c) {
    if constexpr (CPR == 8) return c ^ ((row >> 1) & 7);
    else return c ^ swz_row(row);
}

// s_waitcnt vmcnt(n) (other counters untouched), and vmcnt(n) + lgkmcnt(0)
template <int n>
__device__ __forceinline__ void attn_wait_vmcnt() {
    static_assert(n >= 0 && n < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((0x0f70 & ~0xc00f) | (n & 15) | ((n >> 4) << 14));
}
template <int n>
__device__ __forceinline__ void attn_wait_vmcnt_lgkm0() {
    static_assert(n >= 0 && n < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt(0x0070 | (n & 15) | ((n >> 4) << 14));
}


template <int D, bool CAUSAL, int OUT_DT>
__global__ __launch_bounds__(AQ * 2, 1) void sage_attn_kernel(
    const int8_t* __restrict__ Q, const int8_t* __restrict__ K, const uint16_t* __restrict__ Vt,
    const float* __restrict__ q_scale, const float* __restrict__ k_scale, void* __restrict__ out,
    int S, int BH, float sm_log2) {
    // Every rounding step is spelled out (explicit fmaf where fused), so all
    // output-type instantiations compute identical values.
#pragma clang fp contract(off)
    using C = AttnCfg<D>;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[ANSLOT * C::STAGE];

    // Heads are laid out XCD-contiguously: workgroups are dispatched
    // round-robin over the 8 XCDs, and all query blocks of a head run on one
    // XCD, so that head's K/V tiles are shared in one L2.
    const int nqb = div_up(S, AQ);
    const int nwg = nqb * BH;
    int logical;
    {
        const int bid = blockIdx.x, xcd = bid & 7, local = bid >> 3, per = nwg >> 3, extra = nwg & 7;
        logical = (xcd < extra) ? xcd * (per + 1) + local : extra * (per + 1) + (xcd - extra) * per + local;
    }
    const int h = logical / nqb;
    const int qb = logical % nqb;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31;
    const int half = lane >> 5;
    const int nkt = div_up(S, KTILE);
    const int q_idx = qb * AQ + wave * 32 + l32;

    // Q fragments: lane's query row, bytes [half*D/2, half*D/2 + D/2).
    v4i qf[C::KSTEPS];
    {
        const int qr = q_idx < S ? q_idx : S - 1;
        const int8_t* qp = Q + (static_cast<int64_t>(h) * S + qr) * D + half * (D / 2);
#pragma unroll
        for (int s = 0; s < C::KSTEPS; ++s) qf[s] = reinterpret_cast<const v4i*>(qp)[s];
    }
    // Q scale of the reference's per-thread group (128-token blocks of 32 groups)
    const int nq = div_up(S, QBLK) * 32;
    const int qs_idx = q_idx < S ? q_idx : S - 1;
    const float qsc = q_scale[static_cast<int64_t>(h) * nq + (qs_idx / QBLK) * 32 +
                              ((qs_idx % QBLK) / 32) * 8 + (qs_idx & 7)];
    const float* ksh = k_scale + static_cast<int64_t>(h) * (nkt * 4);

    int kt_end = nkt;
    if (CAUSAL) {
        const int lim = (qb + 1) * AQ < S ? (qb + 1) * AQ : S;
        kt_end = div_up(lim, KTILE);
    }

    const int8_t* Kh = K + static_cast<int64_t>(h) * S * D;
    const uint16_t* Vh = Vt + static_cast<int64_t>(h) * nkt * D * KTILE;

    // DMA of tile kt into ring slot `slot`: instruction j of the tile (1 KB)
    // is issued by wave j % 8; tiles past the end re-fetch the last tile
    // into an idle slot, so every wave issues the same count per tile.
    auto issue_tile = [&](int kt, int slot) {
        kt = kt < kt_end ? kt : kt_end - 1;
        uint8_t* base = lds + slot * C::STAGE;
#pragma unroll
        for (int i = 0; i < C::PER_WAVE; ++i) {
            int j = wave + AWAVES * i;
            j = j < C::NI ? j : j - AWAVES;  // a duplicate of this wave's previous piece
            if (j < C::K_INSTR) {
                constexpr int RPI = 1024 / D;  // K rows per instruction
                const int row = j * RPI + lane / C::K_CPR;
                const int chunk = swz_chunk<C::K_CPR>(row, lane % C::K_CPR);
                int tok = kt * KTILE + row;
                tok = tok < S ? tok : S - 1;  // rows past S are loaded but masked
                __builtin_amdgcn_global_load_lds(
                    (gbl_ptr_t)(Kh + static_cast<int64_t>(tok) * D + chunk * 16),
                    (lds_ptr_t)(base + j * 1024), 16, 0, 0);
            } else {
                const int jj = j - C::K_INSTR;
                const int row = jj * 8 + (lane >> 3);  // d row of V^T
                const int chunk = swz_chunk<8>(row, lane & 7);
                __builtin_amdgcn_global_load_lds(
                    (gbl_ptr_t)(Vh + (static_cast<int64_t>(kt) * D + row) * KTILE + chunk * 8),
                    (lds_ptr_t)(base + C::K_BYTES + jj * 1024), 16, 0, 0);
            }
        }
    };

    v16f o[C::DT];
#pragma unroll
    for (int t = 0; t < C::DT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[t][r] = 0.0f;
    float m = -5000000.0f;  // running max (base-2 scaled), as the reference
    float dsum = 0.0f;      // this lane-half's share of the row sum

#pragma unroll
    for (int p = 0; p < AHEAD; ++p) issue_tile(p, p);
    attn_wait_vmcnt<C::KEEP>();  // tiles 0 and 1 have landed
    __builtin_amdgcn_s_barrier();

    // S^T = K Q^T of the tile in ring slot `slot`: blocks of keys
    // 32*kb + (8*(r/4) + 4*half + r%4), query l32. The K fragments are read
    // (qk_load) at the start of the softmax, well before the MFMAs that use
    // them (qk_mma) at its end.
    auto qk_load = [&](int slot, v4i (&kf)[2 * C::KSTEPS]) {
        const uint8_t* kb_lds = lds + slot * C::STAGE;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const int row = kb * 32 + l32;
#pragma unroll
            for (int s = 0; s < C::KSTEPS; ++s) {
                const int chunk = swz_chunk<C::K_CPR>(row, half * C::KSTEPS + s);
                kf[kb * C::KSTEPS + s] = *reinterpret_cast<const v4i*>(kb_lds + row * D + chunk * 16);
            }
        }
    };
    auto qk_mma = [&](const v4i (&kf)[2 * C::KSTEPS], v16i (&acc)[2]) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[kb][r] = 0;
#pragma unroll
            for (int s = 0; s < C::KSTEPS; ++s)
                acc[kb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(kf[kb * C::KSTEPS + s], qf[s], acc[kb], 0, 0, 0);
        }
    };

    // Each 64-key step is two phases. Softmax(kt): the tile max, the lazy
    // rescale of O and the row sum, P = exp2(s * mult - m) as fp16 for the
    // four 16-key groups (VALU), then QK^T of tile kt+1 into the same score
    // registers (MFMA). PV(kt): O^T += V^T P^T for the four groups (MFMA).
    // Waves 0-3 run softmax(kt) then PV(kt) in step kt; waves 4-7 run
    // PV(kt-1) then softmax(kt), so on every SIMD (one wave of each group)
    // one wave's MFMAs overlap the other's VALU. Each wave applies the same
    // operations to O, the row sum and P in the same order either way (the
    // rescale for tile kt after the PV of tile kt-1, before that of kt), so
    // both groups compute what a single sequence of steps computes. Tiles
    // kt-1 (V, for waves 4-7), kt and kt+1 are resident during step kt.
    v16i sacc[2];
    {
        v4i kf[2 * C::KSTEPS];
        qk_load(0, kf);
        qk_mma(kf, sacc);
    }
    const bool lag = wave >= AWAVES / 2;  // waves 4-7 run PV one step late
    v8h p[4];
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 ones = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};

    // K scales of the tile being processed: each step loads the next tile's
    // after its own softmax, so the load is in flight during the PV phase
    // and the hand-off rather than in front of the tile max.
    float4 ks_cur = *reinterpret_cast<const float4*>(ksh);
    auto softmax = [&](int kt, auto masked_c) {
        constexpr bool MASKED = decltype(masked_c)::value;
        // the next tile's K fragments (past the last tile the slot holds a
        // re-fetched valid tile whose scores are not used)
        v4i kf[2 * C::KSTEPS];
        qk_load((kt + 1) % ANSLOT, kf);
        __builtin_amdgcn_sched_barrier(0);
        const float4 ks4 = ks_cur;
        const float ks_lo = half ? ks4.z : ks4.x;
        const float ks_hi = half ? ks4.w : ks4.y;
        const float mul_lo = sm_log2 * (qsc * ks_lo);
        const float mul_hi = sm_log2 * (qsc * ks_hi);
        const int kbase = kt * KTILE;
        auto key_ok = [&](int kb, int r) {
            const int key = kbase + kb * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
            bool ok = key < S;
            if (CAUSAL) ok = ok && key <= q_idx;
            return ok;
        };
        // tile max: integer max per scale group, then one multiply each
        // (max of fl(acc*c) equals fl(max(acc)*c) for c > 0).
        int mx_lo = INT32_MIN, mx_hi = INT32_MIN;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                int a = sacc[kb][r];
                if constexpr (MASKED) {
                    if (!key_ok(kb, r)) a = INT32_MIN;
                }
                if ((r & 2) == 0) mx_lo = max(mx_lo, a);
                else mx_hi = max(mx_hi, a);
            }
        float mt = -5000000.0f;
        if (mx_lo != INT32_MIN) mt = fmaxf(mt, static_cast<float>(mx_lo) * mul_lo);
        if (mx_hi != INT32_MIN) mt = fmaxf(mt, static_cast<float>(mx_hi) * mul_hi);
        mt = max_lane_halves(mt);
        // Lazy rescale: the reference max m moves (and O, d are rescaled) only
        // when the tile max exceeds it by more than kRescaleSlack (log2
        // units). Otherwise P = exp2(s - m) <= 2^kRescaleSlack, exact in fp16
        // range; O and d use the same m, so O/d is unchanged in exact
        // arithmetic and only the fp16 rounding points of P shift.
        const bool bump = mt > m + kRescaleSlack;
        const float m_new = bump ? mt : m;
        const float o_scale = __builtin_amdgcn_exp2f(m - m_new);
        m = m_new;
        // Lanes that did not move multiply by exactly 1.
        if (__ballot(bump)) {
            dsum *= o_scale;
#pragma unroll
            for (int t = 0; t < C::DT; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[t][r] *= o_scale;
        }
        // P = exp2(acc * mult - m) -> fp16 (round to nearest, in pairs) per
        // 16-key group t; the row sum of the fp16 P accumulates in fp32 with
        // v_dot2_f32_f16.
        const float neg_m = -m_new;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int kb = t >> 1;
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                const int r = 8 * (t & 1) + e;
                const float mul = (r & 2) ? mul_hi : mul_lo;
                float p0 = __builtin_amdgcn_exp2f(fmaf(static_cast<float>(sacc[kb][r]), mul, neg_m));
                float p1 = __builtin_amdgcn_exp2f(fmaf(static_cast<float>(sacc[kb][r + 1]), mul, neg_m));
                if constexpr (MASKED) {
                    if (!key_ok(kb, r)) p0 = 0.0f;
                    if (!key_ok(kb, r + 1)) p1 = 0.0f;
                }
                const h2 ph = __builtin_convertvector((f2){p0, p1}, h2);
                p[t][e] = ph.x;
                p[t][e + 1] = ph.y;
                dsum = __builtin_amdgcn_fdot2(ph, ones, dsum, false);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        qk_mma(kf, sacc);  // the next tile's scores
    };

    auto pv = [&](int kt) {
        const uint8_t* vb_lds = lds + (kt % ANSLOT) * C::STAGE + C::K_BYTES;
        v8h vf[2][C::DT];
        auto read_v = [&](int t, v8h* dst) {
#pragma unroll
            for (int dt = 0; dt < C::DT; ++dt) {
                const int row = dt * 32 + l32;
                const int chunk = swz_chunk<8>(row, 2 * t + half);
                dst[dt] = *reinterpret_cast<const v8h*>(vb_lds + row * (2 * KTILE) + chunk * 16);
            }
        };
        read_v(0, vf[0]);
        read_v(1, vf[1]);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int dt = 0; dt < C::DT; ++dt)
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[t & 1][dt], p[t], o[dt], 0, 0, 0);
            if (t + 2 < 4) read_v(t + 2, vf[t & 1]);
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    // MASKED tiles (the tail past S, and for causal the tiles that reach
    // the block's diagonal) evaluate the per-key validity; the others skip
    // it.
    auto step = [&](int kt, auto masked_c) {
        issue_tile(kt + AHEAD, (kt + AHEAD) % ANSLOT);
        __builtin_amdgcn_sched_barrier(0);
        if (lag && kt > 0) pv(kt - 1);
        softmax(kt, masked_c);
        ks_cur = *reinterpret_cast<const float4*>(ksh + (kt + 1 < nkt ? kt + 1 : nkt - 1) * 4);
        if (!lag) pv(kt);
        // hand-off: this wave's LDS reads are done and its share of tile
        // kt+2 has landed; the barrier makes every wave's share visible and
        // frees slot kt-1 (last read by waves 4-7 in this step) for the DMA
        // issued at the start of step kt+1.
        attn_wait_vmcnt_lgkm0<C::KEEP>();
        __builtin_amdgcn_s_barrier();
    };

    // Tiles wholly inside [0, S) (and, for causal, wholly below the block's
    // first query) need no masking.
    int kt_full = S / KTILE;
    if (CAUSAL) kt_full = min(kt_full, (qb * AQ) / KTILE);
    kt_full = min(kt_full, kt_end);
    int kt = 0;
    for (; kt < kt_full; ++kt) step(kt, std::false_type{});
    for (; kt < kt_end; ++kt) step(kt, std::true_type{});
    if (lag) pv(kt_end - 1);
    attn_wait_vmcnt<0>();  // drain the re-fetches issued by the last steps

    // combine the two lane-halves' row sums, normalise, store.
    const float dtot = dsum + __shfl_xor(dsum, 32, 64);
    if (q_idx >= S) return;
    const float rcp = 1.0f / dtot;
    const int64_t orow = (static_cast<int64_t>(h) * S + q_idx) * D;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d0 = dt * 32 + 8 * g + 4 * half;
            uint16_t hv[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                // O * (1/d) is rounded to fp32 and then to fp16, as the
                // reference does; the empty asm keeps the compiler from
                // fusing both roundings into one v_fma_mix.
                float t = o[dt][4 * g + c] * rcp;
                asm volatile("" : "+v"(t));
                hv[c] = f32_to_f16(t);
            }
            if (OUT_DT == QIMG_FP16) {
                uint16_t* op = reinterpret_cast<uint16_t*>(out) + orow + d0;
                *reinterpret_cast<uint2*>(op) = make_uint2(hv[0] | (static_cast<uint32_t>(hv[1]) << 16),
                                                           hv[2] | (static_cast<uint32_t>(hv[3]) << 16));
            } else if (OUT_DT == QIMG_FP32) {
                float* op = reinterpret_cast<float*>(out) + orow + d0;
                *reinterpret_cast<v4f*>(op) = (v4f){f16_to_f32(hv[0]), f16_to_f32(hv[1]),
                                                    f16_to_f32(hv[2]), f16_to_f32(hv[3])};
            } else {
                uint16_t* op = reinterpret_cast<uint16_t*>(out) + orow + d0;
                uint16_t b[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) b[c] = f32_to_bf16(f16_to_f32(hv[c]));
                *reinterpret_cast<uint2*>(op) = make_uint2(b[0] | (static_cast<uint32_t>(b[1]) << 16),
                                                           b[2] | (static_cast<uint32_t>(b[3]) << 16));
            }
        }
    }
}

// The joint block's Q straight from the text and image linears' fp32
// outputs to int8: the RMSNorm + RoPE + fp16 of joint_heads_f16_kernel
// (block_ops.hip), then the Sage Q quantization of quant_q_kernel, without
// the fp16 Q in HBM. One wave per (head, 32-token slice) and no workgroup
// barriers: a Q scale group (tokens g, g + 8, g + 16, g + 24 of a slice)
// never leaves its slice, so each wave quantizes its own. Phase 1 is the
// heads kernel's per-token code (lane l holds dims 2l, 2l+1; the same wave
// sum, FMAs and fp16 rounding) into a wave-private LDS buffer; in phase 2
// lane 8g + j holds dims 16j .. +16 of group g's four tokens, and the
// group's max is taken over its eight lanes. The int8 values and scales are
// those of the two kernels run one after the other. (A workgroup per 128
// tokens of two heads, with barriers between the phases, has half as many
// waves in flight: the C4 block's qk_norm category measured 40 -> 35 us,
// together with quant_k128_kernel for K.) D = 128.
__global__ __launch_bounds__(256) void heads_quant_q_wave_kernel(const float* __restrict__ txt,
                                                                 const float* __restrict__ img,
                                                                 const uint16_t* __restrict__ w_txt,
                                                                 const uint16_t* __restrict__ w_img,
                                                                 const float* __restrict__ pe,
                                                                 int8_t* __restrict__ q_out,
                                                                 float* __restrict__ q_scale, int n_txt, int n_img,
                                                                 int batch, int H, float eps) {
    constexpr int D = 128, HD = D / 2, PITCH = HD + 1;
    __shared__ uint32_t rows_all[4][32 * PITCH];
    const int S = n_txt + n_img;
    const int BH = batch * H;
    const int nslice = div_up(S, QBLK) * 4;  // every slice of every 128-token block (their scales are written)
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int unit = blockIdx.x * 4 + wave;  // slice-major, head fastest: a workgroup's waves share pe rows
    if (unit >= nslice * BH) return;         // whole waves; no barrier below
    const int slice = unit / BH;
    const int bh = unit - slice * BH;
    const int b = bh / H, h = bh - b * H;
    uint32_t* rows = rows_all[wave];

    // phase 1
    const uint32_t wpt = reinterpret_cast<const uint32_t*>(w_txt)[lane];
    const uint32_t wpi = reinterpret_cast<const uint32_t*>(w_img)[lane];
    for (int t0 = 0; t0 < 32; t0 += HQ_BATCH) {
        float2 x[HQ_BATCH];
        v4f p[HQ_BATCH];
#pragma unroll
        for (int k = 0; k < HQ_BATCH; ++k) {
            const int tok = slice * 32 + t0 + k;
            x[k] = make_float2(0.0f, 0.0f);
            p[k] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
            if (tok < S) {
                const float* row = tok < n_txt ? txt + (static_cast<int64_t>(b) * n_txt + tok) * H * D
                                               : img + (static_cast<int64_t>(b) * n_img + tok - n_txt) * H * D;
                x[k] = reinterpret_cast<const float2*>(row + h * D)[lane];
                p[k] = reinterpret_cast<const v4f*>(pe)[static_cast<int64_t>(tok) * HD + lane];
            }
        }
#pragma unroll
        for (int k = 0; k < HQ_BATCH; ++k) {
            const int tok = slice * 32 + t0 + k;
            const uint32_t wp = tok < n_txt ? wpt : wpi;
            const float w0 = bf16_to_f32(static_cast<uint16_t>(wp & 0xffffu));
            const float w1 = bf16_to_f32(static_cast<uint16_t>(wp >> 16));
            float2 y = x[k];
            const float ss = wave_sum_dpp(__builtin_fmaf(y.x, y.x, y.y * y.y));
            const float rms = rsqrtf(ss / D + eps);
            y.x = y.x * rms * w0;
            y.y = y.y * rms * w1;
            const float o0 = __builtin_fmaf(y.x, p[k].x, y.y * p[k].y);
            const float o1 = __builtin_fmaf(y.x, p[k].z, y.y * p[k].w);
            rows[(t0 + k) * PITCH + lane] =
                static_cast<uint32_t>(f32_to_f16(o0)) | (static_cast<uint32_t>(f32_to_f16(o1)) << 16);
        }
    }
    // LDS operations of one wave complete in order; keep the compiler from
    // moving the reads of other lanes' words above the writes
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");

    // phase 2: group g = lane / 8, dims 16 j .. +16 with j = lane % 8
    const int g = lane >> 3, j = lane & 7;
    uint32_t raw[4][8];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            raw[i][c] = rows[(g + 8 * i) * PITCH + 8 * j + c];
            amax = fmaxf(amax, fabsf(f16_to_f32(static_cast<uint16_t>(raw[i][c] & 0xffffu))));
            amax = fmaxf(amax, fabsf(f16_to_f32(static_cast<uint16_t>(raw[i][c] >> 16))));
        }
#pragma unroll
    for (int off = 1; off < 8; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    const float a = fmaxf(1e-7f, amax);  // the reference starts its max at 1e-7
    const float scale = a / 127.0f + 1e-7f;
    const int nq = div_up(S, QBLK) * 32;
    if (j == 0) q_scale[static_cast<int64_t>(bh) * nq + (slice >> 2) * 32 + (slice & 3) * 8 + g] = scale;
    const float inv = 1.0f / scale;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int tok = slice * 32 + g + 8 * i;
        if (tok >= S) continue;
        u32x4 pk;
#pragma unroll
        for (int wd = 0; wd < 4; ++wd) {
            const uint32_t r0 = raw[i][2 * wd], r1 = raw[i][2 * wd + 1];
            pk[wd] = i8x4_rne_sat(f16_to_f32(static_cast<uint16_t>(r0 & 0xffffu)) * inv,
                                  f16_to_f32(static_cast<uint16_t>(r0 >> 16)) * inv,
                                  f16_to_f32(static_cast<uint16_t>(r1 & 0xffffu)) * inv,
                                  f16_to_f32(static_cast<uint16_t>(r1 >> 16)) * inv);
        }
        *reinterpret_cast<u32x4*>(q_out + (static_cast<int64_t>(bh) * S + tok) * D + 16 * j) = pk;
    }
}

template <int D, bool CAUSAL>
hipError_t launch_attn_dt(const int8_t* q, const int8_t* k, const uint16_t* vt, const float* qs,
                          const float* ks, void* out, int out_dt, int BH, int S, float sm_log2,
                          hipStream_t stream) {
    const dim3 grid(div_up(S, AQ) * BH);
    const dim3 block(AQ * 2);
    if (out_dt == QIMG_FP16)
        hipLaunchKernelGGL((sage_attn_kernel<D, CAUSAL, QIMG_FP16>), grid, block, 0, stream, q, k, vt, qs, ks,
                           out, S, BH, sm_log2);
    else if (out_dt == QIMG_FP32)
        hipLaunchKernelGGL((sage_attn_kernel<D, CAUSAL, QIMG_FP32>), grid, block, 0, stream, q, k, vt, qs, ks,
                           out, S, BH, sm_log2);
    else
        hipLaunchKernelGGL((sage_attn_kernel<D, CAUSAL, QIMG_BF16>), grid, block, 0, stream, q, k, vt, qs, ks,
                           out, S, BH, sm_log2);
    return hipGetLastError();
}

}  // namespace

int64_t sage_vt_bytes(int BH, int S, int D) {
    return static_cast<int64_t>(BH) * div_up(S, KTILE) * KTILE * D * 2;
}

static int64_t align256(int64_t v) { return (v + 255) & ~static_cast<int64_t>(255); }

int64_t sage_scratch_layout(int BH, int S, int D, void* base, SageScratch* out) {
    const int64_t nqkv = static_cast<int64_t>(BH) * S * D;
    const int64_t o_q = 0;
    const int64_t o_k = o_q + align256(nqkv);
    const int64_t o_vt = o_k + align256(nqkv);
    const int64_t o_qs = o_vt + align256(sage_vt_bytes(BH, S, D));
    const int64_t o_ks = o_qs + align256(static_cast<int64_t>(BH) * div_up(S, QBLK) * 32 * 4);
    const int64_t o_mu = o_ks + align256(static_cast<int64_t>(BH) * div_up(S, KTILE) * 4 * 4);
    const int64_t total = o_mu + align256(static_cast<int64_t>(BH) * D * 4);
    if (out && base) {
        char* b = static_cast<char*>(base);
        out->q_i8 = reinterpret_cast<int8_t*>(b + o_q);
        out->k_i8 = reinterpret_cast<int8_t*>(b + o_k);
        out->v_t = reinterpret_cast<uint16_t*>(b + o_vt);
        out->q_scale = reinterpret_cast<float*>(b + o_qs);
        out->k_scale = reinterpret_cast<float*>(b + o_ks);
        out->k_mean = reinterpret_cast<float*>(b + o_mu);
    }
    return total;
}

hipError_t launch_sage_k_mean(const uint16_t* k, float* mean, int BH, int S, int D,
                              hipStream_t stream) {
    hipLaunchKernelGGL(k_mean_kernel, dim3(BH * (D / KM_DIMS)), dim3(256), 0, stream, k, mean, S, D);
    return hipGetLastError();
}

hipError_t launch_sage_quant_q(const uint16_t* q, int8_t* q_out, float* q_scale, int BH, int S,
                               int D, hipStream_t stream) {
    dim3 grid(div_up(S, QBLK), BH);
    if (D == 128)
        hipLaunchKernelGGL(quant_q_kernel<128>, grid, dim3(256), 0, stream, q, q_out, q_scale, S);
    else
        hipLaunchKernelGGL(quant_q_kernel<64>, grid, dim3(256), 0, stream, q, q_out, q_scale, S);
    return hipGetLastError();
}

hipError_t launch_sage_quant_k(const uint16_t* k, const float* mean, int8_t* k_out,
                               float* k_scale, int BH, int S, int D, hipStream_t stream) {
    dim3 grid(div_up(S, KTILE), BH);
    if (D == 128)
        hipLaunchKernelGGL(quant_k128_kernel, grid, dim3(128), 0, stream, k, mean, k_out, k_scale, S);
    else
        hipLaunchKernelGGL(quant_k_kernel<64>, grid, dim3(128), 0, stream, k, mean, k_out, k_scale, S);
    return hipGetLastError();
}

hipError_t launch_heads_quant_q(const float* txt, const float* img, const uint16_t* w_txt, const uint16_t* w_img,
                                const float* pe, int8_t* q_out, float* q_scale, int n_txt, int n_img, int batch, int H,
                                float eps, hipStream_t stream) {
    const int S = n_txt + n_img;
    if (S == 0 || batch == 0 || H == 0) return hipSuccess;
    const int64_t units = static_cast<int64_t>(div_up(S, QBLK)) * 4 * batch * H;
    hipLaunchKernelGGL(heads_quant_q_wave_kernel, dim3(static_cast<unsigned>((units + 3) / 4)), dim3(256), 0, stream,
                       txt, img, w_txt, w_img, pe, q_out, q_scale, n_txt, n_img, batch, H, eps);
    return hipGetLastError();
}

hipError_t launch_sage_tail_fill(uint16_t* v_t, float* q_scale, int BH, int S, hipStream_t stream) {
    const bool v_tail = S % KTILE != 0;
    const bool q_tail = q_scale != nullptr && div_up(S, 32) < div_up(S, QBLK) * 4;
    if (BH == 0 || S == 0 || (!v_tail && !q_tail)) return hipSuccess;
    hipLaunchKernelGGL(sage_tail_fill_kernel<128>, dim3(BH), dim3(128), 0, stream, v_t, q_tail ? q_scale : nullptr, S);
    return hipGetLastError();
}

hipError_t launch_heads_v_relayout(const float* txt, const float* img, uint16_t* v_t, int n_txt, int n_img,
                                   int batch, int H, hipStream_t stream) {
    const int S = n_txt + n_img;
    if (S == 0 || batch == 0 || H == 0) return hipSuccess;
    hipLaunchKernelGGL(heads_v_relayout_kernel<128>, dim3(div_up(S, KTILE), batch * H), dim3(256), 0, stream, txt,
                       img, v_t, n_txt, n_img, H);
    return hipGetLastError();
}

hipError_t launch_sage_attn(const int8_t* q, const int8_t* k, const uint16_t* v,
                            const float* q_scale, const float* k_scale, void* out, int out_dtype,
                            int BH, int S, int D, float sm_scale, int causal, uint16_t* v_t,
                            hipStream_t stream) {
    dim3 vgrid(div_up(S, KTILE), BH);
    if (D == 128)
        hipLaunchKernelGGL(v_relayout_kernel<128>, vgrid, dim3(256), 0, stream, v, v_t, S);
    else
        hipLaunchKernelGGL(v_relayout_kernel<64>, vgrid, dim3(256), 0, stream, v, v_t, S);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_sage_attn_vt(q, k, v_t, q_scale, k_scale, out, out_dtype, BH, S, D, sm_scale, causal, stream);
}

int64_t sage_attn_workgroups(int BH, int S) { return static_cast<int64_t>(div_up(S, AQ)) * BH; }

hipError_t launch_sage_attn_vt(const int8_t* q, const int8_t* k, const uint16_t* v_t, const float* q_scale,
                               const float* k_scale, void* out, int out_dtype, int BH, int S, int D, float sm_scale,
                               int causal, hipStream_t stream) {
    const float sm_log2 = sm_scale * 1.44269504088896340736f;
    if (D == 128)
        return causal ? launch_attn_dt<128, true>(q, k, v_t, q_scale, k_scale, out, out_dtype, BH, S, sm_log2, stream)
                      : launch_attn_dt<128, false>(q, k, v_t, q_scale, k_scale, out, out_dtype, BH, S, sm_log2, stream);
    return causal ? launch_attn_dt<64, true>(q, k, v_t, q_scale, k_scale, out, out_dtype, BH, S, sm_log2, stream)
                  : launch_attn_dt<64, false>(q, k, v_t, q_scale, k_scale, out, out_dtype, BH, S, sm_log2, stream);
}

}  // namespace qimg
