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
// Tiling (CDNA4, wave64): a 512-thread workgroup owns a 256x256 output tile,
// eight waves in a 2x4 arrangement each own 128x64 = 8x4 MFMA 16x16 blocks
// for int8 (v_mfma_i32_16x16x64_i8) or 4x2 32x32 blocks for e4m3
// (v_mfma_scale_f32_32x32x64_f8f6f4 with unit scales) and bf16, 128
// accumulator registers per wave. Two waves per
// SIMD let one wave's LDS reads and waits overlap the other's MFMAs
// (measured 7-9% faster than four waves of 128x128). Both operands are
// K-major [rows, K] as the reference stores them (TN GEMM). Plain launches
// can also run narrower tiles, chosen where they take fewer rounds of the
// CUs: int8 256x224 (waves 4 x 2 of 64x112) or 256x192 (waves of 128x48),
// e4m3 and bf16 256x192 (waves 4 x 2 of 64x96); 4352 x 3072 is 238 tiles of
// 256x224 in one round, 4096 x 3072 256 tiles of 256x192.
//
// K advances 128 bytes per stage through a two-slot LDS ring (2 x 64 KB):
// while one stage is consumed the next is in flight. Stages are filled by
// direct global->LDS DMA (global_load_lds_dwordx4): no VGPR staging and no
// ds_write instructions. Each DMA instruction writes 1 KB = 8 LDS rows of
// 128 bytes, so every lane octet reads one whole 128-byte cache line: on
// gfx950 a DMA instruction that touches 16 half lines (64-byte rows) moves
// half the bytes per unit time of one that touches 8 full lines (measured
// 62 vs 122 GB/s per CU from L2), which outweighs the shallower ring. Lane i
// fetches the global chunk that the row's XOR swizzle places at physical
// chunk i%8, swizzle(row) = (row >> 1) & 7, so MFMA fragment reads of 16
// consecutive rows at one logical chunk hit distinct LDS banks. Stage
// hand-off uses s_waitcnt + s_barrier rather than __syncthreads(), whose
// workgroup fence would drain every outstanding DMA; it sits before the last
// k-step of a stage, right after the reads of that k-step's fragments, and
// the refill of the freed slot is issued as soon as the barrier passes. The
// LDS fragment reads for the next k-step are interleaved with the current
// k-step's MFMAs (sched_group_barrier), so with one wave per SIMD the matrix
// core is fed without waiting on LDS latency.
//
// The tile's activation scales, weight scales and bias are loaded into
// registers at kernel start and written to LDS (in ring space) after the main
// loop, so the epilogue reads them without global latency.
//
// K ordering: a stage row holds eight 16-byte chunks. Lane group q = lane/16
// of an int8 16x16 fragment takes chunk 4s + q in k-step s (two 64-byte
// k-steps per stage); lane half h of a 32x32 fragment takes chunk 4h + s
// (bf16: four 32-byte k-steps) or chunks 4h + 2s and 4h + 2s + 1 (e4m3: two
// 64-byte k-steps) in k-step s. Both operands use the same assignment, so
// each dot product covers every k exactly once and the int8 result is exact.
#include <atomic>
#include <type_traits>

#include "qimg_device.h"
#include "qimg_internal.h"

namespace qimg {

namespace {

constexpr int BM = 256;
constexpr int BN = 256;
constexpr int BK = 128;    // bytes of K per stage
constexpr int NSLOT = 2;   // LDS ring depth (2 x 64 KB)
constexpr int NWAVES = 8;                    // two waves per SIMD
constexpr int WAVES_N = 4;                   // waves across N (2 across M)
constexpr int NTHR = 64 * NWAVES;
constexpr int WTM = BM / (NWAVES / WAVES_N);  // wave tile: 128 x 64
constexpr int WTN = BN / WAVES_N;
constexpr int TM = WTM / 32;  // 32x32 blocks per wave
constexpr int TN = WTN / 32;
constexpr int DMA_ROWS = 1024 / BK;           // rows per DMA instruction
constexpr int NDMA = BM / (NWAVES * DMA_ROWS);  // DMA instructions per operand per wave per stage
constexpr int OP_BYTES = BM * BK;              // one operand's share of a stage (32 KB)
// The ring holds the A slots then the W slots (A slot s at s*OP_BYTES, W
// slot s at (NSLOT + s)*OP_BYTES), and each wave issues a stage's A DMAs
// before its W DMAs. (Measured 5-7% faster than slots of [A|W] with the two
// operands' DMAs interleaved.)
constexpr int LDS_BYTES = 2 * NSLOT * OP_BYTES;
// Epilogue scales and bias reuse the end of the ring once the main loop is
// done (the output staging uses its start: 8 waves x 32 rows x 272 bytes).
constexpr int SCALE_OFF = LDS_BYTES - 4 * 256 * 4;  // as, ws, bias, gate
static_assert(NWAVES * 32 * (BN / WAVES_N * 4 + 16) <= SCALE_OFF, "output staging overlaps the scales");
static_assert(2 * NDMA == TM * TN, "the int8 loop issues one refill DMA per MFMA of a k-step");
constexpr int GROUP_M = 4;  // tile rows per group in the tile order
constexpr int div_up_c(int a, int b) { return (a + b - 1) / b; }
// Cache policy of the operand DMA: sc0 (measured ~10% faster than the
// default policy at the MMDiT shapes; the non-temporal policy is slower).
constexpr int kDmaPolicy = 1;


// 128-byte rows hold 8 chunks. ds_read_b128 serves 16 lanes per cycle from
// 64 banks (256 bytes), i.e. 16 consecutive fragment rows: 8 of them even
// and 8 odd, each parity covering one 128-byte half of the banks, so the
// physical chunk must differ within each parity: chunk ^ ((row >> 1) & 7).
__device__ __forceinline__ int swz8(int row) { return (row >> 1) & 7; }

__device__ __forceinline__ int lds_addr(int row, int chunk) {
    return row * BK + ((chunk ^ swz8(row)) << 4);
}


// sched_group_barrier instruction classes
constexpr int SG_MFMA = 0x008;
constexpr int SG_VMEM = 0x010;
constexpr int SG_DS_READ = 0x100;
#define SGB(mask, n) __builtin_amdgcn_sched_group_barrier((mask), (n), 0)


// Operand kinds: int8 (v_mfma_i32_32x32x32_i8), e4m3
// (v_mfma_scale_f32_32x32x64_f8f6f4) and bf16 (v_mfma_f32_32x32x16_bf16;
// a 32-byte k-step is 16 bf16, so the int8 loop, ring and fragment layout
// serve it unchanged with K counted in bytes).
constexpr int OP_I8 = 0;
constexpr int OP_F8 = 1;
constexpr int OP_BF16 = 2;
// The int8 product on 16x16 MFMA blocks (v_mfma_i32_16x16x64_i8): the same
// operand bytes per op from LDS, a quarter of the accumulator updates per
// instruction, and a higher sustained clock under a full matrix-core load on
// this chip (a register-only loop runs 16x16x64 at 3.8-3.9 POP/s and 2.1-2.3
// GHz, 32x32x32 at 3.5-3.7 POP/s and 1.7-1.8 GHz). The main loop keeps the
// accumulators as 16x16 blocks and hands them to the epilogue in the 32x32
// blocks' register layout (remapped through LDS) only where an attention
// layout is written; plain launches dequantize and stage the 16x16 blocks
// directly.
// (e4m3 stays on 32x32x64: a 16x16x128 loop of the same tiling measured 2-8%
// slower at the 1328x1328 step's shapes.)
constexpr int OP_I8_16 = 3;

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

template <int OP>
struct Acc {
    typedef v16f type;
};
template <>
struct Acc<OP_I8> {
    typedef v16i type;
};
template <>
struct Acc<OP_I8_16> {
    typedef v16i type;
};

// One GEMM of a launch: out[M,N] = epilogue(A[M,K] . W[N,K]^T), `tiles` =
// its number of BM x BN tiles.
struct TileProblem {
    const uint8_t* A;
    const uint8_t* W;
    const float* as;
    const float* ws;
    const uint16_t* bias;
    void* out;
    const float* gate;  // non-null: out = out + gate[n] * value (fp32 out)
    int M, N, K, tiles;  // K in bytes
    int accumulate;      // bf16 operands: out = out + product before the bias (fp32 out)
    // hk > 0: the output goes to an attention operand layout (HeadsOut kind
    // hk: heads hH, S tokens per sequence, rows are tokens hoff + r % hn of
    // sequences hb0 + r / hn)
    int hk, hH, hS, hoff, hn, hb0;
    const uint16_t* hnorm;
    const float* hpe;
    float* hqs;
    float heps;
};

// Element offset in the V^T tile layout [seq * heads + head][ceil(S/64)][128]
// [64] of row r (token off + r % n of sequence b0 + r / n) and column c (dim
// c % 128 of head c / 128): a key's position in its 64-key tile swaps bits 2
// and 3 of the key (the layout the attention kernel's PV fragments read).
__device__ __forceinline__ int64_t vt_index(int r, int c, int heads, int S, int off, int n, int b0) {
    const int q = r / n;
    const int b = b0 + q;
    const int s = off + (r - q * n);
    const int key = s & 63;
    const int pos = (key & ~12) | ((key & 4) << 1) | ((key & 8) >> 1);
    return ((static_cast<int64_t>(b * heads + (c >> 7)) * ((S + 63) >> 6) + (s >> 6)) * 128 + (c & 127)) * 64 + pos;
}

// The GEMMs of one launch: tiles [0, p[0].tiles) are problem 0, the next
// p[1].tiles problem 1, and so on (e.g. the image- and text-stream q, k and v
// linears of a joint block: each alone leaves CUs idle in its last round).
constexpr int kMaxProblems = 8;
struct TileProblems {
    TileProblem p[kMaxProblems];
    int n, total;
};

// HD: the launch may hold problems with attention-layout outputs
// (TileProblem::hk; an instance of its own, so that the extra epilogues
// leave the others' register allocation alone).
// TW: the tile's width, 256, 224 (MID_BN) or 192 (NARROW_BN). The narrower
// tiles serve plain launches whose 256x256 tiles would leave CUs idle:
// 4096 x 3072 is 192 tiles of 256x256 on 256 CUs, a quarter of the chip
// idle for the whole launch, but 256 tiles of 256x192, one round with every
// CU busy; 4352 x 3072 is 204 tiles of 256x256 but 238 of 256x224.
//  - int8 256x192: waves of 128 x 48 = 8 x 3 blocks of 16x16; a stage's W
//    share is 192 rows, 3 DMA instructions per wave.
//  - int8 256x224: 224 columns are not four waves of whole 16x16 blocks, so the
//    waves are arranged 4 x 2, each 64 x 112 = 4 x 7 blocks; the W DMA still
//    fills 256 rows (4 instructions per wave, the last 32 rows unread), so
//    every wave runs the same instruction stream.
//  - e4m3 and bf16 256x192 (32x32 blocks): waves 4 x 2 of 64 x 96 = 2 x 3
//    blocks.
// TH: the tile's height, 256 or 128 (SMALL_BM, with TW = 128: four waves
// 2 x 2 of 64 x 64 and a 64 KB ring, two workgroups per CU; for problems
// too small to fill the CUs with 256-row tiles).
constexpr int NARROW_BN = 192;
constexpr int MID_BN = 224;
constexpr int SMALL_BM = 128;
template <int OP, int OUT_DT, bool GELU, bool HD = false, int TW = BN, int TH = BM>
__global__ __launch_bounds__(TH == SMALL_BM ? 256 : NTHR, TH == SMALL_BM ? 2 : 1) void gemm_w8a8_kernel(
    TileProblems P) {
    constexpr bool BF = OP == OP_BF16;
    constexpr bool M16 = OP == OP_I8_16;
    static_assert(TW == BN || (!HD && (((TW == NARROW_BN || TW == MID_BN) && M16) ||
                                       (TW == NARROW_BN && (OP == OP_F8 || OP == OP_BF16)) ||
                                       (TW == SMALL_BM && TH == SMALL_BM && M16))),
                  "the narrower tiles serve the plain int8 (16x16 blocks), e4m3 and bf16 epilogues");
    static_assert(TH == BM || (TH == SMALL_BM && TW == SMALL_BM), "128-row tiles are 128 x 128");
    // (these hide the file-scope 256 x 256 values inside the kernel)
    constexpr bool SMALL = TH == SMALL_BM;
    constexpr int BM = TH;                                   // tile height
    constexpr int NWAVES = SMALL ? 4 : 8;                    // two waves per SIMD (over two workgroups if SMALL)
    constexpr int NDMA = BM / (NWAVES * DMA_ROWS);           // A DMA instructions per wave per stage
    constexpr int OP_BYTES = BM * BK;                        // one operand's slot
    constexpr int LDS_BYTES = 2 * NSLOT * OP_BYTES;
    constexpr int SCALE_OFF = LDS_BYTES - 4 * 256 * 4;       // as, ws, bias, gate
    constexpr int WVN = (SMALL || TW == MID_BN || (TW == NARROW_BN && !M16)) ? 2 : WAVES_N;  // waves across N
    constexpr int BN = TW;                           // tile width
    constexpr int WTM = BM / (NWAVES / WVN);         // wave tile: 128 or 64 rows
    constexpr int TM = WTM / 32;                     // 32-row blocks of a wave
    constexpr int WTN = BN / WVN;                    // wave tile width (64, 112 or 48)
    constexpr int TN = WTN / 32;                     // 32x32 blocks across a wave (256 wide only)
    constexpr int TN16 = WTN / 16;                   // 16x16 blocks across a wave
    constexpr int NDMA_W = div_up_c(BN, NWAVES * DMA_ROWS);  // W DMA instructions per wave per stage
    static_assert(WTN % (M16 ? 16 : 32) == 0 && NDMA_W * NWAVES * DMA_ROWS * BK <= OP_BYTES, "wave tile or W slot");
    static_assert(NWAVES * 32 * (WTN * 4 + 16) <= SCALE_OFF, "output staging overlaps the scales");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[LDS_BYTES];
    float* s_as = reinterpret_cast<float*>(lds + SCALE_OFF);
    float* s_ws = s_as + 256;
    float* s_bias = s_ws + 256;
    float* s_gate = s_bias + 256;

    // Several problems can share the grid (TileProblems): find this tile's.
    int logical = xcd_remap(blockIdx.x, P.total);
    int pi = 0;
    while (pi + 1 < P.n && logical >= P.p[pi].tiles) {
        logical -= P.p[pi].tiles;
        ++pi;
    }
    pi = __builtin_amdgcn_readfirstlane(pi);
    const TileProblem& pr = P.p[pi];
    const uint8_t* __restrict__ A = pr.A;
    const uint8_t* __restrict__ W = pr.W;
    const float* __restrict__ as = pr.as;
    const float* __restrict__ ws = pr.ws;
    const uint16_t* __restrict__ bias = pr.bias;
    void* __restrict__ out = pr.out;
    const float* __restrict__ gate = pr.gate;
    const bool accumulate = BF && pr.accumulate;
    const int M = pr.M;
    const int N = pr.N;
    const int K = pr.K;

    const int tiles_n = (N + BN - 1) / BN;
    const int tiles_m = (M + BM - 1) / BM;
    // A problem whose tile count was computed for another width than this
    // kernel's would index tiles past its output (and divide by a group
    // height of zero below): its workgroups do nothing instead.
    if (pr.tiles != tiles_m * tiles_n) return;
    // Grouped tile order: groups of GROUP_M tile rows, column-major inside a
    // group, so the 32 tiles an XCD runs at once form a 4 x 8 block that
    // shares 4 activation slices and 8 weight slices in that XCD's L2.
    const int gsz = GROUP_M * tiles_n;
    const int first_m = (logical / gsz) * GROUP_M;
    const int gm = (tiles_m - first_m) < GROUP_M ? (tiles_m - first_m) : GROUP_M;
    const int tm_idx = first_m + (logical % gsz) % gm;
    const int tn_idx = (logical % gsz) / gm;
    const int m0 = tm_idx * BM;
    const int n0 = tn_idx * BN;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WVN;
    const int wn = wave % WVN;
    const bool has_bias = bias != nullptr;
    const bool has_gate = gate != nullptr;

    // epilogue operands for this tile (clamped indices; only stored
    // outputs use them)
    // (loaded now, written to LDS after the main loop; the bias load is
    // branch-free so it stays in flight behind the DMA stream)
    const int et = tid & 255;  // threads 0..255 own one row / column each
    const int e_n = n0 + et < N ? n0 + et : N - 1;
    float e_as = 1.0f, e_ws = 1.0f, e_gate = 0.0f;
    uint16_t e_braw = 0;
    if constexpr (BF) {  // (no scales or gate with bf16 operands)
        if (has_bias) e_braw = bias[e_n];
    } else {
        e_as = as[m0 + et < M ? m0 + et : M - 1];
        e_ws = ws[e_n];
        const uint16_t* bsrc = has_bias ? bias : reinterpret_cast<const uint16_t*>(ws);
        e_braw = bsrc[e_n];
        e_gate = (has_gate ? gate : ws)[e_n];
    }

    // DMA assignment: wave w, instruction i fills LDS rows
    // DMA_ROWS*(NWAVES*i + w) .. +DMA_ROWS of the A tile (and the same rows
    // of the W tile); lane -> row +lane/8, physical chunk lane%8.
    const uint8_t* a_src[NDMA];
    const uint8_t* w_src[NDMA_W];
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
        const int r = DMA_ROWS * (NWAVES * i + wave) + (lane >> 3);
        const int c = (lane & 7) ^ swz8(r);
        int gm = m0 + r;
        gm = gm < M ? gm : M - 1;  // clamp: rows past M are computed, never stored
        a_src[i] = A + static_cast<int64_t>(gm) * K + c * 16;
        if (i < NDMA_W) {
            int gn = n0 + r;
            gn = gn < N ? gn : N - 1;
            w_src[i] = W + static_cast<int64_t>(gn) * K + c * 16;
        }
    }

    typedef typename Acc<OP>::type acc_t;
    acc_t acc[TM][TN];
    // 16x16 blocks of the wave tile (2 TM x 2 TN), for the M16 kinds
    // (one 16x16 block: lane l holds rows 4(l/16) .. +3 of column l%16)
    typedef v4i acc16_t;
    acc16_t acc16[2 * TM][TN16];
    if constexpr (M16) {
#pragma unroll
        for (int i = 0; i < 2 * TM; ++i)
#pragma unroll
            for (int j = 0; j < TN16; ++j) acc16[i][j] = acc16_t{};
    } else {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
    }

    const int KT = K / BK;

    // Both loops run their last two stages as a separate copy of the stage
    // body with no refill, so no stage is fetched twice and no branch
    // separates the refill DMAs from the MFMAs they are interleaved with.
    auto issue_stage = [&](int kt, int slot) {
        kt = kt < KT ? kt : KT - 1;  // (the prologue's stage 1 when K is one stage)
        const int koff = kt * BK;
        uint8_t* abase = lds + slot * OP_BYTES;
        uint8_t* wbase = lds + (NSLOT + slot) * OP_BYTES;
#pragma unroll
        for (int i = 0; i < NDMA; ++i) {
            const int rowblk = DMA_ROWS * (NWAVES * i + wave);
            __builtin_amdgcn_global_load_lds((gbl_ptr_t)(a_src[i] + koff),
                                             (lds_ptr_t)(abase + rowblk * BK), 16, 0, kDmaPolicy);
        }
#pragma unroll
        for (int i = 0; i < NDMA_W; ++i) {
            const int rowblk = DMA_ROWS * (NWAVES * i + wave);
            __builtin_amdgcn_global_load_lds((gbl_ptr_t)(w_src[i] + koff),
                                             (lds_ptr_t)(wbase + rowblk * BK), 16, 0, kDmaPolicy);
        }
    };

    const int frag_row = lane & 31;
    const int half = lane >> 5;
    int arow[TM], wrow[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) arow[i] = wm * WTM + i * 32 + frag_row;
#pragma unroll
    for (int j = 0; j < TN; ++j) wrow[j] = wn * WTN + j * 32 + frag_row;
    // (16x16 fragments: lane l reads row l%16 of its block, lane group q16)
    const int q16 = lane >> 4;
    int arow16[2 * TM], wrow16[TN16];
#pragma unroll
    for (int i = 0; i < 2 * TM; ++i) arow16[i] = wm * WTM + i * 16 + (lane & 15);
#pragma unroll
    for (int j = 0; j < TN16; ++j) wrow16[j] = wn * WTN + j * 16 + (lane & 15);

    // prologue: stages 0 and 1 in flight; wait for stage 0.
    issue_stage(0, 0);
    issue_stage(1, 1);
    wait_vmcnt<NDMA + NDMA_W>();
    __builtin_amdgcn_s_barrier();

    // Hand-off before a stage's last k-step, right after that k-step's
    // fragment reads were issued: this wave's reads of the current slot are
    // complete (so the refill DMA issued next cannot overwrite data still
    // being read), the next stage has landed (vmcnt 0: it is the only DMA in
    // flight), then the workgroup barrier makes every wave's share visible
    // and tells every wave the current slot is free.
    auto handoff = [&]() {
        __builtin_amdgcn_sched_barrier(0);
        wait_lgkmcnt0();
        wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    };

    if constexpr (OP == OP_I8 || OP == OP_BF16) {
        // Four 32-byte k-steps per stage; the fragments of k-step s+1 are read
        // while k-step s's 16 MFMAs run, and the next stage's k-step 0 is
        // read during k-step 3. The sched_group_barrier sequences pin that
        // interleave (the default schedule sinks every LDS read to just before
        // its first use, which serialises them with the MFMAs). An MFMA leads
        // each pair so its wait on the previous reads does not also wait on
        // the read just issued.
        v4i fa0[TM], fw0[TN], fa1[TM], fw1[TN];
        auto read_frags = [&](v4i* fa, v4i* fw, int slot, int ks) {
            const uint8_t* la = lds + slot * OP_BYTES;
            const uint8_t* lw = lds + (NSLOT + slot) * OP_BYTES;
            const int chunk = 4 * half + ks;
#pragma unroll
            for (int i = 0; i < TM; ++i) fa[i] = *reinterpret_cast<const v4i*>(la + lds_addr(arow[i], chunk));
#pragma unroll
            for (int j = 0; j < TN; ++j) fw[j] = *reinterpret_cast<const v4i*>(lw + lds_addr(wrow[j], chunk));
        };
        auto mfma_all = [&](const v4i* fa, const v4i* fw) {
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    if constexpr (BF)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, fw[j]),
                                                                             __builtin_bit_cast(v8bf, fa[i]),
                                                                             acc[i][j], 0, 0, 0);
                    else
                        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fw[j], fa[i], acc[i][j], 0, 0, 0);
                }
        };
        auto interleave = [&]() {
#pragma unroll
            for (int i = 0; i < TM + TN; ++i) {
                SGB(SG_MFMA, 1);
                SGB(SG_DS_READ, 1);
            }
            SGB(SG_MFMA, TM * TN - (TM + TN));
            __builtin_amdgcn_sched_barrier(0);
        };
        // One stage; REFILL (a std::bool_constant) says whether it refills
        // its slot with stage kt + 2. The last two stages take the copy
        // without it, so no branch separates the refill DMAs from the MFMAs
        // and they are issued one after each MFMA of the last k-step instead
        // of all at once after the barrier, where eight waves' 64 DMAs queue
        // in front of the matrix core (measured 1-3% faster).
        auto stage = [&](int kt, auto refill) {
            const int slot = kt & 1;
            read_frags(fa1, fw1, slot, 1);
            mfma_all(fa0, fw0);
            interleave();
            read_frags(fa0, fw0, slot, 2);
            mfma_all(fa1, fw1);
            interleave();
            read_frags(fa1, fw1, slot, 3);
            mfma_all(fa0, fw0);
            interleave();
            handoff();
            if constexpr (decltype(refill)::value) issue_stage(kt + 2, slot);
            // (the compiler keeps these reads after the refill DMAs, which
            // write LDS)
            read_frags(fa0, fw0, slot ^ 1, 0);
            mfma_all(fa1, fw1);
            if constexpr (decltype(refill)::value) {
                constexpr int NM = TM * TN, NV = NDMA + NDMA_W;
                constexpr int VQ = NV / NM, VR = NV % NM;  // DMAs per MFMA, and the first VR MFMAs' extra one
#pragma unroll
                for (int i = 0; i < NM; ++i) {
                    SGB(SG_MFMA, 1);
                    if (i < VR) {
                        SGB(SG_VMEM, VQ + 1);
                    } else if constexpr (VQ > 0) {
                        SGB(SG_VMEM, VQ);
                    }
                    if (i < TM + TN) SGB(SG_DS_READ, 1);
                }
                __builtin_amdgcn_sched_barrier(0);
            } else {
                interleave();
            }
        };
        read_frags(fa0, fw0, 0, 0);
        int kt = 0;
        for (; kt + 2 < KT; ++kt) stage(kt, std::true_type{});
        for (; kt < KT; ++kt) stage(kt, std::false_type{});
    } else if constexpr (OP == OP_F8) {
        // Two 64-byte k-steps per stage (v_mfma_scale_f32_32x32x64_f8f6f4,
        // unit scales), with the same read-ahead and hand-off.
        v8i fa0[TM], fw0[TN], fa1[TM], fw1[TN];
        auto read_frags = [&](v8i* fa, v8i* fw, int slot, int ks) {
            const uint8_t* la = lds + slot * OP_BYTES;
            const uint8_t* lw = lds + (NSLOT + slot) * OP_BYTES;
            const int c0 = 4 * half + 2 * ks;
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const v4i lo4 = *reinterpret_cast<const v4i*>(la + lds_addr(arow[i], c0));
                const v4i hi4 = *reinterpret_cast<const v4i*>(la + lds_addr(arow[i], c0 + 1));
                fa[i] = (v8i){lo4.x, lo4.y, lo4.z, lo4.w, hi4.x, hi4.y, hi4.z, hi4.w};
            }
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const v4i lo4 = *reinterpret_cast<const v4i*>(lw + lds_addr(wrow[j], c0));
                const v4i hi4 = *reinterpret_cast<const v4i*>(lw + lds_addr(wrow[j], c0 + 1));
                fw[j] = (v8i){lo4.x, lo4.y, lo4.z, lo4.w, hi4.x, hi4.y, hi4.z, hi4.w};
            }
        };
        auto mfma_all = [&](const v8i* fa, const v8i* fw) {
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fw[j], fa[i], acc[i][j], 0, 0, 0,
                                                                                127, 0, 127);
        };
        auto interleave = [&]() {
#pragma unroll
            for (int i = 0; i < TM + TN; ++i) {
                SGB(SG_MFMA, 1);
                SGB(SG_DS_READ, 2);
            }
            SGB(SG_MFMA, TM * TN - (TM + TN));
            __builtin_amdgcn_sched_barrier(0);
        };
        auto stage = [&](int kt, auto refill) {
            const int slot = kt & 1;
            read_frags(fa1, fw1, slot, 1);
            mfma_all(fa0, fw0);
            interleave();
            handoff();
            if constexpr (decltype(refill)::value) issue_stage(kt + 2, slot);
            read_frags(fa0, fw0, slot ^ 1, 0);
            mfma_all(fa1, fw1);
            // the refill DMAs spread over the first MFMAs (measured 2-5%
            // faster than issuing them all before the first MFMA): each
            // MFMA of the k-step is followed by its share of the stage's
            // DMAs and, while they last, one fragment's two reads
            if constexpr (decltype(refill)::value) {
                constexpr int NM = TM * TN, NV = NDMA + NDMA_W;
                constexpr int VQ = NV / NM, VR = NV % NM;  // DMAs per MFMA, and the first VR MFMAs' extra one
#pragma unroll
                for (int i = 0; i < NM; ++i) {
                    SGB(SG_MFMA, 1);
                    if (i < VR) {
                        SGB(SG_VMEM, VQ + 1);
                    } else if constexpr (VQ > 0) {
                        SGB(SG_VMEM, VQ);
                    }
                    if (i < TM + TN) SGB(SG_DS_READ, 2);
                }
                __builtin_amdgcn_sched_barrier(0);
            } else {
                interleave();
            }
        };
        read_frags(fa0, fw0, 0, 0);
        int kt = 0;
        for (; kt + 2 < KT; ++kt) stage(kt, std::true_type{});
        for (; kt < KT; ++kt) stage(kt, std::false_type{});
    } else if constexpr (OP == OP_I8_16) {
        // Two 64-byte k-steps per stage of v_mfma_i32_16x16x64_i8 over the
        // wave's 8 x 4 blocks of 16x16: lane group q = lane/16 of a fragment
        // takes logical chunk 4s + q in k-step s (both operands alike), the
        // fragments of k-step s+1 read during k-step s, the refill DMAs
        // spread over the first MFMAs after the hand-off.
        v4i fa0[2 * TM], fw0[TN16], fa1[2 * TM], fw1[TN16];
        auto read_frags = [&](v4i* fa, v4i* fw, int slot, int ks) {
            const uint8_t* la = lds + slot * OP_BYTES;
            const uint8_t* lw = lds + (NSLOT + slot) * OP_BYTES;
            const int chunk = 4 * ks + q16;
#pragma unroll
            for (int i = 0; i < 2 * TM; ++i) fa[i] = *reinterpret_cast<const v4i*>(la + lds_addr(arow16[i], chunk));
#pragma unroll
            for (int j = 0; j < TN16; ++j) fw[j] = *reinterpret_cast<const v4i*>(lw + lds_addr(wrow16[j], chunk));
        };
        auto mfma_all = [&](const v4i* fa, const v4i* fw) {
#pragma unroll
            for (int i = 0; i < 2 * TM; ++i)
#pragma unroll
                for (int j = 0; j < TN16; ++j)
                    acc16[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fw[j], fa[i], acc16[i][j], 0, 0, 0);
        };
        constexpr int NF = 2 * TM + TN16;     // fragment reads per k-step
        constexpr int NM = 2 * TM * TN16;     // MFMAs per k-step
        auto interleave = [&]() {
#pragma unroll
            for (int i = 0; i < NF; ++i) {
                SGB(SG_MFMA, 1);
                SGB(SG_DS_READ, 1);
            }
            SGB(SG_MFMA, NM - NF);
            __builtin_amdgcn_sched_barrier(0);
        };
        auto stage = [&](int kt, auto refill) {
            const int slot = kt & 1;
            read_frags(fa1, fw1, slot, 1);
            mfma_all(fa0, fw0);
            interleave();
            handoff();
            if constexpr (decltype(refill)::value) issue_stage(kt + 2, slot);
            read_frags(fa0, fw0, slot ^ 1, 0);
            mfma_all(fa1, fw1);
            if constexpr (decltype(refill)::value) {
#pragma unroll
                for (int i = 0; i < NM; ++i) {
                    SGB(SG_MFMA, 1);
                    if (i < NDMA + NDMA_W) SGB(SG_VMEM, 1);
                    if (i < NF) SGB(SG_DS_READ, 1);
                }
                __builtin_amdgcn_sched_barrier(0);
            } else {
                interleave();
            }
        };
        read_frags(fa0, fw0, 0, 0);
        int kt = 0;
        for (; kt + 2 < KT; ++kt) stage(kt, std::true_type{});
        for (; kt < KT; ++kt) stage(kt, std::false_type{});
    }

    // Wait for every wave to leave the ring, then publish the epilogue
    // operands in ring space.
    wait_vmcnt<0>();
    __syncthreads();
    // Interior tiles (the common case) take paths with no per-element
    // bounds checks.
    const bool interior = (m0 + BM <= M) && (n0 + BN <= N) && ((N & 3) == 0);
    // (int8 launches are stored straight from the 16x16 blocks: the plain
    // path and the attention-layout paths below read acc16; the 32x32-layout
    // paths at the end serve e4m3 and bf16)
    if (tid < 256) {
        s_as[tid] = e_as;
        s_ws[tid] = e_ws;
        // an absent bias is -0.0f: adding it leaves every value unchanged
        // (-0.0 included), so the epilogue adds it without a select
        s_bias[tid] = has_bias ? bf16_to_f32(e_braw) : -0.0f;
        s_gate[tid] = e_gate;
    }
    __syncthreads();

    if constexpr (M16) {
      if (!HD || pr.hk == 0) {
        // Plain int8 launches: each lane holds 4 consecutive columns of one
        // row per 16x16 block (columns 16j + 4(l/16) .. +3 of row
        // 16i + l%16: D = W x A is indexed [n][m]). They are dequantized with
        // the arithmetic of the 32x32-layout paths below and written to the
        // wave's staging rows (32 at a time, padded by 16 bytes), which are
        // stored 16 bytes a lane, 1 KB per instruction; rows past M and
        // columns past N are skipped there. (Stored directly, 16 rows x 64
        // bytes per instruction, the fp32 GEMM measured 10-15% slower.)
        constexpr int ESZ = (OUT_DT == QIMG_FP32) ? 4 : 2;
        constexpr int ROWB = WTN * ESZ;
        constexpr int PITCH = ROWB + 16;
        constexpr int CPR = ROWB / 16;  // 16-byte chunks per staged row
        constexpr int EPC = 16 / ESZ;   // elements per chunk
        constexpr int NIT = 32 * CPR / 64;
        uint8_t* stage = lds + wave * (32 * PITCH);
        const bool gated = OUT_DT == QIMG_FP32 && has_gate;
        const bool vec = (N % EPC) == 0;
        const bool fast = interior && vec;  // (bf16 chunks need N % 8 == 0)
        // The weight scales and bias of the lane's columns stay in registers
        // for up to 4 blocks across; wider waves (7 blocks: 112 registers
        // with the residual prefetch beside 112 accumulators) read them from
        // LDS at each use instead.
        constexpr bool WREG = TN16 <= 4;
        v4f wv[WREG ? TN16 : 1], bv[WREG ? TN16 : 1];
        if constexpr (WREG) {
#pragma unroll
            for (int j = 0; j < TN16; ++j) {
                const int nl = wn * WTN + 16 * j + 4 * q16;
                wv[j] = *reinterpret_cast<const v4f*>(s_ws + nl);
                bv[j] = *reinterpret_cast<const v4f*>(s_bias + nl);
            }
        }
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int rb = m0 + wm * WTM + i * 32;  // first row of the block
            const int cb = n0 + wn * WTN;           // first column of the wave
            uint8_t* obase = reinterpret_cast<uint8_t*>(out) + (static_cast<int64_t>(rb) * N + cb) * ESZ;
            v4f res[NIT];
            if (gated) {
#pragma unroll
                for (int it = 0; it < NIT; ++it) {
                    const int idx = it * 64 + lane;
                    const int r = idx / CPR, c = cb + (idx % CPR) * EPC;
                    const float* o = reinterpret_cast<const float*>(obase + static_cast<int64_t>(r) * N * ESZ) +
                                     (idx % CPR) * EPC;
                    if (fast || (rb + r < M && vec && c + EPC <= N)) {
                        res[it] = *reinterpret_cast<const v4f*>(o);
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e) res[it][e] = (rb + r < M && c + e < N) ? o[e] : 0.0f;
                    }
                }
            }
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const int rl = 16 * b + (lane & 15);
                const float sa = s_as[wm * WTM + i * 32 + rl];
#pragma unroll
                for (int j = 0; j < TN16; ++j) {
                    const int nl = wn * WTN + 16 * j + 4 * q16;
                    const v4f wj = WREG ? wv[j] : *reinterpret_cast<const v4f*>(s_ws + nl);
                    const v4f bj = WREG ? bv[j] : *reinterpret_cast<const v4f*>(s_bias + nl);
                    float v[4];
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        const int e = acc16[2 * i + b][j][c];
                        float t;
                        {
#pragma clang fp contract(off)
                            t = static_cast<float>(e) * sa * wj[c];
                            t = t + bj[c];
                        }
                        if (GELU) t = gelu_tanh_fast(t);
                        v[c] = t;
                    }
                    uint8_t* dst = stage + rl * PITCH + (16 * j + 4 * q16) * ESZ;
                    if constexpr (OUT_DT == QIMG_FP32)
                        *reinterpret_cast<v4f*>(dst) = (v4f){v[0], v[1], v[2], v[3]};
                    else
                        *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
                }
            }
            // LDS operations of one wave complete in order; the empty asm
            // keeps the compiler from moving the reads above the writes.
            asm volatile("" ::: "memory");
#pragma unroll
            for (int it = 0; it < NIT; ++it) {
                const int idx = it * 64 + lane;
                const int r = idx / CPR;
                const int c16 = idx % CPR;
                const int c = cb + c16 * EPC;
                v4i val = *reinterpret_cast<const v4i*>(stage + r * PITCH + c16 * 16);
                if (gated) {
                    // gate_add_fp32f (cuda_kernels.cu:2181-2189): out + gate[n] * value
                    const v4f t = __builtin_bit_cast(v4f, val);
                    const v4f gv = *reinterpret_cast<const v4f*>(s_gate + wn * WTN + c16 * 4);
                    const v4f rv = res[it];
                    val = __builtin_bit_cast(v4i, (v4f){__builtin_fmaf(gv[0], t[0], rv[0]),
                                                        __builtin_fmaf(gv[1], t[1], rv[1]),
                                                        __builtin_fmaf(gv[2], t[2], rv[2]),
                                                        __builtin_fmaf(gv[3], t[3], rv[3])});
                }
                uint8_t* o = obase + static_cast<int64_t>(r) * N * ESZ + c16 * 16;
                if (fast || (rb + r < M && vec && c + EPC <= N)) {
                    *reinterpret_cast<v4i*>(o) = val;
                } else if (ESZ == 2 && (N & 3) == 0) {
                    // bf16 with N % 8 == 4: 8-byte halves (a chunk starts at
                    // a multiple of 8 columns, so each half is wholly in or
                    // out)
                    const u32x4 u = __builtin_bit_cast(u32x4, val);
                    if (rb + r < M && c + 4 <= N) *reinterpret_cast<uint2*>(o) = make_uint2(u[0], u[1]);
                    if (rb + r < M && c + 8 <= N) *reinterpret_cast<uint2*>(o + 8) = make_uint2(u[2], u[3]);
                } else if (rb + r < M) {
                    const u32x4 u = __builtin_bit_cast(u32x4, val);
#pragma unroll
                    for (int e = 0; e < EPC; ++e) {
                        if (c + e >= N) break;
                        const uint32_t word = u[(e * ESZ) / 4];
                        if constexpr (ESZ == 4)
                            reinterpret_cast<uint32_t*>(o)[e] = word;
                        else
                            reinterpret_cast<uint16_t*>(o)[e] = static_cast<uint16_t>(word >> (16 * (e & 1)));
                    }
                }
            }
            asm volatile("" ::: "memory");
        }
        return;
      }
    }

    if constexpr (HD && OUT_DT == QIMG_FP32 && !BF && !GELU) {
        if (pr.hk == HEADS_K || pr.hk == HEADS_Q) {
            // K or Q heads (the tile is two whole heads), in steps of 64 rows
            // (32 of each wave row wm): (A) every wave stores its dequantized
            // fp32 values in the shared tile T [64][256]; (B) wave w takes
            // tokens 8w .. 8w + 7 of the step, both heads: RMSNorm, RoPE and
            // fp16 with the arithmetic of joint_heads_f16_kernel (lane l holds
            // dims 2l, 2l + 1; the same wave sum and fused multiply-adds), K
            // stored at once, Q kept in R [64][2][128]; (C) for Q, waves 0-3
            // take one (32-token slice, head) each and quantize it as the
            // second phase of heads_quant_q_wave_kernel (lane 8g + j holds
            // dims 16j .. +16 of tokens g, g + 8, g + 16, g + 24). Rows past
            // M count as zeros, as tokens past S do there.
            constexpr int TP = BN + 4;      // T pitch (floats)
            constexpr int RP = 2 * 64 + 4;  // R pitch (32-bit words of two fp16)
            static_assert(64 * TP * 4 + 64 * RP * 4 <= SCALE_OFF, "heads staging overlaps the scales");
            float* T = reinterpret_cast<float*>(lds);
            uint32_t* R = reinterpret_cast<uint32_t*>(lds + 64 * TP * 4);
            const int H = pr.hH, S = pr.hS, hoff = pr.hoff, hn = pr.hn, hb0 = pr.hb0;
            const bool isq = pr.hk == HEADS_Q;
            const float heps = pr.heps;
            const float* __restrict__ pe = pr.hpe;
            const uint32_t wp = reinterpret_cast<const uint32_t*>(pr.hnorm)[lane];
            const float w0 = bf16_to_f32(static_cast<uint16_t>(wp & 0xffffu));
            const float w1 = bf16_to_f32(static_cast<uint16_t>(wp >> 16));
            const int hfirst = n0 >> 7;  // the tile's first head
            const int row = lane & 31;
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                // this step's tokens and their RoPE rows (the loads in flight
                // during (A))
                v4f p[8];
                int tb[8], ts[8];
                bool ok[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const int tr = wave * 8 + k;
                    const int r = m0 + (tr >> 5) * WTM + i * 32 + (tr & 31);
                    ok[k] = r < M;
                    const int q = ok[k] ? r / hn : 0;
                    tb[k] = hb0 + q;
                    ts[k] = hoff + (ok[k] ? r - q * hn : 0);
                    p[k] = ok[k] ? reinterpret_cast<const v4f*>(pe)[static_cast<int64_t>(ts[k]) * 64 + lane]
                                 : (v4f){0.0f, 0.0f, 0.0f, 0.0f};
                }
                // (A)
                if constexpr (M16) {
                    // (lane l of 16x16 block (2i + b, j) holds columns
                    // 16j + 4(l/16) .. +3 of row 16b + l%16 of the block)
#pragma unroll
                    for (int b = 0; b < 2; ++b) {
                        const int rl = 16 * b + (lane & 15);
                        const float sa = s_as[wm * WTM + i * 32 + rl];
#pragma unroll
                        for (int j = 0; j < TN16; ++j) {
                            const int nl = wn * WTN + 16 * j + 4 * q16;
                            const v4f wv = *reinterpret_cast<const v4f*>(s_ws + nl);
                            const v4f bb = *reinterpret_cast<const v4f*>(s_bias + nl);
                            float v[4];
#pragma unroll
                            for (int c = 0; c < 4; ++c) {
                                const int e = acc16[2 * i + b][j][c];
                                {
#pragma clang fp contract(off)
                                    v[c] = static_cast<float>(e) * sa * wv[c];
                                    v[c] = v[c] + bb[c];
                                }
                            }
                            *reinterpret_cast<v4f*>(T + (wm * 32 + rl) * TP + nl) = (v4f){v[0], v[1], v[2], v[3]};
                        }
                    }
                } else {
                    const float sa = s_as[wm * WTM + i * 32 + row];
#pragma unroll
                    for (int j = 0; j < TN; ++j)
#pragma unroll
                        for (int g = 0; g < 4; ++g) {
                            float v[4];
                            const int nl = wn * WTN + j * 32 + 4 * half + 8 * g;
                            const v4f wv = *reinterpret_cast<const v4f*>(s_ws + nl);
                            const v4f bb = *reinterpret_cast<const v4f*>(s_bias + nl);
#pragma unroll
                            for (int c = 0; c < 4; ++c) {
                                {
#pragma clang fp contract(off)
                                    v[c] = static_cast<float>(acc[i][j][4 * g + c]) * sa * wv[c];
                                    v[c] = v[c] + bb[c];
                                }
                            }
                            *reinterpret_cast<v4f*>(T + (wm * 32 + row) * TP + wn * WTN + j * 32 + 8 * g + 4 * half) =
                                (v4f){v[0], v[1], v[2], v[3]};
                        }
                }
                __syncthreads();
                // (B)
                {
                    // all 16 (token, head) rows computed in one branch-free
                    // block (their latencies overlap), then stored
                    uint32_t pk[16];
#pragma unroll
                    for (int u = 0; u < 16; ++u) {
                        const int k = u >> 1, hh = u & 1;
                        float2 y = *reinterpret_cast<const float2*>(T + (wave * 8 + k) * TP + hh * 128 + 2 * lane);
                        const float ss = wave_sum_dpp(__builtin_fmaf(y.x, y.x, y.y * y.y));
                        const float rms = rsqrtf(ss / 128 + heps);
                        y.x = y.x * rms * w0;
                        y.y = y.y * rms * w1;
                        const float o0 = __builtin_fmaf(y.x, p[k].x, y.y * p[k].y);
                        const float o1 = __builtin_fmaf(y.x, p[k].z, y.y * p[k].w);
                        pk[u] = static_cast<uint32_t>(f32_to_f16(o0)) | (static_cast<uint32_t>(f32_to_f16(o1)) << 16);
                    }
                    if (isq) {
#pragma unroll
                        for (int u = 0; u < 16; ++u)
                            R[(wave * 8 + (u >> 1)) * RP + (u & 1) * 64 + lane] = ok[u >> 1] ? pk[u] : 0u;
                    } else {
#pragma unroll
                        for (int u = 0; u < 16; ++u) {
                            const int k = u >> 1;
                            if (ok[k]) {
                                const int64_t bh = static_cast<int64_t>(tb[k]) * H + hfirst + (u & 1);
                                reinterpret_cast<uint32_t*>(out)[(bh * S + ts[k]) * 64 + lane] = pk[u];
                            }
                        }
                    }
                }
                __syncthreads();  // T is free for the next step; R is complete
                // (C)
                if (isq && wave < 4) {
                    const int blk = wave >> 1, hh = wave & 1;
                    const int r0 = m0 + blk * WTM + i * 32;
                    if (r0 < M) {
                        const int q0 = r0 / hn;
                        const int s0 = hoff + r0 - q0 * hn;  // a multiple of 32
                        const int64_t bh = static_cast<int64_t>(hb0 + q0) * H + hfirst + hh;
                        const int g = lane >> 3, jj = lane & 7;
                        uint32_t raw[4][8];
                        float amax = 0.0f;
#pragma unroll
                        for (int ii = 0; ii < 4; ++ii)
#pragma unroll
                            for (int c = 0; c < 8; ++c) {
                                raw[ii][c] = R[(blk * 32 + g + 8 * ii) * RP + hh * 64 + 8 * jj + c];
                                amax = fmaxf(amax, fabsf(f16_to_f32(static_cast<uint16_t>(raw[ii][c] & 0xffffu))));
                                amax = fmaxf(amax, fabsf(f16_to_f32(static_cast<uint16_t>(raw[ii][c] >> 16))));
                            }
#pragma unroll
                        for (int off = 1; off < 8; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
                        const float a = fmaxf(1e-7f, amax);  // the reference starts its max at 1e-7
                        const float scale = a / 127.0f + 1e-7f;
                        const int nq = ((S + 127) / 128) * 32;
                        const int slice = s0 >> 5;
                        if (jj == 0) pr.hqs[bh * nq + (slice >> 2) * 32 + (slice & 3) * 8 + g] = scale;
                        const float inv = 1.0f / scale;
#pragma unroll
                        for (int ii = 0; ii < 4; ++ii) {
                            if (r0 + g + 8 * ii >= M) continue;
                            u32x4 pk;
#pragma unroll
                            for (int wd = 0; wd < 4; ++wd) {
                                const uint32_t a0 = raw[ii][2 * wd], a1 = raw[ii][2 * wd + 1];
                                pk[wd] = i8x4_rne_sat(f16_to_f32(static_cast<uint16_t>(a0 & 0xffffu)) * inv,
                                                      f16_to_f32(static_cast<uint16_t>(a0 >> 16)) * inv,
                                                      f16_to_f32(static_cast<uint16_t>(a1 & 0xffffu)) * inv,
                                                      f16_to_f32(static_cast<uint16_t>(a1 >> 16)) * inv);
                            }
                            *reinterpret_cast<u32x4*>(reinterpret_cast<int8_t*>(out) +
                                                      (bh * S + s0 + g + 8 * ii) * 128 + 16 * jj) = pk;
                        }
                    }
                }
            }
            return;
        }
    }

    if constexpr (M16 && HD) {
        // V^T output (HEADS_V; K and Q returned above, plain problems before
        // them), every tile: each wave stages a 32-row block as fp16 in a
        // private LDS buffer from the 16x16 blocks, then lane l reads column
        // l (one head dim) down the 32 rows. When the rows are 32 consecutive
        // keys of one sequence starting at a multiple of 32, all below M,
        // they fill half of one key tile's 128-byte row for that dim: four
        // 16-byte stores in position order. Otherwise each value in range is
        // stored at its own position. (A wave's 64 columns lie in one head;
        // N is a multiple of 128, so they are all in range or all out.)
        constexpr int PH = WTN + 4;  // staging pitch in fp16 elements (136 bytes)
        uint16_t* stg = reinterpret_cast<uint16_t*>(lds + wave * (32 * PH * 2));
        uint16_t* vo = reinterpret_cast<uint16_t*>(out);
        const int vh = pr.hH, vS = pr.hS, voff = pr.hoff, vn = pr.hn, vb0 = pr.hb0;
        const int col = n0 + wn * WTN + lane;
        const bool cols_in = n0 + wn * WTN < N;
        v4f wv[TN16], bv[TN16];
#pragma unroll
        for (int j = 0; j < TN16; ++j) {
            const int nl = wn * WTN + 16 * j + 4 * q16;
            wv[j] = *reinterpret_cast<const v4f*>(s_ws + nl);
            bv[j] = *reinterpret_cast<const v4f*>(s_bias + nl);
        }
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const int rl = 16 * b + (lane & 15);
                const float sa = s_as[wm * WTM + i * 32 + rl];
#pragma unroll
                for (int j = 0; j < TN16; ++j) {
                    uint16_t hv[4];
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        const int e = acc16[2 * i + b][j][c];
                        float t;
                        {
#pragma clang fp contract(off)
                            t = static_cast<float>(e) * sa * wv[j][c];
                            t = t + bv[j][c];
                        }
                        hv[c] = f32_to_f16(t);
                    }
                    *reinterpret_cast<uint2*>(stg + rl * PH + 16 * j + 4 * q16) =
                        make_uint2(hv[0] | (static_cast<uint32_t>(hv[1]) << 16),
                                   hv[2] | (static_cast<uint32_t>(hv[3]) << 16));
                }
            }
            // LDS operations of one wave complete in order; the empty asm
            // keeps the compiler from moving the reads above the writes.
            asm volatile("" ::: "memory");
            const int r0 = m0 + wm * WTM + i * 32;
            if (cols_in && r0 < M) {
                const int b0 = r0 / vn;
                const int s0 = voff + r0 - b0 * vn;
                if (r0 + 32 <= M && (r0 + 31) / vn == b0 && (s0 & 31) == 0) {
                    uint16_t* dst = vo + vt_index(r0, col, vh, vS, voff, vn, vb0);
#pragma unroll
                    for (int qq = 0; qq < 4; ++qq) {
                        u32x4 w4;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int p = 8 * qq + 2 * e;
                            const int k = (p & ~12) | ((p & 4) << 1) | ((p & 8) >> 1);  // key at positions p, p + 1
                            w4[e] = stg[k * PH + lane] | (static_cast<uint32_t>(stg[(k + 1) * PH + lane]) << 16);
                        }
                        *reinterpret_cast<u32x4*>(dst + 8 * qq) = w4;
                    }
                } else {
                    for (int t = 0; t < 32 && r0 + t < M; ++t)
                        vo[vt_index(r0 + t, col, vh, vS, voff, vn, vb0)] = stg[t * PH + lane];
                }
            }
            asm volatile("" ::: "memory");  // the next block's writes go after these reads
        }
        return;
    }
    if constexpr (!M16) {
        // Epilogue. The MFMA was issued as D = W_frag x A_frag, so the 32x32
        // block is indexed [n][m]: lane holds m = lane%32 and n rows
        // 8*(r/4) + 4*(lane/32) + r%4. Each lane therefore owns one output row
        // per block and 16 columns in four runs of 4 consecutive n, stored as
        // one 16-byte (fp32) or 8-byte (bf16) write per run.
        // edge tiles still store whole 4-column groups with one vector store
        // when the row is in range (rows past M are skipped below)
        const bool vec_n = (N & 3) == 0;
        const bool vt = HD && OUT_DT == QIMG_FP32 && !BF && pr.hk == HEADS_V;
        if (interior && (vt || ((OUT_DT == QIMG_FP32 || !has_gate) && !accumulate))) {  // (no gate with bf16 outputs)
            // The lane's weight scales and bias stay in registers for up to
            // two blocks across; wider waves (3 blocks: 96 registers beside
            // 96 accumulators and the residual prefetch) read each run of 4
            // from LDS at its use instead.
            constexpr bool WREG = TN <= 2;
            float wsv[WREG ? TN : 1][16], bv[WREG ? TN : 1][16];
            if constexpr (WREG) {
#pragma unroll
                for (int j = 0; j < TN; ++j)
#pragma unroll
                    for (int q = 0; q < 16; ++q) {
                        const int nl = wn * WTN + j * 32 + 4 * half + 8 * (q >> 2) + (q & 3);
                        wsv[j][q] = s_ws[nl];
                        bv[j][q] = s_bias[nl];
                    }
            }
            if constexpr (HD) if (vt) {  // (HD instances are 256 wide: WREG)
                // V^T output: each wave stages a 32-row block as fp16 [row][column]
                // in a private LDS buffer, then lane l reads column l (one head dim)
                // down the 32 rows. When the rows are 32 consecutive keys of one
                // sequence starting at a multiple of 32 they fill half of one key
                // tile's 128-byte row for that dim: four 16-byte stores in position
                // order. Otherwise each value is stored at its own position.
                constexpr int PH = WTN + 4;  // staging pitch in fp16 elements (136 bytes)
                uint16_t* stg = reinterpret_cast<uint16_t*>(lds + wave * (32 * PH * 2));
                uint16_t* vo = reinterpret_cast<uint16_t*>(out);
                const int vh = pr.hH, vS = pr.hS, voff = pr.hoff, vn = pr.hn, vb0 = pr.hb0;
                const int row = lane & 31;
                const int col = n0 + wn * WTN + lane;
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    const float sa = s_as[wm * WTM + i * 32 + row];
#pragma unroll
                    for (int j = 0; j < TN; ++j)
#pragma unroll
                        for (int g = 0; g < 4; ++g) {
                            uint16_t h[4];
#pragma unroll
                            for (int c = 0; c < 4; ++c) {
                                float t;
                                {
#pragma clang fp contract(off)
                                    t = static_cast<float>(acc[i][j][4 * g + c]) * sa * wsv[j][4 * g + c];
                                    t = t + bv[j][4 * g + c];
                                }
                                if (GELU) t = gelu_tanh_fast(t);
                                h[c] = f32_to_f16(t);
                            }
                            *reinterpret_cast<uint2*>(stg + row * PH + j * 32 + 8 * g + 4 * half) =
                                make_uint2(h[0] | (static_cast<uint32_t>(h[1]) << 16), h[2] | (static_cast<uint32_t>(h[3]) << 16));
                        }
                    // LDS operations of one wave complete in order; the empty asm
                    // keeps the compiler from moving the reads above the writes.
                    asm volatile("" ::: "memory");
                    const int r0 = m0 + wm * WTM + i * 32;
                    const int b0 = r0 / vn;
                    const int s0 = voff + r0 - b0 * vn;
                    if ((r0 + 31) / vn == b0 && (s0 & 31) == 0) {
                        uint16_t* dst = vo + vt_index(r0, col, vh, vS, voff, vn, vb0);
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            u32x4 wv;
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                const int p = 8 * q + 2 * e;
                                const int k = (p & ~12) | ((p & 4) << 1) | ((p & 8) >> 1);  // key at positions p, p + 1
                                wv[e] = stg[k * PH + lane] | (static_cast<uint32_t>(stg[(k + 1) * PH + lane]) << 16);
                            }
                            *reinterpret_cast<u32x4*>(dst + 8 * q) = wv;
                        }
                    } else {
                        for (int t = 0; t < 32; ++t) vo[vt_index(r0 + t, col, vh, vS, voff, vn, vb0)] = stg[t * PH + lane];
                    }
                    asm volatile("" ::: "memory");  // the next block's writes go after these reads
                }
                return;
            }
            // Interior tiles: each wave stages one 32-row block at a time in a
            // private LDS buffer (rows padded by 16 bytes: conflict-free for both
            // the row-per-lane writes and the row-major reads), then stores it
            // row-contiguously, 1 KB (eight whole 128-byte lines) per store
            // instruction. The direct stores below touch 32 rows per instruction;
            // staging measured 3-6% faster for the whole fp32 GEMM at K = 3072,
            // bit-identical. A gated residual is read the same way, row by row,
            // each 32-row block's before its values are computed.
            constexpr int ESZ = (OUT_DT == QIMG_FP32) ? 4 : 2;
            constexpr int ROWB = WTN * ESZ;
            constexpr int PITCH = ROWB + 16;
            constexpr int CPR = ROWB / 16;  // 16-byte chunks per staged row
            constexpr int NIT = 32 * CPR / 64;  // 16-byte chunks per lane per 32-row block
            uint8_t* stage = lds + wave * (32 * PITCH);
            const bool gated = OUT_DT == QIMG_FP32 && has_gate;
            auto block_base = [&](int i) {
                return reinterpret_cast<uint8_t*>(out) +
                       (static_cast<int64_t>(m0 + wm * WTM + i * 32) * N + n0 + wn * WTN) * ESZ;
            };
            v4f res[NIT];
            auto load_res = [&](int i, v4f* r) {
                const uint8_t* b = block_base(i);
#pragma unroll
                for (int it = 0; it < NIT; ++it) {
                    const int idx = it * 64 + lane;
                    r[it] = *reinterpret_cast<const v4f*>(b + static_cast<int64_t>(idx / CPR) * N * ESZ + (idx % CPR) * 16);
                }
            };

            const int row = lane & 31;
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                if (gated) load_res(i, res);
                const float sa = s_as[wm * WTM + i * 32 + row];
#pragma unroll
                for (int j = 0; j < TN; ++j) {
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int nl = wn * WTN + j * 32 + 4 * half + 8 * g;
                        const v4f wg = WREG ? (v4f){wsv[j][4 * g], wsv[j][4 * g + 1], wsv[j][4 * g + 2], wsv[j][4 * g + 3]}
                                            : *reinterpret_cast<const v4f*>(s_ws + nl);
                        const v4f bg = WREG ? (v4f){bv[j][4 * g], bv[j][4 * g + 1], bv[j][4 * g + 2], bv[j][4 * g + 3]}
                                            : *reinterpret_cast<const v4f*>(s_bias + nl);
                        float v[4];
#pragma unroll
                        for (int c = 0; c < 4; ++c) {
                            float t;
                            if constexpr (BF) {
                                t = acc[i][j][4 * g + c] + bg[c];
                                if (GELU) t = gelu_tanh(t);
                            } else {
                                {
#pragma clang fp contract(off)
                                    t = static_cast<float>(acc[i][j][4 * g + c]) * sa * wg[c];
                                    t = t + bg[c];
                                }
                                if (GELU) t = gelu_tanh_fast(t);
                            }
                            v[c] = t;
                        }
                        uint8_t* dst = stage + row * PITCH + (j * 32 + 8 * g + 4 * half) * ESZ;
                        if (OUT_DT == QIMG_FP32)
                            *reinterpret_cast<v4f*>(dst) = (v4f){v[0], v[1], v[2], v[3]};
                        else
                            *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
                    }
                }
                // LDS operations of one wave complete in order; the empty asm
                // keeps the compiler from moving the reads above the writes.
                asm volatile("" ::: "memory");
                uint8_t* obase = block_base(i);
#pragma unroll
                for (int it = 0; it < NIT; ++it) {
                    const int idx = it * 64 + lane;
                    const int r = idx / CPR;
                    const int c16 = idx % CPR;
                    v4i val = *reinterpret_cast<const v4i*>(stage + r * PITCH + c16 * 16);
                    if (gated) {
                        // gate_add_fp32f (cuda_kernels.cu:2181-2189): out + gate[n] * value
                        const v4f t = __builtin_bit_cast(v4f, val);
                        const v4f gv = *reinterpret_cast<const v4f*>(s_gate + wn * WTN + c16 * 4);
                        const v4f rv = res[it];
                        val = __builtin_bit_cast(v4i, (v4f){__builtin_fmaf(gv[0], t[0], rv[0]), __builtin_fmaf(gv[1], t[1], rv[1]),
                                                            __builtin_fmaf(gv[2], t[2], rv[2]), __builtin_fmaf(gv[3], t[3], rv[3])});
                    }
                    *reinterpret_cast<v4i*>(obase + static_cast<int64_t>(r) * N * ESZ + c16 * 16) = val;
                }
                asm volatile("" ::: "memory");
            }
            return;
        }
        // V^T output: each of this lane's rows' offset at dim 0 of the wave's
        // head (the wave's WTN columns lie in one head)
        int64_t vrow[TM];
        if (vt) {
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int m = m0 + wm * WTM + i * 32 + (lane & 31);
                vrow[i] = m < M ? vt_index(m, (n0 + wn * WTN) & ~127, pr.hH, pr.hS, pr.hoff, pr.hn, pr.hb0) : 0;
            }
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int nj = n0 + wn * WTN + j * 32 + 4 * half;
            float wsv[16], bv[16], gv[16];
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int nl = nj - n0 + 8 * g + c;
                    wsv[4 * g + c] = s_ws[nl];
                    bv[4 * g + c] = s_bias[nl];
                    gv[4 * g + c] = s_gate[nl];
                }
            // Gated residual (gate_add_fp32f, cuda_kernels.cu:2181-2189), or the
            // values a bf16 product accumulates onto: the tile's old values are
            // all loaded before its first store.
            v4f res[TM][4];
            if (OUT_DT == QIMG_FP32 && (has_gate || accumulate)) {
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    const int m = m0 + wm * WTM + i * 32 + (lane & 31);
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int nb = nj + 8 * g;
                        const float* o = reinterpret_cast<const float*>(out) + static_cast<int64_t>(m) * N + nb;
                        if (interior || (m < M && vec_n && nb + 4 <= N)) {
                            res[i][g] = *reinterpret_cast<const v4f*>(o);
                        } else {
#pragma unroll
                            for (int c = 0; c < 4; ++c) res[i][g][c] = (m < M && nb + c < N) ? o[c] : 0.0f;
                        }
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int m = m0 + wm * WTM + i * 32 + (lane & 31);
                if (!interior && m >= M) continue;
                const float sa = s_as[m - m0];
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int nb = nj + 8 * g;
                    float v[4];
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        float t;
                        if constexpr (BF) {
                            // (linear_forward_bf16 order: GEMM with beta = 1,
                            // then bias_add_fp32, then gelu_fp32)
                            t = acc[i][j][4 * g + c];
                            if (OUT_DT == QIMG_FP32 && accumulate) t = t + res[i][g][c];
                            t = t + bv[4 * g + c];
                            if (GELU) t = gelu_tanh(t);
                        } else {
                            {
#pragma clang fp contract(off)
                                t = static_cast<float>(acc[i][j][4 * g + c]) * sa * wsv[4 * g + c];
                                t = t + bv[4 * g + c];
                            }
                            if (GELU) t = gelu_tanh_fast(t);
                            if (OUT_DT == QIMG_FP32 && has_gate) t = __builtin_fmaf(gv[4 * g + c], t, res[i][g][c]);
                        }
                        v[c] = t;
                    }
                    if (vt) {
                        // (nb .. nb + 3 lie in one head: row base + dim * 64)
                        uint16_t* o = reinterpret_cast<uint16_t*>(out) + vrow[i] + static_cast<int64_t>(nb & 127) * 64;
#pragma unroll
                        for (int c = 0; c < 4; ++c)
                            if (nb + c < N) o[64 * c] = f32_to_f16(v[c]);
                    } else if (OUT_DT == QIMG_FP32) {
                        float* o = reinterpret_cast<float*>(out) + static_cast<int64_t>(m) * N + nb;
                        if (interior || (vec_n && nb + 4 <= N)) {
                            *reinterpret_cast<v4f*>(o) = (v4f){v[0], v[1], v[2], v[3]};
                        } else {
#pragma unroll
                            for (int c = 0; c < 4; ++c)
                                if (nb + c < N) o[c] = v[c];
                        }
                    } else {
                        uint16_t* o = reinterpret_cast<uint16_t*>(out) + static_cast<int64_t>(m) * N + nb;
                        if (interior || (vec_n && nb + 4 <= N)) {
                            *reinterpret_cast<uint2*>(o) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
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

// Stand-alone dequant epilogue for an int32 product held in memory
// (dequantize_and_bias / dequantize_bias_gelu, cuda_kernels.cu:2623-2668):
// the same per-element arithmetic as the fused epilogue above, so a caller
// that runs its own integer GEMM gets bit-identical output.
__global__ __launch_bounds__(256) void dequant_bias_kernel(const int32_t* __restrict__ acc,
                                                           const float* __restrict__ as,
                                                           const float* __restrict__ ws,
                                                           const uint16_t* __restrict__ bias,
                                                           float* __restrict__ out, int M, int N,
                                                           int gelu) {
    const int64_t total = static_cast<int64_t>(M) * N;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
        const int m = static_cast<int>(i / N);
        const int n = static_cast<int>(i - static_cast<int64_t>(m) * N);
        float t;
        {
#pragma clang fp contract(off)
            t = static_cast<float>(acc[i]) * as[m] * ws[n];
            if (bias) t = t + bf16_to_f32(bias[n]);
        }
        if (gelu) t = gelu_tanh_fast(t);
        out[i] = t;
    }
}

// tw: the tile width, BN, MID_BN (int8) or NARROW_BN (int8, e4m3, bf16);
// narrower tiles take no attention-layout outputs. Every problem's tile
// count is checked against the width before the launch.
template <int OP, int OUT_DT, bool GELU>
hipError_t launch_tiled(const TileProblems& P, hipStream_t stream, int tw = BN, int th = BM) {
    bool hd = false;
    int64_t total = 0;
    for (int i = 0; i < P.n; ++i) {
        const TileProblem& p = P.p[i];
        hd = hd || p.hk > 0;
        // every problem's tiles counted for the tile size launched
        if (tw <= 0 || th <= 0 || p.tiles != ((p.M + th - 1) / th) * ((p.N + tw - 1) / tw))
            return hipErrorInvalidValue;
        total += p.tiles;
    }
    if (total != P.total) return hipErrorInvalidValue;
    if (th != BM) {
        if constexpr (OP == OP_I8_16) {
            if (hd || th != SMALL_BM || tw != SMALL_BM) return hipErrorInvalidValue;
            hipLaunchKernelGGL((gemm_w8a8_kernel<OP, OUT_DT, GELU, false, SMALL_BM, SMALL_BM>), dim3(P.total),
                               dim3(256), 0, stream, P);
            return hipGetLastError();
        }
        return hipErrorInvalidValue;
    }
    if (tw != BN) {
        if (hd) return hipErrorInvalidValue;
        if constexpr (OP == OP_I8_16 || OP == OP_F8 || OP == OP_BF16) {
            if (tw == NARROW_BN) {
                hipLaunchKernelGGL((gemm_w8a8_kernel<OP, OUT_DT, GELU, false, NARROW_BN>), dim3(P.total), dim3(NTHR),
                                   0, stream, P);
                return hipGetLastError();
            }
        }
        if constexpr (OP == OP_I8_16) {
            if (tw == MID_BN) {
                hipLaunchKernelGGL((gemm_w8a8_kernel<OP, OUT_DT, GELU, false, MID_BN>), dim3(P.total), dim3(NTHR), 0,
                                   stream, P);
                return hipGetLastError();
            }
        }
        return hipErrorInvalidValue;
    } else if (hd) {
        if constexpr (OUT_DT == QIMG_FP32 && !GELU && OP != OP_BF16)
            hipLaunchKernelGGL((gemm_w8a8_kernel<OP, OUT_DT, GELU, true>), dim3(P.total), dim3(NTHR), 0, stream, P);
        else
            return hipErrorInvalidValue;
    } else {
        hipLaunchKernelGGL((gemm_w8a8_kernel<OP, OUT_DT, GELU>), dim3(P.total), dim3(NTHR), 0, stream, P);
    }
    return hipGetLastError();
}

// One or two problems as a TileProblems (p1.tiles may be 0).
TileProblems problems(const TileProblem& p0, const TileProblem& p1) {
    TileProblems P{};
    P.p[0] = p0;
    P.n = 1;
    if (p1.tiles > 0) P.p[P.n++] = p1;
    P.total = p0.tiles + p1.tiles;
    return P;
}

// bn, bm: the tile size the problem will be launched with (BN, MID_BN or
// NARROW_BN wide; BM or SMALL_BM high)
TileProblem tile_problem(const void* a, const float* as, int M, int K, const void* w, const float* ws, int N,
                         const uint16_t* bias, void* out, const float* gate, int bn = BN, int bm = BM) {
    return {static_cast<const uint8_t*>(a), static_cast<const uint8_t*>(w), as, ws, bias, out, gate, M, N, K,
            ((M + bm - 1) / bm) * ((N + bn - 1) / bn), 0};
}

// tw, th must be the tile size P's tile counts were computed for
// (tile_problem's bn, bm).
template <bool FP8>
hipError_t dispatch_tiled(const TileProblems& P, int out_dt, int gelu, hipStream_t stream, int tw, int th = BM) {
    constexpr int OP = FP8 ? OP_F8 : OP_I8_16;
    if (out_dt == QIMG_FP32)
        return gelu ? launch_tiled<OP, QIMG_FP32, true>(P, stream, tw, th)
                    : launch_tiled<OP, QIMG_FP32, false>(P, stream, tw, th);
    return gelu ? launch_tiled<OP, QIMG_BF16, true>(P, stream, tw, th)
                : launch_tiled<OP, QIMG_BF16, false>(P, stream, tw, th);
}

}  // namespace

static std::atomic<int> g_linear_kernel{QIMG_LINEAR_AUTO};

// Compute units of the current device (queried once per device).
int device_cu_count() {
    constexpr int kMaxDev = 64;
    static std::atomic<int> cache[kMaxDev];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return 0;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
        cache[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

// Tiles of w columns and h rows that cover M x N.
static int64_t tiles_of(int M, int N, int w, int h = BM) {
    return static_cast<int64_t>((M + h - 1) / h) * ((N + w - 1) / w);
}

// The cost of running `tiles` tiles of width w, in 256x256-tile-widths of
// the slowest CU: its rounds of the CUs, each weighted by the tile's share
// of a 256x256 tile's work.
static int64_t tile_cost(int64_t tiles, int w, int cus) { return (tiles + cus - 1) / cus * w; }

// The tile with the least tile_cost for `tiles_wh(w, h)` tiles of w x h
// (the largest of equals): 256 rows of 256, 224 or 192 columns, or int8
// 128 x 128 (two workgroups per CU: 2 x cus tiles a round, each round half
// a 256 x 256 round's time); the kernels on 32x32 blocks (e4m3, bf16) take
// 256 or 192 columns (a 224-wide tile's waves do not divide into them).
struct TileSize {
    int tw, th;
};
template <class F>
static TileSize best_tile(F tiles_wh, int cus, bool blocks32) {
    TileSize best{BN, BM};
    int64_t c_best = tile_cost(tiles_wh(BN, BM), BN, cus);
    const TileSize cand[3] = {{MID_BN, BM}, {NARROW_BN, BM}, {SMALL_BM, SMALL_BM}};
    for (const TileSize& t : cand) {
        if (blocks32 && t.tw != NARROW_BN) continue;
        const int64_t c = t.th == SMALL_BM ? tile_cost(tiles_wh(t.tw, t.th), SMALL_BM, 2 * cus)
                                           : tile_cost(tiles_wh(t.tw, t.th), t.tw, cus);
        if (c < c_best) {
            c_best = c;
            best = t;
        }
    }
    return best;
}

// The large-tile plan of an automatic choice (K % 128 == 0, not a small-M
// case): rows [0, m_big) on the large tiles, the rest on smaller ones (int8:
// 128x128 tiles, e4m3: the 64x64 kernel), and the tile width.
//  - One tile per CU at a time. When the last round of 256x256 tiles would
//    be mostly idle, the trailing tile rows (at most two) go to the smaller
//    tiles, which spread them over every CU (M = 4352 = 4096 + 256 rows,
//    N = 12288: 816 tiles = 3 rounds + 48 tiles; the 48 become 192 tiles of
//    128x128, or 768 of 64x64).
//  - Otherwise the tile whose rounds, each weighted by the tile's share of
//    a 256x256 tile's time, add up to least (best_tile): 4096 x 3072 runs
//    256 tiles of 256x192 in one round (192 tiles of 256x256 leave a quarter
//    of the CUs idle), int8 4352 x 3072 238 tiles of 256x224 (204 of
//    256x256, 272 of 256x192), 4096 x 12288 stays on 256x256 (3 rounds; 4
//    of 256x192), 6889 x 3072 432 tiles of 256x192 (two rounds, as 324 of
//    256x256), int8 2048 x 3072 384 tiles of 128x128 (one round of two per
//    CU).
struct LargePlan {
    int m_big;
    int tw;
    int th = BM;
};
static LargePlan large_plan(int M, int N, int K, bool fp8) {
    LargePlan plan{M, BN};
    const int cus = device_cu_count();
    if (cus <= 0) return plan;
    const int tiles_n = (N + BN - 1) / BN;
    const int tiles_m = (M + BM - 1) / BM;
    const int64_t total = static_cast<int64_t>(tiles_m) * tiles_n;
    const int64_t rounds = (total + cus - 1) / cus;
    const int64_t tail = total - (rounds - 1) * cus;
    if (rounds > 1 && tail * 2 < cus) {
        for (int r = 1; r <= 2 && r < tiles_m; ++r) {
            if (static_cast<int64_t>(tiles_m - r) * tiles_n <= (rounds - 1) * cus) {
                plan.m_big = (tiles_m - r) * BM;
                break;
            }
        }
    }
    if (plan.m_big < M && !small_m_fits(M - plan.m_big, N, K)) plan.m_big = M;
    if (plan.m_big == M) {
        const TileSize t = best_tile([&](int w, int h) { return tiles_of(M, N, w, h); }, cus, fp8);
        plan.tw = t.tw;
        plan.th = t.th;
    }
    return plan;
}

// bf16 x [M, K] times w [N, K]^T into fp32 out with the large tiles (K %
// 64 == 0), as linear_forward_bf16_bf16in computes it: out (+)= product,
// then + bias, then GELU. The tile width (256 or 192) by best_tile, or as
// QIMG_LINEAR_LARGE_TILE / QIMG_LINEAR_LARGE_192 force it.
hipError_t launch_gemm_bf16_large(const uint16_t* x, int M, int K, const uint16_t* w, int N, const uint16_t* bias,
                                  float* out, int gelu, int accumulate, hipStream_t stream) {
    if (M == 0 || N == 0) return hipSuccess;
    if ((K * 2) % BK != 0) return hipErrorInvalidValue;
    const int choice = g_linear_kernel.load(std::memory_order_relaxed);
    const int cus = device_cu_count();
    const int tw = choice == QIMG_LINEAR_LARGE_TILE ? BN
                   : choice == QIMG_LINEAR_LARGE_192 ? NARROW_BN
                   : cus > 0 ? best_tile([&](int w_, int h_) { return tiles_of(M, N, w_, h_); }, cus, true).tw
                             : BN;
    TileProblem p0 = tile_problem(x, nullptr, M, K * 2, w, nullptr, N, bias, out, nullptr, tw);
    p0.accumulate = accumulate;
    const TileProblems P = problems(p0, TileProblem{});
    return gelu ? launch_tiled<OP_BF16, QIMG_FP32, true>(P, stream, tw)
                : launch_tiled<OP_BF16, QIMG_FP32, false>(P, stream, tw);
}

int set_linear_kernel(int which) { return g_linear_kernel.exchange(which); }

int get_linear_kernel() { return g_linear_kernel.load(); }

hipError_t launch_dequant_bias(const int32_t* acc, const float* as, const float* ws, const uint16_t* bias,
                              float* out, int M, int N, int gelu, hipStream_t stream) {
    const int64_t total = static_cast<int64_t>(M) * N;
    if (total == 0) return hipSuccess;
    const int64_t want = (total + 255) / 256;
    const int blocks = static_cast<int>(want < 16384 ? want : 16384);
    hipLaunchKernelGGL(dequant_bias_kernel, dim3(blocks), dim3(256), 0, stream, acc, as, ws, bias, out, M, N,
                       gelu);
    return hipGetLastError();
}

hipError_t launch_linear_prequantized(const void* act_q, const float* act_scales, int M, int K,
                                      const void* w_q, const float* w_scales, int N, int mode,
                                      const uint16_t* bias, void* out, int out_dtype, int gelu,
                                      hipStream_t stream, const float* gate, float* tmp) {
    if (M == 0 || N == 0) return hipSuccess;
    if (gate != nullptr && (out_dtype != QIMG_FP32 || tmp == nullptr)) return hipErrorInvalidValue;
    const bool fp8 = (mode == QIMG_QM_FP8_HADAMARD);
    // Rows [r0, M) computed by a kernel without the gated epilogue: into
    // tmp, then out = out + gate * tmp.
    auto gate_rest = [&](int r0) -> hipError_t {
        const int64_t off = static_cast<int64_t>(r0) * N;
        float* o = static_cast<float*>(out) + off;
        return launch_gate_add(o, gate, tmp + off, o, M - r0, N, stream);
    };
    const int choice = g_linear_kernel.load(std::memory_order_relaxed);
    int small = small_m_variant(M, N, K);
    if ((K % 64) == 0 && choice != QIMG_LINEAR_AUTO)
        small = choice == QIMG_LINEAR_SMALL_32 ? 1
                : choice == QIMG_LINEAR_SMALL_64 ? 2
                : choice == QIMG_LINEAR_GEMV     ? 3
                                                 : 0;
    // int8 of at least 128 rows and kMidTileMin tiles of 256x256 takes the
    // large-tile plan, which includes 128x128 tiles (at 32-63 tiles they
    // measured faster than the 64x64 ones: 1024 x 3072 x 3072 19.2 against
    // 23.4 us; below 128 rows most of such a tile would be empty)
    if (choice == QIMG_LINEAR_AUTO && !fp8 && small == 2 && (K % BK) == 0 && M >= SMALL_BM &&
        tiles_of(M, N, BN) >= kMidTileMin)
        small = 0;
    // the large tiles need K % 128 == 0; other multiples of 64 take 64x64 tiles
    if (small == 0 && (K % BK) != 0 && small_m_fits(M, N, K)) small = 2;
    if (small != 0) {
        hipError_t e = launch_linear_small_m(act_q, act_scales, M, K, w_q, w_scales, N, mode, bias,
                                             gate ? tmp : out, out_dtype, gelu, small, stream);
        return e != hipSuccess || !gate ? e : gate_rest(0);
    }
    if ((K % BK) == 0) {
        // (large_plan: the tail-row split and the tile width)
        LargePlan plan{M, choice == QIMG_LINEAR_LARGE_192           ? NARROW_BN
                          : choice == QIMG_LINEAR_LARGE_224 && !fp8 ? MID_BN
                          : choice == QIMG_LINEAR_LARGE_128 && !fp8 ? SMALL_BM
                                                                    : BN};
        if (choice == QIMG_LINEAR_LARGE_128 && !fp8) plan.th = SMALL_BM;
        if (choice == QIMG_LINEAR_AUTO) plan = large_plan(M, N, K, fp8);
        const int m_big = plan.m_big;
        const TileProblems P = problems(
            tile_problem(act_q, act_scales, m_big, K, w_q, w_scales, N, bias, out, gate, plan.tw, plan.th),
            TileProblem{});
        hipError_t e = fp8 ? dispatch_tiled<true>(P, out_dtype, gelu, stream, plan.tw, plan.th)
                           : dispatch_tiled<false>(P, out_dtype, gelu, stream, plan.tw, plan.th);
        if (e != hipSuccess || m_big == M) return e;
        const int esz = out_dtype == QIMG_FP32 ? 4 : 2;
        if (!fp8) {
            // int8 tail rows on 128x128 tiles, with the gated epilogue when
            // there is one (the fc1 tail at 4352 x 12288 x 3072: 192 tiles,
            // 21.4 against 23.1 us on the 64x64 kernel)
            const TileProblems Pt = problems(
                tile_problem(static_cast<const uint8_t*>(act_q) + static_cast<int64_t>(m_big) * K, act_scales + m_big,
                             M - m_big, K, w_q, w_scales, N, bias,
                             static_cast<uint8_t*>(out) + static_cast<int64_t>(m_big) * N * esz, gate, SMALL_BM,
                             SMALL_BM),
                TileProblem{});
            return dispatch_tiled<false>(Pt, out_dtype, gelu, stream, SMALL_BM, SMALL_BM);
        }
        void* rest = gate ? static_cast<void*>(tmp + static_cast<int64_t>(m_big) * N)
                          : static_cast<void*>(static_cast<uint8_t*>(out) + static_cast<int64_t>(m_big) * N * esz);
        e = launch_linear_small_m(static_cast<const uint8_t*>(act_q) + static_cast<int64_t>(m_big) * K,
                                  act_scales + m_big, M - m_big, K, w_q, w_scales, N, mode, bias, rest, out_dtype,
                                  gelu, 2, stream);
        return e != hipSuccess || !gate ? e : gate_rest(m_big);
    }
    const int64_t total = static_cast<int64_t>(M) * N;
    const int blocks = static_cast<int>((total + 255) / 256);
    if (fp8) return hipErrorInvalidValue;  // e4m3 needs K % 64 == 0 (checked by the caller) and fitting sizes
    hipLaunchKernelGGL(gemm_i8_simple_kernel, dim3(blocks), dim3(256), 0, stream,
                       static_cast<const int8_t*>(act_q), static_cast<const int8_t*>(w_q),
                       act_scales, w_scales, bias, gate ? static_cast<void*>(tmp) : out, M, N, K, out_dtype, gelu);
    hipError_t e = hipGetLastError();
    return e != hipSuccess || !gate ? e : gate_rest(0);
}

// Two linears of the same mode, output type and epilogue in one launch
// when the second one's tiles fit into the first one's last round
// (transformer.cu runs the image- and text-stream linears of a block back to
// back: at 4096 image tokens the N = 3072 linears are 192 tiles on 256 CUs,
// and the text stream's 256 rows are one more tile row). Otherwise the two
// run one after the other through launch_linear_prequantized. Each output
// element is computed exactly as in a launch of its own.
hipError_t launch_linear_pair(const LinearArgs& a, const LinearArgs& b, int mode, int out_dtype, int gelu,
                              hipStream_t stream) {
    auto single = [&](const LinearArgs& x) {
        return launch_linear_prequantized(x.act_q, x.act_scales, x.M, x.K, x.w_q, x.w_scales, x.N, mode, x.bias,
                                          x.out, out_dtype, gelu, stream, x.gate, x.tmp);
    };
    const bool fp8 = mode == QIMG_QM_FP8_HADAMARD;
    // (int8 images of at least kMidTileMin tiles of 256x256 pair up too: on
    // 128x128 tiles when those are best)
    bool pair = a.M > 0 && a.N > 0 && b.M > 0 && b.N > 0 &&
                g_linear_kernel.load(std::memory_order_relaxed) == QIMG_LINEAR_AUTO && (a.K % BK) == 0 &&
                (b.K % BK) == 0 &&
                (small_m_variant(a.M, a.N, a.K) == 0 ||
                 (!fp8 && a.M >= SMALL_BM && tiles_of(a.M, a.N, BN) >= kMidTileMin));
    TileSize ts{BN, BM};
    if (pair) {
        const int cus = device_cu_count();
        const int64_t ta = tiles_of(a.M, a.N, BN);
        const int64_t tb = tiles_of(b.M, b.N, BN);
        const int64_t rounds = cus > 0 ? (ta + cus - 1) / cus : 0;
        const int64_t tail = ta - (rounds - 1) * cus;
        // no extra round, and not a case for the tail-row split of a lone launch
        pair = cus > 0 && ta + tb <= rounds * cus && !(rounds > 1 && tail * 2 < cus);
        // the tile for both (int8 4096 + 256 rows of N = 3072: 238 tiles of
        // 256x224 in one round, against 204 of 256x256)
        if (pair)
            ts = best_tile([&](int w, int h) { return tiles_of(a.M, a.N, w, h) + tiles_of(b.M, b.N, w, h); }, cus,
                           fp8);
    }
    if (!pair) {
        hipError_t e = a.M > 0 ? single(a) : hipSuccess;
        return e != hipSuccess || b.M == 0 ? e : single(b);
    }
    if ((a.gate || b.gate) && out_dtype != QIMG_FP32) return hipErrorInvalidValue;
    const TileProblem p0 =
        tile_problem(a.act_q, a.act_scales, a.M, a.K, a.w_q, a.w_scales, a.N, a.bias, a.out, a.gate, ts.tw, ts.th);
    const TileProblem p1 =
        tile_problem(b.act_q, b.act_scales, b.M, b.K, b.w_q, b.w_scales, b.N, b.bias, b.out, b.gate, ts.tw, ts.th);
    const TileProblems P = problems(p0, p1);
    return fp8 ? dispatch_tiled<true>(P, out_dtype, gelu, stream, ts.tw, ts.th)
               : dispatch_tiled<false>(P, out_dtype, gelu, stream, ts.tw, ts.th);
}

// Up to kMaxProblems linears of one mode, output type and epilogue in one
// launch of the large tiles (the joint block's q, k and v of both streams: at
// 4096 + 256 tokens each pair is 204 tiles on 256 CUs, together 612 tiles in
// 2.4 rounds instead of three launches of one round each; 4352 x 9216 x 3072
// measured 131 us against 3 x 48 us). Returns hipErrorNotSupported, having
// launched nothing, when the kernel choice is not automatic, a linear does
// not fit the large tiles or the whole launch has fewer tiles than a single
// linear needs to be given the large tiles (small_m_variant's threshold); the
// caller then runs them one by one. Each output element is computed exactly
// as in a launch of its own.
static_assert(kMaxLinearMulti == kMaxProblems, "the multi-linear limit is the launch's problem table");

static hipError_t build_linear_multi(const LinearArgs* list, int n, int out_dtype, int gelu, TileProblems& P) {
    if (n < 1 || n > kMaxProblems || g_linear_kernel.load(std::memory_order_relaxed) != QIMG_LINEAR_AUTO)
        return hipErrorNotSupported;
    P = TileProblems{};
    for (int i = 0; i < n; ++i) {
        const LinearArgs& a = list[i];
        if (a.M <= 0 || a.N <= 0 || (a.K % BK) != 0) return hipErrorNotSupported;
        if (a.gate && out_dtype != QIMG_FP32) return hipErrorInvalidValue;
        TileProblem t = tile_problem(a.act_q, a.act_scales, a.M, a.K, a.w_q, a.w_scales, a.N, a.bias, a.out, a.gate);
        if (a.heads != nullptr) {
            const HeadsOut& h = *a.heads;
            const bool qk = h.kind == HEADS_K || h.kind == HEADS_Q;
            if (out_dtype != QIMG_FP32 || gelu || a.gate || h.kind < HEADS_V || h.kind > HEADS_Q || h.heads <= 0 ||
                a.N != 128 * h.heads || h.n <= 0 || a.M % h.n != 0 || h.off < 0 || h.off + h.n > h.S || h.b0 < 0 ||
                (qk && (h.norm == nullptr || h.pe == nullptr || a.N % BN != 0)) ||
                (h.kind == HEADS_Q && (h.q_scale == nullptr || h.off % 32 != 0 || (a.M != h.n && h.n % 32 != 0))))
                return hipErrorInvalidValue;
            t.hk = h.kind;
            t.hH = h.heads;
            t.hS = h.S;
            t.hoff = h.off;
            t.hn = h.n;
            t.hb0 = h.b0;
            t.hnorm = h.norm;
            t.hpe = h.pe;
            t.hqs = h.q_scale;
            t.heps = h.eps;
        }
        P.p[P.n++] = t;
        P.total += t.tiles;
    }
    // as many tiles as a lone linear needs to be given the large tiles
    // (a problem of one sequence's rows may be smaller: C5's per-sequence Q
    // slices of 2025 rows at batch 2 are 96 tiles each)
    if (P.total < kSmallMTileLimit) return hipErrorNotSupported;
    return hipSuccess;
}

hipError_t check_linear_multi(const LinearArgs* list, int n, int out_dtype, int gelu) {
    TileProblems P;
    return build_linear_multi(list, n, out_dtype, gelu, P);
}

hipError_t launch_linear_multi(const LinearArgs* list, int n, int mode, int out_dtype, int gelu,
                               hipStream_t stream) {
    TileProblems P;
    const hipError_t r = build_linear_multi(list, n, out_dtype, gelu, P);
    if (r != hipSuccess) return r;
    return mode == QIMG_QM_FP8_HADAMARD ? dispatch_tiled<true>(P, out_dtype, gelu, stream, BN)
                                        : dispatch_tiled<false>(P, out_dtype, gelu, stream, BN);
}

}  // namespace qimg
