// mmdit_block.hip — one MMDiT joint block (transformer.cu:506-817) as a
// sequence of this library's kernels on one stream.
//
// Differences from the reference's order of work, none of which changes a
// value:
//  - the two modulation linears (img_mod, txt_mod) share one activation
//    quantization of silu(t_emb) (the reference quantizes the same vector
//    twice);
//  - RMSNorm + concat/transpose + RoPE of Q and K is one kernel per tensor,
//    and the V concat/transpose writes fp16 only (the fp32 copy the
//    reference also writes feeds nothing on the Sage path);
//  - the attention writes fp16 and the split reads it (the reference
//    widens to fp32 first; fp16 -> fp32 is exact);
//  - the LayerNorm + modulate before QKV and before fc1 writes the int8
//    input of those linears directly (no fp32 copy of the normalized rows);
//  - the gated residuals after the out-projection and after fc2 are applied
//    in the GEMM epilogue (one fused multiply-add, as the gate-add kernel);
//  - the image- and text-stream linears of q, k, v, out-proj and fc2 share
//    a launch when the text tiles fit the image GEMM's last tile round;
//  - the K mean and the K quantization run on a second stream, beside
//    the Q and V preparation and the Q quantization (fork and join by events, which a graph
//    capture of the calling stream records as dependencies);
//  - buffers whose producer has been consumed are reused (q/k/v of each
//    stream hold the attention output, the projection and the MLP output);
//  - `batch` sequences of equal lengths that share t_emb and pe (the two
//    classifier-free-guidance forwards of main.cu:761-773) can run as one:
//    the linears see batch * n rows, the attention batch * 24 heads; each
//    row and head computes exactly what it computes alone.
#include "qimg_device.h"
#include "qimg_internal.h"

namespace qimg {

namespace {

constexpr int DIM = 3072;
constexpr int HEADS = 24;
constexpr int HEAD_DIM = 128;
constexpr int MLP = 12288;
constexpr float EPS = 1e-6f;

inline int64_t al256(int64_t b) { return (b + 255) & ~int64_t{255}; }

// A second stream (default priority) and two events per device and host
// thread, created on first use and kept for the life of the process: the K
// mean (a sequential sum that keeps 48-96 CUs busy for tens of
// microseconds) runs beside the Q/V preparation. Thread-local, so that
// concurrent callers never share an event.
struct SideStream {
    hipStream_t stream = nullptr;
    hipEvent_t fork = nullptr;
    hipEvent_t join = nullptr;
};

hipError_t side_stream(SideStream** out) {
    constexpr int kMaxDev = 64;
    thread_local SideStream per_dev[kMaxDev];
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDev) return hipErrorInvalidDevice;
    SideStream& f = per_dev[dev];
    if (f.stream == nullptr) {
        SideStream n;
        if ((e = hipStreamCreateWithFlags(&n.stream, hipStreamNonBlocking)) != hipSuccess) return e;
        if ((e = hipEventCreateWithFlags(&n.fork, hipEventDisableTiming)) != hipSuccess) return e;
        if ((e = hipEventCreateWithFlags(&n.join, hipEventDisableTiming)) != hipSuccess) return e;
        f = n;
    }
    *out = &f;
    return hipSuccess;
}

}  // namespace

int64_t mmdit_block_scratch_layout(int n_img, int n_txt, int batch, void* base, BlockScratch* out) {
    const int S = n_img + n_txt;
    const int64_t ri = int64_t{batch} * n_img;  // image rows of all sequences
    const int64_t rt = int64_t{batch} * n_txt;
    const int64_t mmax = ri > rt ? ri : (rt > 1 ? rt : 1);
    uint8_t* p = static_cast<uint8_t*>(base);
    int64_t off = 0;
    auto take = [&](int64_t bytes) {
        uint8_t* r = p ? p + off : nullptr;
        off += al256(bytes);
        return r;
    };
    BlockScratch w{};
    w.t_silu = reinterpret_cast<float*>(take(4 * DIM));
    w.mod_q = take(DIM);
    w.mod_scale = reinterpret_cast<float*>(take(4));
    for (int i = 0; i < 2; ++i) {
        w.img_mods[i] = reinterpret_cast<float*>(take(4 * 6 * DIM));
        w.txt_mods[i] = reinterpret_cast<float*>(take(4 * 6 * DIM));
    }
    w.img_norm = reinterpret_cast<float*>(take(4 * ri * DIM));
    w.txt_norm = reinterpret_cast<float*>(take(4 * rt * DIM));
    w.act_q = take(mmax * MLP);
    w.act_scales = reinterpret_cast<float*>(take(4 * mmax));
    w.act_q_txt = take((rt > 1 ? rt : 1) * MLP);
    w.act_scales_txt = reinterpret_cast<float*>(take(4 * (rt > 1 ? rt : 1)));
    for (int i = 0; i < 3; ++i) {
        w.img_qkv[i] = reinterpret_cast<float*>(take(4 * ri * DIM));
        w.txt_qkv[i] = reinterpret_cast<float*>(take(4 * rt * DIM));
    }
    // fp16 K for its mean and quantization (Q goes straight to int8, V to
    // the attention's Vt layout)
    w.k16 = reinterpret_cast<uint16_t*>(take(int64_t{2} * batch * S * DIM));
    w.attn16 = reinterpret_cast<uint16_t*>(take(int64_t{2} * batch * S * DIM));
    w.img_mlp = reinterpret_cast<float*>(take(4 * ri * MLP));
    w.txt_mlp = reinterpret_cast<float*>(take(4 * rt * MLP));
    const int64_t sage = sage_scratch_layout(HEADS * batch, S > 0 ? S : 1, HEAD_DIM, nullptr, nullptr);
    w.sage = take(sage);
    w.sage_bytes = sage;
    if (out) *out = w;
    return off;
}

hipError_t run_mmdit_block(const qimg_mmdit_block& b, float* img, float* txt, const float* t_emb, const float* pe,
                           int n_img, int n_txt, int batch, const BlockScratch& w, float* prof_ms, hipStream_t s,
                           bool t_ready, int mods_set, bool mods_ready, const qimg_mmdit_block* next,
                           bool* next_ready) {
    if (next_ready) *next_ready = false;
    const int S = n_img + n_txt;
    // row counts of the img / txt streams over all sequences
    const int Mi = batch * n_img;
    const int Mt = batch * n_txt;
    hipEvent_t ev[QIMG_PROF_COUNT + 1] = {};
    const bool prof = prof_ms != nullptr;
    hipError_t e = hipSuccess;
#define QIMG_TRY(x)              \
    do {                         \
        e = (x);                 \
        if (e != hipSuccess) goto done; \
    } while (0)
    // Work forked to the side stream is joined back before any return, an
    // error exit included: a graph capture then holds no unjoined fork, and
    // in eager use no side-stream work outlives the call.
    SideStream* forked = nullptr;
    auto fork = [&](SideStream* f) -> hipError_t {
        hipError_t r = hipEventRecord(f->fork, s);
        if (r == hipSuccess) r = hipStreamWaitEvent(f->stream, f->fork, 0);
        if (r == hipSuccess) forked = f;
        return r;
    };
    // (the caller has recorded f->join on the side stream after its work)
    auto join = [&](SideStream* f) -> hipError_t {
        const hipError_t r = hipStreamWaitEvent(s, f->join, 0);
        if (r == hipSuccess) forked = nullptr;
        return r;
    };
    if (prof) {
        for (auto& x : ev) QIMG_TRY(hipEventCreate(&x));
    }
    {
        auto mark = [&](int c) -> hipError_t { return prof ? hipEventRecord(ev[c], s) : hipSuccess; };
        auto gemm = [&](const uint8_t* qa, const float* sa, int M, const qimg_qlinear& l, float* out, int gelu,
                        hipStream_t st) {
            return launch_linear_prequantized(qa, sa, M, l.K, l.w, l.scales, l.N, l.mode, l.bias, out, QIMG_FP32,
                                              gelu, st);
        };
        auto quant = [&](const float* x, int M, const qimg_qlinear& l) {
            return launch_fwht_quant(x, QIMG_FP32, M, l.K, l.hbs, l.mode, w.act_q, w.act_scales, s);
        };
        auto linear = [&](const float* x, int M, const qimg_qlinear& l, float* out, int gelu) -> hipError_t {
            if (M == 0) return hipSuccess;
            hipError_t r = quant(x, M, l);
            return r != hipSuccess ? r : gemm(w.act_q, w.act_scales, M, l, out, gelu, s);
        };
        auto same_quant = [](const qimg_qlinear& a, const qimg_qlinear& c) {
            return a.K == c.K && a.hbs == c.hbs && a.mode == c.mode;
        };
        // quantized activations of the image (act_q) and text (act_q_txt)
        // streams live side by side, so that the two streams' linears can
        // share a launch
        auto quant_txt = [&](const float* x, int M, const qimg_qlinear& l, hipStream_t st) {
            return launch_fwht_quant(x, QIMG_FP32, M, l.K, l.hbs, l.mode, w.act_q_txt, w.act_scales_txt, st);
        };
        // One linear of each stream over the stream's quantized activations;
        // gate != nullptr adds the gated residual into `out` (the stream
        // itself), with `tmp` for rows computed without the fused epilogue.
        auto gemm_pair = [&](int Mi_, const qimg_qlinear& li, float* oi, const float* gi, float* ti, int Mt_,
                             const qimg_qlinear& lt, float* ot, const float* gt, float* tt, int gelu) -> hipError_t {
            const LinearArgs a{w.act_q, w.act_scales, Mi_, li.K, li.w, li.scales, li.N, li.bias, oi, gi, ti};
            const LinearArgs c{w.act_q_txt, w.act_scales_txt, Mt_, lt.K, lt.w, lt.scales, lt.N, lt.bias, ot, gt, tt};
            if (li.mode == lt.mode) return launch_linear_pair(a, c, li.mode, QIMG_FP32, gelu, s);
            const LinearArgs none{};
            hipError_t r = launch_linear_pair(a, none, li.mode, QIMG_FP32, gelu, s);
            return r != hipSuccess ? r : launch_linear_pair(none, c, lt.mode, QIMG_FP32, gelu, s);
        };

        // modulation: silu(t_emb) -> img_mod / txt_mod (transformer.cu:506-515)
        QIMG_TRY(mark(QIMG_PROF_MODULATION));
        // silu(t_emb) and its quantization are the same for every block of a
        // call: computed by the first block (and again where img_mod's
        // quantization changes), then kept in their own buffers
        float* const imods = w.img_mods[mods_set];
        float* const tmods = w.txt_mods[mods_set];
        // both modulation linears in one GEMV launch where they share the
        // activation quantization (int8 or e4m3; the reference's weights)
        auto mods_pair = [&](const qimg_mmdit_block& mb, float* io, float* to, hipStream_t st) -> bool {
            if (!same_quant(mb.img_mod, mb.txt_mod) ||
                (mb.img_mod.mode != QIMG_QM_INT8_HADAMARD && mb.img_mod.mode != QIMG_QM_FP8_HADAMARD))
                return false;
            const LinearArgs mi{w.mod_q, w.mod_scale, 1, mb.img_mod.K, mb.img_mod.w, mb.img_mod.scales,
                                mb.img_mod.N, mb.img_mod.bias, io, nullptr, nullptr};
            const LinearArgs mt{w.mod_q, w.mod_scale, 1, mb.txt_mod.K, mb.txt_mod.w, mb.txt_mod.scales,
                                mb.txt_mod.N, mb.txt_mod.bias, to, nullptr, nullptr};
            return launch_gemv_pair(w.mod_q, w.mod_scale, 1, mb.img_mod.K, mi, mt, mb.img_mod.mode, QIMG_FP32, st,
                                    &e);
        };
        if (!mods_ready) {
            if (!t_ready) {
                QIMG_TRY(launch_silu(t_emb, w.t_silu, DIM, s));
                QIMG_TRY(launch_fwht_quant(w.t_silu, QIMG_FP32, 1, b.img_mod.K, b.img_mod.hbs, b.img_mod.mode,
                                           w.mod_q, w.mod_scale, s));
            }
            const bool mods_done = mods_pair(b, imods, tmods, s);
            if (mods_done && e != hipSuccess) goto done;
            if (!mods_done) {
                QIMG_TRY(gemm(w.mod_q, w.mod_scale, 1, b.img_mod, imods, 0, s));
                if (same_quant(b.img_mod, b.txt_mod)) {
                    QIMG_TRY(gemm(w.mod_q, w.mod_scale, 1, b.txt_mod, tmods, 0, s));
                } else {
                    QIMG_TRY(linear(w.t_silu, 1, b.txt_mod, tmods, 0));
                }
            }
        }
        // chunks: shift1, scale1, gate1, shift2, scale2, gate2
        const float* im = imods;
        const float* tm = tmods;

        // LayerNorm + modulate (transformer.cu:526-540), then QKV with one
        // activation quant per stream (transformer.cu:557-606). When the
        // three linears of a stream share the quantization (always, for the
        // reference's weights) the LayerNorm writes their int8 input
        // directly. The image and text linears of each of q, k, v share a
        // launch.
        const qimg_qlinear* il[3] = {&b.to_q, &b.to_k, &b.to_v};
        const qimg_qlinear* tl[3] = {&b.add_q_proj, &b.add_k_proj, &b.add_v_proj};
        const bool share_i = same_quant(*il[0], *il[1]) && same_quant(*il[0], *il[2]);
        const bool share_t = same_quant(*tl[0], *tl[1]) && same_quant(*tl[0], *tl[2]);
        QIMG_TRY(mark(QIMG_PROF_ATTN_NORM));
        // (both streams' rows in one launch when their quantizations agree:
        // the few text rows' latency then hides behind the image rows)
        if (share_i && share_t && same_quant(*il[0], *tl[0])) {
            QIMG_TRY(launch_ln_fwht_quant_pair(img, im + 0 * DIM, im + 1 * DIM, Mi, w.act_q, w.act_scales, txt,
                                               tm + 0 * DIM, tm + 1 * DIM, Mt, w.act_q_txt, w.act_scales_txt, DIM,
                                               il[0]->hbs, il[0]->mode, EPS, s));
        } else {
            if (share_i)
                QIMG_TRY(launch_ln_fwht_quant(img, im + 0 * DIM, im + 1 * DIM, Mi, DIM, il[0]->hbs, il[0]->mode, EPS,
                                              w.act_q, w.act_scales, s));
            else
                QIMG_TRY(launch_layernorm_modulate(img, im + 0 * DIM, im + 1 * DIM, w.img_norm, Mi, DIM, EPS, s));
            if (share_t)
                QIMG_TRY(launch_ln_fwht_quant(txt, tm + 0 * DIM, tm + 1 * DIM, Mt, DIM, tl[0]->hbs, tl[0]->mode,
                                              EPS, w.act_q_txt, w.act_scales_txt, s));
            else
                QIMG_TRY(launch_layernorm_modulate(txt, tm + 0 * DIM, tm + 1 * DIM, w.txt_norm, Mt, DIM, EPS, s));
        }

        QIMG_TRY(mark(QIMG_PROF_QKV_GEMM));
        auto qkv_gemm = [&](int i) -> hipError_t {
            hipError_t r = hipSuccess;
            if (!share_i && Mi) r = quant(w.img_norm, Mi, *il[i]);
            if (r == hipSuccess && !share_t && Mt) r = quant_txt(w.txt_norm, Mt, *tl[i], s);
            return r != hipSuccess ? r
                                   : gemm_pair(Mi, *il[i], w.img_qkv[i], nullptr, nullptr, Mt, *tl[i], w.txt_qkv[i],
                                               nullptr, nullptr, 0);
        };
        SideStream* side = nullptr;
        QIMG_TRY(side_stream(&side));
        // The next block's modulation GEMV pair (the same quantized
        // silu(t_emb) row when its img_mod quantizes alike) runs on the side
        // stream into the other chunk set, which no work of this block reads;
        // the side stream's next join, at the latest the one at the end of
        // this block, orders it before the next block. It goes where CUs
        // would otherwise idle: beside the attention when that has at least
        // two rounds of workgroups (its workgroups then take CUs as attention
        // workgroups retire, and the attention left to run absorbs them;
        // 6889 + 512 tokens, 2.7 and 5.4 rounds: 0.6-0.9% per step), else
        // beside the K linears' launch, whose last round leaves CUs free
        // (4096 + 256 tokens: 204 tiles on 256 CUs; beside that shape's
        // 1.6-round attention the GEMV outlasted it and slowed the
        // out-projection).
        const bool pre_next = next && next_ready && same_quant(next->img_mod, b.img_mod);
        const int cus = device_cu_count();
        const bool next_beside_attn =
            pre_next && cus > 0 && sage_attn_workgroups(HEADS * batch, S) >= 2 * static_cast<int64_t>(cus);
        auto next_mods = [&]() -> hipError_t {
            hipError_t r = fork(side);
            if (r != hipSuccess) return r;
            const bool done_ = mods_pair(*next, w.img_mods[mods_set ^ 1], w.txt_mods[mods_set ^ 1], side->stream);
            if (done_ && e != hipSuccess) return e;
            r = hipEventRecord(side->join, side->stream);
            if (r == hipSuccess) *next_ready = done_;
            return r;
        };
        SageScratch ss;
        sage_scratch_layout(HEADS * batch, S, HEAD_DIM, w.sage, &ss);
        // When both streams' three linears share their input quantization and
        // every linear has the same mode, the linears write the attention's
        // operands from their epilogues: K as RMSNorm + RoPE fp16, Q also
        // quantized to the Sage int8 (when its 32-token slices lie inside one
        // linear: n_txt a multiple of 32, the image rows split per sequence
        // unless n_img is one too), V in the V^T tile layout. K's two linears
        // go first so that its mean and quantization run on the side stream
        // beside the Q and V linears (one launch of three to seven problems).
        bool merged = false, q_fused = false;
        const int nsplit = (batch > 1 && n_img % 32 != 0) ? batch : 1;
        const bool q_ok = n_txt % 32 == 0 && nsplit <= 4;
        HeadsOut hq_img[4], hv_img[4], hq_txt{}, hk_img{}, hk_txt{}, hv_txt{};
        if (share_i && share_t && Mi > 0 && Mt > 0) {
            bool same_mode = true;
            for (int i = 0; i < 3; ++i)
                same_mode = same_mode && il[i]->mode == il[0]->mode && tl[i]->mode == il[0]->mode;
            if (same_mode) {
                auto args = [&](int i, bool img, int rows, int row0, void* out, const HeadsOut* h) {
                    const qimg_qlinear& l = img ? *il[i] : *tl[i];
                    const uint8_t* aq = static_cast<const uint8_t*>(img ? w.act_q : w.act_q_txt);
                    const float* as = img ? w.act_scales : w.act_scales_txt;
                    LinearArgs a{aq + static_cast<int64_t>(row0) * l.K, as + row0, rows, l.K, l.w, l.scales, l.N,
                                 l.bias, out, nullptr, nullptr};
                    a.heads = h;
                    return a;
                };
                hk_img = HeadsOut{HEADS_K, HEADS, S, n_txt, n_img, 0, b.norm_k, pe, nullptr, EPS};
                hk_txt = HeadsOut{HEADS_K, HEADS, S, 0, n_txt, 0, b.norm_added_k, pe, nullptr, EPS};
                const LinearArgs ks[2] = {args(1, true, Mi, 0, w.k16, &hk_img), args(1, false, Mt, 0, w.k16, &hk_txt)};
                // the Q and V linears: nsplit image Q problems (at most 4),
                // the text Q, up to 2 image V problems and the text V
                static_assert(4 + 1 + 2 + 1 <= kMaxLinearMulti, "the Q/V launch holds at most eight linears");
                LinearArgs qv[kMaxLinearMulti];
                int n = 0;
                if (q_ok) {
                    for (int q = 0; q < nsplit; ++q) {
                        hq_img[q] = HeadsOut{HEADS_Q, HEADS, S, n_txt, n_img, q * (batch / nsplit), b.norm_q, pe,
                                             ss.q_scale, EPS};
                        qv[n++] = args(0, true, Mi / nsplit, q * (Mi / nsplit), ss.q_i8, &hq_img[q]);
                    }
                    hq_txt = HeadsOut{HEADS_Q, HEADS, S, 0, n_txt, 0, b.norm_added_q, pe, ss.q_scale, EPS};
                    qv[n++] = args(0, false, Mt, 0, ss.q_i8, &hq_txt);
                } else {
                    qv[n++] = args(0, true, Mi, 0, w.img_qkv[0], nullptr);
                    qv[n++] = args(0, false, Mt, 0, w.txt_qkv[0], nullptr);
                }
                // (V rows split per sequence as Q's: a 32-row block then
                // fills half of one key tile's rows, stored whole)
                const int vsplit = (n_txt % 32 == 0 && nsplit <= 2) ? nsplit : 1;
                for (int q = 0; q < vsplit; ++q) {
                    hv_img[q] = HeadsOut{HEADS_V, HEADS, S, n_txt, n_img, q * (batch / vsplit), nullptr, nullptr,
                                         nullptr, EPS};
                    qv[n++] = args(2, true, Mi / vsplit, q * (Mi / vsplit), ss.v_t, &hv_img[q]);
                }
                hv_txt = HeadsOut{HEADS_V, HEADS, S, 0, n_txt, 0, nullptr, nullptr, nullptr, EPS};
                qv[n++] = args(2, false, Mt, 0, ss.v_t, &hv_txt);
                // Both launches are validated before the first is issued, so
                // a refusal falls back to the unmerged path with nothing run.
                hipError_t r = check_linear_multi(ks, 2, QIMG_FP32, 0);
                if (r == hipSuccess) r = check_linear_multi(qv, n, QIMG_FP32, 0);
                if (r == hipSuccess) {
                    QIMG_TRY(launch_linear_multi(ks, 2, il[0]->mode, QIMG_FP32, 0, s));
                    merged = true;
                    if (pre_next && !next_beside_attn) QIMG_TRY(next_mods());
                    QIMG_TRY(fork(side));
                    QIMG_TRY(launch_sage_k_mean(w.k16, ss.k_mean, HEADS * batch, S, HEAD_DIM, side->stream));
                    QIMG_TRY(launch_sage_quant_k(w.k16, ss.k_mean, ss.k_i8, ss.k_scale, HEADS * batch, S, HEAD_DIM,
                                                 side->stream));
                    QIMG_TRY(hipEventRecord(side->join, side->stream));
                    QIMG_TRY(launch_linear_multi(qv, n, il[0]->mode, QIMG_FP32, 0, s));
                    q_fused = q_ok;
                } else if (r != hipErrorNotSupported) {
                    e = r;
                    goto done;
                }
            }
        }
        if (!merged) {
            // K first: its RMSNorm + concat + transpose + RoPE -> fp16
            // (transformer.cu:617-666), then its mean and quantization
            // (sageattention_sm80.cu:759-773, 826-886) on the side stream beside
            // the q and v linears and the Q / V preparation.
            QIMG_TRY(qkv_gemm(1));
            QIMG_TRY(launch_joint_heads_f16(w.txt_qkv[1], w.img_qkv[1], b.norm_added_k, b.norm_k, pe, w.k16, n_txt,
                                            n_img, batch, HEADS, EPS, s));
            QIMG_TRY(fork(side));
            QIMG_TRY(launch_sage_k_mean(w.k16, ss.k_mean, HEADS * batch, S, HEAD_DIM, side->stream));
            QIMG_TRY(launch_sage_quant_k(w.k16, ss.k_mean, ss.k_i8, ss.k_scale, HEADS * batch, S, HEAD_DIM,
                                         side->stream));
            QIMG_TRY(hipEventRecord(side->join, side->stream));
            QIMG_TRY(qkv_gemm(0));
            QIMG_TRY(qkv_gemm(2));
        }
        // Q: RMSNorm + RoPE + fp16 and the Sage int8 quantization in one pass
        QIMG_TRY(mark(QIMG_PROF_QK_NORM));
        if (!q_fused)
            QIMG_TRY(launch_heads_quant_q(w.txt_qkv[0], w.img_qkv[0], b.norm_added_q, b.norm_q, pe, ss.q_i8,
                                          ss.q_scale, n_txt, n_img, batch, HEADS, EPS, s));
        QIMG_TRY(mark(QIMG_PROF_CONCAT_TRANSPOSE));
        // V: fp16 straight into the attention's Vt tile layout (by the linears'
        // epilogue when merged, which leaves the tail keys' zeros, and the
        // scales of slices without tokens when Q is fused, to set)
        if (merged)
            QIMG_TRY(launch_sage_tail_fill(ss.v_t, q_fused ? ss.q_scale : nullptr, HEADS * batch, S, s));
        else
            QIMG_TRY(launch_heads_v_relayout(w.txt_qkv[2], w.img_qkv[2], ss.v_t, n_txt, n_img, batch, HEADS, s));
        QIMG_TRY(mark(QIMG_PROF_ROPE));

        // SageAttention, sm_scale = 1/sqrt(128) (transformer.cu:676-684)
        QIMG_TRY(mark(QIMG_PROF_ATTENTION));
        QIMG_TRY(join(side));
        QIMG_TRY(launch_sage_attn_vt(ss.q_i8, ss.k_i8, ss.v_t, ss.q_scale, ss.k_scale, w.attn16, QIMG_FP16,
                                     HEADS * batch, S, HEAD_DIM, 1.0f / sqrtf(128.0f), 0, s));
        if (next_beside_attn) QIMG_TRY(next_mods());

        // transpose + split back to the streams (transformer.cu:693-703),
        // read by the out-projection quantization straight from the fp16
        // attention output; out projections (transformer.cu:723-732) with
        // the gate1 residual (transformer.cu:740-746) in their epilogue, the
        // k buffers taking rows a kernel without that epilogue computes
        QIMG_TRY(mark(QIMG_PROF_TRANSPOSE_SPLIT));
        const bool heads_i = b.to_out.hbs >= 16 && b.to_out.K == DIM;
        const bool heads_t = b.to_add_out.hbs >= 16 && b.to_add_out.K == DIM;
        if (!heads_i || !heads_t) {
            // q buffers are free now
            QIMG_TRY(launch_split_heads(w.attn16, w.txt_qkv[0], w.img_qkv[0], n_txt, n_img, batch, HEADS, s));
        }
        QIMG_TRY(mark(QIMG_PROF_OUT_GEMM));
        if (heads_i && heads_t && same_quant(b.to_out, b.to_add_out)) {
            QIMG_TRY(launch_heads_fwht_quant_pair(w.attn16, batch, HEADS, S, n_txt, n_img, b.to_out.hbs,
                                                  b.to_out.mode, w.act_q, w.act_scales, w.act_q_txt,
                                                  w.act_scales_txt, s));
        } else {
            if (Mi) {
                if (heads_i)
                    QIMG_TRY(launch_heads_fwht_quant(w.attn16, batch, HEADS, S, n_txt, n_img, b.to_out.hbs,
                                                     b.to_out.mode, w.act_q, w.act_scales, s));
                else
                    QIMG_TRY(quant(w.img_qkv[0], Mi, b.to_out));
            }
            if (Mt) {
                if (heads_t)
                    QIMG_TRY(launch_heads_fwht_quant(w.attn16, batch, HEADS, S, 0, n_txt, b.to_add_out.hbs,
                                                     b.to_add_out.mode, w.act_q_txt, w.act_scales_txt, s));
                else
                    QIMG_TRY(quant_txt(w.txt_qkv[0], Mt, b.to_add_out, s));
            }
        }
        QIMG_TRY(gemm_pair(Mi, b.to_out, img, im + 2 * DIM, w.img_qkv[1], Mt, b.to_add_out, txt, tm + 2 * DIM,
                           w.txt_qkv[1], 0));
        QIMG_TRY(mark(QIMG_PROF_GATE_ATTN));

        // LayerNorm + modulate (transformer.cu:754-764) straight into the
        // fc1 input quantization
        QIMG_TRY(mark(QIMG_PROF_MLP_NORM));
        if (same_quant(b.img_mlp_fc1, b.txt_mlp_fc1)) {
            QIMG_TRY(launch_ln_fwht_quant_pair(img, im + 3 * DIM, im + 4 * DIM, Mi, w.act_q, w.act_scales, txt,
                                               tm + 3 * DIM, tm + 4 * DIM, Mt, w.act_q_txt, w.act_scales_txt, DIM,
                                               b.img_mlp_fc1.hbs, b.img_mlp_fc1.mode, EPS, s));
        } else {
            QIMG_TRY(launch_ln_fwht_quant(img, im + 3 * DIM, im + 4 * DIM, Mi, DIM, b.img_mlp_fc1.hbs,
                                          b.img_mlp_fc1.mode, EPS, w.act_q, w.act_scales, s));
            QIMG_TRY(launch_ln_fwht_quant(txt, tm + 3 * DIM, tm + 4 * DIM, Mt, DIM, b.txt_mlp_fc1.hbs,
                                          b.txt_mlp_fc1.mode, EPS, w.act_q_txt, w.act_scales_txt, s));
        }

        // GELU MLP (transformer.cu:780-808): fc1 of each stream on its own.
        // With e4m3 weights fc1 is run without its GELU and the fc2-input
        // quantization applies it to the values it loads (the same function
        // of the same fp32 values: the same quantized bytes; C5 step
        // measured faster, the int8 block equal).
        const bool gelu_i = b.img_mlp_fc1.mode == QIMG_QM_FP8_HADAMARD &&
                            fwht_quant_gelu_supported(b.img_mlp_fc2.K, b.img_mlp_fc2.hbs);
        const bool gelu_t = b.txt_mlp_fc1.mode == QIMG_QM_FP8_HADAMARD &&
                            fwht_quant_gelu_supported(b.txt_mlp_fc2.K, b.txt_mlp_fc2.hbs);
        QIMG_TRY(mark(QIMG_PROF_MLP_GEMM));
        // The text stream's fc1 and fc2-input quantization run on the side
        // stream beside the image fc2-input quantization, which is HBM-bound
        // and leaves the matrix cores idle (they start once the image fc1,
        // which fills every CU, is done).
        if (Mi) QIMG_TRY(gemm(w.act_q, w.act_scales, Mi, b.img_mlp_fc1, w.img_mlp, gelu_i ? 0 : 1, s));
        if (Mt) {
            hipStream_t st = s;
            if (Mi) {
                QIMG_TRY(fork(side));
                st = side->stream;
            }
            QIMG_TRY(gemm(w.act_q_txt, w.act_scales_txt, Mt, b.txt_mlp_fc1, w.txt_mlp, gelu_t ? 0 : 1, st));
            if (gelu_t)
                QIMG_TRY(launch_fwht_quant_gelu(w.txt_mlp, Mt, b.txt_mlp_fc2.K, b.txt_mlp_fc2.hbs, b.txt_mlp_fc2.mode,
                                                w.act_q_txt, w.act_scales_txt, st));
            else
                QIMG_TRY(quant_txt(w.txt_mlp, Mt, b.txt_mlp_fc2, st));
            if (Mi) QIMG_TRY(hipEventRecord(side->join, side->stream));
        }
        if (Mi) {
            if (gelu_i)
                QIMG_TRY(launch_fwht_quant_gelu(w.img_mlp, Mi, b.img_mlp_fc2.K, b.img_mlp_fc2.hbs, b.img_mlp_fc2.mode,
                                                w.act_q, w.act_scales, s));
            else
                QIMG_TRY(quant(w.img_mlp, Mi, b.img_mlp_fc2));
        }
        if (Mt && Mi) QIMG_TRY(join(side));
        // both fc2 in one launch, with the gate2 residual (transformer.cu:
        // 812-818) in their epilogue
        QIMG_TRY(gemm_pair(Mi, b.img_mlp_fc2, img, im + 5 * DIM, w.img_qkv[2], Mt, b.txt_mlp_fc2, txt, tm + 5 * DIM,
                           w.txt_qkv[2], 0));
        QIMG_TRY(mark(QIMG_PROF_GATE_MLP));
        if (forked != nullptr) QIMG_TRY(join(forked));
        QIMG_TRY(mark(QIMG_PROF_COUNT));

        if (prof) {
            QIMG_TRY(hipEventSynchronize(ev[QIMG_PROF_COUNT]));
            for (int c = 0; c < QIMG_PROF_COUNT; ++c) {
                float ms = 0.0f;
                QIMG_TRY(hipEventElapsedTime(&ms, ev[c], ev[c + 1]));
                prof_ms[c] += ms;
            }
        }
    }
done:
#undef QIMG_TRY
    if (forked != nullptr) {
        // error exit between a fork and its join: join whatever the side
        // stream has queued (the first error is the one returned)
        if (hipEventRecord(forked->join, forked->stream) == hipSuccess) (void)hipStreamWaitEvent(s, forked->join, 0);
    }
    if (prof)
        for (auto& x : ev)
            if (x) (void)hipEventDestroy(x);
    return e;
}

}  // namespace qimg
