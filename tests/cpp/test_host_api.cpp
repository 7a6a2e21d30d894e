// test_host_api.cpp — exercises the reference-signature C++ layer
// (qwen-image.cu_amd/host/kernels.h) the way the reference's forward pass
// calls it (transformer.cu:563-606, 680-689, 785-807), and checks every
// result against the CPU oracle (oracle/qimg_oracle.h).
//
//   test_host_api                    GPU parity cases; exit 0 when all pass
//   test_host_api --expect-error C   run case C, which must be rejected by the
//                                    host-side checks before any HIP call (the
//                                    process then exits 1 with a message, as
//                                    the reference's asserts do); no GPU needed
#include <cmath>
#include <cstdlib>
#include <unistd.h>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "checkpoint.h"
#include "kernels.h"
#include "qimg_oracle.h"

namespace {

int g_fail = 0;

struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed * 0x9E3779B97F4A7C15ull + 1) {}
    uint32_t next() {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        return static_cast<uint32_t>(s >> 32);
    }
    float uniform() { return (next() + 0.5f) * (1.0f / 4294967296.0f); }
    float normal() {
        const float u = uniform(), v = uniform();
        return std::sqrt(-2.0f * std::log(u)) * std::cos(6.2831853f * v);
    }
};

std::vector<uint16_t> bf16_normal(Rng& r, size_t n, float sigma) {
    std::vector<uint16_t> v(n);
    for (auto& x : v) x = or_f32_to_bf16(r.normal() * sigma);
    return v;
}

std::vector<float> f32_normal(Rng& r, size_t n, float sigma) {
    std::vector<float> v(n);
    for (auto& x : v) x = r.normal() * sigma;
    return v;
}

template <typename T>
Tensor upload(const std::vector<T>& h, std::vector<int64_t> dims, DType dt) {
    Tensor t = Tensor::alloc(dims, dt);
    t.from_host(h.data(), h.size() * sizeof(T));
    return t;
}

template <typename T>
std::vector<T> download(const Tensor& t) {
    std::vector<T> h(t.nbytes() / sizeof(T));
    t.to_host(h.data());
    return h;
}

void report(const char* name, bool ok, const std::string& detail = "") {
    printf("%s %s %s\n", ok ? "ok  " : "FAIL", name, detail.c_str());
    fflush(stdout);
    if (!ok) ++g_fail;
}

// Oracle chain a5 -> a7 -> a8 (fp32 or bf16 input) -> fp32 [M,N].
std::vector<float> oracle_linear(const void* x, bool bf16, int M, int K, const std::vector<int8_t>& wq,
                                 const std::vector<float>& ws, int N, int hbs, const uint16_t* bias, bool gelu) {
    std::vector<int8_t> q(static_cast<size_t>(M) * K);
    std::vector<float> s(M);
    or_quantize_activation(x, bf16 ? 1 : 0, M, K, hbs, q.data(), s.data());
    std::vector<int32_t> c(static_cast<size_t>(M) * N);
    or_gemm_s8s8s32(q.data(), wq.data(), M, N, K, 0, M, c.data());
    std::vector<float> out(static_cast<size_t>(M) * N);
    or_dequant_epilogue(c.data(), s.data(), ws.data(), bias, M, N, gelu ? 1 : 0, out.data());
    return out;
}

double max_abs_diff(const std::vector<float>& a, const std::vector<float>& b) {
    double m = 0;
    for (size_t i = 0; i < a.size(); ++i) m = std::fmax(m, std::fabs(static_cast<double>(a[i]) - b[i]));
    return m;
}

double max_abs(const std::vector<float>& a) {
    double m = 0;
    for (float v : a) m = std::fmax(m, std::fabs(v));
    return m;
}

void case_tensor_api() {
    Rng r(1);
    std::vector<float> h = f32_normal(r, 6 * 5, 1.0f);
    Tensor t = upload(h, {6, 5}, DType::FP32);
    Tensor c = t.clone();
    Tensor s = c.slice(2, 4);
    Tensor v = s.view({10});
    std::vector<float> got = download<float>(v);
    bool ok = got.size() == 10 && std::memcmp(got.data(), h.data() + 10, 40) == 0 && t.numel() == 30 &&
              s.shape[0] == 2 && s.shape[1] == 5 && !s.owns_data && c.owns_data;
    Tensor moved = std::move(c);
    ok = ok && moved.owns_data && c.data == nullptr;
    report("tensor_api", ok);
}

void case_weight_quant(QuantMode mode, int N, int K) {
    Rng r(N + K);
    std::vector<uint16_t> w = bf16_normal(r, static_cast<size_t>(N) * K, 0.02f);
    Tensor wt = upload(w, {N, K}, DType::BF16);
    QuantizedWeight qw = mode == QuantMode::INT8_HADAMARD ? quantize_weight_tensor(wt) : quantize_weight_tensor_fp8(wt);
    std::vector<uint8_t> gq = download<uint8_t>(qw.data);
    std::vector<float> gs = download<float>(qw.scales);
    std::vector<uint8_t> rq(static_cast<size_t>(N) * K);
    std::vector<float> rs(N);
    int hbs = 0;
    if (mode == QuantMode::INT8_HADAMARD) {
        hbs = or_quantize_weight_bf16(w.data(), N, K, reinterpret_cast<int8_t*>(rq.data()), rs.data());
    } else {
        std::vector<float> wf(w.size());
        for (size_t i = 0; i < w.size(); ++i) wf[i] = or_bf16_to_f32(w[i]);
        hbs = or_hadamard_block_size(K);
        or_fwht_rows(wf.data(), N, K, hbs);
        or_quant_rows_fp8(wf.data(), N, K, rq.data(), rs.data());
    }
    const bool ok = qw.had_block_size == hbs && gq == rq && gs == rs &&
                    qw.data.dtype == (mode == QuantMode::INT8_HADAMARD ? DType::INT8 : DType::FP8_E4M3);
    report(mode == QuantMode::INT8_HADAMARD ? "quantize_weight_tensor" : "quantize_weight_tensor_fp8", ok);
}

void case_linear(bool bf16_in, int M, int N, int K, bool with_bias, bool gelu) {
    Rng r(M * 7 + N * 3 + K);
    std::vector<uint16_t> w = bf16_normal(r, static_cast<size_t>(N) * K, 0.02f);
    std::vector<uint16_t> b = bf16_normal(r, N, 0.01f);
    std::vector<float> xf = f32_normal(r, static_cast<size_t>(M) * K, 1.0f);
    std::vector<uint16_t> xb(xf.size());
    for (size_t i = 0; i < xf.size(); ++i) xb[i] = or_f32_to_bf16(xf[i]);

    Tensor wt = upload(w, {N, K}, DType::BF16);
    QuantizedWeight qw = quantize_weight_tensor(wt);
    Tensor bias = upload(b, {N}, DType::BF16);
    Tensor x = bf16_in ? upload(xb, {M, K}, DType::BF16) : upload(xf, {M, K}, DType::FP32);
    Tensor out = Tensor::alloc({M, N}, DType::FP32);
    Tensor scratch = Tensor::alloc({int8_scratch_bytes(M, K, N)}, DType::UINT8);
    if (bf16_in)
        linear_forward_int8_bf16in(x, qw, with_bias ? &bias : nullptr, out, scratch, gelu);
    else
        linear_forward_quantized(x, qw, with_bias ? &bias : nullptr, out, scratch, gelu);
    HIP_CHECK(hipDeviceSynchronize());
    std::vector<float> got = download<float>(out);

    std::vector<int8_t> wq(static_cast<size_t>(N) * K);
    std::vector<float> ws(N);
    const int hbs = or_quantize_weight_bf16(w.data(), N, K, wq.data(), ws.data());
    std::vector<float> ref = oracle_linear(bf16_in ? static_cast<const void*>(xb.data()) : xf.data(), bf16_in, M, K,
                                           wq, ws, N, hbs, with_bias ? b.data() : nullptr, gelu);
    char name[128];
    snprintf(name, sizeof(name), "linear %s M=%d N=%d K=%d bias=%d gelu=%d", bf16_in ? "bf16in" : "fp32in", M, N, K,
             with_bias, gelu);
    // No GELU: the epilogue is the reference's operation order, bit-exact.
    // GELU: tanh evaluated through exp2/rcp on the GPU, ~1e-6 relative.
    const double d = max_abs_diff(got, ref);
    const bool ok = gelu ? d <= 2e-6 * (max_abs(ref) + 1.0) : d == 0.0;
    char det[64];
    snprintf(det, sizeof(det), "max|diff|=%.3g", d);
    report(name, ok, det);
}

void case_prequantized_and_dequant() {
    const int M = 129, N = 384, K = 3072;
    Rng r(99);
    std::vector<uint16_t> w = bf16_normal(r, static_cast<size_t>(N) * K, 0.02f);
    std::vector<uint16_t> b = bf16_normal(r, N, 0.01f);
    std::vector<float> xf = f32_normal(r, static_cast<size_t>(M) * K, 1.0f);
    Tensor qwt = upload(w, {N, K}, DType::BF16);
    QuantizedWeight qw = quantize_weight_tensor(qwt);
    Tensor x = upload(xf, {M, K}, DType::FP32);
    Tensor qa = Tensor::alloc({M, K}, DType::INT8);
    Tensor sa = Tensor::alloc({M}, DType::FP32);
    quantize_activation_int8_hadamard_fp32(static_cast<const float*>(x.data), static_cast<int8_t*>(qa.data),
                                           static_cast<float*>(sa.data), M, K, qw.had_block_size);
    Tensor bias = upload(b, {N}, DType::BF16);
    Tensor out = Tensor::alloc({M, N}, DType::FP32);
    Tensor scratch;
    linear_forward_int8_prequantized(static_cast<const int8_t*>(qa.data), static_cast<const float*>(sa.data), M, K,
                                     qw, &bias, out, scratch, false);
    HIP_CHECK(hipDeviceSynchronize());
    std::vector<float> got = download<float>(out);
    std::vector<int8_t> wq(static_cast<size_t>(N) * K);
    std::vector<float> ws(N);
    const int hbs = or_quantize_weight_bf16(w.data(), N, K, wq.data(), ws.data());
    std::vector<float> ref = oracle_linear(xf.data(), false, M, K, wq, ws, N, hbs, b.data(), false);
    report("linear_forward_int8_prequantized", max_abs_diff(got, ref) == 0.0);

    // separate dequant pass on an oracle int32 product
    std::vector<int8_t> q(static_cast<size_t>(M) * K);
    std::vector<float> s(M);
    or_quantize_activation(xf.data(), 0, M, K, hbs, q.data(), s.data());
    std::vector<int32_t> c(static_cast<size_t>(M) * N);
    or_gemm_s8s8s32(q.data(), wq.data(), M, N, K, 0, M, c.data());
    Tensor ct = upload(c, {M, N}, DType::INT32);
    Tensor st = upload(s, {M}, DType::FP32);
    Tensor wst = upload(ws, {N}, DType::FP32);
    Tensor o2 = Tensor::alloc({M, N}, DType::FP32);
    dequantize_and_bias(static_cast<const int32_t*>(ct.data), static_cast<const float*>(st.data),
                        static_cast<const float*>(wst.data), static_cast<const __hip_bfloat16*>(bias.data),
                        static_cast<float*>(o2.data), M, N);
    HIP_CHECK(hipDeviceSynchronize());
    report("dequantize_and_bias", max_abs_diff(download<float>(o2), ref) == 0.0);
}

void case_fp8_linear() {
    const int M = 200, N = 256, K = 3072;
    Rng r(5);
    std::vector<uint16_t> w = bf16_normal(r, static_cast<size_t>(N) * K, 0.02f);
    std::vector<uint16_t> xb = bf16_normal(r, static_cast<size_t>(M) * K, 1.0f);
    Tensor wt = upload(w, {N, K}, DType::BF16);
    QuantizedWeight qw = quantize_weight_tensor_fp8(wt);
    Tensor x = upload(xb, {M, K}, DType::BF16);
    Tensor out = Tensor::alloc({M, N}, DType::FP32);
    Tensor scratch = Tensor::alloc({int8_scratch_bytes(M, K, N)}, DType::UINT8);
    linear_forward_quantized_bf16in(x, qw, nullptr, out, scratch);
    HIP_CHECK(hipDeviceSynchronize());
    std::vector<float> got = download<float>(out);
    // float64 product of the unquantized operands (H orthonormal, so the
    // rotation cancels): the e4m3 path must stay within the stated bar.
    double num = 0, den = 0, dot = 0, na = 0, nb = 0, mx = 0;
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            double e = 0;
            for (int k = 0; k < K; ++k)
                e += static_cast<double>(or_bf16_to_f32(xb[static_cast<size_t>(m) * K + k])) *
                     or_bf16_to_f32(w[static_cast<size_t>(n) * K + k]);
            const double g = got[static_cast<size_t>(m) * N + n];
            num = std::fmax(num, std::fabs(g - e));
            mx = std::fmax(mx, std::fabs(e));
            dot += g * e;
            na += g * g;
            nb += e * e;
        }
    (void)den;
    const double rel = num / mx, cos = dot / std::sqrt(na * nb);
    char det[96];
    snprintf(det, sizeof(det), "max-rel=%.3g cos=%.6f", rel, cos);
    report("linear fp8 bf16in vs float64", rel <= 5e-2 && cos >= 0.999, det);
}

void case_sage(int BH, int S, int D, bool causal) {
    Rng r(BH * S + D);
    const size_t n = static_cast<size_t>(BH) * S * D;
    std::vector<uint16_t> q(n), k(n), v(n);
    for (size_t i = 0; i < n; ++i) {
        q[i] = or_f32_to_f16(r.normal());
        k[i] = or_f32_to_f16(r.normal() + 0.5f);
        v[i] = or_f32_to_f16(r.normal());
    }
    Tensor qt = upload(q, {BH, S, D}, DType::FP16), kt = upload(k, {BH, S, D}, DType::FP16),
           vt = upload(v, {BH, S, D}, DType::FP16);
    Tensor ot = Tensor::alloc({BH, S, D}, DType::FP32);
    const float scale = 1.0f / std::sqrt(static_cast<float>(D));
    attention_forward_sage_sm80_fp16io(static_cast<const __half*>(qt.data), static_cast<const __half*>(kt.data),
                                       static_cast<const __half*>(vt.data), static_cast<float*>(ot.data), scale, BH,
                                       S, D, causal);
    HIP_CHECK(hipDeviceSynchronize());
    std::vector<float> got = download<float>(ot);
    std::vector<uint16_t> ref16(n);
    or_sage_attention_fp16io(q.data(), k.data(), v.data(), BH, S, D, scale, causal ? 1 : 0, ref16.data());
    std::vector<float> ref(n);
    for (size_t i = 0; i < n; ++i) ref[i] = or_f16_to_f32(ref16[i]);
    const double d = max_abs_diff(got, ref);
    char name[96], det[64];
    snprintf(name, sizeof(name), "attention_forward_sage_sm80_fp16io BH=%d S=%d D=%d causal=%d", BH, S, D, causal);
    snprintf(det, sizeof(det), "max|diff|=%.3g", d);
    report(name, d <= 2e-3 * max_abs(ref) + 2e-3, det);
}

// Host-side rejections: fake device pointers that must never be touched.
// The reference's TransformerWeights::Block field names (transformer.h:94-140),
// which mmdit_block_view reads.
struct RefBlock {
    QuantizedWeight img_mod_weight, txt_mod_weight, to_q_weight, to_k_weight, to_v_weight, add_q_proj_weight,
        add_k_proj_weight, add_v_proj_weight, to_out_weight, to_add_out_weight, img_mlp_fc1_weight,
        img_mlp_fc2_weight, txt_mlp_fc1_weight, txt_mlp_fc2_weight;
    Tensor img_mod_bias, txt_mod_bias, to_q_bias, to_k_bias, to_v_bias, add_q_proj_bias, add_k_proj_bias,
        add_v_proj_bias, to_out_bias, to_add_out_bias, img_mlp_fc1_bias, img_mlp_fc2_bias, txt_mlp_fc1_bias,
        txt_mlp_fc2_bias;
    Tensor norm_q_weight, norm_k_weight, norm_added_q_weight, norm_added_k_weight;
};

// The block loop through the C++ layer (batch 2, one TransformerWeights::
// Block-shaped struct) against the C ABI's one-block entry point run on each
// sequence alone: bit-identical.
void case_block_loop() {
    Rng r(99);
    RefBlock b;
    const int D = 3072, F = 12288;
    auto lin = [&](QuantizedWeight& w, Tensor& bias, int N, int K) {
        std::vector<uint16_t> h(static_cast<size_t>(N) * K);
        for (auto& x : h) x = or_f32_to_bf16((r.uniform() - 0.5f) * 0.07f);
        Tensor wt = upload(h, {N, K}, DType::BF16);
        w = quantize_weight_tensor(wt);
        bias = upload(bf16_normal(r, N, 0.01f), {N}, DType::BF16);
    };
    lin(b.img_mod_weight, b.img_mod_bias, 6 * D, D);
    lin(b.txt_mod_weight, b.txt_mod_bias, 6 * D, D);
    lin(b.to_q_weight, b.to_q_bias, D, D);
    lin(b.to_k_weight, b.to_k_bias, D, D);
    lin(b.to_v_weight, b.to_v_bias, D, D);
    lin(b.add_q_proj_weight, b.add_q_proj_bias, D, D);
    lin(b.add_k_proj_weight, b.add_k_proj_bias, D, D);
    lin(b.add_v_proj_weight, b.add_v_proj_bias, D, D);
    lin(b.to_out_weight, b.to_out_bias, D, D);
    lin(b.to_add_out_weight, b.to_add_out_bias, D, D);
    lin(b.img_mlp_fc1_weight, b.img_mlp_fc1_bias, F, D);
    lin(b.img_mlp_fc2_weight, b.img_mlp_fc2_bias, D, F);
    lin(b.txt_mlp_fc1_weight, b.txt_mlp_fc1_bias, F, D);
    lin(b.txt_mlp_fc2_weight, b.txt_mlp_fc2_bias, D, F);
    for (Tensor* t : {&b.norm_q_weight, &b.norm_k_weight, &b.norm_added_q_weight, &b.norm_added_k_weight}) {
        std::vector<uint16_t> h(128);
        for (auto& x : h) x = or_f32_to_bf16(1.0f + 0.1f * r.normal());
        *t = upload(h, {128}, DType::BF16);
    }
    const int n_img = 64, n_txt = 16, S = n_img + n_txt;
    std::vector<float> hi = f32_normal(r, 2 * n_img * D, 1.0f), ht = f32_normal(r, 2 * n_txt * D, 1.0f);
    std::vector<float> hte = f32_normal(r, D, 1.0f), hpe(static_cast<size_t>(S) * 256);
    for (int s = 0; s < S; ++s)
        for (int j = 0; j < 64; ++j) {
            const float a = 0.01f * s * (j + 1), c = std::cos(a), sn = std::sin(a);
            float* p = &hpe[(static_cast<size_t>(s) * 64 + j) * 4];
            p[0] = c, p[1] = -sn, p[2] = sn, p[3] = c;
        }
    Tensor img = upload(hi, {2 * n_img, D}, DType::FP32), txt = upload(ht, {2 * n_txt, D}, DType::FP32);
    Tensor temb = upload(hte, {D}, DType::FP32), pe = upload(hpe, {S, 64, 4}, DType::FP32);
    std::vector<qimg_mmdit_block> table{mmdit_block_view(b)};
    float prof[QIMG_PROF_COUNT];
    mmdit_blocks_forward(table, img, txt, temb, pe, 2, prof);
    std::vector<float> gi = download<float>(img), gt = download<float>(txt);
    bool ok = true;
    const int64_t bytes = qimg_mmdit_block_scratch_bytes(n_img, n_txt);
    Tensor scratch = Tensor::alloc({bytes}, DType::UINT8);
    for (int q = 0; q < 2; ++q) {
        std::vector<float> si(hi.begin() + q * n_img * D, hi.begin() + (q + 1) * n_img * D);
        std::vector<float> st(ht.begin() + q * n_txt * D, ht.begin() + (q + 1) * n_txt * D);
        Tensor i1 = upload(si, {n_img, D}, DType::FP32), t1 = upload(st, {n_txt, D}, DType::FP32);
        const int rc = qimg_mmdit_block_forward(&table[0], static_cast<float*>(i1.data), static_cast<float*>(t1.data),
                                                static_cast<const float*>(temb.data),
                                                static_cast<const float*>(pe.data), n_img, n_txt, scratch.data,
                                                bytes, nullptr, nullptr);
        HIP_CHECK(hipDeviceSynchronize());
        std::vector<float> ri = download<float>(i1), rt = download<float>(t1);
        ok = ok && rc == QIMG_OK && std::memcmp(ri.data(), gi.data() + q * n_img * D, ri.size() * 4) == 0 &&
             std::memcmp(rt.data(), gt.data() + q * n_txt * D, rt.size() * 4) == 0;
    }
    double total = 0;
    for (float v : prof) total += v;
    for (float v : gi) ok = ok && std::isfinite(v);
    report("mmdit_blocks_forward", ok && total > 0, "batch 2 vs two single-sequence blocks");
}

int expect_error(const std::string& c) {
    void* fake = reinterpret_cast<void*>(0x10000);
    Tensor x = Tensor::wrap(fake, {4, 64}, DType::FP32);
    Tensor out = Tensor::wrap(fake, {4, 8}, DType::FP32);
    Tensor scratch = Tensor::wrap(fake, {1 << 20}, DType::UINT8);
    QuantizedWeight w;
    w.data = Tensor::wrap(fake, {8, 64}, DType::INT8);
    w.scales = Tensor::wrap(fake, {8}, DType::FP32);
    w.had_block_size = 64;
    if (c == "out_shape") {
        Tensor bad = Tensor::wrap(fake, {4, 9}, DType::FP32);
        linear_forward_int8(x, w, nullptr, bad, scratch);
    } else if (c == "x_dtype") {
        Tensor xb = Tensor::wrap(fake, {4, 64}, DType::BF16);
        linear_forward_int8(xb, w, nullptr, out, scratch);
    } else if (c == "weight_k") {
        Tensor x2 = Tensor::wrap(fake, {4, 128}, DType::FP32);
        linear_forward_quantized(x2, w, nullptr, out, scratch);
    } else if (c == "bf16_out_dtype") {
        QuantizedWeight wb;
        wb.mode = QuantMode::BF16;
        wb.data = Tensor::wrap(fake, {8, 64}, DType::BF16);
        Tensor out16 = Tensor::wrap(fake, {4, 8}, DType::BF16);
        linear_forward_quantized(x, wb, nullptr, out16, scratch);
    } else if (c == "mode_int4") {
        w.mode = QuantMode::INT4_SVD;  // no low-rank factors
        linear_forward_quantized(x, w, nullptr, out, scratch);
    } else if (c == "awq_m") {
        w.mode = QuantMode::INT4_AWQ;
        w.awq_OC = 8;
        w.awq_IC = 64;
        linear_forward_quantized(x, w, nullptr, out, scratch);
    } else if (c == "scratch") {
        Tensor small = Tensor::wrap(fake, {16}, DType::UINT8);
        linear_forward_int8(x, w, nullptr, out, small);
    } else if (c == "hbs") {
        w.had_block_size = 48;
        linear_forward_int8(x, w, nullptr, out, scratch);
    } else if (c == "sage_head_dim") {
        attention_forward_sage_sm80_fp16io(static_cast<const __half*>(fake), static_cast<const __half*>(fake),
                                           static_cast<const __half*>(fake), static_cast<float*>(fake), 0.1f, 2, 64,
                                           96);
    } else if (c == "block_pe") {
        Tensor img = Tensor::wrap(fake, {64, 3072}, DType::FP32);
        Tensor txt = Tensor::wrap(fake, {16, 3072}, DType::FP32);
        Tensor temb = Tensor::wrap(fake, {3072}, DType::FP32);
        Tensor pe = Tensor::wrap(fake, {64, 64, 4}, DType::FP32);
        std::vector<qimg_mmdit_block> table(1);
        mmdit_blocks_forward(table, img, txt, temb, pe);
    } else {
        fprintf(stderr, "unknown case %s\n", c.c_str());
        return 2;
    }
    fprintf(stderr, "case %s was not rejected\n", c.c_str());
    return 3;
}

}  // namespace

// Quantized weights through the checkpoint format (transformer.h:146-199):
// written with SafeTensorsWriter, read back with SafeTensorsLoader and
// load_quantized_weight, the device bytes, scales, mode and Hadamard block
// must be those that were written; a BF16 weight loads as BF16 or, when
// asked, quantized as quantize_weight_tensor quantizes it.
void case_checkpoint_roundtrip() {
    Rng r(11);
    const int N = 64, K = 3072;
    std::vector<uint16_t> w = bf16_normal(r, static_cast<size_t>(N) * K, 0.02f);
    Tensor wt = upload(w, {N, K}, DType::BF16);
    QuantizedWeight q8 = quantize_weight_tensor(wt);
    QuantizedWeight qf = quantize_weight_tensor_fp8(wt);
    const std::vector<uint8_t> d8 = download<uint8_t>(q8.data), df = download<uint8_t>(qf.data);
    const std::vector<float> s8 = download<float>(q8.scales), sf = download<float>(qf.scales);
    SafeTensorsWriter wr;
    wr.add("transformer_blocks.0.attn.to_q.weight", "I8", {N, K}, d8.data(), d8.size());
    wr.add("transformer_blocks.0.attn.to_q.weight.__scales__", "F32", {N}, s8.data(), s8.size() * 4);
    wr.add("fp8.weight", "F8_E4M3", {N, K}, df.data(), df.size());
    wr.add("fp8.weight.__scales__", "F32", {N}, sf.data(), sf.size() * 4);
    wr.add("img_in.weight", "BF16", {N, K}, w.data(), w.size() * 2);
    const char* tmp = getenv("TMPDIR");
    const std::string path = std::string(tmp ? tmp : "/tmp") + "/qimg_ckpt_roundtrip_" + std::to_string(getpid()) +
                             ".safetensors";
    bool ok = wr.write(path);
    SafeTensorsLoader ld;
    ok = ok && ld.load_file(path);
    if (ok) {
        ok = detect_checkpoint(ld) == CheckpointKind::INT8 && ld.names().size() == 5;
        QuantizedWeight a = load_quantized_weight(ld, "transformer_blocks.0.attn.to_q.weight");
        QuantizedWeight b = load_quantized_weight(ld, "fp8.weight");
        QuantizedWeight c = load_quantized_weight(ld, "img_in.weight");
        QuantizedWeight d = load_quantized_weight(ld, "img_in.weight", false);
        ok = ok && a.mode == QuantMode::INT8_HADAMARD && a.had_block_size == 1024 && a.data.dtype == DType::INT8 &&
             download<uint8_t>(a.data) == d8 && download<float>(a.scales) == s8;
        ok = ok && b.mode == QuantMode::FP8_HADAMARD && b.had_block_size == 1024 &&
             b.data.dtype == DType::FP8_E4M3 && download<uint8_t>(b.data) == df && download<float>(b.scales) == sf;
        ok = ok && c.mode == QuantMode::BF16 && download<uint16_t>(c.data) == w;
        ok = ok && d.mode == QuantMode::INT8_HADAMARD && download<uint8_t>(d.data) == d8 &&
             download<float>(d.scales) == s8;
    }
    remove(path.c_str());
    report("checkpoint_roundtrip", ok);
}

// QuantMode::BF16 weights through the dispatchers (transformer.cu:400, 418
// call linear_forward_quantized_bf16in; :876, :894 linear_forward_quantized):
// integer-valued operands, exact in bf16 and in any fp32 summation order, so
// the output must equal the int64 product plus the bias.
void case_bf16_mode(bool bf16_in, int M, int N, int K) {
    Rng r(M + 5 * N + K + bf16_in);
    std::vector<float> xf(static_cast<size_t>(M) * K), wf(static_cast<size_t>(N) * K);
    for (auto& v : xf) v = static_cast<float>(static_cast<int>(r.next() % 9) - 4);
    for (auto& v : wf) v = static_cast<float>(static_cast<int>(r.next() % 9) - 4);
    std::vector<uint16_t> xb(xf.size()), wb(wf.size()), b(N);
    for (size_t i = 0; i < xf.size(); ++i) xb[i] = or_f32_to_bf16(xf[i]);
    for (size_t i = 0; i < wf.size(); ++i) wb[i] = or_f32_to_bf16(wf[i]);
    for (auto& v : b) v = or_f32_to_bf16(static_cast<float>(static_cast<int>(r.next() % 17) - 8));
    QuantizedWeight qw;
    qw.mode = QuantMode::BF16;
    qw.data = upload(wb, {N, K}, DType::BF16);
    Tensor bias = upload(b, {N}, DType::BF16);
    Tensor x = bf16_in ? upload(xb, {M, K}, DType::BF16) : upload(xf, {M, K}, DType::FP32);
    Tensor out = Tensor::alloc({M, N}, DType::FP32);
    Tensor scratch = Tensor::alloc({16}, DType::UINT8);  // the BF16 path needs none
    if (bf16_in)
        linear_forward_quantized_bf16in(x, qw, &bias, out, scratch);
    else
        linear_forward_quantized(x, qw, &bias, out, scratch);
    HIP_CHECK(hipDeviceSynchronize());
    std::vector<float> got = download<float>(out);
    double d = 0;
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            int64_t acc = 0;
            for (int k = 0; k < K; ++k)
                acc += static_cast<int64_t>(xf[static_cast<size_t>(m) * K + k]) *
                       static_cast<int64_t>(wf[static_cast<size_t>(n) * K + k]);
            const double want = static_cast<double>(acc) + or_bf16_to_f32(b[n]);
            d = std::fmax(d, std::fabs(got[static_cast<size_t>(m) * N + n] - want));
        }
    char name[96], det[64];
    snprintf(name, sizeof(name), "bf16-mode linear %s M=%d N=%d K=%d", bf16_in ? "bf16in" : "fp32in", M, N, K);
    snprintf(det, sizeof(det), "max|diff|=%.3g", d);
    report(name, d == 0.0, det);
}

// INT4_SVD through linear_forward_quantized[_bf16in] (cuda_kernels.cu:
// 4599-4635). The low-rank up factor is zero, so the output is the residual
// alone: W4A4 (nunchaku form, loaded as transformer.h:202-279 does: row-major
// nibbles swizzled into qweight_mma) is then bit-exact against the oracle's
// activation quant + W4A4 GEMM; W4A16 against float64 within an fp32
// summation bound.
void case_int4(bool w4a4, bool bf16_in, int M, int N, int K) {
    Rng r(M * 7 + N + K + w4a4 * 2 + bf16_in);
    const int gs = 64, G = K / gs, rank = 32;
    std::vector<float> xf = f32_normal(r, static_cast<size_t>(M) * K, 1.0f);
    std::vector<uint16_t> xb(xf.size());
    for (size_t i = 0; i < xf.size(); ++i) {
        xb[i] = or_f32_to_bf16(xf[i]);
        xf[i] = or_bf16_to_f32(xb[i]);  // the same values either way
    }
    std::vector<uint16_t> b(N), up(static_cast<size_t>(N) * rank, 0);
    for (auto& v : b) v = or_f32_to_bf16(r.normal() * 0.01f);
    std::vector<uint16_t> down = bf16_normal(r, static_cast<size_t>(K) * rank, 0.05f);
    std::vector<float> sm(K);
    for (auto& v : sm) v = 0.5f + r.uniform();
    QuantizedWeight qw;
    qw.mode = QuantMode::INT4_SVD;
    qw.group_size = gs;
    qw.svd_rank = rank;
    qw.svd_up = upload(up, {N, rank}, DType::BF16);
    qw.svd_down = upload(down, {K, rank}, DType::BF16);
    std::vector<float> want(static_cast<size_t>(M) * N, 0.0f);
    double tol = 0;
    if (w4a4) {
        std::vector<uint8_t> wq(static_cast<size_t>(N) * K / 2);
        for (auto& v : wq) v = static_cast<uint8_t>(r.next());
        std::vector<float> ws(static_cast<size_t>(G) * N);
        for (auto& v : ws) v = 0.001f + 0.01f * r.uniform();
        qw.nunchaku_swizzle = true;
        qw.had_block_size = 1;
        qw.smooth = upload(sm, {K}, DType::FP32);
        qw.qweight_rowmajor = upload(wq, {N, K / 2}, DType::UINT8);
        qw.wscales_rowmajor = upload(ws, {G, N}, DType::FP32);
        qw.qweight_mma = Tensor::alloc({static_cast<int64_t>(G) * ((N + 7) / 8) * 256}, DType::UINT8);
        swizzle_w4a4_weights_mma(static_cast<const uint8_t*>(qw.qweight_rowmajor.data),
                                 static_cast<uint32_t*>(qw.qweight_mma.data), N, K, gs);
        HIP_CHECK(hipDeviceSynchronize());
        qw.qweight_rowmajor.free_data();
        std::vector<uint8_t> pk(static_cast<size_t>(M) * K / 2);
        std::vector<float> as(static_cast<size_t>(G) * M);
        or_quant_act_int4(xf.data(), sm.data(), M, K, gs, nullptr, pk.data(), as.data());
        or_w4a4_gemm(pk.data(), wq.data(), as.data(), ws.data(), M, N, K, gs, 1, b.data(), 0, M, want.data());
    } else {
        std::vector<float> resid = f32_normal(r, static_cast<size_t>(N) * K, 0.02f);
        std::vector<uint8_t> q4(static_cast<size_t>(N) * K / 2);
        std::vector<float> s4(static_cast<size_t>(N) * G);
        or_quant_int4_nf4(resid.data(), N, K, gs, q4.data(), s4.data());
        const int hbs = K & -K;
        qw.had_block_size = hbs;
        qw.nf4_grid = true;
        qw.qweight = upload(q4, {N, K / 2}, DType::UINT8);
        qw.scales4 = upload(s4, {N, G}, DType::FP32);
        std::vector<float> xr = xf;
        or_fwht_rows(xr.data(), M, K, hbs);
        std::vector<uint16_t> deq(static_cast<size_t>(N) * K);
        or_dequant_int4_bf16(q4.data(), s4.data(), N, K, gs, 1, 0, 0, deq.data());
        for (int m = 0; m < M; ++m)
            for (int n = 0; n < N; ++n) {
                double acc = 0, mag = 0;
                for (int k = 0; k < K; ++k) {
                    const double p = static_cast<double>(or_bf16_to_f32(or_f32_to_bf16(xr[static_cast<size_t>(m) * K + k]))) *
                                     or_bf16_to_f32(deq[static_cast<size_t>(n) * K + k]);
                    acc += p;
                    mag += std::fabs(p);
                }
                want[static_cast<size_t>(m) * N + n] = static_cast<float>(acc + or_bf16_to_f32(b[n]));
                tol = std::fmax(tol, 8 * std::sqrt(static_cast<double>(K)) * std::ldexp(mag, -24) + 1e-6);
            }
    }
    Tensor bias = upload(b, {N}, DType::BF16);
    Tensor x = bf16_in ? upload(xb, {M, K}, DType::BF16) : upload(xf, {M, K}, DType::FP32);
    Tensor out = Tensor::alloc({M, N}, DType::FP32);
    Tensor scratch = Tensor::alloc({int4_scratch_bytes(M, K, N, rank)}, DType::UINT8);
    if (bf16_in)
        linear_forward_quantized_bf16in(x, qw, &bias, out, scratch);
    else
        linear_forward_quantized(x, qw, &bias, out, scratch);
    HIP_CHECK(hipDeviceSynchronize());
    const double d = max_abs_diff(download<float>(out), want);
    char name[96], det[64];
    snprintf(name, sizeof(name), "int4 %s linear %s M=%d N=%d K=%d", w4a4 ? "W4A4" : "W4A16",
             bf16_in ? "bf16in" : "fp32in", M, N, K);
    snprintf(det, sizeof(det), "max|diff|=%.3g tol=%.3g", d, tol);
    report(name, d <= tol, det);
}

// INT4_AWQ (M = 1) through linear_forward_quantized, loaded as
// transformer.h:427-456 does (repack at load): bit-exact against the oracle.
void case_awq(int OC, int IC) {
    Rng r(OC + IC);
    const int gs = 64, nc = 6;
    std::vector<int32_t> q(static_cast<size_t>(OC / 4) * (IC / 2));
    for (auto& v : q) v = static_cast<int32_t>(r.next());
    std::vector<uint16_t> ws(static_cast<size_t>(IC / gs) * OC), wz(ws.size()), b(OC);
    for (auto& v : ws) v = or_f32_to_bf16(0.001f + 0.01f * r.uniform());
    for (auto& v : wz) v = or_f32_to_bf16(0.1f * r.normal());
    for (auto& v : b) v = or_f32_to_bf16(0.01f * r.normal());
    std::vector<float> x = f32_normal(r, IC, 1.0f);
    QuantizedWeight qw;
    qw.mode = QuantMode::INT4_AWQ;
    Tensor raw = upload(q, {OC / 4, IC / 2}, DType::INT32);
    qw.awq_wscales = upload(ws, {IC / gs, OC}, DType::BF16);
    qw.awq_wzeros = upload(wz, {IC / gs, OC}, DType::BF16);
    qw.awq_OC = OC;
    qw.awq_IC = IC;
    qw.awq_group_size = gs;
    qw.awq_num_components = nc;
    qw.awq_qweight = Tensor::alloc({IC / 8, OC}, DType::INT32);
    repack_awq_to_transposed(static_cast<const int32_t*>(raw.data), static_cast<int32_t*>(qw.awq_qweight.data), OC, IC);
    HIP_CHECK(hipDeviceSynchronize());
    Tensor xt = upload(x, {1, IC}, DType::FP32), bias = upload(b, {OC}, DType::BF16);
    Tensor out = Tensor::alloc({1, OC}, DType::FP32), scratch = Tensor::alloc({16}, DType::UINT8);
    linear_forward_quantized(xt, qw, &bias, out, scratch);
    HIP_CHECK(hipDeviceSynchronize());
    std::vector<int32_t> rep(static_cast<size_t>(IC / 8) * OC);
    or_awq_repack(q.data(), OC, IC, rep.data());
    std::vector<float> want(OC);
    or_awq_gemv(x.data(), rep.data(), ws.data(), wz.data(), b.data(), OC, IC, gs, nc, want.data());
    const double d = max_abs_diff(download<float>(out), want);
    char name[96], det[64];
    snprintf(name, sizeof(name), "awq linear OC=%d IC=%d", OC, IC);
    snprintf(det, sizeof(det), "max|diff|=%.3g", d);
    report(name, d == 0.0, det);
}

int main(int argc, char** argv) {
    if (argc == 3 && std::string(argv[1]) == "--expect-error") return expect_error(argv[2]);
    case_tensor_api();
    case_weight_quant(QuantMode::INT8_HADAMARD, 3072, 3072);
    case_weight_quant(QuantMode::INT8_HADAMARD, 256, 12288);
    case_weight_quant(QuantMode::FP8_HADAMARD, 512, 3072);
    case_linear(false, 300, 320, 3072, true, false);
    case_linear(true, 64, 256, 12288, true, false);
    case_linear(true, 257, 255, 1024, false, false);
    case_linear(false, 96, 512, 3072, true, true);
    case_linear(true, 1, 18432 / 8, 3072, true, false);
    case_prequantized_and_dequant();
    case_fp8_linear();
    case_bf16_mode(true, 64, 3072, 64);     // img_in
    case_bf16_mode(true, 32, 512, 3584);    // txt_in (a slice of N)
    case_bf16_mode(false, 1, 6144, 3072);   // norm_out
    case_bf16_mode(false, 96, 64, 3072);    // proj_out
    case_int4(true, false, 96, 384, 3072);
    case_int4(true, true, 33, 256, 1024);
    case_int4(false, false, 40, 256, 3072);
    case_int4(false, true, 17, 128, 1024);
    case_awq(18432, 3072);                  // the modulation layer
    case_awq(96, 128);
    case_sage(2, 300, 128, false);
    case_sage(3, 129, 64, true);
    case_block_loop();
    case_checkpoint_roundtrip();
    printf("%s: %d failure(s)\n", g_fail ? "FAILED" : "PASSED", g_fail);
    return g_fail ? 1 : 0;
}
