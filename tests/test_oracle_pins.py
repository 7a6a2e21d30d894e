"""Pins the CPU oracle against facts fixed independently of its own code:
closed forms, explicit Hadamard matrices, library conversions (numpy, torch),
brute-force integer products, hand-derived known answers for the reference's
stage order and scale-group layout, and float64 attention/linear algebra.

No reference source is executed: the reference is CUDA and cannot be built
here, and it ships no golden vectors for this path.

What these checks cannot pin: the reference binary is compiled with
--use_fast_math (Makefile:11), so its `127.0f / amax`, `1.0f / scale`,
rsqrtf, tanhf and ex2.approx are approximations. The oracle (and the GPU
path) use correctly rounded division and rsqrt, so a value that lands exactly
on an int8 rounding tie can round differently from a CUDA run of the
reference. Nothing in the reference's tree records such a run.
"""
import math

import numpy as np
import pytest
import scipy.linalg
import torch

# ------------------------------------------------------------------ a1


def test_hadamard_block_size_closed_form(oracle):
    for K in range(1, 5000):
        hbs = oracle.hadamard_block_size(K)
        # largest power of two dividing K
        assert K % hbs == 0 and (K // hbs) % 2 == 1 and hbs & (hbs - 1) == 0
    assert [oracle.hadamard_block_size(k) for k in (3072, 12288, 256, 64, 3584)] == [1024, 4096, 256, 64, 512]


# ------------------------------------------------------------------ a2


@pytest.mark.parametrize("n", [2, 4, 8, 16, 32, 64, 128, 256, 512, 1024, 2048, 4096])
def test_fwht_matches_explicit_hadamard(oracle, n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal((3, n)).astype(np.float32)
    H = scipy.linalg.hadamard(n).astype(np.float64) / math.sqrt(n)
    ref = x.astype(np.float64) @ H.T
    got = oracle.fwht_rows(x, n).astype(np.float64)
    assert np.max(np.abs(got - ref)) <= 1e-6 * math.sqrt(math.log2(n) + 1) * np.max(np.abs(ref)) + 1e-6


def test_fwht_block_diagonal(oracle):
    rng = np.random.default_rng(1)
    K, hbs = 3072, 1024
    x = rng.standard_normal((2, K)).astype(np.float32)
    H = scipy.linalg.hadamard(hbs).astype(np.float64) / 32.0
    ref = np.concatenate([x[:, i * hbs:(i + 1) * hbs].astype(np.float64) @ H.T for i in range(3)], axis=1)
    got = oracle.fwht_rows(x, hbs)
    assert np.max(np.abs(got - ref)) < 1e-4


def test_fwht_involution_and_parseval(oracle):
    rng = np.random.default_rng(2)
    x = rng.standard_normal((4, 12288)).astype(np.float32)
    y = oracle.fwht_rows(x, 4096)
    np.testing.assert_allclose(np.sum(y.astype(np.float64) ** 2, 1), np.sum(x.astype(np.float64) ** 2, 1),
                               rtol=1e-5)
    np.testing.assert_allclose(oracle.fwht_rows(y, 4096), x, atol=2e-5)


def test_fwht_stage_order_known_answer(oracle):
    # Hand evaluation of cuda_kernels.cu:2226-2241 (half = 1 first, then 2)
    # on x = [1, 2^-24, -1, 0] in fp32:
    #   half=1: [1 + 2^-24 -> 1 (tie to even), 1 - 2^-24, -1, -1]
    #   half=2: [0, -2^-24, 2, 2 - 2^-24 -> 2 (tie to even)]
    # then * rsqrt(4) = 0.5 (exact). Running half=2 first would instead give
    # [2^-24, -2^-24, 2, 2] * 0.5, so this pins the stage order.
    e = 2.0 ** -24
    x = np.array([[1.0, e, -1.0, 0.0]], np.float32)
    got = oracle.fwht_rows(x, 4)
    np.testing.assert_array_equal(got, np.array([[0.0, -e, 2.0, 2.0]], np.float32) * np.float32(0.5))


def test_fwht_norm_values(oracle):
    assert oracle.lib().or_fwht_norm(1024) == 1.0 / 32
    assert oracle.lib().or_fwht_norm(4096) == 1.0 / 64
    assert oracle.lib().or_fwht_norm(256) == 1.0 / 16
    assert oracle.lib().or_fwht_norm(512) == float(np.float32(1.0 / math.sqrt(512.0)))


# ------------------------------------------------------------------ a3


def test_quant_rows_special_cases(oracle):
    K = 64
    x = np.zeros((6, K), np.float32)
    x[1, 5] = 5.0          # positive spike
    x[2, 7] = -5.0         # negative spike
    # amax = 127 -> inv = 1 exactly; halves round to even
    x[3, :7] = [127.0, 2.5, 3.5, -2.5, 0.5, 1.5, 126.5]
    x[4, :3] = [1e-30, -1e-30, 0.0]     # tiny amax
    x[5, :] = -3.0                      # constant row
    q, s = oracle.quant_rows_int8(x)
    assert s[0] == 0.0 and not q[0].any()
    assert q[1, 5] == 127 and np.count_nonzero(q[1]) == 1 and s[1] == np.float32(5.0) / np.float32(127.0)
    assert q[2, 7] == -127 and np.count_nonzero(q[2]) == 1
    assert list(q[3, :7]) == [127, 2, 4, -2, 0, 2, 126]
    assert list(q[4, :3]) == [127, -127, 0]
    assert (q[5] == -127).all()


def test_quant_rows_properties(oracle):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((64, 3072)) * rng.uniform(0.01, 100, (64, 1))).astype(np.float32)
    q, s = oracle.quant_rows_int8(x)
    assert np.abs(q.astype(np.int32)).max() <= 127
    amax = np.abs(x).max(1)
    assert (np.abs(q[np.arange(64), np.abs(x).argmax(1)]) == 127).all()
    np.testing.assert_array_equal(s, amax / np.float32(127.0))
    err = np.abs(q.astype(np.float64) * s[:, None] - x)
    assert (err <= s[:, None] * 0.5 * (1 + 1e-5) + 1e-12).all()


# ------------------------------------------------------------------ conversions


def test_f16_conversion_matches_numpy(oracle):
    rng = np.random.default_rng(4)
    v = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 1000,
        rng.standard_normal(5000).astype(np.float32) * 1e-5,   # fp16 subnormals
        np.array([65504.0, 65519.0, 65520.0, 1e6, 6e-8, 3e-8, 2.98e-8, -0.0, 0.0], np.float32)])
    L = oracle.lib()
    got = np.array([L.or_f32_to_f16(float(t)) for t in v], np.uint16)
    with np.errstate(over="ignore"):
        np.testing.assert_array_equal(got, v.astype(np.float16).view(np.uint16))
    back = np.array([L.or_f16_to_f32(int(b)) for b in got[:3000]], np.float32)
    np.testing.assert_array_equal(back, got[:3000].view(np.float16).astype(np.float32))


def test_bf16_conversion_matches_torch(oracle):
    rng = np.random.default_rng(5)
    v = rng.standard_normal(50000).astype(np.float32) * np.float32(10.0) ** rng.integers(-20, 20, 50000)
    got = oracle.bf16_bits_from_f32(v)
    ref = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(got, ref)


def test_e4m3_conversion_matches_torch(oracle):
    rng = np.random.default_rng(6)
    v = np.concatenate([rng.uniform(-448, 448, 20000), rng.standard_normal(5000) * 0.01,
                        np.array([448.0, -448.0, 0.0, 2 ** -9, 2 ** -10, 3 * 2 ** -11, 0.015625])]).astype(np.float32)
    L = oracle.lib()
    got = np.array([L.or_f32_to_e4m3(float(t)) for t in v], np.uint8)
    ref = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(got, ref)
    np.testing.assert_array_equal(oracle.e4m3_to_f32(got), torch.from_numpy(ref).view(torch.float8_e4m3fn).float().numpy())


# ------------------------------------------------------------------ a7, a8, a9


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (7, 13, 64), (33, 65, 300), (64, 128, 3072)])
def test_int_gemm_brute_force(oracle, M, N, K):
    rng = np.random.default_rng(M * N + K)
    a = rng.integers(-128, 128, (M, K), dtype=np.int8)
    w = rng.integers(-128, 128, (N, K), dtype=np.int8)
    ref = a.astype(np.int64) @ w.astype(np.int64).T
    np.testing.assert_array_equal(oracle.gemm_s8s8s32(a, w), ref.astype(np.int32))


def test_epilogue_against_float64(oracle):
    rng = np.random.default_rng(7)
    M, N = 40, 96
    c = rng.integers(-2 ** 24, 2 ** 24, (M, N)).astype(np.int32)
    sa = rng.uniform(1e-4, 1e-2, M).astype(np.float32)
    sw = rng.uniform(1e-4, 1e-2, N).astype(np.float32)
    bias = oracle.bf16_bits_from_f32(rng.standard_normal(N).astype(np.float32))
    bf = oracle.bf16_bits_to_f32(bias).astype(np.float64)
    lin = c.astype(np.float64) * sa[:, None] * sw[None, :] + bf[None, :]
    out = oracle.dequant_epilogue(c, sa, sw, bias, gelu=False)
    np.testing.assert_allclose(out, lin, rtol=1e-6, atol=1e-6)
    g = oracle.dequant_epilogue(c, sa, sw, bias, gelu=True)
    gref = 0.5 * lin * (1 + np.tanh(math.sqrt(2 / math.pi) * (lin + 0.044715 * lin ** 3)))
    np.testing.assert_allclose(g, gref, rtol=1e-5, atol=1e-5)


def _metrics(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    rel = np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30)
    cos = float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-300))
    return rel, cos


@pytest.mark.parametrize("K,N", [(3072, 256), (12288, 128), (256, 64)])
def test_w8a8_linear_against_float64_matmul(oracle, K, N):
    # x H (w H)^T = x w^T for the orthonormal symmetric block Hadamard H, so
    # the quantized linear must approximate the plain product.
    rng = np.random.default_rng(K + N)
    M = 64
    x = rng.standard_normal((M, K)).astype(np.float32)
    w_bits = oracle.bf16_bits_from_f32((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    b_bits = oracle.bf16_bits_from_f32((rng.standard_normal(N) * 0.01).astype(np.float32))
    wq, ws, hbs = oracle.quantize_weight_bf16(w_bits)
    assert hbs == K & -K
    out = oracle.linear_w8a8(x, wq, ws, hbs, b_bits)
    ref = x.astype(np.float64) @ oracle.bf16_bits_to_f32(w_bits).reshape(N, K).astype(np.float64).T \
        + oracle.bf16_bits_to_f32(b_bits).astype(np.float64)
    rel, cos = _metrics(out, ref)
    assert rel <= 2e-2 and cos >= 0.999, (rel, cos)


def test_weight_quant_is_rotation_then_rowquant(oracle):
    rng = np.random.default_rng(8)
    w_bits = oracle.bf16_bits_from_f32(rng.standard_normal((16, 3072)).astype(np.float32))
    q, s, hbs = oracle.quantize_weight_bf16(w_bits)
    q2, s2 = oracle.quant_rows_int8(oracle.fwht_rows(oracle.bf16_bits_to_f32(w_bits).reshape(16, 3072), hbs))
    np.testing.assert_array_equal(q, q2)
    np.testing.assert_array_equal(s, s2)
    # activation path on the same fp32 data agrees with the weight path
    qa, sa = oracle.quantize_activation(w_bits, hbs)
    np.testing.assert_array_equal(qa, q)
    np.testing.assert_array_equal(sa, s)


def test_fp8_linear_against_float64_matmul(oracle):
    rng = np.random.default_rng(9)
    M, N, K = 48, 96, 3072
    x = rng.standard_normal((M, K)).astype(np.float32)
    w_bits = oracle.bf16_bits_from_f32((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    wq, ws, hbs = oracle.quantize_weight_fp8(w_bits)
    xq, xs = oracle.quantize_activation_fp8(x, hbs)
    assert np.abs(oracle.e4m3_to_f32(xq)).max() == 448.0
    out = oracle.gemm_fp8_epilogue(xq, wq, xs, ws)
    ref = x.astype(np.float64) @ oracle.bf16_bits_to_f32(w_bits).reshape(N, K).astype(np.float64).T
    rel, cos = _metrics(out, ref)
    assert rel <= 5e-2 and cos >= 0.999, (rel, cos)


# ------------------------------------------------------------------ Sage


def test_sage_k_mean_sequential_sum(oracle):
    rng = np.random.default_rng(10)
    k = rng.standard_normal((3, 1000, 64)).astype(np.float16)
    mean = oracle.sage_k_mean(k)
    # np.add.accumulate is a left-to-right fp32 running sum: the reference's
    # single-thread loop, computed by an independent routine.
    seq = np.add.accumulate(k.astype(np.float32), axis=1, dtype=np.float32)[:, -1, :]
    np.testing.assert_array_equal(mean, seq / np.float32(1000))
    np.testing.assert_allclose(mean, k.astype(np.float64).mean(1), atol=1e-5)


def test_sage_q_scale_groups_known_answer(oracle):
    # Per sageattention_sm80.cu:787-812 the scale at index b*32 + w*8 + g
    # covers tokens b*128 + w*32 + g + 8i (i < 4). With token t filled with
    # the value t + 1 the group maximum is its last token + 1.
    S, D = 256, 64
    q = np.broadcast_to((np.arange(S, dtype=np.float32) + 1)[None, :, None], (1, S, D)).astype(np.float16)
    qi, qs = oracle.sage_quant_q(q)
    for b in range(2):
        for w in range(4):
            for g in range(8):
                amax = np.float32(b * 128 + w * 32 + g + 24 + 1)
                assert qs[0, b * 32 + w * 8 + g] == amax / np.float32(127) + np.float32(1e-7)
    # group (b=0, w=0, g=7) = tokens 7, 15, 23, 31 (values 8..32): the last
    # maps to 127, the first to rne(8 * 127 / 32) = 32
    assert (qi[0, 31] == 127).all() and (qi[0, 7] == 32).all()


def test_sage_k_scale_groups_known_answer(oracle):
    # Per sageattention_sm80.cu:839-870 the scale at index b*4 + g covers
    # tokens b*64 + 2g + {0,1} + 8i (i < 8). Values k = t+1 and a zero mean
    # (mean passed explicitly) make each group's max its last token + 1.
    S, D = 128, 64
    k = np.broadcast_to((np.arange(S, dtype=np.float32) + 1)[None, :, None], (1, S, D)).astype(np.float16)
    ki, ks = oracle.sage_quant_k(k, np.zeros((1, D), np.float32))
    for b in range(2):
        for g in range(4):
            amax = np.float32(b * 64 + 2 * g + 1 + 56 + 1)
            assert ks[0, b * 4 + g] == amax / np.float32(127) + np.float32(1e-7)


def _attn64(q, k, v, scale, causal):
    s = np.einsum("hqd,hkd->hqk", q, k) * scale
    if causal:
        S = q.shape[1]
        s = np.where(np.tril(np.ones((S, S), bool))[None], s, -np.inf)
    s -= s.max(-1, keepdims=True)
    p = np.exp(s)
    return np.einsum("hqk,hkd->hqd", p / p.sum(-1, keepdims=True), v)


@pytest.mark.parametrize("S,D,causal", [(200, 128, False), (64, 64, False), (1, 128, False),
                                        (333, 128, True), (130, 64, True)])
def test_sage_attention_against_float64(oracle, S, D, causal):
    rng = np.random.default_rng(S * D + causal)
    BH = 2
    q = rng.standard_normal((BH, S, D)).astype(np.float16)
    k = (rng.standard_normal((BH, S, D)) + 0.5).astype(np.float16)   # non-zero mean exercises smoothing
    v = rng.standard_normal((BH, S, D)).astype(np.float16)
    scale = 1.0 / math.sqrt(D)
    out = oracle.sage_attention_fp16io(q, k, v, scale, causal).astype(np.float64)
    # tight: float64 attention on the oracle's own dequantized Q/K
    mean = oracle.sage_k_mean(k)
    qi, qs = oracle.sage_quant_q(q)
    ki, ks = oracle.sage_quant_k(k, mean)
    t = np.arange(S)
    qsc = qs[:, (t // 128) * 32 + ((t % 128) // 32) * 8 + t % 8]
    ksc = ks[:, (t // 64) * 4 + (t % 8) // 2]
    qd = qi.astype(np.float64) * qsc[..., None]
    kd = ki.astype(np.float64) * ksc[..., None]
    tight = _attn64(qd, kd, v.astype(np.float64), scale, causal)
    assert np.max(np.abs(out - tight)) <= 4e-3 * np.max(np.abs(tight)) + 1e-3
    # loose: unquantized attention at the stated tolerance
    ref = _attn64(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64), scale, causal)
    rel, cos = _metrics(out, ref)
    assert rel <= 2e-2 and cos >= 0.999, (rel, cos)


def test_linear_bf16_oracle_pins(oracle):
    """The BF16-mode linear's oracle: integer-valued operands (exact in bf16,
    every partial sum exact in fp32) equal the int64 product plus the bias;
    fp32 inputs are rounded as torch rounds to bfloat16 (an independent
    implementation of nearest even); GELU is the tanh form at known points."""
    import torch
    rng = np.random.default_rng(41)
    M, N, K = 9, 13, 3584
    xi = rng.integers(-4, 5, (M, K))
    wi = rng.integers(-4, 5, (N, K))
    b = oracle.bf16_bits_from_f32(rng.integers(-8, 9, N).astype(np.float32))
    out, mag = oracle.linear_bf16(xi.astype(np.float32), oracle.bf16_bits_from_f32(wi.astype(np.float32)), b)
    np.testing.assert_array_equal(out, (xi @ wi.T + oracle.bf16_bits_to_f32(b)[None]).astype(np.float64))
    np.testing.assert_array_equal(mag, np.abs(xi) @ np.abs(wi).T)
    # one-hot weights pick bf16(x) exactly
    x = rng.standard_normal((5, 64)).astype(np.float32) * 3
    eye = oracle.bf16_bits_from_f32(np.eye(64, dtype=np.float32))
    got, _ = oracle.linear_bf16(x, eye)
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(got.astype(np.float32), want)
    # bf16 inputs are used as given
    got16, _ = oracle.linear_bf16(oracle.bf16_bits_from_f32(x), eye)
    np.testing.assert_array_equal(got16, got)
    g = oracle.gelu_tanh64(np.array([0.0, 10.0, -10.0, 1.0]))
    assert g[0] == 0.0 and abs(g[1] - 10.0) < 1e-12 and abs(g[2]) < 1e-12
    assert abs(g[3] - 0.8411919906) < 1e-9  # 0.5 (1 + tanh(0.7978845608 * 1.044715))
