"""GPU parity: the fused quantized linear against the oracle.

* The integer product is checked exactly: with unit scales and no bias the
  fp32 output is fl(acc), the correctly rounded int32 dot product.
* The dequant epilogue (no GELU) follows the reference's operation order
  without contraction, so it is compared bit for bit as well.
* GELU (tanhf), bf16 outputs and e4m3 accumulation order are checked against
  tolerances: max|a-b|/max|b| <= 2e-2 and cosine >= 0.999 (the stated bar),
  plus much tighter bounds where the arithmetic allows.
* At the full layer shapes the oracle runs on a sample of rows.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _metrics(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    rel = np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30)
    cos = float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-300))
    return rel, cos


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _bf16_dev(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(DEV).view(torch.bfloat16)


def _qw(qimg, q, s, hbs, mode=0):
    return qimg.QuantizedWeight(_dev(q), _dev(s), hbs, mode)


KERNELS = {"auto": 0, "large": 1, "small32": 2, "small64": 3, "gemv": 4, "w192": 5, "w224": 6, "t128": 7}


@pytest.mark.parametrize("kernel", list(KERNELS))
@pytest.mark.parametrize("M,N,K", [
    (256, 256, 64), (1, 64, 64), (7, 300, 192), (300, 7, 128), (256, 256, 128), (129, 384, 384),
    (513, 520, 3072),
    (257, 255, 1024), (64, 3072, 3072), (4096, 3072, 3072),
])
def test_int8_gemm_exact(qimg, oracle, M, N, K, kernel):
    """Every kernel choice gives the exact int32 product (fp32 out with unit
    scales is fl(acc))."""
    if kernel in ("small32", "gemv") and M * N > 2 ** 22:
        pytest.skip("32x32 tiles at this size only repeat the small-shape cases")
    rng = np.random.default_rng(M + 3 * N + 7 * K)
    a = rng.integers(-128, 128, (M, K), dtype=np.int8)
    w = rng.integers(-128, 128, (N, K), dtype=np.int8)
    ones_m = np.ones(M, np.float32)
    ones_n = np.ones(N, np.float32)
    rows = (0, M) if M * N * K <= 2 ** 31 else None
    with qimg.linear_kernel(KERNELS[kernel]):
        out = qimg.linear_forward_prequantized(_dev(a), _dev(ones_m), _qw(qimg, w, ones_n, 1))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    if rows is None:  # full-size: check a sample of rows
        idx = np.unique(np.concatenate([[0, M - 1], rng.integers(0, M, 62)]))
        ref = (a[idx].astype(np.int64) @ w.astype(np.int64).T).astype(np.float32)
        np.testing.assert_array_equal(got[idx], ref)
    else:
        ref = oracle.gemm_s8s8s32(a, w).astype(np.float32)
        np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("M,N,K,with_bias", [(300, 320, 3072, True), (64, 256, 12288, True),
                                             (130, 200, 256, False), (5, 96, 100, True)])
def test_int8_linear_fp32_bit_exact(qimg, oracle, M, N, K, with_bias):
    rng = np.random.default_rng(M * N + K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w_bits = oracle.bf16_bits_from_f32((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    b_bits = oracle.bf16_bits_from_f32((rng.standard_normal(N) * 0.01).astype(np.float32)) if with_bias else None
    wq, ws, hbs = oracle.quantize_weight_bf16(w_bits)
    ref = oracle.linear_w8a8(x, wq, ws, hbs, b_bits)
    out = qimg.linear_forward_quantized(_dev(x), _qw(qimg, wq, ws, hbs),
                                        None if b_bits is None else _bf16_dev(b_bits))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), ref)


def test_int8_linear_gelu_and_bf16_out(qimg, oracle):
    rng = np.random.default_rng(21)
    M, N, K = 320, 512, 3072
    x_bits = oracle.bf16_bits_from_f32(rng.standard_normal((M, K)).astype(np.float32))
    w_bits = oracle.bf16_bits_from_f32((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    b_bits = oracle.bf16_bits_from_f32((rng.standard_normal(N) * 0.01).astype(np.float32))
    wq, ws, hbs = oracle.quantize_weight_bf16(w_bits)
    qw = _qw(qimg, wq, ws, hbs)
    ref_g = oracle.linear_w8a8(x_bits, wq, ws, hbs, b_bits, gelu=True)
    ref = oracle.linear_w8a8(x_bits, wq, ws, hbs, b_bits, gelu=False)
    xd, bd = _bf16_dev(x_bits), _bf16_dev(b_bits)
    g = qimg.linear_forward_quantized(xd, qw, bd, apply_gelu=True)
    o16 = qimg.linear_forward_quantized(xd, qw, bd, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    np.testing.assert_allclose(g.cpu().numpy(), ref_g, rtol=2e-6, atol=2e-6)
    np.testing.assert_array_equal(o16.float().cpu().numpy(),
                                  oracle.bf16_bits_to_f32(oracle.bf16_bits_from_f32(ref)).reshape(M, N))
    # end to end against the unquantized product (the stated tolerance)
    xf = oracle.bf16_bits_to_f32(x_bits).reshape(M, K).astype(np.float64)
    wf = oracle.bf16_bits_to_f32(w_bits).reshape(N, K).astype(np.float64)
    exact = xf @ wf.T + oracle.bf16_bits_to_f32(b_bits)
    rel, cos = _metrics(o16.float().cpu().numpy(), exact)
    assert rel <= 2e-2 and cos >= 0.999, (rel, cos)


@pytest.mark.parametrize("M,N,K", [(256, 256, 3072), (100, 300, 12288), (4352, 512, 3072)])
def test_fp8_linear(qimg, oracle, M, N, K):
    rng = np.random.default_rng(M + N + K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w_bits = oracle.bf16_bits_from_f32((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    b_bits = oracle.bf16_bits_from_f32((rng.standard_normal(N) * 0.01).astype(np.float32))
    wq, ws, hbs = oracle.quantize_weight_fp8(w_bits)
    xq, xs = oracle.quantize_activation_fp8(x, hbs)
    rows = (0, min(M, 256))
    ref = oracle.gemm_fp8_epilogue(xq, wq, xs, ws, b_bits, rows=rows)[rows[0]:rows[1]]
    qw = _qw(qimg, wq, ws, hbs, mode=qimg.FP8_HADAMARD)
    out = qimg.linear_forward_quantized(_dev(x), qw, _bf16_dev(b_bits))
    torch.cuda.synchronize()
    got = out.cpu().numpy()[rows[0]:rows[1]]
    # fp32 accumulation order differs from the float64 oracle sum only
    scale = np.abs(ref).max()
    assert np.max(np.abs(got - ref)) <= 1e-5 * scale * np.sqrt(K / 64), np.max(np.abs(got - ref))
    exact = x[rows[0]:rows[1]].astype(np.float64) @ oracle.bf16_bits_to_f32(w_bits).reshape(N, K).astype(np.float64).T \
        + oracle.bf16_bits_to_f32(b_bits)
    rel, cos = _metrics(got, exact)
    assert rel <= 5e-2 and cos >= 0.999, (rel, cos)


@pytest.mark.parametrize("M,N,K", [(600, 518, 512), (777, 1000, 256), (1100, 3076, 1024), (6889, 3072, 1024)])
def test_fp8_tile_widths(qimg, oracle, M, N, K):
    """e4m3 on 256x256 and 256x192 tiles (waves 4 x 2 of 64x96): each
    output's k-sum runs through the same MFMA sequence, so the two widths
    agree bit for bit (fp32 and bf16 out, GELU), on ragged tiles too (last
    tiles of 134, 40, 4 and 0 columns), and both are within the fp32
    accumulation-order bound of the oracle's float64 sum: the fp32 output,
    the bf16 output (plus its rounding) and the GELU output (plus the
    GELU approximation's error)."""
    rng = np.random.default_rng(M + 7 * N + K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w_bits = oracle.bf16_bits_from_f32((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    b_bits = oracle.bf16_bits_from_f32((rng.standard_normal(N) * 0.01).astype(np.float32))
    wq, ws, hbs = oracle.quantize_weight_fp8(w_bits)
    xq, xs = oracle.quantize_activation_fp8(x, hbs)
    qw = _qw(qimg, wq, ws, hbs, mode=qimg.FP8_HADAMARD)
    xd, bd = _dev(x), _bf16_dev(b_bits)
    outs = {}
    for kernel in ("large", "w192"):
        with qimg.linear_kernel(KERNELS[kernel]):
            outs[kernel] = (qimg.linear_forward_quantized(xd, qw, bd),
                            qimg.linear_forward_quantized(xd, qw, bd, out_dtype=torch.bfloat16),
                            qimg.linear_forward_quantized(xd, qw, bd, apply_gelu=True))
    torch.cuda.synchronize()
    for a, b in zip(outs["large"], outs["w192"]):
        assert torch.equal(a, b)
    rows = (0, min(M, 300))
    ref = oracle.gemm_fp8_epilogue(xq, wq, xs, ws, b_bits, rows=rows)[rows[0]:rows[1]]
    got = outs["w192"][0].cpu().numpy()[rows[0]:rows[1]]
    bound = 1e-5 * np.abs(ref).max() * np.sqrt(K / 64)
    assert np.max(np.abs(got - ref)) <= bound
    # bf16 out: the round-to-nearest of a value within that bound (half a
    # bf16 ulp is at most 2^-8 relative)
    got_h = outs["w192"][1].float().cpu().numpy()[rows[0]:rows[1]]
    assert np.all(np.abs(got_h - ref) <= np.abs(ref) * 2.0 ** -8 + 1.01 * bound)
    # GELU: the bound carried through GELU (slope below 1.13) plus the
    # GELU approximation's own 2e-6
    ref_g = oracle.gemm_fp8_epilogue(xq, wq, xs, ws, b_bits, gelu=True, rows=rows)[rows[0]:rows[1]]
    got_g = outs["w192"][2].cpu().numpy()[rows[0]:rows[1]]
    assert np.max(np.abs(got_g - ref_g)) <= 1.13 * bound + 2e-6 * np.abs(ref_g).max()


@pytest.mark.slow
def test_mlp_pair_full_size_sampled(qimg, oracle):
    """MMDiT MLP at M=4352: fc1 (3072->12288, GELU) -> FWHT(4096)+quant -> fc2,
    checked on sampled rows against the oracle chain and the float64 MLP."""
    rng = np.random.default_rng(0)
    M, D, H = 4352, 3072, 12288
    x_bits = oracle.bf16_bits_from_f32(rng.standard_normal((M, D)).astype(np.float32))
    w1 = oracle.bf16_bits_from_f32((rng.standard_normal((H, D)) * 0.02).astype(np.float32))
    w2 = oracle.bf16_bits_from_f32((rng.standard_normal((D, H)) * 0.02).astype(np.float32))
    b1 = oracle.bf16_bits_from_f32((rng.standard_normal(H) * 0.01).astype(np.float32))
    b2 = oracle.bf16_bits_from_f32((rng.standard_normal(D) * 0.01).astype(np.float32))
    qw1 = qimg.quantize_weight_tensor(_bf16_dev(w1))
    qw2 = qimg.quantize_weight_tensor(_bf16_dev(w2))
    h = qimg.linear_forward_quantized(_bf16_dev(x_bits), qw1, _bf16_dev(b1), apply_gelu=True)
    y = qimg.linear_forward_quantized(h, qw2, _bf16_dev(b2), out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    idx = np.unique(np.concatenate([[0, 4095, 4096, M - 1], rng.integers(0, M, 28)]))
    w1q, w1s, _ = oracle.quantize_weight_bf16(w1)
    w2q, w2s, _ = oracle.quantize_weight_bf16(w2)
    np.testing.assert_array_equal(qw1.data.cpu().numpy(), w1q)
    np.testing.assert_array_equal(qw2.scales.cpu().numpy(), w2s)
    h_ref = oracle.linear_w8a8(x_bits[idx], w1q, w1s, 1024, b1, gelu=True)
    h_got = h.cpu().numpy()[idx]
    np.testing.assert_allclose(h_got, h_ref, rtol=2e-6, atol=2e-6)
    y_ref = oracle.linear_w8a8(h_got, w2q, w2s, 4096, b2)
    y_got = y.float().cpu().numpy()[idx]
    rel, cos = _metrics(y_got, y_ref)
    assert rel <= 1e-2 and cos >= 0.99999, (rel, cos)
    xf = oracle.bf16_bits_to_f32(x_bits).reshape(M, D)[idx].astype(np.float64)
    w1f = oracle.bf16_bits_to_f32(w1).reshape(H, D).astype(np.float64)
    w2f = oracle.bf16_bits_to_f32(w2).reshape(D, H).astype(np.float64)
    t = xf @ w1f.T + oracle.bf16_bits_to_f32(b1)
    t = 0.5 * t * (1 + np.tanh(0.7978845608 * (t + 0.044715 * t ** 3)))
    exact = t @ w2f.T + oracle.bf16_bits_to_f32(b2)
    # The reference algorithm itself is ~6% max-rel from exact math here: the
    # FWHT folds the GELU output's positive mean into one coefficient per
    # 4096-block, which then sets the per-token int8 scale of fc2's input.
    # The GPU must be as close to exact math as the oracle chain is.
    y_chain = oracle.linear_w8a8(h_ref, w2q, w2s, 4096, b2)
    rel_o, cos_o = _metrics(y_chain, exact)
    rel, cos = _metrics(y_got, exact)
    assert rel <= rel_o * 1.05 + 1e-3 and cos >= cos_o - 1e-4, (rel, cos, rel_o, cos_o)
    assert cos_o >= 0.99


def test_dequantize_and_bias_matches_oracle_and_fused(qimg, oracle):
    """The stand-alone epilogue (dequantize_and_bias / dequantize_bias_gelu)
    on an oracle int32 product: bit-exact without GELU, and identical to the
    fused GEMM epilogue with GELU."""
    rng = np.random.default_rng(31)
    M, N, K = 200, 264, 3072
    x = rng.standard_normal((M, K)).astype(np.float32)
    w_bits = oracle.bf16_bits_from_f32((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    b_bits = oracle.bf16_bits_from_f32((rng.standard_normal(N) * 0.01).astype(np.float32))
    wq, ws, hbs = oracle.quantize_weight_bf16(w_bits)
    q, s = oracle.quantize_activation(x, hbs)
    c = oracle.gemm_s8s8s32(q, wq)
    got = qimg.dequantize_and_bias(_dev(c), _dev(s), _dev(ws), _bf16_dev(b_bits))
    got_g = qimg.dequantize_and_bias(_dev(c), _dev(s), _dev(ws), _bf16_dev(b_bits), apply_gelu=True)
    fused_g = qimg.linear_forward_prequantized(_dev(q), _dev(s), _qw(qimg, wq, ws, hbs), _bf16_dev(b_bits),
                                               apply_gelu=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.cpu().numpy(), oracle.dequant_epilogue(c, s, ws, b_bits))
    np.testing.assert_array_equal(got_g.cpu().numpy(), fused_g.cpu().numpy())
    np.testing.assert_allclose(got_g.cpu().numpy(), oracle.dequant_epilogue(c, s, ws, b_bits, gelu=True),
                               rtol=2e-6, atol=2e-6)


@pytest.mark.parametrize("M,N,K", [(4100, 3076, 1024), (600, 518, 512), (777, 1000, 256), (513, 264, 3072)])
@pytest.mark.parametrize("kernel", ["large", "w192", "w224", "t128"])
def test_large_tile_epilogue_edges(qimg, oracle, M, N, K, kernel):
    """The 256-row tiles' int8 epilogue (256, 224 and 192 columns) on ragged
    tiles: rows past M, N % 4 = 2 (element stores), N % 8 = 4 (bf16
    half-chunk stores), N % 8 = 0, and last tiles of 4, 40, 72 and 134
    columns (192 wide) or 164, 70, 104 and 40 (224 wide). fp32 out bit-exact against the oracle's dequant of the int32
    product, bf16 out its RNE rounding, GELU identical to the stand-alone
    epilogue kernel."""
    rng = np.random.default_rng(M + 5 * N + K)
    a = rng.integers(-128, 128, (M, K), dtype=np.int8)
    w = rng.integers(-128, 128, (N, K), dtype=np.int8)
    s = (rng.random(M) * 1e-3 + 1e-5).astype(np.float32)
    ws = (rng.random(N) * 1e-3 + 1e-5).astype(np.float32)
    b_bits = oracle.bf16_bits_from_f32((rng.standard_normal(N) * 0.01).astype(np.float32))
    c = oracle.gemm_s8s8s32(a, w)
    ref = oracle.dequant_epilogue(c, s, ws, b_bits)
    qw = _qw(qimg, w, ws, 1)
    ad, sd, bd = _dev(a), _dev(s), _bf16_dev(b_bits)
    with qimg.linear_kernel(KERNELS[kernel]):
        o32 = qimg.linear_forward_prequantized(ad, sd, qw, bd)
        o16 = qimg.linear_forward_prequantized(ad, sd, qw, bd, out_dtype=torch.bfloat16)
        og = qimg.linear_forward_prequantized(ad, sd, qw, bd, apply_gelu=True)
    sep_g = qimg.dequantize_and_bias(_dev(c), sd, _dev(ws), bd, apply_gelu=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(o32.cpu().numpy(), ref)
    np.testing.assert_array_equal(o16.float().cpu().numpy(),
                                  oracle.bf16_bits_to_f32(oracle.bf16_bits_from_f32(ref)).reshape(M, N))
    assert torch.equal(og, sep_g)


@pytest.mark.parametrize("M", [33, 129, 257, 1000, 1024, 2049, 4095, 4352, 6889])
@pytest.mark.parametrize("N", [1000, 3072, 12288])
def test_int8_auto_dispatch_exact(qimg, M, N):
    """The automatic choice over M and N around the dispatcher's
    boundaries (the 64x64 small tiles, 128x128 tiles from 128 rows and 32
    tiles of 256x256, 256-row tiles 192, 224 or 256 wide, the trailing tile
    rows split off to 128x128 tiles): every row of a sample is the exact
    int32 product, fp32 out, and bf16 out its rounding."""
    K = 256
    rng = np.random.default_rng(M * 7 + N)
    a = rng.integers(-128, 128, (M, K), dtype=np.int8)
    w = rng.integers(-128, 128, (N, K), dtype=np.int8)
    ones_m = np.ones(M, np.float32)
    qw = _qw(qimg, w, np.ones(N, np.float32), 1)
    ad, sd = _dev(a), _dev(ones_m)
    o32 = qimg.linear_forward_prequantized(ad, sd, qw)
    o16 = qimg.linear_forward_prequantized(ad, sd, qw, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    idx = np.unique(np.concatenate([[0, M - 1], np.arange(0, M, max(1, M // 16)), rng.integers(0, M, 24),
                                    np.arange(max(0, M - 300), M, 37)]))
    ref = (a[idx].astype(np.int64) @ w.astype(np.int64).T).astype(np.float32)
    np.testing.assert_array_equal(o32.cpu().numpy()[idx], ref)
    np.testing.assert_array_equal(o16.float().cpu().numpy()[idx], torch.from_numpy(ref).bfloat16().float().numpy())


@pytest.mark.parametrize("M,N,K", [(3328, 2560, 128), (3328, 2560, 320), (4352, 3072, 1024)])
def test_int8_gemm_partial_round_shapes_exact(qimg, oracle, M, N, K):
    """Tile counts that do not fill whole rounds of the 256 CUs (130 and 204
    tiles), with short and long K: exact, and identical on repeated calls."""
    rng = np.random.default_rng(M + N + K)
    a = rng.integers(-128, 128, (M, K), dtype=np.int8)
    w = rng.integers(-128, 128, (N, K), dtype=np.int8)
    qw = _qw(qimg, w, np.ones(N, np.float32), 1)
    ad, ones_m = _dev(a), _dev(np.ones(M, np.float32))
    out1 = qimg.linear_forward_prequantized(ad, ones_m, qw)
    out2 = qimg.linear_forward_prequantized(ad, ones_m, qw)
    torch.cuda.synchronize()
    assert torch.equal(out1, out2)
    idx = np.unique(np.concatenate([[0, M - 1], np.arange(0, M, 97), rng.integers(0, M, 40)]))
    ref = (a[idx].astype(np.int64) @ w.astype(np.int64).T).astype(np.float32)
    np.testing.assert_array_equal(out1.cpu().numpy()[idx], ref)


@pytest.mark.parametrize("M,N,K", [(1, 18432, 3072), (1, 3072, 256), (2, 18432, 3072), (3, 1000, 1088),
                                   (4, 3072, 12288), (17, 3072, 3072), (256, 3072, 3072), (256, 12288, 3072),
                                   (256, 3072, 12288)])
def test_small_m_shapes_exact(qimg, oracle, M, N, K):
    """The step-level and text-stream shapes: modulation (M = 1 or 2 CFG rows,
    N = 18432), the timestep MLP (K = 256), text linears (M = 256). The int32
    product is exact against float64 (|acc| < 2^53) under the automatic
    choice and under the large-tile kernel."""
    rng = np.random.default_rng(M * 7 + N + K)
    a = rng.integers(-128, 128, (M, K), dtype=np.int8)
    w = rng.integers(-128, 128, (N, K), dtype=np.int8)
    ref = (a.astype(np.float64) @ w.astype(np.float64).T).astype(np.float32)
    ad, wd = _dev(a), _qw(qimg, w, np.ones(N, np.float32), 1)
    sd = _dev(np.ones(M, np.float32))
    got_auto = qimg.linear_forward_prequantized(ad, sd, wd)
    with qimg.linear_kernel(qimg.LINEAR_LARGE_TILE):
        got_large = qimg.linear_forward_prequantized(ad, sd, wd)
    with qimg.linear_kernel(qimg.LINEAR_SMALL_32):
        got_s32 = qimg.linear_forward_prequantized(ad, sd, wd)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got_auto.cpu().numpy(), ref)
    np.testing.assert_array_equal(got_large.cpu().numpy(), ref)
    np.testing.assert_array_equal(got_s32.cpu().numpy(), ref)


@pytest.mark.parametrize("M,N,K,gelu", [(1, 18432, 3072, False), (1, 3072, 256, True), (2, 3000, 3072, True),
                                        (256, 3072, 3072, False),
                                        (256, 12288, 3072, True), (40, 200, 12288, False)])
def test_small_m_linear_matches_oracle(qimg, oracle, M, N, K, gelu):
    """Full linear (activation FWHT + quant, GEMM, dequant epilogue) at the
    small-M shapes: fp32 out bit-exact against the oracle without GELU and
    within 2e-6 with it; bf16 out is the RNE rounding of the fp32 out."""
    rng = np.random.default_rng(M + N * 3 + K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w_bits = oracle.bf16_bits_from_f32((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    b_bits = oracle.bf16_bits_from_f32((rng.standard_normal(N) * 0.01).astype(np.float32))
    wq, ws, hbs = oracle.quantize_weight_bf16(w_bits)
    ref = oracle.linear_w8a8(x, wq, ws, hbs, b_bits, gelu=gelu)
    qw = _qw(qimg, wq, ws, hbs)
    out = qimg.linear_forward_quantized(_dev(x), qw, _bf16_dev(b_bits), apply_gelu=gelu)
    o16 = qimg.linear_forward_quantized(_dev(x), qw, _bf16_dev(b_bits), apply_gelu=gelu, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    if gelu:
        np.testing.assert_allclose(got, ref, rtol=2e-6, atol=2e-6)
    else:
        np.testing.assert_array_equal(got, ref)
    np.testing.assert_array_equal(o16.float().cpu().numpy(),
                                  oracle.bf16_bits_to_f32(oracle.bf16_bits_from_f32(got)).reshape(M, N))


@pytest.mark.parametrize("M,N,K", [(1, 18432, 3072), (2, 5000, 12288), (3, 1000, 3072), (4, 130, 1024),
                                   (256, 3072, 3072), (9, 100, 12288)])
def test_small_m_fp8(qimg, oracle, M, N, K):
    """e4m3 at small M (M <= 4: the vector-ALU GEMV, fp32 FMAs of the
    widened bytes; longer K in two alternating register sets): the oracle's
    float64 sum of the exact e4m3 products, within the fp32
    accumulation-order bound; the small and large kernels agree to the
    same bound."""
    rng = np.random.default_rng(M + N + K + 5)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w_bits = oracle.bf16_bits_from_f32((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    b_bits = oracle.bf16_bits_from_f32((rng.standard_normal(N) * 0.01).astype(np.float32))
    wq, ws, hbs = oracle.quantize_weight_fp8(w_bits)
    xq, xs = oracle.quantize_activation_fp8(x, hbs)
    ref = oracle.gemm_fp8_epilogue(xq, wq, xs, ws, b_bits, rows=(0, M))
    qw = _qw(qimg, wq, ws, hbs, mode=qimg.FP8_HADAMARD)
    got = qimg.linear_forward_quantized(_dev(x), qw, _bf16_dev(b_bits))
    got_h = qimg.linear_forward_quantized(_dev(x), qw, _bf16_dev(b_bits), out_dtype=torch.bfloat16)
    got_g = qimg.linear_forward_quantized(_dev(x), qw, _bf16_dev(b_bits), apply_gelu=True)
    with qimg.linear_kernel(qimg.LINEAR_LARGE_TILE):
        got_l = qimg.linear_forward_quantized(_dev(x), qw, _bf16_dev(b_bits))
    torch.cuda.synchronize()
    bound = 1e-5 * np.abs(ref).max() * np.sqrt(K / 64)
    assert np.max(np.abs(got.cpu().numpy() - ref)) <= bound
    assert np.max(np.abs(got_l.cpu().numpy() - ref)) <= bound
    # bf16 out within the bound plus half a bf16 ulp; GELU within the bound
    # through GELU's slope plus the approximation's error
    assert np.all(np.abs(got_h.float().cpu().numpy() - ref) <= np.abs(ref) * 2.0 ** -8 + 1.01 * bound)
    ref_g = oracle.gemm_fp8_epilogue(xq, wq, xs, ws, b_bits, gelu=True, rows=(0, M))
    assert np.max(np.abs(got_g.cpu().numpy() - ref_g)) <= 1.13 * bound + 2e-6 * np.abs(ref_g).max()


@pytest.mark.parametrize("M,N,K", [(4352, 12288, 3072), (4400, 12288, 1024), (4352, 12288, 256)])
def test_tail_round_split_exact(qimg, oracle, M, N, K):
    """When the last round of 256x256 tiles would be mostly idle, the automatic
    choice runs the trailing tile rows on the 64x64 kernel (here rows 4096..M).
    The result is identical to the all-large-tile run and exact on sampled
    rows from both parts (including the ragged end of M)."""
    rng = np.random.default_rng(M + N + K)
    a = rng.integers(-128, 128, (M, K), dtype=np.int8)
    w = rng.integers(-128, 128, (N, K), dtype=np.int8)
    sa = (rng.random(M) * 0.01 + 1e-3).astype(np.float32)
    sw = (rng.random(N) * 0.01 + 1e-3).astype(np.float32)
    b_bits = oracle.bf16_bits_from_f32((rng.standard_normal(N) * 0.01).astype(np.float32))
    ad, qw, bd, sd = _dev(a), _qw(qimg, w, sw, 1), _bf16_dev(b_bits), _dev(sa)
    got = qimg.linear_forward_prequantized(ad, sd, qw, bd, apply_gelu=True)
    with qimg.linear_kernel(qimg.LINEAR_LARGE_TILE):
        big = qimg.linear_forward_prequantized(ad, sd, qw, bd, apply_gelu=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.cpu().numpy(), big.cpu().numpy())
    idx = np.unique(np.concatenate([[0, 4095, 4096, M - 1], rng.integers(0, M, 12)]))
    c = (a[idx].astype(np.float64) @ w.astype(np.float64).T).astype(np.int32)
    ref = oracle.dequant_epilogue(c, sa[idx], sw, b_bits, gelu=True)
    np.testing.assert_allclose(got.cpu().numpy()[idx], ref, rtol=2e-6, atol=2e-6)
