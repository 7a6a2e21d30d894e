"""GPU parity of the INT4 paths (cuda_kernels.cu:2864-4532) through the C ABI.

Integer, byte and layout work is bit-exact against the oracle: dequantized
bf16 weights, INT4 weight codes and scales (NF4 and linear), INT4
activation codes, scales and bf16 copies, the W4A4 GEMM (its per-group fp32
order is the reference's, so every tiling gives the oracle's bits), the AWQ
repack, dequant and GEMV, and the nunchaku / LoRA conversions.

The composite INT4 linear (low-rank branch through bf16 GEMMs whose fp32
summation order is cuBLAS's, not the reference's source) is held to the
oracle's composite within 1e-3 of the output scale, and to float64 math of
the same quantized operands at the stated bar (max-rel 2e-2, cos 0.999).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _u8(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.uint8)).to(DEV)


def _f32(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(DEV)


def _bf16_bits_dev(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(DEV).view(torch.bfloat16)


def _bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("N,K,gs", [(3072, 3072, 64), (24, 136, 8), (7, 256, 128)])
@pytest.mark.parametrize("form", ["nf4", "linear", "signed_gn"])
def test_dequant_int4_bit_exact(qimg, oracle, N, K, gs, form):
    rng = np.random.default_rng(N + K + gs + len(form))
    qw = rng.integers(0, 256, (N, K // 2)).astype(np.uint8)
    gn = form == "signed_gn"
    sc = rng.uniform(0.001, 2, (K // gs, N) if gn else (N, K // gs)).astype(np.float32)
    nf4, signed = form == "nf4", form == "signed_gn"
    got = qimg.dequantize_int4_to_bf16(_u8(qw), _f32(sc), K, gs, nf4_grid=nf4, scales_gn=gn, signed_int4=signed)
    torch.cuda.synchronize()
    want = oracle.dequant_int4_bf16(qw, sc, K, gs, nf4=nf4, scales_gn=gn, signed_int4=signed)
    np.testing.assert_array_equal(_bits(got), want)


@pytest.mark.parametrize("N,K,gs", [(3072, 3072, 64), (64, 256, 128), (5, 64, 32), (3, 96, 6)])
@pytest.mark.parametrize("nf4", [True, False])
def test_quantize_int4_weight_bit_exact(qimg, oracle, N, K, gs, nf4):
    rng = np.random.default_rng(N * 3 + K + nf4)
    r = (rng.standard_normal((N, K)) * rng.uniform(0.001, 0.1, (N, 1))).astype(np.float32)
    r[0, :gs] = 0.0
    r[-1, 1] = 7.0 * 2.5 / 7.0  # a value on a rounding boundary of its group
    qw, sc = qimg.quantize_int4_per_group(_f32(r), gs, nf4_grid=nf4)
    torch.cuda.synchronize()
    qw_ref, sc_ref = oracle.quant_int4_weight(r, gs, nf4=nf4)
    np.testing.assert_array_equal(sc.cpu().numpy(), sc_ref)
    np.testing.assert_array_equal(qw.cpu().numpy(), qw_ref)


@pytest.mark.parametrize("M,K,gs", [(4096, 3072, 64), (37, 3072, 128), (3, 64, 32), (1, 128, 64)])
@pytest.mark.parametrize("smooth", [False, True])
def test_quantize_activation_int4_bit_exact(qimg, oracle, M, K, gs, smooth):
    rng = np.random.default_rng(M + K + gs + smooth)
    x = (rng.standard_normal((M, K)) * rng.uniform(0.1, 5, (M, 1))).astype(np.float32)
    x[0, :gs] = 0.0
    sm = rng.uniform(0.25, 4, K).astype(np.float32) if smooth else None
    if smooth:
        pk, sc, bf = qimg.quantize_activation_int4(_f32(x), gs, smooth=_f32(sm), want_bf16=True)
        pk_r, sc_r, bf_r = oracle.quant_act_int4(x, gs, smooth=sm, want_bf16=True)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_bits(bf), bf_r)
    else:
        pk, sc = qimg.quantize_activation_int4(_f32(x), gs)
        pk_r, sc_r = oracle.quant_act_int4(x, gs)
        torch.cuda.synchronize()
    np.testing.assert_array_equal(sc.cpu().numpy(), sc_r)
    np.testing.assert_array_equal(pk.cpu().numpy(), pk_r)


def _rows(M, rng, k=24):
    return np.unique(np.concatenate([[0, M - 1], rng.integers(0, M, k)]))


@pytest.mark.parametrize("M,N,K,gs", [(4096, 3072, 3072, 64), (100, 200, 128, 64), (33, 130, 256, 128),
                                      (1, 64, 64, 64)])
@pytest.mark.parametrize("accumulate", [False, True])
def test_w4a4_gemm_bit_exact(qimg, oracle, M, N, K, gs, accumulate):
    rng = np.random.default_rng(M + N + K + accumulate)
    ap = rng.integers(0, 256, (M, K // 2)).astype(np.uint8)
    wp = rng.integers(0, 256, (N, K // 2)).astype(np.uint8)
    asc = rng.uniform(0.001, 0.5, (K // gs, M)).astype(np.float32)
    wsc = rng.uniform(0.001, 0.05, (K // gs, N)).astype(np.float32)
    bias = oracle.bf16_bits_from_f32(rng.standard_normal(N).astype(np.float32) * 0.1)
    base = rng.standard_normal((M, N)).astype(np.float32)
    out = _f32(base) if accumulate else None
    got = qimg.w4a4_gemm(_u8(ap), _u8(wp), _f32(asc), _f32(wsc), K, gs, bias=_bf16_bits_dev(bias), out=out,
                         accumulate=accumulate)
    torch.cuda.synchronize()
    idx = _rows(M, rng)
    g = got.cpu().numpy()
    for m in idx:
        want = oracle.w4a4_gemm(ap, wp, asc, wsc, K, gs, bias_bits=bias,
                                out=base[m:m + 1] if accumulate else None, rows=(int(m), int(m) + 1))
        np.testing.assert_array_equal(g[m:m + 1], want)


def test_awq_paths_bit_exact(qimg, oracle):
    rng = np.random.default_rng(2)
    OC, IC, gs, nc = 18432, 3072, 64, 6   # the modulation layer (6 x 3072 outputs)
    qw = rng.integers(-2 ** 31, 2 ** 31, (OC // 4, IC // 2), dtype=np.int64).astype(np.int32)
    ws = oracle.bf16_bits_from_f32(rng.uniform(0.001, 0.02, (IC // gs, OC)).astype(np.float32))
    wz = oracle.bf16_bits_from_f32(rng.uniform(-0.1, 0.1, (IC // gs, OC)).astype(np.float32))
    b = oracle.bf16_bits_from_f32(rng.standard_normal(OC).astype(np.float32) * 0.01)
    x = rng.standard_normal(IC).astype(np.float32)
    qw_d = torch.from_numpy(qw).to(DEV)
    rep = qimg.repack_awq_to_transposed(qw_d, OC, IC)
    torch.cuda.synchronize()
    rep_r = oracle.awq_repack(qw, OC, IC)
    np.testing.assert_array_equal(rep.cpu().numpy(), rep_r)
    out = qimg.linear_forward_awq(_f32(x), rep, _bf16_bits_dev(ws), _bf16_bits_dev(wz), OC, IC,
                                  bias=_bf16_bits_dev(b), group_size=gs, num_components=nc)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy()[0], oracle.awq_gemv(x, rep_r, ws, wz, OC, IC, gs, nc, bias_bits=b))
    OCs, ICs = 96, 256
    deq = qimg.dequantize_awq_to_bf16(qw_d[:OCs // 4, :ICs // 2].contiguous(), _bf16_bits_dev(ws[:ICs // gs, :OCs]),
                                      _bf16_bits_dev(wz[:ICs // gs, :OCs]), OCs, ICs, gs, nc)
    torch.cuda.synchronize()
    want = oracle.dequant_awq_bf16(np.ascontiguousarray(qw[:OCs // 4, :ICs // 2]), ws[:ICs // gs, :OCs],
                                   wz[:ICs // gs, :OCs], OCs, ICs, gs, nc)
    np.testing.assert_array_equal(_bits(deq), want)


@pytest.mark.parametrize("N,K,G", [(3072, 3072, 48), (128, 256, 2)])
def test_nunchaku_conversions_bit_exact(qimg, oracle, N, K, G):
    rng = np.random.default_rng(N + G)
    q_sw = rng.integers(0, 256, N * K // 2).astype(np.uint8)
    s_sw = oracle.bf16_bits_from_f32(rng.uniform(0.001, 0.1, N * G).astype(np.float32))
    q, s = qimg.unswizzle_nunchaku_weights(_u8(q_sw), _bf16_bits_dev(s_sw), N, K, G)
    deq = qimg.dequantize_nunchaku_to_bf16(_u8(q_sw), _bf16_bits_dev(s_sw), N, K, G)
    torch.cuda.synchronize()
    q_r, s_r = oracle.unswizzle_nunchaku(q_sw, s_sw, N, K, G)
    np.testing.assert_array_equal(q.cpu().numpy(), q_r)
    np.testing.assert_array_equal(s.cpu().numpy(), s_r)
    np.testing.assert_array_equal(_bits(deq), oracle.dequant_nunchaku_bf16(q_sw, s_sw, N, K, G))


@pytest.mark.parametrize("rows,cols,is_down", [(3072, 32, True), (3072, 32, False), (48, 64, True)])
def test_lora_unswizzle_bit_exact(qimg, oracle, rows, cols, is_down):
    rng = np.random.default_rng(rows + cols + is_down)
    packed = rng.integers(0, 2 ** 16, rows * cols).astype(np.uint16)
    got = qimg.unswizzle_lora_weights(_bf16_bits_dev(packed), rows, cols, is_down)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(got), oracle.unswizzle_lora(packed, rows, cols, is_down))


def _int4_case(oracle, rng, M, N, K, r, gs, w4a4, smooth, nf4=True, hbs=1):
    x = rng.standard_normal((M, K)).astype(np.float32)
    resid = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    down = oracle.bf16_bits_from_f32((rng.standard_normal((K, r)) * 0.05).astype(np.float32)) if r else None
    up = oracle.bf16_bits_from_f32((rng.standard_normal((N, r)) * 0.05).astype(np.float32)) if r else None
    sm = rng.uniform(0.5, 2, K).astype(np.float32) if smooth else None
    bias = oracle.bf16_bits_from_f32(rng.standard_normal(N).astype(np.float32) * 0.01)
    case = dict(x=x, down=down, up=up, sm=sm, bias=bias)
    if w4a4:
        q = rng.integers(-7, 8, (N, K))
        case["wp"] = ((q[:, 0::2] & 0xF) | ((q[:, 1::2] & 0xF) << 4)).astype(np.uint8)
        case["ws"] = rng.uniform(0.001, 0.01, (K // gs, N)).astype(np.float32)
    else:
        case["qw"], case["s4"] = oracle.quant_int4_weight(resid, gs, nf4=nf4)
    return case


def _int4_oracle(oracle, c, rows, N, K, r, gs, w4a4, nf4, hbs, gelu):
    """The reference's linear_forward_int4 composed from oracle parts on the
    given rows; the bf16 GEMMs as float64 sums rounded to fp32 (their
    accumulation order is cuBLAS's)."""
    x = c["x"][rows]
    v = x / c["sm"] if c["sm"] is not None else x
    v = v.astype(np.float32)
    xs = oracle.bf16_bits_to_f32(oracle.bf16_bits_from_f32(v)).reshape(v.shape).astype(np.float64)
    lora = np.zeros((len(rows), N))
    lora_exact = np.zeros((len(rows), N))
    if r:
        down = oracle.bf16_bits_to_f32(c["down"]).reshape(K, r).astype(np.float64)
        up = oracle.bf16_bits_to_f32(c["up"]).reshape(N, r).astype(np.float64)
        lr = (xs @ down).astype(np.float32)
        lr16 = oracle.bf16_bits_to_f32(oracle.bf16_bits_from_f32(lr)).reshape(lr.shape).astype(np.float64)
        lora = (lr16 @ up.T).astype(np.float32)
        lora_exact = (xs @ down) @ up.T
    b = oracle.bf16_bits_to_f32(c["bias"]).astype(np.float64)
    if w4a4:
        pk, sc = oracle.quant_act_int4(v, gs)
        res = oracle.w4a4_gemm(pk, c["wp"], sc, c["ws"], K, gs).astype(np.float64)
        # float64 of the same quantized operands
        qa = pk
        a_n = np.empty((len(rows), K), np.int64)
        a_n[:, 0::2] = qa & 0xF
        a_n[:, 1::2] = qa >> 4
        a_n = np.where(a_n >= 8, a_n - 16, a_n)
        w_n = np.empty((N, K), np.int64)
        w_n[:, 0::2] = c["wp"] & 0xF
        w_n[:, 1::2] = c["wp"] >> 4
        w_n = np.where(w_n >= 8, w_n - 16, w_n)
        G = K // gs
        d = np.einsum("mgk,ngk->gmn", a_n.reshape(-1, G, gs), w_n.reshape(N, G, gs)).astype(np.float64)
        res_exact = np.einsum("gmn,gm,gn->mn", d, sc.astype(np.float64), c["ws"].astype(np.float64))
        want = lora.astype(np.float64) + (res.astype(np.float32) + b.astype(np.float32)).astype(np.float64)
    else:
        xr = v.copy()
        if hbs > 1:
            xr = oracle.fwht_rows(xr, hbs)
        xr16 = oracle.bf16_bits_to_f32(oracle.bf16_bits_from_f32(xr)).reshape(xr.shape).astype(np.float64)
        deq = oracle.dequant_int4_bf16(c["qw"], c["s4"], K, gs, nf4=nf4)
        w = oracle.bf16_bits_to_f32(deq).reshape(N, K).astype(np.float64)
        res = xr16 @ w.T
        res_exact = res
        want = lora.astype(np.float64) + res + b
    exact = lora_exact + res_exact + b
    if gelu:
        want = oracle.gelu_tanh64(want)
        exact = oracle.gelu_tanh64(exact)
    return want, exact


@pytest.mark.parametrize("M,N,K,r,gs,w4a4,smooth,nf4,hbs,gelu", [
    (256, 3072, 3072, 32, 64, False, False, True, 1024, False),   # W4A16, NF4, Hadamard
    (4096, 3072, 3072, 32, 64, False, True, True, 1024, True),    # W4A16 at 4096 tokens (large-tile residual)
    (300, 3072, 3072, 32, 64, False, True, False, 1024, True),    # linear INT4, smooth + Hadamard, GELU
    (64, 512, 1024, 16, 128, False, True, True, 1, False),        # smooth only
    (256, 3072, 3072, 32, 64, True, True, True, 1, False),        # W4A4 (nunchaku form)
    (40, 256, 512, 32, 128, True, False, True, 1, True),          # W4A4, GELU
    (17, 128, 256, 0, 64, False, False, True, 256, False),        # no low-rank factor
])
def test_linear_int4(qimg, oracle, M, N, K, r, gs, w4a4, smooth, nf4, hbs, gelu):
    rng = np.random.default_rng(M + N + K + r + gs + w4a4 + smooth)
    c = _int4_case(oracle, rng, M, N, K, r, gs, w4a4, smooth, nf4, hbs)
    dev = lambda a: None if a is None else _f32(a)
    bdev = lambda a: None if a is None else _bf16_bits_dev(a)
    w = qimg.Int4Weight(N, K, gs, svd_up=bdev(c["up"]), svd_down=bdev(c["down"]),
                        qweight=None if w4a4 else _u8(c["qw"]), scales4=None if w4a4 else _f32(c["s4"]),
                        nf4_grid=nf4, had_block_size=hbs, w4a4_qweight=_u8(c["wp"]) if w4a4 else None,
                        w4a4_wscales=_f32(c["ws"]) if w4a4 else None, smooth=dev(c["sm"]))
    out = qimg.linear_forward_int4(_f32(c["x"]), w, bias=_bf16_bits_dev(c["bias"]), apply_gelu=gelu)
    torch.cuda.synchronize()
    rows = _rows(M, rng, 16)
    got = out.cpu().numpy()[rows].astype(np.float64)
    assert np.isfinite(got).all()
    want, exact = _int4_oracle(oracle, c, rows, N, K, r, gs, w4a4, nf4, hbs, gelu)
    assert np.max(np.abs(got - want)) <= 1e-3 * np.max(np.abs(want)) + 1e-6, np.max(np.abs(got - want))
    a, e = got.ravel(), exact.ravel()
    rel = np.max(np.abs(a - e)) / np.max(np.abs(e))
    cos = float(a @ e / (np.linalg.norm(a) * np.linalg.norm(e)))
    assert rel <= 2e-2 and cos >= 0.999, (rel, cos)


@pytest.mark.parametrize("M,N,K,r,gs,smooth,gelu", [
    (256, 3072, 3072, 32, 64, True, False),   # the W4A4 case's nunchaku weights through W4A16
    (40, 256, 512, 16, 128, False, True),
])
def test_linear_int4_nunchaku_w4a16(qimg, oracle, M, N, K, r, gs, smooth, gelu):
    """The reference's W4A16 fallback for nunchaku weights
    (cuda_kernels.cu:4443-4470): the row-major two's complement nibbles and
    [K/gs, N] scales dequantized to bf16 (signed, scales_gn), times bf16 of
    the smoothed x with no rotation, onto the low-rank product, then the
    bias and GELU."""
    rng = np.random.default_rng(7 * M + N + K + r + gs + smooth)
    c = _int4_case(oracle, rng, M, N, K, r, gs, True, smooth)
    dev = lambda a: None if a is None else _f32(a)
    bdev = lambda a: None if a is None else _bf16_bits_dev(a)
    w = qimg.Int4Weight(N, K, gs, svd_up=bdev(c["up"]), svd_down=bdev(c["down"]), qweight=_u8(c["wp"]),
                        scales4=_f32(c["ws"]), had_block_size=1024, nf4_grid=True, smooth=dev(c["sm"]),
                        w4a16_nunchaku=True)
    out = qimg.linear_forward_int4(_f32(c["x"]), w, bias=_bf16_bits_dev(c["bias"]), apply_gelu=gelu)
    torch.cuda.synchronize()
    rows = _rows(M, rng, 16)
    got = out.cpu().numpy()[rows].astype(np.float64)
    assert np.isfinite(got).all()
    # the oracle's W4A16 composite with the nunchaku dequantization
    x = c["x"][rows]
    v = (x / c["sm"] if c["sm"] is not None else x).astype(np.float32)
    xs = oracle.bf16_bits_to_f32(oracle.bf16_bits_from_f32(v)).reshape(v.shape).astype(np.float64)
    lora = np.zeros((len(rows), N))
    if r:
        down = oracle.bf16_bits_to_f32(c["down"]).reshape(K, r).astype(np.float64)
        up = oracle.bf16_bits_to_f32(c["up"]).reshape(N, r).astype(np.float64)
        lr = (xs @ down).astype(np.float32)
        lr16 = oracle.bf16_bits_to_f32(oracle.bf16_bits_from_f32(lr)).reshape(lr.shape).astype(np.float64)
        lora = (lr16 @ up.T).astype(np.float32)
    deq = oracle.dequant_int4_bf16(c["wp"], c["ws"], K, gs, nf4=False, scales_gn=True, signed_int4=True)
    wd = oracle.bf16_bits_to_f32(deq).reshape(N, K).astype(np.float64)
    want = lora.astype(np.float64) + xs @ wd.T + oracle.bf16_bits_to_f32(c["bias"]).astype(np.float64)
    if gelu:
        want = oracle.gelu_tanh64(want)
    assert np.max(np.abs(got - want)) <= 1e-3 * np.max(np.abs(want)) + 1e-6, np.max(np.abs(got - want))
    # and not the W4A4 result on the same weights (activations kept in bf16)
    w4 = qimg.Int4Weight(N, K, gs, svd_up=bdev(c["up"]), svd_down=bdev(c["down"]), w4a4_qweight=_u8(c["wp"]),
                         w4a4_wscales=_f32(c["ws"]), smooth=dev(c["sm"]))
    out4 = qimg.linear_forward_int4(_f32(c["x"]), w4, bias=_bf16_bits_dev(c["bias"]), apply_gelu=gelu)
    torch.cuda.synchronize()
    assert not torch.equal(out, out4)


def test_linear_int4_rejects_bad_arguments(qimg):
    x = torch.zeros(4, 128, device=DEV)
    w = qimg.Int4Weight(64, 128, 64)  # neither residual form
    with pytest.raises(qimg.QimgError):
        qimg.linear_forward_int4(x, w)
    q = torch.zeros(64, 64, dtype=torch.uint8, device=DEV)
    s = torch.zeros(2, 64, device=DEV)
    w = qimg.Int4Weight(64, 128, 96, w4a4_qweight=q, w4a4_wscales=s)  # W4A4 group size 96
    with pytest.raises(qimg.QimgError):
        qimg.linear_forward_int4(x, w)
    L = qimg.lib()
    scratch = torch.zeros(16, dtype=torch.uint8, device=DEV)
    st = qimg.Int4Weight(64, 128, 64, w4a4_qweight=q, w4a4_wscales=s).struct()
    import ctypes
    assert L.qimg_linear_int4(qimg._ptr(x), 4, ctypes.byref(st), None, qimg._ptr(x), 0, qimg._ptr(scratch), 16,
                              None) == 3  # scratch too small
