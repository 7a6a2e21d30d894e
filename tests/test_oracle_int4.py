"""Pins of the INT4 oracle (oracle/qimg_oracle_int4.c, cuda_kernels.cu:
2864-4532) by checks that do not restate its formulas:

* dequantization against numpy/torch conversions of each code, including
  all 16 codes of every form;
* the quantizers by their defining properties: the group's absmax element
  maps to the extreme code, every value lands within half a step (linear)
  or on the nearest grid point in float64 (NF4), half-way values round away
  from zero (CUDA roundf);
* the W4A4 GEMM against int64 brute-force dot products and float64 sums,
  exactly where every fp32 operation is exact (power-of-two scales);
* the AWQ GEMV against float64 dot products, exactly on small integers;
* the layout conversions (AWQ repack/dequant, nunchaku weights and
  scales, LoRA factors) as permutations: every source element is reached
  exactly once, and the two reference routes to the same dequantized
  weight (direct nunchaku dequant; unswizzle then dequant) agree.
"""
import numpy as np
import pytest
import torch


def _bf16(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def _pack(nib):
    nib = np.asarray(nib, np.uint8)
    return (nib[:, 0::2] & 0xF) | ((nib[:, 1::2] & 0xF) << 4)


def _unpack(p):
    p = np.asarray(p, np.uint8)
    out = np.empty((p.shape[0], p.shape[1] * 2), np.uint8)
    out[:, 0::2] = p & 0xF
    out[:, 1::2] = p >> 4
    return out


def _signed(n):
    n = np.asarray(n, np.int64)
    return np.where(n >= 8, n - 16, n)


def test_nf4_grid_is_sorted_symmetric_endpoints(oracle):
    g = oracle.NF4_GRID.astype(np.float64)
    assert np.all(np.diff(g) > 0) and g[0] == -1.0 and g[7] == 0.0 and g[15] == 1.0


@pytest.mark.parametrize("nf4,signed_int4,gn", [(True, False, False), (False, False, False), (False, True, True),
                                                (True, False, True)])
def test_dequant_int4_every_code(oracle, nf4, signed_int4, gn):
    rng = np.random.default_rng(int(nf4) * 4 + int(signed_int4) * 2 + int(gn))
    N, K, gs = 8, 64, 32
    codes = np.tile(np.arange(16, dtype=np.uint8), (N, K // 16))
    rng.shuffle(codes, axis=1)
    scales = rng.uniform(0.01, 3, (N, K // gs)).astype(np.float32)
    sc_arg = np.ascontiguousarray(scales.T) if gn else scales
    got = oracle.dequant_int4_bf16(_pack(codes), sc_arg, K, gs, nf4=nf4, scales_gn=gn, signed_int4=signed_int4)
    if nf4:
        vals = oracle.NF4_GRID[codes]
    elif signed_int4:
        vals = _signed(codes).astype(np.float32)
    else:
        vals = codes.astype(np.float32) - 8
    want = _bf16(vals * np.repeat(scales, gs, axis=1))
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("nf4", [True, False])
def test_weight_quant_properties(oracle, nf4):
    rng = np.random.default_rng(11 + nf4)
    N, K, gs = 16, 256, 64
    r = (rng.standard_normal((N, K)) * rng.uniform(0.01, 2, (N, 1))).astype(np.float32)
    r[3, 64:128] = 0.0  # an all-zero group: scale 0, the zero code
    qw, sc = oracle.quant_int4_weight(r, gs, nf4=nf4)
    codes = _unpack(qw).astype(np.int64)
    g = r.reshape(N, K // gs, gs).astype(np.float64)
    amax = np.abs(g).max(-1)
    np.testing.assert_array_equal(sc, (amax if nf4 else amax.astype(np.float32) / np.float32(7)).astype(np.float32))
    c = codes.reshape(N, K // gs, gs)
    # the absmax element takes an extreme code
    idx = np.abs(g).argmax(-1)
    top = np.take_along_axis(c, idx[..., None], -1)[..., 0]
    sgn = np.sign(np.take_along_axis(g, idx[..., None], -1)[..., 0])
    nz = amax > 0
    if nf4:
        assert np.all(top[nz & (sgn > 0)] == 15) and np.all(top[nz & (sgn < 0)] == 0)
        # nearest grid point in float64 (ties excluded by a margin)
        grid = oracle.NF4_GRID.astype(np.float64)
        n = g / np.where(amax > 0, amax, 1)[..., None]
        d = np.abs(n[..., None] - grid)
        best = d.argmin(-1)
        ds = np.sort(d, -1)
        clear = (ds[..., 1] - ds[..., 0]) > 1e-6
        assert np.all((c == best)[clear])
        assert np.all(c[3, 1] == 7)  # zero group -> code of 0.0
    else:
        assert np.all(top[nz & (sgn > 0)] == 15) and np.all(top[nz & (sgn < 0)] == 1)
        step = amax / 7
        err = np.abs(g - (c - 8) * step[..., None])
        assert np.all(err <= step[..., None] * (0.5 + 1e-6))
        assert np.all(c[3, 1] == 8)


def test_linear_int4_rounds_half_away_from_zero(oracle):
    # amax = 7 -> inv = 1: values x.5 sit exactly half-way
    row = np.array([7.0, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 3.49] + [0.0] * 24, np.float32)
    qw, sc = oracle.quant_int4_weight(row[None], 32, nf4=False)
    c = _unpack(qw)[0].astype(np.int64) - 8
    assert sc[0, 0] == 1.0
    np.testing.assert_array_equal(c[:8], [7, 3, -3, 1, -1, 2, -2, 3])


def test_activation_int4_properties(oracle):
    rng = np.random.default_rng(5)
    M, K, gs = 6, 256, 64
    x = (rng.standard_normal((M, K)) * 3).astype(np.float32)
    x[0, 0] = 7 * 0.5  # half-way after scaling? checked through the generic bound below
    sm = rng.uniform(0.5, 2.0, K).astype(np.float32)
    pk, sc, bf = oracle.quant_act_int4(x, gs, smooth=sm, want_bf16=True)
    v = (x / sm).astype(np.float32)
    np.testing.assert_array_equal(bf, _bf16(v))
    g = v.reshape(M, K // gs, gs).astype(np.float64)
    amax = np.abs(g).max(-1)
    np.testing.assert_array_equal(sc, (amax.astype(np.float32) / np.float32(7)).T)
    q = _signed(_unpack(pk)).reshape(M, K // gs, gs)
    assert q.min() >= -7 and q.max() <= 7
    step = amax / 7
    assert np.all(np.abs(g - q * step[..., None]) <= step[..., None] * (0.5 + 1e-6))
    pk2, sc2 = oracle.quant_act_int4(v, gs)
    np.testing.assert_array_equal(pk2, pk)
    np.testing.assert_array_equal(sc2, sc)


def test_w4a4_gemm_int64_and_exact_scales(oracle):
    rng = np.random.default_rng(9)
    M, N, K, gs = 5, 7, 256, 64
    G = K // gs
    a = rng.integers(-8, 8, (M, K))
    w = rng.integers(-8, 8, (N, K))
    a[0, :] = -8  # extreme nibbles
    w[0, :] = -8
    ap, wp = _pack(a & 0xF), _pack(w & 0xF)
    # power-of-two scales: every fp32 product and sum below is exact
    asc = (2.0 ** rng.integers(-6, 3, (G, M))).astype(np.float32)
    wsc = (2.0 ** rng.integers(-6, 3, (G, N))).astype(np.float32)
    d = np.einsum("mgk,ngk->gmn", a.reshape(M, G, gs), w.reshape(N, G, gs))  # int64
    want = np.einsum("gmn,gm,gn->mn", d.astype(np.float64), asc.astype(np.float64), wsc.astype(np.float64))
    bias = _bf16(rng.standard_normal(N).astype(np.float32) * 0)  # zero bias keeps the sum exact
    got = oracle.w4a4_gemm(ap, wp, asc, wsc, K, gs, bias_bits=bias)
    np.testing.assert_array_equal(got.astype(np.float64), want)
    # accumulate into existing values
    base = np.full((M, N), 0.5, np.float32)
    got2 = oracle.w4a4_gemm(ap, wp, asc, wsc, K, gs, out=base)
    np.testing.assert_array_equal(got2.astype(np.float64), want + 0.5)
    # general scales: within the fp32 rounding of G products and sums
    asc = rng.uniform(0.01, 1, (G, M)).astype(np.float32)
    wsc = rng.uniform(0.01, 1, (G, N)).astype(np.float32)
    want = np.einsum("gmn,gm,gn->mn", d.astype(np.float64), asc.astype(np.float64), wsc.astype(np.float64))
    got = oracle.w4a4_gemm(ap, wp, asc, wsc, K, gs).astype(np.float64)
    mag = np.einsum("gmn,gm,gn->mn", np.abs(d).astype(np.float64), asc.astype(np.float64), wsc.astype(np.float64))
    assert np.all(np.abs(got - want) <= 4 * G * 2.0 ** -24 * mag + 1e-30)


def _awq_pack(Q):
    """Inverse of the kInterleave=4 address map written from the layout
    comment (cuda_kernels.cu:2992-3001): q for (oc, ic) sits in int16 column
    (ic/64)*64 + (oc%4)*16 + ((ic%64)/32)*8 + ic%8 of row oc/4, nibble
    (ic/8)%4 of that 16-bit half."""
    OC, IC = Q.shape
    words = np.zeros((OC // 4, IC // 2), np.uint32)
    for oc in range(OC):
        for ic in range(IC):
            i16 = (ic // 64) * 64 + (oc % 4) * 16 + ((ic % 64) // 32) * 8 + ic % 8
            words[oc // 4, i16 // 2] |= np.uint32(int(Q[oc, ic]) << ((i16 % 2) * 16 + ((ic // 8) % 4) * 4))
    return words.view(np.int32)


def test_awq_layout_round_trip(oracle):
    rng = np.random.default_rng(3)
    OC, IC, gs, nc = 24, 128, 64, 6
    Q = rng.integers(0, 16, (OC, IC))
    qw = _awq_pack(Q)
    rep = oracle.awq_repack(qw, OC, IC).view(np.uint32)
    for ig in range(IC // 8):
        for k in range(8):
            np.testing.assert_array_equal((rep[ig] >> (4 * k)) & 0xF, Q[:, ig * 8 + k])
    ws = _bf16(rng.uniform(0.01, 0.1, (IC // gs, OC)).astype(np.float32))
    wz = _bf16(rng.uniform(-0.5, 0.5, (IC // gs, OC)).astype(np.float32))
    deq = oracle.dequant_awq_bf16(qw, ws, wz, OC, IC, gs, nc)
    s = oracle.bf16_bits_to_f32(ws).reshape(ws.shape)
    z = oracle.bf16_bits_to_f32(wz).reshape(wz.shape)
    dim = OC // nc
    for so in range(OC):
        nk = (so % dim) * nc + so // dim
        w = (Q[nk].astype(np.float32) * np.repeat(s[:, nk], gs)).astype(np.float32) + np.repeat(z[:, nk], gs)
        np.testing.assert_array_equal(deq[so], _bf16(w.astype(np.float32)))


def test_awq_gemv_float64(oracle):
    rng = np.random.default_rng(4)
    OC, IC, gs, nc = 24, 256, 64, 6
    Q = rng.integers(0, 16, (OC, IC))
    rep = oracle.awq_repack(_awq_pack(Q), OC, IC)
    # exact case: integer inputs, scale 1, zero -8 (bf16-exact), small sums
    ws = _bf16(np.ones((IC // gs, OC), np.float32))
    wz = _bf16(np.full((IC // gs, OC), -8.0, np.float32))
    x = rng.integers(-3, 4, IC).astype(np.float32)
    b = _bf16(rng.integers(-4, 5, OC).astype(np.float32))
    got = oracle.awq_gemv(x, rep, ws, wz, OC, IC, gs, nc, bias_bits=b)
    dim = OC // nc
    want = np.empty(OC)
    for nk in range(OC):
        so = (nk % nc) * dim + nk // nc
        want[so] = float((Q[nk] - 8) @ x.astype(np.int64)) + float(oracle.bf16_bits_to_f32(b)[so])
    np.testing.assert_array_equal(got.astype(np.float64), want)
    # general values: within the fp32 error of an in-order sum
    ws = _bf16(rng.uniform(0.01, 0.1, (IC // gs, OC)).astype(np.float32))
    wz = _bf16(rng.uniform(-0.5, 0.5, (IC // gs, OC)).astype(np.float32))
    x = rng.standard_normal(IC).astype(np.float32)
    got = oracle.awq_gemv(x, rep, ws, wz, OC, IC, gs, nc).astype(np.float64)
    s = oracle.bf16_bits_to_f32(ws).reshape(ws.shape).astype(np.float64)
    z = oracle.bf16_bits_to_f32(wz).reshape(wz.shape).astype(np.float64)
    for nk in range(OC):
        so = (nk % nc) * dim + nk // nc
        w = Q[nk] * np.repeat(s[:, nk], gs) + np.repeat(z[:, nk], gs)
        assert abs(got[so] - w @ x) <= 2 * IC * 2.0 ** -24 * (np.abs(w) @ np.abs(x)) + 1e-6


def _nibble_sources(oracle, N, K, G):
    """For every row-major output nibble of the nunchaku unswizzle, the index
    of the swizzled source nibble, read back 4 bits at a time."""
    n_nib = N * K
    src = np.arange(n_nib, dtype=np.int64)
    out = np.zeros((N, K), np.int64)
    s_sw = np.zeros(N * G, np.uint16)
    for sh in range(0, 24, 4):
        nib = ((src >> sh) & 0xF).astype(np.uint8)
        q_sw = (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8)
        q_rm, _ = oracle.unswizzle_nunchaku(q_sw, s_sw, N, K, G)
        out |= _unpack(q_rm).astype(np.int64) << sh
    return out


def test_nunchaku_unswizzle_is_a_permutation(oracle):
    N, K, G = 128, 128, 2
    srcs = _nibble_sources(oracle, N, K, G)
    assert np.array_equal(np.sort(srcs.ravel()), np.arange(N * K))
    # scales: every swizzled bf16 scale lands once
    s_sw = np.arange(N * G, dtype=np.uint16)
    _, s_rm = oracle.unswizzle_nunchaku(np.zeros(N * K // 2, np.uint8), s_sw, N, K, G)
    vals = (s_rm.view(np.uint32) >> 16).astype(np.int64)
    assert np.array_equal(np.sort(vals.ravel()), np.arange(N * G))


def test_nunchaku_dequant_routes_agree(oracle):
    rng = np.random.default_rng(8)
    N, K, G = 256, 256, 4
    q_sw = rng.integers(0, 256, N * K // 2).astype(np.uint8)
    s_sw = _bf16(rng.uniform(0.01, 1.0, N * G).astype(np.float32))
    direct = oracle.dequant_nunchaku_bf16(q_sw, s_sw, N, K, G)
    q_rm, s_rm = oracle.unswizzle_nunchaku(q_sw, s_sw, N, K, G)
    via = oracle.dequant_int4_bf16(q_rm, s_rm, K, K // G, nf4=False, scales_gn=True, signed_int4=True)
    np.testing.assert_array_equal(direct, via)


@pytest.mark.parametrize("is_down", [False, True])
def test_lora_unswizzle_is_a_permutation(oracle, is_down):
    rows, cols = 64, 48
    packed = np.arange(rows * cols, dtype=np.uint16)
    out = oracle.unswizzle_lora(packed, rows, cols, is_down).astype(np.int64)
    assert np.array_equal(np.sort(out.ravel()), np.arange(rows * cols))
