"""GPU parity at the shapes of the 60-block e4m3 denoising step at 1328x1328
(main.cu:761-773 around transformer.cu:497-836): a 166x166 latent in 2x2
patches gives 6889 image tokens, plus 512 text tokens (S = 7401); weights
are e4m3 with per-channel scales behind the same FWHT front end as int8; the
two classifier-free-guidance forwards run as one batch-2 forward, so each
image linear sees 13778 rows and each text linear 1024.

* The e4m3 linears over 13778 rows under the automatic kernel choice: fc1
  (2544 tiles of 256x256 on rows [0, 13568) and the 210 tail rows on 64x64
  tiles, with GELU), fc2 (K = 12288, three tile rounds) and a 3072x3072
  projection, against the oracle on sampled rows of both parts, and against
  the all-large-tile run.
* The block, stage by stage at batch 1 and batch 2: every stage through the
  C-ABI operations, checked against the oracle on the GPU's own inputs of
  that stage (sampled rows for the row-wise stages, the Q/K int8 values and
  scales in full at S = 7401, a 128-query window of every head for the
  attention), then the fused block entry point equal bit for bit to the
  composition. At batch 2 the fused block runs the text-stream q, k, v,
  out-projection and fc2 in the image linears' launches with the gated
  residual in their epilogue; the composition mirrors those kernel choices.
* Batch 2 against two batch-1 forwards over two blocks: bit for bit with
  int8 weights (exact accumulation); with e4m3 weights a text-stream linear
  runs 256x256 tiles at batch 2 (1024 rows) and 64x64 tiles at batch 1
  (512 rows), whose fp32 accumulation orders differ, so the two are held to
  the block's own sensitivity to rounding-level input changes, measured in
  the same test.

e4m3 products are exact and the GPU sums them in fp32 in a different order
than the oracle's float64 sum: a linear's output is held to
1e-5 * max|ref| * sqrt(K / 64) (plus 2e-6 relative after GELU's tanh).
"""
import math

import numpy as np
import pytest
import torch

from blockutil import (DEV, cu_count, dev, gpu_block, metrics, oracle_entries,
                       pair_in_one_launch)

pytestmark = pytest.mark.gpu
N_IMG, N_TXT, D = 6889, 512, 3072
LATENT = 166  # 1328 / 8; 2x2 patches -> 83 x 83 = 6889 tokens


def _fp8_bound(ref, K):
    return 1e-5 * float(np.abs(ref).max()) * math.sqrt(K / 64)


def _rows(t, idx):
    """Rows `idx` of a device tensor, on the host (only those rows move)."""
    return t[torch.as_tensor(np.asarray(idx), device=t.device)].cpu().numpy()


@pytest.fixture(scope="module")
def blk():
    from oracle import block
    return block


@pytest.mark.parametrize("N,K,gelu", [(12288, 3072, True), (3072, 12288, False), (3072, 3072, False)])
def test_c5_fp8_linear_13778_rows(qimg, oracle, N, K, gelu):
    """fc1 / fc2 / a projection over the batch-2 image rows, e4m3."""
    M = 2 * N_IMG
    g = torch.Generator(device=DEV).manual_seed(N + K)
    x = torch.randn(M, K, generator=g, device=DEV)
    wb = (torch.randn(N, K, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    bias = (torch.randn(N, generator=g, device=DEV) * 0.01).to(torch.bfloat16)
    qw = qimg.quantize_weight_tensor(wb, mode=qimg.FP8_HADAMARD)
    # the weight quantization at this shape, bit-exact
    w_bits = wb.view(torch.int16).cpu().numpy().view(np.uint16)
    wq, ws, hbs = oracle.quantize_weight_fp8(w_bits)
    np.testing.assert_array_equal(qw.data.cpu().numpy().view(np.uint8), wq)
    np.testing.assert_array_equal(qw.scales.cpu().numpy(), ws)
    assert qw.had_block_size == hbs == K & -K
    aq, asc = qimg.quantize_activation_hadamard(x, hbs, qimg.FP8_HADAMARD)
    auto = qimg.linear_forward_prequantized(aq, asc, qw, bias, apply_gelu=gelu)
    with qimg.linear_kernel(qimg.LINEAR_LARGE_TILE):
        large = qimg.linear_forward_prequantized(aq, asc, qw, bias, apply_gelu=gelu)
    torch.cuda.synchronize()
    rng = np.random.default_rng(N * 7 + K)
    # rows from the large-tile part, the tail rows and the two sequences' seam
    idx = np.unique(np.concatenate([[0, 255, 256, N_IMG - 1, N_IMG, 13567, 13568, M - 1],
                                    rng.integers(0, M, 20)]))
    rq, rs = oracle.quantize_activation_fp8(_rows(x, idx), hbs)
    np.testing.assert_array_equal(_rows(aq, idx), rq)
    np.testing.assert_array_equal(_rows(asc, idx), rs)
    b_bits = bias.view(torch.int16).cpu().numpy().view(np.uint16)
    ref = oracle.gemm_fp8_epilogue(rq, wq, rs, ws, b_bits, gelu=gelu)
    bound = _fp8_bound(ref, K) + (2e-6 * float(np.abs(ref).max()) if gelu else 0.0)
    got = _rows(auto, idx)
    assert np.max(np.abs(got - ref)) <= bound, np.max(np.abs(got - ref))
    # every row: the automatic choice (tail rows on 64x64 tiles) against the
    # all-large-tile run, each within the bound of the same exact sum
    assert float((auto - large).abs().max()) <= 2 * bound
    assert bool(torch.isfinite(auto).all())


def _stagewise(qimg, oracle, blk, W, B, N, n_img, n_txt, batch, seed):
    """Stage-by-stage composition of the block at batch `batch` (see the
    module docstring) and the fused entry point against it."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    img = torch.randn(batch * n_img, D, generator=g, device=DEV)
    txt = torch.randn(batch * n_txt, D, generator=g, device=DEV)
    t_emb = torch.randn(D, generator=g, device=DEV)
    pe_np = qimg.qwen_image_pe(LATENT, LATENT, 2, n_txt)
    assert pe_np.shape == (n_img + n_txt, 64, 4)
    pe = dev(pe_np)
    rng = np.random.default_rng(seed + 1)
    h = lambda t: t.cpu().numpy()
    ref = oracle_entries(W, B)
    norm_bits = {n: h(v.view(torch.int16)).view(np.uint16) for n, v in N.items()}
    cus = cu_count()
    Mi, Mt = batch * n_img, batch * n_txt

    def rows_of(M, k=20):
        seams = [0, M - 1] + [s * n for n in (n_img, n_txt) for s in range(1, batch) if s * n < M]
        return np.unique(np.concatenate([seams, rng.integers(0, M, k)]).astype(np.int64))

    def check_lin(x, got, name, gelu):
        idx = rows_of(x.shape[0])
        want = blk.qlinear(ref[name], _rows(x, idx), gelu)
        K = x.shape[1]
        bound = _fp8_bound(want, K) if ref[name][4] == 1 else 1e-5 * float(np.abs(want).max())
        if gelu:
            bound += 2e-6 * float(np.abs(want).max())
        assert np.max(np.abs(_rows(got, idx) - want)) <= bound, name

    def lin(x, name, gelu=False, large=False):
        if large:
            with qimg.linear_kernel(qimg.LINEAR_LARGE_TILE):
                got = qimg.linear_forward_quantized(x, W[name], B[name], apply_gelu=gelu)
        else:
            got = qimg.linear_forward_quantized(x, W[name], B[name], apply_gelu=gelu)
        check_lin(x, got, name, gelu)
        return got

    def pair(xi, ni, xt, nt, gelu=False):
        """An image/text linear pair as the block runs it: the text linear
        in the image linear's launch (256x256 tiles) when the dispatcher
        pairs them."""
        N_out = W[ni].data.shape[0]
        together = pair_in_one_launch(xi.shape[0], N_out, xt.shape[0], N_out, cus)
        return lin(xi, ni, gelu), lin(xt, nt, gelu, large=together)

    def ln(x, shift, scale):
        got = qimg.layer_norm_modulate(x, shift.contiguous(), scale.contiguous())
        idx = rows_of(x.shape[0])
        np.testing.assert_allclose(_rows(got, idx), blk.layer_norm_modulate(_rows(x, idx), h(shift), h(scale)),
                                   rtol=2e-5, atol=2e-5)
        return got

    def gate(x, gt, y):
        got = qimg.gate_add(x, gt.contiguous(), y)
        idx = rows_of(x.shape[0])
        np.testing.assert_allclose(_rows(got, idx), blk.gate_add(_rows(x, idx), h(gt), _rows(y, idx)),
                                   rtol=1e-6, atol=1e-6)
        return got

    ts = qimg.silu(t_emb)
    np.testing.assert_allclose(h(ts), blk.silu(h(t_emb)), rtol=2e-6, atol=1e-7)
    mi = lin(ts.view(1, D), "img_mod").view(6, D)
    mt = lin(ts.view(1, D), "txt_mod").view(6, D)
    xi, xt = ln(img, mi[0], mi[1]), ln(txt, mt[0], mt[1])
    qkv = [pair(xi, a, xt, b) for a, b in (("to_q", "add_q_proj"), ("to_k", "add_k_proj"),
                                           ("to_v", "add_v_proj"))]
    # per sequence: RMSNorm + RoPE heads (fp16), V heads; then all
    # batch x 24 heads through the attention
    heads = [[], [], []]
    for s in range(batch):
        for i, (wt, wi) in enumerate((("norm_added_q", "norm_q"), ("norm_added_k", "norm_k"), (None, None))):
            ti = qkv[i][1][s * n_txt:(s + 1) * n_txt]
            ii = qkv[i][0][s * n_img:(s + 1) * n_img]
            if wt is None:
                got = qimg.joint_heads_f16(ti, ii)
                np.testing.assert_array_equal(h(got), blk.concat_transpose(h(ti), h(ii)).astype(np.float16))
            else:
                got = qimg.joint_heads_f16(ti, ii, N[wt], N[wi], pe)
                if s == 0:
                    want = blk.rope_f16(blk.concat_transpose(blk.rms_norm_heads(h(ti), norm_bits[wt]),
                                                             blk.rms_norm_heads(h(ii), norm_bits[wi])), pe_np)
                    gg, r = h(got).astype(np.float64), want.astype(np.float64)
                    assert np.all(np.abs(gg - r) <= 2.0 ** -10 * np.abs(r) + 2.0 ** -14 * np.abs(r).max())
            heads[i].append(got)
    q16, k16, v16 = (torch.cat(x, 0) for x in heads)
    # Q/K int8 values and scales in full
    km = qimg.sage_k_mean(k16)
    qi, qs = qimg.sage_quant_q(q16)
    ki, ks = qimg.sage_quant_k(k16, km)
    qh, kh = h(q16), h(k16)
    rq, rqs = oracle.sage_quant_q(qh)
    rkm = oracle.sage_k_mean(kh)
    rk, rks = oracle.sage_quant_k(kh, rkm)
    np.testing.assert_array_equal(h(km), rkm)
    np.testing.assert_array_equal(h(qi), rq)
    np.testing.assert_array_equal(h(qs), rqs)
    np.testing.assert_array_equal(h(ki), rk)
    np.testing.assert_array_equal(h(ks), rks)
    scale = 1 / np.sqrt(128.0)
    att = qimg.attention_forward_sage_fp16io(q16, k16, v16, scale, out_dtype=torch.float16)
    S = n_img + n_txt
    for q0 in (n_txt - 64, S - 128):  # the text/image seam and the ragged end
        want = oracle.sage_attn(rq, rk, h(v16), rqs, rks, scale, False, rows=(q0, q0 + 128))[:, q0:q0 + 128]
        got = h(att)[:, q0:q0 + 128].astype(np.float32)
        want = want.astype(np.float32)
        assert np.max(np.abs(got - want)) <= 2e-3 * np.abs(want).max() + 2e-3
        rel, cos = metrics(got, want)
        assert rel <= 2e-2 and cos >= 0.999, (rel, cos)
    # back to the streams
    parts = [qimg.split_heads(att[s * 24:(s + 1) * 24], n_txt) for s in range(batch)]
    for s in range(batch):
        rt, ri = blk.split(h(att[s * 24:(s + 1) * 24]), n_txt)
        np.testing.assert_array_equal(h(parts[s][0]), rt)
        np.testing.assert_array_equal(h(parts[s][1]), ri)
    at = torch.cat([p[0] for p in parts], 0)
    ai = torch.cat([p[1] for p in parts], 0)
    oi, ot = pair(ai, "to_out", at, "to_add_out")
    x1i, x1t = gate(img, mi[2], oi), gate(txt, mt[2], ot)
    hi = lin(ln(x1i, mi[3], mi[4]), "img_mlp_fc1", gelu=True)
    ht = lin(ln(x1t, mt[3], mt[4]), "txt_mlp_fc1", gelu=True)
    yi, yt = pair(hi, "img_mlp_fc2", ht, "txt_mlp_fc2")
    fi, ft = gate(x1i, mi[5], yi), gate(x1t, mt[5], yt)
    table = qimg.BlockTable([(W, B, N)])
    img_d, txt_d = img.clone(), txt.clone()
    qimg.mmdit_blocks_forward(table, img_d.view(batch, n_img, D), txt_d.view(batch, n_txt, D), t_emb, pe)
    torch.cuda.synchronize()
    assert torch.isfinite(img_d).all()
    assert torch.equal(img_d, fi)
    assert torch.equal(txt_d, ft)
    return Mi, Mt


@pytest.fixture(scope="module")
def c5_fp8(qimg):
    return gpu_block(qimg, 51, mode=1)


@pytest.mark.parametrize("batch", [1, 2])
def test_c5_block_fp8_full_size_stagewise(qimg, oracle, blk, c5_fp8, batch):
    W, B, N = c5_fp8
    Mi, Mt = _stagewise(qimg, oracle, blk, W, B, N, N_IMG, N_TXT, batch, seed=60 + batch)
    if batch == 2 and cu_count() == 256:
        # the composition really covered the paired launches
        assert pair_in_one_launch(Mi, 3072, Mt, 3072, 256)


def _two_blocks(qimg, mode, seed):
    W, B, N = gpu_block(qimg, seed, mode=mode)
    W2, B2, N2 = gpu_block(qimg, seed + 1, mode=mode)
    return [(W, B, N), (W2, B2, N2)]


@pytest.mark.parametrize("mode", [0, 1])
def test_c5_batched_cfg_pair_against_two_forwards(qimg, mode):
    """Two blocks over the CFG pair at 6889 + 512 tokens, batched against
    each sequence alone (see the module docstring for the e4m3 bar)."""
    blocks = _two_blocks(qimg, mode, 70 + mode)
    table = qimg.BlockTable(blocks)
    g = torch.Generator(device=DEV).manual_seed(80 + mode)
    img = torch.randn(2, N_IMG, D, generator=g, device=DEV)
    txt = torch.randn(2, N_TXT, D, generator=g, device=DEV)
    t_emb = torch.randn(D, generator=g, device=DEV)
    pe = dev(qimg.qwen_image_pe(LATENT, LATENT, 2, N_TXT))
    ib, tb = img.clone(), txt.clone()
    qimg.mmdit_blocks_forward(table, ib, tb, t_emb, pe)
    seq = []
    for s in range(2):
        i1, t1 = img[s].clone(), txt[s].clone()
        qimg.mmdit_blocks_forward(table, i1, t1, t_emb, pe)
        seq.append((i1, t1))
    # the same forward on rounding-level perturbed inputs: the block's own
    # sensitivity, the bar for kernels with different fp32 summation orders
    noise = torch.randn(N_IMG, D, generator=g, device=DEV)
    ip, tp = img[0] * (1 + 1e-6 * noise), txt[0].clone()
    qimg.mmdit_blocks_forward(table, ip, tp, t_emb, pe)
    torch.cuda.synchronize()
    assert torch.isfinite(ib).all() and torch.isfinite(tb).all()
    if mode == 0:
        for s in range(2):
            assert torch.equal(ib[s], seq[s][0]), s
            assert torch.equal(tb[s], seq[s][1]), s
        return
    h = lambda t: t.cpu().numpy()
    rel_self, cos_self = metrics(h(ip), h(seq[0][0]))
    for s in range(2):
        for got, want in ((ib[s], seq[s][0]), (tb[s], seq[s][1])):
            rel, cos = metrics(h(got), h(want))
            assert cos >= 0.999, (s, rel, cos)
            assert rel <= max(2e-2, 2.5 * rel_self), (s, rel, rel_self)
            assert 1 - cos <= max(1e-5, 2.5 * (1 - cos_self)), (s, cos, cos_self)


def test_c5_int8_block_same_for_every_kernel_choice(qimg):
    """int8 weights at 6889 + 512 tokens, batch 2: the automatic choice
    (paired text linears, the fc1 tail rows on 64x64 tiles, small-M
    modulation) and the all-large-tile run give the same bits."""
    W, B, N = gpu_block(qimg, 90)
    table = qimg.BlockTable([(W, B, N)])
    g = torch.Generator(device=DEV).manual_seed(91)
    img = torch.randn(2, N_IMG, D, generator=g, device=DEV)
    txt = torch.randn(2, N_TXT, D, generator=g, device=DEV)
    t_emb = torch.randn(D, generator=g, device=DEV)
    pe = dev(qimg.qwen_image_pe(LATENT, LATENT, 2, N_TXT))
    outs = []
    for choice in (qimg.LINEAR_AUTO, qimg.LINEAR_LARGE_TILE):
        i, t = img.clone(), txt.clone()
        with qimg.linear_kernel(choice):
            qimg.mmdit_blocks_forward(table, i, t, t_emb, pe)
        torch.cuda.synchronize()
        outs.append((i, t))
    assert torch.isfinite(outs[0][0]).all()
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1], outs[1][1])
