"""GPU parity: SageAttention. K mean, Q/K int8 values and scales must be
bit-exact against the oracle; the attention output is compared with the
oracle (same quantized inputs; differences come only from exp2/rcp ulps and
fp32 summation order inside the MFMAs) and with float64 attention on the
unquantized inputs at the stated tolerance."""
import math

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


def _inputs(BH, S, D, seed, kshift=0.5):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((BH, S, D)).astype(np.float16)
    k = (rng.standard_normal((BH, S, D)) + kshift).astype(np.float16)
    v = rng.standard_normal((BH, S, D)).astype(np.float16)
    return q, k, v


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


@pytest.mark.parametrize("BH,S,D", [(2, 300, 128), (3, 64, 64), (1, 1, 128), (24, 4352, 128), (2, 129, 64)])
def test_sage_quant_bit_exact(qimg, oracle, BH, S, D):
    q, k, v = _inputs(BH, S, D, BH * S + D)
    mean_ref = oracle.sage_k_mean(k)
    qi_ref, qs_ref = oracle.sage_quant_q(q)
    ki_ref, ks_ref = oracle.sage_quant_k(k, mean_ref)
    kd = _dev(k)
    mean = qimg.sage_k_mean(kd)
    qi, qs = qimg.sage_quant_q(_dev(q))
    ki, ks = qimg.sage_quant_k(kd, mean)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(mean.cpu().numpy(), mean_ref)
    np.testing.assert_array_equal(qs.cpu().numpy(), qs_ref)
    np.testing.assert_array_equal(ks.cpu().numpy(), ks_ref)
    np.testing.assert_array_equal(qi.cpu().numpy(), qi_ref)
    np.testing.assert_array_equal(ki.cpu().numpy(), ki_ref)


def _attn64(q, k, v, scale, causal):
    s = np.einsum("hqd,hkd->hqk", q, k) * scale
    if causal:
        S = q.shape[1]
        s = np.where(np.tril(np.ones((S, S), bool))[None], s, -np.inf)
    s -= s.max(-1, keepdims=True)
    p = np.exp(s)
    return np.einsum("hqk,hkd->hqd", p / p.sum(-1, keepdims=True), v)


@pytest.mark.parametrize("BH,S,D,causal", [
    (2, 300, 128, False), (2, 64, 128, False), (1, 1, 128, False), (2, 200, 64, False),
    (2, 333, 128, True), (1, 130, 64, True), (2, 1000, 128, False),
    # key-tile (64) and query-block (256) boundaries
    (1, 63, 128, False), (1, 65, 128, True), (1, 256, 128, True), (1, 257, 64, False), (1, 513, 128, True),
    (1, 512, 64, True),
])
def test_sage_attention_vs_oracle(qimg, oracle, BH, S, D, causal):
    q, k, v = _inputs(BH, S, D, S * D + causal)
    scale = 1.0 / math.sqrt(D)
    ref = oracle.sage_attention_fp16io(q, k, v, scale, causal).astype(np.float32)
    out = qimg.attention_forward_sage_fp16io(_dev(q), _dev(k), _dev(v), scale, causal=causal)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    # same quantized operands: only ulp-level exp2/rcp and summation-order
    # differences, amplified at most by one fp16 rounding of P and of O
    assert np.max(np.abs(got - ref)) <= 2e-3 * np.max(np.abs(ref)) + 2e-3, np.max(np.abs(got - ref))
    rel, cos = _metrics(got, ref)
    assert cos >= 0.99999, cos
    exact = _attn64(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64), scale, causal)
    rel, cos = _metrics(got, exact)
    assert rel <= 2e-2 and cos >= 0.999, (rel, cos)


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_sage_output_dtypes(qimg, dt):
    rng = np.random.default_rng(5)
    q, k, v = _inputs(2, 256, 128, 5)
    o32 = qimg.attention_forward_sage_fp16io(_dev(q), _dev(k), _dev(v), 0.0883883, out_dtype=torch.float32)
    o32b = qimg.attention_forward_sage_fp16io(_dev(q), _dev(k), _dev(v), 0.0883883, out_dtype=torch.float32)
    o = qimg.attention_forward_sage_fp16io(_dev(q), _dev(k), _dev(v), 0.0883883, out_dtype=dt)
    torch.cuda.synchronize()
    assert torch.equal(o32, o32b), "attention is not run-to-run deterministic"
    # fp32 output is the fp16 result widened (the reference's half_to_float)
    assert torch.equal(o32.half().float(), o32)
    assert torch.equal(o.float(), o32.to(dt).float())


def test_sage_attention_graph_replays(qimg):
    """The entry point's launches (K mean, Q/K quantization, V relayout,
    attention) captured into a HIP graph replay to the eager result, with the
    output and scratch cleared and eager work between replays."""
    q, k, v = _inputs(4, 777, 128, 11)
    qd, kd, vd = _dev(q), _dev(k), _dev(v)
    scratch = torch.empty(qimg.sage_scratch_bytes(4, 777, 128), dtype=torch.uint8, device=DEV)
    ref = qimg.attention_forward_sage_fp16io(qd, kd, vd, 0.0883883, scratch=scratch)
    out = torch.empty_like(ref)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up on the capture stream
        qimg.attention_forward_sage_fp16io(qd, kd, vd, 0.0883883, out=out, scratch=scratch)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        qimg.attention_forward_sage_fp16io(qd, kd, vd, 0.0883883, out=out, scratch=scratch)
    for rep in range(3):
        out.zero_()
        scratch.zero_()
        junk = torch.randn(1 << 20, device=DEV).sum()  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), rep
        del junk
    del graph


@pytest.mark.slow
def test_sage_joint_attention_full_size_sampled(qimg, oracle):
    """Config: 24 heads, S = 4352 (256 txt + 4096 img), D = 128, sampled rows."""
    BH, S, D = 24, 4352, 128
    q, k, v = _inputs(BH, S, D, 0, kshift=0.3)
    scale = 1.0 / math.sqrt(128.0)
    out = qimg.attention_forward_sage_fp16io(_dev(q), _dev(k), _dev(v), scale)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    mean = oracle.sage_k_mean(k)
    qi, qs = oracle.sage_quant_q(q)
    ki, ks = oracle.sage_quant_k(k, mean)
    for r0 in (0, 2048, 4224):
        ref = oracle.sage_attn(qi, ki, v, qs, ks, scale, rows=(r0, r0 + 128))[:, r0:r0 + 128].astype(np.float32)
        g = got[:, r0:r0 + 128]
        assert np.max(np.abs(g - ref)) <= 2e-3 * np.max(np.abs(ref)) + 2e-3


@pytest.mark.slow
def test_sage_joint_attention_c3_inputs(qimg, oracle):
    """C3 on its configured inputs: Q, K, V fp32 N(0,1) rows of the 256 text
    and 4096 image tokens ([tokens, 24 x 128]); per-head RMSNorm (eps 1e-6,
    weight 1) and the Qwen-Image RoPE (qwen_image_pe(128, 128, 2, 256), text
    first) on Q and K; concatenated text first and transposed to fp16 [24,
    4352, 128] (cuda_kernels.cu:1656-1687, 1935-1962; transformer.cu:106-130,
    617-674). The operands are made by the oracle's restatement on the CPU,
    and the GPU's joint_heads_f16 is checked against them at its own bar; the
    attention is then compared with the oracle on 128-query windows of every
    head (text rows, the first image rows, a middle window and the ragged
    tail) and with float64 attention at the stated tolerance."""
    from oracle import block as blk
    n_txt, n_img, H, D = 256, 4096, 24, 128
    S = n_txt + n_img
    rng = np.random.default_rng(31)
    rows = [rng.standard_normal((n, H * D)).astype(np.float32) for n in (n_txt, n_img) * 3]
    ones = oracle.bf16_bits_from_f32(np.ones(D, np.float32))
    pe = qimg.qwen_image_pe(128, 128, 2, n_txt)
    q = blk.rope_f16(blk.concat_transpose(blk.rms_norm_heads(rows[0], ones), blk.rms_norm_heads(rows[1], ones)), pe)
    k = blk.rope_f16(blk.concat_transpose(blk.rms_norm_heads(rows[2], ones), blk.rms_norm_heads(rows[3], ones)), pe)
    v = blk.concat_transpose(rows[4], rows[5]).astype(np.float16)
    # the library's pre-attention pass on the same rows, at its own bar
    ones_d = torch.ones(D, dtype=torch.bfloat16, device=DEV)
    qg = qimg.joint_heads_f16(_dev(rows[0]), _dev(rows[1]), ones_d, ones_d, _dev(pe))
    torch.cuda.synchronize()
    r = q.astype(np.float64)
    assert np.all(np.abs(qg.cpu().numpy().astype(np.float64) - r) <= 2.0 ** -10 * np.abs(r) + 2.0 ** -14 * np.abs(r).max())
    scale = 1.0 / math.sqrt(128.0)
    out = qimg.attention_forward_sage_fp16io(_dev(q), _dev(k), _dev(v), scale, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    mean = oracle.sage_k_mean(k)
    qi, qs = oracle.sage_quant_q(q)
    ki, ks = oracle.sage_quant_k(k, mean)
    qd, kd, vd = (_dev(a) for a in (q, k, v))
    qi_g, qs_g = qimg.sage_quant_q(qd)
    mean_g = qimg.sage_k_mean(kd)
    ki_g, ks_g = qimg.sage_quant_k(kd, mean_g)
    torch.cuda.synchronize()
    # int8 Q/K values and scales bit-exact on these inputs too
    np.testing.assert_array_equal(mean_g.cpu().numpy(), mean)
    np.testing.assert_array_equal(qi_g.cpu().numpy(), qi)
    np.testing.assert_array_equal(qs_g.cpu().numpy(), qs)
    np.testing.assert_array_equal(ki_g.cpu().numpy(), ki)
    np.testing.assert_array_equal(ks_g.cpu().numpy(), ks)
    for r0 in (0, 256, 2112, S - 128):
        ref = oracle.sage_attn(qi, ki, v, qs, ks, scale, rows=(r0, r0 + 128))[:, r0:r0 + 128].astype(np.float32)
        # bf16 output: one bf16 rounding (2^-9 relative) on top of the fp16 bar
        ref_b = torch.from_numpy(ref).to(torch.bfloat16).float().numpy()
        g = got[:, r0:r0 + 128]
        assert np.max(np.abs(g - ref_b)) <= 2e-3 * np.max(np.abs(ref)) + 2e-3 + 2.0 ** -8 * np.max(np.abs(ref)), r0
    # float64 attention on the unquantized fp16 operands, one window of every head
    r0 = 2112
    s64 = np.matmul(q[:, r0:r0 + 128].astype(np.float64), k.astype(np.float64).transpose(0, 2, 1)) * scale
    s64 -= s64.max(-1, keepdims=True)
    p64 = np.exp(s64)
    exact = np.matmul(p64 / p64.sum(-1, keepdims=True), v.astype(np.float64))
    rel, cos = _metrics(got[:, r0:r0 + 128], exact)
    assert rel <= 2e-2 and cos >= 0.999, (rel, cos)
