"""The HIP path on the committed fixture inputs (tests/golden/hotpath_golden.npz):
quantized values and scales bit-exact, linear outputs bit-exact (no GELU) or
within 2e-6 (GELU), attention within the same bound as the oracle parity test."""
import math
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "hotpath_golden.npz")


@pytest.fixture(scope="module")
def g():
    with np.load(GOLDEN, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _bf16(bits):
    return _dev(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


def test_fwht(qimg, g):
    for tag, hbs in (("fwht64", 64), ("fwht1024", 1024)):
        x = _dev(g[f"{tag}_x"])
        qimg.fwht_inplace(x, hbs)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(x.cpu().numpy(), g[f"{tag}_y"])


@pytest.mark.parametrize("tag,hbs,bf16", [("act_f32", 1024, False), ("act_bf16", 4096, True), ("act_512", 512, True)])
def test_activation_quant(qimg, g, tag, hbs, bf16):
    x = _bf16(g[f"{tag}_x"]) if bf16 else _dev(g[f"{tag}_x"])
    q, s = qimg.quantize_activation_hadamard(x, hbs)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(q.cpu().numpy(), g[f"{tag}_q"])
    np.testing.assert_array_equal(s.cpu().numpy(), g[f"{tag}_s"])


def test_weight_quant_and_linear(qimg, g):
    qw = qimg.quantize_weight_tensor(_bf16(g["wq_w"]))
    np.testing.assert_array_equal(qw.data.cpu().numpy(), g["wq_q"])
    np.testing.assert_array_equal(qw.scales.cpu().numpy(), g["wq_s"])
    lw = qimg.quantize_weight_tensor(_bf16(g["lin_w"]))
    out = qimg.linear_forward_quantized(_bf16(g["lin_x"]), lw, _bf16(g["lin_b"]))
    outg = qimg.linear_forward_quantized(_bf16(g["lin_x"]), lw, _bf16(g["lin_b"]), apply_gelu=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), g["lin_out"])
    np.testing.assert_allclose(outg.cpu().numpy(), g["lin_out_gelu"], rtol=2e-6, atol=2e-6)


def test_fp8_quant(qimg, g):
    q, s = qimg.quantize_activation_hadamard(_dev(g["fp8_x"]), 1024, mode=qimg.FP8_HADAMARD)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(q.cpu().numpy(), g["fp8_q"])
    np.testing.assert_array_equal(s.cpu().numpy(), g["fp8_s"])


@pytest.mark.parametrize("tag", ["sage128", "sage64c"])
def test_sage(qimg, g, tag):
    q, k, v = _dev(g[f"{tag}_q"]), _dev(g[f"{tag}_k"]), _dev(g[f"{tag}_v"])
    mean = qimg.sage_k_mean(k)
    qi, qs = qimg.sage_quant_q(q)
    ki, ks = qimg.sage_quant_k(k, mean)
    causal = bool(g[f"{tag}_causal"])
    out = qimg.attention_forward_sage_fp16io(q, k, v, 1.0 / math.sqrt(q.shape[2]), causal=causal,
                                             out_dtype=torch.float16)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(mean.cpu().numpy(), g[f"{tag}_mean"])
    for a, b in ((qi, "qi"), (qs, "qs"), (ki, "ki"), (ks, "ks")):
        np.testing.assert_array_equal(a.cpu().numpy(), g[f"{tag}_{b}"])
    ref = g[f"{tag}_out"].astype(np.float32)
    got = out.float().cpu().numpy()
    assert np.max(np.abs(got - ref)) <= 2e-3 * np.max(np.abs(ref)) + 2e-3
