"""The committed fixtures (tests/golden/hotpath_golden.npz, made by
tests/golden/make_golden.py) against the oracle: every output is recomputed
from the stored inputs and must match bit for bit, so a change to the oracle
that alters any result fails here."""
import math
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "hotpath_golden.npz")


@pytest.fixture(scope="module")
def g():
    with np.load(GOLDEN, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def test_fwht(oracle, g):
    np.testing.assert_array_equal(oracle.fwht_rows(g["fwht64_x"], 64), g["fwht64_y"])
    np.testing.assert_array_equal(oracle.fwht_rows(g["fwht1024_x"], 1024), g["fwht1024_y"])


@pytest.mark.parametrize("tag,hbs,bf16", [("act_f32", 1024, False), ("act_bf16", 4096, True), ("act_512", 512, True)])
def test_activation_quant(oracle, g, tag, hbs, bf16):
    q, s = oracle.quantize_activation(g[f"{tag}_x"], hbs, is_bf16=bf16)
    np.testing.assert_array_equal(q, g[f"{tag}_q"])
    np.testing.assert_array_equal(s, g[f"{tag}_s"])


def test_weight_quant_and_linear(oracle, g):
    q, s, hbs = oracle.quantize_weight_bf16(g["wq_w"])
    np.testing.assert_array_equal(q, g["wq_q"])
    np.testing.assert_array_equal(s, g["wq_s"])
    wq, ws, hbs = oracle.quantize_weight_bf16(g["lin_w"])
    np.testing.assert_array_equal(oracle.linear_w8a8(g["lin_x"], wq, ws, hbs, g["lin_b"]), g["lin_out"])
    np.testing.assert_array_equal(oracle.linear_w8a8(g["lin_x"], wq, ws, hbs, g["lin_b"], gelu=True),
                                  g["lin_out_gelu"])


def test_fp8_quant(oracle, g):
    q, s = oracle.quantize_activation_fp8(g["fp8_x"], 1024)
    np.testing.assert_array_equal(q, g["fp8_q"])
    np.testing.assert_array_equal(s, g["fp8_s"])


@pytest.mark.parametrize("tag", ["sage128", "sage64c"])
def test_sage(oracle, g, tag):
    q, k, v = g[f"{tag}_q"], g[f"{tag}_k"], g[f"{tag}_v"]
    mean = oracle.sage_k_mean(k)
    np.testing.assert_array_equal(mean, g[f"{tag}_mean"])
    qi, qs = oracle.sage_quant_q(q)
    ki, ks = oracle.sage_quant_k(k, mean)
    for a, b in ((qi, "qi"), (qs, "qs"), (ki, "ki"), (ks, "ks")):
        np.testing.assert_array_equal(a, g[f"{tag}_{b}"])
    out = oracle.sage_attention_fp16io(q, k, v, 1.0 / math.sqrt(q.shape[2]), bool(g[f"{tag}_causal"]))
    np.testing.assert_array_equal(out, g[f"{tag}_out"])
