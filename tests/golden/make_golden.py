#!/usr/bin/env python3
"""Writes tests/golden/hotpath_golden.npz: small seeded inputs of the hot path
and the CPU oracle's outputs for them.

The reference ships no golden vectors for this path (its only known-answer
test, test_philox.cu, covers latent noise), so these fixtures are the oracle's
own outputs, produced after the oracle passed its independent pins
(tests/test_oracle_pins.py). They freeze those results: tests/test_golden.py
recomputes them with the oracle (bit-exact), and tests/test_gpu_golden.py runs
the HIP path on the same inputs.

    python tests/golden/make_golden.py
"""
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as o  # noqa: E402

OUT = os.path.join(HERE, "hotpath_golden.npz")


def make() -> dict:
    rng = np.random.default_rng(20261201)
    g = {}
    # a2: FWHT, two block sizes
    g["fwht64_x"] = rng.standard_normal((3, 192)).astype(np.float32)
    g["fwht64_y"] = o.fwht_rows(g["fwht64_x"], 64)
    g["fwht1024_x"] = rng.standard_normal((2, 3072)).astype(np.float32)
    g["fwht1024_y"] = o.fwht_rows(g["fwht1024_x"], 1024)
    # a5: activation FWHT + int8 (fp32 in, hbs 1024; bf16 in, hbs 4096 and 512)
    x = (rng.standard_normal((8, 3072)) * rng.uniform(0.1, 10, (8, 1))).astype(np.float32)
    x[0] = 0.0                                   # all-zero row: scale 0, q 0
    x[1, 5] = 100.0                              # spike
    g["act_f32_x"] = x
    g["act_f32_q"], g["act_f32_s"] = o.quantize_activation(x, 1024, is_bf16=False)
    g["act_bf16_x"] = o.bf16_bits_from_f32(rng.standard_normal((4, 12288)).astype(np.float32))
    g["act_bf16_q"], g["act_bf16_s"] = o.quantize_activation(g["act_bf16_x"], 4096, is_bf16=True)
    g["act_512_x"] = o.bf16_bits_from_f32(rng.standard_normal((3, 3584)).astype(np.float32))
    g["act_512_q"], g["act_512_s"] = o.quantize_activation(g["act_512_x"], 512, is_bf16=True)
    # a4: weight quantization
    g["wq_w"] = o.bf16_bits_from_f32((rng.standard_normal((16, 3072)) * 0.02).astype(np.float32))
    g["wq_q"], g["wq_s"], _ = o.quantize_weight_bf16(g["wq_w"])
    # a9: linear (bf16 in), with and without GELU
    g["lin_x"] = o.bf16_bits_from_f32(rng.standard_normal((16, 3072)).astype(np.float32))
    g["lin_w"] = o.bf16_bits_from_f32((rng.standard_normal((40, 3072)) * 0.02).astype(np.float32))
    g["lin_b"] = o.bf16_bits_from_f32((rng.standard_normal(40) * 0.01).astype(np.float32))
    wq, ws, hbs = o.quantize_weight_bf16(g["lin_w"])
    g["lin_out"] = o.linear_w8a8(g["lin_x"], wq, ws, hbs, g["lin_b"])
    g["lin_out_gelu"] = o.linear_w8a8(g["lin_x"], wq, ws, hbs, g["lin_b"], gelu=True)
    # fp8 (e4m3) activation quantization
    g["fp8_x"] = rng.standard_normal((4, 3072)).astype(np.float32)
    g["fp8_q"], g["fp8_s"] = o.quantize_activation_fp8(g["fp8_x"], 1024)
    # a12-a17: SageAttention, non-causal D=128 and causal D=64
    for tag, (BH, S, D, causal) in {"sage128": (2, 200, 128, False), "sage64c": (1, 130, 64, True)}.items():
        q = rng.standard_normal((BH, S, D)).astype(np.float16)
        k = (rng.standard_normal((BH, S, D)) + 0.5).astype(np.float16)
        v = rng.standard_normal((BH, S, D)).astype(np.float16)
        mean = o.sage_k_mean(k)
        qi, qs = o.sage_quant_q(q)
        ki, ks = o.sage_quant_k(k, mean)
        g[f"{tag}_q"], g[f"{tag}_k"], g[f"{tag}_v"] = q, k, v
        g[f"{tag}_mean"], g[f"{tag}_qi"], g[f"{tag}_qs"], g[f"{tag}_ki"], g[f"{tag}_ks"] = mean, qi, qs, ki, ks
        g[f"{tag}_out"] = o.sage_attention_fp16io(q, k, v, 1.0 / math.sqrt(D), causal)
        g[f"{tag}_causal"] = np.array(causal)
    return g


if __name__ == "__main__":
    g = make()
    np.savez_compressed(OUT, **g)
    print(f"wrote {OUT}: {len(g)} arrays, {os.path.getsize(OUT)} bytes")
