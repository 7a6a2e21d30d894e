"""CPU checks of the block's host-side pieces: the RoPE table generator
(qwen_image_pe, a restatement of rope.h:9-160) and the oracle's block
operations (oracle/block.py), pinned by invariants rather than by their own
formulas."""
import math

import numpy as np
import pytest


@pytest.fixture(scope="module")
def blk():
    from oracle import block
    return block


@pytest.fixture(scope="module")
def q():
    import qimg_amd
    return qimg_amd


def _angles(pos, dim, theta=10000.0):
    half = dim // 2
    return np.array([[p / theta ** ((2.0 * j) / dim) for j in range(half)] for p in pos])


def test_qwen_image_pe_layout_and_values(q):
    # 128x128 latent, patch 2 -> 64x64 = 4096 image tokens; 256 text tokens first
    pe = q.qwen_image_pe(128, 128, 2, 256)
    assert pe.shape == (4352, 64, 4) and pe.dtype == np.float32
    # every (cos, -sin, sin, cos) quadruple is a rotation
    np.testing.assert_allclose(pe[..., 0], pe[..., 3])
    np.testing.assert_allclose(pe[..., 1], -pe[..., 2])
    np.testing.assert_allclose(pe[..., 0] ** 2 + pe[..., 2] ** 2, 1.0, atol=1e-6)
    # text token j sits at position 64 + j * 256/255 on all three axes
    for j in (0, 1, 255):
        p = 64 + j * 256.0 / 255.0
        ang = np.concatenate([_angles([p], d)[0] for d in (16, 56, 56)])
        np.testing.assert_allclose(pe[j, :, 0], np.cos(ang), atol=2e-4)
        np.testing.assert_allclose(pe[j, :, 2], np.sin(ang), atol=2e-4)
    # image token (r, c) -> axes (0, r - 32, c - 32)
    for r, c in ((0, 0), (31, 40), (63, 63)):
        t = 256 + r * 64 + c
        ang = np.concatenate([_angles([0.0], 16)[0], _angles([r - 32.0], 56)[0], _angles([c - 32.0], 56)[0]])
        np.testing.assert_allclose(pe[t, :, 0], np.cos(ang), atol=2e-5)
        np.testing.assert_allclose(pe[t, :, 2], np.sin(ang), atol=2e-5)


def test_layer_norm_modulate_invariants(blk):
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((5, 3072)) * 7 + 3).astype(np.float32)
    y = blk.layer_norm_modulate(x, np.zeros(3072, np.float32), np.zeros(3072, np.float32))
    np.testing.assert_allclose(y.mean(1), 0, atol=1e-5)
    np.testing.assert_allclose(y.std(1), 1, rtol=1e-4)
    z = blk.layer_norm_modulate(x, np.full(3072, 2, np.float32), np.full(3072, 1, np.float32))
    np.testing.assert_allclose(z, 2 * y + 2, rtol=1e-5, atol=1e-5)


def test_rms_norm_rope_split_invariants(blk):
    from oracle import oracle as o
    rng = np.random.default_rng(1)
    txt = rng.standard_normal((3, 3072)).astype(np.float32)
    img = (rng.standard_normal((5, 3072)) * 4).astype(np.float32)
    ones = o.bf16_bits_from_f32(np.ones(128, np.float32))
    r = blk.rms_norm_heads(img, ones).reshape(5, 24, 128)
    np.testing.assert_allclose(np.sqrt((r.astype(np.float64) ** 2).mean(-1)), 1, rtol=1e-5)
    x = blk.concat_transpose(txt, img)
    assert x.shape == (24, 8, 128)
    np.testing.assert_array_equal(x[3, 0], txt[0, 3 * 128:4 * 128])
    np.testing.assert_array_equal(x[3, 3], img[0, 3 * 128:4 * 128])
    ident = np.zeros((8, 64, 4), np.float32)
    ident[..., 0] = ident[..., 3] = 1
    np.testing.assert_array_equal(blk.rope_f16(x, ident), x.astype(np.float16))
    ang = rng.uniform(-math.pi, math.pi, (8, 64))
    pe = np.stack([np.cos(ang), -np.sin(ang), np.sin(ang), np.cos(ang)], -1).astype(np.float32)
    y = blk.rope_f16(x, pe).astype(np.float64)
    n0 = x[..., 0::2] ** 2 + x[..., 1::2] ** 2
    n1 = y[..., 0::2] ** 2 + y[..., 1::2] ** 2
    np.testing.assert_allclose(n1, n0, rtol=3e-3, atol=1e-3)
    st, si = blk.split(x, 3)
    np.testing.assert_array_equal(st, txt)
    np.testing.assert_array_equal(si, img)


def test_silu_against_independent_forms(blk):
    """silu(x) = x * sigmoid(x): against scipy's logistic function in float64,
    the closed values at 0 and the large-|x| limits (x and 0), and the
    symmetry silu(x) - silu(-x) = x."""
    from scipy.special import expit
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(4096) * 4, [0.0, 30.0, -30.0, 1e-3, -1e-3]]).astype(np.float32)
    y = blk.silu(x)
    want = x.astype(np.float64) * expit(x.astype(np.float64))
    np.testing.assert_allclose(y, want, rtol=3e-7, atol=1e-12)
    assert y[-5] == 0.0 and y[-4] == np.float32(30.0) and abs(y[-3]) < 1e-11
    np.testing.assert_allclose(y.astype(np.float64) - blk.silu(-x), x, rtol=1e-6, atol=1e-6)


def test_gate_add_against_float64(blk):
    """x + gate * y with one fp32 rounding of the product and one of the sum,
    or fewer: within one fp32 ulp of each of the two operations of the
    float64 result; gate 0 returns x and gate 1 is the plain sum."""
    rng = np.random.default_rng(4)
    x = rng.standard_normal((7, 3072)).astype(np.float32)
    y = (rng.standard_normal((7, 3072)) * 3).astype(np.float32)
    g = rng.standard_normal(3072).astype(np.float32)
    got = blk.gate_add(x, g, y).astype(np.float64)
    exact = x.astype(np.float64) + g.astype(np.float64)[None] * y.astype(np.float64)
    ulp = np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64)
    prod_ulp = np.spacing(np.abs(g[None] * y)).astype(np.float64)
    assert np.all(np.abs(got - exact) <= ulp + prod_ulp)
    np.testing.assert_array_equal(blk.gate_add(x, np.zeros(3072, np.float32), y), x)
    np.testing.assert_array_equal(blk.gate_add(x, np.ones(3072, np.float32), y), x + y)
