"""GPU parity: the BF16-mode linear (QuantMode::BF16; linear_forward_bf16 /
_bf16in, cuda_kernels.cu:4534-4596) at the shapes of the four layers a
quantized checkpoint keeps in bf16 (img_in 3072x64, txt_in 3072x3584,
norm_out 6144x3072, proj_out 64x3072; transformer.cu:396-419, 874-895).

* Integer-valued operands (exact in bf16, every partial sum exact in fp32)
  give the int64 product plus the bias bit for bit, whatever the summation
  order: this catches a dropped, repeated or misplaced term.
* One-hot weights return bf16(x): the fp32 -> bf16 rounding (nearest even)
  bit for bit.
* Random N(0,1) activations and N(0,0.02) weights against the oracle's
  exactly summed product: within 8 sqrt(K) 2^-24 sum_k |x_k w_k| (the size of
  an fp32 summation error, with margin; the order of cuBLAS's accumulation
  is not part of the reference's sources), GELU within 1e-5; and against
  unrounded float64 math at the stated bar (max-rel 2e-2, cosine 0.999).
"""
import math

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

# (M, N, K): img_in / proj_out at 4096, 6889 and 13778 (CFG pair) image
# tokens, txt_in at 256 / 512 / 1024 text tokens, norm_out at M = 1 and 2
LAYERS = [(4096, 3072, 64), (6889, 3072, 64), (13778, 3072, 64),
          (256, 3072, 3584), (512, 3072, 3584), (1024, 3072, 3584),
          (1, 6144, 3072), (2, 6144, 3072),
          (4096, 64, 3072), (6889, 64, 3072), (13778, 64, 3072)]
# ragged tiles and K not a multiple of 32 (the one-thread-per-output kernel)
RAGGED = [(7, 300, 96), (130, 70, 160), (33, 65, 32), (5, 17, 100), (3, 40, 8)]
# bf16 x with at least 128 tiles of 256x256 (the large-tile kernel; the INT4
# linear's residual GEMM): a full-tile shape and a ragged one
LARGE = [(4096, 3072, 3072), (1000, 12288, 3072)]


def _bf16_dev(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(DEV).view(torch.bfloat16)


def _rows(M, rng, k=48):
    return np.unique(np.concatenate([[0, M - 1], rng.integers(0, M, k)]))


@pytest.mark.parametrize("M,N,K", LAYERS + RAGGED + LARGE)
@pytest.mark.parametrize("x_fp32", [True, False])
def test_linear_bf16_integer_operands_exact(qimg, oracle, M, N, K, x_fp32):
    rng = np.random.default_rng(M * 3 + N + K + x_fp32)
    xi = rng.integers(-4, 5, (M, K)).astype(np.float32)
    wi = rng.integers(-4, 5, (N, K)).astype(np.float32)
    b = oracle.bf16_bits_from_f32(rng.integers(-8, 9, N).astype(np.float32))
    x = torch.from_numpy(xi).to(DEV)
    if not x_fp32:
        x = x.to(torch.bfloat16)
    w = torch.from_numpy(wi).to(DEV).to(torch.bfloat16)
    out = qimg.linear_forward_bf16(x, w, _bf16_dev(b))
    torch.cuda.synchronize()
    idx = _rows(M, rng)
    want = (xi[idx].astype(np.int64) @ wi.T.astype(np.int64)).astype(np.float64) + oracle.bf16_bits_to_f32(b)
    np.testing.assert_array_equal(out.cpu().numpy()[idx], want.astype(np.float32))


@pytest.mark.parametrize("M,N,K", [(4096, 3072, 3072), (4100, 3076, 1024)])
def test_linear_bf16_large_tile_widths(qimg, oracle, M, N, K):
    """bf16 x on the large tiles, 256 and 256x192 wide (waves 4 x 2 of
    64x96): each output's k-sum runs through the same MFMA sequence, so the
    widths agree bit for bit, with and without GELU, on ragged tiles too
    (last tiles of 4 columns and 4 rows); and the values match the oracle's
    integer-operand answer exactly."""
    rng = np.random.default_rng(M + 2 * N + K)
    xi = rng.integers(-4, 5, (M, K)).astype(np.float32)
    wi = rng.integers(-4, 5, (N, K)).astype(np.float32)
    b = oracle.bf16_bits_from_f32(rng.integers(-8, 9, N).astype(np.float32))
    x = torch.from_numpy(xi).to(DEV).to(torch.bfloat16)
    w = torch.from_numpy(wi).to(DEV).to(torch.bfloat16)
    bd = _bf16_dev(b)
    outs = {}
    for choice in (qimg.LINEAR_LARGE_TILE, qimg.LINEAR_LARGE_192):
        with qimg.linear_kernel(choice):
            outs[choice] = (qimg.linear_forward_bf16(x, w, bd), qimg.linear_forward_bf16(x, w, bd, apply_gelu=True))
    torch.cuda.synchronize()
    for a, c in zip(outs[qimg.LINEAR_LARGE_TILE], outs[qimg.LINEAR_LARGE_192]):
        assert torch.equal(a, c)
    idx = _rows(M, rng)
    want = (xi[idx].astype(np.int64) @ wi.T.astype(np.int64)).astype(np.float64) + oracle.bf16_bits_to_f32(b)
    np.testing.assert_array_equal(outs[qimg.LINEAR_LARGE_192][0].cpu().numpy()[idx], want.astype(np.float32))


@pytest.mark.parametrize("M,K", [(300, 64), (17, 3584), (4, 96)])
def test_linear_bf16_rounds_fp32_input_to_nearest_even(qimg, oracle, M, K):
    rng = np.random.default_rng(M + K)
    x = (rng.standard_normal((M, K)) * 5).astype(np.float32)
    # exact ties between two bf16 values, both parities, and values that
    # round across a binade
    u = x.view(np.uint32)
    u[:, 0::7] = (u[:, 0::7] & 0xFFFF0000) | 0x8000
    u[:, 3::11] = (u[:, 3::11] & 0xFFFE0000) | 0x18000
    u[:, 5::13] |= 0x7FFF
    eye = np.eye(K, dtype=np.float32)
    got = qimg.linear_forward_bf16(torch.from_numpy(x).to(DEV), torch.from_numpy(eye).to(DEV).to(torch.bfloat16))
    torch.cuda.synchronize()
    want = oracle.bf16_bits_to_f32(oracle.bf16_bits_from_f32(x)).reshape(M, K)
    np.testing.assert_array_equal(got.cpu().numpy(), want)


@pytest.mark.parametrize("M,N,K,x_fp32,gelu",
                         [(M, N, K, xf, g) for (M, N, K) in LAYERS + RAGGED[:2]
                          for (xf, g) in [(True, False), (False, False), (True, True)]]
                         + [(M, N, K, False, g) for (M, N, K) in LARGE for g in (False, True)])
def test_linear_bf16_random_vs_oracle(qimg, oracle, M, N, K, x_fp32, gelu):
    rng = np.random.default_rng(M + 7 * N + K + 2 * x_fp32 + gelu)
    g = torch.Generator(device=DEV).manual_seed(M + N + K)
    x = torch.randn(M, K, generator=g, device=DEV)
    if not x_fp32:
        x = x.to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    bias = (torch.randn(N, generator=g, device=DEV) * 0.01).to(torch.bfloat16)
    out = qimg.linear_forward_bf16(x, w, bias, apply_gelu=gelu)
    torch.cuda.synchronize()
    idx = _rows(M, rng)
    xs = x[torch.as_tensor(idx, device=DEV)]
    xh = xs.cpu().numpy() if x_fp32 else xs.view(torch.int16).cpu().numpy().view(np.uint16)
    w_bits = w.view(torch.int16).cpu().numpy().view(np.uint16)
    b_bits = bias.view(torch.int16).cpu().numpy().view(np.uint16)
    want, mag = oracle.linear_bf16(xh, w_bits, b_bits, gelu=gelu)
    got = out[torch.as_tensor(idx, device=DEV)].cpu().numpy().astype(np.float64)
    assert np.isfinite(got).all()
    if gelu:
        assert np.max(np.abs(got - want)) <= 1e-5 * max(1.0, np.abs(want).max())
    else:
        bound = 8 * math.sqrt(K) * 2.0 ** -24 * mag + 2.0 ** -24 * np.abs(want)
        assert np.all(np.abs(got - want) <= bound), np.max(np.abs(got - want) / bound)
    # the stated bar against unrounded float64 math
    xf = xs.float().cpu().numpy().astype(np.float64)
    exact = xf @ w.float().cpu().numpy().astype(np.float64).T + bias.float().cpu().numpy()
    if gelu:
        exact = oracle.gelu_tanh64(exact)
    a, e = got.ravel(), exact.ravel()
    rel = np.max(np.abs(a - e)) / np.max(np.abs(e))
    cos = float(a @ e / (np.linalg.norm(a) * np.linalg.norm(e)))
    assert rel <= 2e-2 and cos >= 0.999, (rel, cos)


def test_linear_bf16_rejects_bad_arguments(qimg):
    x = torch.zeros(4, 64, device=DEV)
    w = torch.zeros(8, 64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(qimg.QimgError):
        qimg.linear_forward_bf16(x, w.float())   # fp32 weights
    with pytest.raises(qimg.QimgError):
        qimg.linear_forward_bf16(x, torch.zeros(8, 32, dtype=torch.bfloat16, device=DEV))  # K mismatch
    L = qimg.lib()
    assert L.qimg_linear_bf16(qimg._ptr(x), 2, 4, 64, qimg._ptr(w), 8, None, qimg._ptr(x), 0, None) == 1  # fp16 x
