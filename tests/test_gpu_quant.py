"""GPU parity: fused FWHT + quantization kernels against the oracle.
Quantized values and scales must be bit-exact."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _bf16_dev(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(DEV).view(torch.bfloat16)


@pytest.mark.parametrize("M,K,in_bf16", [
    (4096, 3072, True),      # C1 img activations (bf16 in)
    (256, 3072, False),      # txt activations, fp32 in (the reference's path)
    (64, 12288, False),      # fc2 input, hbs 4096
    (1, 3072, False),        # modulation / timestep row
    (33, 256, True),         # K = 256 (timestep linear_1)
    (5, 3584, True),         # hbs 512 (odd power of two: non-exact norm)
    (3, 96, False),          # hbs 32
    (7, 24, False),          # hbs 8: scalar path
    (4, 17, True),           # hbs 1: plain per-token quantization
])
def test_activation_quant_int8_bit_exact(qimg, oracle, M, K, in_bf16):
    rng = np.random.default_rng(M * 131 + K)
    x = (rng.standard_normal((M, K)) * rng.uniform(0.1, 10, (M, 1))).astype(np.float32)
    hbs = K & -K
    if in_bf16:
        bits = oracle.bf16_bits_from_f32(x)
        q_ref, s_ref = oracle.quantize_activation(bits, hbs, is_bf16=True)
        xd = _bf16_dev(bits)
    else:
        q_ref, s_ref = oracle.quantize_activation(x, hbs, is_bf16=False)
        xd = torch.from_numpy(x).to(DEV)
    q, s = qimg.quantize_activation_hadamard(xd, hbs)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)


@pytest.mark.parametrize("M,K,in_bf16,fp8", [
    (300, 12288, False, False),   # fc2 input: three 4096-blocks
    (37, 12288, True, True),
    (6, 8192, False, False),      # hbs 4096 given explicitly: two blocks
    (3, 16384, True, False),      # four blocks
    (5, 16384, False, True),
])
def test_activation_quant_4096_blocks_bit_exact(qimg, oracle, M, K, in_bf16, fp8):
    """Rows of 2-4 Hadamard blocks of 4096 (the block-by-block kernel)."""
    rng = np.random.default_rng(M * 7 + K + fp8)
    x = (rng.standard_normal((M, K)) * rng.uniform(0.1, 10, (M, 1))).astype(np.float32)
    x[0, :] = 0.0  # an all-zero row: scale 0, all-zero values
    mode = qimg.FP8_HADAMARD if fp8 else qimg.INT8_HADAMARD
    ref = oracle.quantize_activation_fp8 if fp8 else oracle.quantize_activation
    if in_bf16:
        bits = oracle.bf16_bits_from_f32(x)
        q_ref, s_ref = ref(bits, 4096)
        xd = _bf16_dev(bits)
    else:
        q_ref, s_ref = ref(x, 4096)
        xd = torch.from_numpy(x).to(DEV)
    q, s = qimg.quantize_activation_hadamard(xd, 4096, mode=mode)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(q.cpu().numpy().view(np.uint8), q_ref.view(np.uint8))


@pytest.mark.parametrize("M,K,in_bf16,fp8", [
    (5, 1024, False, False),      # one 1024-block per row
    (7, 2048, True, True),
    (4353, 3072, True, True),     # rows not a multiple of four
    (2, 4096, True, False),       # four blocks
    (9, 4096, False, True),
])
def test_activation_quant_1024_blocks_bit_exact(qimg, oracle, M, K, in_bf16, fp8):
    """Rows of 1-4 Hadamard blocks of 1024 (one wave per row)."""
    rng = np.random.default_rng(M * 5 + K + fp8)
    x = (rng.standard_normal((M, K)) * rng.uniform(0.1, 10, (M, 1))).astype(np.float32)
    x[M - 1, :] = 0.0  # an all-zero row: scale 0, all-zero values
    mode = qimg.FP8_HADAMARD if fp8 else qimg.INT8_HADAMARD
    ref = oracle.quantize_activation_fp8 if fp8 else oracle.quantize_activation
    if in_bf16:
        bits = oracle.bf16_bits_from_f32(x)
        q_ref, s_ref = ref(bits, 1024)
        xd = _bf16_dev(bits)
    else:
        q_ref, s_ref = ref(x, 1024)
        xd = torch.from_numpy(x).to(DEV)
    q, s = qimg.quantize_activation_hadamard(xd, 1024, mode=mode)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(q.cpu().numpy().view(np.uint8), q_ref.view(np.uint8))


@pytest.mark.parametrize("M,K", [(128, 3072), (16, 12288), (3, 64)])
def test_activation_quant_fp8_bit_exact(qimg, oracle, M, K):
    rng = np.random.default_rng(K + 7)
    x = rng.standard_normal((M, K)).astype(np.float32)
    hbs = K & -K
    q_ref, s_ref = oracle.quantize_activation_fp8(x, hbs)
    q, s = qimg.quantize_activation_hadamard(torch.from_numpy(x).to(DEV), hbs, mode=qimg.FP8_HADAMARD)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)


def test_e4m3_rounding_at_every_tie(qimg, oracle):
    """The e4m3 conversion of the quantizers against the oracle's, on values
    chosen to decide the rounding: every midpoint between adjacent e4m3
    magnitudes (ties go to the even code), one fp32 ulp either side of each
    midpoint, the subnormal range (quantum 2^-9, ties at odd multiples of
    2^-10), values just under 448, zeros and random magnitudes, both signs.
    Each row's first value is 448, so the row scale is exactly 1 and the
    stored code is the conversion of the value itself (hbs = 1: no
    transform)."""
    codes = oracle.e4m3_to_f32(np.arange(0, 0x7f, dtype=np.uint8)).astype(np.float64)  # +0 .. 448
    mids = (codes[:-1] + codes[1:]) / 2
    m32 = mids.astype(np.float32)
    vals = np.concatenate([m32, np.nextafter(m32, np.float32(0)), np.nextafter(m32, np.float32(np.inf)),
                           codes.astype(np.float32), np.float32([2.0 ** -10, 3 * 2.0 ** -10, 2.0 ** -11, 1e-30, 0.0,
                                                                 447.9, 447.99997, 448.0])])
    rng = np.random.default_rng(4)
    vals = np.concatenate([vals, (rng.random(2000) * 448).astype(np.float32),
                           (2.0 ** rng.uniform(-12, 8.8, 2000)).astype(np.float32)])
    vals = np.concatenate([vals, -vals])
    K = 4096
    rows = -(-vals.size // (K - 1))
    x = np.zeros((rows, K), np.float32)
    x[:, 0] = 448.0
    x.reshape(-1)[np.flatnonzero(np.tile(np.arange(K) > 0, rows))[:vals.size]] = vals
    q_ref, s_ref = oracle.quantize_activation_fp8(x, 1)
    assert np.all(s_ref == np.float32(1.0))
    q, s = qimg.quantize_activation_hadamard(torch.from_numpy(x).to(DEV), 1, mode=qimg.FP8_HADAMARD)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)
    # ties really are ties and round to the even code in the oracle
    tie_codes = q_ref.reshape(-1)[np.flatnonzero(np.tile(np.arange(K) > 0, rows))[:m32.size]]
    assert np.all((tie_codes & 1) == 0)


def test_int8_rounding_at_every_tie(qimg, oracle):
    """The int8 conversion of the quantizers (clamp, round half to even)
    against the oracle on every half-integer in range, one fp32 ulp either
    side of each, the integers and random values, both signs. Each row's
    first value is 127, so the row scale is exactly 1 and the stored value is
    the rounding of the value itself (hbs = 1: no transform)."""
    half = np.arange(-127, 127, dtype=np.float64) + 0.5
    h32 = half.astype(np.float32)
    vals = np.concatenate([h32, np.nextafter(h32, np.float32(-np.inf)), np.nextafter(h32, np.float32(np.inf)),
                           np.arange(-127, 128, dtype=np.float32), np.float32([126.99999, -126.99999, 0.0, -0.0, 1e-30])])
    rng = np.random.default_rng(5)
    vals = np.concatenate([vals, ((rng.random(3000) * 2 - 1) * 127).astype(np.float32)])
    K = 4096
    rows = -(-vals.size // (K - 1))
    x = np.zeros((rows, K), np.float32)
    x[:, 0] = 127.0
    idx = np.flatnonzero(np.tile(np.arange(K) > 0, rows))[:vals.size]
    x.reshape(-1)[idx] = vals
    q_ref, s_ref = oracle.quantize_activation(x, 1, is_bf16=False)
    assert np.all(s_ref == np.float32(1.0))
    q, s = qimg.quantize_activation_hadamard(torch.from_numpy(x).to(DEV), 1)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)
    ties = q_ref.reshape(-1)[idx[:h32.size]].astype(np.int64)
    assert np.all(ties % 2 == 0)


def test_activation_quant_special_rows(qimg, oracle):
    K = 3072
    x = np.zeros((4, K), np.float32)
    x[1, 17] = 3.0
    x[2, :] = -1.0
    x[3, ::7] = 1e-30
    q_ref, s_ref = oracle.quantize_activation(x, 1024, is_bf16=False)
    q, s = qimg.quantize_activation_hadamard(torch.from_numpy(x).to(DEV), 1024)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)
    assert s_ref[0] == 0 and not q_ref[0].any()


@pytest.mark.parametrize("N,K,mode", [(3072, 3072, 0), (12288, 3072, 0), (3072, 12288, 0),
                                      (18432, 3072, 0), (512, 3072, 1), (256, 12288, 1)])
def test_weight_quant_bit_exact(qimg, oracle, N, K, mode):
    rng = np.random.default_rng(N + K + mode)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    bits = oracle.bf16_bits_from_f32(w)
    if mode == 0:
        q_ref, s_ref, hbs_ref = oracle.quantize_weight_bf16(bits)
    else:
        q_ref, s_ref, hbs_ref = oracle.quantize_weight_fp8(bits)
    qw = qimg.quantize_weight_tensor(_bf16_dev(bits), mode=mode)
    assert qw.had_block_size == hbs_ref
    np.testing.assert_array_equal(qw.scales.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(qw.data.cpu().numpy().view(np.uint8), q_ref.view(np.uint8))


def test_fwht_inplace_and_per_row(qimg, oracle):
    rng = np.random.default_rng(11)
    x = rng.standard_normal((300, 3072)).astype(np.float32)
    xd = torch.from_numpy(x).to(DEV)
    qimg.fwht_inplace(xd, 1024)
    torch.cuda.synchronize()
    ref = oracle.fwht_rows(x, 1024)
    np.testing.assert_array_equal(xd.cpu().numpy(), ref)
    q, s = qimg.quantize_per_row_fp32(xd)
    q_ref, s_ref = oracle.quant_rows_int8(ref)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)


@pytest.mark.parametrize("K,hbs,in_bf16,fp8", [
    (12288, 4096, False, False),  # the MLP's fc2 input
    (12288, 4096, False, True),
    (3072, 1024, True, False),    # the fc1 input
])
def test_activation_quant_row_split_identical(qimg, K, hbs, in_bf16, fp8):
    """Quantization is row-wise: 4352 rows in one call equal rows 0-4095 and
    4096-4351 in two calls (each call picks its kernel from its own row
    count), as a caller that splits the image and text rows over two
    streams relies on."""
    M, MI = 4352, 4096
    g = torch.Generator(device="cpu").manual_seed(K + fp8)
    x = (torch.randn(M, K, generator=g) * torch.rand(M, 1, generator=g) * 10).to(DEV)
    if in_bf16:
        x = x.to(torch.bfloat16)
    mode = qimg.FP8_HADAMARD if fp8 else qimg.INT8_HADAMARD
    q_all, s_all = qimg.quantize_activation_hadamard(x, hbs, mode=mode)
    q_a, s_a = qimg.quantize_activation_hadamard(x[:MI], hbs, mode=mode)
    q_b, s_b = qimg.quantize_activation_hadamard(x[MI:], hbs, mode=mode)
    torch.cuda.synchronize()
    assert torch.equal(s_all, torch.cat([s_a, s_b]))
    assert torch.equal(q_all.view(torch.uint8), torch.cat([q_a.view(torch.uint8), q_b.view(torch.uint8)]))


def test_quant_repeatable_and_empty(qimg):
    x = torch.randn(64, 3072, device=DEV)
    a = qimg.quantize_activation_hadamard(x, 1024)
    b = qimg.quantize_activation_hadamard(x, 1024)
    torch.cuda.synchronize()
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    e = qimg.quantize_activation_hadamard(torch.empty(0, 3072, device=DEV), 1024)
    assert e[0].shape == (0, 3072)
