"""C-ABI checks that need no GPU: the library loads, exports every symbol the
public header declares, and rejects bad arguments on the host before any HIP
call (status codes instead of the reference's abort)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qimg_hot.h")

FAKE = ctypes.c_void_p(0x10000)  # never dereferenced: validation fails first


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(qimg_[a-z0-9_]+)\s*\(", text)))


def test_header_symbols_exported(qimg):
    names = _declared()
    assert len(names) >= 17
    lib = ctypes.CDLL(qimg.LIB_PATH)
    for n in names:
        assert hasattr(lib, n), f"{n} declared in qimg_hot.h but not exported"
    assert set(names) == set(qimg.EXPORTED)


def test_sizing_helpers(qimg):
    L = qimg.lib()
    assert L.qimg_hadamard_block_size(3072) == 1024
    assert L.qimg_hadamard_block_size(12288) == 4096
    # int8_scratch_bytes (cuda_kernels.cuh:311-319) at the C1 shape
    a = ((max(4096 * 3072, 4096 * 3072) * 4 + 255) & ~255) + ((4096 * 3072 + 255) & ~255) + ((4096 * 4 + 255) & ~255)
    assert L.qimg_int8_scratch_bytes(4096, 3072, 3072) == a
    assert L.qimg_sage_scratch_bytes(24, 4352, 128) > 2 * 24 * 4352 * 128
    assert L.qimg_status_string(3) == b"scratch too small"


def _err(qimg):
    return qimg.lib().qimg_last_error().decode()


def test_linear_rejects_bad_arguments(qimg):
    L = qimg.lib()
    # null input
    assert L.qimg_linear(None, 0, 4, 64, FAKE, FAKE, 8, 64, 0, None, FAKE, 0, 0, FAKE, 1 << 20, None) == 1
    # K not a multiple of hbs
    assert L.qimg_linear(FAKE, 0, 4, 96, FAKE, FAKE, 8, 64, 0, None, FAKE, 0, 0, FAKE, 1 << 20, None) == 1
    assert "multiple of hbs" in _err(qimg)
    # hbs not a power of two
    assert L.qimg_linear(FAKE, 0, 4, 96, FAKE, FAKE, 8, 96, 0, None, FAKE, 0, 0, FAKE, 1 << 20, None) == 1
    # bad dtype / mode / out dtype
    assert L.qimg_linear(FAKE, 3, 4, 64, FAKE, FAKE, 8, 64, 0, None, FAKE, 0, 0, FAKE, 1 << 20, None) == 1
    assert L.qimg_linear(FAKE, 0, 4, 64, FAKE, FAKE, 8, 64, 7, None, FAKE, 0, 0, FAKE, 1 << 20, None) == 1
    assert L.qimg_linear(FAKE, 0, 4, 64, FAKE, FAKE, 8, 64, 0, None, FAKE, 2, 0, FAKE, 1 << 20, None) == 1
    # undersized scratch
    assert L.qimg_linear(FAKE, 0, 4, 64, FAKE, FAKE, 8, 64, 0, None, FAKE, 0, 0, FAKE, 16, None) == 3
    assert "scratch" in _err(qimg)
    # fp8 needs K % 64 == 0
    assert L.qimg_linear(FAKE, 0, 4, 48, FAKE, FAKE, 8, 16, 1, None, FAKE, 0, 0, FAKE, 1 << 20, None) == 2
    # row too long for the fused kernel
    assert L.qimg_linear(FAKE, 0, 4, 65536, FAKE, FAKE, 8, 65536, 0, None, FAKE, 0, 0, FAKE, 1 << 30, None) == 2
    # empty problem is a no-op success
    assert L.qimg_linear(FAKE, 0, 0, 64, FAKE, FAKE, 8, 64, 0, None, FAKE, 0, 0, FAKE, 0, None) == 0


def test_prequantized_rejects_bad_arguments(qimg):
    L = qimg.lib()
    assert L.qimg_linear_prequantized(None, FAKE, 4, 64, FAKE, FAKE, 8, 0, None, FAKE, 0, 0, None) == 1
    assert L.qimg_linear_prequantized(FAKE, FAKE, -1, 64, FAKE, FAKE, 8, 0, None, FAKE, 0, 0, None) == 1
    assert L.qimg_linear_prequantized(ctypes.c_void_p(0x10004), FAKE, 4, 128, FAKE, FAKE, 8, 0, None, FAKE,
                                      0, 0, None) == 1
    assert "aligned" in _err(qimg)
    assert L.qimg_linear_prequantized(FAKE, FAKE, 4, 96, FAKE, FAKE, 8, 1, None, FAKE, 0, 0, None) == 2


def test_quantize_rejects_bad_arguments(qimg):
    L = qimg.lib()
    assert L.qimg_quantize_activation(FAKE, 2, 4, 64, 64, 0, FAKE, FAKE, None) == 1   # fp16 input
    assert L.qimg_quantize_activation(FAKE, 0, 4, 64, 3, 0, FAKE, FAKE, None) == 1    # hbs not pow2
    assert L.qimg_quantize_activation(FAKE, 0, 4, 64, 128, 0, FAKE, FAKE, None) == 1  # hbs > K
    assert L.qimg_quantize_weight(FAKE, 1, 0, 64, 0, FAKE, FAKE, None, None) == 1
    assert L.qimg_fwht_inplace(None, 4, 64, 64, None) == 1
    assert L.qimg_quantize_per_row_fp32(FAKE, None, FAKE, 4, 64, None) == 1
    # every device pointer must be 16-byte aligned
    odd = ctypes.c_void_p(0x10004)
    assert L.qimg_quantize_activation(odd, 0, 4, 64, 64, 0, FAKE, FAKE, None) == 1
    assert "aligned" in _err(qimg)
    assert L.qimg_quantize_weight(FAKE, 1, 8, 64, 0, odd, FAKE, None, None) == 1
    assert L.qimg_linear(FAKE, 0, 4, 64, odd, FAKE, 8, 64, 0, None, FAKE, 0, 0, FAKE, 1 << 20, None) == 1
    assert L.qimg_linear_prequantized(FAKE, FAKE, 4, 128, FAKE, FAKE, 8, 0, None, odd, 0, 0, None) == 1
    assert L.qimg_sage_k_mean(odd, FAKE, 1, 64, 128, None) == 1
    assert L.qimg_fwht_inplace(odd, 4, 64, 64, None) == 1


def test_linear_noalloc_rejects_oversize_on_the_host(qimg):
    """M*K beyond the static scratch is refused before any HIP call."""
    L = qimg.lib()
    assert L.qimg_linear_noalloc(FAKE, 1, 8192, 12288, FAKE, FAKE, 64, 4096, 0, None, FAKE, 0, 0, None) == 3
    assert "static" in _err(qimg)
    assert L.qimg_linear_noalloc(None, 1, 8, 64, FAKE, FAKE, 64, 64, 0, None, FAKE, 0, 0, None) == 1
    assert L.qimg_linear_noalloc(FAKE, 1, 0, 64, FAKE, FAKE, 64, 64, 0, None, FAKE, 0, 0, None) == 0


def test_sage_rejects_bad_arguments(qimg):
    L = qimg.lib()
    args = (FAKE, FAKE, FAKE, FAKE, 0)
    assert L.qimg_sage_attention(*args, ctypes.c_float(0.1), 2, 64, 96, 0, FAKE, 1 << 30, None) == 2
    assert "head_dim" in _err(qimg)
    assert L.qimg_sage_attention(*args, ctypes.c_float(0.1), 0, 64, 128, 0, FAKE, 1 << 30, None) == 1
    assert L.qimg_sage_attention(*args, ctypes.c_float(0.1), 2, 64, 128, 0, FAKE, 100, None) == 3
    assert L.qimg_sage_attention(FAKE, FAKE, FAKE, FAKE, 4, ctypes.c_float(0.1), 2, 64, 128, 0, FAKE,
                                 1 << 30, None) == 1
    assert L.qimg_sage_attn_quantized(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 0, 2, 64, 128, ctypes.c_float(0.1), 0,
                                      FAKE, 10, None) == 3
    assert L.qimg_sage_quant_q(None, FAKE, FAKE, 1, 64, 128, None) == 1
    assert L.qimg_sage_k_mean(FAKE, FAKE, 1, 64, 32, None) == 2


def test_block_wrappers_refuse_operands_of_other_sizes(qimg):
    """The block entry points read the RoPE table at all n_img + n_txt
    positions (and img / txt / t_emb at the sizes the token counts give):
    the Python wrappers refuse a table made for another grid before any call
    into the library. 64 image tokens are an 8 x 8 latent grid, i.e.
    qwen_image_pe(16, 16, 2, n_txt); (8, 8) gives 16 positions."""
    import torch

    img = torch.zeros((2, 64, 3072))
    txt = torch.zeros((2, 16, 3072))
    t_emb = torch.zeros(3072)
    short = torch.from_numpy(qimg.qwen_image_pe(8, 8, 2, 16))
    good = torch.from_numpy(qimg.qwen_image_pe(16, 16, 2, 16))
    assert good.shape[0] == 80 and short.shape[0] == 32
    with pytest.raises(ValueError, match="pe has 8192 elements, 20480 expected"):
        qimg.mmdit_blocks_forward(None, img, txt, t_emb, short)
    with pytest.raises(ValueError, match="pe has"):
        qimg.mmdit_block_forward({}, {}, {}, img[0], txt[0], t_emb, short)
    with pytest.raises(ValueError, match="t_emb has"):
        qimg.mmdit_blocks_forward(None, img, txt, torch.zeros(3071), good)
    with pytest.raises(ValueError, match="float32"):
        qimg.mmdit_blocks_forward(None, img, txt, t_emb, good.double())
