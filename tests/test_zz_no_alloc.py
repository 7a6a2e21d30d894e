"""qimg_linear_noalloc (the allocation-free quantized linear) through the C
ABI, against qimg_linear (the caller-scratch entry point that runs the same
kernels) on identical inputs: two calls in a row, the second smaller, each
equal bit for bit; no device memory taken by the calls; sizes beyond the
static scratch rejected before any launch."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _ptr(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _noalloc(qimg, x, qw, bias, out, gelu):
    L = qimg.lib()
    M, K = x.shape
    N = qw.data.shape[0]
    st = L.qimg_linear_noalloc(_ptr(x), qimg._DT[x.dtype], M, K, _ptr(qw.data), _ptr(qw.scales), N,
                               qw.had_block_size, qw.mode, _ptr(bias), _ptr(out), qimg._DT[out.dtype],
                               int(gelu), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    return st


def _case(qimg, g, M, K, N, mode, x_dtype, out_dtype, gelu):
    x = torch.randn(M, K, generator=g, device=DEV).to(x_dtype)
    w = (torch.randn(N, K, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    bias = (torch.randn(N, generator=g, device=DEV) * 0.01).to(torch.bfloat16)
    qw = qimg.quantize_weight_tensor(w, mode=mode)
    ref = qimg.linear_forward_quantized(x, qw, bias, apply_gelu=gelu, out_dtype=out_dtype)
    out = torch.full((M, N), float("nan"), dtype=out_dtype, device=DEV)
    return x, qw, bias, ref, out


def test_linear_noalloc_matches_linear(qimg):
    g = torch.Generator(device=DEV).manual_seed(7)
    # the MLP's fc2 input at 4352 tokens (53.5 MB of quantized activations,
    # close to the static array's size), then a smaller e4m3 linear with GELU
    big = _case(qimg, g, 4352, 12288, 3072, qimg.INT8_HADAMARD, torch.bfloat16, torch.float32, False)
    small = _case(qimg, g, 300, 3072, 1000, qimg.FP8_HADAMARD, torch.float32, torch.bfloat16, True)
    torch.cuda.synchronize()
    for x, qw, bias, ref, out in (big, small):
        assert _noalloc(qimg, x, qw, bias, out, gelu=qw.mode == qimg.FP8_HADAMARD) == 0, qimg.lib().qimg_last_error()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), (x.shape, qw.mode)
    # repeated calls take no device memory (the array was mapped with the
    # library's code object)
    x, qw, bias, ref, out = small
    free0 = torch.cuda.mem_get_info()[0]
    for _ in range(3):
        assert _noalloc(qimg, x, qw, bias, out, gelu=True) == 0
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0
    assert torch.equal(out, ref)


def test_linear_noalloc_rejects_oversize(qimg):
    L = qimg.lib()
    x = torch.zeros(8192, 12288, dtype=torch.bfloat16, device=DEV)
    qw = qimg.QuantizedWeight(torch.zeros(64, 12288, dtype=torch.int8, device=DEV),
                              torch.ones(64, device=DEV), 4096, qimg.INT8_HADAMARD)
    out = torch.zeros(8192, 64, device=DEV)
    assert _noalloc(qimg, x, qw, None, out, gelu=False) == 3
    assert b"static" in L.qimg_last_error()
    torch.cuda.synchronize()
    assert not out.any()
