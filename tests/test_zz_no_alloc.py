"""qimg_linear_noalloc (the allocation-free quantized linear) through the C
ABI, against qimg_linear (the caller-scratch entry point that runs the same
kernels) on identical inputs: two calls in a row, the second smaller, each
equal bit for bit; the call captured in a graph in global capture mode
(which any allocation during the capture fails) and replayed between eager
calls; sizes beyond the static scratch rejected before any launch."""
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
    # The call is captured into a graph in global capture mode, where an
    # allocation (hipMalloc, hipFree) by this process during the capture
    # fails it: so the call allocates nothing, whatever other processes on
    # the GPU do. Each replay, with eager work on the same buffers between
    # the replays, gives the eager result again.
    x, qw, bias, ref, out = small
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, capture_error_mode="global"):
        st = _noalloc(qimg, x, qw, bias, out, gelu=True)
    assert st == 0, qimg.lib().qimg_last_error()
    for i in range(3):
        out.fill_(float("nan"))
        big[4].fill_(0.0)
        assert _noalloc(qimg, *big[:3], big[4], gelu=False) == 0  # eager use of the same static array
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), i
        assert torch.equal(big[4], big[3]), i


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
