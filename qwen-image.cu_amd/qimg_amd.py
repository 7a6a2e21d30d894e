"""Python binding of the gfx950 hot-path library (lib/libqimg_hot.so).

Mirrors the reference's operator surface (cuda_kernels.cuh) on torch device
tensors: names, argument meaning and error behaviour follow the reference,
except that failures raise QimgError instead of aborting the process.

There is no CPU fallback: every operator runs the HIP kernels, and importing
this module fails loudly when the library has not been built.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libqimg_hot.so")

QIMG_OK, QIMG_ERR_INVALID_ARG, QIMG_ERR_UNSUPPORTED, QIMG_ERR_SCRATCH, QIMG_ERR_HIP = range(5)
FP32, BF16, FP16, INT8, INT32, FP8_E4M3 = range(6)
INT8_HADAMARD, FP8_HADAMARD = 0, 1
(LINEAR_AUTO, LINEAR_LARGE_TILE, LINEAR_SMALL_32, LINEAR_SMALL_64, LINEAR_GEMV, LINEAR_LARGE_192,
 LINEAR_LARGE_224, LINEAR_LARGE_128) = range(8)

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float

_SIGS = {
    "qimg_status_string": (ctypes.c_char_p, [_I]),
    "qimg_last_error": (ctypes.c_char_p, []),
    "qimg_version": (ctypes.c_char_p, []),
    "qimg_hadamard_block_size": (_I, [_I]),
    "qimg_int8_scratch_bytes": (_I64, [_I, _I, _I]),
    "qimg_fwht_inplace": (_I, [_P, _I, _I, _I, _P]),
    "qimg_quantize_per_row_fp32": (_I, [_P, _P, _P, _I, _I, _P]),
    "qimg_quantize_activation": (_I, [_P, _I, _I, _I, _I, _I, _P, _P, _P]),
    "qimg_quantize_weight": (_I, [_P, _I, _I, _I, _I, _P, _P, ctypes.POINTER(_I), _P]),
    "qimg_linear_prequantized": (_I, [_P, _P, _I, _I, _P, _P, _I, _I, _P, _P, _I, _I, _P]),
    "qimg_dequantize_bias": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _P]),
    "qimg_set_linear_kernel": (_I, [_I]),
    "qimg_get_linear_kernel": (_I, []),
    "qimg_linear": (_I, [_P, _I, _I, _I, _P, _P, _I, _I, _I, _P, _P, _I, _I, _P, _I64, _P]),
    "qimg_linear_noalloc": (_I, [_P, _I, _I, _I, _P, _P, _I, _I, _I, _P, _P, _I, _I, _P]),
    "qimg_linear_bf16": (_I, [_P, _I, _I, _I, _P, _I, _P, _P, _I, _P]),
    "qimg_dequantize_int4_bf16": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _P]),
    "qimg_quantize_int4_per_group": (_I, [_P, _P, _P, _I, _I, _I, _I, _P]),
    "qimg_quantize_activation_int4": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "qimg_fused_smooth_bf16_quant": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _P]),
    "qimg_w4a4_gemm": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P]),
    "qimg_int4_scratch_bytes": (_I64, [_I, _I, _I, _I]),
    "qimg_linear_int4": (_I, [_P, _I, _P, _P, _P, _I, _P, _I64, _P]),
    "qimg_bf16_to_fp32": (_I, [_P, _P, _I64, _P]),
    "qimg_smooth_hadamard": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "qimg_awq_repack": (_I, [_P, _P, _I, _I, _P]),
    "qimg_dequantize_awq_bf16": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "qimg_linear_awq": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "qimg_unswizzle_nunchaku_weights": (_I, [_P, _P, _P, _P, _I, _I, _I, _P]),
    "qimg_dequantize_nunchaku_bf16": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "qimg_unswizzle_lora_weights": (_I, [_P, _P, _I, _I, _I, _P]),
    "qimg_sage_scratch_bytes": (_I64, [_I, _I, _I]),
    "qimg_sage_k_mean": (_I, [_P, _P, _I, _I, _I, _P]),
    "qimg_sage_quant_q": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "qimg_sage_quant_k": (_I, [_P, _P, _P, _P, _I, _I, _I, _P]),
    "qimg_sage_attn_quantized": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _P, _I64, _P]),
    "qimg_sage_attention": (_I, [_P, _P, _P, _P, _I, _F, _I, _I, _I, _I, _P, _I64, _P]),
    "qimg_silu": (_I, [_P, _P, _I64, _P]),
    "qimg_layernorm_modulate": (_I, [_P, _P, _P, _P, _I, _I, _F, _P]),
    "qimg_layernorm_modulate_quant": (_I, [_P, _P, _P, _I, _I, _I, _I, _F, _P, _P, _P]),
    "qimg_joint_heads_f16": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _F, _P]),
    "qimg_split_heads": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "qimg_gate_add": (_I, [_P, _P, _P, _P, _I, _I, _P]),
    "qimg_mmdit_block_scratch_bytes": (_I64, [_I, _I]),
    "qimg_mmdit_block_forward": (_I, [_P, _P, _P, _P, _P, _I, _I, _P, _I64, _P, _P]),
    "qimg_mmdit_blocks_scratch_bytes": (_I64, [_I, _I, _I]),
    "qimg_mmdit_blocks_forward": (_I, [_P, _I, _P, _P, _P, _P, _I, _I, _I, _P, _I64, _P, _P]),
}

EXPORTED = tuple(_SIGS)


class QimgError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"[{status}] {message}")
        self.status = status


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    if not os.path.exists(path):
        raise ImportError(f"{path} is missing: build it with qwen-image.cu_amd/build.py "
                          "(or __graft_entry__.build())")
    lib = ctypes.CDLL(path)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_lib = load_library()


def lib() -> ctypes.CDLL:
    return _lib


# ---- quantized checkpoint files (include/qimg_ckpt.h, libqimg_host.so) ----
HOST_LIB_PATH = os.path.join(os.path.dirname(LIB_PATH), "libqimg_host.so")
_CS = ctypes.c_char_p
_CKPT_SIGS = {
    "qimg_st_writer_new": (_P, []),
    "qimg_st_writer_add": (_I, [_P, _CS, _CS, _P, _I, _P, ctypes.c_size_t]),
    "qimg_st_writer_write": (_I, [_P, _CS]),
    "qimg_st_writer_free": (None, [_P]),
    "qimg_checkpoint_kind": (_I, [_CS, _CS, _I]),
    "qimg_quantize_checkpoint": (_I, [_CS, _CS, _I, _I, _CS, _I]),
}
CKPT_EXPORTED = tuple(_CKPT_SIGS)
CHECKPOINT_KINDS = {0: "bf16", 1: "int8", 2: "fp8"}
_host = None


def host_lib() -> ctypes.CDLL:
    global _host
    if _host is None:
        if not os.path.exists(HOST_LIB_PATH):
            raise ImportError(f"{HOST_LIB_PATH} is missing: build it with qwen-image.cu_amd/build.py")
        h = ctypes.CDLL(HOST_LIB_PATH)
        for name, (res, args) in _CKPT_SIGS.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _host = h
    return _host


def write_safetensors(path: str, tensors) -> None:
    """tensors: iterable of (name, dtype string, shape, bytes-like), written
    in that order with the reference's safetensors writer layout."""
    h = host_lib()
    w = h.qimg_st_writer_new()
    if not w:
        raise MemoryError("qimg_st_writer_new")
    try:
        for name, dtype, shape, data in tensors:
            buf = bytes(data)
            shp = (ctypes.c_int64 * max(1, len(shape)))(*shape)
            if h.qimg_st_writer_add(w, name.encode(), dtype.encode(), shp, len(shape), buf, len(buf)) != 0:
                raise ValueError(f"qimg_st_writer_add rejected {name!r}")
        if h.qimg_st_writer_write(w, path.encode()) != 0:
            raise OSError(f"failed to write {path}")
    finally:
        h.qimg_st_writer_free(w)


def checkpoint_kind(path: str) -> str:
    """'bf16', 'int8' or 'fp8' (transformer.h:146-156); raises ValueError on
    an unreadable or malformed checkpoint or an unknown dtype."""
    err = ctypes.create_string_buffer(512)
    k = host_lib().qimg_checkpoint_kind(path.encode(), err, len(err))
    if k < 0:
        raise ValueError(err.value.decode())
    return CHECKPOINT_KINDS[k]


def quantize_checkpoint(in_path: str, out_path: str, mode: int = INT8_HADAMARD,
                        num_blocks: int = 60) -> None:
    """The offline quantizer (quantize.cu): BF16 checkpoint -> I8 / F8_E4M3 +
    .__scales__ on the current device."""
    err = ctypes.create_string_buffer(1024)
    if host_lib().qimg_quantize_checkpoint(in_path.encode(), out_path.encode(), mode, num_blocks, err,
                                           len(err)) != 0:
        raise ValueError(err.value.decode())


def _check(status: int) -> None:
    if status != QIMG_OK:
        raise QimgError(status, _lib.qimg_last_error().decode())


def _ptr(t):
    if t is None:
        return None
    return ctypes.c_void_p(t.data_ptr())


def _stream(device=None):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


_DT = {torch.float32: FP32, torch.bfloat16: BF16, torch.float16: FP16, torch.int8: INT8,
       torch.int32: INT32, torch.float8_e4m3fn: FP8_E4M3, torch.uint8: FP8_E4M3}
_TORCH = {FP32: torch.float32, BF16: torch.bfloat16, FP16: torch.float16}


def _dev(t: torch.Tensor, name: str):
    if not t.is_cuda:
        raise QimgError(QIMG_ERR_INVALID_ARG, f"{name} must be a device tensor")
    if not t.is_contiguous():
        raise QimgError(QIMG_ERR_INVALID_ARG, f"{name} must be contiguous")


# --------------------------------------------------------------- helpers
def hadamard_block_size(K: int) -> int:
    """cuda_kernels.cuh:253"""
    return int(_lib.qimg_hadamard_block_size(int(K)))


def int8_scratch_bytes(M: int, K: int, N: int) -> int:
    """cuda_kernels.cuh:311-319"""
    return int(_lib.qimg_int8_scratch_bytes(int(M), int(K), int(N)))


@dataclass
class QuantizedWeight:
    """cuda_kernels.cuh:187-245 (the INT8/FP8 fields)."""
    data: torch.Tensor       # [N, K] int8 (INT8_HADAMARD) or uint8 e4m3 bits (FP8_HADAMARD)
    scales: torch.Tensor     # [N] fp32
    had_block_size: int
    mode: int = INT8_HADAMARD


# --------------------------------------------------------- quantization
def fwht_inplace(data: torch.Tensor, had_block_size: int) -> torch.Tensor:
    """cuda_kernels.cu:2209-2254 on fp32 [M, K] rows, in place."""
    _dev(data, "data")
    M, K = data.shape
    _check(_lib.qimg_fwht_inplace(_ptr(data), M, K, int(had_block_size), _stream()))
    return data


def quantize_per_row_fp32(x: torch.Tensor):
    """cuda_kernels.cu:2385-2416 -> (int8 [M,K], fp32 [M])."""
    _dev(x, "x")
    M, K = x.shape
    q = torch.empty((M, K), dtype=torch.int8, device=x.device)
    s = torch.empty((M,), dtype=torch.float32, device=x.device)
    _check(_lib.qimg_quantize_per_row_fp32(_ptr(x), _ptr(q), _ptr(s), M, K, _stream()))
    return q, s


def quantize_activation_hadamard(x: torch.Tensor, had_block_size: int, mode: int = INT8_HADAMARD):
    """quantize_activation_int8_hadamard_{fp32,bf16} (cuda_kernels.cu:2603-2619);
    FP8_HADAMARD gives e4m3 bytes (uint8) with scale amax/448."""
    _dev(x, "x")
    M, K = x.shape
    qdt = torch.int8 if mode == INT8_HADAMARD else torch.uint8
    q = torch.empty((M, K), dtype=qdt, device=x.device)
    s = torch.empty((M,), dtype=torch.float32, device=x.device)
    _check(_lib.qimg_quantize_activation(_ptr(x), _DT[x.dtype], M, K, int(had_block_size), int(mode),
                                         _ptr(q), _ptr(s), _stream()))
    return q, s


def quantize_weight_tensor(w: torch.Tensor, mode: int = INT8_HADAMARD) -> QuantizedWeight:
    """cuda_kernels.cu:2830-2862: bf16 [N,K] -> FWHT(K & -K) -> per-row quant."""
    _dev(w, "weight")
    N, K = w.shape
    qdt = torch.int8 if mode == INT8_HADAMARD else torch.uint8
    q = torch.empty((N, K), dtype=qdt, device=w.device)
    s = torch.empty((N,), dtype=torch.float32, device=w.device)
    hbs = _I(0)
    _check(_lib.qimg_quantize_weight(_ptr(w), _DT[w.dtype], N, K, int(mode), _ptr(q), _ptr(s),
                                     ctypes.byref(hbs), _stream()))
    return QuantizedWeight(q, s, int(hbs.value), mode)


# ---------------------------------------------------------------- linear
def linear_forward_prequantized(act_q: torch.Tensor, act_scales: torch.Tensor, weight: QuantizedWeight,
                                bias: torch.Tensor | None = None, apply_gelu: bool = False,
                                out: torch.Tensor | None = None, out_dtype=torch.float32) -> torch.Tensor:
    """linear_forward_int8_prequantized (cuda_kernels.cu:2734-2773), epilogue fused."""
    _dev(act_q, "act_q")
    M, K = act_q.shape
    N = weight.data.shape[0]
    if weight.data.shape[1] != K:
        raise QimgError(QIMG_ERR_INVALID_ARG, f"weight K {weight.data.shape[1]} != activation K {K}")
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=act_q.device)
    _check(_lib.qimg_linear_prequantized(_ptr(act_q), _ptr(act_scales), M, K, _ptr(weight.data),
                                         _ptr(weight.scales), N, int(weight.mode), _ptr(bias), _ptr(out),
                                         _DT[out.dtype], int(bool(apply_gelu)), _stream()))
    return out


def set_linear_kernel(which: int) -> int:
    """Select the quantized-linear kernel process-wide (LINEAR_AUTO,
    LINEAR_LARGE_TILE, LINEAR_SMALL_32, LINEAR_SMALL_64, LINEAR_GEMV,
    LINEAR_LARGE_192, LINEAR_LARGE_224, LINEAR_LARGE_128); returns the previous choice. Every
    choice gives the same int8 results."""
    prev = int(_lib.qimg_get_linear_kernel())
    _check(_lib.qimg_set_linear_kernel(int(which)))
    return prev


class linear_kernel:
    """Context manager: run the enclosed linears with one kernel choice."""

    def __init__(self, which: int):
        self.which = which
        self.prev = None

    def __enter__(self):
        self.prev = set_linear_kernel(self.which)
        return self

    def __exit__(self, *exc):
        set_linear_kernel(self.prev)
        return False


def dequantize_and_bias(acc: torch.Tensor, act_scales: torch.Tensor, w_scales: torch.Tensor,
                        bias: torch.Tensor | None = None, apply_gelu: bool = False) -> torch.Tensor:
    """dequantize_and_bias / dequantize_bias_gelu (cuda_kernels.cu:2623-2668):
    int32 [M,N] -> fp32 [M,N]."""
    _dev(acc, "acc")
    M, N = acc.shape
    out = torch.empty((M, N), dtype=torch.float32, device=acc.device)
    _check(_lib.qimg_dequantize_bias(_ptr(acc), _ptr(act_scales), _ptr(w_scales), _ptr(bias), _ptr(out), M, N,
                                     int(bool(apply_gelu)), _stream()))
    return out


def linear_forward_quantized(x: torch.Tensor, weight: QuantizedWeight, bias: torch.Tensor | None = None,
                             out: torch.Tensor | None = None, scratch: torch.Tensor | None = None,
                             apply_gelu: bool = False, out_dtype=torch.float32) -> torch.Tensor:
    """linear_forward_quantized / _bf16in (cuda_kernels.cu:4599-4635) for the
    INT8/FP8 Hadamard modes: x fp32 or bf16 [M,K] -> out [M,N]."""
    _dev(x, "x")
    M, K = x.shape
    N = weight.data.shape[0]
    if weight.data.shape[1] != K:
        raise QimgError(QIMG_ERR_INVALID_ARG, f"weight K {weight.data.shape[1]} != activation K {K}")
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=x.device)
    if scratch is None:
        scratch = torch.empty((int8_scratch_bytes(M, K, N),), dtype=torch.uint8, device=x.device)
    _check(_lib.qimg_linear(_ptr(x), _DT[x.dtype], M, K, _ptr(weight.data), _ptr(weight.scales), N,
                            int(weight.had_block_size), int(weight.mode), _ptr(bias), _ptr(out),
                            _DT[out.dtype], int(bool(apply_gelu)), _ptr(scratch), scratch.numel(),
                            _stream()))
    return out


def linear_forward_bf16(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None,
                        apply_gelu: bool = False, out: torch.Tensor | None = None) -> torch.Tensor:
    """linear_forward_bf16 / _bf16in (cuda_kernels.cu:4534-4596), the
    QuantMode::BF16 path: x fp32 (rounded to bf16 in the kernel) or bf16
    [M,K], weight bf16 [N,K], bias bf16 [N] -> fp32 [M,N] (+ GELU-tanh)."""
    _dev(x, "x")
    _dev(weight, "weight")
    if weight.dtype != torch.bfloat16:
        raise QimgError(QIMG_ERR_INVALID_ARG, "weight must be bfloat16")
    M, K = x.shape
    N = weight.shape[0]
    if weight.shape[1] != K:
        raise QimgError(QIMG_ERR_INVALID_ARG, f"weight K {weight.shape[1]} != activation K {K}")
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32, device=x.device)
    _check(_lib.qimg_linear_bf16(_ptr(x), _DT[x.dtype], M, K, _ptr(weight), N, _ptr(bias), _ptr(out),
                                 int(bool(apply_gelu)), _stream()))
    return out


# ------------------------------------------------------------- INT4 paths
def dequantize_int4_to_bf16(qweight: torch.Tensor, scales: torch.Tensor, K: int, group_size: int,
                            nf4_grid: bool = True, scales_gn: bool = False, signed_int4: bool = False) -> torch.Tensor:
    """dequantize_int4_to_bf16 (cuda_kernels.cu:2876-2929): packed [N, K/2]
    uint8 -> bf16 [N, K]."""
    _dev(qweight, "qweight")
    N = qweight.shape[0]
    out = torch.empty((N, K), dtype=torch.bfloat16, device=qweight.device)
    _check(_lib.qimg_dequantize_int4_bf16(_ptr(qweight), _ptr(scales), _ptr(out), N, K, group_size, int(nf4_grid),
                                          int(scales_gn), int(signed_int4), _stream()))
    return out


def quantize_int4_per_group(residual: torch.Tensor, group_size: int, nf4_grid: bool = True):
    """quantize_int4_per_group (NF4, cuda_kernels.cu:3290-3368) or the linear
    INT4 quantizer (:3226-3288): fp32 [N, K] -> (packed [N, K/2], scales [N, K/gs])."""
    _dev(residual, "residual")
    N, K = residual.shape
    qw = torch.empty((N, K // 2), dtype=torch.uint8, device=residual.device)
    sc = torch.empty((N, K // group_size), dtype=torch.float32, device=residual.device)
    _check(_lib.qimg_quantize_int4_per_group(_ptr(residual), _ptr(qw), _ptr(sc), N, K, group_size, int(nf4_grid),
                                             _stream()))
    return qw, sc


def quantize_activation_int4(x: torch.Tensor, group_size: int, smooth: torch.Tensor | None = None,
                             want_bf16: bool = False):
    """quantize_activation_int4 (cuda_kernels.cu:3575-3648) or, with smooth /
    the bf16 copy, fused_smooth_bf16_quant (:3650-3730): fp32 [M, K] ->
    (packed [M, K/2], scales [K/gs, M][, bf16 [M, K]])."""
    _dev(x, "x")
    M, K = x.shape
    pk = torch.empty((M, K // 2), dtype=torch.uint8, device=x.device)
    sc = torch.empty((K // group_size, M), dtype=torch.float32, device=x.device)
    if smooth is None and not want_bf16:
        _check(_lib.qimg_quantize_activation_int4(_ptr(x), _ptr(pk), _ptr(sc), M, K, group_size, _stream()))
        return pk, sc
    bf = torch.empty((M, K), dtype=torch.bfloat16, device=x.device)
    _check(_lib.qimg_fused_smooth_bf16_quant(_ptr(x), _ptr(smooth), _ptr(bf), _ptr(pk), _ptr(sc), M, K, group_size,
                                             _stream()))
    return pk, sc, bf


def w4a4_gemm(act_packed: torch.Tensor, wgt_packed: torch.Tensor, act_scales: torch.Tensor, wgt_scales: torch.Tensor,
              K: int, group_size: int, bias: torch.Tensor | None = None, out: torch.Tensor | None = None,
              accumulate: bool = False) -> torch.Tensor:
    """w4a4_gemm (cuda_kernels.cu:4257-4313) over row-major packed weights."""
    _dev(act_packed, "act_packed")
    M, N = act_packed.shape[0], wgt_packed.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32, device=act_packed.device)
    _check(_lib.qimg_w4a4_gemm(_ptr(act_packed), _ptr(wgt_packed), _ptr(act_scales), _ptr(wgt_scales), _ptr(out), M, N,
                               K, group_size, int(bool(accumulate)), _ptr(bias), _stream()))
    return out


class _Int4Weight(ctypes.Structure):
    _fields_ = [("N", _I), ("K", _I), ("rank", _I), ("group_size", _I), ("nf4_grid", _I), ("had_block_size", _I),
                ("qweight", _P), ("scales4", _P), ("w4a4_qweight", _P), ("w4a4_wscales", _P), ("svd_up", _P),
                ("svd_down", _P), ("smooth", _P), ("w4a16_nunchaku", _I)]


class Int4Weight:
    """The INT4_SVD fields of QuantizedWeight (cuda_kernels.cuh:194-213).
    W4A4 when w4a4_qweight (two's complement [N, K/2]) and w4a4_wscales
    ([K/gs, N]) are given, else W4A16 over qweight / scales4 ([N, K/gs]).
    w4a16_nunchaku: the reference's W4A16 fallback for nunchaku weights
    (cuda_kernels.cu:4443-4470): qweight holds two's complement nibbles,
    scales4 is [K/gs, N], and x is not rotated."""

    def __init__(self, N, K, group_size, svd_up=None, svd_down=None, qweight=None, scales4=None, nf4_grid=True,
                 had_block_size=1, w4a4_qweight=None, w4a4_wscales=None, smooth=None, w4a16_nunchaku=False):
        self.N, self.K, self.group_size = N, K, group_size
        self.svd_up, self.svd_down = svd_up, svd_down
        self.rank = 0 if svd_up is None else int(svd_up.shape[1])
        self.qweight, self.scales4, self.nf4_grid, self.had_block_size = qweight, scales4, nf4_grid, had_block_size
        self.w4a4_qweight, self.w4a4_wscales, self.smooth = w4a4_qweight, w4a4_wscales, smooth
        self.w4a16_nunchaku = w4a16_nunchaku

    def struct(self) -> _Int4Weight:
        def p(t):
            return None if t is None else t.data_ptr()
        return _Int4Weight(self.N, self.K, self.rank, self.group_size, int(bool(self.nf4_grid)),
                           int(self.had_block_size), p(self.qweight), p(self.scales4), p(self.w4a4_qweight),
                           p(self.w4a4_wscales), p(self.svd_up), p(self.svd_down), p(self.smooth),
                           int(bool(self.w4a16_nunchaku)))


def int4_scratch_bytes(M: int, K: int, N: int, svd_rank: int) -> int:
    """int4_scratch_bytes (cuda_kernels.cuh:475-487), or more where needed."""
    return int(_lib.qimg_int4_scratch_bytes(M, K, N, svd_rank))


def linear_forward_int4(x: torch.Tensor, weight: Int4Weight, bias: torch.Tensor | None = None,
                        apply_gelu: bool = False, out: torch.Tensor | None = None,
                        scratch: torch.Tensor | None = None) -> torch.Tensor:
    """linear_forward_int4 (cuda_kernels.cu:4332-4532): x fp32 [M, K] -> fp32 [M, N]."""
    _dev(x, "x")
    if x.dtype != torch.float32:
        raise QimgError(QIMG_ERR_INVALID_ARG, "x must be float32")
    M, K = x.shape
    if K != weight.K:
        raise QimgError(QIMG_ERR_INVALID_ARG, f"weight K {weight.K} != activation K {K}")
    if out is None:
        out = torch.empty((M, weight.N), dtype=torch.float32, device=x.device)
    if scratch is None:
        scratch = torch.empty((int4_scratch_bytes(M, K, weight.N, weight.rank),), dtype=torch.uint8, device=x.device)
    st = weight.struct()
    _check(_lib.qimg_linear_int4(_ptr(x), M, ctypes.byref(st), _ptr(bias), _ptr(out), int(bool(apply_gelu)),
                                 _ptr(scratch), scratch.numel(), _stream()))
    return out


def smooth_hadamard(x: torch.Tensor, smooth: torch.Tensor | None, had_block_size: int,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """apply_smooth_div / smooth_hadamard_inplace (cuda_kernels.cu:2257-2324):
    FWHT_hbs(x / smooth) fp32 [M, K] (out may be x)."""
    _dev(x, "x")
    M, K = x.shape
    if out is None:
        out = torch.empty_like(x)
    _check(_lib.qimg_smooth_hadamard(_ptr(x), _ptr(smooth), _ptr(out), M, K, int(had_block_size), _stream()))
    return out


def repack_awq_to_transposed(qweight_awq: torch.Tensor, OC: int, IC: int) -> torch.Tensor:
    """repack_awq_to_transposed (cuda_kernels.cu:3059-3102): int32 [OC/4, IC/2] -> [IC/8, OC]."""
    _dev(qweight_awq, "qweight_awq")
    out = torch.empty((IC // 8, OC), dtype=torch.int32, device=qweight_awq.device)
    _check(_lib.qimg_awq_repack(_ptr(qweight_awq), _ptr(out), OC, IC, _stream()))
    return out


def dequantize_awq_to_bf16(qweight_awq, wscales, wzeros, OC, IC, group_size=64, num_components=6) -> torch.Tensor:
    """dequantize_awq_to_bf16 (cuda_kernels.cu:3002-3057): bf16 [OC, IC]."""
    _dev(qweight_awq, "qweight_awq")
    out = torch.empty((OC, IC), dtype=torch.bfloat16, device=qweight_awq.device)
    _check(_lib.qimg_dequantize_awq_bf16(_ptr(qweight_awq), _ptr(wscales), _ptr(wzeros), _ptr(out), OC, IC,
                                         group_size, num_components, _stream()))
    return out


def linear_forward_awq(x: torch.Tensor, qweight_repacked: torch.Tensor, wscales: torch.Tensor, wzeros: torch.Tensor,
                       OC: int, IC: int, bias: torch.Tensor | None = None, group_size: int = 64,
                       num_components: int = 6) -> torch.Tensor:
    """linear_forward_awq (cuda_kernels.cu:3155-3179): x fp32 [IC] (or [1, IC]) -> fp32 [1, OC]."""
    _dev(x, "x")
    out = torch.empty((1, OC), dtype=torch.float32, device=x.device)
    _check(_lib.qimg_linear_awq(_ptr(x), _ptr(qweight_repacked), _ptr(wscales), _ptr(wzeros), _ptr(bias), _ptr(out),
                                OC, IC, group_size, num_components, _stream()))
    return out


def unswizzle_nunchaku_weights(qweight_swizzled: torch.Tensor, wscales_swizzled: torch.Tensor, N: int, K: int,
                               num_groups: int):
    """unswizzle_nunchaku_weights (cuda_kernels.cu:3431-3499): -> (packed
    [N, K/2] uint8, fp32 scales [num_groups, N])."""
    _dev(qweight_swizzled, "qweight_swizzled")
    q = torch.empty((N, K // 2), dtype=torch.uint8, device=qweight_swizzled.device)
    sc = torch.empty((num_groups, N), dtype=torch.float32, device=qweight_swizzled.device)
    _check(_lib.qimg_unswizzle_nunchaku_weights(_ptr(qweight_swizzled), _ptr(wscales_swizzled), _ptr(q), _ptr(sc), N,
                                                K, num_groups, _stream()))
    return q, sc


def dequantize_nunchaku_to_bf16(qweight_swizzled, wscales_swizzled, N, K, num_groups) -> torch.Tensor:
    """dequantize_nunchaku_to_bf16 (cuda_kernels.cu:2932-2998): bf16 [N, K]."""
    _dev(qweight_swizzled, "qweight_swizzled")
    out = torch.empty((N, K), dtype=torch.bfloat16, device=qweight_swizzled.device)
    _check(_lib.qimg_dequantize_nunchaku_bf16(_ptr(qweight_swizzled), _ptr(wscales_swizzled), _ptr(out), N, K,
                                              num_groups, _stream()))
    return out


def unswizzle_lora_weights(packed: torch.Tensor, rows: int, cols: int, is_down: bool) -> torch.Tensor:
    """unswizzle_lora_weights (cuda_kernels.cu:3503-3572): bf16 [rows, cols]."""
    _dev(packed, "packed")
    out = torch.empty((rows, cols), dtype=torch.bfloat16, device=packed.device)
    _check(_lib.qimg_unswizzle_lora_weights(_ptr(packed), _ptr(out), rows, cols, int(bool(is_down)), _stream()))
    return out


# ---------------------------------------------------------- SageAttention
def sage_scratch_bytes(BH: int, S: int, D: int) -> int:
    return int(_lib.qimg_sage_scratch_bytes(BH, S, D))


def sage_k_mean(k: torch.Tensor) -> torch.Tensor:
    """sageattention_sm80.cu:759-773"""
    _dev(k, "k")
    BH, S, D = k.shape
    mean = torch.empty((BH, D), dtype=torch.float32, device=k.device)
    _check(_lib.qimg_sage_k_mean(_ptr(k), _ptr(mean), BH, S, D, _stream()))
    return mean


def sage_quant_q(q: torch.Tensor):
    """sageattention_sm80.cu:775-824"""
    _dev(q, "q")
    BH, S, D = q.shape
    qi = torch.empty((BH, S, D), dtype=torch.int8, device=q.device)
    qs = torch.empty((BH, (S + 127) // 128 * 32), dtype=torch.float32, device=q.device)
    _check(_lib.qimg_sage_quant_q(_ptr(q), _ptr(qi), _ptr(qs), BH, S, D, _stream()))
    return qi, qs


def sage_quant_k(k: torch.Tensor, mean: torch.Tensor):
    """sageattention_sm80.cu:826-886"""
    _dev(k, "k")
    BH, S, D = k.shape
    ki = torch.empty((BH, S, D), dtype=torch.int8, device=k.device)
    ks = torch.empty((BH, (S + 63) // 64 * 4), dtype=torch.float32, device=k.device)
    _check(_lib.qimg_sage_quant_k(_ptr(k), _ptr(mean), _ptr(ki), _ptr(ks), BH, S, D, _stream()))
    return ki, ks


def sage_attn_quantized(q_i8, k_i8, v, q_scale, k_scale, sm_scale, causal=False, out_dtype=torch.float16,
                        scratch=None):
    """qk_int_sv_f16_attn_kernel (sageattention_sm80.cu:47-674) on pre-quantized Q/K."""
    BH, S, D = q_i8.shape
    out = torch.empty((BH, S, D), dtype=out_dtype, device=q_i8.device)
    if scratch is None:
        scratch = torch.empty((sage_scratch_bytes(BH, S, D),), dtype=torch.uint8, device=q_i8.device)
    _check(_lib.qimg_sage_attn_quantized(_ptr(q_i8), _ptr(k_i8), _ptr(v), _ptr(q_scale), _ptr(k_scale),
                                         _ptr(out), _DT[out_dtype], BH, S, D, float(sm_scale),
                                         int(bool(causal)), _ptr(scratch), scratch.numel(), _stream()))
    return out


def attention_forward_sage_fp16io(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
                                  causal: bool = False, out: torch.Tensor | None = None,
                                  out_dtype=torch.float32, scratch: torch.Tensor | None = None):
    """attention_forward_sage_sm80_fp16io (sageattention_sm80.cu:965-1027):
    fp16 [BH,S,D] q,k,v -> out [BH,S,D] (fp32 by default, as the reference)."""
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _dev(t, n)
        if t.dtype != torch.float16:
            raise QimgError(QIMG_ERR_INVALID_ARG, f"{n} must be float16")
    BH, S, D = q.shape
    if out is None:
        out = torch.empty((BH, S, D), dtype=out_dtype, device=q.device)
    if scratch is None:
        scratch = torch.empty((max(sage_scratch_bytes(BH, S, D), 1),), dtype=torch.uint8, device=q.device)
    _check(_lib.qimg_sage_attention(_ptr(q), _ptr(k), _ptr(v), _ptr(out), _DT[out.dtype], float(scale),
                                    BH, S, D, int(bool(causal)), _ptr(scratch), scratch.numel(), _stream()))
    return out


# ------------------------------------------------------- MMDiT joint block
HIDDEN, HEADS, HEAD_DIM, MLP_DIM = 3072, 24, 128, 12288
PROF_CATEGORIES = ("modulation", "attn_norm", "qkv_gemm", "qk_norm", "concat_transpose", "rope", "attention",
                   "transpose_split", "out_gemm", "gate_attn", "mlp_norm", "mlp_gemm", "gate_mlp")


def silu(x: torch.Tensor) -> torch.Tensor:
    """silu_fp32 (cuda_kernels.cu:1881-1893)."""
    _dev(x, "x")
    out = torch.empty_like(x)
    _check(_lib.qimg_silu(_ptr(x), _ptr(out), x.numel(), _stream()))
    return out


def layer_norm_modulate(x: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """layer_norm_modulate_fp32 (cuda_kernels.cu:1799-1859): fp32 [rows, dim]."""
    _dev(x, "x")
    rows, dim = x.shape
    out = torch.empty_like(x)
    _check(_lib.qimg_layernorm_modulate(_ptr(x), _ptr(shift), _ptr(scale), _ptr(out), rows, dim, float(eps),
                                        _stream()))
    return out


def layer_norm_modulate_quant(x: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor, had_block_size: int,
                              mode: int = INT8_HADAMARD, eps: float = 1e-6):
    """layer_norm_modulate_fp32 then fwht_quantize_fp32 (cuda_kernels.cu:1799-1859,
    2493-2601) in one pass: (int8 or e4m3 bytes [rows, dim], fp32 scales [rows])."""
    _dev(x, "x")
    rows, dim = x.shape
    q = torch.empty((rows, dim), dtype=torch.int8 if mode == INT8_HADAMARD else torch.uint8, device=x.device)
    s = torch.empty((rows,), dtype=torch.float32, device=x.device)
    _check(_lib.qimg_layernorm_modulate_quant(_ptr(x), _ptr(shift), _ptr(scale), rows, dim, int(had_block_size),
                                              int(mode), float(eps), _ptr(q), _ptr(s), _stream()))
    return q, s


def joint_heads_f16(txt: torch.Tensor, img: torch.Tensor, norm_txt=None, norm_img=None, pe=None,
                    eps: float = 1e-6) -> torch.Tensor:
    """RMSNorm per head + txt-first concat + [S,H,D] -> [H,S,D] + RoPE -> fp16
    (cuda_kernels.cu:1656-1692, transformer.cu:106-130, cuda_kernels.cu:1935-1971).
    Without norm weights only the concat/transpose/fp16 (the V path)."""
    n_txt, n_img = txt.shape[0], img.shape[0]
    H = txt.shape[1] // HEAD_DIM
    out = torch.empty((H, n_txt + n_img, HEAD_DIM), dtype=torch.float16, device=txt.device)
    _check(_lib.qimg_joint_heads_f16(_ptr(txt), _ptr(img), _ptr(norm_txt), _ptr(norm_img), _ptr(pe), _ptr(out),
                                     n_txt, n_img, H, float(eps), _stream()))
    return out


def split_heads(attn: torch.Tensor, n_txt: int):
    """transpose_split_fused_fp32 (transformer.cu:84-104) from fp16 [H,S,128]."""
    H, S, _ = attn.shape
    txt = torch.empty((n_txt, H * HEAD_DIM), dtype=torch.float32, device=attn.device)
    img = torch.empty((S - n_txt, H * HEAD_DIM), dtype=torch.float32, device=attn.device)
    _check(_lib.qimg_split_heads(_ptr(attn), _ptr(txt), _ptr(img), n_txt, S - n_txt, H, _stream()))
    return txt, img


def gate_add(x: torch.Tensor, gate: torch.Tensor, y: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """gate_add_fp32f (cuda_kernels.cu:2181-2197): x + gate[c] * y."""
    rows, dim = x.shape
    if out is None:
        out = torch.empty_like(x)
    _check(_lib.qimg_gate_add(_ptr(x), _ptr(gate), _ptr(y), _ptr(out), rows, dim, _stream()))
    return out


def qwen_image_pe(h: int, w: int, patch_size: int = 2, context_len: int = 256, theta: float = 10000.0,
                  axes_dim=(16, 56, 56)):
    """RoPE::gen_qwen_image_pe (rope.h:154-160) for batch 1: [context_len +
    (h/p)*(w/p), 64, 4] float32 rows of (cos, -sin, sin, cos), text tokens
    first. Host-side, in float32 like the reference's std::vector<float>."""
    import numpy as np

    h_len = (h + patch_size // 2) // patch_size
    w_len = (w + patch_size // 2) // patch_size
    t0 = max(h_len, w_len)
    f32 = np.float32

    def linspace(a, b, n):
        if n == 1:
            return np.array([a], f32)
        step = f32((f32(b) - f32(a)) / f32(n - 1))
        return np.array([f32(a) + f32(i) * step for i in range(n)], f32)

    txt = linspace(t0, context_len + t0, context_len)
    ids = [np.stack([txt, txt, txt], 1)]
    rows = linspace(-(h_len // 2), -(h_len // 2) + h_len - 1, h_len)
    cols = linspace(-(w_len // 2), -(w_len // 2) + w_len - 1, w_len)
    img = np.zeros((h_len * w_len, 3), f32)
    img[:, 1] = np.repeat(rows, w_len)
    img[:, 2] = np.tile(cols, h_len)
    ids = np.concatenate(ids + [img], 0)
    parts = []
    for axis, dim in enumerate(axes_dim):
        half = dim // 2
        scale = linspace(0.0, (dim * 1.0 - 2.0) / dim, half)
        omega = np.array([f32(1.0) / f32(np.power(np.float32(theta), s, dtype=np.float32)) for s in scale], f32)
        ang = (ids[:, axis:axis + 1] * omega[None, :]).astype(f32)
        c, s = np.cos(ang).astype(f32), np.sin(ang).astype(f32)
        parts.append(np.stack([c, -s, s, c], -1))
    return np.ascontiguousarray(np.concatenate(parts, 1), dtype=np.float32)


class _QLinear(ctypes.Structure):
    _fields_ = [("w", _P), ("scales", _P), ("N", _I), ("K", _I), ("hbs", _I), ("mode", _I), ("bias", _P)]


_BLOCK_LINEARS = ("img_mod", "txt_mod", "to_q", "to_k", "to_v", "add_q_proj", "add_k_proj", "add_v_proj",
                  "to_out", "to_add_out", "img_mlp_fc1", "img_mlp_fc2", "txt_mlp_fc1", "txt_mlp_fc2")
_BLOCK_NORMS = ("norm_q", "norm_k", "norm_added_q", "norm_added_k")


class _Block(ctypes.Structure):
    _fields_ = [(n, _QLinear) for n in _BLOCK_LINEARS] + [(n, _P) for n in _BLOCK_NORMS]


def mmdit_block_scratch_bytes(n_img: int, n_txt: int, batch: int = 1) -> int:
    return int(_lib.qimg_mmdit_blocks_scratch_bytes(int(n_img), int(n_txt), int(batch)))


def _block_struct(weights: dict, biases: dict, norms: dict, b=None):
    b = _Block() if b is None else b
    for n in _BLOCK_LINEARS:
        qw = weights[n]
        N, K = qw.data.shape
        bias = biases.get(n)
        setattr(b, n, _QLinear(qw.data.data_ptr(), qw.scales.data_ptr(), N, K, int(qw.had_block_size),
                               int(qw.mode), bias.data_ptr() if bias is not None else None))
    for n in _BLOCK_NORMS:
        setattr(b, n, norms[n].data_ptr())
    return b


class BlockTable:
    """A C array of qimg_mmdit_block for a list of (weights, biases, norms)
    dicts, built once: the tensors must outlive the table."""

    def __init__(self, blocks):
        self.n = len(blocks)
        self.array = (_Block * self.n)()
        for i, (w, b, nr) in enumerate(blocks):
            _block_struct(w, b, nr, self.array[i])


def _check_block_operands(fn: str, img: torch.Tensor, txt: torch.Tensor, t_emb: torch.Tensor, pe: torch.Tensor,
                          n_img: int, n_txt: int, batch: int) -> None:
    """The block entry points take bare pointers and read every operand at
    the sizes the token counts imply (the RoPE table for all n_img + n_txt
    positions): a tensor of another size would be read out of bounds, so it
    is refused here."""
    want = {"img": (img, batch * n_img * 3072), "txt": (txt, batch * n_txt * 3072), "t_emb": (t_emb, 3072),
            "pe": (pe, (n_img + n_txt) * 64 * 4)}
    for name, (t, n) in want.items():
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError(f"{fn}: {name} must be a contiguous float32 tensor")
        if t.numel() != n:
            raise ValueError(f"{fn}: {name} has {t.numel()} elements, {n} expected"
                             + (f" (a RoPE table of {n_img + n_txt} positions x 64 x 4, qwen_image_pe)"
                                if name == "pe" else ""))
        if t.device != img.device:
            raise ValueError(f"{fn}: {name} is on {t.device}, img on {img.device}")


def mmdit_blocks_forward(table: "BlockTable", img: torch.Tensor, txt: torch.Tensor, t_emb: torch.Tensor,
                         pe: torch.Tensor, scratch: torch.Tensor | None = None, profile: bool = False):
    """The block loop (transformer.cu:497-836) over every block of `table`.
    img [batch, n_img, 3072] / txt [batch, n_txt, 3072] fp32 (or 2-D for
    batch 1) are updated in place; the sequences share t_emb and pe. With
    profile=True returns {category: ms} summed over the blocks."""
    batch = img.shape[0] if img.dim() == 3 else 1
    n_img = img.shape[-2]
    n_txt = txt.shape[-2]
    if txt.dim() == 3 and txt.shape[0] != batch:
        raise ValueError("img and txt batch differ")
    _check_block_operands("mmdit_blocks_forward", img, txt, t_emb, pe, n_img, n_txt, batch)
    if scratch is None:
        scratch = torch.empty((mmdit_block_scratch_bytes(n_img, n_txt, batch),), dtype=torch.uint8,
                              device=img.device)
    prof = (ctypes.c_float * len(PROF_CATEGORIES))() if profile else None
    _check(_lib.qimg_mmdit_blocks_forward(ctypes.addressof(table.array), table.n, _ptr(img), _ptr(txt), _ptr(t_emb),
                                          _ptr(pe), n_img, n_txt, batch, _ptr(scratch), scratch.numel(),
                                          ctypes.addressof(prof) if profile else None, _stream()))
    if profile:
        return {n: float(prof[i]) for i, n in enumerate(PROF_CATEGORIES)}
    return None


def mmdit_block_forward(weights: dict, biases: dict, norms: dict, img: torch.Tensor, txt: torch.Tensor,
                        t_emb: torch.Tensor, pe: torch.Tensor, scratch: torch.Tensor | None = None,
                        profile: bool = False):
    """One MMDiT joint block (transformer.cu:506-817), img [n_img, 3072] and
    txt [n_txt, 3072] fp32 updated in place. `weights` maps the names of
    TransformerWeights::Block (img_mod, to_q, ..., txt_mlp_fc2) to
    QuantizedWeight, `biases` the same names to bf16 [N] tensors, `norms`
    norm_q / norm_k / norm_added_q / norm_added_k to bf16 [128]. With
    profile=True returns {category: ms} (the stream is synchronised)."""
    n_img, n_txt = img.shape[0], txt.shape[0]
    _check_block_operands("mmdit_block_forward", img, txt, t_emb, pe, n_img, n_txt, 1)
    b = _block_struct(weights, biases, norms)
    if scratch is None:
        scratch = torch.empty((mmdit_block_scratch_bytes(n_img, n_txt),), dtype=torch.uint8, device=img.device)
    prof = (ctypes.c_float * len(PROF_CATEGORIES))() if profile else None
    _check(_lib.qimg_mmdit_block_forward(ctypes.addressof(b), _ptr(img), _ptr(txt), _ptr(t_emb), _ptr(pe), n_img,
                                         n_txt, _ptr(scratch), scratch.numel(),
                                         ctypes.addressof(prof) if profile else None, _stream()))
    if profile:
        return {n: float(prof[i]) for i, n in enumerate(PROF_CATEGORIES)}
    return None
