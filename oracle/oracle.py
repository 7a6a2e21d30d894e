"""numpy front end of the CPU oracle (oracle/qimg_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, the smoke check and the bench's
CPU-baseline leg to produce expected values. Product code never imports it.

Each wrapper names the reference function it restates (file:line relative to
the qwen-image.cu tree); the C source holds the arithmetic.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libqimg_oracle.so")
_lib = None

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float

_SIGS = {
    "or_bf16_to_f32": (_F, [ctypes.c_uint16]),
    "or_f32_to_bf16": (ctypes.c_uint16, [_F]),
    "or_f16_to_f32": (_F, [ctypes.c_uint16]),
    "or_f32_to_f16": (ctypes.c_uint16, [_F]),
    "or_f32_to_e4m3": (ctypes.c_uint8, [_F]),
    "or_e4m3_to_f32": (_F, [ctypes.c_uint8]),
    "or_hadamard_block_size": (_I, [_I]),
    "or_fwht_norm": (_F, [_I]),
    "or_fwht_rows": (None, [_P, _I64, _I, _I]),
    "or_quant_rows_int8": (None, [_P, _I64, _I, _P, _P]),
    "or_quantize_weight_bf16": (_I, [_P, _I, _I, _P, _P]),
    "or_quantize_activation": (None, [_P, _I, _I64, _I, _I, _P, _P]),
    "or_gemm_s8s8s32": (None, [_P, _P, _I64, _I, _I, _I64, _I64, _P]),
    "or_dequant_epilogue": (None, [_P, _P, _P, _P, _I64, _I, _I, _P]),
    "or_quant_rows_fp8": (None, [_P, _I64, _I, _P, _P]),
    "or_gemm_fp8_epilogue": (None, [_P, _P, _P, _P, _P, _I64, _I, _I, _I64, _I64, _I, _P]),
    "or_sage_k_mean": (None, [_P, _I, _I, _I, _P]),
    "or_sage_quant_q": (None, [_P, _I, _I, _I, _P, _P]),
    "or_sage_quant_k": (None, [_P, _P, _I, _I, _I, _P, _P]),
    "or_sage_attn": (None, [_P, _P, _P, _P, _P, _I, _I, _I, _F, _I, _I, _I, _P]),
    "or_sage_attention_fp16io": (None, [_P, _P, _P, _I, _I, _I, _F, _I, _P]),
    "or_dequant_int4_bf16": (None, [_P, _P, _I, _I, _I, _I, _I, _I, _P]),
    "or_quant_int4_linear": (None, [_P, _I, _I, _I, _P, _P]),
    "or_quant_int4_nf4": (None, [_P, _I, _I, _I, _P, _P]),
    "or_quant_act_int4": (None, [_P, _P, _I, _I, _I, _P, _P, _P]),
    "or_w4a4_gemm": (None, [_P, _P, _P, _P, _I64, _I, _I, _I, _I, _P, _I64, _I64, _P]),
    "or_awq_repack": (None, [_P, _I, _I, _P]),
    "or_dequant_awq_bf16": (None, [_P, _P, _P, _I, _I, _I, _I, _P]),
    "or_awq_gemv": (None, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "or_unswizzle_nunchaku": (None, [_P, _P, _I, _I, _I, _P, _P]),
    "or_dequant_nunchaku_bf16": (None, [_P, _P, _I, _I, _I, _P]),
    "or_unswizzle_lora": (None, [_P, _I, _I, _I, _P]),
    "or_set_threads": (None, [_I]),
    "or_get_threads": (_I, []),
}


def build() -> str:
    """Compile the oracle with its Makefile (gcc); returns the library path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def set_threads(n: int) -> None:
    lib().or_set_threads(int(n))


def get_threads() -> int:
    return int(lib().or_get_threads())


# ---------------------------------------------------------------- dtypes
def bf16_bits_from_f32(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns (uint16), round to nearest even."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def e4m3_to_f32(b: np.ndarray) -> np.ndarray:
    L = lib()
    lut = np.array([L.or_e4m3_to_f32(i) for i in range(256)], dtype=np.float32)
    return lut[np.asarray(b, dtype=np.uint8)]


# ---------------------------------------------------------- quantization
def hadamard_block_size(K: int) -> int:
    """cuda_kernels.cuh:253"""
    return int(lib().or_hadamard_block_size(int(K)))


def fwht_rows(x: np.ndarray, hbs: int) -> np.ndarray:
    """cuda_kernels.cu:2209-2254 (returns a transformed copy)."""
    y = np.array(x, dtype=np.float32, order="C", copy=True)
    M, K = y.shape
    lib().or_fwht_rows(_ptr(y), M, K, int(hbs))
    return y


def quant_rows_int8(x: np.ndarray):
    """cuda_kernels.cu:2385-2416 -> (int8 [M,K], fp32 scales [M])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    q = np.empty((M, K), np.int8)
    s = np.empty((M,), np.float32)
    lib().or_quant_rows_int8(_ptr(x), M, K, _ptr(q), _ptr(s))
    return q, s


def quantize_weight_bf16(w_bits: np.ndarray):
    """cuda_kernels.cu:2830-2862 -> (int8 [N,K], scales [N], hbs)."""
    w_bits = np.ascontiguousarray(w_bits, dtype=np.uint16)
    N, K = w_bits.shape
    q = np.empty((N, K), np.int8)
    s = np.empty((N,), np.float32)
    hbs = lib().or_quantize_weight_bf16(_ptr(w_bits), N, K, _ptr(q), _ptr(s))
    return q, s, int(hbs)


def quantize_activation(x: np.ndarray, hbs: int, is_bf16: bool | None = None):
    """cuda_kernels.cu:2493-2619. x is fp32, or uint16 bf16 bit patterns."""
    if is_bf16 is None:
        is_bf16 = x.dtype == np.uint16
    x = np.ascontiguousarray(x, dtype=np.uint16 if is_bf16 else np.float32)
    M, K = x.shape
    q = np.empty((M, K), np.int8)
    s = np.empty((M,), np.float32)
    lib().or_quantize_activation(_ptr(x), int(bool(is_bf16)), M, K, int(hbs), _ptr(q), _ptr(s))
    return q, s


def gemm_s8s8s32(a: np.ndarray, w: np.ndarray, rows: tuple[int, int] | None = None) -> np.ndarray:
    """cuda_kernels.cu:2711-2721; returns C[M,N] int32 (rows outside `rows` are 0)."""
    a = np.ascontiguousarray(a, dtype=np.int8)
    w = np.ascontiguousarray(w, dtype=np.int8)
    M, K = a.shape
    N = w.shape[0]
    m0, m1 = rows if rows is not None else (0, M)
    c = np.zeros((M, N), np.int32)
    lib().or_gemm_s8s8s32(_ptr(a), _ptr(w), M, N, K, m0, m1, _ptr(c))
    return c


def dequant_epilogue(c: np.ndarray, a_scales, w_scales, bias_bits=None, gelu=False) -> np.ndarray:
    """cuda_kernels.cu:2623-2668"""
    c = np.ascontiguousarray(c, dtype=np.int32)
    M, N = c.shape
    a_scales = np.ascontiguousarray(a_scales, dtype=np.float32)
    w_scales = np.ascontiguousarray(w_scales, dtype=np.float32)
    out = np.empty((M, N), np.float32)
    b = None if bias_bits is None else np.ascontiguousarray(bias_bits, dtype=np.uint16)
    lib().or_dequant_epilogue(_ptr(c), _ptr(a_scales), _ptr(w_scales),
                              None if b is None else _ptr(b), M, N, int(bool(gelu)), _ptr(out))
    return out


def linear_w8a8(x, w_q, w_scales, hbs, bias_bits=None, gelu=False):
    """cuda_kernels.cu:2674-2827 composition (a5 -> a7 -> a8)."""
    q, s = quantize_activation(x, hbs)
    c = gemm_s8s8s32(q, w_q)
    return dequant_epilogue(c, s, w_scales, bias_bits, gelu)


def gelu_tanh64(v):
    """gelu_fp32 (cuda_kernels.cu:1863-1871): 0.5 v (1 + tanh(c (v + 0.044715 v^3))),
    c = 0.7978845608, evaluated in float64."""
    v = np.asarray(v, np.float64)
    return 0.5 * v * (1.0 + np.tanh(0.7978845608 * (v + 0.044715 * v ** 3)))


def linear_bf16(x, w_bits, bias_bits=None, gelu=False):
    """linear_forward_bf16 / linear_forward_bf16_bf16in (cuda_kernels.cu:4534-4596).

    x fp32 is rounded to bf16 (fp32_to_bf16, cuda_kernels.cu:33-42:
    __float2bfloat16, nearest even); uint16 x is taken as bf16 bits. The
    bf16 x bf16 products are summed exactly (float64) and rounded once to
    fp32: cuBLAS's fp32 accumulation order is outside the reference's
    sources, so the summation order is not pinned and callers compare within
    a bound on the fp32 rounding of a K-term sum. Then + bias in fp32
    (bias_add_fp32, :1510-1517) and GELU (gelu_fp32) when asked.
    Returns (out float64 [M,N], sum_k |x_k w_k| [M,N] for error bounds)."""
    if np.asarray(x).dtype == np.uint16:
        xb = bf16_bits_to_f32(x).reshape(np.shape(x))
    else:
        xb = bf16_bits_to_f32(bf16_bits_from_f32(np.asarray(x, np.float32))).reshape(np.shape(x))
    w = bf16_bits_to_f32(w_bits).reshape(np.shape(w_bits)).astype(np.float64)
    xd = xb.astype(np.float64)
    acc = (xd @ w.T).astype(np.float32)
    mag = np.abs(xd) @ np.abs(w).T
    if bias_bits is not None:
        acc = (acc + bf16_bits_to_f32(bias_bits)[None, :]).astype(np.float32)
    out = acc.astype(np.float64)
    if gelu:
        out = gelu_tanh64(out)
    return out, mag


# ---------------------------------------------------------------- fp8
def quant_rows_fp8(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    q = np.empty((M, K), np.uint8)
    s = np.empty((M,), np.float32)
    lib().or_quant_rows_fp8(_ptr(x), M, K, _ptr(q), _ptr(s))
    return q, s


def quantize_weight_fp8(w_bits: np.ndarray):
    w = bf16_bits_to_f32(w_bits).reshape(w_bits.shape)
    hbs = hadamard_block_size(w.shape[1])
    if hbs > 1:
        w = fwht_rows(w, hbs)
    q, s = quant_rows_fp8(w)
    return q, s, hbs


def quantize_activation_fp8(x: np.ndarray, hbs: int):
    xf = bf16_bits_to_f32(x).reshape(x.shape) if x.dtype == np.uint16 else np.asarray(x, np.float32)
    if hbs > 1:
        xf = fwht_rows(xf, hbs)
    return quant_rows_fp8(xf)


def gemm_fp8_epilogue(a_q, w_q, a_scales, w_scales, bias_bits=None, gelu=False, rows=None):
    a_q = np.ascontiguousarray(a_q, dtype=np.uint8)
    w_q = np.ascontiguousarray(w_q, dtype=np.uint8)
    M, K = a_q.shape
    N = w_q.shape[0]
    m0, m1 = rows if rows is not None else (0, M)
    out = np.zeros((M, N), np.float32)
    a_scales = np.ascontiguousarray(a_scales, dtype=np.float32)
    w_scales = np.ascontiguousarray(w_scales, dtype=np.float32)
    b = None if bias_bits is None else np.ascontiguousarray(bias_bits, dtype=np.uint16)
    lib().or_gemm_fp8_epilogue(_ptr(a_q), _ptr(w_q), _ptr(a_scales), _ptr(w_scales),
                               None if b is None else _ptr(b), M, N, K, m0, m1,
                               int(bool(gelu)), _ptr(out))
    return out


# ---------------------------------------------------------- SageAttention
def sage_k_mean(k_f16: np.ndarray) -> np.ndarray:
    """sageattention_sm80.cu:759-773; k is float16 [BH,S,D]."""
    k = np.ascontiguousarray(k_f16, dtype=np.float16)
    BH, S, D = k.shape
    mean = np.empty((BH, D), np.float32)
    lib().or_sage_k_mean(_ptr(k), BH, S, D, _ptr(mean))
    return mean


def sage_quant_q(q_f16: np.ndarray):
    """sageattention_sm80.cu:775-824"""
    q = np.ascontiguousarray(q_f16, dtype=np.float16)
    BH, S, D = q.shape
    out = np.empty((BH, S, D), np.int8)
    sc = np.empty((BH, (S + 127) // 128 * 32), np.float32)
    lib().or_sage_quant_q(_ptr(q), BH, S, D, _ptr(out), _ptr(sc))
    return out, sc


def sage_quant_k(k_f16: np.ndarray, mean: np.ndarray):
    """sageattention_sm80.cu:826-886"""
    k = np.ascontiguousarray(k_f16, dtype=np.float16)
    BH, S, D = k.shape
    mean = np.ascontiguousarray(mean, dtype=np.float32)
    out = np.empty((BH, S, D), np.int8)
    sc = np.empty((BH, (S + 63) // 64 * 4), np.float32)
    lib().or_sage_quant_k(_ptr(k), _ptr(mean), BH, S, D, _ptr(out), _ptr(sc))
    return out, sc


def sage_attn(q_i8, k_i8, v_f16, q_scale, k_scale, sm_scale, causal=False, rows=None):
    """sageattention_sm80.cu:47-674 -> float16 [BH,S,D] (rows outside `rows` are 0)."""
    q_i8 = np.ascontiguousarray(q_i8, dtype=np.int8)
    k_i8 = np.ascontiguousarray(k_i8, dtype=np.int8)
    v = np.ascontiguousarray(v_f16, dtype=np.float16)
    BH, S, D = q_i8.shape
    q0, q1 = rows if rows is not None else (0, S)
    out = np.zeros((BH, S, D), np.float16)
    lib().or_sage_attn(_ptr(q_i8), _ptr(k_i8), _ptr(v),
                       _ptr(np.ascontiguousarray(q_scale, np.float32)),
                       _ptr(np.ascontiguousarray(k_scale, np.float32)),
                       BH, S, D, float(sm_scale), int(bool(causal)), q0, q1, _ptr(out))
    return out


def sage_attention_fp16io(q, k, v, sm_scale, causal=False) -> np.ndarray:
    """sageattention_sm80.cu:965-1027 composition; returns float16 [BH,S,D]."""
    q = np.ascontiguousarray(q, dtype=np.float16)
    k = np.ascontiguousarray(k, dtype=np.float16)
    v = np.ascontiguousarray(v, dtype=np.float16)
    BH, S, D = q.shape
    out = np.empty((BH, S, D), np.float16)
    lib().or_sage_attention_fp16io(_ptr(q), _ptr(k), _ptr(v), BH, S, D, float(sm_scale),
                                   int(bool(causal)), _ptr(out))
    return out


# ---- INT4 paths (cuda_kernels.cu:2864-4532; arithmetic in qimg_oracle_int4.c) ----

NF4_GRID = np.array([-1.0, -0.6962, -0.5251, -0.3949, -0.2844, -0.1848, -0.0911, 0.0,
                     0.0796, 0.1609, 0.2461, 0.3379, 0.4407, 0.5626, 0.7230, 1.0], np.float32)


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def dequant_int4_bf16(qw, scales, K, group_size, nf4=True, scales_gn=False, signed_int4=False):
    """dequantize_int4_to_bf16 (cuda_kernels.cu:2876-2929): bf16 bits [N, K]."""
    qw = _c(qw, np.uint8); scales = _c(scales, np.float32)
    N = qw.shape[0]
    out = np.empty((N, K), np.uint16)
    lib().or_dequant_int4_bf16(_ptr(qw), _ptr(scales), N, K, group_size, int(nf4), int(scales_gn),
                               int(signed_int4), _ptr(out))
    return out


def quant_int4_weight(r, group_size, nf4=True):
    """quantize_int4_per_group (NF4, cuda_kernels.cu:3290-3368) or the linear
    INT4 quantizer (:3226-3288): packed [N, K/2], scales [N, K/gs]."""
    r = _c(r, np.float32)
    N, K = r.shape
    qw = np.empty((N, K // 2), np.uint8)
    sc = np.empty((N, K // group_size), np.float32)
    (lib().or_quant_int4_nf4 if nf4 else lib().or_quant_int4_linear)(_ptr(r), N, K, group_size, _ptr(qw), _ptr(sc))
    return qw, sc


def quant_act_int4(x, group_size, smooth=None, want_bf16=False):
    """quantize_activation_int4 (cuda_kernels.cu:3575-3648), or with smooth /
    bf16 copy fused_smooth_bf16_quant (:3650-3730): packed [M, K/2], scales
    [G, M] (and bf16 bits [M, K])."""
    x = _c(x, np.float32)
    M, K = x.shape
    pk = np.empty((M, K // 2), np.uint8)
    sc = np.empty((K // group_size, M), np.float32)
    bf = np.empty((M, K), np.uint16) if want_bf16 else None
    sm = None if smooth is None else _c(smooth, np.float32)
    lib().or_quant_act_int4(_ptr(x), None if sm is None else _ptr(sm), M, K, group_size,
                            None if bf is None else _ptr(bf), _ptr(pk), _ptr(sc))
    return (pk, sc, bf) if want_bf16 else (pk, sc)


def w4a4_gemm(act, wgt, a_scales, w_scales, K, group_size, bias_bits=None, out=None, rows=None):
    """w4a4_gemm (cuda_kernels.cu:4257-4313, kernels :3732-3854 / :4117-4255).
    out (fp32 [M, N] or the given rows) is accumulated into when given."""
    act = _c(act, np.uint8); wgt = _c(wgt, np.uint8)
    a_scales = _c(a_scales, np.float32); w_scales = _c(w_scales, np.float32)
    M, N = act.shape[0], wgt.shape[0]
    m0, m1 = rows if rows is not None else (0, M)
    acc = out is not None
    o = _c(out, np.float32).copy() if acc else np.empty((m1 - m0, N), np.float32)
    b = None if bias_bits is None else _c(bias_bits, np.uint16)
    lib().or_w4a4_gemm(_ptr(act), _ptr(wgt), _ptr(a_scales), _ptr(w_scales), M, N, K, group_size, int(acc),
                       None if b is None else _ptr(b), m0, m1, _ptr(o))
    return o


def awq_repack(qw, OC, IC):
    """repack_awq_to_transposed (cuda_kernels.cu:3059-3102): [IC/8, OC] int32."""
    qw = _c(qw, np.int32)
    out = np.empty((IC // 8, OC), np.int32)
    lib().or_awq_repack(_ptr(qw), OC, IC, _ptr(out))
    return out


def dequant_awq_bf16(qw, wscales_bits, wzeros_bits, OC, IC, group_size, ncomp):
    """dequantize_awq_to_bf16 (cuda_kernels.cu:3002-3057): bf16 bits [OC, IC]."""
    out = np.empty((OC, IC), np.uint16)
    lib().or_dequant_awq_bf16(_ptr(_c(qw, np.int32)), _ptr(_c(wscales_bits, np.uint16)),
                              _ptr(_c(wzeros_bits, np.uint16)), OC, IC, group_size, ncomp, _ptr(out))
    return out


def awq_gemv(x, qw_rep, wscales_bits, wzeros_bits, OC, IC, group_size, ncomp, bias_bits=None):
    """linear_forward_awq / awq_gemv_repacked_kernel (cuda_kernels.cu:3106-3179), x [IC]."""
    out = np.empty(OC, np.float32)
    b = None if bias_bits is None else _c(bias_bits, np.uint16)
    lib().or_awq_gemv(_ptr(_c(x, np.float32)), _ptr(_c(qw_rep, np.int32)), _ptr(_c(wscales_bits, np.uint16)),
                      _ptr(_c(wzeros_bits, np.uint16)), None if b is None else _ptr(b), OC, IC, group_size, ncomp,
                      _ptr(out))
    return out


def unswizzle_nunchaku(q_sw, s_sw_bits, N, K, G):
    """unswizzle_nunchaku_weights (cuda_kernels.cu:3431-3499): row-major
    packed [N, K/2] and fp32 scales [G, N]."""
    q = np.empty((N, K // 2), np.uint8)
    s = np.empty((G, N), np.float32)
    lib().or_unswizzle_nunchaku(_ptr(_c(q_sw, np.uint8)), _ptr(_c(s_sw_bits, np.uint16)), N, K, G, _ptr(q), _ptr(s))
    return q, s


def dequant_nunchaku_bf16(q_sw, s_sw_bits, N, K, G):
    """dequantize_nunchaku_to_bf16 (cuda_kernels.cu:2932-2998): bf16 bits [N, K]."""
    out = np.empty((N, K), np.uint16)
    lib().or_dequant_nunchaku_bf16(_ptr(_c(q_sw, np.uint8)), _ptr(_c(s_sw_bits, np.uint16)), N, K, G, _ptr(out))
    return out


def unswizzle_lora(packed_bits, rows, cols, is_down):
    """unswizzle_lora_weights (cuda_kernels.cu:3503-3572): bf16 bits [rows, cols]."""
    out = np.empty((rows, cols), np.uint16)
    lib().or_unswizzle_lora(_ptr(_c(packed_bits, np.uint16)), rows, cols, int(is_down), _ptr(out))
    return out
