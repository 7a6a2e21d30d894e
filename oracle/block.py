"""CPU restatement of one MMDiT joint block (transformer.cu:506-817).

TEST INFRASTRUCTURE ONLY: imported by tests/ and the bench's CPU-baseline leg
to produce expected values. Product code never imports it.

The element-wise / per-row operations are restated in numpy float32 with
float64 reductions (the reference reduces in fp32 trees; the difference is a
few ulp, inside the block tolerance). The quantized linears and the
SageAttention go through the C oracle (oracle.linear_w8a8,
oracle.sage_attention_fp16io), which is bit-exact for int8 values and scales.
"""
from __future__ import annotations

import numpy as np

from . import oracle as o

DIM, HEADS, HEAD_DIM, MLP = 3072, 24, 128, 12288
F32 = np.float32


def silu(x):
    """silu_fp32_kernel (cuda_kernels.cu:1881-1887)."""
    x = np.asarray(x, F32)
    return (x / (F32(1) + np.exp(-x))).astype(F32)


def layer_norm_modulate(x, shift, scale, eps=1e-6):
    """layer_norm_modulate_fp32_kernel (cuda_kernels.cu:1799-1853)."""
    x = np.asarray(x, F32)
    mean = (x.astype(np.float64).sum(1, keepdims=True) / x.shape[1]).astype(F32)
    d = (x - mean).astype(F32)
    var = (d.astype(np.float64) ** 2).sum(1, keepdims=True) / x.shape[1]
    inv = (1.0 / np.sqrt(var + eps)).astype(F32)
    return (d * inv * (F32(1) + np.asarray(scale, F32)) + np.asarray(shift, F32)).astype(F32)


def rms_norm_heads(x, w_bits, eps=1e-6):
    """rms_norm_fp32_kernel (cuda_kernels.cu:1656-1687) over rows of 128."""
    n = x.shape[0]
    r = np.asarray(x, F32).reshape(n * HEADS, HEAD_DIM)
    ss = (r.astype(np.float64) ** 2).sum(1, keepdims=True)
    rms = (1.0 / np.sqrt(ss / HEAD_DIM + eps)).astype(F32)
    w = o.bf16_bits_to_f32(np.asarray(w_bits, np.uint16)).reshape(1, HEAD_DIM)
    return (r * rms * w).astype(F32).reshape(n, DIM)


def concat_transpose(txt, img):
    """concat_transpose_fused_fp32 (transformer.cu:106-130): text first,
    [S, H, D] -> [H, S, D]."""
    x = np.concatenate([np.asarray(txt, F32), np.asarray(img, F32)], 0)
    return np.ascontiguousarray(x.reshape(-1, HEADS, HEAD_DIM).transpose(1, 0, 2))


def rope_f16(x, pe):
    """rope_apply_fp32_to_fp16_kernel (cuda_kernels.cu:1935-1962) on
    [H, S, 128] with pe [S, 64, 4] = (cos, -sin, sin, cos)."""
    x0 = x[..., 0::2]
    x1 = x[..., 1::2]
    p = np.asarray(pe, F32)[None]
    out = np.empty_like(x)
    out[..., 0::2] = x0 * p[..., 0] + x1 * p[..., 1]
    out[..., 1::2] = x0 * p[..., 2] + x1 * p[..., 3]
    return out.astype(np.float16)


def split(attn, n_txt):
    """transpose_split_fused_fp32 (transformer.cu:84-104)."""
    a = np.asarray(attn, F32).transpose(1, 0, 2).reshape(-1, DIM)
    return a[:n_txt].copy(), a[n_txt:].copy()


def gate_add(x, gate, y):
    """gate_add_fp32f_kernel (cuda_kernels.cu:2181-2189)."""
    return (np.asarray(x, F32) + np.asarray(gate, F32)[None] * np.asarray(y, F32)).astype(F32)


def qlinear(entry, x, gelu=False):
    """One quantized linear: entry = (w_q, w_scales, hbs, bias_bits) for
    int8 + Hadamard (cuda_kernels.cu:2674-2827), or the same with a fifth
    element 1 for e4m3 weights and activations behind the same FWHT."""
    wq, ws, hbs, b = entry[:4]
    x = np.asarray(x, F32)
    if len(entry) > 4 and entry[4] == 1:
        aq, asc = o.quantize_activation_fp8(x, hbs)
        return o.gemm_fp8_epilogue(aq, wq, asc, ws, b, gelu=gelu)
    return o.linear_w8a8(x, wq, ws, hbs, b, gelu=gelu)


def mmdit_block(q, img, txt, t_emb, pe):
    """One block as transformer.cu:506-817. `q` maps the block's linear names
    (img_mod, to_q, ..., txt_mlp_fc2) to qlinear entries and norm_q / norm_k /
    norm_added_q / norm_added_k to bf16 bits [128]. Returns the updated
    (img, txt)."""
    def lin(x, name, gelu=False):
        return qlinear(q[name], x, gelu)

    n_txt = txt.shape[0]
    ts = silu(t_emb).reshape(1, DIM)
    im = lin(ts, "img_mod").reshape(6, DIM)
    tm = lin(ts, "txt_mod").reshape(6, DIM)
    img_n = layer_norm_modulate(img, im[0], im[1])
    txt_n = layer_norm_modulate(txt, tm[0], tm[1])
    iq, ik, iv = lin(img_n, "to_q"), lin(img_n, "to_k"), lin(img_n, "to_v")
    tq, tk, tv = lin(txt_n, "add_q_proj"), lin(txt_n, "add_k_proj"), lin(txt_n, "add_v_proj")
    iq, ik = rms_norm_heads(iq, q["norm_q"]), rms_norm_heads(ik, q["norm_k"])
    tq, tk = rms_norm_heads(tq, q["norm_added_q"]), rms_norm_heads(tk, q["norm_added_k"])
    q16 = rope_f16(concat_transpose(tq, iq), pe)
    k16 = rope_f16(concat_transpose(tk, ik), pe)
    v16 = concat_transpose(tv, iv).astype(np.float16)
    attn = o.sage_attention_fp16io(q16, k16, v16, 1.0 / np.sqrt(128.0), False)
    ta, ia = split(attn, n_txt)
    img = gate_add(img, im[2], lin(ia, "to_out"))
    txt = gate_add(txt, tm[2], lin(ta, "to_add_out"))
    img_n = layer_norm_modulate(img, im[3], im[4])
    txt_n = layer_norm_modulate(txt, tm[3], tm[4])
    img = gate_add(img, im[5], lin(lin(img_n, "img_mlp_fc1", gelu=True), "img_mlp_fc2"))
    txt = gate_add(txt, tm[5], lin(lin(txt_n, "txt_mlp_fc1", gelu=True), "txt_mlp_fc2"))
    return img, txt
