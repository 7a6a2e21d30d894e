"""Offline quantizer (qimg_quantize_checkpoint, quantize.cu:110-161,
462-539) on the GPU: a small BF16 checkpoint with every tensor of the
reference's list for two blocks is quantized to I8 and to F8_E4M3; the
output's tensor order must equal the list read from quantize.cu
(tests/golden/quantize_plan.json), every quantized weight and scale must
equal the oracle's bit for bit, and copied tensors keep their bytes with
the reference's dtype labels. The output is parsed here from its raw
header, independently of the library's reader."""
import json
import os
import struct

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
PLAN = json.load(open(os.path.join(HERE, "golden", "quantize_plan.json")))["plan"]
NBLK = 2


def plan(nblk):
    glob = [(n, q) for n, q in PLAN if "{i}" not in n]
    blk = [(n, q) for n, q in PLAN if "{i}" in n]
    return glob + [(n.replace("{i}", str(i)), q) for i in range(nblk) for n, q in blk]


def weight_shape(name):
    if "img_mod" in name:
        return (16, 3072)   # hbs 1024
    if name.endswith("net.2.weight"):
        return (8, 96)      # hbs 32
    return (24, 256)


def make_checkpoint(path):
    from safetensors.torch import save_file
    g = torch.Generator().manual_seed(7)
    t = {}
    for name, q in plan(NBLK):
        if q:
            t[name] = (torch.randn(weight_shape(name), generator=g) * 0.05).to(torch.bfloat16)
        elif name == "txt_norm.weight":
            t[name] = torch.randn(64, generator=g)                        # F32, kept F32
        elif name.endswith("norm_q.weight"):
            t[name] = torch.randn(128, generator=g).to(torch.float16)    # labelled BF16, as the reference
        else:
            t[name] = torch.randn(16, generator=g).to(torch.bfloat16)
    save_file(t, path)
    return t


def read_raw(path):
    raw = open(path, "rb").read()
    n = struct.unpack("<Q", raw[:8])[0]
    header = json.loads(raw[8:8 + n])
    data = raw[8 + n:]
    return header, lambda e: data[e["data_offsets"][0]:e["data_offsets"][1]]


@pytest.mark.parametrize("mode", ["int8", "fp8"])
def test_quantize_checkpoint_matches_oracle(qimg, oracle, tmp_path, mode):
    src = str(tmp_path / "bf16.safetensors")
    dst = str(tmp_path / f"{mode}.safetensors")
    tensors = make_checkpoint(src)
    print(f"quantize_checkpoint mode={mode} blocks={NBLK}", flush=True)
    qimg.quantize_checkpoint(src, dst, qimg.INT8_HADAMARD if mode == "int8" else qimg.FP8_HADAMARD, NBLK)
    header, blob = read_raw(dst)
    expect = []
    for n, q in plan(NBLK):
        expect += [n, n + ".__scales__"] if q else [n]
    assert list(header) == expect
    for name, q in plan(NBLK):
        e = header[name]
        src_t = tensors[name]
        if not q:
            assert e["dtype"] == ("F32" if src_t.dtype == torch.float32 else "BF16")
            assert e["shape"] == list(src_t.shape)
            assert blob(e) == src_t.contiguous().view(torch.uint8).numpy().tobytes()
            continue
        bits = src_t.view(torch.int16).numpy().view(np.uint16)
        N, K = bits.shape
        if mode == "int8":
            q_ref, s_ref, _ = oracle.quantize_weight_bf16(bits)
            assert e["dtype"] == "I8"
        else:
            q_ref, s_ref, _ = oracle.quantize_weight_fp8(bits)
            assert e["dtype"] == "F8_E4M3"
        assert e["shape"] == [N, K]
        got = np.frombuffer(blob(e), np.uint8).reshape(N, K)
        assert np.array_equal(got, np.ascontiguousarray(q_ref).view(np.uint8)), name
        es = header[name + ".__scales__"]
        assert es["dtype"] == "F32" and es["shape"] == [N]
        assert np.array_equal(np.frombuffer(blob(es), np.float32).view(np.uint32),
                              np.asarray(s_ref, np.float32).view(np.uint32)), name
    assert qimg.checkpoint_kind(dst) == mode
    assert qimg.checkpoint_kind(src) == "bf16"
