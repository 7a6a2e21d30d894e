"""Quantized checkpoint format, host side (no GPU): the safetensors writer
against the reference's SafeTensorsWriter bytes (tests/golden/
st_writer_ref.safetensors, written by safetensors_writer.h), the reader and
checkpoint detection against files written by the `safetensors` package,
error paths, and the C ABI of include/qimg_ckpt.h."""
import json
import os
import re
import struct

import numpy as np
import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
GOLDEN = os.path.join(HERE, "golden")

# the tensors oracle/st_writer_ref.cpp hands to the reference writer
REF_TENSORS = [
    ("transformer_blocks.0.attn.to_q.weight", "I8", [2, 3], np.array([0, 1, -2, 3, -128, 127], np.int8).tobytes()),
    ("transformer_blocks.0.attn.to_q.weight.__scales__", "F32", [2], np.array([1.5, -2.0], np.float32).tobytes()),
    ('quote"name\\x', "BF16", [1], np.array([0x3F80], np.uint16).tobytes()),
    ("scalar", "F32", [], np.array([3.25], np.float32).tobytes()),
    ("empty", "U8", [0], b""),
    ("e4m3", "F8_E4M3", [2, 2], bytes([0x00, 0x38, 0xB8, 0x7E])),
]


def test_ckpt_header_symbols_exported(qimg):
    text = open(os.path.join(ROOT, "include", "qimg_ckpt.h")).read()
    names = set(re.findall(r"\b(qimg_\w+)\s*\(", text))
    assert names == set(qimg.CKPT_EXPORTED)
    h = qimg.host_lib()
    for n in names:
        assert hasattr(h, n), f"{n} declared in qimg_ckpt.h but not exported"


def test_writer_bytes_equal_reference_writer(qimg, tmp_path):
    p = str(tmp_path / "w.safetensors")
    qimg.write_safetensors(p, REF_TENSORS)
    ref = open(os.path.join(GOLDEN, "st_writer_ref.safetensors"), "rb").read()
    assert open(p, "rb").read() == ref


def test_writer_output_reads_with_safetensors_package(qimg, tmp_path):
    from safetensors.torch import load_file
    p = str(tmp_path / "w.safetensors")
    qimg.write_safetensors(p, REF_TENSORS)
    t = load_file(p)
    assert t["transformer_blocks.0.attn.to_q.weight"].tolist() == [[0, 1, -2], [3, -128, 127]]
    assert t["transformer_blocks.0.attn.to_q.weight.__scales__"].tolist() == [1.5, -2.0]
    assert t['quote"name\\x'].dtype == torch.bfloat16 and t['quote"name\\x'].item() == 1.0
    assert t["scalar"].shape == () and t["scalar"].item() == 3.25
    assert t["empty"].numel() == 0
    assert t["e4m3"].dtype == torch.float8_e4m3fn
    assert t["e4m3"].float().flatten().tolist() == [0.0, 1.0, -1.0, 448.0]
    # header length and padding (8 + len is a multiple of 8, padded with spaces)
    raw = open(p, "rb").read()
    n = struct.unpack("<Q", raw[:8])[0]
    header = raw[8:8 + n].decode()
    assert (8 + n) % 8 == 0 and header.rstrip(" ").endswith("}") and len(header) - len(header.rstrip(" ")) < 8
    assert list(json.loads(header)) == [e[0] for e in REF_TENSORS]  # insertion order


@pytest.mark.parametrize("dtype,kind", [(torch.bfloat16, "bf16"), (torch.int8, "int8"),
                                        (torch.float8_e4m3fn, "fp8")])
def test_checkpoint_kind(qimg, tmp_path, dtype, kind):
    from safetensors.torch import save_file
    w = torch.zeros(4, 8).to(dtype)
    tensors = {"transformer_blocks.0.attn.to_q.weight": w, "img_in.weight": torch.zeros(2, 2, dtype=torch.bfloat16)}
    if kind != "bf16":
        tensors["transformer_blocks.0.attn.to_q.weight.__scales__"] = torch.ones(4)
    f = str(tmp_path / "x.safetensors")
    save_file(tensors, f)
    assert qimg.checkpoint_kind(f) == kind
    # a directory holding model.safetensors (load_model_dir)
    d = tmp_path / "dir"
    d.mkdir()
    save_file(tensors, str(d / "model.safetensors"))
    assert qimg.checkpoint_kind(str(d)) == kind


def test_sharded_index(qimg, tmp_path):
    from safetensors.torch import save_file
    save_file({"img_in.weight": torch.zeros(2, 2, dtype=torch.bfloat16)}, str(tmp_path / "a.safetensors"))
    save_file({"transformer_blocks.0.attn.to_q.weight": torch.zeros(2, 2, dtype=torch.int8)},
              str(tmp_path / "b.safetensors"))
    idx = {"metadata": {}, "weight_map": {"img_in.weight": "a.safetensors",
                                          "transformer_blocks.0.attn.to_q.weight": "b.safetensors"}}
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps(idx))
    assert qimg.checkpoint_kind(str(tmp_path)) == "int8"


def test_unknown_dtype_is_an_error(qimg, tmp_path):
    """The reference prints "Unknown dtype" and skips the tensor; here the
    load fails and names it."""
    from safetensors.torch import save_file
    f = str(tmp_path / "x.safetensors")
    save_file({"transformer_blocks.0.attn.to_q.weight": torch.zeros(2, 2, dtype=torch.float64)}, f)
    with pytest.raises(ValueError, match="unknown dtype 'F64'.*to_q.weight"):
        qimg.checkpoint_kind(f)


def test_malformed_files_are_errors(qimg, tmp_path):
    good = str(tmp_path / "g.safetensors")
    qimg.write_safetensors(good, REF_TENSORS)
    raw = open(good, "rb").read()
    n = struct.unpack("<Q", raw[:8])[0]
    cases = {
        "truncated_header": raw[:20],
        "length_past_end": struct.pack("<Q", len(raw)) + raw[8:],
        "bad_json": raw[:8] + raw[8:8 + n].replace(b'"dtype"', b'"dtype" ', 1)[:-2] + b"]]" + raw[8 + n:],
        "data_past_end": raw[:-1],
        "offsets_vs_shape": raw.replace(b'"shape":[2,3]', b'"shape":[3,3]', 1),
        "empty_file": b"",
    }
    for name, data in cases.items():
        f = str(tmp_path / f"{name}.safetensors")
        open(f, "wb").write(data)
        with pytest.raises(ValueError):
            qimg.checkpoint_kind(f)
    with pytest.raises(ValueError, match="No such|no safetensors"):
        qimg.checkpoint_kind(str(tmp_path / "missing_dir"))


def test_quantizer_rejects_incomplete_checkpoint(qimg, tmp_path):
    """Fails on the first missing tensor of the list, before any device work."""
    from safetensors.torch import save_file
    f = str(tmp_path / "x.safetensors")
    save_file({"img_in.weight": torch.zeros(2, 2, dtype=torch.bfloat16)}, f)
    with pytest.raises(ValueError, match="tensor not found.*timestep_embedder.linear_1.weight"):
        qimg.quantize_checkpoint(f, str(tmp_path / "o.safetensors"), qimg.INT8_HADAMARD, 1)
    with pytest.raises(ValueError, match="mode"):
        qimg.quantize_checkpoint(f, str(tmp_path / "o.safetensors"), 7, 1)
    assert not os.path.exists(tmp_path / "o.safetensors")


def test_plan_fixture():
    d = json.load(open(os.path.join(GOLDEN, "quantize_plan.json")))
    plan = d["plan"]
    glob = [p for p in plan if "{i}" not in p[0]]
    blk = [p for p in plan if "{i}" in p[0]]
    assert len(glob) == 13 and len(blk) == 32
    assert sum(q for _, q in glob) == 2 and sum(q for _, q in blk) == 14
    assert all(n.endswith(".weight") for n, q in plan if q)


def test_metadata_and_escaped_names(qimg, tmp_path):
    """__metadata__ is skipped (safetensors.h:71); JSON escapes in names
    (\\u sequences, written by the safetensors package for non-ASCII) are
    decoded, so the probe name is found."""
    from safetensors.torch import save_file
    f = str(tmp_path / "m.safetensors")
    save_file({"transformer_blocks.0.attn.to_q.weight": torch.zeros(2, 2, dtype=torch.int8),
               "transformer_blocks.0.attn.to_q.weight.__scales__": torch.ones(2),
               "café.weight": torch.zeros(1)}, f, metadata={"format": "pt", "quote": 'a"b'})
    assert qimg.checkpoint_kind(f) == "int8"
    # the same header hand-escaped with \u sequences
    raw = open(f, "rb").read()
    n = struct.unpack("<Q", raw[:8])[0]
    hdr = raw[8:8 + n].decode()
    esc = hdr.replace("transformer_blocks.0", "\\u0074ransformer_blocks.0")
    pad = (8 - (8 + len(esc.encode())) % 8) % 8
    esc_b = (esc + " " * pad).encode()
    g = str(tmp_path / "e.safetensors")
    open(g, "wb").write(struct.pack("<Q", len(esc_b)) + esc_b + raw[8 + n:])
    assert qimg.checkpoint_kind(g) == "int8"
