"""Writes the checkpoint-format fixtures (run in a container that has the
reference sources; the files it writes are committed):

  st_writer_ref.safetensors  the reference's SafeTensorsWriter
                             (safetensors_writer.h) run on the fixed tensors of
                             oracle/st_writer_ref.cpp (built by `make -C oracle ref`)
  quantize_plan.json         the tensor order of the reference's offline
                             quantizer (quantize.cu:462-539, the INT8 branch),
                             read from that file's quantize_weight / passthrough
                             calls; block tensors carry a "{i}" placeholder
"""
import json
import os
import re
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF = os.environ.get("QIMG_REFERENCE", "/root/reference")


def writer_fixture():
    subprocess.run(["make", "-C", os.path.join(ROOT, "oracle"), "ref", f"REF={REF}"], check=True)
    out = os.path.join(HERE, "st_writer_ref.safetensors")
    subprocess.run([os.path.join(ROOT, "oracle", "_ref", "st_writer_ref"), out], check=True)
    return out


def quantize_plan():
    src = open(os.path.join(REF, "quantize.cu")).read()
    body = src[src.index("// --- Timestep embedding ---"):src.index("writer.write(cfg.output)")]
    body = re.sub(r"quantize_fused_qkv\([^;]*\);", "", body, flags=re.S)  # the INT4 fused branch
    plan = []
    for fn, prefix, name in re.findall(r'\b(quantize_weight|passthrough)\((prefix \+ )?"([^"]+)"\)', body):
        full = ("transformer_blocks.{i}." if prefix else "") + name
        plan.append([full, fn == "quantize_weight"])
    out = os.path.join(HERE, "quantize_plan.json")
    with open(out, "w") as f:
        json.dump({"source": "quantize.cu:462-539", "blocks": 60, "plan": plan}, f, indent=0)
        f.write("\n")
    return out, len(plan)


if __name__ == "__main__":
    print(writer_fixture())
    print(*quantize_plan())
