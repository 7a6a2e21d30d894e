"""Build recipe for the gfx950 hot-path library.

Compiles every HIP source under csrc/ with hipcc for gfx950 only and links
them into `qwen-image.cu_amd/lib/libqimg_hot.so` (the C ABI declared in
include/qimg_hot.h). The C++ reference-signature host layer (host/) is built
into `lib/libqimg_host.so` on top of it.

    python qwen-image.cu_amd/build.py            # build both
    python qwen-image.cu_amd/build.py --jobs 4
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
HOST = os.path.join(HERE, "host")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "lib")
HOT_SO = os.path.join(LIB, "libqimg_hot.so")
HOST_SO = os.path.join(LIB, "libqimg_host.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# Packed fp32 VALU ops are disabled: the compiler would otherwise form
# v_pk_{add,mul,fma}_f32 from scalar float code.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]

SOURCES = ["hadamard_quant.hip", "gemm_w8a8.hip", "sage_attention.hip", "capi.hip"]
HOST_SOURCES = ["kernels.cpp"]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError("command failed:\n  " + " ".join(cmd) + "\n" + r.stdout)
    return r.stdout


def _compile(src: str, out: str, extra=()):
    cmd = [HIPCC, *HIP_FLAGS, *extra, "-I", os.path.join(ROOT, "include"), "-c", src, "-o", out]
    _run(cmd)
    return out


def build(jobs: int = 4, verbose: bool = True) -> str:
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIB, exist_ok=True)
    objs = []
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        futs = []
        for s in SOURCES:
            o = os.path.join(OBJ, os.path.splitext(s)[0] + ".o")
            futs.append(ex.submit(_compile, os.path.join(CSRC, s), o))
            objs.append(o)
        for s in HOST_SOURCES:
            p = os.path.join(HOST, s)
            if os.path.exists(p):
                o = os.path.join(OBJ, "host_" + os.path.splitext(s)[0] + ".o")
                futs.append(ex.submit(_compile, p, o, ("-x", "hip", "-I", HOST)))
        for f in futs:
            f.result()
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", HOT_SO, *objs])
    host_objs = [os.path.join(OBJ, "host_" + os.path.splitext(s)[0] + ".o") for s in HOST_SOURCES
                 if os.path.exists(os.path.join(HOST, s))]
    if host_objs:
        _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", HOST_SO, *host_objs,
              "-L", LIB, "-lqimg_hot", "-Wl,-rpath,$ORIGIN"])
    if verbose:
        print(f"built {HOT_SO}")
    return HOT_SO


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=4)
    a = ap.parse_args()
    build(a.jobs)
    sys.exit(0)
