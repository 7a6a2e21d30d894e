"""Build recipe for the gfx950 hot-path libraries.

    lib/libqimg_hot.so   the kernels + C ABI (include/qimg_hot.h), from csrc/
    lib/libqimg_host.so  the reference-signature C++ layer (host/kernels.h)
                         over the C ABI
    lib/libqimg_probe.so the matrix-core rate probe bench.py reports the
                         kernels against (csrc/mfma_probe.hip; no product
                         code links it)
    tests/cpp/_build/test_host_api
                         the C++ layer's parity test program (links the CPU
                         oracle, so it is built only after oracle/ is)

Everything is compiled with hipcc for gfx950 only.

    python qwen-image.cu_amd/build.py            # libraries
    python qwen-image.cu_amd/build.py --tests    # libraries + test program
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
PROBE_SO = os.path.join(LIB, "libqimg_probe.so")
TEST_SRC = os.path.join(ROOT, "tests", "cpp", "test_host_api.cpp")
TEST_BIN = os.path.join(ROOT, "tests", "cpp", "_build", "test_host_api")
ORACLE_DIR = os.path.join(ROOT, "oracle")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# Packed fp32 VALU ops are disabled: the compiler would otherwise form
# v_pk_{add,mul,fma}_f32 from scalar float code.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]

SOURCES = ["hadamard_quant.hip", "gemm_w8a8.hip", "gemm_small_m.hip", "gemm_bf16.hip", "sage_attention.hip", "block_ops.hip",
           "mmdit_block.hip", "capi.hip", "linear_noalloc.hip", "int4.hip", "capi_int4.hip"]
HOST_SOURCES = ["kernels.cpp", "checkpoint.cpp"]
PROBE_SOURCE = "mfma_probe.hip"


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
    hot_objs, host_objs = [], []
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        futs = []
        for s in SOURCES:
            o = os.path.join(OBJ, os.path.splitext(s)[0] + ".o")
            futs.append(ex.submit(_compile, os.path.join(CSRC, s), o))
            hot_objs.append(o)
        for s in HOST_SOURCES:
            o = os.path.join(OBJ, "host_" + os.path.splitext(s)[0] + ".o")
            futs.append(ex.submit(_compile, os.path.join(HOST, s), o, ("-x", "hip", "-I", HOST)))
            host_objs.append(o)
        probe_obj = os.path.join(OBJ, "mfma_probe.o")
        futs.append(ex.submit(_compile, os.path.join(CSRC, PROBE_SOURCE), probe_obj))
        for f in futs:
            f.result()
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", HOT_SO, *hot_objs])
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", HOST_SO, *host_objs,
          "-L", LIB, "-lqimg_hot", "-Wl,-rpath,$ORIGIN"])
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", PROBE_SO, probe_obj])
    if verbose:
        print(f"built {HOT_SO}, {HOST_SO} and {PROBE_SO}")
    return HOT_SO


def build_tests(verbose: bool = True) -> str:
    """The C++ layer's test program; needs oracle/_build/libqimg_oracle.so."""
    oracle_lib = os.path.join(ORACLE_DIR, "_build")
    if not os.path.exists(os.path.join(oracle_lib, "libqimg_oracle.so")):
        raise RuntimeError("build the oracle first: make -C oracle")
    os.makedirs(os.path.dirname(TEST_BIN), exist_ok=True)
    rel_lib = os.path.relpath(LIB, os.path.dirname(TEST_BIN))
    rel_oracle = os.path.relpath(oracle_lib, os.path.dirname(TEST_BIN))
    _run([HIPCC, *HIP_FLAGS, "-x", "hip", "-I", HOST, "-I", os.path.join(ROOT, "include"), "-I", ORACLE_DIR,
          TEST_SRC, "-o", TEST_BIN, "-L", LIB, "-lqimg_host", "-lqimg_hot", "-L", oracle_lib, "-lqimg_oracle",
          f"-Wl,-rpath,$ORIGIN/{rel_lib}:$ORIGIN/{rel_oracle}"])
    if verbose:
        print(f"built {TEST_BIN}")
    return TEST_BIN


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=4)
    ap.add_argument("--tests", action="store_true")
    a = ap.parse_args()
    build(a.jobs)
    if a.tests:
        build_tests()
    sys.exit(0)
