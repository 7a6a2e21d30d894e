"""The reference-signature C++ layer (qwen-image.cu_amd/host/kernels.h) via its
test program tests/cpp/test_host_api.cpp.

* CPU: invalid calls are rejected on the host before any HIP call, printing
  "qimg: <function>: <reason>" and exiting with status 1 (the reference's
  assert/exit behaviour, cuda_kernels.cu:2681-2686, sageattention_sm80.cu:975-978).
* GPU: the program runs the operators the way transformer.cu calls them and
  checks each against the CPU oracle (bit-exact where the arithmetic allows).
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "_build", "test_host_api")

REJECTIONS = {
    "out_shape": "linear_forward_int8: out is [4, 9], expected [4, 8]",
    "x_dtype": "linear_forward_int8: x must be FP32",
    "weight_k": "linear_forward_quantized: weight K=64 != input K=128",
    "mode_int4": "linear_forward_int4: svd_up [N, r] and svd_down [K, r] must be BF16",
    "awq_m": "linear_forward_awq: AWQ GEMV only supports M=1 (got 4)",
    "bf16_out_dtype": "linear_forward_quantized: out must be FP32",
    "scratch": "scratch 16 bytes < required",
    "hbs": "hbs=48 is not a power of two",
    "sage_head_dim": "head_dim 96 not supported",
    "block_pe": "mmdit_blocks_forward: pe must be [80, 64, 4]",
}


def _bin():
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is missing: run __graft_entry__.build()")
    return BIN


@pytest.mark.parametrize("case", sorted(REJECTIONS))
def test_host_layer_rejects_before_any_hip_call(case):
    r = subprocess.run([_bin(), "--expect-error", case], capture_output=True, text=True, timeout=60,
                       env={**os.environ, "HIP_VISIBLE_DEVICES": ""})
    assert r.returncode == 1, (r.returncode, r.stdout, r.stderr)
    assert r.stderr.startswith("qimg: ") and REJECTIONS[case] in r.stderr, r.stderr


@pytest.mark.gpu
def test_host_layer_parity_on_gpu():
    r = subprocess.run([_bin()], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "PASSED: 0 failure(s)" in r.stdout
