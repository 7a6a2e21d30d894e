#!/usr/bin/env python3
"""Benchmark of the quantized-linear hot path on one MI355X.

Workload (one "step"): the MMDiT MLP pair at M = 4352 tokens (4096 image +
256 text):
    x bf16 [4352, 3072] --FWHT(1024)+int8--> fc1 3072->12288 (+bias, GELU-tanh,
    fp32 out, as the reference writes it) --FWHT(4096)+int8--> fc2 12288->3072
    (+bias, bf16 out)
with random N(0, 0.02) weights quantized by the library (W8A8 + Hadamard).
fc1 is issued as the two kernel launches one M = 4352 call makes (rows
0-4095 on the 256 x 256 tiles, rows 4096-4351 on the 128 x 128 tiles), as two
calls, so that each kernel is timed; the output is that of the single call.
Inputs are resident in HBM before timing. value = 2*M*N*K summed over both
GEMMs (657.13 GOP) / measured time, in TFLOP/s (int8 ops). The K timed steps
run twice: eagerly on one stream, with HIP events around each launch (the
per-kernel times), then as K back-to-back replays of the step captured in one
HIP graph between one event pair (the step time, span / K). In the graph,
rows 4096-4351 (their fc1 and fc2-input quantization) run on a second stream
beside rows 0-4095's fc1 and quantization, and fc2 joins the two; the output
must equal the eager steps' bit for bit. The one-stream step as a graph is
reported beside it.

Also printed in the same JSON line:
  roofline     the dominant kernel's achieved rate vs the int8 MFMA peak,
               from HIP events recorded around each launch in the eager steps
  cpu_baseline the CPU oracle (oracle/qimg_oracle.c, OpenMP) running the same
               MLP pair on the host cores
  extra        single linear (M=4096, 3072x3072), SageAttention (24 heads,
               S=4352, D=128), activation-quant bandwidth, and the small-M
               linears (modulation M=1/2 as HBM GB/s, text-stream M=256), and
               one MMDiT joint block at 4096 + 256 tokens (ms/block and the
               13-category split of transformer.cu:487-490), and the 60-block
               e4m3 step at 1328x1328 (6889 + 512 tokens, two CFG branches,
               sequential and batched)

    python bench.py [--steps K] [--warmup W] [--gpus 1]
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "qwen-image.cu_amd"))

METRIC = "quant-GEMM TFLOP/s (% MFMA peak); ms/MMDiT block @4096 img tokens"
PEAK_INT8_TOPS = 5033.0     # MI355X dense int8 MFMA
PEAK_FP16_TFLOPS = 2517.0   # MI355X dense fp16/bf16 MFMA
PEAK_HBM_GBS = 8000.0


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "mlp4352_hbm_traffic.txt")


def _traffic_from_profiles(kernel):
    """HBM bytes per launch of `kernel` (a key of the timed launch list)
    measured by rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs of this script,
    each scaled by the same counter's reading for a plain copy of known size;
    kept in profiles/mlp4352_hbm_traffic.txt as
    'traffic_bytes_per_launch <kernel>: N' lines. None if not measured."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    key = f"traffic_bytes_per_launch {kernel}:"
    for line in open(TRAFFIC_FILE):
        if line.startswith(key):
            try:
                return float(line.split(":", 1)[1])
            except ValueError:
                return None
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--ramp-s", type=float, default=1.0,
                    help="seconds of untimed steps before the warmup, so clocks are up when timing starts")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--calib-copy", action="store_true",
                    help="only run a plain 256 MiB device copy (HBM counter calibration) and exit")
    ap.add_argument("--c5-steps", type=int, default=20, help="timed steps of the 60-block C5 leg")
    ap.add_argument("--profile-commands", metavar="DIR",
                    help="print the rocprofv3 runs behind profiles/*.txt (output under DIR), one 'name<TAB>command' "
                         "line each, and exit")
    ap.add_argument("--summarize", metavar="DIR",
                    help="write the profiles/*.txt summaries from the CSVs of those runs under DIR, and exit")
    ap.add_argument("--profile-all", metavar="DIR",
                    help="run every --profile-commands run (each a child process under its own time limit, in "
                         "order, stopping at the first failure), then --summarize DIR; this process does not touch "
                         "the GPU itself")
    ap.add_argument("--summary-out", default=os.path.join(ROOT, "profiles"),
                    help="directory the --summarize files go to (default: profiles/)")
    ap.add_argument("--profile-set", choices=sorted(PROFILE_SETS),
                    help="only run the named group of measured workloads a few times each, untimed, for "
                         "rocprofv3 counter runs, and exit")
    args = ap.parse_args()

    if args.profile_commands:
        for name, cmd in _profile_commands(args.profile_commands):
            print(f"{name}\t{cmd}")
        return
    if args.profile_all:
        import shlex
        import subprocess
        args.profile_all = os.path.abspath(args.profile_all)
        os.makedirs(args.profile_all, exist_ok=True)
        for name, cmd in _profile_commands(args.profile_all):
            limit = 600 if name == "kt" else 240
            print(f"profile run {name}", flush=True)
            with open(os.path.join(args.profile_all, f"{name}.log"), "w") as log:
                r = subprocess.run(["timeout", "-s", "KILL", str(limit)] + shlex.split(cmd), stdout=log,
                                   stderr=subprocess.STDOUT, cwd=ROOT)
            if r.returncode != 0:
                print(f"profile run {name} failed: exit {r.returncode} (log {args.profile_all}/{name}.log)")
                sys.exit(1)
        args.summarize = args.profile_all
    if args.summarize:
        for f in _summarize(os.path.abspath(args.summarize), args.summary_out):
            print(os.path.join(args.summary_out, f))
        return

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this library has no multi-GPU path "
              "(run with --gpus 1).", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    if args.calib_copy:
        _calib_copy(torch)
        return

    import qimg_amd as q

    if args.profile_set:
        PROFILE_SETS[args.profile_set](q, torch, torch.device("cuda:0"))
        torch.cuda.synchronize()
        print(json.dumps({"profile_set": args.profile_set, "done": True}))
        return

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    g = torch.Generator(device="cpu").manual_seed(0)
    M, D, H = 4352, 3072, 12288

    # ---- synthetic inputs (seeded), weights quantized by the library
    x = torch.randn(M, D, generator=g).to(torch.bfloat16).to(dev)
    w1 = (torch.randn(H, D, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(D, H, generator=g) * 0.02).to(torch.bfloat16)
    b1 = (torch.randn(H, generator=g) * 0.01).to(torch.bfloat16)
    b2 = (torch.randn(D, generator=g) * 0.01).to(torch.bfloat16)
    qw1 = q.quantize_weight_tensor(w1.to(dev))
    qw2 = q.quantize_weight_tensor(w2.to(dev))
    b1d, b2d = b1.to(dev), b2.to(dev)
    h = torch.empty(M, H, dtype=torch.float32, device=dev)
    y = torch.empty(M, D, dtype=torch.bfloat16, device=dev)
    a1 = torch.empty(M, D, dtype=torch.int8, device=dev)
    s1 = torch.empty(M, dtype=torch.float32, device=dev)
    a2 = torch.empty(M, H, dtype=torch.int8, device=dev)
    s2 = torch.empty(M, dtype=torch.float32, device=dev)
    L = q.lib()
    stream = torch.cuda.current_stream(dev)
    P = q._ptr

    # fc1 of the 4352 rows is issued as the two kernel launches one
    # qimg_linear_prequantized call of M = 4352 makes (the dispatcher sends
    # rows 0-4095 to the 256 x 256 tiles, 768 tiles = exactly three rounds on
    # 256 CUs, and the trailing tile row to the 128 x 128 tiles), as two
    # calls, so that HIP events time each kernel; the outputs and the
    # one-stream step time equal those of the single call (measured
    # in-process: 395.4 against 395.9 us per step). extra.fc1_single_call_ms
    # times fc1 as that single call (its two kernels back to back, without
    # the events between them).
    MI, MT = 4096, M - 4096

    # (the stream is read at each call, so the same launches can be captured)
    def quant(src, dt, rows, K, hbs, dst, sc):
        q._check(L.qimg_quantize_activation(P(src), dt, rows, K, hbs, q.INT8_HADAMARD, P(dst), P(sc),
                                            q._stream(dev)))

    def gemm(act, sc, rows, w, bias, out, out_dt, gelu):
        q._check(L.qimg_linear_prequantized(P(act), P(sc), rows, act.shape[1], P(w.data), P(w.scales),
                                            w.data.shape[0], q.INT8_HADAMARD, P(bias), P(out), out_dt,
                                            gelu, q._stream(dev)))

    names = ["quant_fc1_in", "gemm_fc1", "gemm_fc1_tail", "quant_fc2_in", "gemm_fc2"]
    launches = [
        lambda: quant(x, q.BF16, M, D, 1024, a1, s1),
        lambda: gemm(a1, s1, MI, qw1, b1d, h, q.FP32, 1),
        lambda: gemm(a1[MI:], s1[MI:], MT, qw1, b1d, h[MI:], q.FP32, 1),
        lambda: quant(h, q.FP32, M, H, 4096, a2, s2),
        lambda: gemm(a2, s2, M, qw2, b2d, y, q.BF16, 0),
    ]

    def step(evs=None):
        cur = torch.cuda.current_stream(dev)
        for j, f in enumerate(launches):
            if evs is not None:
                evs[j].record(cur)
            f()
        if evs is not None:
            evs[len(launches)].record(cur)

    # The timed step: the same work, with rows 4096-4351 (fc1 on the 128 x 128
    # tiles, then their fc2-input quantization) on a second stream from the
    # fc1-input quantization on, so that they fill the CUs the main rows' fc1
    # rounds leave free and overlap the main rows' fc2-input quantization
    # (row-wise, so the quantized rows are the same bits); fc2 joins both.
    side = torch.cuda.Stream(dev)

    def step_two_streams():
        cur = torch.cuda.current_stream(dev)
        launches[0]()
        side.wait_stream(cur)
        with torch.cuda.stream(side):
            launches[2]()
            quant(h[MI:], q.FP32, MT, H, 4096, a2[MI:], s2[MI:])
        launches[1]()
        quant(h, q.FP32, MI, H, 4096, a2, s2)
        cur.wait_stream(side)
        launches[4]()

    # Clock ramp: the GPU raises its clocks only under sustained load (the
    # first few milliseconds of a burst run ~15% slower), so the step runs
    # untimed for --ramp-s seconds before the W warmup steps.
    t_ramp = time.perf_counter()
    while time.perf_counter() - t_ramp < args.ramp_s:
        for _ in range(20):
            step()
        torch.cuda.synchronize()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    K = args.steps
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(len(names) + 1)] for _ in range(K)]
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for i in range(K):
        step(ev[i])
    stop.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    total_ms = start.elapsed_time(stop)
    # medians over the K timed steps (per step, and per launch)
    step_ms = [ev[i][0].elapsed_time(ev[i][len(names)]) for i in range(K)]
    ms_step_eager = float(np.median(step_ms))
    per_kernel_ms = {n: float(np.median([ev[i][j].elapsed_time(ev[i][j + 1]) for i in range(K)]))
                     for j, n in enumerate(names)}
    y_eager = y.clone()

    # ---- the step on two streams captured as one HIP graph (without the host
    # launch gaps), replayed K times back to back between one event pair:
    # ms_per_step and value are that span / K (the throughput of consecutive
    # steps). Bracketing each replay with its own event pair instead adds a
    # gap per replay on some boxes (graph slower than eager); that median is
    # reported beside it, and so is the one-stream step as a graph.
    def graph_of(fn):
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            fn()
        torch.cuda.synchronize()
        return gr

    def replay_span(gr):
        t_ramp = time.perf_counter()
        while time.perf_counter() - t_ramp < min(args.ramp_s, 0.3):
            for _ in range(20):
                gr.replay()
            torch.cuda.synchronize()
        for _ in range(args.warmup):
            gr.replay()
        g0 = torch.cuda.Event(enable_timing=True)
        g1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        g0.record(stream)
        for i in range(K):
            gr.replay()
        g1.record(stream)
        torch.cuda.synchronize()
        return g0.elapsed_time(g1) / K, time.perf_counter() - t0

    graph = graph_of(step_two_streams)
    y.zero_()
    ms_step, wall_graph = replay_span(graph)
    # every replay computes what the eager one-stream steps computed
    graph_equals_eager = bool(torch.equal(y, y_eager))
    gev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(K)]
    torch.cuda.synchronize()
    for i in range(K):
        gev[i][0].record(stream)
        graph.replay()
        gev[i][1].record(stream)
    torch.cuda.synchronize()
    ms_step_bracketed = float(np.median([a.elapsed_time(b) for a, b in gev]))
    del graph
    graph = graph_of(step)
    y.zero_()
    ms_step_one_stream, _ = replay_span(graph)
    graph_equals_eager = graph_equals_eager and bool(torch.equal(y, y_eager))
    del graph
    # fc1 of all 4352 rows as one call (the dispatcher sends the trailing tile
    # row to the small tiles), for comparison with the split above
    ms_fc1_single = _time(torch, lambda: gemm(a1, s1, M, qw1, b1d, h, q.FP32, 1), iters=21)
    gemm_ops = 2.0 * M * D * H
    total_ops = 2 * gemm_ops
    value = total_ops / (ms_step * 1e-3) / 1e12

    # ---- roofline of the dominant kernel (main-stream launches)
    dom = max(per_kernel_ms, key=per_kernel_ms.get)
    if dom.startswith("gemm"):
        rows, Kd, Nd, ob = {"gemm_fc1": (MI, D, H, 4), "gemm_fc1_tail": (MT, D, H, 4),
                            "gemm_fc2": (M, H, D, 2)}[dom]
        dom_ops = 2.0 * rows * Kd * Nd
        achieved = dom_ops / (per_kernel_ms[dom] * 1e-3) / 1e12
        traffic = _traffic_from_profiles(dom)
        # algorithmic bytes: int8 activations + int8 weights + output + scales + bias
        gbytes = rows * Kd + Nd * Kd + rows * Nd * ob + 4 * (rows + Nd) + 2 * Nd
        kname = {"gemm_fc1": f"gemm_w8a8_kernel (int8, 16x16x64 MFMA), fc1 rows 0-4095: {rows}x{Nd}x{Kd}, "
                             "768 tiles of 256x256 = 3 rounds on 256 CUs",
                 "gemm_fc1_tail": f"gemm_w8a8_kernel (int8, 16x16x64 MFMA), fc1 rows 4096-4351: {rows}x{Nd}x{Kd}, "
                                  "192 tiles of 128x128, two per CU",
                 "gemm_fc2": f"gemm_w8a8_kernel (int8, 16x16x64 MFMA), fc2 {rows}x{Nd}x{Kd}"}[dom]
        roof = {"kernel": kname, "bound": "mfma", "achieved": round(achieved, 1),
                "peak": PEAK_INT8_TOPS, "unit": "TFLOP/s", "frac": round(achieved / PEAK_INT8_TOPS, 4),
                "traffic": traffic, "ops_per_launch": dom_ops, "bytes_per_launch": gbytes,
                "avg_launch_ms": round(per_kernel_ms[dom], 4)}
    else:
        rows = M
        Kd = D if dom == "quant_fc1_in" else H
        nbytes = rows * Kd * (2 if dom == "quant_fc1_in" else 4) + rows * Kd + 4 * rows
        achieved = nbytes / (per_kernel_ms[dom] * 1e-3) / 1e9
        roof = {"kernel": f"FWHT + int8 quantization ({dom})", "bound": "hbm", "achieved": round(achieved, 1),
                "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                "traffic": _traffic_from_profiles(dom), "bytes_per_launch": nbytes,
                "avg_launch_ms": round(per_kernel_ms[dom], 4)}

    extra = {"per_kernel_ms_median": {k: round(v, 4) for k, v in per_kernel_ms.items()},
             "fc1_single_call_ms": round(ms_fc1_single, 4),
             "fc1_single_call_tflops": round(2.0 * M * D * H / ms_fc1_single / 1e9, 1),
             "step_timing": "K back-to-back replays of the two-stream step captured as one HIP graph, span / K",
             "ms_per_step_graph_bracketed_median": round(ms_step_bracketed, 4),
             "ms_per_step_one_stream_graph": round(ms_step_one_stream, 4),
             "ms_per_step_eager": round(ms_step_eager, 4), "ms_per_step_eager_mean": round(total_ms / K, 4),
             "graph_equals_eager": graph_equals_eager,
             "wall_s_timed_eager": round(wall, 3), "wall_s_timed_graph": round(wall_graph, 3)}
    if not args.no_extra:
        extra.update(_extra(q, torch, dev, c5_steps=args.c5_steps))

    # ---- CPU baseline: the oracle on the same MLP pair (and, as a by-product,
    # a parity spot check of this run's GPU output on sampled rows)
    cpu = None
    if not args.no_cpu_baseline:
        cpu = _cpu_baseline(np, torch, x, w1, w2, b1, b2, y, M, D, H)
        cpu["c3_attention"] = _cpu_baseline_sage(np, torch, q, dev)

    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": K,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "MMDiT MLP pair, M=4352 tokens (4096 image + 256 text): FWHT1024+int8 quant, "
                               "fc1 3072->12288 +bias+GELU-tanh (fp32; rows 0-4095 and 4096-4351 as two launches), "
                               "FWHT4096+int8 quant, fc2 12288->3072 +bias (bf16); rows 4096-4351's fc1 and "
                               "fc2-input quant on a second stream",
                   "M": M, "hidden": D, "mlp": H, "weights": "N(0,0.02) -> W8A8 + Hadamard",
                   "frac_of_int8_peak": round(value / PEAK_INT8_TOPS, 4)},
        "roofline": roof,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line))


def _calib_copy(torch):
    """A plain device-to-device copy of 256 MiB, five times: the known-size
    reference that FETCH_SIZE / WRITE_SIZE readings are scaled by."""
    n = 256 << 20
    src = torch.ones(n // 4, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calib_copy_bytes": n, "copies": 5}))


def _time_cycle(torch, fns, iters=10, min_calls=20, ramp_s=0.2):
    """Median GPU time per call of `fns` (run in turn): the calls are captured
    into one HIP graph (at least `min_calls` calls) and the graph is replayed
    between two events, so host launch overhead is not part of the figure."""
    reps = max(1, -(-min_calls // len(fns)))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for f in fns:
            f()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(reps):
            for f in fns:
                f()
    # replay untimed for a while first: clocks ramp up under sustained load
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < ramp_s:
        graph.replay()
        torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    ts = []
    for _ in range(iters):
        e0.record()
        graph.replay()
        e1.record()
        e1.synchronize()
        ts.append(e0.elapsed_time(e1) / (reps * len(fns)))
    del graph
    return float(sorted(ts)[len(ts) // 2])


def _time(torch, fn, iters=10):
    return _time_cycle(torch, [fn], iters=iters)


def _c3_inputs(q, torch, dev, seed=3):
    """The C3 attention operands as the joint block makes them: fp32 N(0,1)
    Q, K, V rows of the 256 text and 4096 image tokens ([tokens, 24 x 128],
    drawn from torch.Generator('cpu').manual_seed(seed) in the order q_txt,
    q_img, k_txt, k_img, v_txt, v_img), per-head RMSNorm (eps 1e-6, weight 1)
    and RoPE (qwen_image_pe(128, 128, 2, 256)) on Q and K, text first, fp16
    [24, 4352, 128] (joint_heads_f16: cuda_kernels.cu:1656-1687, 1935-1962,
    transformer.cu:106-130, 617-674)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    n_txt, n_img = 256, 4096
    rows = [torch.randn(n, 3072, generator=g).to(dev) for n in (n_txt, n_img) * 3]
    ones = torch.ones(128, dtype=torch.bfloat16, device=dev)
    pe = torch.from_numpy(q.qwen_image_pe(128, 128, 2, n_txt)).to(dev)
    q16 = q.joint_heads_f16(rows[0], rows[1], ones, ones, pe)
    k16 = q.joint_heads_f16(rows[2], rows[3], ones, ones, pe)
    v16 = q.joint_heads_f16(rows[4], rows[5])
    torch.cuda.synchronize()
    return q16, k16, v16


PROBE_KINDS = {  # qimg_probe_mfma kind: (name, ops per instruction, spec peak in TOP/s, cycles per instruction)
    0: ("v_mfma_i32_32x32x32_i8", 65536, PEAK_INT8_TOPS, 32),
    1: ("v_mfma_i32_16x16x64_i8", 32768, PEAK_INT8_TOPS, 16),
    2: ("v_mfma_scale_f32_32x32x64_f8f6f4 (e4m3)", 131072, 5033.0, 64),
    3: ("v_mfma_f32_32x32x16_f16", 32768, PEAK_FP16_TFLOPS, 32),
    4: ("v_mfma_f32_32x32x16_bf16", 32768, PEAK_FP16_TFLOPS, 32),
    5: ("v_mfma_scale_f32_16x16x128_f8f6f4 (e4m3)", 65536, 5033.0, 32),
    6: ("v_mfma_f32_16x16x32_f16", 16384, PEAK_FP16_TFLOPS, 16),
}


def _mfma_ceiling(torch, dev, launches=12, timed=3):
    """The matrix cores' sustained rate on this GPU (lib/libqimg_probe.so,
    csrc/mfma_probe.hip): a register-only loop of one MFMA form on every SIMD
    (one or two waves per SIMD), `launches` back-to-back launches of ~10-20
    ms, the median of the last `timed` taken (the clock ramps under load). The
    shader clock comes from the waves' own s_memtime / s_memrealtime (100
    MHz) counters. frac_of_spec = rate / the spec peak (2.4 GHz);
    clock_ghz x 1024 SIMDs x ops per cycle is what that clock allows."""
    import ctypes
    import numpy as np
    lib = ctypes.CDLL(os.path.join(ROOT, "qwen-image.cu_amd", "lib", "libqimg_probe.so"))
    lib.qimg_probe_mfma.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                    ctypes.c_void_p, ctypes.c_void_p]
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    stream = torch.cuda.current_stream(dev)
    res = {}
    for kind, (name, ops, peak, cyc) in PROBE_KINDS.items():
        per_iter = lib.qimg_probe_mfma_per_iter(kind)
        iters = max(1, int(2.0e7 // (per_iter * cyc)))  # ~10 ms per wave at 2 GHz
        for wps in (1, 2):
            waves = cus * wps * 4
            clocks = torch.zeros(4 * waves, dtype=torch.int64, device=dev)
            sink = torch.zeros(cus * wps * 256, dtype=torch.int32, device=dev)
            ts = []
            for i in range(launches):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                st = lib.qimg_probe_mfma(kind, wps, cus, iters, ctypes.c_void_p(clocks.data_ptr()),
                                         ctypes.c_void_p(sink.data_ptr()), ctypes.c_void_p(stream.cuda_stream))
                e1.record(stream)
                if st != 0:
                    raise RuntimeError(f"qimg_probe_mfma({kind}, {wps}) failed: {st}")
                e1.synchronize()
                ts.append(e0.elapsed_time(e1))
            c = clocks.cpu().numpy().reshape(-1, 4).astype(np.float64)
            ghz = float(np.median((c[:, 1] - c[:, 0]) / np.maximum(c[:, 3] - c[:, 2], 1) * 0.1))
            ms = float(np.median(ts[-timed:]))
            total = float(ops) * per_iter * iters * waves
            tops = total / ms / 1e9
            res[f"{name} wps{wps}"] = {"tops": round(tops, 1), "frac_of_spec": round(tops / peak, 4),
                                       "clock_ghz": round(ghz, 3),
                                       "frac_at_clock": round(tops * 1e12 / (ops / cyc * 1024 * ghz * 1e9), 4),
                                       "ms": round(ms, 3)}
            del clocks, sink
    return res


def _vendor_gemms(torch, dev, iters=20):
    """hipBLASLt (through torch._int_mm and torch._scaled_mm) on this box at
    the quantized linears' shapes, as a vendor-library reference point: int8
    x int8 -> int32 [M, N] (no dequant epilogue) and e4m3 x e4m3 -> bf16
    with unit scales; each the median of `iters` eager calls between
    events. Operands are A [M, K] row-major times W [N, K] row-major (W^T
    passed as a column-major [K, N] view), as this library's GEMMs take them."""
    g = torch.Generator(device=dev).manual_seed(21)
    res = {}
    shapes = {"C1 4096x3072x3072": (4096, 3072, 3072), "fc1 4352x12288x3072": (4352, 12288, 3072),
              "fc2 4352x3072x12288": (4352, 3072, 12288), "C5 fc1 13778x12288x3072": (13778, 12288, 3072),
              "C5 fc2 13778x3072x12288": (13778, 3072, 12288)}
    f8 = getattr(torch, "float8_e4m3fn", None)
    for tag, (M, N, K) in shapes.items():
        a = torch.randint(-127, 128, (M, K), generator=g, device=dev, dtype=torch.int8)
        w = torch.randint(-127, 128, (N, K), generator=g, device=dev, dtype=torch.int8)
        ops = 2.0 * M * N * K
        entry = {}

        def timed(fn):
            for _ in range(3):
                fn()
            torch.cuda.synchronize()
            ts = []
            for _ in range(iters):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                fn()
                e1.record()
                ts.append((e0, e1))
            torch.cuda.synchronize()
            return sorted(e0.elapsed_time(e1) for e0, e1 in ts)[iters // 2]

        try:
            ms = timed(lambda: torch._int_mm(a, w.t()))
            entry["int8_ms"] = round(ms, 4)
            entry["int8_tops"] = round(ops / ms / 1e9, 1)
            entry["int8_frac_of_spec"] = round(ops / ms / 1e9 / PEAK_INT8_TOPS, 4)
        except Exception as ex:  # noqa: BLE001 - reported, not fatal
            entry["int8_error"] = str(ex)[:200]
        if f8 is not None:
            try:
                af = (torch.randn(M, K, generator=g, device=dev) * 0.5).to(f8)
                wf = (torch.randn(N, K, generator=g, device=dev) * 0.5).to(f8)
                one = torch.ones((), device=dev)
                ms = timed(lambda: torch._scaled_mm(af, wf.t(), scale_a=one, scale_b=one, out_dtype=torch.bfloat16))
                entry["e4m3_ms"] = round(ms, 4)
                entry["e4m3_tflops"] = round(ops / ms / 1e9, 1)
                entry["e4m3_frac_of_spec"] = round(ops / ms / 1e9 / 5033.0, 4)
                del af, wf
            except Exception as ex:  # noqa: BLE001
                entry["e4m3_error"] = str(ex)[:200]
        res[tag] = entry
        del a, w
    return res


def _extra(q, torch, dev, c5_steps=20):
    out = {}
    g = torch.Generator(device="cpu").manual_seed(0)
    # C1: single linear, M=4096, 3072x3072 (bf16 in, fp32 out as the reference)
    M, K, N = 4096, 3072, 3072
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    b = (torch.randn(N, generator=g) * 0.01).to(torch.bfloat16).to(dev)
    qw = q.quantize_weight_tensor(w)
    o32 = torch.empty(M, N, device=dev)
    scratch = torch.empty(q.int8_scratch_bytes(M, K, N), dtype=torch.uint8, device=dev)
    aq, asc = q.quantize_activation_hadamard(x, 1024)
    ms_lin = _time(torch, lambda: q.linear_forward_quantized(x, qw, b, out=o32, scratch=scratch))
    ms_gemm = _time(torch, lambda: q.linear_forward_prequantized(aq, asc, qw, b, out=o32))
    ops = 2.0 * M * N * K
    out["linear_c1_ms"] = round(ms_lin, 4)
    out["linear_c1_tflops"] = round(ops / ms_lin / 1e9, 1)
    out["linear_c1_gemm_only_tflops"] = round(ops / ms_gemm / 1e9, 1)
    # the same linear with bf16 out (the config's output type; fp32 above is
    # the reference's linear_forward_quantized output)
    o16 = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    ms_lin16 = _time(torch, lambda: q.linear_forward_quantized(x, qw, b, out=o16, scratch=scratch))
    ms_gemm16 = _time(torch, lambda: q.linear_forward_prequantized(aq, asc, qw, b, out=o16))
    out["linear_c1_bf16out_ms"] = round(ms_lin16, 4)
    out["linear_c1_bf16out_tflops"] = round(ops / ms_lin16 / 1e9, 1)
    out["linear_c1_bf16out_gemm_only_tflops"] = round(ops / ms_gemm16 / 1e9, 1)
    out["linear_c1_gemm_only_frac"] = round(ops / ms_gemm / 1e9 / 5033.0, 4)
    out["linear_c1_bf16out_gemm_only_frac"] = round(ops / ms_gemm16 / 1e9 / 5033.0, 4)
    ms_q = _time(torch, lambda: q.quantize_activation_hadamard(x, 1024))
    out["act_quant_c1_gbs"] = round((M * K * 3 + 4 * M) / ms_q / 1e6, 1)
    # C3: SageAttention, 24 heads, S = 4352 (256 text + 4096 image tokens),
    # D = 128, on its configured inputs: Q, K, V fp32 N(0,1) as the text and
    # image streams' [tokens, 24 x 128] rows; Q and K get the per-head RMSNorm
    # (eps 1e-6, weight 1) and the Qwen-Image RoPE of a 64 x 64 latent grid
    # (qwen_image_pe(128, 128, 2, 256), text tokens first), all three are
    # concatenated text first and transposed to fp16 [24, 4352, 128] by
    # joint_heads_f16 (the block's pre-attention pass). Output: fp16 [24,
    # 4352, 128] (head-major, what the block's out-projection quantization
    # reads) and bf16 in the same layout; the config's bf16 [1, 4352, 24,
    # 128] is the same values with heads and tokens swapped.
    q16, k16, v16 = _c3_inputs(q, torch, dev)
    BH, S, Dh = q16.shape
    ao = torch.empty(BH, S, Dh, dtype=torch.float16, device=dev)
    ab = torch.empty(BH, S, Dh, dtype=torch.bfloat16, device=dev)
    sscr = torch.empty(q.sage_scratch_bytes(BH, S, Dh), dtype=torch.uint8, device=dev)
    sc = 1.0 / math.sqrt(128.0)
    ms_att = _time(torch, lambda: q.attention_forward_sage_fp16io(q16, k16, v16, sc, out=ao, scratch=sscr),
                   iters=21)
    ms_att_bf = _time(torch, lambda: q.attention_forward_sage_fp16io(q16, k16, v16, sc, out=ab, scratch=sscr),
                      iters=21)
    qi, qs = q.sage_quant_q(q16)
    km = q.sage_k_mean(k16)
    ki, ks = q.sage_quant_k(k16, km)
    ms_core = _time(torch, lambda: q.sage_attn_quantized(qi, ki, v16, qs, ks, sc, scratch=sscr), iters=21)
    flops = 4.0 * BH * S * S * Dh
    out["sage_c3_inputs"] = ("Q,K,V fp32 N(0,1) [4352, 24x128] (256 txt + 4096 img); RMSNorm (eps 1e-6, w 1) + "
                             "RoPE(qwen_image_pe(128,128,2,256)) on Q,K; fp16 [24,4352,128] via joint_heads_f16")
    out["sage_c3_output"] = "fp16 [24,4352,128] head-major (sage_c3_ms); bf16 same layout (sage_c3_bf16out_ms)"
    out["sage_c3_ms"] = round(ms_att, 4)
    out["sage_c3_bf16out_ms"] = round(ms_att_bf, 4)
    out["sage_c3_tflops"] = round(flops / ms_att / 1e9, 1)
    out["sage_c3_attn_kernel_ms"] = round(ms_core, 4)
    out["sage_c3_attn_kernel_tflops"] = round(flops / ms_core / 1e9, 1)
    out["sage_c3_frac_of_mixed_peak"] = round(flops / ms_att / 1e9 / 3355.0, 4)
    out["sage_c3_attn_kernel_frac_of_mixed_peak"] = round(flops / ms_core / 1e9 / 3355.0, 4)
    del q16, k16, v16, ao, ab, sscr, qi, ki, km
    # Small M: modulation (M = 1, and 2 rows for a CFG pair; 18432 x 3072)
    # and text-stream linears (M = 256). HBM bytes = int8 weights + scales +
    # bias + activations + fp32 outputs, each once. Each call uses the next
    # of several weight copies (> 600 MB in all), so weights come from HBM
    # and not from the 256 MB last-level cache, as in a forward pass.
    for tag, (M, N, K, gelu) in {"mod_m1": (1, 18432, 3072, False), "mod_m2": (2, 18432, 3072, False),
                                 "txt_qkv_m256": (256, 3072, 3072, False),
                                 "txt_fc1_m256": (256, 12288, 3072, True),
                                 "txt_fc2_m256": (256, 3072, 12288, False)}.items():
        x = torch.randn(M, K, generator=g).to(dev)
        w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(dev)
        b = (torch.randn(N, generator=g) * 0.01).to(torch.bfloat16).to(dev)
        qw0 = q.quantize_weight_tensor(w)
        del w
        copies = max(2, -(-600_000_000 // (N * K)))
        qws = [q.QuantizedWeight(qw0.data.clone(), qw0.scales.clone(), qw0.had_block_size, qw0.mode)
               for _ in range(copies)]
        o32 = torch.empty(M, N, device=dev)
        scratch = torch.empty(q.int8_scratch_bytes(M, K, N), dtype=torch.uint8, device=dev)
        aq, asc = q.quantize_activation_hadamard(x, qw0.had_block_size)

        def gemm(qw):
            return lambda: q.linear_forward_prequantized(aq, asc, qw, b, apply_gelu=gelu, out=o32)

        def lin(qw):
            return lambda: q.linear_forward_quantized(x, qw, b, out=o32, scratch=scratch, apply_gelu=gelu)

        ms_g = _time_cycle(torch, [gemm(w_) for w_ in qws])
        ms_l = _time_cycle(torch, [lin(w_) for w_ in qws])
        with q.linear_kernel(q.LINEAR_LARGE_TILE):
            ms_big = _time_cycle(torch, [gemm(w_) for w_ in qws])
        if M <= 32:
            with q.linear_kernel(q.LINEAR_SMALL_32):
                out[f"{tag}_mfma32_gemm_us"] = round(_time_cycle(torch, [gemm(w_) for w_ in qws]) * 1e3, 2)
        nbytes = N * K + 4 * N + 2 * N + M * K + 4 * M + 4 * M * N
        out[f"{tag}_gemm_us"] = round(ms_g * 1e3, 2)
        out[f"{tag}_gemm_gbs"] = round(nbytes / ms_g / 1e6, 1)
        out[f"{tag}_gemm_tops"] = round(2.0 * M * N * K / ms_g / 1e9, 1)
        out[f"{tag}_linear_us"] = round(ms_l * 1e3, 2)
        out[f"{tag}_large_tile_gemm_us"] = round(ms_big * 1e3, 2)
        del qws, qw0
    out.update(_block_c4(q, torch, dev, g))
    out.update(_step_c5(q, torch, dev, steps=c5_steps))
    out["mfma_ceiling"] = _mfma_ceiling(torch, dev)
    out["hipblaslt_reference"] = _vendor_gemms(torch, dev)
    return out


def _step_c5(q, torch, dev, n_blocks=60, steps=20):
    """One denoising step's transformer blocks at 1328x1328: 60 MMDiT joint
    blocks over 6889 image + 512 text tokens with e4m3 weights (FWHT front
    end, N(0, 0.02) weights, N(0, 0.01) biases, RMSNorm weights 1), for the
    two classifier-free-guidance branches (main.cu:761-773), run as two
    sequential forwards and as one forward of batch 2. The weights (20.4 GB)
    are drawn on the GPU; every block has its own. Each figure is the median
    of `steps` steps, each between its own pair of events."""
    n_img, n_txt, D, F = 83 * 83, 512, 3072, 12288
    gen = torch.Generator(device=dev).manual_seed(5)
    shapes = {"img_mod": (6 * D, D), "txt_mod": (6 * D, D)}
    for n in ("to_q", "to_k", "to_v", "add_q_proj", "add_k_proj", "add_v_proj", "to_out", "to_add_out"):
        shapes[n] = (D, D)
    for s in ("img", "txt"):
        shapes[f"{s}_mlp_fc1"] = (F, D)
        shapes[f"{s}_mlp_fc2"] = (D, F)
    ones = torch.ones(128, dtype=torch.bfloat16, device=dev)
    norms = {n: ones for n in ("norm_q", "norm_k", "norm_added_q", "norm_added_k")}
    t_build = time.perf_counter()
    blocks = []
    for _ in range(n_blocks):
        W, B = {}, {}
        for n, (N, K) in shapes.items():
            w = (torch.randn(N, K, generator=gen, device=dev) * 0.02).to(torch.bfloat16)
            W[n] = q.quantize_weight_tensor(w, mode=q.FP8_HADAMARD)
            B[n] = (torch.randn(N, generator=gen, device=dev) * 0.01).to(torch.bfloat16)
            del w
        blocks.append((W, B, norms))
    table = q.BlockTable(blocks)
    torch.cuda.synchronize()
    build_s = time.perf_counter() - t_build
    img0 = torch.randn(n_img, D, generator=gen, device=dev)
    txts = [torch.randn(n_txt, D, generator=gen, device=dev) for _ in range(2)]
    t_emb = torch.randn(D, generator=gen, device=dev)
    pe = torch.from_numpy(q.qwen_image_pe(166, 166, 2, n_txt)).to(dev)
    assert pe.shape[0] == n_img + n_txt
    sc1 = torch.empty(q.mmdit_block_scratch_bytes(n_img, n_txt, 1), dtype=torch.uint8, device=dev)
    sc2 = torch.empty(q.mmdit_block_scratch_bytes(n_img, n_txt, 2), dtype=torch.uint8, device=dev)
    seq = [(img0.clone(), t.clone()) for t in txts]
    bat_img = torch.stack([img0, img0]).contiguous()
    bat_txt = torch.stack(txts).contiguous()

    def run_seq():
        for i, t in seq:
            q.mmdit_blocks_forward(table, i, t, t_emb, pe, scratch=sc1)

    def run_bat():
        q.mmdit_blocks_forward(table, bat_img, bat_txt, t_emb, pe, scratch=sc2)

    res, spread = {}, {}
    for tag, fn in (("seq", run_seq), ("batched", run_bat)):
        fn()  # warm-up step
        torch.cuda.synchronize()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        for e0, e1 in ev:
            e0.record()
            fn()
            e1.record()
        torch.cuda.synchronize()
        ts = sorted(e0.elapsed_time(e1) for e0, e1 in ev)
        res[tag] = ts[len(ts) // 2]
        spread[tag] = (ts[0], ts[-1])
    prof = q.mmdit_blocks_forward(table, bat_img, bat_txt, t_emb, pe, scratch=sc2, profile=True)
    finite = all(bool(torch.isfinite(x).all().item()) for x in (bat_img, bat_txt, seq[0][0], seq[1][1]))
    S = n_img + n_txt
    lin = 0.0
    for n, (N, K) in shapes.items():
        rows = 1 if n.endswith("_mod") else (n_txt if n.startswith(("txt", "add_")) or n == "to_add_out" else n_img)
        lin += 2.0 * rows * N * K
    att = 4.0 * 24 * S * S * 128
    step_ops = 2 * n_blocks * (lin + att)
    del table, blocks
    return {"step_c5_seq_ms": round(res["seq"], 2), "step_c5_batched_ms": round(res["batched"], 2),
            "step_c5_timing": f"median of {steps} steps each (min-max: seq {spread['seq'][0]:.2f}-"
                              f"{spread['seq'][1]:.2f}, batched {spread['batched'][0]:.2f}-{spread['batched'][1]:.2f} ms)",
            "step_c5_top": round(step_ops / 1e12, 2),
            "step_c5_seq_tflops": round(step_ops / res["seq"] / 1e9, 1),
            "step_c5_batched_tflops": round(step_ops / res["batched"] / 1e9, 1),
            "step_c5_batched_categories_ms": {k: round(v, 3) for k, v in prof.items()},
            "step_c5_weights_build_s": round(build_s, 1), "step_c5_finite": finite}


def _block_c4(q, torch, dev, g, copies=2, blocks=8, profiled=10):
    """One MMDiT joint block at 4096 image + 256 text tokens
    (transformer.cu:497-836): W8A8 + Hadamard linears with N(0, 0.02)
    weights and N(0, 0.01) biases, RMSNorm weights 1, the Qwen-Image RoPE
    table for a 64x64 latent grid, SageAttention. `copies` weight sets
    (340 MB each) alternate so weights stream from HBM as in a 60-block
    forward. ms/block: the median over 21 replays of a HIP graph of one
    qimg_mmdit_blocks_forward call over `blocks` consecutive blocks, divided
    by `blocks` (block_c4_single_call_ms: the same blocks as single-block
    calls); the 13-category split from events around each category (no
    synchronisation between categories), averaged over the blocks of eager
    multi-block calls (`profiled` blocks or more)."""
    n_img, n_txt, D, MLPD = 4096, 256, 3072, 12288
    shapes = {"img_mod": (6 * D, D), "txt_mod": (6 * D, D)}
    for n in ("to_q", "to_k", "to_v", "add_q_proj", "add_k_proj", "add_v_proj", "to_out", "to_add_out"):
        shapes[n] = (D, D)
    for s in ("img", "txt"):
        shapes[f"{s}_mlp_fc1"] = (MLPD, D)
        shapes[f"{s}_mlp_fc2"] = (D, MLPD)
    sets = []
    for _ in range(copies):
        W, B = {}, {}
        for n, (N, K) in shapes.items():
            w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(dev)
            W[n] = q.quantize_weight_tensor(w)
            B[n] = (torch.randn(N, generator=g) * 0.01).to(torch.bfloat16).to(dev)
            del w
        sets.append((W, B))
    ones = torch.ones(128, dtype=torch.bfloat16, device=dev)
    norms = {n: ones for n in ("norm_q", "norm_k", "norm_added_q", "norm_added_k")}
    img = torch.randn(n_img, D, generator=g).to(dev)
    txt = torch.randn(n_txt, D, generator=g).to(dev)
    t_emb = torch.randn(D, generator=g).to(dev)
    pe = torch.from_numpy(q.qwen_image_pe(128, 128, 2, n_txt)).to(dev)
    scratch = torch.empty(q.mmdit_block_scratch_bytes(n_img, n_txt), dtype=torch.uint8, device=dev)
    img0, txt0 = img.clone(), txt.clone()

    # The blocks as a forward runs them: one qimg_mmdit_blocks_forward call
    # over `blocks` blocks (silu(t_emb) and its quantization once per call,
    # as in the 60-block step); the single-block entry point, which redoes
    # them in every call as transformer.cu:506-512 does per block, is timed
    # beside it.
    table = q.BlockTable([(sets[i % copies][0], sets[i % copies][1], norms) for i in range(blocks)])

    def block(i):
        W, B = sets[i % copies]
        return lambda: q.mmdit_block_forward(W, B, norms, img, txt, t_emb, pe, scratch=scratch)

    ms_graph = _time_cycle(torch, [lambda: q.mmdit_blocks_forward(table, img, txt, t_emb, pe, scratch=scratch)],
                           iters=21, min_calls=1, ramp_s=0.5) / blocks
    fns = [block(i) for i in range(blocks)]
    ms_single = _time_cycle(torch, fns, iters=21, min_calls=blocks, ramp_s=0.5)
    img.copy_(img0)
    txt.copy_(txt0)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    q.mmdit_blocks_forward(table, img, txt, t_emb, pe, scratch=scratch)
    torch.cuda.synchronize()
    ms_eager = (time.perf_counter() - t0) * 1e3 / blocks
    cats = {}
    for _ in range(max(1, profiled // blocks)):
        for k, v in q.mmdit_blocks_forward(table, img, txt, t_emb, pe, scratch=scratch, profile=True).items():
            cats[k] = cats.get(k, 0.0) + v / (blocks * max(1, profiled // blocks))
    finite = bool(torch.isfinite(img).all().item() and torch.isfinite(txt).all().item())
    S = n_img + n_txt
    lin_ops = sum(2.0 * (n_img if not n.startswith(("txt", "add_")) and n != "to_add_out" else n_txt) * N * K
                  for n, (N, K) in shapes.items() if not n.endswith("_mod"))
    lin_ops += 2 * 2.0 * shapes["img_mod"][0] * D
    att_ops = 4.0 * 24 * S * S * 128
    return {"block_c4_ms": round(ms_graph, 4), "block_c4_eager_ms": round(ms_eager, 4),
            "block_c4_single_call_ms": round(ms_single, 4),
            "block_c4_gop": round((lin_ops + att_ops) / 1e9, 2),
            "block_c4_tflops": round((lin_ops + att_ops) / ms_graph / 1e9, 1),
            "block_c4_categories_ms": {k: round(v, 4) for k, v in cats.items()},
            "block_c4_finite": finite}


def _cpu_baseline(np, torch, x, w1, w2, b1, b2, y_gpu, M, D, H, min_seconds=10.0, max_runs=20):
    """The oracle (oracle/qimg_oracle.c, OpenMP over rows) computing the same
    MLP pair on the host cores: weight quantization is done once (it is not
    part of a step), then FWHT+quant, exact int32 GEMM, dequant+bias+GELU,
    FWHT(4096)+quant, GEMM, dequant+bias, repeated until at least
    `min_seconds` of CPU work. The first run's output also checks this run's
    GPU output on sampled rows."""
    from oracle import oracle as o

    def bits(t):
        return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)

    threads = o.get_threads()
    xb = bits(x)
    w1q, w1s, _ = o.quantize_weight_bf16(bits(w1))
    w2q, w2s, _ = o.quantize_weight_bf16(bits(w2))
    b1b, b2b = bits(b1), bits(b2)

    def step():
        hq, hs = o.quantize_activation(xb, 1024)
        hh = o.dequant_epilogue(o.gemm_s8s8s32(hq, w1q), hs, w1s, b1b, gelu=True)
        q2, s2 = o.quantize_activation(hh, 4096)
        return o.dequant_epilogue(o.gemm_s8s8s32(q2, w2q), s2, w2s, b2b, gelu=False)

    runs, t0 = 0, time.perf_counter()
    y_ref = step()
    runs += 1
    while time.perf_counter() - t0 < min_seconds and runs < max_runs:
        step()
        runs += 1
    dt = time.perf_counter() - t0
    ops = 2 * 2.0 * M * D * H
    rows = [0, 1234, 4095, 4096, 4351]
    y_ref_r = np.stack([o.bf16_bits_to_f32(o.bf16_bits_from_f32(y_ref[r])) for r in rows])
    y_got = y_gpu[rows].float().cpu().numpy()
    parity_rel = float(np.max(np.abs(y_got - y_ref_r)) / np.max(np.abs(y_ref_r)))
    return {"value": round(runs * ops / dt / 1e12, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"full MLP pair (M={M}) through the C oracle, {runs} runs in {dt:.1f} s",
            "cpu": _cpu_model(), "gpu_parity_max_rel_5rows": parity_rel}


def _cpu_model():
    """The host CPU as /proc/cpuinfo and sysfs describe it: model name,
    family/model/stepping, logical CPUs visible to this process, and the
    widest x86 vector extension present."""
    info = {}
    try:
        for line in open("/proc/cpuinfo"):
            if ":" in line:
                k, v = (t.strip() for t in line.split(":", 1))
                info.setdefault(k, v)
    except OSError:
        return "unknown"
    flags = info.get("flags", "").split()
    vec = next((f for f in ("avx512f", "avx2", "avx") if f in flags), "none")
    try:
        visible = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        visible = os.cpu_count()
    return (f"{info.get('model name', '?')} (family {info.get('cpu family', '?')} model {info.get('model', '?')} "
            f"stepping {info.get('stepping', '?')}, {visible} logical CPUs visible, {vec})")


def _cpu_baseline_sage(np, torch, q, dev, min_seconds=10.0, heads_per_run=2):
    """The C3 attention (24 heads, S = 4352, D = 128, sm_scale 1/sqrt(128), on
    the configured inputs of _c3_inputs: RMSNorm + RoPE on Q and K) through
    the oracle's SageAttention (K mean, per-thread Q/K int8 quant, integer
    QK^T, online softmax, fp16 PV) on the host cores, `heads_per_run` heads at
    a time over successive heads until `min_seconds` of CPU work; the first
    sample's heads are also compared with the GPU's output."""
    from oracle import oracle as o
    q16, k16, v16 = _c3_inputs(q, torch, dev)
    BH, S, D = q16.shape
    qh, kh, vh = (t.cpu().numpy() for t in (q16, k16, v16))
    sc = 1.0 / math.sqrt(128.0)
    heads = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < min_seconds and heads < BH:
        h0, h1 = heads, min(BH, heads + heads_per_run)
        ref = o.sage_attention_fp16io(qh[h0:h1], kh[h0:h1], vh[h0:h1], sc)
        if h0 == 0:
            ref0 = ref.astype(np.float32)
        heads = h1
    dt = time.perf_counter() - t0
    # GPU parity on the first sample's heads
    got = q.attention_forward_sage_fp16io(q16[:heads_per_run].contiguous(), k16[:heads_per_run].contiguous(),
                                          v16[:heads_per_run].contiguous(), sc, out_dtype=torch.float16)
    worst = float(np.max(np.abs(got.float().cpu().numpy() - ref0)) / np.max(np.abs(ref0)))
    flops = 4.0 * heads * S * S * D
    return {"value": round(flops / dt / 1e9, 2), "unit": "GFLOP/s", "cores": o.get_threads(), "kind": "port",
            "sample": f"{heads} of the 24 heads (S={S}, D={D}, RMSNorm+RoPE inputs) through the C oracle's "
                      f"SageAttention in {dt:.1f} s",
            "gpu_max_rel_vs_oracle": worst}


# ---- workloads for rocprofv3 counter runs (bench.py --profile-set NAME):
# each runs its kernels a few times, untimed; the counters per dispatch are
# read from the profiler's output by kernel name and grid size.
def _profile_gemm(q, torch, dev, reps=4):
    """Large-tile GEMMs: C1 (4096 x 3072 x 3072, int8, fp32 out + bias), the
    MLP pair at 4352 tokens (int8; fc1 GELU fp32 out, fc2 bf16 out), and the
    batch-2 e4m3 fc1 / fc2 of the 1328x1328 step (13778 rows)."""
    g = torch.Generator(device=dev).manual_seed(11)

    def problem(M, N, K, mode):
        a = torch.randn(M, K, generator=g, device=dev)
        w = (torch.randn(N, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        qw = q.quantize_weight_tensor(w, mode=mode)
        aq, asc = q.quantize_activation_hadamard(a, qw.had_block_size, mode)
        b = (torch.randn(N, generator=g, device=dev) * 0.01).to(torch.bfloat16)
        return aq, asc, qw, b

    for (M, N, K, mode, gelu, odt) in ((4096, 3072, 3072, q.INT8_HADAMARD, False, torch.float32),
                                       (4352, 12288, 3072, q.INT8_HADAMARD, True, torch.float32),
                                       (4352, 3072, 12288, q.INT8_HADAMARD, False, torch.bfloat16),
                                       (13778, 12288, 3072, q.FP8_HADAMARD, True, torch.float32),
                                       (13778, 3072, 12288, q.FP8_HADAMARD, False, torch.float32)):
        aq, asc, qw, b = problem(M, N, K, mode)
        out = torch.empty(M, N, dtype=odt, device=dev)
        for _ in range(reps):
            q.linear_forward_prequantized(aq, asc, qw, b, apply_gelu=gelu, out=out)
        torch.cuda.synchronize()
        del aq, asc, qw, b, out


def _profile_sage(q, torch, dev, reps=4):
    """SageAttention at C3 (24 heads, S = 4352, on the C3 leg's RMSNorm +
    RoPE inputs): K mean, Q/K quantization and the attention kernel; and the
    K mean of the batch-2 1328x1328 block (48 heads, S = 7401)."""
    g = torch.Generator(device=dev).manual_seed(12)
    for BH, S in ((24, 4352), (48, 7401)):
        if BH == 24:
            qh, kh, vh = _c3_inputs(q, torch, dev)
        else:
            kh = torch.randn(BH, S, 128, generator=g, device=dev).half()
        scratch = torch.empty(q.sage_scratch_bytes(BH, S, 128), dtype=torch.uint8, device=dev)
        for _ in range(reps):
            km = q.sage_k_mean(kh)
            if BH == 24:
                qi, qs = q.sage_quant_q(qh)
                ki, ks = q.sage_quant_k(kh, km)
                q.sage_attn_quantized(qi, ki, vh, qs, ks, 1.0 / math.sqrt(128.0), scratch=scratch)
        torch.cuda.synchronize()
        del kh, scratch


def _profile_small_m(q, torch, dev, reps=3):
    """The small-M linears (GEMM only) as bench.py's extra leg runs them:
    modulation (M = 1 and 2, 18432 x 3072) and the text-stream linears at
    M = 256, each over weight copies totalling > 600 MB so the weights come
    from HBM."""
    g = torch.Generator(device=dev).manual_seed(13)
    for M, N, K, gelu in ((1, 18432, 3072, False), (2, 18432, 3072, False), (256, 3072, 3072, False),
                          (256, 12288, 3072, True), (256, 3072, 12288, False)):
        x = torch.randn(M, K, generator=g, device=dev)
        w = (torch.randn(N, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        qw0 = q.quantize_weight_tensor(w)
        b = (torch.randn(N, generator=g, device=dev) * 0.01).to(torch.bfloat16)
        copies = max(2, -(-600_000_000 // (N * K)))
        qws = [q.QuantizedWeight(qw0.data.clone(), qw0.scales.clone(), qw0.had_block_size, qw0.mode)
               for _ in range(copies)]
        aq, asc = q.quantize_activation_hadamard(x, qw0.had_block_size)
        out = torch.empty(M, N, device=dev)
        for _ in range(reps):
            for qw in qws:
                q.linear_forward_prequantized(aq, asc, qw, b, apply_gelu=gelu, out=out)
        torch.cuda.synchronize()
        del qws, qw0, w, out


def _profile_quant(q, torch, dev, reps=4):
    """Activation FWHT + quantization passes: the fc1 input (bf16 4352 x
    3072, block 1024), the fc2 input (fp32 4352 x 12288, block 4096, int8)
    and the batch-2 e4m3 fc2 input of the 1328x1328 block (13778 x 12288);
    and the LayerNorm + modulate + quantization of 4096 x 3072 rows."""
    g = torch.Generator(device=dev).manual_seed(14)
    for M, K, hbs, mode, dt in ((4352, 3072, 1024, q.INT8_HADAMARD, torch.bfloat16),
                                (4352, 12288, 4096, q.INT8_HADAMARD, torch.float32),
                                (13778, 12288, 4096, q.FP8_HADAMARD, torch.float32)):
        x = torch.randn(M, K, generator=g, device=dev).to(dt)
        for _ in range(reps):
            q.quantize_activation_hadamard(x, hbs, mode)
        torch.cuda.synchronize()
        del x
    x = torch.randn(4096, 3072, generator=g, device=dev)
    shift = torch.randn(3072, generator=g, device=dev)
    scale = torch.randn(3072, generator=g, device=dev) * 0.1
    for _ in range(reps):
        q.layer_norm_modulate_quant(x, shift, scale, 1024, q.INT8_HADAMARD)
    torch.cuda.synchronize()


PROFILE_SETS = {"gemm": _profile_gemm, "sage": _profile_sage, "small_m": _profile_small_m,
                "quant": _profile_quant}


# ---- the rocprofv3 runs behind profiles/*.txt (bench.py --profile-commands
# DIR prints them, one "name<TAB>command" line each, to be run in order from
# any directory) and their summaries (bench.py --summarize DIR --summary-out
# OUT turns the CSVs those runs leave under DIR into OUT/*.txt, the files kept
# under profiles/). Counter conventions:
#  - FETCH_SIZE / WRITE_SIZE are KiB per dispatch between L2 and memory (L2
#    misses and write-backs; last-level-cache hits count as fetches), each
#    scaled by what the same counter reads for a plain device copy of 256 MiB
#    (the calib_* runs);
#  - MfmaUtil = sum(SQ_VALU_MFMA_BUSY_CYCLES) / (GRBM_GUI_ACTIVE per XCD x
#    1024 SIMDs), GRBM_GUI_ACTIVE being read summed over the 8 XCDs; the clock
#    is GRBM cycles per XCD / duration.
PMC_MFMA = ("SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE SQ_BUSY_CYCLES SQ_WAVE_CYCLES SQ_INSTS_VALU_MFMA_MOPS_I8 "
            "SQ_INSTS_VALU_MFMA_MOPS_F8 SQ_INSTS_VALU_MFMA_MOPS_F16")
KT_ARGS = "--steps 10 --warmup 3 --ramp-s 0.3 --no-cpu-baseline --c5-steps 3"
MLP_ARGS = "--steps 3 --warmup 1 --ramp-s 0.2 --no-cpu-baseline --no-extra"


def _profile_commands(d):
    """(name, command) of every profiling run, output under directory d; the
    commands run from the repository root (paths under it are given relative
    to it)."""
    bench = "bench.py"
    if os.path.isabs(d) and os.path.commonpath([os.path.realpath(d), os.path.realpath(ROOT)]) == \
            os.path.realpath(ROOT):
        d = os.path.relpath(os.path.realpath(d), os.path.realpath(ROOT))
    out = []
    for set_ in ("gemm", "sage", "small_m", "quant"):
        for pass_, ctr in (("mfma", PMC_MFMA), ("fetch", "FETCH_SIZE"), ("write", "WRITE_SIZE")):
            if pass_ == "mfma" and set_ in ("small_m", "quant"):
                continue
            out.append((f"{set_}_{pass_}", f"rocprofv3 --kernel-trace --pmc {ctr} --output-format csv "
                                           f"-d {d}/{set_}_{pass_} -o p -- python3 {bench} --profile-set {set_}"))
    for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
        out.append((f"calib_{ctr}", f"rocprofv3 --kernel-trace --pmc {ctr} --output-format csv -d {d}/calib_{ctr} "
                                    f"-o p -- python3 {bench} --calib-copy"))
        out.append((f"mlp_{ctr}", f"rocprofv3 --kernel-trace --pmc {ctr} --output-format csv -d {d}/mlp_{ctr} "
                                  f"-o p -- python3 {bench} {MLP_ARGS}"))
    out.append(("kt", f"rocprofv3 --kernel-trace --stats --output-format csv -d {d}/kt -o b -- "
                      f"python3 {bench} {KT_ARGS}"))
    return out


def _short_kernel(n):
    n = n.replace("(anonymous namespace)::", "").replace("void ", "")
    return n.split(">(")[0] + ">" if ">(" in n else n.split("(")[0]


def _csv(d, pattern):
    import csv
    import glob
    f = sorted(glob.glob(os.path.join(d, "**", pattern), recursive=True))
    if not f:
        raise FileNotFoundError(f"no {pattern} under {d}")
    return list(csv.DictReader(open(f[0])))


def _dispatches(d):
    """Dispatches of one counter run in dispatch order: name, workgroups,
    duration (kernel trace), counters (summed over the run's instances)."""
    import collections
    per = collections.OrderedDict()
    for r in _csv(d, "*counter_collection.csv"):
        k = int(r["Dispatch_Id"])
        if k not in per:
            per[k] = {"name": _short_kernel(r["Kernel_Name"]), "wgs": int(r["Grid_Size"]) // int(r["Workgroup_Size"]),
                      "us": (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3,
                      "c": collections.defaultdict(float)}
        per[k]["c"][r["Counter_Name"]] += float(r["Counter_Value"])
    try:
        for r in _csv(d, "*kernel_trace.csv"):
            k = int(r["Dispatch_Id"])
            if k in per:
                per[k]["us"] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
    except FileNotFoundError:
        pass
    return [per[k] for k in sorted(per)]


def _pick(ds, name, wgs, skip=0):
    """Dispatches of kernel `name` (its name up to the template arguments'
    end) with `wgs` workgroups, after the first `skip` of them."""
    return [x for x in ds if x["name"] == name and x["wgs"] == wgs][skip:]


def _med(xs, key=None):
    import statistics
    return statistics.median(x["c"][key] if key else x["us"] for x in xs)


def _calibration(d):
    out = {}
    lines = []
    for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
        ds = [x for x in _dispatches(os.path.join(d, f"calib_{ctr}")) if "copyBuffer" in x["name"] or
              "copy" in x["name"].lower()]
        v = _med(ds, ctr)
        out[ctr] = (256 * 1024) / v
        lines.append(f"{ctr} reads {v:.1f} KiB for a 256 MiB device copy -> x{out[ctr]:.4f}")
    cmds = dict(_profile_commands(d))
    hdr = ["HBM counters: FETCH_SIZE / WRITE_SIZE KiB per dispatch (TCC <-> memory), each scaled by its reading for a "
           "plain 256 MiB device copy: " + "; ".join(lines),
           f"calibration commands: {cmds['calib_FETCH_SIZE']}  (and WRITE_SIZE)"]
    return out, hdr


def _traffic_table(rows):
    out = [" launch                          n   med_us   fetch_MB  write_MB  traffic_MB  algo_MB  traffic/algo  "
           "algo_GB/s  frac_HBM  kernel (workgroups)"]
    for label, name, wgs, n, us, fb, wb, algo in rows:
        out.append(f" {label:30s} {n:3d} {us:8.2f} {fb / 1e6:10.1f} {wb / 1e6:9.1f} {(fb + wb) / 1e6:11.1f} "
                   f"{algo / 1e6:8.1f} {(fb + wb) / algo:12.2f} {algo / us / 1e3:10.0f} {algo / us / 1e3 / 8000:9.3f}  "
                   f"{name} ({wgs})")
    return out


def _summarize(d, outdir):
    """profiles/*.txt from the runs of _profile_commands(d)."""
    import statistics
    os.makedirs(outdir, exist_ok=True)
    cmds = dict(_profile_commands(d))
    cal, cal_hdr = _calibration(d)
    written = []

    def traffic_rows(set_, picks):
        fd, wd = _dispatches(os.path.join(d, f"{set_}_fetch")), _dispatches(os.path.join(d, f"{set_}_write"))
        rows = []
        for label, name, wgs, algo, skip in picks:
            f, w = _pick(fd, name, wgs, skip), _pick(wd, name, wgs, skip)
            if not f or not w:
                raise RuntimeError(f"{set_}: no dispatches of {name} ({wgs})")
            rows.append((label, name, wgs, len(f), statistics.median(x["us"] for x in f + w),
                         _med(f, "FETCH_SIZE") * 1024 * cal["FETCH_SIZE"],
                         _med(w, "WRITE_SIZE") * 1024 * cal["WRITE_SIZE"], algo))
        return rows

    def write(fname, lines):
        open(os.path.join(outdir, fname), "w").write("\n".join(lines) + "\n")
        written.append(fname)

    # -- GEMMs (bench.py --profile-set gemm: each shape 4 times)
    G = [("C1 4096x3072x3072 i8 fp32", "qimg::gemm_w8a8_kernel<3, 0, false, false, 192, 256>", 256, 4096, 3072, 3072, 4,
          "I8"),
         ("fc1 rows 0-4095 of 4352 i8", "qimg::gemm_w8a8_kernel<3, 0, true, false, 256, 256>", 768, 4096, 12288, 3072, 4, "I8"),
         ("fc1 rows 4096-4351 i8", "qimg::gemm_w8a8_kernel<3, 0, true, false, 128, 128>", 192, 256, 12288, 3072, 4,
          "I8"),
         ("fc2 4352x3072x12288 i8 bf16", "qimg::gemm_w8a8_kernel<3, 1, false, false, 224, 256>", 238, 4352, 3072, 12288, 2,
          "I8"),
         ("C5 fc1 rows 0-13567 e4m3", "qimg::gemm_w8a8_kernel<1, 0, true, false, 256, 256>", 2544, 13568, 12288, 3072, 4, "F8"),
         ("C5 fc1 rows 13568-13777 e4m3", "qimg::gemm_small_dma_kernel<true, 2, 2, 2, 0, true, 64>", 768, 210, 12288,
          3072, 4, "F8"),
         ("C5 fc2 13778x3072x12288 e4m3", "qimg::gemm_w8a8_kernel<1, 0, false, false, 256, 256>", 648, 13778, 3072, 12288, 4,
          "F8")]
    md = _dispatches(os.path.join(d, "gemm_mfma"))
    lines = ["# MFMA utilisation and HBM traffic of the quantized-linear GEMMs",
             f"command (MFMA pass): {cmds['gemm_mfma']}",
             f"command (HBM passes): {cmds['gemm_fetch']}  (and WRITE_SIZE into gemm_write)",
             "workloads (bench.py _profile_gemm): C1 linear, the MLP pair at 4352 tokens, the batch-2 e4m3 fc1/fc2 of the",
             "1328x1328 step (13778 rows); int8/e4m3 operands, fp32 out (fc2 at 4352: bf16), 4 launches each, medians.",
             "ops = SQ_INSTS_VALU_MFMA_MOPS_{I8,F8} x 512 (checked against 2MNK); frac = ops/s / 5033 TOP/s (2.4 GHz "
             "spec peak); frac@clk = ops/s / (2048 ops/clk/SIMD x 1024 SIMDs x measured clock).", "",
             " launch                          med_us  clock_GHz  MfmaUtil   ops_G   2MNK_G   TOP/s    frac  frac@clk"]
    for label, name, wgs, M_, N_, K_, ob, mode in G:
        r = _pick(md, name, wgs)
        if not r:
            raise RuntimeError(f"gemm_mfma: no dispatches of {name} ({wgs})")
        us = _med(r)
        grbm = _med(r, "GRBM_GUI_ACTIVE") / 8
        util = _med(r, "SQ_VALU_MFMA_BUSY_CYCLES") / (grbm * 1024)
        ops = _med(r, f"SQ_INSTS_VALU_MFMA_MOPS_{mode}") * 512
        clk = grbm / us / 1e3
        tops = 2.0 * M_ * N_ * K_ / us / 1e6
        lines.append(f" {label:30s} {us:8.2f} {clk:10.2f} {util:9.3f} {ops / 1e9:7.1f} {2 * M_ * N_ * K_ / 1e9:8.1f} "
                     f"{tops:7.0f} {tops * 1e12 / 5033e12:7.3f} {tops * 1e12 / (2048 * 1024 * clk * 1e9):9.3f}")
    picks = [(label, name, wgs, M_ * K_ + N_ * K_ + M_ * N_ * ob + 4 * (M_ + N_) + 2 * N_, 0)
             for label, name, wgs, M_, N_, K_, ob, mode in G]
    lines += ["", "HBM traffic per launch (algorithmic bytes = A + W + out + scales + bias, each once)"] + cal_hdr + \
        [""] + _traffic_table(traffic_rows("gemm", picks))
    write("gemm_mfma_hbm_counters.txt", lines)

    # -- SageAttention (bench.py --profile-set sage)
    BH, S_, D_ = 24, 4352, 128
    fl = 4.0 * BH * S_ * S_ * D_
    sd = _dispatches(os.path.join(d, "sage_mfma"))
    att = _pick(sd, "qimg::sage_attn_kernel<128, false, 2>", 408)
    lines = ["# SageAttention at 24 heads x 4352 tokens x 128 (and the K mean of the batch-2 1328x1328 block, 48 x 7401)",
             f"command (MFMA pass): {cmds['sage_mfma']}",
             f"command (HBM passes): {cmds['sage_fetch']}  (and WRITE_SIZE into sage_write)",
             "inputs: Q, K, V as the C3 leg makes them (RMSNorm + RoPE on Q and K, fp16 [24, 4352, 128]);",
             "attention flops = 4 x BH x S^2 x D (half int8 QK^T, half fp16 PV); mixed peak 3355 TFLOP/s", "",
             " launch                      med_us  clock_GHz  MfmaUtil  i8_ops_G  f16_ops_G  TFLOP/s  frac_mixed"]
    us = _med(att)
    grbm = _med(att, "GRBM_GUI_ACTIVE") / 8
    lines.append(f" {'attention 24x4352x128':26s} {us:8.2f} {grbm / us / 1e3:9.2f} "
                 f"{_med(att, 'SQ_VALU_MFMA_BUSY_CYCLES') / (grbm * 1024):9.3f} "
                 f"{_med(att, 'SQ_INSTS_VALU_MFMA_MOPS_I8') * 512 / 1e9:9.1f} "
                 f"{_med(att, 'SQ_INSTS_VALU_MFMA_MOPS_F16') * 512 / 1e9:10.1f} {fl / us / 1e6:8.0f} "
                 f"{fl / us / 1e6 / 3355:11.3f}")
    nq = (S_ + 127) // 128
    picks = [("attention 24x4352x128", "qimg::sage_attn_kernel<128, false, 2>", 408,
              2 * BH * S_ * D_ + 2 * BH * S_ * D_ + 2 * BH * S_ * D_ + 4 * BH * nq * 32 * 2, 0),
             ("K mean 24x4352x128", "qimg::k_mean_kernel", 96, BH * S_ * D_ * 2 + BH * D_ * 4, 0),
             ("K mean 48x7401x128", "qimg::k_mean_kernel", 192, 48 * 7401 * D_ * 2 + 48 * D_ * 4, 0),
             ("Q quant 24x4352x128", "qimg::quant_q_kernel<128>", 816, BH * S_ * D_ * 3 + 4 * BH * nq * 32, 0),
             ("K quant 24x4352x128", "qimg::quant_k128_kernel", 1632, BH * S_ * D_ * 3 + 4 * BH * ((S_ + 63) // 64) * 4,
              0)]
    lines += ["", "HBM traffic per launch (algorithmic: attention = int8 Q, K + fp16 V in + fp16 out + scales; quant = "
              "fp16 in + int8 out + scales; K mean = fp16 K in)"] + cal_hdr + [""] + \
        _traffic_table(traffic_rows("sage", picks))
    write("sage_c3_counters.txt", lines)

    # -- small M (bench.py --profile-set small_m)
    fd = _dispatches(os.path.join(d, "small_m_fetch"))
    shapes = [("mod M=1 18432x3072", 1, 18432, 3072), ("mod M=2 18432x3072", 2, 18432, 3072),
              ("txt qkv M=256 3072x3072", 256, 3072, 3072), ("txt fc1 M=256 12288x3072", 256, 12288, 3072),
              ("txt fc2 M=256 3072x12288", 256, 3072, 12288)]
    # the GEMM kernels of each shape, in order: the first kernel with >= 6
    # consecutive dispatches after the previous shape's
    import itertools
    groups = [(k, len(list(g))) for k, g in itertools.groupby(
        (x for x in fd if "gemv" in x["name"] or "gemm_small" in x["name"] or "gemm_w8a8" in x["name"]),
        key=lambda x: (x["name"], x["wgs"]))]
    keys = [k for k, n in groups if n >= 6]
    if len(keys) != len(shapes):
        raise RuntimeError(f"small_m: expected {len(shapes)} GEMM kernels, found {keys}")
    picks = [(label, k[0], k[1], N_ * K_ + 6 * N_ + M_ * K_ + 4 * M_ + 4 * M_ * N_, 0)
             for (label, M_, N_, K_), k in zip(shapes, keys)]
    lines = ["# HBM traffic of the small-M linears (GEMM only; bench.py _profile_small_m: every call reads the next of",
             "# several weight copies, > 600 MB in all, so the weights come from HBM)",
             f"command: {cmds['small_m_fetch']}  (and WRITE_SIZE into small_m_write)",
             "algorithmic bytes = int8 weights + scales + bias + activations + fp32 output, each once"] + cal_hdr + \
        [""] + _traffic_table(traffic_rows("small_m", picks))
    write("small_m_hbm_traffic.txt", lines)

    # -- activation quant (bench.py --profile-set quant)
    fd = _dispatches(os.path.join(d, "quant_fetch"))
    groups = [(k, len(list(g))) for k, g in itertools.groupby(
        (x for x in fd if x["name"].startswith("qimg::")), key=lambda x: (x["name"], x["wgs"]))]
    keys = [k for k, n in groups if n >= 4]
    Q = [("fc1 input bf16 4352x3072 hbs1024", 4352 * 3072 * 3 + 4 * 4352),
         ("fc2 input fp32 4352x12288 hbs4096", 4352 * 12288 * 5 + 4 * 4352),
         ("C5 fc2 input fp32 13778x12288 e4m3", 13778 * 12288 * 5 + 4 * 13778),
         ("LN+mod+quant 4096x3072", 4096 * 3072 * 5 + 4 * 4096 + 2 * 3072 * 4)]
    if len(keys) != len(Q):
        raise RuntimeError(f"quant: expected {len(Q)} kernels, found {keys}")
    picks = [(label, k[0], k[1], algo, 0) for (label, algo), k in zip(Q, keys)]
    lines = ["# HBM traffic of the activation FWHT + quantization passes (bench.py _profile_quant)",
             f"command: {cmds['quant_fetch']}  (and WRITE_SIZE into quant_write)",
             "algorithmic bytes = input (bf16 2 B or fp32 4 B) + 1-byte output + fp32 scales"] + cal_hdr + [""] + \
        _traffic_table(traffic_rows("quant", picks))
    write("quant_hbm_traffic.txt", lines)

    # -- the bench step's launches (MLP pair at 4352 tokens); read by the
    # bench line's roofline.traffic
    M_, D_, H_, MI = 4352, 3072, 12288, 4096
    step_kernels = {  # launch: (kernel, workgroups, algorithmic bytes)
        "quant_fc1_in": ("qimg::fwht_quant_wave_rows_kernel<qimg::RowsLoader<unsigned short>, (qimg::RowOut)0, 3, "
                         "qimg::RowDest>", M_ // 4, M_ * D_ * 2 + M_ * D_ + 4 * M_),
        "gemm_fc1": ("qimg::gemm_w8a8_kernel<3, 0, true, false, 256, 256>", 768,
                     MI * D_ + H_ * D_ + MI * H_ * 4 + 4 * (MI + H_) + 2 * H_),
        "gemm_fc1_tail": ("qimg::gemm_w8a8_kernel<3, 0, true, false, 128, 128>", 192,
                          256 * D_ + H_ * D_ + 256 * H_ * 4 + 4 * (256 + H_) + 2 * H_),
        "quant_fc2_in": ("qimg::fwht_quant_blocks_kernel<float, (qimg::RowOut)0, 3, false>", M_,
                         M_ * H_ * 4 + M_ * H_ + 4 * M_),
        "gemm_fc2": ("qimg::gemm_w8a8_kernel<3, 1, false, false, 224, 256>", 238,
                     M_ * H_ + D_ * H_ + M_ * D_ * 2 + 4 * (M_ + D_) + 2 * D_),
    }
    fd = _dispatches(os.path.join(d, "mlp_FETCH_SIZE"))
    wd = _dispatches(os.path.join(d, "mlp_WRITE_SIZE"))
    lines = ["# HBM-side traffic per launch of the bench step's kernels (MLP pair at 4352 tokens)",
             f"command (fetch): {cmds['mlp_FETCH_SIZE']}",
             f"command (write): {cmds['mlp_WRITE_SIZE']}"] + cal_hdr + [
             "medians over every dispatch of the launch's kernel and grid in the run; gemm_fc1 = rows 0-4095 on the "
             "256x256 tiles, gemm_fc1_tail = rows 4096-4351 on the 128x128 tiles", "",
             " launch            n  FETCH_KiB  WRITE_KiB  fetch_MB  write_MB  traffic_MB  algorithmic_MB  kernel"]
    tr = {}
    for k, (name, wgs, algo) in step_kernels.items():
        f, w = _pick(fd, name, wgs), _pick(wd, name, wgs)
        if not f or not w:
            raise RuntimeError(f"mlp: no dispatches of {name} ({wgs})")
        fk, wk = _med(f, "FETCH_SIZE"), _med(w, "WRITE_SIZE")
        fb, wb = fk * 1024 * cal["FETCH_SIZE"], wk * 1024 * cal["WRITE_SIZE"]
        tr[k] = fb + wb
        lines.append(f" {k:16s} {len(f):3d} {fk:10.1f} {wk:10.1f} {fb / 1e6:9.1f} {wb / 1e6:9.1f} {(fb + wb) / 1e6:11.1f} "
                     f"{algo / 1e6:15.1f}  {name} ({wgs})")
    lines.append("")
    for k, v in tr.items():
        lines.append(f"traffic_bytes_per_launch {k}: {v:.0f}")
    write("mlp4352_hbm_traffic.txt", lines)

    # -- kernel traces of the bench command (the MLP step and its legs)
    write("mlp4352_kernel_trace.txt", _kt_stats_summary(d, cmds["kt"]))
    trace = sorted(_csv(os.path.join(d, "kt"), "*kernel_trace.csv"), key=lambda r: int(r["Start_Timestamp"]))
    write("block_c4_4096img_256txt_kernel_trace.txt",
          _block_summary(trace, 4096, 256, "# Kernel trace of one MMDiT joint block, 4096 image + 256 text tokens, "
                         "int8 (bench.py C4 leg)", cmds["kt"], "work: 1218.66 GOP per block (linears 985.92, "
                         "attention 232.73)"))
    write("step_c5_fp8_6889img_512txt_kernel_trace.txt",
          _block_summary(trace, 2 * 6889, 2 * 512, "# Kernel trace of one block of the 60-block e4m3 step, 6889 image "
                         "+ 512 text tokens, CFG pair batched (bench.py C5 leg)", cmds["kt"],
                         "work: 2 x 2349.57 GOP per block (the two CFG branches)"))
    return written


def _kt_stats_summary(d, cmd):
    rows = _csv(os.path.join(d, "kt"), "*kernel_stats.csv")
    rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
    lines = ["# Kernel trace: the bench command (MLP pair at 4352 tokens and its extra legs: C1 linear, SageAttention "
             "24x4352x128, small-M linears, C4 block, C5 step, MFMA probe, hipBLASLt reference)",
             f"command: {cmd}", "source: rocprofv3 --kernel-trace --stats (kernel_stats.csv), durations in microseconds",
             "", " calls     avg_us    total_us    pct  kernel"]
    for r in rows[:60]:
        lines.append(f"{int(r['Calls']):6d} {float(r['AverageNs']) / 1e3:10.3f} {float(r['TotalDurationNs']) / 1e3:11.3f}"
                     f" {float(r['Percentage']):6.2f}  {_short_kernel(r['Name'])}")
    return lines


def _block_summary(trace, img_rows, txt_rows, title, cmd, ops_note):
    """Median duration of each kernel of one joint block over every traced
    block whose image-stream LayerNorm covers img_rows rows (blocks run from
    their modulation GEMV to the next one; kernels are matched across blocks
    by name, grid and occurrence, since the two streams' start order varies)."""
    import collections
    import statistics

    def is_mod(r):
        n = r["Kernel_Name"]
        return "gemv_i8_kernel" in n or "gemm_small_dma_kernel<true, 1, 1, 4" in n or \
            "gemm_small_dma_kernel<false, 1, 1, 4" in n
    idx = []
    for i, r in enumerate(trace):
        if is_mod(r) and (i == 0 or not is_mod(trace[i - 1])):
            j = i - 2 if i >= 2 and "silu_kernel" in trace[i - 2]["Kernel_Name"] else i
            idx.append(j)
    blocks = []
    for a, b in zip(idx, idx[1:] + [len(trace)]):
        seq = trace[a:b]
        ln = [r for r in seq if "LnLoader" in r["Kernel_Name"]]
        # (a workgroup per row, a wave per row in fours, or in eights)
        if ln and int(ln[0]["Grid_Size_X"]) in (img_rows * 256, (img_rows + 3) // 4 * 256,
                                                 (img_rows + txt_rows + 3) // 4 * 256,
                                                 (img_rows + 7) // 8 * 512, (img_rows + txt_rows + 7) // 8 * 512):
            blocks.append(seq)
    if not blocks:
        return [title, f"command: {cmd}", "no block found in the trace"]
    n = collections.Counter(len(b) for b in blocks).most_common(1)[0][0]
    blocks = [b for b in blocks if len(b) == n]

    def keyed(block):
        seen = collections.Counter()
        out = collections.OrderedDict()
        for r in block:
            k = (r["Kernel_Name"], int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]))
            out[k + (seen[k],)] = r
            seen[k] += 1
        return out
    kb = [keyed(b) for b in blocks]
    keys = [k for k in kb[0] if all(k in x for x in kb)]
    lines = [title, f"command: {cmd}",
             "source: rocprofv3 --kernel-trace (kernel_trace.csv); median duration of each kernel over "
             f"{len(blocks)} blocks (matched by kernel and grid), microseconds", ops_note, "",
             " pos   median_us  grid_threads x wg  kernel"]
    tot = 0.0
    for j, k in enumerate(keys):
        dur = statistics.median((int(x[k]["End_Timestamp"]) - int(x[k]["Start_Timestamp"])) / 1e3 for x in kb)
        tot += dur
        r = kb[0][k]
        lines.append(f" {j:3d} {dur:11.2f}  {k[1]:12d} x {int(r['Workgroup_Size_X']):3d}  {_short_kernel(r['Kernel_Name'])}")
    span = statistics.median((int(b[-1]["End_Timestamp"]) - int(b[0]["Start_Timestamp"])) / 1e3 for b in blocks)
    lines += ["", f"sum of kernel durations per block: {tot:.1f} us; first start to last end: {span:.1f} us",
              "(the side stream's kernels (the K mean and quantization, the text fc1 and its fc2-input quantization; "
              "in multi-block calls also the next block's modulation GEMV, beside the attention where that has two "
              "or more rounds of workgroups, which then heads the list, else beside the K linears' launch) overlap "
              "the main stream's; the span is the block time)"]
    return lines


if __name__ == "__main__":
    main()
