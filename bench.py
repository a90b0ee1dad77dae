#!/usr/bin/env python3
"""Benchmark of the fused Linear+bias+ReLU hot path on one MI355X.

Workload (the metric's headline layer): fp32 X[8192,4096] . W[4096,4096] +
b[4096] -> ReLU forward, then the fused backward (dX, dW, db) from dY.  One
step = c3hip_linear_fwd + c3hip_linear_bwd, i.e. the three GEMM launches
(forward, dX, dW+db).  Algorithmic work per step: 6*M*N*K flop
(2MNK forward, 4MNK backward); bias, mask and db are timed but not counted.

Inputs are synthetic (X ~ N(0,1), W ~ N(0,1/4096), b ~ N(0,0.01) read as
variance, dY ~ N(0,1)) and already resident in HBM when timing starts.

Printed: one JSON line with the metric, the roofline of the dominant kernel
(HIP events around each of its launches inside the timed loop), the bf16
variant of the same step and the eight elementwise ops at 2^28 fp32 elements
as extra lines of evidence, and the CPU baseline: the oracle's sequential
restatement of the reference loops, timed on one host core on a row/column
slice of the same layer and scaled to the full layer.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "fused GEMM+bias+ReLU fwd+bwd TFLOP/s & % MFMA peak; elementwise GB/s"
PEAK_FP32_TFLOPS = 157.3
PEAK_BF16_TFLOPS = 2516.6
PEAK_HBM_GBS = 8000.0
M, K, N = 8192, 4096, 4096


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true", help="skip the bf16 and elementwise evidence lines")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain copy-like stream (scale: read 2^26 fp32, write 2^26 fp32) three times; "
                         "its FETCH_SIZE/WRITE_SIZE counters calibrate the HBM traffic figures")
    return ap.parse_args()


def copy_calibration():
    import torch

    from c3_amd import native as C

    C.init(0)
    n = 1 << 26
    a = torch.randn(n, device="cuda:0")
    o = torch.empty(n, device="cuda:0")
    s = torch.cuda.current_stream().cuda_stream
    for _ in range(3):
        C.elementwise(C.EW_SCALE, C.F32, a.data_ptr(), None, 0.5, o.data_ptr(), n, 0, s)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration": {"kernel": "c3_ew_scale_f32_v", "read_bytes": 4 * n,
                                           "write_bytes": 4 * n, "launches": 3}}), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration()
        return

    import torch

    from c3_amd import native as C

    C.init(0)
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    s = stream.cuda_stream
    g = torch.Generator(device=dev)
    g.manual_seed(0xC3)
    X = torch.randn(M, K, device=dev, generator=g)
    W = torch.randn(K, N, device=dev, generator=g) / 64.0
    b = torch.randn(N, device=dev, generator=g) * 0.1
    dY = torch.randn(M, N, device=dev, generator=g)
    Y = torch.empty(M, N, device=dev)
    dX = torch.empty(M, K, device=dev)
    dW = torch.empty(K, N, device=dev)
    db = torch.empty(N, device=dev)

    def fwd():
        C.linear_fwd(C.F32, X.data_ptr(), W.data_ptr(), b.data_ptr(), Y.data_ptr(), M, K, N, C.ACT_RELU, s)

    def bwd_dx():
        C.linear_bwd(C.F32, X.data_ptr(), W.data_ptr(), Y.data_ptr(), dY.data_ptr(), dX.data_ptr(), None, None,
                     M, K, N, C.ACT_RELU, s)

    def bwd_dw():
        C.linear_bwd(C.F32, X.data_ptr(), W.data_ptr(), Y.data_ptr(), dY.data_ptr(), None, dW.data_ptr(),
                     db.data_ptr(), M, K, N, C.ACT_RELU, s)

    # A step is the forward and the full backward; the backward is issued as
    # its two kernels so events can bracket each (same launches as one
    # c3hip_linear_bwd call with dX, dW and db).
    kernels = [("gemm_fwd_bias_relu", fwd), ("gemm_dx_mask", bwd_dx), ("gemm_dw_mask_db", bwd_dw)]
    for _ in range(args.warmup):
        for _, fn in kernels:
            fn()
    torch.cuda.synchronize()

    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(len(kernels) + 1)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        ev[i][0].record(stream)
        for j, (_, fn) in enumerate(kernels):
            fn()
            ev[i][j + 1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per_kernel_ms = {name: sum(ev[i][j].elapsed_time(ev[i][j + 1]) for i in range(args.steps)) / args.steps
                     for j, (name, _) in enumerate(kernels)}
    step_ms = sum(ev[i][0].elapsed_time(ev[i][-1]) for i in range(args.steps)) / args.steps
    flop_step = 6.0 * M * N * K
    value = flop_step / (step_ms * 1e-3) / 1e12
    wall_tflops = flop_step * args.steps / wall / 1e12

    dom = max(per_kernel_ms, key=per_kernel_ms.get)
    dom_ms = per_kernel_ms[dom]
    dom_achieved = 2.0 * M * N * K / (dom_ms * 1e-3) / 1e12
    roofline = {"bound": "mfma", "kernel": dom, "achieved": round(dom_achieved, 2), "peak": PEAK_FP32_TFLOPS,
                "unit": "TFLOP/s", "frac": round(dom_achieved / PEAK_FP32_TFLOPS, 4),
                "avg_launch_ms": round(dom_ms, 4), "traffic": _traffic(dom)}

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (X~N(0,1), W~N(0,1/4096), b~N(0,0.01), dY~N(0,1); resident in HBM)",
        "config": {"workload": "fused Linear+bias+ReLU fwd+bwd (dX, dW, db), fp32", "M": M, "K": K, "N": N,
                   "flop_per_step": flop_step, "parallelism": "single GPU"},
        "frac_of_fp32_peak": round(value / PEAK_FP32_TFLOPS, 4),
        "wall_clock_tflops": round(wall_tflops, 2),
        "per_kernel_ms": {k: round(v, 4) for k, v in per_kernel_ms.items()},
        "roofline": roofline,
    }
    if not args.no_extras:
        out["bf16"] = bench_bf16(torch, C, dev, s, args)
        out["elementwise"] = bench_elementwise(torch, C, dev, s)
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)


def _traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE, scaled by the copy-stream calibration), or None."""
    p = ROOT / "profiles" / "traffic_fp32_linear_8192x4096x4096.md"
    try:
        for line in p.read_text().splitlines():
            if line.startswith("traffic-json:"):
                return json.loads(line.split(":", 1)[1]).get(kernel, {}).get("bytes_per_launch")
    except (ValueError, OSError):
        pass
    return None


def bench_bf16(torch, C, dev, s, args):
    """Same step with bf16 X, W, dY, Y, dX (fp32 accumulation; dW, db fp32)."""
    g = torch.Generator(device=dev)
    g.manual_seed(0xB16)
    X = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
    W = (torch.randn(K, N, device=dev, generator=g) / 64.0).to(torch.bfloat16)
    b = torch.randn(N, device=dev, generator=g) * 0.1
    dY = torch.randn(M, N, device=dev, generator=g).to(torch.bfloat16)
    Y = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
    dX = torch.empty(M, K, device=dev, dtype=torch.bfloat16)
    dW = torch.empty(K, N, device=dev)
    db = torch.empty(N, device=dev)

    def step():
        C.linear_fwd(C.BF16, X.data_ptr(), W.data_ptr(), b.data_ptr(), Y.data_ptr(), M, K, N, C.ACT_RELU, s)
        C.linear_bwd(C.BF16, X.data_ptr(), W.data_ptr(), Y.data_ptr(), dY.data_ptr(), dX.data_ptr(), dW.data_ptr(),
                     db.data_ptr(), M, K, N, C.ACT_RELU, s)

    for _ in range(args.warmup):
        step()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    tf = 6.0 * M * N * K / (ms * 1e-3) / 1e12
    return {"workload": "same layer, bf16 storage, fp32 accumulate", "ms_per_step": round(ms, 4),
            "tflops": round(tf, 2), "frac_of_bf16_peak": round(tf / PEAK_BF16_TFLOPS, 4)}


def bench_elementwise(torch, C, dev, s, n=1 << 28, iters=10):
    """The eight elementwise ops over 2^28 fp32 elements (1 GiB per operand, far
    above the 256 MB Infinity Cache), algorithmic bytes: 12 B/elem binary,
    8 B/elem unary."""
    a = torch.randn(n, device=dev)
    bb = torch.rand(n, device=dev) * 1.5 + 0.5
    o = torch.empty(n, device=dev)
    res = {}
    for name, code in C.EW_OPS.items():
        nbytes = (12 if code in (C.EW_ADD, C.EW_SUB, C.EW_MUL, C.EW_DIV, C.EW_RELU_BWD) else 8) * n
        fn = lambda: C.elementwise(code, C.F32, a.data_ptr(), bb.data_ptr(), 0.5, o.data_ptr(), n, 0, s)  # noqa
        fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(iters):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / iters
        gbs = nbytes / (ms * 1e-3) / 1e9
        res[name] = {"GB/s": round(gbs, 1), "frac_of_hbm_peak": round(gbs / PEAK_HBM_GBS, 4)}
    return {"n": n, "ops": res}


def cpu_baseline():
    """The oracle (C restatement of the reference's JIT'd loops: 64x64 i/j
    tiles, sequential k, no FMA) on one host core, over a slice of the same
    layer: 32 rows of Y (forward), 32 rows of dX and 32 rows of dW (about
    15 s on one core).  Each output row of a GEMM costs the same, so the
    slice rate is the full layer's rate: TFLOP/s = slice flop / slice seconds."""
    import numpy as np

    from oracle import oracle as O

    rows = 32
    X = O.normal(1, (rows, K))
    W = O.normal(2, (K, N), 0.0, 1.0 / 64.0)
    b = O.normal(3, N, 0.0, 0.1)
    dY = O.normal(4, (rows, N))
    Xm = O.normal(5, (M, rows))      # X[:, k-slice] for the dW rows
    dZm = O.normal(6, (M, N))        # dZ for the dW slice
    t0 = time.perf_counter()
    Y = O.linear_fwd(X, W, b, 1)
    t1 = time.perf_counter()
    dZ = O.relu_mask_mul(Y, dY)
    O.matmul(dZ, W, transB=True)
    t2 = time.perf_counter()
    O.matmul(Xm, dZm, transA=True)
    t3 = time.perf_counter()
    flop = 2.0 * rows * N * K * 2 + 2.0 * rows * M * N
    secs = t3 - t0
    del np
    return {"value": round(flop / secs / 1e12, 6), "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": f"oracle on {rows} rows of Y ({t1 - t0:.1f}s), {rows} rows of dX ({t2 - t1:.1f}s) and "
                      f"{rows} rows of dW ({t3 - t2:.1f}s) of the {M}x{K}x{N} layer, one core; "
                      f"full fwd+bwd step extrapolates to {6.0 * M * N * K / (flop / secs) / 3600:.1f} h",
            "host_cpu": _cpu_model()}


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip() + f" ({os.cpu_count()} logical cpus visible)"
    except OSError:
        pass
    return None


if __name__ == "__main__":
    main()
