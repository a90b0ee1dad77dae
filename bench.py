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
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the evidence beside the headline (bf16 layer and sweep, elementwise, MLP steps)")
    ap.add_argument("--elementwise-profile", action="store_true",
                    help="only run each of the eight elementwise ops over 2^LOG2N fp32 elements (random data), "
                         "rotating over SETS operand sets, for rocprofv3 kernel-trace and FETCH_SIZE/WRITE_SIZE "
                         "summaries of the streams")
    ap.add_argument("--log2n", type=int, default=28, help="--elementwise-profile: elements per operand (2^LOG2N)")
    ap.add_argument("--sets", type=int, default=1, help="--elementwise-profile: operand sets rotated over")
    ap.add_argument("--gemm-compare", action="store_true",
                    help="only run the bf16 forward GEMM (c3hip_linear_fwd, bias + ReLU) and torch.matmul "
                         "(hipBLASLt) alternately at 8192x4096x4096 and 16384x8192x8192 on random data, for "
                         "rocprofv3 kernel-trace and MFMA-busy/clock counter summaries of both")
    ap.add_argument("--bf16-gemm-kinds", action="store_true",
                    help="only run the three bf16 GEMMs of a Linear layer (forward with bias + ReLU, dX, dW) at "
                         "16384x8192x8192 on the size heuristic's kernels, 10 launches each, for rocprofv3 "
                         "counter summaries of the bf16 GEMM kernels")
    ap.add_argument("--bf16-sweep-only", action="store_true",
                    help="only run the bf16 M x K x N sweep (one JSON line), for a rocprofv3 kernel trace "
                         "summarised per shape")
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


def elementwise_profile(log2n=28, sets=1, reps=3):
    """Each elementwise op `reps` times per operand set, rotating over `sets`
    sets (sets > 1 keeps each launch's operands out of the Infinity Cache)."""
    import torch

    from c3_amd import native as C

    C.init(0)
    n = 1 << log2n
    g = torch.Generator(device="cuda:0")
    g.manual_seed(0xE7)
    bufs = [(torch.randn(n, device="cuda:0", generator=g), torch.rand(n, device="cuda:0", generator=g) * 1.5 + 0.5,
             torch.empty(n, device="cuda:0")) for _ in range(sets)]
    s = torch.cuda.current_stream().cuda_stream
    for name, code in C.EW_OPS.items():
        for _ in range(reps):
            for a, b, o in bufs:
                C.elementwise(code, C.F32, a.data_ptr(), b.data_ptr(), 0.5, o.data_ptr(), n, 0, s)
    torch.cuda.synchronize()
    print(json.dumps({"elementwise_profile": {"n": n, "operand_sets": sets, "launches_per_op": reps * sets,
                                              "ops": list(C.EW_OPS)}}), flush=True)


def bf16_gemm_kinds(m=16384, k=8192, n=8192, reps=10):
    """The forward (bias + ReLU), dX and dW GEMMs of a bf16 Linear layer,
    each `reps` times, through c3hip_linear_fwd / c3hip_linear_bwd (dX alone,
    dW alone, no activation: each call is exactly one GEMM launch)."""
    import torch

    from c3_amd import native as C

    C.init(0)
    dev = torch.device("cuda:0")
    s = torch.cuda.current_stream().cuda_stream
    g = torch.Generator(device=dev)
    g.manual_seed(0xB1A6)
    X = torch.randn(m, k, device=dev, generator=g).to(torch.bfloat16)
    W = (torch.randn(k, n, device=dev, generator=g) / float(k) ** 0.5).to(torch.bfloat16)
    b = torch.randn(n, device=dev, generator=g) * 0.1
    dZ = torch.randn(m, n, device=dev, generator=g).to(torch.bfloat16)
    Y = torch.empty(m, n, device=dev, dtype=torch.bfloat16)
    dX = torch.empty(m, k, device=dev, dtype=torch.bfloat16)
    dW = torch.empty(k, n, device=dev)
    for _ in range(reps):
        C.linear_fwd(C.BF16, X.data_ptr(), W.data_ptr(), b.data_ptr(), Y.data_ptr(), m, k, n, C.ACT_RELU, s)
    for _ in range(reps):
        C.linear_bwd(C.BF16, None, W.data_ptr(), None, dZ.data_ptr(), dX.data_ptr(), None, None, m, k, n,
                     C.ACT_NONE, s)
    for _ in range(reps):
        C.linear_bwd(C.BF16, X.data_ptr(), None, None, dZ.data_ptr(), None, dW.data_ptr(), None, m, k, n,
                     C.ACT_NONE, s)
    torch.cuda.synchronize()
    print(json.dumps({"bf16_gemm_kinds": {"shape": f"{m}x{k}x{n}", "launches_per_kind": reps}}), flush=True)


def gemm_compare(reps=10, rounds=3):
    """bf16 forward GEMM of this backend (c3hip_linear_fwd with bias and ReLU)
    against torch.matmul (hipBLASLt's kernel; no bias) on the same random
    operands, alternating in rounds so both see the same clock and power
    state.  Prints the event-timed TFLOP/s of each; the kernel durations,
    MFMA busy and clock come from rocprofv3 over this same command."""
    import torch

    from c3_amd import native as C

    C.init(0)
    dev = torch.device("cuda:0")
    s = torch.cuda.current_stream().cuda_stream
    g = torch.Generator(device=dev)
    g.manual_seed(0xB1A5)
    out = {}
    for (m, k, n) in [(8192, 4096, 4096), (16384, 8192, 8192)]:
        X = torch.randn(m, k, device=dev, generator=g).to(torch.bfloat16)
        W = (torch.randn(k, n, device=dev, generator=g) / float(k) ** 0.5).to(torch.bfloat16)
        b = torch.randn(n, device=dev, generator=g) * 0.1
        Y = torch.empty(m, n, device=dev, dtype=torch.bfloat16)
        Yt = torch.empty(m, n, device=dev, dtype=torch.bfloat16)

        def ours():
            C.linear_fwd(C.BF16, X.data_ptr(), W.data_ptr(), b.data_ptr(), Y.data_ptr(), m, k, n, C.ACT_RELU, s)

        def theirs():
            torch.matmul(X, W, out=Yt)

        times = {"c3hip_linear_fwd": [], "torch.matmul (hipBLASLt)": []}
        for _ in range(rounds):
            for name, fn in (("c3hip_linear_fwd", ours), ("torch.matmul (hipBLASLt)", theirs)):
                fn()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                torch.cuda.synchronize()
                e0.record()
                for _ in range(reps):
                    fn()
                e1.record()
                torch.cuda.synchronize()
                times[name].append(e0.elapsed_time(e1) / reps)
        out[f"{m}x{k}x{n}"] = {name: round(2.0 * m * n * k / (sorted(v)[len(v) // 2] * 1e-3) / 1e12, 1)
                               for name, v in times.items()}
        del X, W, b, Y, Yt
        torch.cuda.empty_cache()
    print(json.dumps({"gemm_compare_tflops": out, "launches_per_kernel_and_shape": rounds * (reps + 1)}), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration()
        return
    if args.elementwise_profile:
        elementwise_profile(args.log2n, args.sets)
        return
    if args.gemm_compare:
        gemm_compare()
        return
    if args.bf16_gemm_kinds:
        bf16_gemm_kinds()
        return

    import torch

    from c3_amd import native as C

    C.init(0)
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    if args.bf16_sweep_only:
        print(json.dumps({"bf16_sweep": bench_bf16_sweep(torch, C, dev, stream.cuda_stream)}), flush=True)
        return
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

    def bwd():
        C.linear_bwd(C.F32, X.data_ptr(), W.data_ptr(), Y.data_ptr(), dY.data_ptr(), dX.data_ptr(), dW.data_ptr(),
                     db.data_ptr(), M, K, N, C.ACT_RELU, s)

    # A step is c3hip_linear_fwd + c3hip_linear_bwd (dX, dW, db): the forward
    # GEMM, then the backward's dZ = mask(Y) dY pass (with the db partials and
    # their final sum) and the dX and dW GEMMs on dZ.  Each launch is timed on
    # its stream by the library's launch timing.
    def step():
        fwd()
        bwd()

    for _ in range(args.warmup):
        step()
    step_ms, wall, kt = _timed_steps(torch, C, stream, step, args.steps)
    flop_step = 6.0 * M * N * K
    value = flop_step / (step_ms * 1e-3) / 1e12
    wall_tflops = flop_step * args.steps / wall / 1e12
    per_kernel_ms = {k: v["avg_ms"] for k, v in kt.items()}

    # Each of the three GEMMs does 2 M N K flop per launch; the slowest is the dominant kernel.
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
        out["bf16_sweep"] = bench_bf16_sweep(torch, C, dev, s)
        out["elementwise"] = {"2^28": bench_elementwise(torch, C, dev, s, 1 << 28, sets=1),
                              "2^24": bench_elementwise(torch, C, dev, s, 1 << 24, sets=8)}
        out["backward_chain"] = bench_backward_chain(torch, C, dev, s)
        out["mlp_784_256_128_10_fp32"] = bench_mlp(torch, C, dev, s, [784, 256, 128, 10], 128, C.F32,
                                                   steps=200, uniform_x=True, graph=True)
        out["mlp_deep_bf16"] = bench_mlp(torch, C, dev, s, [4096, 8192, 8192, 8192, 4096, 1000], 16384, C.BF16,
                                         steps=10, uniform_x=False, timed_kernels=True)
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)


def _timed_steps(torch, C, stream, step, steps):
    """Time `steps` back-to-back steps with HIP events on `stream` (the step
    time, and the host wall time), then the same number again with the
    library's launch timing on, for each kernel's duration (events around
    every launch add a little time between kernels, so that second loop does
    not give the step time).  Returns (ms per step, wall s, kernel table)."""
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    step_ms = e0.elapsed_time(e1) / steps
    C.set_launch_timing(True)
    try:
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        kt = _kernel_table(C.launch_timings(), steps)
    finally:
        C.set_launch_timing(False)
    return step_ms, wall, kt


def _kernel_table(records, steps):
    """Per kernel name: launches per step, mean and total duration per step (ms),
    from the library's launch timing records [(name, ms), ...] of `steps` steps."""
    agg = {}
    for name, ms in records:
        agg.setdefault(name, []).append(ms)
    return {n: {"launches_per_step": round(len(v) / steps, 3), "avg_ms": round(sum(v) / len(v), 4),
                "ms_per_step": round(sum(v) / steps, 4)} for n, v in agg.items()}


def _traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE, scaled by the copy-stream calibration), or None."""
    p = ROOT / "profiles" / "traffic_fp32_linear_8192x4096x4096.md"
    try:
        for line in p.read_text().splitlines():
            if line.startswith("traffic-json:"):
                for entry in json.loads(line.split(":", 1)[1]).values():
                    if entry.get("kernel") == kernel:
                        return entry.get("bytes_per_launch")
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
    ms, _, kt = _timed_steps(torch, C, torch.cuda.current_stream(), step, args.steps)
    tf = 6.0 * M * N * K / (ms * 1e-3) / 1e12
    # The forward GEMM does 2 M N K flop per launch, the backward's dX and dW
    # 4 M N K together, in one launch (c3_gemm_bf16_bwd_*) or two; the
    # backward pre-pass (dZ and the db partials) is an HBM stream.
    gemms = {k: v for k, v in kt.items() if k.startswith("c3_gemm_")}
    dom = max(gemms, key=lambda k: gemms[k]["avg_ms"])
    dom_flop = (4.0 if dom.startswith("c3_gemm_bf16_bwd_") else 2.0) * M * N * K
    ach = dom_flop / (gemms[dom]["avg_ms"] * 1e-3) / 1e12
    return {"workload": "same layer, bf16 storage, fp32 accumulate", "ms_per_step": round(ms, 4),
            "tflops": round(tf, 2), "frac_of_bf16_peak": round(tf / PEAK_BF16_TFLOPS, 4), "kernels": kt,
            "roofline": {"bound": "mfma", "kernel": dom, "achieved": round(ach, 2), "peak": PEAK_BF16_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(ach / PEAK_BF16_TFLOPS, 4),
                         "avg_launch_ms": gemms[dom]["avg_ms"], "traffic": None}}


def bench_elementwise(torch, C, dev, s, n, sets, iters=10):
    """The eight elementwise ops over n fp32 elements.  Algorithmic bytes:
    12 B/elem binary, 8 B/elem unary.  With sets > 1 the launches rotate over
    that many operand sets so that each launch reads memory the previous ones
    did not touch (2^24 elements: 8 sets of 192 MiB, above the 256 MB
    Infinity Cache)."""
    bufs = [(torch.randn(n, device=dev), torch.rand(n, device=dev) * 1.5 + 0.5, torch.empty(n, device=dev))
            for _ in range(sets)]
    # Device pointers taken once: a 2^24 launch runs ~30 us on the GPU, about
    # what three data_ptr() calls and the list indexing cost on the host.
    ptrs = [(a.data_ptr(), bb.data_ptr(), o.data_ptr()) for a, bb, o in bufs]
    ew = C.elementwise
    res = {}
    for name, code in C.EW_OPS.items():
        nbytes = (12 if code in (C.EW_ADD, C.EW_SUB, C.EW_MUL, C.EW_DIV, C.EW_RELU_BWD) else 8) * n

        def fn(i):
            pa, pb, po = ptrs[i % sets]
            ew(code, C.F32, pa, pb, 0.5, po, n, 0, s)

        for i in range(sets):
            fn(i)
        total = iters * sets
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for i in range(total):
            fn(i)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / total
        gbs = nbytes / (ms * 1e-3) / 1e9
        res[name] = {"GB/s": round(gbs, 1), "frac_of_hbm_peak": round(gbs / PEAK_HBM_GBS, 4)}
    del bufs
    torch.cuda.empty_cache()
    return {"n": n, "operand_sets": sets, "ops": res}


def bench_backward_chain(torch, C, dev, s, n=1 << 26, iters=10):
    """Fused backward chains over n fp32 elements against the same nodes run one
    by one.  Algorithmic bytes of a w-node chain: 4 * (1 + 2w) per element
    (grad and w forward inputs read, w upstream grads written); one by one the
    nodes move 4 * 3w (Neg: 8 B per element)."""
    chains = {"ReLU+Sigmoid": [C.CHAIN_RELU, C.CHAIN_SIGMOID], "Sigmoid+Tanh": [C.CHAIN_SIGMOID, C.CHAIN_TANH],
              "ReLU+Log+Neg+Exp": [C.CHAIN_RELU, C.CHAIN_LOG, C.CHAIN_NEG, C.CHAIN_EXP]}
    single = {C.CHAIN_RELU: (C.EW_RELU_BWD, True), C.CHAIN_SIGMOID: (C.EW_SIGMOID_BWD, True),
              C.CHAIN_TANH: (C.EW_TANH_BWD, True), C.CHAIN_EXP: (C.EW_EXP_BWD, True),
              C.CHAIN_LOG: (C.EW_DIV, False), C.CHAIN_NEG: (C.EW_NEG, False)}
    g = torch.randn(n, device=dev)
    xs = [torch.rand(n, device=dev) * 4.0 + 0.25 for _ in range(4)]
    outs = [torch.empty(n, device=dev) for _ in range(4)]

    def timed(fn):
        fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(iters):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / iters

    res = {}
    for name, nodes in chains.items():
        w = len(nodes)

        def fused():
            C.backward_chain(C.F32, g.data_ptr(), [x.data_ptr() for x in xs[:w]], nodes,
                             [o.data_ptr() for o in outs[:w]], n, s)

        def one_by_one():
            cur = g
            for k, node in enumerate(nodes):
                op, x_first = single[node]
                if node == C.CHAIN_NEG:
                    C.elementwise(op, C.F32, cur.data_ptr(), None, 0.0, outs[k].data_ptr(), n, 0, s)
                elif x_first:
                    C.elementwise(op, C.F32, xs[k].data_ptr(), cur.data_ptr(), 0.0, outs[k].data_ptr(), n, 0, s)
                else:
                    C.elementwise(op, C.F32, cur.data_ptr(), xs[k].data_ptr(), 0.0, outs[k].data_ptr(), n, 0, s)
                cur = outs[k]

        ms_f, ms_u = timed(fused), timed(one_by_one)
        gbs = 4.0 * (1 + 2 * w) * n / (ms_f * 1e-3) / 1e9
        res[name] = {"fused_ms": round(ms_f, 4), "one_by_one_ms": round(ms_u, 4), "speedup": round(ms_u / ms_f, 3),
                     "fused_GB/s": round(gbs, 1), "frac_of_hbm_peak": round(gbs / PEAK_HBM_GBS, 4)}
    del g, xs, outs
    torch.cuda.empty_cache()
    return {"n": n, "chains": res}


SWEEP = [(m, k, n) for m in (1024, 4096, 16384) for k in (1024, 4096, 8192) for n in (1024, 4096, 8192)]


def bench_bf16_sweep(torch, C, dev, s, reps=5, groups=3, warmup=3):
    """bf16 Linear+bias+ReLU forward + fused backward over the M x K x N sweep
    {1024, 4096, 16384} x {1024, 4096, 8192} x {1024, 4096, 8192}: TFLOP/s of
    the step (6 M N K flop) per shape, after `warmup` steps: the median over
    `groups` groups of events around `reps` back-to-back steps."""
    g = torch.Generator(device=dev)
    g.manual_seed(0x5EE9)
    res = {}
    for (m, k, n) in SWEEP:
        X = torch.randn(m, k, device=dev, generator=g).to(torch.bfloat16)
        W = (torch.randn(k, n, device=dev, generator=g) / float(k) ** 0.5).to(torch.bfloat16)
        b = torch.randn(n, device=dev, generator=g) * 0.1
        dY = torch.randn(m, n, device=dev, generator=g).to(torch.bfloat16)
        Y = torch.empty(m, n, device=dev, dtype=torch.bfloat16)
        dX = torch.empty(m, k, device=dev, dtype=torch.bfloat16)
        dW = torch.empty(k, n, device=dev)
        db = torch.empty(n, device=dev)

        def step():
            C.linear_fwd(C.BF16, X.data_ptr(), W.data_ptr(), b.data_ptr(), Y.data_ptr(), m, k, n, C.ACT_RELU, s)
            C.linear_bwd(C.BF16, X.data_ptr(), W.data_ptr(), Y.data_ptr(), dY.data_ptr(), dX.data_ptr(),
                         dW.data_ptr(), db.data_ptr(), m, k, n, C.ACT_RELU, s)

        for _ in range(warmup):
            step()
        times = []
        for _ in range(groups):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record()
            for _ in range(reps):
                step()
            e1.record()
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1) / reps)
        ms = sorted(times)[len(times) // 2]
        res[f"{m}x{k}x{n}"] = round(6.0 * m * n * k / (ms * 1e-3) / 1e12, 1)
        del X, W, b, dY, Y, dX, dW, db
    torch.cuda.empty_cache()
    vals = sorted(res.values())
    return {"workload": "bf16 Linear+bias+ReLU fwd+bwd step per shape, TFLOP/s", "tflops": res,
            "median_tflops": vals[len(vals) // 2], "min_tflops": vals[0], "max_tflops": vals[-1]}


def bench_mlp(torch, C, dev, s, dims, batch, dtype, steps, uniform_x, graph=False, timed_kernels=False):
    """Train step of an MLP (ReLU between layers, softmax-CE, SGD) through the
    dispatch flow (c3_amd/trainer.py: region kernels from RegionFusionRegistry,
    fused backwards from C3BackwardCapture, JIT cache warm), after warm-up
    until every layer runs on an installed kernel.  Flop per step: 6 * batch
    * sum(K*N) (forward 2x, backward 4x including the first layer's dX)."""
    from c3_amd import trainer as T

    g = torch.Generator(device=dev)
    g.manual_seed(0xC3)
    tr = T.MlpTrainer(dims, batch, dtype)
    keep = []
    for l in range(len(dims) - 1):
        bound = (6.0 / dims[l]) ** 0.5
        w = (torch.rand(dims[l], dims[l + 1], device=dev, generator=g) * 2 - 1) * bound
        wp, bp = tr.params(l)
        C.cast(C.F32, dtype, w.data_ptr(), wp, w.numel(), s)  # biases stay zero
        keep.append(w)
    x = torch.rand(batch, dims[0], device=dev, generator=g) if uniform_x else \
        torch.randn(batch, dims[0], device=dev, generator=g)
    xd = x if dtype == C.F32 else x.to(torch.bfloat16)
    lbl = torch.randint(0, dims[-1], (batch,), device=dev, generator=g, dtype=torch.int32)
    torch.cuda.synchronize()
    lr = 1e-3
    warm = tr.warm_up(xd.data_ptr(), lbl.data_ptr(), lr, 16, s)
    st0 = tr.stats()
    loss0 = tr.step(xd.data_ptr(), lbl.data_ptr(), lr, True, s)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        tr.step(xd.data_ptr(), lbl.data_ptr(), lr, False, s)
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / steps
    kt = None
    if timed_kernels:
        # The same steps again with every launch timed (kernel durations only).
        C.set_launch_timing(True)
        try:
            for _ in range(steps):
                tr.step(xd.data_ptr(), lbl.data_ptr(), lr, False, s)
            torch.cuda.synchronize()
            kt = _kernel_table(C.launch_timings(), steps)
        finally:
            C.set_launch_timing(False)
    loss1 = tr.step(xd.data_ptr(), lbl.data_ptr(), lr, True, s)
    st1 = tr.stats()
    graph_ms = None
    if graph:
        # The same step captured as one HIP graph (on a side stream: the
        # default stream cannot be captured) and replayed.
        side = torch.cuda.Stream()
        with torch.cuda.stream(side):
            tr.capture(xd.data_ptr(), lbl.data_ptr(), lr, side.cuda_stream)
            for _ in range(3):
                tr.replay(side.cuda_stream)
            g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            side.synchronize()
            g0.record(side)
            for _ in range(steps):
                tr.replay(side.cuda_stream)
            g1.record(side)
            side.synchronize()
        graph_ms = g0.elapsed_time(g1) / steps
    tr.close()
    del keep, x, xd, lbl
    torch.cuda.empty_cache()
    # Forward 2·B·in·out per layer; backward dW 2·B·in·out per layer and dX
    # 2·B·in·out for every layer but the first (the data batch needs no gradient).
    macs = [batch * dims[l] * dims[l + 1] for l in range(len(dims) - 1)]
    flop = 6.0 * sum(macs) - 2.0 * macs[0]
    tf = flop / (ms * 1e-3) / 1e12
    peak = PEAK_FP32_TFLOPS if dtype == C.F32 else PEAK_BF16_TFLOPS
    extra = {}
    if kt is not None:
        # The step's GEMM flop (every layer's forward and dW, every layer's dX
        # but the first) over the summed durations of its GEMM launches.
        gemm_ms = sum(v["ms_per_step"] for k, v in kt.items() if k.startswith("c3_gemm_"))
        ach = flop / (gemm_ms * 1e-3) / 1e12
        extra = {"kernels": kt, "roofline": {
            "bound": "mfma", "kernel": "all GEMM launches of the step", "achieved": round(ach, 2), "peak": peak,
            "unit": "TFLOP/s", "frac": round(ach / peak, 4), "gemm_ms_per_step": round(gemm_ms, 4),
            "traffic": None}}
    return {**extra, "dims": dims, "batch": batch, "dtype": "fp32" if dtype == C.F32 else "bf16",
            "ms_per_step": round(ms, 4), "us_per_step_wall": round(wall / steps * 1e6, 1),
            "tflops": round(tf, 3), "frac_of_peak": round(tf / peak, 4), "flop_per_step": flop,
            "input_grad": "not computed for the first layer (its input is the data batch)",
            "warm_up_steps": warm, "region_hits_timed": st1["region_hits"] - st0["region_hits"],
            "backward_hits_timed": st1["backward_hits"] - st0["backward_hits"],
            "eager_ops_timed": st1["eager_ops"] - st0["eager_ops"],
            "fully_dispatched": bool(st1["fully_dispatched"]),
            "loss_before": round(loss0, 5), "loss_after": round(loss1, 5),
            **({"graph_replay_us_per_step": round(graph_ms * 1e3, 2),
                "graph_replay_tflops": round(flop / (graph_ms * 1e-3) / 1e12, 3)} if graph_ms else {})}


def cpu_baseline():
    """The oracle (C restatement of the reference's JIT'd loops: 64x64 i/j
    tiles, sequential k, no FMA), run on the host, for every workload in
    the bench: the headline layer and both sweeps on row slices (each output
    row of a GEMM costs the same, so a slice's rate is the whole layer's;
    the extrapolated full-step time is stated), the small MLP's full train
    step, and the eight elementwise ops.  One core, as the reference runs
    its GEMM kernels (serially, src/C3/C3Engine.cpp:168); relu-bwd, a
    two-node graph the reference runs on up to 8 threads for n >= 262144
    (src/C3/C3Engine.cpp:165-206), also on min(cores, 8) threads."""
    import numpy as np

    from oracle import oracle as O

    t_all = time.perf_counter()
    head = _cpu_layer_slices(O, np, M, K, N, rows=16)
    out = {"value": round(head["tflops"], 6), "unit": "TFLOP/s", "cores": 1, "kind": "port",
           "sample": f"oracle on {head['rows']} rows of Y, of dX and of dW of the {M}x{K}x{N} fp32 layer, one "
                     f"core ({head['sample_s']:.1f} s); the full fwd+bwd step extrapolates to "
                     f"{head['full_step_s'] / 3600:.2f} h",
           "host_cpu": _cpu_model(),
           "mlp_784_256_128_10_fp32": _cpu_mlp(O, np),
           "elementwise": _cpu_elementwise(O, np),
           "bf16_sweep": _cpu_sweep(O, np),
           "mlp_deep_bf16": _cpu_deep_mlp(O, np)}
    out["total_cpu_s"] = round(time.perf_counter() - t_all, 1)
    return out


def _fill(np, shape, seed, scale=1.0):
    """Normal-looking values for timing runs (no denormals): a seeded block
    tiled over the shape (generating every element would dominate the run)."""
    blk = np.random.default_rng(seed).standard_normal(1 << 16).astype(np.float32) * scale
    return np.resize(blk, shape).astype(np.float32)


def _cpu_layer_slices(O, np, m, k, n, rows):
    """Oracle time of `rows` rows of Y (forward with bias and ReLU), `rows`
    rows of dX (dZ . W^T) and `rows` rows of dW (X^T . dZ, a full sequential
    k = m sum each) of an m x k x n layer, with the full layer's leading
    dimensions; the full step is m / rows forward and dX slices and k / rows
    dW slices."""
    X = _fill(np, (rows, k), 1)
    W = _fill(np, (k, n), 2, 1.0 / 64.0)
    b = _fill(np, n, 3, 0.1)
    dZ = _fill(np, (rows, n), 4)
    Xk = _fill(np, (m, rows), 5)       # X[:, k-slice] for the dW rows
    dZm = _fill(np, (m, n), 6)
    t0 = time.perf_counter()
    O.linear_fwd(X, W, b, 1)
    t1 = time.perf_counter()
    O.matmul(dZ, W, transB=True)
    t2 = time.perf_counter()
    O.matmul(Xk, dZm, transA=True)
    t3 = time.perf_counter()
    full = (t1 - t0) * m / rows + (t2 - t1) * m / rows + (t3 - t2) * k / rows
    return {"rows": rows, "sample_s": t3 - t0, "full_step_s": full, "tflops": 6.0 * m * n * k / full / 1e12}


def _cpu_sweep(O, np):
    """The bf16 sweep on the oracle (bf16 values widened to fp32 run the same
    loops): 1024x1024x1024 as a full fwd + bwd step (dZ from the ReLU mask),
    the other 26 shapes by one-row slices as in _cpu_layer_slices."""
    m = k = n = 1024
    X, W = O.round_bf16(_fill(np, (m, k), 11)), O.round_bf16(_fill(np, (k, n), 12, 1.0 / 32.0))
    b, dY = _fill(np, n, 13, 0.1), O.round_bf16(_fill(np, (m, n), 14))
    t0 = time.perf_counter()
    Y = O.linear_fwd(X, W, b, 1)
    O.linear_bwd(X, W, Y, dY, 1)
    full = time.perf_counter() - t0
    res = {"1024x1024x1024": {"full_step_s": round(full, 3), "tflops": round(6.0 * m * n * k / full / 1e12, 6),
                              "sample": "full step"}}
    for (mm, kk, nn) in SWEEP:
        if (mm, kk, nn) == (1024, 1024, 1024):
            continue
        r = _cpu_layer_slices(O, np, mm, kk, nn, rows=1)
        res[f"{mm}x{kk}x{nn}"] = {"full_step_s": round(r["full_step_s"], 1), "tflops": round(r["tflops"], 6),
                                  "sample": f"1-row slices, {r['sample_s']:.2f} s"}
    return {"cores": 1, "kind": "port", "shapes": res}


def _cpu_deep_mlp(O, np):
    """The 4096-8192-8192-8192-4096-1000 MLP at batch 16384 on the oracle,
    layer by layer on one-row slices (the first layer without dX, as on the
    GPU); the full step's time is extrapolated (CE and SGD are O(M N), left
    out)."""
    dims, B = [4096, 8192, 8192, 8192, 4096, 1000], 16384
    total, sample, layers = 0.0, 0.0, []
    for l in range(len(dims) - 1):
        r = _cpu_layer_slices(O, np, B, dims[l], dims[l + 1], rows=1)
        # Remove the first layer's dX share (same cost as its forward share).
        full = r["full_step_s"] * (2.0 / 3.0 if l == 0 else 1.0)
        total += full
        sample += r["sample_s"]
        layers.append(round(full, 1))
    macs = [B * dims[l] * dims[l + 1] for l in range(len(dims) - 1)]
    flop = 6.0 * sum(macs) - 2.0 * macs[0]
    return {"cores": 1, "kind": "port", "full_step_s": round(total, 1), "tflops": round(flop / total / 1e12, 6),
            "per_layer_full_s": layers, "sample": f"1-row slices of every layer ({sample:.1f} s), extrapolated"}


def _cpu_mlp(O, np, reps=20, warmup=3):
    """One full train step of the 784-256-128-10 MLP (batch 128) in the
    oracle on one core: forward, softmax-CE, backward, SGD; median of reps
    after warm-up steps."""
    dims, B = [784, 256, 128, 10], 128
    X = O.uniform(1, (B, 784))
    Ws = [O.uniform(2 + l, (dims[l], dims[l + 1]), -(6.0 / dims[l]) ** 0.5, (6.0 / dims[l]) ** 0.5)
          for l in range(3)]
    bs = [np.zeros(dims[l + 1], np.float32) for l in range(3)]
    lbl = O.labels(9, B, 10)
    times = []
    for it in range(warmup + reps):
        t0 = time.perf_counter()
        acts = [X]
        for l in range(3):
            acts.append(O.linear_fwd(acts[-1], Ws[l], bs[l], 1 if l < 2 else 0))
        _, g = O.softmax_ce(acts[3], lbl)
        for l in reversed(range(3)):
            # Same work as the GPU step: no gradient for the data batch.
            want = ("dX", "dW", "db") if l > 0 else ("dW", "db")
            g, dW, db = O.linear_bwd(acts[l], Ws[l], acts[l + 1], g, 1 if l < 2 else 0, want=want)
            O.sgd_update(Ws[l], dW, 1e-3)
            O.sgd_update(bs[l], db, 1e-3)
        if it >= warmup:
            times.append(time.perf_counter() - t0)
    ms = sorted(times)[reps // 2] * 1e3
    macs = [B * dims[l] * dims[l + 1] for l in range(3)]
    flop = 6.0 * sum(macs) - 2.0 * macs[0]
    return {"ms_per_step": round(ms, 3), "tflops": round(flop / (ms * 1e-3) / 1e12, 6), "cores": 1,
            "kind": "port", "sample": f"median of {reps} full steps after {warmup} warm-up steps"}


def _cpu_elementwise(O, np):
    """The eight oracle elementwise ops over 2^24 (median of 3) and 2^28 (one
    run) fp32 elements on one core, GB/s of algorithmic traffic; relu-bwd
    also split over min(cores, 8) threads (ctypes releases the GIL during
    the oracle call, so the chunks run in parallel)."""
    from concurrent.futures import ThreadPoolExecutor

    threads = min(os.cpu_count() or 1, 8)
    res = {}
    for log2n, reps in ((24, 3), (28, 1)):
        n = 1 << log2n
        a = _fill(np, n, 21)
        b = np.abs(_fill(np, n, 22)) + np.float32(0.5)
        ops = {}
        for name, code in (("add", O.EW_ADD), ("sub", O.EW_SUB), ("mul", O.EW_MUL), ("div", O.EW_DIV),
                           ("relu", O.EW_RELU), ("relu_bwd", O.EW_RELU_BWD), ("neg", O.EW_NEG),
                           ("scale", O.EW_SCALE)):
            binary = code in O.EW_BINARY
            times = []
            for _ in range(reps):
                t0 = time.perf_counter()
                O.elementwise(code, a, b if binary else None, alpha=0.5)
                times.append(time.perf_counter() - t0)
            ops[name] = round((12 if binary else 8) * n / sorted(times)[reps // 2] / 1e9, 2)
        chunks = [(i * n // threads, (i + 1) * n // threads) for i in range(threads)]
        with ThreadPoolExecutor(threads) as ex:
            times = []
            for _ in range(reps):
                t0 = time.perf_counter()
                list(ex.map(lambda c: O.elementwise(O.EW_RELU_BWD, a[c[0]:c[1]], b[c[0]:c[1]]), chunks))
                times.append(time.perf_counter() - t0)
        ops[f"relu_bwd_{threads}_threads"] = round(12 * n / sorted(times)[reps // 2] / 1e9, 2)
        res[f"2^{log2n}"] = ops
        del a, b
    return {"GB/s": res, "cores": 1, "threads_relu_bwd": threads, "kind": "port",
            "sample": "n = 2^24 median of 3, n = 2^28 one run"}


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
