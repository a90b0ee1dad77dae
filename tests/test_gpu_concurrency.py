"""Concurrent use of the C ABI from several host threads, one stream each.

The reference requires its kernels to be re-entrant and dispatches from
several host threads (include/C3/LinalgElementwiseGen.h:58,
src/C3/C3KernelRegistry.cpp:94-111).  Here four threads each run the fused
Linear forward + backward (fp32 on the one-launch small path and on the large
tiles, bf16 with its pre-pass workspace) and two elementwise ops on their own
stream, several times over; every result must equal the one computed alone on
the default stream, bit for bit.  ctypes releases the GIL during the calls, so
the launches really overlap.
"""
import threading

import numpy as np
import pytest
import torch

from c3_amd import native as N
from tests.parity import dev, dev_bf16, empty, host, ptr

pytestmark = pytest.mark.gpu

# Small fp32 layers (one-launch backward), bf16 (pre-pass workspace from the
# stream-ordered pool, direct kernels), and an fp32 layer whose forward runs
# on 256x128 tiles and whose backward takes two launches.
CASES = [("fp32", 300, 260, 200), ("fp32", 128, 256, 128), ("bf16", 256, 512, 384), ("fp32", 4096, 256, 2048)]


def _ints(seed, shape):
    return np.random.default_rng(seed).integers(-2, 3, size=shape).astype(np.float32)


def _make(case, seed):
    dt, M, K, Nn = case
    bf = dt == "bf16"
    up = dev_bf16 if bf else dev
    tdt = torch.bfloat16 if bf else torch.float32
    X, W, b, dY = _ints(seed, (M, K)), _ints(seed + 1, (K, Nn)), _ints(seed + 2, Nn), _ints(seed + 3, (M, Nn))
    a = np.random.default_rng(seed + 4).standard_normal(M * Nn).astype(np.float32)
    d = np.random.default_rng(seed + 5).uniform(0.5, 2.0, M * Nn).astype(np.float32)
    ins = dict(X=up(X), W=up(W), b=dev(b), dY=up(dY), a=dev(a), d=dev(d))
    outs = dict(Y=empty((M, Nn), dtype=tdt), dX=empty((M, K), dtype=tdt), dW=empty((K, Nn)), db=empty(Nn),
                e1=empty(M * Nn), e2=empty(M * Nn))
    return ins, outs


def _run(case, ins, outs, stream):
    dt, M, K, Nn = case
    code = N.BF16 if dt == "bf16" else N.F32
    N.linear_fwd(code, ptr(ins["X"]), ptr(ins["W"]), ptr(ins["b"]), ptr(outs["Y"]), M, K, Nn, N.ACT_RELU, stream)
    N.linear_bwd(code, ptr(ins["X"]), ptr(ins["W"]), ptr(outs["Y"]), ptr(ins["dY"]), ptr(outs["dX"]), ptr(outs["dW"]),
                 ptr(outs["db"]), M, K, Nn, N.ACT_RELU, stream)
    n = M * Nn
    N.elementwise(N.EW_OPS["div"], N.F32, ptr(ins["a"]), ptr(ins["d"]), 0.0, ptr(outs["e1"]), n, 0, stream)
    N.elementwise(N.EW_OPS["relu_bwd"], N.F32, ptr(ins["a"]), ptr(outs["e1"]), 0.0, ptr(outs["e2"]), n, 0, stream)


def test_threads_on_own_streams_match_single_thread(gpu, stream):
    # Reference: each case alone on the default stream.
    refs = []
    for i, case in enumerate(CASES):
        ins, outs = _make(case, 100 + 10 * i)
        _run(case, ins, outs, stream)
        torch.cuda.synchronize()
        refs.append({k: host(v) for k, v in outs.items()})

    reps = 4
    bufs = [[_make(case, 100 + 10 * i) for _ in range(reps)] for i, case in enumerate(CASES)]
    streams = [torch.cuda.Stream() for _ in CASES]  # default priority
    torch.cuda.synchronize()
    errors = []

    def worker(i):
        try:
            s = streams[i].cuda_stream
            for r in range(reps):
                ins, outs = bufs[i][r]
                _run(CASES[i], ins, outs, s)
            streams[i].synchronize()
        except Exception as e:  # reported after join
            errors.append((i, repr(e)))

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(CASES))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not errors, errors
    torch.cuda.synchronize()
    for i in range(len(CASES)):
        for r in range(reps):
            _, outs = bufs[i][r]
            for k, v in outs.items():
                got = host(v)
                assert np.array_equal(got.view(np.int32), refs[i][k].view(np.int32)), (CASES[i], r, k)
