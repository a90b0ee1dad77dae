"""Call workspaces from the library's per-(device, stream) arena.

A layer backward takes its dZ, column-sum partials and split-K partials from
an arena the library keeps for the stream: each call reuses it from the start
(the stream runs the calls in order), it grows after a stream
synchronisation when a call needed more, a second thread that finds it in use
takes the stream-ordered allocator, and c3hip_shutdown frees it.  Each case
below checks the outputs bit for bit against the same calls made with the
arena switched off (C3_HIP_WORKSPACE_ARENA=0: every workspace from
hipMallocAsync on the stream).
"""
import threading

import numpy as np
import pytest
import torch

from c3_amd import native as N
from oracle import oracle as O
from tests.parity import dev_bf16, host, ptr

pytestmark = pytest.mark.gpu

# (M, K, N): a split-K dW with a pre-pass (1024^3), the largest (grows the
# arena), a small one again (reuses the grown arena from its start).
SHAPES = [(1024, 1024, 1024), (4096, 2048, 4096), (1024, 4096, 1024), (512, 256, 768)]


def _problems(seed, shapes):
    """Inputs on the device, copied before any kernel of the test's own stream reads them."""
    out = []
    for i, (M, K, Nn) in enumerate(shapes):
        s = seed + 7 * i
        X = O.normal(s, (M, K))
        W = O.normal(s + 1, (K, Nn), 0.0, 1.0 / np.sqrt(K))
        Y = O.normal(s + 2, (M, Nn))
        dY = O.normal(s + 3, (M, Nn))
        out.append(((dev_bf16(X), dev_bf16(W), dev_bf16(Y), dev_bf16(dY)), (M, K, Nn)))
    torch.cuda.synchronize()
    return out


def _bwd(stream, bufs, M, K, Nn):
    # Outputs are written in full by the call; torch.empty queues no fill on
    # another stream that could land after the call's writes.
    Xd, Wd, Yd, dYd = bufs
    dX = torch.empty(M, K, device="cuda:0", dtype=torch.bfloat16)
    dW, db = torch.empty(K, Nn, device="cuda:0"), torch.empty(Nn, device="cuda:0")
    N.linear_bwd(N.BF16, ptr(Xd), ptr(Wd), ptr(Yd), ptr(dYd), dX.data_ptr(), ptr(dW), ptr(db), M, K, Nn, 1, stream)
    return dX, dW, db


def _host(outs):
    torch.cuda.synchronize()  # the call's kernels run on the test's own stream
    return [o.view(torch.int16).cpu().numpy() if o.dtype == torch.bfloat16 else host(o) for o in outs]


def _reference(monkeypatch, stream, problems):
    monkeypatch.setenv("C3_HIP_WORKSPACE_ARENA", "0")
    ref = []
    for bufs, (M, K, Nn) in problems:
        ref.append(_host(_bwd(stream, bufs, M, K, Nn)))
        torch.cuda.synchronize()
    monkeypatch.delenv("C3_HIP_WORKSPACE_ARENA")
    return ref


def _same(got, ref):
    for g, r in zip(got, ref):
        assert np.array_equal(g, r)


def test_arena_back_to_back_calls_of_growing_and_shrinking_size(gpu, monkeypatch):
    s = torch.cuda.Stream()
    problems = _problems(0x100, SHAPES)
    ref = _reference(monkeypatch, s.cuda_stream, problems)
    for _ in range(2):  # the first pass grows the arena, the second reuses it
        outs = [_bwd(s.cuda_stream, bufs, *shape) for bufs, shape in problems]  # no synchronisation between calls
        torch.cuda.synchronize()
        for o, r in zip(outs, ref):
            _same(_host(o), r)


def test_arena_two_threads_on_one_stream(gpu, monkeypatch):
    s = torch.cuda.Stream()
    problems = _problems(0x200, SHAPES[:3])
    ref = _reference(monkeypatch, s.cuda_stream, problems)
    results = {}
    errors = []

    def worker(t):
        try:
            torch.cuda.set_device(0)
            outs = []
            for _ in range(3):
                outs.append([_bwd(s.cuda_stream, bufs, *shape) for bufs, shape in problems])
            results[t] = outs
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(2)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for t in range(2):
        for rnd in results[t]:
            for o, r in zip(rnd, ref):
                _same(_host(o), r)


def test_arenas_of_many_streams_are_bounded(gpu, monkeypatch):
    # More streams than the library keeps arenas for (8 per device): the least
    # recently used idle arena is freed (after a device synchronisation) as
    # each new stream arrives; every call still returns the reference bits.
    shape = SHAPES[0]
    problems = _problems(0x400, [shape])
    streams = [torch.cuda.Stream() for _ in range(12)]
    ref = _reference(monkeypatch, streams[0].cuda_stream, problems)
    for rnd in range(2):
        outs = [_bwd(st.cuda_stream, problems[0][0], *shape) for st in streams]
        for o in outs:
            _same(_host(o), ref[0])


def test_arena_freed_by_shutdown_and_rebuilt(gpu, monkeypatch):
    s = torch.cuda.Stream()
    shape = SHAPES[1]
    problems = _problems(0x300, [shape])
    ref = _reference(monkeypatch, s.cuda_stream, problems)
    _same(_host(_bwd(s.cuda_stream, problems[0][0], *shape)), ref[0])
    torch.cuda.synchronize()
    N.shutdown()
    N.init(0)
    _same(_host(_bwd(s.cuda_stream, problems[0][0], *shape)), ref[0])
    torch.cuda.synchronize()
