"""GPU parity of the fused backward chain (c3hip_backward_chain).

The reference merges the backward graphs of a run of single-input nodes into
one multi-output graph (src/C3/C3BackwardCapture.cpp:1140-1210), so each
output is what the node's own backward graph gives.  Here:
  * every output is bit-identical to the single-node GPU kernels run one after
    another (those are pinned against the oracle in test_gpu_math.py);
  * chains of the exact rules (ReLU mask, Log grad/x, Neg) are bit-identical to
    the oracle's composition;
  * chains with transcendental rules agree with the oracle's composition to a
    normwise relative error of 1e-5, NaN/inf positions included;
on the vector path (n a multiple of 4, 16-byte aligned) and the scalar path
(ragged n, offset pointers), with outputs aliasing inputs and skipped outputs.
"""
import itertools

import numpy as np
import pytest
import torch

from c3_amd import native as N
from oracle import oracle as O
from tests.parity import dev, empty, host, ptr

pytestmark = pytest.mark.gpu

RULES = {N.CHAIN_RELU: (N.EW_RELU_BWD, "x_first"), N.CHAIN_SIGMOID: (N.EW_SIGMOID_BWD, "x_first"),
         N.CHAIN_TANH: (N.EW_TANH_BWD, "x_first"), N.CHAIN_EXP: (N.EW_EXP_BWD, "x_first"),
         N.CHAIN_LOG: (N.EW_DIV, "g_first"), N.CHAIN_NEG: (N.EW_NEG, "unary")}
EXACT = {N.CHAIN_RELU, N.CHAIN_LOG, N.CHAIN_NEG}


def inputs(seed, nodes, n):
    g = O.normal(seed, n, 0.0, 2.0)
    xs = []
    for k, node in enumerate(nodes):
        if node == N.CHAIN_NEG:
            xs.append(None)
            continue
        x = O.uniform(seed + 10 + k, n, -5.0, 5.0)
        if node == N.CHAIN_LOG:
            x = np.abs(x) + np.float32(0.25)
        if node == N.CHAIN_RELU:
            x[::7] = 0.0  # the mask's boundary
        xs.append(x)
    return g, xs


def single_node_kernels(nodes, g_dev, x_devs, n, stream):
    """The nodes one by one through c3hip_elementwise."""
    outs = []
    cur = g_dev
    for node, x in zip(nodes, x_devs):
        op, form = RULES[node]
        out = empty(n)
        if form == "x_first":
            N.elementwise(op, N.F32, ptr(x), ptr(cur), 0.0, ptr(out), n, 0, stream)
        elif form == "g_first":
            N.elementwise(op, N.F32, ptr(cur), ptr(x), 0.0, ptr(out), n, 0, stream)
        else:
            N.elementwise(op, N.F32, ptr(cur), None, 0.0, ptr(out), n, 0, stream)
        outs.append(out)
        cur = out
    return outs


def same_bits(a, b, what):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    diff = a.view(np.int32) != b.view(np.int32)
    assert not diff.any(), f"{what}: {int(diff.sum())} elements differ, first at {int(np.argmax(diff))}"


def close_to_oracle(got, ref, what):
    gn, rn = np.isnan(got), np.isnan(ref)
    assert np.array_equal(gn, rn), f"{what}: NaN positions differ"
    gi, ri = np.isinf(got), np.isinf(ref)
    assert np.array_equal(gi, ri) and np.array_equal(got[gi], ref[ri]), f"{what}: infinities differ"
    fin = ~(gn | gi)
    err = np.max(np.abs(got[fin].astype(np.float64) - ref[fin]), initial=0.0)
    scale = np.max(np.abs(ref[fin].astype(np.float64)), initial=0.0)
    assert err <= 1e-5 * scale, f"{what}: normwise rel err {err / max(scale, 1e-300):.3e}"


# Every pair, a spread of triples and the quadruples the window allows.
PAIRS = list(itertools.product(range(6), repeat=2))
LONGER = [(0, 1, 2), (4, 5, 0), (3, 4, 1), (2, 2, 2), (5, 5, 5), (0, 1, 2, 3), (3, 2, 1, 0), (4, 0, 5, 1),
          (1, 1, 1, 1), (0, 4, 0, 4)]


@pytest.mark.parametrize("n", [1 << 16, 1001])
@pytest.mark.parametrize("nodes", [(k,) for k in range(6)] + PAIRS + LONGER,
                         ids=lambda t: "+".join(str(v) for v in t) if isinstance(t, tuple) else str(t))
def test_chain_matches_single_node_kernels(gpu, stream, nodes, n):
    g, xs = inputs(900 + 31 * len(nodes) + sum(nodes), nodes, n)
    g_dev = dev(g)
    x_devs = [None if x is None else dev(x) for x in xs]
    want = single_node_kernels(nodes, g_dev, x_devs, n, stream)
    outs = [empty(n) for _ in nodes]
    N.backward_chain(N.F32, ptr(g_dev), [None if x is None else ptr(x) for x in x_devs], list(nodes),
                     [ptr(o) for o in outs], n, stream)
    with np.errstate(all="ignore"):
        ref = O.backward_chain(list(nodes), g, xs)
    for k in range(len(nodes)):
        got = host(outs[k])
        same_bits(got, host(want[k]), f"output {k} vs single-node kernels")
        if set(nodes[: k + 1]) <= EXACT:
            same_bits(got, ref[k], f"output {k} vs oracle")
        else:
            close_to_oracle(got, ref[k], f"output {k} vs oracle")


def test_chain_unaligned_views_take_the_scalar_path(gpu, stream):
    nodes = [N.CHAIN_SIGMOID, N.CHAIN_RELU, N.CHAIN_LOG]
    n = 4096
    g, xs = inputs(950, nodes, n + 1)
    # One-element offsets: every base address is 4 mod 16.
    g_dev, x_devs = dev(g), [dev(x) for x in xs]
    outs = [empty(n + 1) for _ in nodes]
    N.backward_chain(N.F32, ptr(g_dev) + 4, [ptr(x) + 4 for x in x_devs], nodes, [ptr(o) + 4 for o in outs], n,
                     stream)
    with np.errstate(all="ignore"):
        ref = O.backward_chain(nodes, g[1:], [x[1:] for x in xs])
    for k in range(3):
        got = host(outs[k])[1:]
        close_to_oracle(got, ref[k], f"offset output {k}")
    same_bits(host(outs[2])[1:], O.elementwise(O.EW_DIV, host(outs[1])[1:], xs[2][1:]), "offset Log step")


def test_chain_in_place_and_skipped_outputs(gpu, stream):
    nodes = [N.CHAIN_EXP, N.CHAIN_TANH, N.CHAIN_NEG]
    n = 1 << 14
    g, xs = inputs(960, nodes, n)
    x_devs = [None if x is None else dev(x) for x in xs]
    full = [empty(n) for _ in nodes]
    N.backward_chain(N.F32, ptr(dev(g)), [None if x is None else ptr(x) for x in x_devs], nodes,
                     [ptr(o) for o in full], n, stream)
    # Only the last grad, written over the incoming grad.
    g_dev = dev(g)
    N.backward_chain(N.F32, ptr(g_dev), [None if x is None else ptr(x) for x in x_devs], nodes,
                     [None, None, ptr(g_dev)], n, stream)
    same_bits(host(g_dev), host(full[2]), "in-place last grad")
    # First grad written over node 0's forward input.
    x0 = x_devs[0].clone()
    outs = [x0, empty(n), empty(n)]
    N.backward_chain(N.F32, ptr(dev(g)), [ptr(x0), ptr(x_devs[1]), None], nodes, [ptr(o) for o in outs], n, stream)
    for k in range(3):
        same_bits(host(outs[k]), host(full[k]), f"aliased output {k}")


def test_chain_empty_and_errors(gpu, stream):
    N.backward_chain(N.F32, 0, [0], [N.CHAIN_RELU], [0], 0, stream)  # n = 0: nothing to do
    x = empty(8)
    with pytest.raises(N.C3HipError) as e:
        N.backward_chain(N.BF16, ptr(x), [ptr(x)], [N.CHAIN_RELU], [ptr(x)], 8, stream)
    assert e.value.code == N.ERR_UNSUPPORTED
    for nodes in ([], [0] * 5, [6], [-1]):
        with pytest.raises(N.C3HipError) as e:
            N.backward_chain(N.F32, ptr(x), [ptr(x)] * len(nodes), nodes, [ptr(x)] * len(nodes), 8, stream)
        assert e.value.code == N.ERR_INVALID
    with pytest.raises(N.C3HipError):
        N.backward_chain(N.F32, ptr(x), [None], [N.CHAIN_SIGMOID], [ptr(x)], 8, stream)
    torch.cuda.synchronize()
