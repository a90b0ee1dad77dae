"""Known-answer fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py
from exact integer arithmetic, single IEEE float32 operations and closed forms,
independently of the oracle).

CPU tests pin the oracle to them; GPU tests check the HIP path through the C
ABI against the same files: bit for bit for the integer-exact layer (fp32, and
bf16 with its one final rounding), the elementwise ops and SumReduce; within a
stated bound for softmax cross-entropy.
"""
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"
EW_OPS = {"add": 0, "sub": 1, "mul": 2, "div": 3, "relu": 4, "relu_bwd": 5, "neg": 6, "scale": 7}
EW_BINARY = {"add", "sub", "mul", "div", "relu_bwd"}


def load(name):
    with np.load(GOLDEN / name, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def linear_cases():
    z = load("linear_relu_int.npz")
    names = sorted({k.split("_", 1)[0] for k in z})
    out = []
    for c in names:
        d = {k.split("_", 1)[1]: v for k, v in z.items() if k.startswith(c + "_")}
        for k in ("X", "W", "b", "dY"):
            d[k] = d[k].astype(np.float32)
        d["act"] = int(d["act"])
        out.append(pytest.param(d, id=f"{c}-{d['X'].shape[0]}x{d['X'].shape[1]}x{d['W'].shape[1]}-act{d['act']}"))
    return out


def same_bits(got, ref, signed_zero=True):
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32)
    gn, rn = np.isnan(got), np.isnan(ref)
    assert np.array_equal(gn, rn), f"NaN positions differ ({int((gn != rn).sum())})"
    g, r = got[~gn], ref[~rn]
    if signed_zero:
        bad = g.view(np.int32) != r.view(np.int32)
    else:
        bad = g != r
    assert not bad.any(), f"{int(bad.sum())} elements differ, first at {np.flatnonzero(bad)[:5]}"


def relu_fixup(got, a, ref):
    """relu(-0.0): maxnum leaves the sign of the zero result unspecified."""
    got = np.array(got, np.float32, copy=True)
    neg0 = (a == 0) & np.signbit(a)
    assert np.all(got[neg0] == 0)
    got[neg0] = ref[neg0]
    return got


# ------------------------------------------------------------------ CPU ----
def test_fixtures_present_and_small():
    files = sorted(p.name for p in GOLDEN.glob("*.npz"))
    assert files == ["elementwise_ieee.npz", "linear_relu_int.npz", "softmax_ce_closed.npz", "sum_reduce_int.npz"]
    assert sum((GOLDEN / f).stat().st_size for f in files) < 512 * 1024


@pytest.mark.parametrize("case", linear_cases())
def test_oracle_linear_golden(case):
    c = case
    Y = O.linear_fwd(c["X"], c["W"], c["b"], c["act"])
    same_bits(Y, c["Y"])
    dX, dW, db = O.linear_bwd(c["X"], c["W"], Y, c["dY"], c["act"])
    same_bits(dX, c["dX"])
    same_bits(dW, c["dW"])
    same_bits(db, c["db"])


@pytest.mark.parametrize("op", list(EW_OPS))
def test_oracle_elementwise_golden(op):
    z = load("elementwise_ieee.npz")
    a, b = z["a"], z["b"]
    got = O.elementwise(EW_OPS[op], a, b if op in EW_BINARY else None, alpha=float(z["alpha"]))
    ref = z[f"out_{op}"]
    if op == "relu":
        got = relu_fixup(got, a, ref)
    same_bits(got, ref)


def test_oracle_softmax_ce_golden():
    z = load("softmax_ce_closed.npz")
    loss, d, rows = O.softmax_ce(z["logits"], z["labels"], want_rows=True)
    # fp32 evaluation of the closed forms: a few ulp of log C (2.3) and of the
    # probabilities; 1e-6 absolute covers both with margin.
    np.testing.assert_allclose(rows, z["loss_rows"], rtol=0, atol=1e-6)
    np.testing.assert_allclose(loss, z["loss"], rtol=0, atol=1e-6)
    np.testing.assert_allclose(d, z["dlogits"], rtol=0, atol=1e-7)


def test_oracle_sum_reduce_golden():
    z = load("sum_reduce_int.npz")
    x = z["x"].astype(np.float32)
    same_bits(O.sum_reduce(x, axis=0), z["axis0"])
    same_bits(O.sum_reduce(x, axis=1), z["axis1"])


def test_golden_catches_a_planted_mistake():
    """A bias added before the mask, a transposed W or a dropped bias must
    change the fixture's answer (so the fixtures can tell these apart)."""
    c = linear_cases()[0].values[0]
    X, W, b = c["X"], c["W"], c["b"]
    assert not np.array_equal(np.maximum(X @ W, 0), c["Y"])                    # bias dropped
    assert not np.array_equal(np.maximum(X @ W, 0) + b, c["Y"])               # bias after ReLU
    Wp = W[::-1].copy()
    assert not np.array_equal(np.maximum(X @ Wp + b, 0), c["Y"])              # W rows permuted


# ------------------------------------------------------------------ GPU ----
@pytest.mark.gpu
@pytest.mark.parametrize("case", linear_cases())
def test_gpu_linear_golden_fp32(gpu, stream, case):
    import torch

    from c3_amd import native as N
    from tests.parity import dev, empty, host, ptr

    c = case
    M, K = c["X"].shape
    Nn = c["W"].shape[1]
    Y = empty((M, Nn))
    N.linear_fwd(N.F32, ptr(dev(c["X"])), ptr(dev(c["W"])), ptr(dev(c["b"])), ptr(Y), M, K, Nn, c["act"], stream)
    dX, dW, db = empty((M, K)), empty((K, Nn)), empty(Nn)
    N.linear_bwd(N.F32, ptr(dev(c["X"])), ptr(dev(c["W"])), ptr(Y), ptr(dev(c["dY"])), ptr(dX), ptr(dW), ptr(db),
                 M, K, Nn, c["act"], stream)
    torch.cuda.synchronize()
    same_bits(host(Y), c["Y"])
    same_bits(host(dX), c["dX"])
    same_bits(host(dW), c["dW"])
    same_bits(host(db), c["db"])


@pytest.mark.gpu
@pytest.mark.parametrize("case", linear_cases())
def test_gpu_linear_golden_bf16(gpu, stream, case):
    import torch

    from c3_amd import native as N
    from tests.parity import dev, dev_bf16, empty, host, ptr

    c = case
    M, K = c["X"].shape
    Nn = c["W"].shape[1]
    Y = empty((M, Nn), dtype=torch.bfloat16)
    if K % 8 or Nn % 8:
        # bf16 operands move in 16-byte vectors: K and N must be multiples of
        # 8; anything else is refused with C3HIP_ERR_UNSUPPORTED, not computed.
        with pytest.raises(N.C3HipError) as e:
            N.linear_fwd(N.BF16, ptr(dev_bf16(c["X"])), ptr(dev_bf16(c["W"])), ptr(dev(c["b"])), ptr(Y), M, K, Nn,
                         c["act"], stream)
        assert e.value.code == 2
        return
    N.linear_fwd(N.BF16, ptr(dev_bf16(c["X"])), ptr(dev_bf16(c["W"])), ptr(dev(c["b"])), ptr(Y), M, K, Nn, c["act"],
                 stream)
    dX = empty((M, K), dtype=torch.bfloat16)
    dW, db = empty((K, Nn)), empty(Nn)
    N.linear_bwd(N.BF16, ptr(dev_bf16(c["X"])), ptr(dev_bf16(c["W"])), ptr(Y), ptr(dev_bf16(c["dY"])), ptr(dX),
                 ptr(dW), ptr(db), M, K, Nn, c["act"], stream)
    torch.cuda.synchronize()
    same_bits(host(Y), c["Y_bf16"])
    same_bits(host(dX), c["dX_bf16"])
    same_bits(host(dW), c["dW"])
    same_bits(host(db), c["db"])


@pytest.mark.gpu
@pytest.mark.parametrize("op", list(EW_OPS))
def test_gpu_elementwise_golden(gpu, stream, op):
    import torch

    from c3_amd import native as N
    from tests.parity import dev, empty, host, ptr

    z = load("elementwise_ieee.npz")
    a, b = z["a"], z["b"]
    assert a.size % 4 == 0
    # n = size: the float4 kernel; n = size - 1: the scalar kernel.
    for n in (a.size, a.size - 1):
        out = empty(n)
        N.elementwise(EW_OPS[op], N.F32, ptr(dev(a)), ptr(dev(b)), float(z["alpha"]), ptr(out), n, 0, stream)
        torch.cuda.synchronize()
        got, ref = host(out), z[f"out_{op}"][:n]
        if op == "relu":
            got = relu_fixup(got, a[:n], ref)
        same_bits(got, ref)


@pytest.mark.gpu
def test_gpu_softmax_ce_golden(gpu, stream):
    import torch

    from c3_amd import native as N
    from tests.parity import dev, empty, host, ptr

    z = load("softmax_ce_closed.npz")
    M, C = z["logits"].shape
    rows, d = empty(M), empty((M, C))
    N.softmax_ce(N.F32, ptr(dev(z["logits"])), ptr(dev(z["labels"])), ptr(rows), ptr(d), M, C, stream)
    torch.cuda.synchronize()
    # Device expf/logf are within a few ulp; the same 1e-6 / 1e-7 absolute
    # bounds as the oracle's check hold with margin.
    np.testing.assert_allclose(host(rows), z["loss_rows"], rtol=0, atol=1e-6)
    np.testing.assert_allclose(host(d), z["dlogits"], rtol=0, atol=1e-7)


@pytest.mark.gpu
@pytest.mark.parametrize("axis", [0, 1])
def test_gpu_sum_reduce_golden(gpu, stream, axis):
    import torch

    from c3_amd import native as N
    from tests.parity import dev, empty, host, ptr

    z = load("sum_reduce_int.npz")
    x = z["x"].astype(np.float32)
    M, Nn = x.shape
    out = empty(Nn if axis == 0 else M)
    N.sum_reduce(ptr(dev(x)), ptr(out), M, Nn, axis, stream)
    torch.cuda.synchronize()
    same_bits(host(out), z[f"axis{axis}"])


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_gpu_linear_empty_inner_dimension(gpu, stream, dtype):
    """K = 0: the k-sum is empty, so Y = act(0 + b) and the backward's only
    non-empty output is db = column sum of mask(Y) * dY (dX is M x 0, dW 0 x N)."""
    import torch

    from c3_amd import native as N
    from tests.parity import dev, dev_bf16, empty, host, ptr

    M, K, Nn = 40, 0, 24
    b = ((np.arange(Nn) - 11.5) / 4).astype(np.float32)   # multiples of 1/8: exact in bf16
    dY = np.random.default_rng(7).integers(-2, 3, size=(M, Nn)).astype(np.float32)
    dt, tdt, up = (N.F32, torch.float32, dev) if dtype == "fp32" else (N.BF16, torch.bfloat16, dev_bf16)
    Y = empty((M, Nn), dtype=tdt)
    N.linear_fwd(dt, None, None, ptr(dev(b)), ptr(Y), M, K, Nn, N.ACT_RELU, stream)
    db = empty(Nn)
    N.linear_bwd(dt, None, None, ptr(Y), ptr(up(dY)), None, None, ptr(db), M, K, Nn, N.ACT_RELU, stream)
    torch.cuda.synchronize()
    ref_y = np.broadcast_to(np.maximum(b, 0), (M, Nn))
    same_bits(host(Y), ref_y)            # b's values are exact in bf16
    same_bits(host(db), ((b > 0).astype(np.float32) * dY).sum(0).astype(np.float32))
