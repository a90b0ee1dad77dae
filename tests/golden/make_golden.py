"""Writes the known-answer fixtures in this folder (run: python tests/golden/make_golden.py).

The reference (ShengFlow/C3) holds no golden vectors for the fused
Linear+bias+ReLU path and cannot be built here, so these fixtures are fixed by
mathematics alone, computed with numpy and never with the oracle:

linear_relu_int.npz
    Integer-valued X, W, b, dY (entries in -2..2).  Every partial sum of the
    fused layer is an integer below 2^24, so the fp32 result is the exact
    integer result whatever the summation order: int64 arithmetic gives
    Y = relu(X.W + b) (act 1) or X.W + b (act 0), the ReLU mask Z > 0,
    dZ = mask * dY, dX = dZ.W^T, dW = X^T.dZ, db = column sum of dZ
    (src/C3/C3DialectLowering.cpp:467-610, src/C3/MLIRKernelGen.cpp:610-768,
    src/C3/C3BackwardCapture.cpp:501-528, :618-644, :681-723).  The bf16
    expectations are the same exact integers rounded once to bf16 (round to
    nearest even), the single rounding the bf16 path makes for Y and dX
    (fp32 accumulation of exact products; dW and db stay fp32).
elementwise_ieee.npz
    The eight single-node ops (src/C3/C3DialectLowering.cpp:246-350,
    src/C3/LinalgElementwiseGen.cpp:142-244) over every pair of IEEE special
    values (signed zeros, infinities, NaN, subnormals, extremes) plus random
    normals: add, sub, mul, div are single correctly-rounded float32
    operations (numpy float32, no flush to zero); relu = maxnum(x, 0) (NaN
    gives 0); relu_bwd = (x > 0 ? 1 : 0) * g; neg = sign flip; scale = x * 0.5.
softmax_ce_closed.npz
    Softmax cross-entropy closed forms in float64: equal logits in a row give
    loss log C and dlogits (1/C - onehot) / M; a row whose label logit exceeds
    the others by d gives loss log(1 + (C - 1) e^-d).
sum_reduce_int.npz
    SumReduce over axis 0 and axis 1 of an integer matrix (exact int64 sums;
    src/C3/C3DialectLowering.cpp:382-465).
"""
from __future__ import annotations

from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def bf16_rne(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bf16 (ties to even), returned as float32 (finite inputs)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return r.astype(np.uint32).view(np.float32)


def linear_case(seed: int, M: int, K: int, N: int, act: int) -> dict:
    rng = np.random.default_rng(seed)
    X = rng.integers(-2, 3, size=(M, K)).astype(np.int64)
    W = rng.integers(-2, 3, size=(K, N)).astype(np.int64)
    b = rng.integers(-2, 3, size=N).astype(np.int64)
    dY = rng.integers(-2, 3, size=(M, N)).astype(np.int64)
    Z = X @ W + b
    Y = np.maximum(Z, 0) if act == 1 else Z
    dZ = (Z > 0).astype(np.int64) * dY if act == 1 else dY
    dX = dZ @ W.T
    dW = X.T @ dZ
    db = dZ.sum(axis=0)
    f = lambda a: a.astype(np.float32)  # noqa: E731  (|values| < 2^24: exact)
    i8 = lambda a: a.astype(np.int8)  # noqa: E731  (inputs are stored as int8, read as float32)
    assert max(np.abs(Z).max(), np.abs(dX).max(), np.abs(dW).max(), np.abs(db).max()) < (1 << 24)
    return dict(X=i8(X), W=i8(W), b=i8(b), dY=i8(dY), Y=f(Y), dX=f(dX), dW=f(dW), db=f(db),
                Y_bf16=bf16_rne(f(Y)), dX_bf16=bf16_rne(f(dX)), act=np.int32(act))


def write_linear() -> None:
    cases = {"c0": (0xC3, 37, 70, 33, 1), "c1": (0xC4, 64, 128, 96, 1), "c2": (0xC5, 9, 300, 10, 0),
             "c3": (0xC6, 32, 784, 16, 1), "c4": (0xC7, 37, 72, 40, 1)}
    out = {}
    for name, (seed, M, K, N, act) in cases.items():
        for k, v in linear_case(seed, M, K, N, act).items():
            out[f"{name}_{k}"] = v
    np.savez_compressed(HERE / "linear_relu_int.npz", **out)


SPECIALS = np.array([0.0, -0.0, 1.0, -1.0, 2.0, 0.5, np.inf, -np.inf, np.nan, 1e-40, -1e-40, 1.4e-45,
                     1.1754944e-38, 3.4e38, -3.4e38, 1e-30, 1e30, 3.0, -7.25], dtype=np.float32)


def write_elementwise() -> None:
    a = np.repeat(SPECIALS, len(SPECIALS))
    b = np.tile(SPECIALS, len(SPECIALS))
    rng = np.random.default_rng(0xE1)
    # 19^2 special pairs + 1027 normals = 1388 elements, a multiple of 4 (the
    # vector kernels run it; the first 1387 take the scalar kernels).
    a = np.concatenate([a, rng.standard_normal(1027).astype(np.float32)])
    b = np.concatenate([b, rng.standard_normal(1027).astype(np.float32)])
    half = np.float32(0.5)
    with np.errstate(all="ignore"):
        ref = {
            "add": a + b, "sub": a - b, "mul": a * b, "div": a / b,
            "relu": np.fmax(a, np.float32(0.0)),
            "relu_bwd": np.where(a > 0, np.float32(1.0), np.float32(0.0)).astype(np.float32) * b,
            "neg": -a, "scale": a * half,
        }
    np.savez_compressed(HERE / "elementwise_ieee.npz", a=a, b=b, alpha=half,
                        **{f"out_{k}": v.astype(np.float32) for k, v in ref.items()})


def write_softmax_ce() -> None:
    M, C = 6, 10
    logits = np.zeros((M, C), np.float32)
    labels = np.array([0, 3, 9, 5, 1, 7], np.int32)
    loss = np.zeros(M)
    dl = np.zeros((M, C))
    for i, c in enumerate([0.0, 1.5, -3.0]):           # rows 0-2: equal logits
        logits[i, :] = c
        loss[i] = np.log(C)
        dl[i, :] = 1.0 / C
        dl[i, labels[i]] -= 1.0
    for i, d in zip(range(3, 6), [1.0, 4.0, 12.0]):     # rows 3-5: label logit ahead by d
        logits[i, labels[i]] = d
        loss[i] = np.log1p((C - 1) * np.exp(-d))
        p = np.full(C, np.exp(-d)) / (1 + (C - 1) * np.exp(-d))
        p[labels[i]] = 1.0 / (1 + (C - 1) * np.exp(-d))
        p[labels[i]] -= 1.0
        dl[i, :] = p
    dl /= M
    np.savez_compressed(HERE / "softmax_ce_closed.npz", logits=logits, labels=labels, loss_rows=loss,
                        loss=np.float64(loss.mean()), dlogits=dl)


def write_sum_reduce() -> None:
    rng = np.random.default_rng(0x5E)
    x = rng.integers(-100, 101, size=(75, 130)).astype(np.int64)
    np.savez_compressed(HERE / "sum_reduce_int.npz", x=x.astype(np.int16),
                        axis0=x.sum(axis=0).astype(np.float32), axis1=x.sum(axis=1).astype(np.float32))


if __name__ == "__main__":
    write_linear()
    write_elementwise()
    write_softmax_ce()
    write_sum_reduce()
    for p in sorted(HERE.glob("*.npz")):
        print(p.name, p.stat().st_size, "bytes")
