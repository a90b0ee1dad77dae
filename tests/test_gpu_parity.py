"""GPU parity of the HIP path (through the C ABI) against the oracle.

Integer-valued inputs make every partial sum exact in fp32, so there the GPU
must match the oracle bit for bit whatever its summation order.  Real-valued
inputs are checked with the tolerances in tests/parity.py.
"""
import numpy as np
import pytest
import torch

from c3_amd import native as N
from oracle import oracle as O
from tests.parity import (assert_close_gemm, dev, empty, gemm_bound, host, mask_flips, ptr)

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5


def same_bits(got, ref):
    """Bit equality, with any NaN payload accepted for a NaN."""
    got = np.asarray(got, dtype=np.float32)
    ref = np.asarray(ref, dtype=np.float32)
    gn, rn = np.isnan(got), np.isnan(ref)
    assert np.array_equal(gn, rn), f"NaN positions differ ({int((gn != rn).sum())})"
    g, r = got[~gn].view(np.int32), ref[~rn].view(np.int32)
    bad = g != r
    assert not bad.any(), f"{int(bad.sum())} elements differ in bits, first at {np.flatnonzero(bad)[:5]}"


def ints(seed, shape, lo=-2, hi=2):
    return np.random.default_rng(seed).integers(lo, hi + 1, size=shape).astype(np.float32)


# ------------------------------------------------------------ elementwise ----
SPECIALS = np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan, 1e-40, -1e-40, 3.4e38, -3.4e38, 1e-30],
                    dtype=np.float32)


@pytest.mark.parametrize("op", list(N.EW_OPS))
@pytest.mark.parametrize("n", [1 << 16, 1000003, 12])
def test_elementwise_bit_exact(gpu, stream, op, n):
    code = N.EW_OPS[op]
    a = O.normal(100 + code, n)
    b = O.uniform(200 + code, n, 0.5, 2.0) if op == "div" else O.normal(300 + code, n)
    a[: len(SPECIALS)] = SPECIALS[: min(n, len(SPECIALS))]
    b[: len(SPECIALS)] = SPECIALS[::-1][: min(n, len(SPECIALS))]
    da, db_, out = dev(a), dev(b), empty(n)
    N.elementwise(code, N.F32, ptr(da), ptr(db_), 0.5, ptr(out), n, 0, stream)
    with np.errstate(all="ignore"):
        ref = O.elementwise(code, a, b if code in O.EW_BINARY else None, alpha=0.5)
    if op == "relu":
        # relu(-0.0): the reference's maxnum leaves the sign of the zero unspecified.
        neg0 = (a == 0) & np.signbit(a)
        got = host(out)
        assert np.all(got[neg0] == 0)
        got[neg0] = ref[neg0]
        same_bits(got, ref)
    else:
        same_bits(host(out), ref)


@pytest.mark.parametrize("op", ["add", "sub", "mul", "div", "relu_bwd"])
@pytest.mark.parametrize("bmod", [256, 7, -256, -5])
def test_elementwise_broadcast(gpu, stream, op, bmod):
    code = N.EW_OPS[op]
    n = 256 * 37
    big = O.normal(400, n)
    small = O.uniform(401, abs(bmod), 0.5, 2.0)
    a, b = (big, small) if bmod > 0 else (small, big)
    out = empty(n)
    N.elementwise(code, N.F32, ptr(dev(a)), ptr(dev(b)), 0.0, ptr(out), n, bmod, stream)
    same_bits(host(out), O.elementwise(code, a, b, bmod=bmod))


def test_elementwise_unaligned_pointers(gpu, stream):
    n = 4096
    a, b = O.normal(500, n + 1), O.normal(501, n + 1)
    da, db_ = dev(a), dev(b)
    out = empty(n + 1)
    N.elementwise(N.EW_ADD, N.F32, ptr(da) + 4, ptr(db_) + 4, 0.0, ptr(out) + 4, n, 0, stream)
    same_bits(host(out)[1:], a[1:] + b[1:])


# ----------------------------------------------------------- fused forward ----
FWD_SHAPES = [(128, 784, 256), (128, 256, 128), (128, 128, 10), (256, 512, 384), (67, 45, 33), (1, 1, 1),
              (130, 129, 131), (512, 1024, 1000), (1024, 256, 1024)]


@pytest.mark.parametrize("M,K,Nn", FWD_SHAPES)
@pytest.mark.parametrize("act", [1, 0])
def test_linear_fwd_integer_bit_exact(gpu, stream, M, K, Nn, act):
    X, W, b = ints(1, (M, K)), ints(2, (K, Nn)), ints(3, Nn)
    Y = empty((M, Nn))
    N.linear_fwd(N.F32, ptr(dev(X)), ptr(dev(W)), ptr(dev(b)), ptr(Y), M, K, Nn, act, stream)
    same_bits(host(Y), O.linear_fwd(X, W, b, act))


@pytest.mark.parametrize("M,K,Nn", FWD_SHAPES)
def test_linear_fwd_real(gpu, stream, M, K, Nn):
    X = O.normal(11, (M, K))
    W = O.normal(12, (K, Nn), 0.0, 1.0 / np.sqrt(K))
    b = O.normal(13, Nn, 0.0, 0.1)
    Y = empty((M, Nn))
    N.linear_fwd(N.F32, ptr(dev(X)), ptr(dev(W)), ptr(dev(b)), ptr(Y), M, K, Nn, 1, stream)
    got = host(Y)
    t = O.matmul(X, W)
    z = O.bias_act(t, b, act=0)
    ref = O.bias_act(t, b, act=1)
    bound = gemm_bound(X, W, K)
    assert_close_gemm(got, ref, bound, FP32_TOL, what="Y")
    mask_flips(got, z, bound)


def test_linear_fwd_no_bias_and_k0(gpu, stream):
    M, K, Nn = 64, 32, 48
    X, W = ints(21, (M, K)), ints(22, (K, Nn))
    Y = empty((M, Nn))
    N.linear_fwd(N.F32, ptr(dev(X)), ptr(dev(W)), None, ptr(Y), M, K, Nn, 0, stream)
    same_bits(host(Y), O.matmul(X, W))
    # K = 0: Y = act(bias).
    b = O.normal(23, Nn)
    Y0 = empty((M, Nn))
    N.linear_fwd(N.F32, None, None, ptr(dev(b)), ptr(Y0), M, 0, Nn, 1, stream)
    same_bits(host(Y0), np.tile(np.maximum(b, 0), (M, 1)))


# ---------------------------------------------------------- fused backward ----
BWD_SHAPES = [(128, 784, 256), (128, 128, 10), (256, 512, 384), (67, 45, 33), (1, 1, 1), (130, 129, 131),
              (512, 1000, 1024), (1000, 256, 512)]


def _bwd_inputs(seed, M, K, Nn, integer):
    if integer:
        X, W, b, dY = ints(seed, (M, K)), ints(seed + 1, (K, Nn)), ints(seed + 2, Nn), ints(seed + 3, (M, Nn))
    else:
        X = O.normal(seed, (M, K))
        W = O.normal(seed + 1, (K, Nn), 0.0, 1.0 / np.sqrt(K))
        b = O.normal(seed + 2, Nn, 0.0, 0.1)
        dY = O.normal(seed + 3, (M, Nn))
    Y = O.linear_fwd(X, W, b, 1)
    return X, W, Y, dY


def _run_bwd(stream, X, W, Y, dY, act, want=("dX", "dW", "db")):
    M, K = X.shape
    Nn = W.shape[1]
    dX = empty((M, K)) if "dX" in want else None
    dW = empty((K, Nn)) if "dW" in want else None
    db = empty(Nn) if "db" in want else None
    keep = [dev(X), dev(W), dev(Y), dev(dY)]
    N.linear_bwd(N.F32, ptr(keep[0]), ptr(keep[1]), ptr(keep[2]), ptr(keep[3]), ptr(dX), ptr(dW), ptr(db), M, K,
                 Nn, act, stream)
    return (None if dX is None else host(dX), None if dW is None else host(dW), None if db is None else host(db))


def test_f32_all_k_at_once_kernels_match_the_k_loop(gpu, stream):
    # GEMMs over k <= 128 on the 64x64 register tile with vector-aligned
    # operands issue every k-tile's loads at once (t64x64k kernels); k = 144
    # takes the k loop.  Padding k from 128 to 144 with zero operands (an
    # exact +-0 added to each sum) must leave the real-valued outputs
    # unchanged bit for bit: the forward (289 tiles of 64x64, more than the
    # direct 64x64 tile takes) and the one-launch ReLU backward (dX over
    # k = N, dW over k = M, db).
    rng = np.random.default_rng(0x64)
    M, K, Nn = 1088, 128, 1088
    X = rng.standard_normal((M, K + 16), dtype=np.float32)
    X[:, K:] = 0.0
    W = rng.standard_normal((K + 16, Nn), dtype=np.float32) / np.float32(12.0)
    b = rng.standard_normal(Nn, dtype=np.float32)
    outs = []
    for k in (K, K + 16):
        Yg = empty((M, Nn))
        N.linear_fwd(N.F32, ptr(dev(np.ascontiguousarray(X[:, :k]))), ptr(dev(np.ascontiguousarray(W[:k]))), ptr(dev(b)),
                     ptr(Yg), M, k, Nn, 1, stream)
        outs.append(host(Yg))
    same_bits(outs[0], outs[1])

    M, K, Nn = 128, 96, 128
    X = rng.standard_normal((M + 16, K), dtype=np.float32)
    W = rng.standard_normal((K, Nn + 16), dtype=np.float32) / np.float32(10.0)
    Y = rng.standard_normal((M + 16, Nn + 16), dtype=np.float32)
    dY = rng.standard_normal((M + 16, Nn + 16), dtype=np.float32)
    dY[M:, :] = 0.0
    dY[:, Nn:] = 0.0
    gX, gW, gb = _run_bwd(stream, X[:M], np.ascontiguousarray(W[:, :Nn]), np.ascontiguousarray(Y[:M, :Nn]),
                          np.ascontiguousarray(dY[:M, :Nn]), 1)
    pX, pW, pb = _run_bwd(stream, X, W, Y, dY, 1)
    same_bits(gX, pX[:M])
    same_bits(gW, pW[:, :Nn])
    same_bits(gb, pb[:Nn])


@pytest.mark.parametrize("M,K,Nn,act", [(128, 256, 128, 1), (128, 128, 10, 0), (37, 70, 33, 1), (64, 300, 40, 1),
                                          (200, 96, 130, 0)])
def test_small_bwd_one_launch_matches_two(gpu, stream, monkeypatch, M, K, Nn, act):
    # Small fp32 layers run dX and dW + db in one launch; forcing the 64x64
    # tile takes the two separate launches of the same tile.  Real-valued
    # inputs: the results must agree bit for bit (same tiles, same k order).
    X, W, Y, dY = _bwd_inputs(71, M, K, Nn, False)
    one = _run_bwd(stream, X, W, Y, dY, act)
    monkeypatch.setenv("C3_HIP_GEMM_TILE", "t64x64")
    two = _run_bwd(stream, X, W, Y, dY, act)
    for g1, g2 in zip(one, two):
        same_bits(g1, g2)
    rX, rW, rb = O.linear_bwd(X, W, Y, dY, act)
    assert_close_gemm(one[1], rW, gemm_bound(X.T, O.relu_mask_mul(Y, dY) if act else dY, M), FP32_TOL, what="dW")


@pytest.mark.parametrize("tile", ["t64x64", "t128x128", "t256x128", "t128x256", "t256x128d", "t128x256d", "t256x256d",
                                  "t64x64d"])
@pytest.mark.parametrize("M,K,Nn", [(300, 260, 200), (257, 128, 64), (272, 144, 80)])
def test_every_fp32_tile_bit_exact(gpu, stream, monkeypatch, tile, M, K, Nn):
    # Each tile the planner can pick, forced for every GEMM of the layer
    # (forward, dX with mask, dW with mask and db), on ragged extents.
    monkeypatch.setenv("C3_HIP_GEMM_TILE", tile)
    X, W, Y, dY = _bwd_inputs(61, M, K, Nn, True)
    b = ints(64, Nn)
    Yg = empty((M, Nn))
    N.linear_fwd(N.F32, ptr(dev(X)), ptr(dev(W)), ptr(dev(b)), ptr(Yg), M, K, Nn, 1, stream)
    same_bits(host(Yg), O.linear_fwd(X, W, b, 1))
    gX, gW, gb = _run_bwd(stream, X, W, Y, dY, 1)
    rX, rW, rb = O.linear_bwd(X, W, Y, dY, 1)
    same_bits(gX, rX)
    same_bits(gW, rW)
    same_bits(gb, rb)


@pytest.mark.parametrize("tile", [None, "t64x64", "t128x128", "t256x128", "t128x256", "t256x128d", "t128x256d",
                                  "t256x256d", "t64x64d"])
@pytest.mark.parametrize("M,K,Nn", [(1024, 768, 1536), (300, 260, 200), (2048, 1024, 4096)])
def test_bwd_dz_side_output_matches_masked_launches(gpu, stream, monkeypatch, tile, M, K, Nn):
    # With dX and dW both asked for, the dX kernel also writes dZ = mask(Y) dY
    # and dW + db run on it unmasked; alone, each runs with the mask in its
    # operand loads.  Real-valued inputs: both routes must agree bit for bit.
    if tile:
        monkeypatch.setenv("C3_HIP_GEMM_TILE", tile)
    X = O.normal(81, (M, K))
    W = O.normal(82, (K, Nn), 0.0, 1.0 / np.sqrt(K))
    Y = O.normal(83, (M, Nn))          # the saved output: mixed signs, exact zeros of both signs
    Y[::7, ::5] = 0.0
    Y[3::11, 1::9] = -0.0
    dY = O.normal(84, (M, Nn))
    both = _run_bwd(stream, X, W, Y, dY, 1)
    gx = _run_bwd(stream, X, W, Y, dY, 1, ("dX",))[0]
    _, gw, gb = _run_bwd(stream, X, W, Y, dY, 1, ("dW", "db"))
    same_bits(both[0], gx)
    same_bits(both[1], gw)
    same_bits(both[2], gb)


@pytest.mark.parametrize("pair", [("t256x128d", "t256x128"), ("t128x256d", "t128x256"), ("t256x256d", "t256x128"),
                                  ("t64x64d", "t64x64")])
@pytest.mark.parametrize("M,K,Nn", [(512, 256, 384), (1000, 512, 776), (272, 144, 80), (300, 272, 200)])
def test_f32_direct_tiles_match_register_tiles(gpu, stream, monkeypatch, pair, M, K, Nn):
    # The direct-to-LDS tiles (operands DMA'd into LDS, three stages) multiply
    # in the register tiles' order, so the forward, dX and dW agree bit for bit
    # on real-valued inputs, ragged extents included.  With K, N and M all
    # multiples of 16 the direct backward runs through the dZ pre-pass, whose
    # db sums in another order than the dW kernel's side output: db within the
    # fp32 bound of both against the oracle.
    X = O.normal(91, (M, K))
    W = O.normal(92, (K, Nn), 0.0, 1.0 / np.sqrt(K))
    b = O.normal(93, Nn, 0.0, 0.1)
    dY = O.normal(94, (M, Nn))
    outs = {}
    for tile in pair:
        monkeypatch.setenv("C3_HIP_GEMM_TILE", tile)
        Yg = empty((M, Nn))
        N.linear_fwd(N.F32, ptr(dev(X)), ptr(dev(W)), ptr(dev(b)), ptr(Yg), M, K, Nn, 1, stream)
        Y = host(Yg)
        outs[tile] = (Y,) + _run_bwd(stream, X, W, Y, dY, 1)
    d, r = outs[pair[0]], outs[pair[1]]
    for i, name in enumerate(("Y", "dX", "dW")):
        same_bits(d[i], r[i])
    Y = d[0]
    rb = O.linear_bwd(X, W, Y, dY, 1)[2]
    bound = 2.02 * M * 2.0 ** -24 * np.abs(O.relu_mask_mul(Y, dY).astype(np.float64)).sum(0)
    for gb in (d[3], r[3]):
        assert_close_gemm(gb, rb, bound, FP32_TOL, what="db")


@pytest.mark.parametrize("tile", ["t256x128d", "t128x256d", "t256x256d", "t64x64d"])
@pytest.mark.parametrize("M,K,Nn", [(512, 16, 256), (256, 32, 512), (16, 512, 272), (32, 48, 16), (64, 96, 80)])
def test_f32_direct_tiles_short_k_bit_exact(gpu, stream, monkeypatch, tile, M, K, Nn):
    # One, two and three k-tiles through the three-stage pipeline (the
    # prologue's second tile and the last waits), and extents below one tile:
    # the forward (k = K), dX (k = N) and dW (k = M) on integer inputs against
    # the oracle.
    monkeypatch.setenv("C3_HIP_GEMM_TILE", tile)
    X, W, Y, dY = _bwd_inputs(97, M, K, Nn, True)
    b = ints(98, Nn)
    Yg = empty((M, Nn))
    N.linear_fwd(N.F32, ptr(dev(X)), ptr(dev(W)), ptr(dev(b)), ptr(Yg), M, K, Nn, 1, stream)
    same_bits(host(Yg), O.linear_fwd(X, W, b, 1))
    gX, gW, gb = _run_bwd(stream, X, W, Y, dY, 1)
    rX, rW, rb = O.linear_bwd(X, W, Y, dY, 1)
    same_bits(gX, rX)
    same_bits(gW, rW)
    same_bits(gb, rb)


@pytest.mark.parametrize("tile", [None, "t256x128d", "t256x256d"])
def test_f32_direct_backward_specials(gpu, stream, monkeypatch, tile):
    # The direct route's pre-pass forms dZ = (Y > 0 ? 1 : 0) * dY as one IEEE
    # multiply: -0 and NaN in Y mask to zero, +inf in Y passes dY, a zero mask
    # times an infinite or NaN dY gives NaN, which then reaches its dX row, dW
    # column and db entry.  Integer elsewhere, so every other element is exact.
    if tile:
        monkeypatch.setenv("C3_HIP_GEMM_TILE", tile)
    M, K, Nn = 512, 128, 256
    X, W, Y, dY = _bwd_inputs(99, M, K, Nn, True)
    rng = np.random.default_rng(100)
    for v in (-0.0, np.nan, np.inf, -np.inf):
        Y[rng.integers(0, M, 6), rng.integers(0, Nn, 6)] = v
    for v in (-0.0, np.inf, -np.inf, np.nan):
        dY[rng.integers(0, M, 3), rng.integers(0, Nn, 3)] = v
    gX, gW, gb = _run_bwd(stream, X, W, Y, dY, 1)
    rX, rW, rb = O.linear_bwd(X, W, Y, dY, 1)
    same_bits(gX, rX)
    same_bits(gW, rW)
    same_bits(gb, rb)


@pytest.mark.parametrize("M,K,Nn", BWD_SHAPES)
@pytest.mark.parametrize("act", [1, 0])
def test_linear_bwd_integer_bit_exact(gpu, stream, M, K, Nn, act):
    X, W, Y, dY = _bwd_inputs(31, M, K, Nn, True)
    gX, gW, gb = _run_bwd(stream, X, W, Y, dY, act)
    rX, rW, rb = O.linear_bwd(X, W, Y, dY, act)
    same_bits(gX, rX)
    same_bits(gW, rW)
    same_bits(gb, rb)


@pytest.mark.parametrize("M,K,Nn", BWD_SHAPES)
def test_linear_bwd_real(gpu, stream, M, K, Nn):
    X, W, Y, dY = _bwd_inputs(41, M, K, Nn, False)
    gX, gW, gb = _run_bwd(stream, X, W, Y, dY, 1)
    rX, rW, rb = O.linear_bwd(X, W, Y, dY, 1)
    dZ = O.relu_mask_mul(Y, dY)
    assert_close_gemm(gX, rX, gemm_bound(dZ, W.T, Nn), FP32_TOL, what="dX")
    assert_close_gemm(gW, rW, gemm_bound(X.T, dZ, M), FP32_TOL, what="dW")
    assert_close_gemm(gb, rb, 2.02 * M * 2.0 ** -24 * np.abs(dZ.astype(np.float64)).sum(0), FP32_TOL, what="db")


@pytest.mark.parametrize("want", [("dX",), ("dW",), ("db",), ("dW", "db"), ("dX", "db")])
def test_linear_bwd_optional_outputs(gpu, stream, want):
    M, K, Nn = 96, 80, 72
    X, W, Y, dY = _bwd_inputs(51, M, K, Nn, True)
    got = _run_bwd(stream, X, W, Y, dY, 1, want)
    ref = O.linear_bwd(X, W, Y, dY, 1)
    for g, r, name in zip(got, ref, ("dX", "dW", "db")):
        if name in want:
            same_bits(g, r)
        else:
            assert g is None


def test_linear_bwd_mask_signs_and_nan(gpu, stream):
    # dZ = mask * dY keeps -0 and propagates NaN/Inf from dY: check through db,
    # which is the plain column sum of dZ (one row, so no additions change it).
    M, K, Nn = 1, 4, 8
    X = np.ones((M, K), dtype=np.float32)
    W = np.zeros((K, Nn), dtype=np.float32)
    Y = np.array([[-1, 0, 2, np.nan, -1, -1, 3, 1]], dtype=np.float32)
    dY = np.array([[-3, -2, 5, 1, np.inf, np.nan, -0.0, 7]], dtype=np.float32)
    _, _, gb = _run_bwd(stream, X, W, Y, dY, 1, ("db",))
    _, _, rb = O.linear_bwd(X, W, Y, dY, 1)
    same_bits(gb, rb)
    _, _, gb2 = _run_bwd(stream, X, W, Y, dY, 1, ("dW", "db"))
    same_bits(gb2, rb)


# ------------------------------------------------------------- matmul ----
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,K,Nn", [(96, 64, 80), (130, 67, 129), (512, 256, 512), (4096, 64, 2048)])
def test_matmul_transposes(gpu, stream, ta, tb, M, K, Nn):
    # (4096, 64, 2048): grids large enough for the size heuristic's direct
    # fp32 tiles on A.B, A.B^T and A^T.B (A^T.B^T stays register-staged).
    A = ints(61, (K, M) if ta else (M, K))
    B = ints(62, (Nn, K) if tb else (K, Nn))
    C = empty((M, Nn))
    N.matmul(N.F32, ptr(dev(A)), ptr(dev(B)), ptr(C), M, K, Nn, bool(ta), bool(tb), stream)
    same_bits(host(C), O.matmul(A, B, transA=bool(ta), transB=bool(tb)))
    Ar, Br = O.normal(63, A.shape), O.normal(64, B.shape)
    Cr = empty((M, Nn))
    N.matmul(N.F32, ptr(dev(Ar)), ptr(dev(Br)), ptr(Cr), M, K, Nn, bool(ta), bool(tb), stream)
    ref = O.matmul(Ar, Br, transA=bool(ta), transB=bool(tb))
    bound = gemm_bound(Ar.T if ta else Ar, Br.T if tb else Br, K)
    assert_close_gemm(host(Cr), ref, bound, FP32_TOL, what="C")


# --------------------------------------------------------- sum_reduce ----
@pytest.mark.parametrize("M,Nn", [(1, 1), (100, 37), (5000, 300), (8192, 4096), (65536, 8), (20000, 100)])
@pytest.mark.parametrize("axis", [0, 1])
def test_sum_reduce(gpu, stream, M, Nn, axis):
    x = ints(71, (M, Nn), -50, 50)
    out = empty(Nn if axis == 0 else M)
    N.sum_reduce(ptr(dev(x)), ptr(out), M, Nn, axis, stream)
    same_bits(host(out), O.sum_reduce(x, axis))
    xr = O.normal(72, (M, Nn))
    outr = empty(Nn if axis == 0 else M)
    N.sum_reduce(ptr(dev(xr)), ptr(outr), M, Nn, axis, stream)
    ref = O.sum_reduce(xr, axis)
    L = M if axis == 0 else Nn
    bound = 2.02 * L * 2.0 ** -24 * np.abs(xr.astype(np.float64)).sum(axis)
    assert_close_gemm(host(outr), ref, bound, FP32_TOL, what="sum")


# ------------------------------------------------------------------ bf16 ----
# bf16 storage, fp32 accumulation.  The oracle runs on the bf16-rounded
# inputs; Y and dX are rounded once to bf16 (RNE), dW and db stay fp32.
BF16_TOL = 1e-2
BF16_SHAPES = [(128, 256, 128), (256, 512, 384), (512, 1024, 1000), (1024, 1024, 1024), (136, 72, 264), (8, 8, 8),
               (1, 64, 8)]


def _bf16_round(x):
    return O.round_bf16(x)


@pytest.mark.parametrize("M,K,Nn", BF16_SHAPES)
@pytest.mark.parametrize("act", [1, 0])
def test_bf16_integer_bit_exact(gpu, stream, M, K, Nn, act):
    from tests.parity import dev_bf16

    X, W, b, dY = ints(81, (M, K)), ints(82, (K, Nn)), ints(83, Nn), ints(84, (M, Nn))
    Y = empty((M, Nn), dtype=torch.bfloat16)
    N.linear_fwd(N.BF16, ptr(dev_bf16(X)), ptr(dev_bf16(W)), ptr(dev(b)), ptr(Y), M, K, Nn, act, stream)
    rY = _bf16_round(O.linear_fwd(X, W, b, act))
    same_bits(host(Y), rY)
    dX = empty((M, K), dtype=torch.bfloat16)
    dW, db = empty((K, Nn)), empty(Nn)
    N.linear_bwd(N.BF16, ptr(dev_bf16(X)), ptr(dev_bf16(W)), ptr(Y), ptr(dev_bf16(dY)), ptr(dX), ptr(dW), ptr(db),
                 M, K, Nn, act, stream)
    rX, rW, rb = O.linear_bwd(X, W, rY, dY, act)
    same_bits(host(dX), _bf16_round(rX))
    same_bits(host(dW), rW)
    same_bits(host(db), rb)


@pytest.mark.parametrize("tile", ["d256w8", "d256rq", "d256pp", "d128w4", "d128w4s4", "d64w4", "t64x64", "t128x128",
                                  "t256x128", "t256x256"])
def test_every_bf16_tile_bit_exact(gpu, stream, monkeypatch, tile):
    # Each bf16 kernel family forced for the forward and every backward GEMM,
    # on ragged M and N (the 256x256 tiles run 2x2 blocks with partial edges).
    from tests.parity import dev_bf16

    monkeypatch.setenv("C3_HIP_GEMM_TILE_BF16", tile)
    M, K, Nn = 320, 256, 264
    X, W, b, dY = ints(85, (M, K)), ints(86, (K, Nn)), ints(87, Nn), ints(88, (M, Nn))
    Y = empty((M, Nn), dtype=torch.bfloat16)
    N.linear_fwd(N.BF16, ptr(dev_bf16(X)), ptr(dev_bf16(W)), ptr(dev(b)), ptr(Y), M, K, Nn, 1, stream)
    rY = _bf16_round(O.linear_fwd(X, W, b, 1))
    same_bits(host(Y), rY)
    dX = empty((M, K), dtype=torch.bfloat16)
    dW, db = empty((K, Nn)), empty(Nn)
    N.linear_bwd(N.BF16, ptr(dev_bf16(X)), ptr(dev_bf16(W)), ptr(Y), ptr(dev_bf16(dY)), ptr(dX), ptr(dW), ptr(db),
                 M, K, Nn, 1, stream)
    rX, rW, rb = O.linear_bwd(X, W, rY, dY, 1)
    same_bits(host(dX), _bf16_round(rX))
    same_bits(host(dW), rW)
    same_bits(host(db), rb)


@pytest.mark.parametrize("tile", [None, "d256w8", "d128w4", "d128w4s4", "d64w4"])
@pytest.mark.parametrize("M,K,Nn", [(328, 1000, 264), (301, 1000, 264), (200, 72, 136), (264, 40, 8)])
def test_bf16_direct_k_tail_bit_exact(gpu, stream, monkeypatch, tile, M, K, Nn):
    # k extents that are not multiples of the direct kernels' 64-deep k-tile:
    # forward k = K, dX k = N, dW k = M (any M; the others multiples of 8).
    # The last tile loads only its valid chunks and zero-fills the rest.
    from tests.parity import dev_bf16

    if tile:
        monkeypatch.setenv("C3_HIP_GEMM_TILE_BF16", tile)
    X, W, b, dY = ints(91, (M, K)), ints(92, (K, Nn)), ints(93, Nn), ints(94, (M, Nn))
    Y = empty((M, Nn), dtype=torch.bfloat16)
    N.linear_fwd(N.BF16, ptr(dev_bf16(X)), ptr(dev_bf16(W)), ptr(dev(b)), ptr(Y), M, K, Nn, 1, stream)
    rY = _bf16_round(O.linear_fwd(X, W, b, 1))
    same_bits(host(Y), rY)
    dX = empty((M, K), dtype=torch.bfloat16)
    dW, db = empty((K, Nn)), empty(Nn)
    N.linear_bwd(N.BF16, ptr(dev_bf16(X)), ptr(dev_bf16(W)), ptr(Y), ptr(dev_bf16(dY)), ptr(dX), ptr(dW), ptr(db),
                 M, K, Nn, 1, stream)
    rX, rW, rb = O.linear_bwd(X, W, rY, dY, 1)
    same_bits(host(dX), _bf16_round(rX))
    same_bits(host(dW), rW)
    same_bits(host(db), rb)


@pytest.mark.parametrize("M,K,Nn", BF16_SHAPES)
def test_bf16_real(gpu, stream, M, K, Nn):
    from tests.parity import dev_bf16

    X = _bf16_round(O.normal(91, (M, K)))
    W = _bf16_round(O.normal(92, (K, Nn), 0.0, 1.0 / np.sqrt(K)))
    b = O.normal(93, Nn, 0.0, 0.1)
    dY = _bf16_round(O.normal(94, (M, Nn)))
    Y = empty((M, Nn), dtype=torch.bfloat16)
    N.linear_fwd(N.BF16, ptr(dev_bf16(X)), ptr(dev_bf16(W)), ptr(dev(b)), ptr(Y), M, K, Nn, 1, stream)
    t = O.matmul(X, W)
    z = O.bias_act(t, b, 0)
    rY = O.bias_act(t, b, 1)
    gY = host(Y)
    bound = gemm_bound(X, W, K)
    assert_close_gemm(gY, rY, bound, BF16_TOL, out_round=2.0 ** -8, what="Y bf16")
    mask_flips(gY, z, bound + 2.0 ** -8 * np.abs(z))
    # Backward from the GPU's own Y (its mask is what the backward must use).
    dX = empty((M, K), dtype=torch.bfloat16)
    dW, db = empty((K, Nn)), empty(Nn)
    N.linear_bwd(N.BF16, ptr(dev_bf16(X)), ptr(dev_bf16(W)), ptr(Y), ptr(dev_bf16(dY)), ptr(dX), ptr(dW), ptr(db),
                 M, K, Nn, 1, stream)
    rX, rW, rb = O.linear_bwd(X, W, gY, dY, 1)
    dZ = O.relu_mask_mul(gY, dY)
    assert_close_gemm(host(dX), rX, gemm_bound(dZ, W.T, Nn), BF16_TOL, out_round=2.0 ** -8, what="dX bf16")
    assert_close_gemm(host(dW), rW, gemm_bound(X.T, dZ, M), BF16_TOL, what="dW")
    assert_close_gemm(host(db), rb, 2.02 * M * 2.0 ** -24 * np.abs(dZ.astype(np.float64)).sum(0), BF16_TOL,
                      what="db")


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_bf16_matmul_transposes(gpu, stream, ta, tb):
    from tests.parity import dev_bf16

    M, K, Nn = 136, 200, 264
    A = ints(95, (K, M) if ta else (M, K))
    B = ints(96, (Nn, K) if tb else (K, Nn))
    C = empty((M, Nn), dtype=torch.bfloat16)
    N.matmul(N.BF16, ptr(dev_bf16(A)), ptr(dev_bf16(B)), ptr(C), M, K, Nn, bool(ta), bool(tb), stream)
    same_bits(host(C), _bf16_round(O.matmul(A, B, transA=bool(ta), transB=bool(tb))))


def test_bf16_rejects_unaligned_extents(gpu, stream):
    from tests.parity import dev_bf16

    X, W = dev_bf16(np.ones((16, 12), np.float32)), dev_bf16(np.ones((12, 16), np.float32))
    Y = empty((16, 16), dtype=torch.bfloat16)
    with pytest.raises(N.C3HipError) as ei:
        N.linear_fwd(N.BF16, ptr(X), ptr(W), None, ptr(Y), 16, 12, 16, 1, stream)
    assert ei.value.code == N.ERR_UNSUPPORTED


def test_forced_tile_override(gpu, stream):
    # The calling thread's tile override (c3hip_set_gemm_tile): results are
    # the oracle's bit for bit under every tile; a direct tile on a problem it
    # cannot run is refused, not silently replaced; clearing restores the
    # heuristic.
    from tests.parity import dev_bf16

    M, K, Nn = 300, 264, 200
    X, W, b = ints(95, (M, K)), ints(96, (K, Nn)), ints(97, Nn)
    rY = O.linear_fwd(X, W, b, 1)
    try:
        for tile in N.gemm_tile_names(N.F32):
            N.set_gemm_tile(N.F32, tile)
            Y = empty((M, Nn))
            N.linear_fwd(N.F32, ptr(dev(X)), ptr(dev(W)), ptr(dev(b)), ptr(Y), M, K, Nn, 1, stream)
            same_bits(host(Y), rY)
        for tile in N.gemm_tile_names(N.BF16):
            N.set_gemm_tile(N.BF16, tile)
            Y = empty((M, Nn), dtype=torch.bfloat16)
            args = (N.BF16, ptr(dev_bf16(X)), ptr(dev_bf16(W)), ptr(dev(b)), ptr(Y), M, K, Nn, 1, stream)
            # K = 264 is not a multiple of the direct tiles' 32/64-deep k tile: those
            # with a partial last k-tile run it, the others refuse it.
            if tile.startswith("d") and tile not in ("d256w8", "d128w4", "d128w4s4", "d64w4"):
                with pytest.raises(N.C3HipError) as e:
                    N.linear_fwd(*args)
                assert e.value.code == N.ERR_UNSUPPORTED
                continue
            N.linear_fwd(*args)
            same_bits(host(Y), _bf16_round(rY))
    finally:
        N.set_gemm_tile(N.F32, None)
        N.set_gemm_tile(N.BF16, None)
    Y = empty((M, Nn), dtype=torch.bfloat16)
    N.linear_fwd(N.BF16, ptr(dev_bf16(X)), ptr(dev_bf16(W)), ptr(dev(b)), ptr(Y), M, K, Nn, 1, stream)
    same_bits(host(Y), _bf16_round(rY))


@pytest.mark.parametrize("K", [32, 64, 96, 160])
def test_bf16_pingpong_short_k_bit_exact(gpu, stream, monkeypatch, K):
    # The ping-pong tile keeps up to four 32-deep k tiles in flight; K of one to
    # five tiles covers the prologue and drain paths (fewer tiles than stages).
    from tests.parity import dev_bf16

    monkeypatch.setenv("C3_HIP_GEMM_TILE_BF16", "d256pp")
    M, Nn = 264, 520
    X, W, b, dY = ints(95, (M, K)), ints(96, (K, Nn)), ints(97, Nn), ints(98, (M, Nn))
    Y = empty((M, Nn), dtype=torch.bfloat16)
    N.linear_fwd(N.BF16, ptr(dev_bf16(X)), ptr(dev_bf16(W)), ptr(dev(b)), ptr(Y), M, K, Nn, 1, stream)
    rY = _bf16_round(O.linear_fwd(X, W, b, 1))
    same_bits(host(Y), rY)
    dX = empty((M, K), dtype=torch.bfloat16)
    dW, db = empty((K, Nn)), empty(Nn)
    N.linear_bwd(N.BF16, ptr(dev_bf16(X)), ptr(dev_bf16(W)), ptr(Y), ptr(dev_bf16(dY)), ptr(dX), ptr(dW), ptr(db),
                 M, K, Nn, 1, stream)
    rX, rW, rb = O.linear_bwd(X, W, rY, dY, 1)
    same_bits(host(dX), _bf16_round(rX))
    same_bits(host(dW), rW)
    same_bits(host(db), rb)


# Split-K: a GEMM with fewer than 64 output tiles of 256x256 and a long k
# range runs as k splits with fp32 partials added by c3_splitk_reduce.  Each
# shape splits one GEMM of the layer: (576, 8192, 576) the forward,
# (576, 576, 8192) dX (k = N), (8192, 576, 576) dW (k = M); 576 = 9 x 64, so
# every forced direct tile runs all three GEMMs.
@pytest.mark.parametrize("tile", [None, "d256w8", "d256rq", "d256pp", "d128w4", "d128w4s4", "d64w4"])
@pytest.mark.parametrize("M,K,Nn", [(576, 8192, 576), (576, 576, 8192), (8192, 576, 576)])
def test_bf16_split_k_bit_exact(gpu, stream, monkeypatch, tile, M, K, Nn):
    from tests.parity import dev_bf16

    if tile is None:
        monkeypatch.delenv("C3_HIP_GEMM_TILE_BF16", raising=False)
    else:
        monkeypatch.setenv("C3_HIP_GEMM_TILE_BF16", tile)
    X, W, b, dY = ints(101, (M, K)), ints(102, (K, Nn)), ints(103, Nn), ints(104, (M, Nn))
    Y = empty((M, Nn), dtype=torch.bfloat16)
    N.linear_fwd(N.BF16, ptr(dev_bf16(X)), ptr(dev_bf16(W)), ptr(dev(b)), ptr(Y), M, K, Nn, 1, stream)
    # Integer-valued inputs: every partial sum is an integer below 2^24, so
    # float64 products in any order are exact and equal the oracle's
    # sequential loop (checked against it in test_oracle); this keeps the
    # reference fast at k = 8192.
    X64, W64, dY64 = X.astype(np.float64), W.astype(np.float64), dY.astype(np.float64)
    rY = _bf16_round(np.maximum(X64 @ W64 + b, 0.0).astype(np.float32))
    same_bits(host(Y), rY)
    dX = empty((M, K), dtype=torch.bfloat16)
    dW, db = empty((K, Nn)), empty(Nn)
    N.linear_bwd(N.BF16, ptr(dev_bf16(X)), ptr(dev_bf16(W)), ptr(Y), ptr(dev_bf16(dY)), ptr(dX), ptr(dW), ptr(db),
                 M, K, Nn, 1, stream)
    dZ = np.where(rY > 0, dY64, 0.0)
    same_bits(host(dX), _bf16_round((dZ @ W64.T).astype(np.float32)))
    same_bits(host(dW), (X64.T @ dZ).astype(np.float32))
    same_bits(host(db), dZ.sum(axis=0).astype(np.float32))


# The bf16 layer backward after its pre-pass runs dX, dW and the bias
# gradient's final pass in one launch (c3_gemm_bf16_bwd_<dX tile>[_<dW tile>])
# where the size heuristic puts both GEMMs on direct tiles without a split.
# A forced tile turns the one-launch path off: the separate dX, dW and
# column-sum launches on it (no split on these shapes either) must give the
# same bits on real-valued inputs (every direct tile adds k in the same
# order).  One shape per one-launch kernel, with each activation's pre-pass
# on the smallest, partial last k-tiles in dX (k = N = 1000) and dW
# (k = M = 1000), and shapes whose dX and dW the heuristic alone would put
# on different 128x128 / 256x256 tiles or both on d128w4s4 (both run on
# d128w4 instead; 2048^3 compares against separate d128w4s4 launches).
@pytest.mark.parametrize("M,K,Nn,pair,tile,act", [
    (1000, 1016, 1024, "d64w4", "d64w4", 1), (1000, 1016, 1024, "d64w4", "d64w4", 2),
    (1000, 1016, 1024, "d64w4", "d64w4", 3), (1000, 1016, 1024, "d64w4", "d64w4", 0),
    (1024, 4096, 1024, "d128w4", "d128w4", 1), (2048, 2048, 2048, "d128w4", "d128w4s4", 1),
    (4096, 4096, 4096, "d256w8", "d256w8", 1), (1024, 1024, 4096, "d64w4_d128w4", "d64w4", 1),
    (4096, 1024, 1024, "d128w4_d64w4", "d64w4", 1), (1024, 1024, 1000, "d64w4", "d64w4", 1),
    (1000, 1016, 1000, "d64w4", "d64w4", 3), (1024, 4096, 4096, "d128w4", "d128w4", 1),
    (4096, 1024, 8192, "d128w4", "d128w4", 1)])
def test_bf16_layer_backward_one_launch_matches_separate(gpu, stream, M, K, Nn, pair, tile, act):
    from tests.parity import dev_bf16

    rng = np.random.default_rng(M + K + Nn)
    X = dev_bf16(rng.standard_normal((M, K), dtype=np.float32))
    W = dev_bf16(rng.standard_normal((K, Nn), dtype=np.float32) / np.float32(np.sqrt(K)))
    Y = dev_bf16(rng.standard_normal((M, Nn), dtype=np.float32))
    dY = dev_bf16(rng.standard_normal((M, Nn), dtype=np.float32))

    def bwd():
        dX = empty((M, K), dtype=torch.bfloat16)
        dW, db = empty((K, Nn)), empty(Nn)
        N.set_launch_timing(True)
        try:
            N.linear_bwd(N.BF16, ptr(X), ptr(W), ptr(Y), ptr(dY), ptr(dX), ptr(dW), ptr(db), M, K, Nn, act, stream)
            names = [n for n, _ in N.launch_timings()]
        finally:
            N.set_launch_timing(False)
        return [host(dX), host(dW), host(db)], names

    one, names = bwd()
    assert names == ["c3_dz_colsum_bf16", f"c3_gemm_bf16_bwd_{pair}"], names
    N.set_gemm_tile(N.BF16, tile)
    try:
        sep, names = bwd()
    finally:
        N.set_gemm_tile(N.BF16, None)
    assert names == ["c3_dz_colsum_bf16", "c3_colsum_final_f32", f"c3_gemm_bf16_dx_{tile}",
                     f"c3_gemm_bf16_dw_{tile}"], names
    for got, ref in zip(one, sep):
        same_bits(got, ref)


def test_bf16_layer_backward_mixed_tiles_beyond_the_pair_bound_stay_separate(gpu, stream):
    # dX on 128x128 tiles (512) and dW on 256x256 tiles (2048): on 128x128
    # tiles the pair would be 8704 blocks, past the 4608 the one-launch rule
    # takes, so the GEMMs run as separate launches on their own tiles.
    M, K, Nn = 1024, 8192, 16384
    X, W = empty((M, K), dtype=torch.bfloat16, fill=0.0), empty((K, Nn), dtype=torch.bfloat16, fill=0.0)
    Y, dY = empty((M, Nn), dtype=torch.bfloat16, fill=0.0), empty((M, Nn), dtype=torch.bfloat16, fill=0.0)
    dX = empty((M, K), dtype=torch.bfloat16)
    dW, db = empty((K, Nn)), empty(Nn)
    N.set_launch_timing(True)
    try:
        N.linear_bwd(N.BF16, ptr(X), ptr(W), ptr(Y), ptr(dY), ptr(dX), ptr(dW), ptr(db), M, K, Nn, 1, stream)
        names = [n for n, _ in N.launch_timings()]
    finally:
        N.set_launch_timing(False)
    assert "c3_gemm_bf16_dx_d128w4" in names and "c3_gemm_bf16_dw_d256w8" in names, names
    assert not any(n.startswith("c3_gemm_bf16_bwd_") for n in names), names
    assert not host(dW).any() and not host(db).any()


def test_bf16_split_k_real_values(gpu, stream):
    # Real-valued inputs through the split forward and split dW: the split
    # order differs from the sequential k loop only by rounding.
    from tests.parity import dev_bf16

    M, K, Nn = 576, 8192, 576
    X = _bf16_round(O.normal(111, (M, K)))
    W = _bf16_round(O.normal(112, (K, Nn), 0.0, 1.0 / np.sqrt(K)))
    b = O.normal(113, Nn, 0.0, 0.1)
    Y = empty((M, Nn), dtype=torch.bfloat16)
    N.linear_fwd(N.BF16, ptr(dev_bf16(X)), ptr(dev_bf16(W)), ptr(dev(b)), ptr(Y), M, K, Nn, 1, stream)
    t = O.matmul(X, W)
    rY = O.bias_act(t, b, 1)
    z = O.bias_act(t, b, 0)
    gY = host(Y)
    bound = gemm_bound(X, W, K)
    assert_close_gemm(gY, rY, bound, BF16_TOL, out_round=2.0 ** -8, what="Y bf16 split")
    mask_flips(gY, z, bound + 2.0 ** -8 * np.abs(z))


# Transposed-W forward (bf16, opt-in with C3_HIP_BF16_WT=1): W is transposed
# into a workspace and the GEMM reads both operands k-contiguous.  Same tile,
# split and k order as the plain forward, so the same bits: integer inputs
# against the exact product, real inputs against the plain path bit for bit.
# Shapes: a 256x256-tile forward, a split-K forward, a 128x128-tile forward.
@pytest.mark.parametrize("M,K,Nn", [(4096, 256, 264), (576, 8192, 576), (1000, 512, 1024)])
def test_bf16_fwd_transposed_w(gpu, stream, monkeypatch, M, K, Nn):
    from tests.parity import dev_bf16

    X, W, b = ints(121, (M, K)), ints(122, (K, Nn)), ints(123, Nn)
    want = _bf16_round(np.maximum(X.astype(np.float64) @ W.astype(np.float64) + b, 0.0).astype(np.float32))
    Xr = _bf16_round(O.normal(124, (M, K)))
    Wr = _bf16_round(O.normal(125, (K, Nn), 0.0, 1.0 / np.sqrt(K)))
    br = O.normal(126, Nn, 0.0, 0.1)
    outs = {}
    for mode in ("1", "0", None):
        if mode is None:
            monkeypatch.delenv("C3_HIP_BF16_WT", raising=False)
        else:
            monkeypatch.setenv("C3_HIP_BF16_WT", mode)
        Y = empty((M, Nn), dtype=torch.bfloat16)
        N.linear_fwd(N.BF16, ptr(dev_bf16(X)), ptr(dev_bf16(W)), ptr(dev(b)), ptr(Y), M, K, Nn, 1, stream)
        same_bits(host(Y), want)
        Yr = empty((M, Nn), dtype=torch.bfloat16)
        N.linear_fwd(N.BF16, ptr(dev_bf16(Xr)), ptr(dev_bf16(Wr)), ptr(dev(br)), ptr(Yr), M, K, Nn, 1, stream)
        outs[mode] = host(Yr)
    same_bits(outs["1"], outs["0"])
    same_bits(outs[None], outs["0"])


# fp32 split-K: the 64x64 kernel on fewer than 32 tiles over K >= 512 runs as
# 16-aligned k splits whose fp32 partials c3_splitk_reduce adds (with the bias
# and activation).  (128, 784, 256): the forward splits (a train step's first
# layer); (128, 256, 784): the masked dX splits (k = N = 784) while dW keeps
# its db side output and does not.
@pytest.mark.parametrize("M,K,Nn", [(128, 784, 256), (128, 256, 784), (70, 1000, 90)])
def test_f32_split_k_bit_exact(gpu, stream, M, K, Nn):
    X, W, b = ints(131, (M, K)), ints(132, (K, Nn)), ints(133, Nn)
    Y = empty((M, Nn))
    N.linear_fwd(N.F32, ptr(dev(X)), ptr(dev(W)), ptr(dev(b)), ptr(Y), M, K, Nn, 1, stream)
    rY = O.linear_fwd(X, W, b, 1)
    same_bits(host(Y), rY)
    dY = ints(134, (M, Nn))
    gX, gW, gb = _run_bwd(stream, X, W, rY, dY, 1)
    rX, rW, rb = O.linear_bwd(X, W, rY, dY, 1)
    same_bits(gX, rX)
    same_bits(gW, rW)
    same_bits(gb, rb)


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_f32_split_k_matmul_transposes(gpu, stream, ta, tb):
    M, K, Nn = 96, 1000, 80
    A = ints(141, (K, M) if ta else (M, K))
    B = ints(142, (Nn, K) if tb else (K, Nn))
    C = empty((M, Nn))
    N.matmul(N.F32, ptr(dev(A)), ptr(dev(B)), ptr(C), M, K, Nn, bool(ta), bool(tb), stream)
    same_bits(host(C), O.matmul(A, B, transA=bool(ta), transB=bool(tb)))


@pytest.mark.parametrize("act", [1, 2])
def test_f32_split_k_real(gpu, stream, act):
    M, K, Nn = 128, 784, 256
    X = O.normal(151, (M, K))
    W = O.normal(152, (K, Nn), 0.0, 1.0 / np.sqrt(K))
    b = O.normal(153, Nn, 0.0, 0.1)
    Y = empty((M, Nn))
    N.linear_fwd(N.F32, ptr(dev(X)), ptr(dev(W)), ptr(dev(b)), ptr(Y), M, K, Nn, act, stream)
    t = O.matmul(X, W)
    ref = O.bias_act(t, b, act)
    # ReLU: the GEMM bound; sigmoid is 1/4-Lipschitz and adds a few ulp.
    bound = gemm_bound(X, W, K) + (8.0 * 2.0 ** -24 if act == 2 else 0.0)
    assert_close_gemm(host(Y), ref, bound, FP32_TOL, out_round=(4.0 * 2.0 ** -24 if act == 2 else 0.0), what="Y split")
