"""GPU parity of the transcendental ops (sigmoid, tanh, exp, log and the
single-input backward ops), the three-input Div gradient, and the sigmoid /
tanh activations of the fused Linear layer, through the C ABI against the
oracle.

exp, log and tanh are the device library's on the GPU and libm's in the
oracle; each is within an ulp or two of the exact value, so the two agree to
a few ulp of the result (per-op bounds below, u = 2^-23 relative spacing):
  exp, log:            3 ulp(ref)            tanh:     4 ulp(ref)
  sigmoid:             5 ulp(ref)            exp_bwd:  4 ulp(ref)
  sigmoid_bwd:  16 u |grad| + 4 ulp(ref)     (1 - s cancels near s = 1)
  tanh_bwd:     32 u |grad| + 4 ulp(ref)     (e^x - e^-x cancels near 0)
plus the normwise rel-err 1e-5; NaN and infinity positions must agree, and
the three-input op (IEEE operations only) is bit-exact.
"""
import numpy as np
import pytest
import torch

from c3_amd import native as N
from oracle import oracle as O
from tests.parity import U, assert_close_gemm, dev, dev_bf16, empty, gemm_bound, host, ptr

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5
E = 2.0 ** -23


def ulp(x):
    x = np.abs(np.asarray(x, np.float64))
    return np.maximum(np.spacing(x.astype(np.float32)).astype(np.float64), np.finfo(np.float32).tiny)


def specials_agree(got, ref):
    gn, rn = np.isnan(got), np.isnan(ref)
    assert np.array_equal(gn, rn), f"NaN positions differ ({int((gn != rn).sum())})"
    gi, ri = np.isinf(got), np.isinf(ref)
    assert np.array_equal(gi, ri) and np.array_equal(got[gi], ref[ri]), "infinities differ"
    return ~(gn | gi)


BOUNDS = {
    "exp": lambda ref, g: 3 * ulp(ref),
    "log": lambda ref, g: 3 * ulp(ref),
    "tanh": lambda ref, g: 4 * ulp(ref),
    "sigmoid": lambda ref, g: 5 * ulp(ref),
    "exp_bwd": lambda ref, g: 4 * ulp(ref),
    "sigmoid_bwd": lambda ref, g: 16 * E * np.abs(g) + 4 * ulp(ref),
    "tanh_bwd": lambda ref, g: 32 * E * np.abs(g) + 4 * ulp(ref),
}

SPECIALS = np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan, 1e-40, -1e-40, 88.0, -88.0, 89.0, -89.0,
                     100.0, -100.0, 1e-6, -1e-6, 20.0], dtype=np.float32)


@pytest.mark.parametrize("op", list(N.EW_MATH_OPS))
@pytest.mark.parametrize("n", [1 << 18, 1001])
def test_math_ops_against_oracle(gpu, stream, op, n):
    code = N.EW_MATH_OPS[op]
    a = O.normal(600 + code, n, 0.0, 4.0)
    if op == "log":
        a = np.abs(a) + np.float32(1e-3)
    a[: len(SPECIALS)] = SPECIALS[: min(n, len(SPECIALS))]
    g = O.normal(700 + code, n, 0.0, 2.0)
    binary = code in O.EW_BINARY
    out = empty(n)
    N.elementwise(code, N.F32, ptr(dev(a)), ptr(dev(g)) if binary else None, 0.0, ptr(out), n, 0, stream)
    with np.errstate(all="ignore"):
        ref = O.elementwise(code, a, g if binary else None)
    got = host(out)
    fin = specials_agree(got, ref)
    err = np.abs(got[fin].astype(np.float64) - ref[fin])
    bound = BOUNDS[op](ref[fin].astype(np.float64), g[fin].astype(np.float64))
    assert np.all(err <= bound), f"{op}: {int((err > bound).sum())} elements beyond the bound, worst excess " \
                                 f"{float(np.max(err - bound)):.3e}"
    assert np.max(err) <= FP32_TOL * np.max(np.abs(ref[fin]))


def test_math_closed_forms_on_gpu(gpu, stream):
    z = dev(np.zeros(4, np.float32))
    g = dev(np.full(4, 3.0, np.float32))
    for code, want in [(N.EW_SIGMOID, 0.5), (N.EW_EXP, 1.0), (N.EW_TANH, 0.0), (N.EW_SIGMOID_BWD, 0.75),
                       (N.EW_TANH_BWD, 3.0), (N.EW_EXP_BWD, 3.0)]:
        out = empty(4)
        N.elementwise(code, N.F32, ptr(z), ptr(g), 0.0, ptr(out), 4, 0, stream)
        assert np.all(host(out) == np.float32(want)), code
    out = empty(4)
    N.elementwise(N.EW_LOG, N.F32, ptr(dev(np.ones(4, np.float32))), None, 0.0, ptr(out), 4, 0, stream)
    assert np.all(host(out) == 0.0)


@pytest.mark.parametrize("n", [1 << 20, 37])
def test_div_backward_divisor_bit_exact(gpu, stream, n):
    a = O.normal(610, n)
    b = O.uniform(611, n, 0.5, 2.0)
    c = O.normal(612, n)
    a[:4] = [0.0, -0.0, np.inf, 1.0]
    b[:4] = [1.0, 2.0, 3.0, 0.0]
    out = empty(n)
    N.elementwise3(N.EW3_DIV_BWD_B, N.F32, ptr(dev(a)), ptr(dev(b)), ptr(dev(c)), ptr(out), n, stream)
    with np.errstate(all="ignore"):
        ref = O.elementwise3(O.EW3_DIV_BWD_B, a, b, c)
    got = host(out)
    fin = specials_agree(got, ref)
    assert np.array_equal(got[fin].view(np.int32), ref[fin].view(np.int32))


# ------------------------------------------------ sigmoid / tanh layers ----
ACT_FWD_ULP = {N.ACT_SIGMOID: 5, N.ACT_TANH: 4}
ACT_SLOPE = {N.ACT_SIGMOID: 0.25, N.ACT_TANH: 1.0}   # max |f'|


def ints(seed, shape, lo=-2, hi=2):
    return np.random.default_rng(seed).integers(lo, hi + 1, size=shape).astype(np.float32)


@pytest.mark.parametrize("act", [N.ACT_SIGMOID, N.ACT_TANH])
@pytest.mark.parametrize("M,K,Nn", [(128, 784, 256), (130, 129, 131), (1024, 512, 768)])
def test_linear_sigmoid_tanh_fp32(gpu, stream, act, M, K, Nn):
    # Forward: integer inputs make z exact, so only the activation differs.
    X, W, b = ints(620, (M, K)), ints(621, (K, Nn)), ints(622, Nn)
    Y = empty((M, Nn))
    N.linear_fwd(N.F32, ptr(dev(X)), ptr(dev(W)), ptr(dev(b)), ptr(Y), M, K, Nn, act, stream)
    rY = O.linear_fwd(X, W, b, act)
    got = host(Y)
    assert np.all(np.abs(got.astype(np.float64) - rY) <= ACT_FWD_ULP[act] * ulp(rY))
    # Real inputs: z differs by the GEMM bound, Y by slope x bound + ulps.
    Xr = O.normal(623, (M, K))
    Wr = O.normal(624, (K, Nn), 0.0, 1.0 / np.sqrt(K))
    br = O.normal(625, Nn, 0.0, 0.1)
    Yr = empty((M, Nn))
    N.linear_fwd(N.F32, ptr(dev(Xr)), ptr(dev(Wr)), ptr(dev(br)), ptr(Yr), M, K, Nn, act, stream)
    rYr = O.linear_fwd(Xr, Wr, br, act)
    bound = ACT_SLOPE[act] * gemm_bound(Xr, Wr, K) + ACT_FWD_ULP[act] * ulp(rYr)
    assert_close_gemm(host(Yr), rYr, bound, FP32_TOL, what="Y")
    # Backward from the oracle's Y: dZ = dY * f'(Y) is formed with the same IEEE
    # operations on both sides, so only the GEMM and column-sum orders differ.
    dY = O.normal(626, (M, Nn))
    dX, dW, db = empty((M, K)), empty((K, Nn)), empty(Nn)
    N.linear_bwd(N.F32, ptr(dev(Xr)), ptr(dev(Wr)), ptr(dev(rYr)), ptr(dev(dY)), ptr(dX), ptr(dW), ptr(db),
                 M, K, Nn, act, stream)
    rX, rW, rb = O.linear_bwd(Xr, Wr, rYr, dY, act)
    dZ = O.act_grad(rYr, dY, act)
    assert_close_gemm(host(dX), rX, gemm_bound(dZ, Wr.T, Nn), FP32_TOL, what="dX")
    assert_close_gemm(host(dW), rW, gemm_bound(Xr.T, dZ, M), FP32_TOL, what="dW")
    assert_close_gemm(host(db), rb, 2.02 * M * U * np.abs(dZ.astype(np.float64)).sum(0), FP32_TOL, what="db")


# tile: the size heuristic's kernels, or a forced direct tile, whose forward
# stores whole tiles through LDS (the sigmoid and tanh epilogues on that path).
@pytest.mark.parametrize("tile", [None, "d256w8", "d128w4s4"])
@pytest.mark.parametrize("act", [N.ACT_SIGMOID, N.ACT_TANH])
def test_linear_sigmoid_tanh_bf16(gpu, stream, monkeypatch, act, tile):
    if tile:
        monkeypatch.setenv("C3_HIP_GEMM_TILE_BF16", tile)
    M, K, Nn = 512, 256, 264
    X = O.round_bf16(O.normal(630, (M, K)))
    W = O.round_bf16(O.normal(631, (K, Nn), 0.0, 1.0 / np.sqrt(K)))
    b = O.normal(632, Nn, 0.0, 0.1)
    Y = empty((M, Nn), dtype=torch.bfloat16)
    N.linear_fwd(N.BF16, ptr(dev_bf16(X)), ptr(dev_bf16(W)), ptr(dev(b)), ptr(Y), M, K, Nn, act, stream)
    rY = O.linear_fwd(X, W, b, act)
    bound = ACT_SLOPE[act] * gemm_bound(X, W, K) + ACT_FWD_ULP[act] * ulp(rY)
    assert_close_gemm(host(Y), rY, bound, 1e-2, out_round=2.0 ** -8, what="Y bf16")
    # Backward from the GPU's own bf16 Y: the pre-pass rounds dZ = dY * f'(Y)
    # to bf16 once; the oracle does the same, then the GEMMs differ in order only.
    Yb = host(Y)
    dY = O.round_bf16(O.normal(633, (M, Nn)))
    dX = empty((M, K), dtype=torch.bfloat16)
    dW, db = empty((K, Nn)), empty(Nn)
    N.linear_bwd(N.BF16, ptr(dev_bf16(X)), ptr(dev_bf16(W)), ptr(Y), ptr(dev_bf16(dY)), ptr(dX), ptr(dW), ptr(db),
                 M, K, Nn, act, stream)
    dZ = O.round_bf16(O.act_grad(Yb, dY, act))
    rX = O.matmul(dZ, W, transB=True)
    rW = O.matmul(X, dZ, transA=True)
    rb = O.sum_reduce(dZ, axis=0)
    assert_close_gemm(host(dX), rX, gemm_bound(dZ, W.T, Nn), 1e-2, out_round=2.0 ** -8, what="dX bf16")
    assert_close_gemm(host(dW), rW, gemm_bound(X.T, dZ, M), 1e-2, what="dW bf16")
    assert_close_gemm(host(db), rb, 2.02 * M * U * np.abs(dZ.astype(np.float64)).sum(0), 1e-2, what="db bf16")


@pytest.mark.parametrize("act", [N.ACT_SIGMOID, N.ACT_TANH])
def test_linear_act_backward_against_reference_composition(gpu, stream, act):
    """The fused backward (derivative from the saved output Y) against the
    reference's per-node composition from the pre-activation Z
    (oracle.linear_bwd_from_preact: the activation node's rule recomputed
    from Z through exp, then MatMul and Add backward).  Sigmoid: the same dZ
    bits, so only the GEMM orders differ.  Tanh: dZ differs by at most 16 ulp
    of |dY| (+ 4 ulp) while |z| <= 88, which adds |dZ err| . |W| to the bound."""
    M, K, Nn = 256, 192, 320
    X = O.normal(640, (M, K))
    W = O.normal(641, (K, Nn), 0.0, 2.0 / np.sqrt(K))
    b = O.normal(642, Nn, 0.0, 0.5)
    dY = O.normal(643, (M, Nn))
    Y = empty((M, Nn))
    N.linear_fwd(N.F32, ptr(dev(X)), ptr(dev(W)), ptr(dev(b)), ptr(Y), M, K, Nn, act, stream)
    gY = host(Y)
    dX, dW, db = empty((M, K)), empty((K, Nn)), empty(Nn)
    N.linear_bwd(N.F32, ptr(dev(X)), ptr(dev(W)), ptr(Y), ptr(dev(dY)), ptr(dX), ptr(dW), ptr(db), M, K, Nn, act,
                 stream)
    Z = O.bias_act(O.matmul(X, W), b, act=0)
    assert np.max(np.abs(Z)) <= 88.0
    rX, rW, rb = O.linear_bwd_from_preact(X, W, Z, dY, act)
    dZ = O.act_grad(gY, dY, act)
    dz_err = np.abs(dY).astype(np.float64) * 16 * 2.0 ** -23 + 4 * ulp(dZ) if act == N.ACT_TANH else 0.0 * dZ
    # The GPU's Y differs from tanhf/sigmoid of the oracle's Z by the GEMM bound x slope + a few ulp.
    y_err = ACT_SLOPE[act] * gemm_bound(X, W, K) + ACT_FWD_ULP[act] * ulp(gY)
    dz_err = dz_err + 2.0 * np.abs(dY).astype(np.float64) * y_err
    assert_close_gemm(host(dX), rX, gemm_bound(dZ, W.T, Nn) + dz_err @ np.abs(W.T.astype(np.float64)), FP32_TOL,
                      what="dX")
    assert_close_gemm(host(dW), rW, gemm_bound(X.T, dZ, M) + np.abs(X.T.astype(np.float64)) @ dz_err, FP32_TOL,
                      what="dW")
    assert_close_gemm(host(db), rb, 2.02 * M * U * np.abs(dZ.astype(np.float64)).sum(0) + dz_err.sum(0), FP32_TOL,
                      what="db")
