"""Pins the oracle (oracle/c3_oracle.c) before it is trusted as the checker.

The reference ships no golden vectors for this path (its tests live in the
host framework and are not in the repository), so each oracle function is
pinned by what the mathematics fixes: published known answers, integer
inputs whose sums are exact in fp32, float64 brute force with the standard
error bound, and hand-built cases whose result changes if the summation
order, the FMA contraction, the bias placement or a sign/mask rule changes.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O

U = 2.0 ** -24  # unit roundoff of fp32


def f32(x):
    return np.float32(x)


# ---------------------------------------------------------------- inputs ----
def test_splitmix64_published_sequence():
    # Published SplitMix64 outputs for seed 1234567 (Vigna's splitmix64.c).
    import ctypes

    lib = O.lib()
    lib.oracle_splitmix64_next.restype = ctypes.c_uint64
    lib.oracle_splitmix64_next.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
    s = ctypes.c_uint64(1234567)
    got = [lib.oracle_splitmix64_next(ctypes.byref(s)) for _ in range(5)]
    assert got == [6457827717110365317, 3203168211198807973, 9817491932198370423, 4593380528125082431,
                   16408922859458223821]


def test_fill_distributions():
    x = O.normal(7, 1 << 16)
    assert abs(x.mean()) < 0.02 and abs(x.std() - 1.0) < 0.02
    u = O.uniform(7, 1 << 16, 0.5, 2.0)
    assert u.min() >= 0.5 and u.max() < 2.0 and abs(u.mean() - 1.25) < 0.01
    lb = O.labels(3, 10000, 10)
    assert lb.min() == 0 and lb.max() == 9 and len(np.unique(lb)) == 10
    # Reproducible from the seed.
    assert np.array_equal(O.normal(11, 1001), O.normal(11, 1001))


# ------------------------------------------------------------------ bf16 ----
def test_bf16_round_known_answers():
    one = 1.0
    cases = {
        one: one,
        one + 2.0 ** -8: one,                     # tie -> even (mantissa 0)
        one + 3 * 2.0 ** -8: one + 2.0 ** -6,     # tie -> even (rounds up)
        one + 2.0 ** -8 + 2.0 ** -20: one + 2.0 ** -7,  # above the tie
        -2.5: -2.5,
        65504.0: 65536.0,
    }
    xs = np.array(list(cases), dtype=np.float32)
    assert np.array_equal(O.round_bf16(xs), np.array(list(cases.values()), dtype=np.float32))
    r = O.round_bf16(np.array([np.inf, -np.inf, np.nan], dtype=np.float32))
    assert r[0] == np.inf and r[1] == -np.inf and np.isnan(r[2])


def test_bf16_round_is_nearest():
    x = O.normal(5, 4096, 0.0, 100.0)
    r = O.round_bf16(x).astype(np.float64)
    bits = O.pack_bf16(x)
    assert np.array_equal(O.bf16_bits_to_f32(bits), r.astype(np.float32))
    # Neighbouring bf16 values (one bf16 ulp away) are never closer.
    up = O.bf16_bits_to_f32((bits.astype(np.int32) + 1).astype(np.uint16)).astype(np.float64)
    dn = O.bf16_bits_to_f32((bits.astype(np.int32) - 1).astype(np.uint16)).astype(np.float64)
    xd = x.astype(np.float64)
    assert np.all(np.abs(xd - r) <= np.abs(xd - up)) and np.all(np.abs(xd - r) <= np.abs(xd - dn))


# -------------------------------------------------------------- maxnum ----
def test_maxnum_semantics():
    assert O.maxnum(float("nan"), 0.0) == 0.0
    assert O.maxnum(0.0, float("nan")) == 0.0
    assert O.maxnum(-1.5, 0.0) == 0.0
    assert O.maxnum(2.5, 0.0) == 2.5
    assert math.copysign(1.0, O.maxnum(-0.0, 0.0)) == 1.0  # relu(-0) = +0 in this restatement


# -------------------------------------------------------------- matmul ----
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_matmul_integer_exact(ta, tb):
    rng = np.random.default_rng(1)
    M, K, N = 37, 53, 29
    A = rng.integers(-3, 4, size=(K, M) if ta else (M, K)).astype(np.float32)
    B = rng.integers(-3, 4, size=(N, K) if tb else (K, N)).astype(np.float32)
    ref = (A.T if ta else A).astype(np.int64) @ (B.T if tb else B).astype(np.int64)
    got = O.matmul(A, B, transA=bool(ta), transB=bool(tb))
    assert np.array_equal(got, ref.astype(np.float32))


def test_matmul_float64_error_bound():
    M, K, N = 24, 300, 19
    A = O.normal(21, (M, K))
    B = O.normal(22, (K, N), 0.0, 0.05)
    got = O.matmul(A, B).astype(np.float64)
    exact = A.astype(np.float64) @ B.astype(np.float64)
    bound = 1.01 * K * U * (np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64))
    assert np.all(np.abs(got - exact) <= bound)


def test_matmul_sequential_k_order():
    # Sequential sum from 0.0: ((2^24 + 1) + 1) - 2^24 = 0 in fp32 (each +1 is
    # a tie that rounds back to 2^24).  Pairwise or reordered sums give 1 or 2.
    A = np.array([[2.0 ** 24, 1.0, 1.0, -(2.0 ** 24)]], dtype=np.float32)
    B = np.ones((4, 1), dtype=np.float32)
    assert O.matmul(A, B)[0, 0] == 0.0
    # Reversed k order gives a different value, so the test sees the order.
    assert O.matmul(A[:, ::-1], B)[0, 0] == 2.0


def test_matmul_no_fma_contraction():
    # k0 product: -(1 + 2^-11) exactly; k1 product (1 + 2^-12)^2 = 1 + 2^-11 + 2^-24
    # rounds to 1 + 2^-11 on its own, so the sum is 0.  An FMA would keep 2^-24.
    a1 = 1.0 + 2.0 ** -12
    A = np.array([[-(1.0 + 2.0 ** -11), a1]], dtype=np.float32)
    B = np.array([[1.0], [a1]], dtype=np.float32)
    assert O.matmul(A, B)[0, 0] == 0.0


def test_matmul_tile_does_not_change_bits():
    A = O.normal(31, (70, 45))
    B = O.normal(32, (45, 66))
    assert np.array_equal(O.matmul(A, B, tile=64), O.matmul(A, B, tile=7))


# ----------------------------------------------------- fused forward ----
def test_bias_added_after_accumulation():
    # Products 1 and 2^24, bias 1.  After: (0+1)+2^24 = 2^24 (tie), +1 = 2^24.
    # Bias as the accumulator's initial value would give 1+1+2^24 = 2^24 + 2.
    X = np.array([[1.0, 2.0 ** 24]], dtype=np.float32)
    W = np.ones((2, 1), dtype=np.float32)
    b = np.ones(1, dtype=np.float32)
    assert O.linear_fwd(X, W, b, act=1)[0, 0] == 2.0 ** 24


def test_linear_fwd_special_cases():
    M, K, N = 9, 12, 7
    W = O.normal(41, (K, N))
    b = O.normal(42, N)
    # One-hot rows pick a row of W: Y = relu(W[k] + b).
    X = np.zeros((M, K), dtype=np.float32)
    ks = np.arange(M) % K
    X[np.arange(M), ks] = 1.0
    Y = O.linear_fwd(X, W, b, act=1)
    assert np.array_equal(Y, np.maximum(W[ks] + b, 0).astype(np.float32))
    # W = 0 -> relu(b) in every row; act 0 leaves the bias.
    Wz = np.zeros((K, N), dtype=np.float32)
    assert np.array_equal(O.linear_fwd(O.normal(1, (M, K)), Wz, b, 1), np.tile(np.maximum(b, 0), (M, 1)))
    assert np.array_equal(O.linear_fwd(O.normal(1, (M, K)), Wz, b, 0), np.tile(b, (M, 1)))


def test_bias_act_nan_and_broadcast():
    t = np.array([[np.nan, -1.0, 2.0]], dtype=np.float32)
    b = np.array([0.0, 0.5, -3.0], dtype=np.float32)
    y = O.bias_act(t, b, act=1)
    assert y[0, 0] == 0.0 and y[0, 1] == 0.0 and y[0, 2] == 0.0
    y0 = O.bias_act(t, b, act=0)
    assert np.isnan(y0[0, 0]) and y0[0, 1] == -0.5 and y0[0, 2] == -1.0


# ---------------------------------------------------------- backward ----
def test_relu_mask_mul_signs_and_nans():
    z = np.array([-1.0, -1.0, 2.0, np.nan, -1.0, 0.0, 1e-30], dtype=np.float32)
    g = np.array([3.0, -3.0, -4.0, 5.0, np.inf, 7.0, 2.0], dtype=np.float32)
    out = O.relu_mask_mul(z, g)
    assert out[0] == 0.0 and math.copysign(1, out[0]) == 1
    assert out[1] == 0.0 and math.copysign(1, out[1]) == -1  # 0 * -3 = -0
    assert out[2] == -4.0
    assert out[3] == 0.0                                        # NaN > 0 is false
    assert np.isnan(out[4])                                     # 0 * inf
    assert out[5] == 0.0                                        # 0 > 0 is false
    assert out[6] == 2.0                                        # denormal-free tiny positive


def test_sum_reduce_closed_forms():
    M, N = 513, 37
    ones = np.ones((M, N), dtype=np.float32)
    assert np.array_equal(O.sum_reduce(ones, 0), np.full(N, M, dtype=np.float32))
    assert np.array_equal(O.sum_reduce(ones, 1), np.full(M, N, dtype=np.float32))
    rng = np.random.default_rng(2)
    x = rng.integers(-50, 51, size=(M, N)).astype(np.float32)
    assert np.array_equal(O.sum_reduce(x, 0), x.astype(np.int64).sum(0).astype(np.float32))
    assert np.array_equal(O.sum_reduce(x, 1), x.astype(np.int64).sum(1).astype(np.float32))
    # Sequential order (same construction as the matmul order test).
    col = np.array([[2.0 ** 24], [1.0], [1.0], [-(2.0 ** 24)]], dtype=np.float32)
    assert O.sum_reduce(col, 0)[0] == 0.0


def test_linear_bwd_matches_its_definition():
    M, K, N = 33, 21, 17
    X = O.normal(51, (M, K))
    W = O.normal(52, (K, N), 0.0, 0.3)
    b = O.normal(53, N, 0.0, 0.1)
    Y = O.linear_fwd(X, W, b, 1)
    dY = O.normal(54, (M, N))
    dX, dW, db = O.linear_bwd(X, W, Y, dY, act=1)
    mask = (Y > 0).astype(np.float64)
    dZ = mask * dY
    # Float64 brute force with the gamma_K bound of the fp32 sequential sums.
    ex = dZ @ W.astype(np.float64).T
    assert np.all(np.abs(dX - ex) <= 1.01 * N * U * (np.abs(dZ) @ np.abs(W.astype(np.float64)).T) + 1e-30)
    ew = X.astype(np.float64).T @ dZ
    assert np.all(np.abs(dW - ew) <= 1.01 * M * U * (np.abs(X.astype(np.float64)).T @ np.abs(dZ)) + 1e-30)
    eb = dZ.sum(0)
    assert np.all(np.abs(db - eb) <= 1.01 * M * U * np.abs(dZ).sum(0) + 1e-30)
    # act 0: dZ = dY.
    dX0, dW0, db0 = O.linear_bwd(X, W, Y, dY, act=0)
    assert np.array_equal(db0, O.sum_reduce(dY, 0))
    assert np.array_equal(dX0, O.matmul(dY, W, transB=True))
    # Optional outputs.
    _, dWo, dbo = O.linear_bwd(X, W, Y, dY, act=1, want=("dW", "db"))
    assert np.array_equal(dWo, dW) and np.array_equal(dbo, db)


def test_linear_bwd_db_all_ones():
    M, K, N = 40, 3, 5
    X = np.ones((M, K), dtype=np.float32)
    W = np.ones((K, N), dtype=np.float32)
    Y = np.ones((M, N), dtype=np.float32)
    dY = np.ones((M, N), dtype=np.float32)
    dX, dW, db = O.linear_bwd(X, W, Y, dY, act=1)
    assert np.array_equal(db, np.full(N, M, dtype=np.float32))
    assert np.array_equal(dW, np.full((K, N), M, dtype=np.float32))
    assert np.array_equal(dX, np.full((M, K), N, dtype=np.float32))


# --------------------------------------------------------- elementwise ----
def test_elementwise_matches_ieee_single_ops():
    n = 4099
    a = O.normal(61, n)
    b = O.normal(62, n)
    d = O.uniform(63, n, 0.5, 2.0)
    with np.errstate(all="ignore"):
        assert np.array_equal(O.elementwise(O.EW_ADD, a, b), a + b)
        assert np.array_equal(O.elementwise(O.EW_SUB, a, b), a - b)
        assert np.array_equal(O.elementwise(O.EW_MUL, a, b), a * b)
        assert np.array_equal(O.elementwise(O.EW_DIV, a, d), a / d)
        assert np.array_equal(O.elementwise(O.EW_NEG, a), -a)
        assert np.array_equal(O.elementwise(O.EW_SCALE, a, alpha=0.5), a * np.float32(0.5))
        assert np.array_equal(O.elementwise(O.EW_RELU, a), np.where(a > 0, a, np.float32(0)))
        assert np.array_equal(O.elementwise(O.EW_RELU_BWD, a, b), np.where(a > 0, b, np.float32(0) * b))


def test_elementwise_special_values_and_broadcast():
    a = np.array([1.0, -1.0, 0.0, np.nan], dtype=np.float32)
    z = np.zeros(4, dtype=np.float32)
    with np.errstate(all="ignore"):
        r = O.elementwise(O.EW_DIV, a, z)
    assert r[0] == np.inf and r[1] == -np.inf and np.isnan(r[2]) and np.isnan(r[3])
    assert O.elementwise(O.EW_RELU, a)[3] == 0.0  # maxnum(NaN, 0) = 0
    neg = O.elementwise(O.EW_NEG, np.array([0.0], dtype=np.float32))
    assert math.copysign(1, neg[0]) == -1
    # bmod > 0 broadcasts the rhs row (bias add), bmod < 0 the lhs.
    x = O.normal(71, (6, 8))
    row = O.normal(72, 8)
    assert np.array_equal(O.elementwise(O.EW_ADD, x, row, bmod=8).reshape(6, 8), x + row)
    assert np.array_equal(O.elementwise(O.EW_SUB, row, x, bmod=-8).reshape(6, 8), row - x)


# -------------------------------------------------------- softmax-CE ----
def test_softmax_ce_against_float64():
    M, C = 64, 10
    logits = O.normal(81, (M, C), 0.0, 3.0)
    lbl = O.labels(82, M, C)
    loss, d = O.softmax_ce(logits, lbl)
    L = logits.astype(np.float64)
    m = L.max(1, keepdims=True)
    lse = m[:, 0] + np.log(np.exp(L - m).sum(1))
    ref = float(np.mean(lse - L[np.arange(M), lbl]))
    assert abs(loss - ref) <= 1e-5 * max(1.0, abs(ref))
    p = np.exp(L - lse[:, None])
    p[np.arange(M), lbl] -= 1.0
    assert np.max(np.abs(d - p / M)) <= 1e-6


def test_softmax_ce_closed_forms():
    # Equal logits: every row is uniform, loss = log C, dlogits = (1/C - onehot)/M.
    M, C = 8, 10
    lbl = O.labels(83, M, C)
    loss, d, rows = O.softmax_ce(np.full((M, C), 2.5, np.float32), lbl, want_rows=True)
    assert np.allclose(rows, math.log(C), rtol=0, atol=4 * U * math.log(C) + 1e-7)
    assert abs(loss - math.log(C)) <= 1e-6
    exp = np.full((M, C), (1.0 / C) / M)
    exp[np.arange(M), lbl] -= 1.0 / M
    assert np.max(np.abs(d - exp)) <= 1e-7
    # A dominant correct logit gives loss ~ 0 and gradient ~ 0; a dominant
    # wrong logit gives loss ~ the margin.
    z = np.zeros((2, 4), np.float32)
    z[0, 1] = 50.0
    z[1, 3] = 50.0
    _, d, rows = O.softmax_ce(z, np.array([1, 0], np.int32), want_rows=True)
    assert rows[0] < 1e-20 and abs(rows[1] - 50.0) < 1e-5
    assert abs(d[0]).max() < 1e-20 and abs(d[1, 0] + 0.5) < 1e-7 and abs(d[1, 3] - 0.5) < 1e-7


def test_softmax_ce_gradient_is_the_derivative():
    # Central differences of the float64 mean loss along random directions
    # agree with the oracle's dlogits; a wrong sign, a missing 1/M or a
    # one-hot on the wrong column fails this.
    M, C = 6, 7
    logits = O.normal(84, (M, C), 0.0, 2.0)
    lbl = O.labels(85, M, C)
    _, d = O.softmax_ce(logits, lbl)

    def f(L):
        L = L.astype(np.float64)
        m = L.max(1, keepdims=True)
        return float(np.mean(m[:, 0] + np.log(np.exp(L - m).sum(1)) - L[np.arange(M), lbl]))

    rng = np.random.default_rng(0)
    for _ in range(5):
        v = rng.standard_normal((M, C))
        h = 1e-4
        L64 = logits.astype(np.float64)
        fd = (f(L64 + h * v) - f(L64 - h * v)) / (2 * h)
        assert abs(fd - float(np.sum(d * v))) <= 1e-5
    # Rows of the gradient sum to zero (softmax sums to one).
    assert np.max(np.abs(d.sum(1))) <= 4 * C * U


def test_softmax_ce_shift_invariance():
    M, C = 16, 33
    logits = O.normal(86, (M, C), 0.0, 1.0)
    lbl = O.labels(87, M, C)
    l0, d0, r0 = O.softmax_ce(logits, lbl, want_rows=True)
    l1, d1, r1 = O.softmax_ce(logits + np.float32(64.0), lbl, want_rows=True)
    # x - max is exact for both, so the softmax terms coincide up to the
    # rounding of the shifted inputs (64 + x loses low bits of x).
    assert np.max(np.abs(r0 - r1)) <= 64 * 2 * U * 4
    assert np.max(np.abs(d0 - d1)) <= 1e-5


def test_sgd_update_rounds_the_product_first():
    lr = f32(1 + 2 ** -12)
    g = np.array([1 + 2 ** -12], np.float32)
    w = np.array([1 + 2 ** -11], np.float32)
    out = O.sgd_update(w, g, float(lr))
    step = np.float32(lr * g[0])             # rounded product
    assert out[0] == np.float32(w[0] - step)
    fused = np.float32(float(w[0]) - float(lr) * float(g[0]))  # single rounding
    assert out[0] != fused
    # bf16: 1.0 - 0.5 * 2^-8 = 1 - 2^-9 rounds (ties to even) to 1.0; 1.5 - 0.5 * 0.25 = 1.375.
    wb = O.pack_bf16(np.array([1.0, 1.5], np.float32))
    ob = O.sgd_update(wb, np.array([2.0 ** -8, 0.25], np.float32), 0.5)
    assert np.array_equal(O.bf16_bits_to_f32(ob), np.array([1.0, 1.375], np.float32))



# ------------------------------------------------- transcendental ops ----
def _ulp(x):
    x = np.abs(np.asarray(x, np.float64))
    return np.maximum(np.spacing(x.astype(np.float32)).astype(np.float64), np.finfo(np.float32).tiny)


def test_transcendental_ops_against_float64():
    # libm's expf/logf/tanhf are within an ulp or two of the exact value; the
    # sigmoid chain adds an add and a division.
    x = np.concatenate([np.linspace(-20, 20, 4001), O.normal(91, 4000, 0.0, 3.0)]).astype(np.float32)
    xd = x.astype(np.float64)
    checks = {
        O.EW_EXP: (np.exp(xd), 1.0),
        O.EW_TANH: (np.tanh(xd), 2.0),
        O.EW_SIGMOID: (1.0 / (1.0 + np.exp(-xd)), 3.0),
    }
    for op, (exact, k) in checks.items():
        got = O.elementwise(op, x).astype(np.float64)
        assert np.all(np.abs(got - exact) <= k * _ulp(exact)), O.EW_NAMES[op]
    pos = np.abs(x) + np.float32(1e-3)
    got = O.elementwise(O.EW_LOG, pos).astype(np.float64)
    exact = np.log(pos.astype(np.float64))
    assert np.all(np.abs(got - exact) <= 1.0 * _ulp(exact))


def test_transcendental_closed_forms_and_specials():
    z = np.zeros(1, np.float32)
    assert O.elementwise(O.EW_SIGMOID, z)[0] == 0.5
    assert O.elementwise(O.EW_EXP, z)[0] == 1.0 and O.elementwise(O.EW_TANH, z)[0] == 0.0
    assert O.elementwise(O.EW_LOG, np.ones(1, np.float32))[0] == 0.0
    g = np.array([3.0], np.float32)
    assert O.elementwise(O.EW_SIGMOID_BWD, z, g)[0] == np.float32(0.75)   # 3 * 0.25
    assert O.elementwise(O.EW_TANH_BWD, z, g)[0] == 3.0                  # t = 0
    assert O.elementwise(O.EW_EXP_BWD, z, g)[0] == 3.0
    big = np.array([-200.0, 200.0], np.float32)
    with np.errstate(all="ignore"):
        assert np.array_equal(O.elementwise(O.EW_SIGMOID, big), np.array([0.0, 1.0], np.float32))
        assert np.isinf(O.elementwise(O.EW_EXP, big)[1]) and O.elementwise(O.EW_EXP, big)[0] == 0.0
        assert O.elementwise(O.EW_LOG, np.zeros(1, np.float32))[0] == -np.inf
        assert np.isnan(O.elementwise(O.EW_LOG, -np.ones(1, np.float32))[0])
        # Tanh backward goes through exp like the reference: inf / inf for |x| > ~88.7.
        assert np.all(np.isnan(O.elementwise(O.EW_TANH_BWD, big, np.ones(2, np.float32))))
    # Div's divisor gradient: -((a / (b * b)) * g), exact on powers of two.
    a, b, c = (np.array(v, np.float32) for v in ([1.0, -6.0], [2.0, 0.5], [8.0, 1.0]))
    assert np.array_equal(O.elementwise3(O.EW3_DIV_BWD_B, a, b, c), np.array([-2.0, 24.0], np.float32))


def test_backward_ops_follow_the_reference_graph_order():
    # Sigmoid backward is grad * (s * (1 - s)) and tanh backward recomputes
    # tanh through exp; on random inputs some results differ in the last bit
    # from (grad * s) * (1 - s) and from 1 - tanhf(x)^2, so these pin the order.
    x = O.normal(92, 20000, 0.0, 2.0)
    g = O.normal(93, 20000, 0.0, 3.0)
    f = np.float32
    with np.errstate(all="ignore"):
        e = np.exp(-x.astype(np.float64)).astype(f)
    s = (f(1.0) / (f(1.0) + e)).astype(f)
    want = (g * (s * (f(1.0) - s))).astype(f)
    other = ((g * s) * (f(1.0) - s)).astype(f)
    got = O.elementwise(O.EW_SIGMOID_BWD, x, g)
    exp_ok = O.elementwise(O.EW_EXP, -x)
    same_e = exp_ok == e   # where libm's expf agrees with numpy's rounding of exp
    assert np.array_equal(got[same_e], want[same_e])
    assert np.any(got[same_e] != other[same_e])
    t_tanhf = O.elementwise(O.EW_TANH, x)
    gt = O.elementwise(O.EW_TANH_BWD, x, g)
    via_tanhf = (g * (f(1.0) - t_tanhf * t_tanhf)).astype(f)
    assert np.any(gt != via_tanhf)
    bound = np.abs(g).astype(np.float64) * 16 * 2.0 ** -23 + 4 * _ulp(via_tanhf)
    assert np.all(np.abs(gt.astype(np.float64) - via_tanhf) <= bound)


def test_act_grad_and_epilogue_activations():
    y = np.array([0.0, 0.5, 0.25, -0.5, 2.0], np.float32)
    g = np.array([1.0, 1.0, 2.0, 4.0, -1.0], np.float32)
    assert np.array_equal(O.act_grad(y, g, 1), O.relu_mask_mul(y, g))
    assert np.array_equal(O.act_grad(y, g, 2), g * (y * (np.float32(1) - y)))
    assert np.array_equal(O.act_grad(y, g, 3), g * (np.float32(1) - y * y))
    assert np.array_equal(O.act_grad(y, g, 0), g)
    assert O.act_grad(np.float32([0.5]), np.float32([1.0]), 2)[0] == 0.25
    # Sigmoid/tanh epilogues equal the elementwise ops applied to t + b.
    t = O.normal(94, (16, 24), 0.0, 2.0)
    b = O.normal(95, 24)
    z = O.bias_act(t, b, act=0)
    assert np.array_equal(O.bias_act(t, b, act=2), O.elementwise(O.EW_SIGMOID, z).reshape(z.shape))
    assert np.array_equal(O.bias_act(t, b, act=3), O.elementwise(O.EW_TANH, z).reshape(z.shape))
    # The fused sigmoid backward from Y equals the per-node backward from Z
    # (the per-node graph recomputes the same s = 1/(1+exp(-z))).
    gz = O.normal(96, z.shape)
    y2 = O.bias_act(t, b, act=2)
    assert np.array_equal(O.act_grad(y2, gz, 2), O.elementwise(O.EW_SIGMOID_BWD, z, gz).reshape(z.shape))


def test_fused_tanh_backward_against_the_reference_composition():
    """The fused Linear+Tanh backward forms tanh' from the saved output Y as
    1 - Y*Y; the reference's Tanh node recomputes t from the pre-activation z
    through exp.  For |z| <= 88 they agree within 16 ulp of |g| (plus 4 ulp of
    the result); beyond that the reference's e^z overflows, t = inf/inf = NaN,
    while 1 - Y*Y = 0 (the derivative underflows there).  Both facts are pinned."""
    f = np.float32
    z = np.concatenate([O.normal(97, 20000, 0.0, 3.0), np.array([88.0, -88.0, 89.0, -89.0, 100.0, -1e4], f)])
    g = O.normal(98, z.size, 0.0, 2.0)
    y = O.elementwise(O.EW_TANH, z)
    fused = O.act_grad(y, g, 3)
    with np.errstate(all="ignore"):
        ref = O.elementwise(O.EW_TANH_BWD, z, g)
    small = np.abs(z) <= 88.0
    bound = np.abs(g[small]).astype(np.float64) * 16 * 2.0 ** -23 + 4 * _ulp(ref[small])
    assert np.all(np.abs(fused[small].astype(np.float64) - ref[small]) <= bound)
    big = np.abs(z) >= 89.0
    assert np.all(np.isnan(ref[big])) and np.all(fused[big] == 0.0)
    # The composition routine applies the same rule before its GEMMs.
    X = O.normal(99, (6, 5))
    W = O.normal(100, (5, 4))
    Z = O.normal(101, (6, 4), 0.0, 2.0)
    dY = O.normal(102, (6, 4))
    dX, dW, db = O.linear_bwd_from_preact(X, W, Z, dY, 3)
    dZ = O.elementwise(O.EW_TANH_BWD, Z, dY).reshape(Z.shape)
    assert np.array_equal(dX, O.matmul(dZ, W, transB=True))
    assert np.array_equal(dW, O.matmul(X, dZ, transA=True))
    assert np.array_equal(db, O.sum_reduce(dZ, 0))
    # ReLU: the mask from Z equals the mask from Y = maxnum(Z, 0), so both routes agree bit for bit.
    Y = O.bias_act(Z, np.zeros(4, f), act=1)
    for a, b in zip(O.linear_bwd_from_preact(X, W, Z, dY, 1), O.linear_bwd(X, W, Y, dY, 1)):
        assert np.array_equal(a, b)
