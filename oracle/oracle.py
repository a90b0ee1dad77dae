"""ctypes front end of the oracle (oracle/c3_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker.  The product path never imports
this module.

Arrays are numpy float32 / int32, C-contiguous.  How each restated function
is pinned, and the one property left "parity unpinned" (the exact bits of
the reference's LLVM-JIT output), is stated in c3_oracle.h.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liboracle.so"
_lib = None

EW_ADD, EW_SUB, EW_MUL, EW_DIV, EW_RELU, EW_RELU_BWD, EW_NEG, EW_SCALE = range(8)
EW_NAMES = ["add", "sub", "mul", "div", "relu", "relu_bwd", "neg", "scale", "sigmoid", "tanh", "exp", "log",
            "sigmoid_bwd", "tanh_bwd", "exp_bwd"]
EW_SIGMOID, EW_TANH, EW_EXP, EW_LOG, EW_SIGMOID_BWD, EW_TANH_BWD, EW_EXP_BWD = range(8, 15)
EW3_DIV_BWD_B = 0
EW_BINARY = {EW_ADD, EW_SUB, EW_MUL, EW_DIV, EW_RELU_BWD, EW_SIGMOID_BWD, EW_TANH_BWD, EW_EXP_BWD}

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            raise RuntimeError(f"{_LIB_PATH} is not built; run `make -C oracle` or __graft_entry__.build()")
        L = ctypes.CDLL(str(_LIB_PATH))
        L.oracle_fill_uniform.argtypes = [ctypes.c_uint64, _f32p, _i64, ctypes.c_float, ctypes.c_float]
        L.oracle_fill_normal.argtypes = [ctypes.c_uint64, _f32p, _i64, ctypes.c_float, ctypes.c_float]
        L.oracle_fill_labels.argtypes = [ctypes.c_uint64, _i32p, _i64, ctypes.c_int32]
        L.oracle_round_bf16.argtypes = [_f32p, _f32p, _i64]
        L.oracle_pack_bf16.argtypes = [_f32p, _u16p, _i64]
        L.oracle_maxnum.argtypes = [ctypes.c_float, ctypes.c_float]
        L.oracle_maxnum.restype = ctypes.c_float
        L.oracle_matmul.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, _i64, ctypes.c_int, ctypes.c_int, _i64]
        L.oracle_bias_act.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, ctypes.c_int]
        L.oracle_linear_fwd.argtypes = [_f32p, _f32p, _f32p, _f32p, _i64, _i64, _i64, ctypes.c_int]
        L.oracle_relu_mask_mul.argtypes = [_f32p, _f32p, _f32p, _i64]
        L.oracle_sum_reduce.argtypes = [_f32p, _f32p, _i64, _i64, ctypes.c_int]
        vp = ctypes.c_void_p
        L.oracle_linear_bwd.argtypes = [_f32p, _f32p, _f32p, _f32p, vp, vp, vp, _i64, _i64, _i64, ctypes.c_int]
        L.oracle_elementwise.argtypes = [ctypes.c_int, _f32p, vp, ctypes.c_float, _f32p, _i64, _i64]
        L.oracle_elementwise3.argtypes = [ctypes.c_int, _f32p, _f32p, _f32p, _f32p, _i64]
        L.oracle_act_grad.argtypes = [_f32p, _f32p, _f32p, _i64, ctypes.c_int]
        L.oracle_softmax_ce.argtypes = [_f32p, _i32p, vp, vp, _i64, _i64]
        L.oracle_softmax_ce.restype = ctypes.c_float
        L.oracle_sgd_update.argtypes = [_f32p, _f32p, ctypes.c_float, _i64]
        L.oracle_sgd_update_bf16.argtypes = [_u16p, _f32p, ctypes.c_float, _i64]
        _lib = L
    return _lib


def _c(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


# ---- inputs -----------------------------------------------------------------
def uniform(seed: int, shape, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    out = np.empty(shape, dtype=np.float32)
    lib().oracle_fill_uniform(seed, out.reshape(-1), out.size, lo, hi)
    return out


def normal(seed: int, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(shape, dtype=np.float32)
    lib().oracle_fill_normal(seed, out.reshape(-1), out.size, mean, std)
    return out


def labels(seed: int, n: int, num_classes: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    lib().oracle_fill_labels(seed, out, n, num_classes)
    return out


def round_bf16(x: np.ndarray) -> np.ndarray:
    x = _c(x)
    out = np.empty_like(x)
    lib().oracle_round_bf16(x.reshape(-1), out.reshape(-1), x.size)
    return out


def pack_bf16(x: np.ndarray) -> np.ndarray:
    x = _c(x)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_pack_bf16(x.reshape(-1), out.reshape(-1), x.size)
    return out


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---- kernels ----------------------------------------------------------------
def maxnum(a: float, b: float) -> float:
    return lib().oracle_maxnum(a, b)


def matmul(A, B, transA=False, transB=False, tile=64):
    A, B = _c(A), _c(B)
    M = A.shape[1] if transA else A.shape[0]
    K = A.shape[0] if transA else A.shape[1]
    N = B.shape[0] if transB else B.shape[1]
    KB = B.shape[1] if transB else B.shape[0]
    assert K == KB, (A.shape, B.shape, transA, transB)
    C = np.empty((M, N), dtype=np.float32)
    lib().oracle_matmul(A.reshape(-1), B.reshape(-1), C.reshape(-1), M, K, N, int(transA), int(transB), tile)
    return C


def bias_act(t, b, act=1):
    t, b = _c(t), _c(b)
    M, N = t.shape
    y = np.empty_like(t)
    lib().oracle_bias_act(t.reshape(-1), b, y.reshape(-1), M, N, act)
    return y


def linear_fwd(X, W, b, act=1):
    X, W, b = _c(X), _c(W), _c(b)
    M, K = X.shape
    N = W.shape[1]
    Y = np.empty((M, N), dtype=np.float32)
    lib().oracle_linear_fwd(X.reshape(-1), W.reshape(-1), b, Y.reshape(-1), M, K, N, act)
    return Y


def relu_mask_mul(z, g):
    z, g = _c(z), _c(g)
    out = np.empty_like(z)
    lib().oracle_relu_mask_mul(z.reshape(-1), g.reshape(-1), out.reshape(-1), z.size)
    return out


def sum_reduce(x, axis=0):
    x = _c(x)
    M, N = x.shape
    out = np.empty(N if axis == 0 else M, dtype=np.float32)
    lib().oracle_sum_reduce(x.reshape(-1), out, M, N, axis)
    return out


def linear_bwd(X, W, Y, dY, act=1, want=("dX", "dW", "db")):
    X, W, Y, dY = _c(X), _c(W), _c(Y), _c(dY)
    M, K = X.shape
    N = W.shape[1]
    dX = np.empty((M, K), dtype=np.float32) if "dX" in want else None
    dW = np.empty((K, N), dtype=np.float32) if "dW" in want else None
    db = np.empty(N, dtype=np.float32) if "db" in want else None
    lib().oracle_linear_bwd(X.reshape(-1), W.reshape(-1), Y.reshape(-1), dY.reshape(-1), _ptr(dX), _ptr(dW),
                            _ptr(db), M, K, N, act)
    return dX, dW, db


def elementwise(op, a, b=None, alpha=0.0, bmod=0):
    a = _c(a).reshape(-1)
    n = a.size if bmod >= 0 else (b.size if b is not None else a.size)
    if bmod < 0:
        n = _c(b).size
    bb = None if b is None else _c(b).reshape(-1)
    out = np.empty(n, dtype=np.float32)
    lib().oracle_elementwise(op, a, _ptr(bb), alpha, out, n, bmod)
    return out


def elementwise3(op, a, b, c):
    a, b, c = _c(a).reshape(-1), _c(b).reshape(-1), _c(c).reshape(-1)
    out = np.empty(a.size, dtype=np.float32)
    lib().oracle_elementwise3(op, a, b, c, out, a.size)
    return out


CHAIN_RELU, CHAIN_SIGMOID, CHAIN_TANH, CHAIN_EXP, CHAIN_LOG, CHAIN_NEG = range(6)


def backward_chain(nodes, grad, xs):
    """Upstream grads of a chain of single-input nodes, node 0 downstream:
    g_0 = grad, g_{k+1} = rule_k(g_k, x_k); returns [g_1, ..., g_w].

    The reference merges each node's own backward graph into one
    multi-output graph, feeding node k's output grad to node k+1
    (src/C3/C3BackwardCapture.cpp:1140-1210), so each step is that node's
    rule: ReLU Gt+Mul (:501-528), Sigmoid (:530-567), Tanh (:569-616),
    Exp (:823-849), Log grad/x (:851-872), Neg -grad (:725-741)."""
    rule = {CHAIN_RELU: lambda g, x: elementwise(EW_RELU_BWD, x, g),
            CHAIN_SIGMOID: lambda g, x: elementwise(EW_SIGMOID_BWD, x, g),
            CHAIN_TANH: lambda g, x: elementwise(EW_TANH_BWD, x, g),
            CHAIN_EXP: lambda g, x: elementwise(EW_EXP_BWD, x, g),
            CHAIN_LOG: lambda g, x: elementwise(EW_DIV, g, x),
            CHAIN_NEG: lambda g, x: elementwise(EW_NEG, g)}
    g = _c(grad).reshape(-1)
    outs = []
    for node, x in zip(nodes, xs):
        g = rule[node](g, None if x is None else _c(x).reshape(-1))
        outs.append(g)
    return outs


def act_grad(y, g, act):
    y, g = _c(y), _c(g)
    out = np.empty_like(y)
    lib().oracle_act_grad(y.reshape(-1), g.reshape(-1), out.reshape(-1), y.size, act)
    return out


def linear_bwd_from_preact(X, W, Z, dY, act, want=("dX", "dW", "db")):
    """The reference's per-node backward of a Linear+act layer, from the
    activation's input Z (the Add output, which the reference's autograd
    keeps for the activation node): the activation node's rule -- ReLU Gt+Mul
    (src/C3/C3BackwardCapture.cpp:501-528), Sigmoid and Tanh recomputed from
    Z through exp (:530-616) -- then MatMul's dX, dW (:681-723) and Add's db
    (:618-644).  The fused layer backward gets the output Y instead of Z and
    forms the derivative from Y (act_grad); this composition is what it is
    compared with."""
    rule = {0: None, 1: EW_RELU_BWD, 2: EW_SIGMOID_BWD, 3: EW_TANH_BWD}[act]
    Z, dY = _c(Z), _c(dY)
    dZ = dY if rule is None else elementwise(rule, Z, dY).reshape(Z.shape)
    out = [None, None, None]
    if "dX" in want:
        out[0] = matmul(dZ, W, transB=True)
    if "dW" in want:
        out[1] = matmul(X, dZ, transA=True)
    if "db" in want:
        out[2] = sum_reduce(dZ, 0)
    return tuple(out)


def softmax_ce(logits, lbl, want_grad=True, want_rows=False):
    """Mean CE loss and dlogits (None unless want_grad); with want_rows the
    per-row losses are returned as a third value."""
    logits = _c(logits)
    lbl = np.ascontiguousarray(lbl, dtype=np.int32)
    M, C = logits.shape
    d = np.empty_like(logits) if want_grad else None
    rows = np.empty(M, dtype=np.float32) if want_rows else None
    loss = lib().oracle_softmax_ce(logits.reshape(-1), lbl, _ptr(rows), _ptr(d), M, C)
    return (loss, d, rows) if want_rows else (loss, d)


def sgd_update(w, g, lr):
    """w - lr * g (product rounded first); w fp32 values, or bf16 bit patterns (uint16)."""
    g = _c(g).reshape(-1)
    if np.asarray(w).dtype == np.uint16:
        out = np.array(w, dtype=np.uint16, copy=True)
        lib().oracle_sgd_update_bf16(out.reshape(-1), g, lr, out.size)
        return out
    out = np.array(_c(w), copy=True)
    lib().oracle_sgd_update(out.reshape(-1), g, lr, out.size)
    return out
