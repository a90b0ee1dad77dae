"""ctypes binding of libc3hip.so (the C ABI declared in include/c3hip.h).

This is the binding a Python caller of the backend uses; tests and bench.py
go through it so every GPU result crosses the same C ABI a C/C++ host would
call.  Device pointers and streams are plain integers (for example
``tensor.data_ptr()`` and ``torch.cuda.current_stream().cuda_stream``).

Loading fails loudly when the library is not built: there is no fallback.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_DIR = Path(__file__).resolve().parent / "lib"
LIB_PATH = LIB_DIR / "libc3hip.so"

# Status codes, element types, activations and elementwise ops (include/c3hip.h).
OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_HIP, ERR_NOT_FOUND, ERR_TOO_LARGE = 0, 1, 2, 3, 4, 5
F32, BF16 = 0, 1
ACT_NONE, ACT_RELU, ACT_SIGMOID, ACT_TANH = 0, 1, 2, 3
EW_ADD, EW_SUB, EW_MUL, EW_DIV, EW_RELU, EW_RELU_BWD, EW_NEG, EW_SCALE = range(8)
EW_SIGMOID, EW_TANH, EW_EXP, EW_LOG, EW_SIGMOID_BWD, EW_TANH_BWD, EW_EXP_BWD = range(8, 15)
EW3_DIV_BWD_B = 0
CHAIN_RELU, CHAIN_SIGMOID, CHAIN_TANH, CHAIN_EXP, CHAIN_LOG, CHAIN_NEG = range(6)
CHAIN_MAX_NODES = 4
# Node type names of the backward chain (the host framework's node types).
CHAIN_NODES = {"ReLU": CHAIN_RELU, "Sigmoid": CHAIN_SIGMOID, "Tanh": CHAIN_TANH, "Exp": CHAIN_EXP,
               "Log": CHAIN_LOG, "Neg": CHAIN_NEG}
# The eight single-node ops of the fused path's elementwise set.
EW_OPS = {"add": EW_ADD, "sub": EW_SUB, "mul": EW_MUL, "div": EW_DIV, "relu": EW_RELU,
          "relu_bwd": EW_RELU_BWD, "neg": EW_NEG, "scale": EW_SCALE}
# Transcendental forward ops and the single-input backward ops.
EW_MATH_OPS = {"sigmoid": EW_SIGMOID, "tanh": EW_TANH, "exp": EW_EXP, "log": EW_LOG,
               "sigmoid_bwd": EW_SIGMOID_BWD, "tanh_bwd": EW_TANH_BWD, "exp_bwd": EW_EXP_BWD}

# Every symbol include/c3hip.h declares, with its ctypes signature.
_vp, _i64, _int, _f = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
SIGNATURES = {
    "c3hip_abi_version": (_int, []),
    "c3hip_last_error": (ctypes.c_char_p, []),
    "c3hip_init": (_int, [_int]),
    "c3hip_shutdown": (_int, []),
    "c3hip_load_code_object": (_int, [ctypes.c_char_p, _vp, ctypes.c_size_t]),
    "c3hip_code_object_path": (_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_size_t]),
    "c3hip_set_launch_timing": (_int, [_int]),
    "c3hip_launch_timings": (_int, [ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(_f), _int,
                                    ctypes.POINTER(_int)]),
    "c3hip_elementwise": (_int, [_int, _int, _vp, _vp, _f, _vp, _i64, _i64, _vp]),
    "c3hip_elementwise3": (_int, [_int, _int, _vp, _vp, _vp, _vp, _i64, _vp]),
    "c3hip_set_gemm_tile": (_int, [_int, ctypes.c_char_p]),
    "c3hip_gemm_tile_names": (_int, [_int, ctypes.c_char_p, ctypes.c_size_t]),
    "c3hip_backward_chain": (_int, [_int, _vp, ctypes.POINTER(_vp), ctypes.POINTER(_int), _int,
                                    ctypes.POINTER(_vp), _i64, _vp]),
    "c3hip_matmul": (_int, [_int, _vp, _vp, _vp, _i64, _i64, _i64, _int, _int, _vp]),
    "c3hip_linear_fwd": (_int, [_int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _int, _vp]),
    "c3hip_linear_fwd_noalloc": (_int, [_int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _int, _vp]),
    "c3hip_linear_bwd": (_int, [_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _int, _vp]),
    "c3hip_sum_reduce": (_int, [_vp, _vp, _i64, _i64, _int, _vp]),
    "c3hip_softmax_ce": (_int, [_int, _vp, _vp, _vp, _vp, _i64, _i64, _vp]),
    "c3hip_cast": (_int, [_int, _int, _vp, _vp, _i64, _vp]),
    "c3hip_sgd_update": (_int, [_int, _vp, _vp, _f, _i64, _vp]),
    "c3hip_sgd_update_multi": (_int, [_int, _int, ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_void_p),
                                      ctypes.POINTER(ctypes.c_int64), _f, _vp]),
}


class C3HipError(RuntimeError):
    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed with status {code}: {msg}")
        self.code = code


_lib = None


def load(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """Load libc3hip.so once and attach the signatures."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise RuntimeError(f"{p} is not built: run `python -m c3_amd.build` (no CPU fallback exists)")
    # torch wheels carry their own libamdhip64.so.7.  Importing torch first lets
    # this library bind to that copy (same soname) so device pointers and
    # streams are shared; otherwise two HIP runtimes would end up in one process.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def _check(fn: str, rc: int) -> None:
    if rc != OK:
        raise C3HipError(fn, rc, load().c3hip_last_error().decode(errors="replace"))


def last_error() -> str:
    return load().c3hip_last_error().decode(errors="replace")


def init(device: int = 0) -> None:
    _check("c3hip_init", load().c3hip_init(device))


def shutdown() -> None:
    _check("c3hip_shutdown", load().c3hip_shutdown())


def set_launch_timing(enable: bool) -> None:
    """Bracket every kernel this thread launches through the library with HIP events."""
    _check("c3hip_set_launch_timing", load().c3hip_set_launch_timing(int(enable)))


def launch_timings(max_records: int = 65536, name_len: int = 96) -> list[tuple[str, float]]:
    """(kernel name, ms) of each launch recorded since the last call, in launch order; clears them."""
    names = ctypes.create_string_buffer(max_records * name_len)
    ms = (_f * max_records)()
    cnt = _int()
    _check("c3hip_launch_timings", load().c3hip_launch_timings(names, name_len, ms, max_records, ctypes.byref(cnt)))
    raw = names.raw
    return [(raw[i * name_len:(i + 1) * name_len].split(b"\0", 1)[0].decode(), ms[i]) for i in range(cnt.value)]


def elementwise(op: int, dtype: int, a: int, b: int | None, alpha: float, out: int, n: int, bmod: int = 0,
                stream: int = 0) -> None:
    _check("c3hip_elementwise", load().c3hip_elementwise(op, dtype, a, b, alpha, out, n, bmod, stream))


def elementwise3(op: int, dtype: int, a: int, b: int, c: int, out: int, n: int, stream: int = 0) -> None:
    _check("c3hip_elementwise3", load().c3hip_elementwise3(op, dtype, a, b, c, out, n, stream))


def set_gemm_tile(dtype: int, name: str | None) -> None:
    """Force the calling thread's GEMM tile for dtype (None: size heuristic)."""
    _check("c3hip_set_gemm_tile", load().c3hip_set_gemm_tile(dtype, name.encode() if name else None))


def gemm_tile_names(dtype: int) -> list[str]:
    buf = ctypes.create_string_buffer(512)
    _check("c3hip_gemm_tile_names", load().c3hip_gemm_tile_names(dtype, buf, len(buf)))
    return buf.value.decode().split(",")


def backward_chain(dtype: int, grad: int, xs, nodes, outs, n: int, stream: int = 0) -> None:
    """Fused backward of len(nodes) single-input nodes (node 0 downstream);
    xs[k] is node k's forward input (None for Neg), outs[k] its upstream grad
    (None: not stored)."""
    w = len(nodes)
    xa = (_vp * max(w, 1))(*[x or None for x in xs])
    oa = (_vp * max(w, 1))(*[o or None for o in outs])
    na = (_int * max(w, 1))(*nodes)
    _check("c3hip_backward_chain", load().c3hip_backward_chain(dtype, grad, xa, na, w, oa, n, stream))


def matmul(dtype: int, A: int, B: int, C: int, M: int, K: int, N: int, transA: bool = False,
           transB: bool = False, stream: int = 0) -> None:
    _check("c3hip_matmul", load().c3hip_matmul(dtype, A, B, C, M, K, N, int(transA), int(transB), stream))


def linear_fwd(dtype: int, X: int, W: int, b: int | None, Y: int, M: int, K: int, N: int, act: int = ACT_RELU,
               stream: int = 0) -> None:
    _check("c3hip_linear_fwd", load().c3hip_linear_fwd(dtype, X, W, b, Y, M, K, N, act, stream))


# Bytes of c3hip_linear_fwd_noalloc's per-device static scratch (C3HIP_NOALLOC_SCRATCH_BYTES).
NOALLOC_SCRATCH_BYTES = 32 << 20


def linear_fwd_noalloc(dtype: int, X: int, W: int, b: int | None, Y: int, M: int, K: int, N: int,
                       act: int = ACT_RELU, stream: int = 0) -> None:
    """c3hip_linear_fwd with its workspace in the library's static scratch (no allocation)."""
    _check("c3hip_linear_fwd_noalloc", load().c3hip_linear_fwd_noalloc(dtype, X, W, b, Y, M, K, N, act, stream))


def linear_bwd(dtype: int, X: int | None, W: int | None, Y: int | None, dY: int, dX: int | None, dW: int | None,
               db: int | None, M: int, K: int, N: int, act: int = ACT_RELU, stream: int = 0) -> None:
    _check("c3hip_linear_bwd", load().c3hip_linear_bwd(dtype, X, W, Y, dY, dX, dW, db, M, K, N, act, stream))


def sum_reduce(inp: int, out: int, M: int, N: int, axis: int = 0, stream: int = 0) -> None:
    _check("c3hip_sum_reduce", load().c3hip_sum_reduce(inp, out, M, N, axis, stream))


def softmax_ce(dtype: int, logits: int, labels: int, loss_rows: int | None, dlogits: int | None, M: int, C: int,
               stream: int = 0) -> None:
    _check("c3hip_softmax_ce", load().c3hip_softmax_ce(dtype, logits, labels, loss_rows, dlogits, M, C, stream))


def cast(src_dtype: int, dst_dtype: int, inp: int, out: int, n: int, stream: int = 0) -> None:
    _check("c3hip_cast", load().c3hip_cast(src_dtype, dst_dtype, inp, out, n, stream))


def sgd_update(dtype: int, w: int, g: int, lr: float, n: int, stream: int = 0) -> None:
    _check("c3hip_sgd_update", load().c3hip_sgd_update(dtype, w, g, lr, n, stream))


SGD_MAX_TENSORS = 16


def sgd_update_multi(dtype: int, ws, gs, ns, lr: float, stream: int = 0) -> None:
    """c3hip_sgd_update on several parameters of one dtype in one launch."""
    k = len(ws)
    W = (ctypes.c_void_p * max(k, 1))(*ws)
    G = (ctypes.c_void_p * max(k, 1))(*gs)
    Nn = (ctypes.c_int64 * max(k, 1))(*ns)
    _check("c3hip_sgd_update_multi", load().c3hip_sgd_update_multi(dtype, k, W, G, Nn, lr, stream))
