"""ctypes binding of the MLP train-step harness in libc3core.so
(c3_amd/csrc/host/include/C3/MlpTrainer.h).

The harness plays the host framework's part around C3: it walks the forward
op trace through RegionFusionRegistry / C3KernelRegistry dispatch (with
C3HotPathManager compiling regions in the background), runs softmax-CE,
the backward through C3BackwardCapture, and an SGD update, all on the GPU.
Pointers are device pointers (for example ``tensor.data_ptr()``).
"""
from __future__ import annotations

import ctypes
from pathlib import Path

from c3_amd import native

CORE_PATH = Path(__file__).resolve().parent / "lib" / "libc3core.so"

_vp, _i64, _int, _f = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
SIGNATURES = {
    "c3mlp_last_error": (ctypes.c_char_p, []),
    "c3mlp_create": (_int, [_int, ctypes.POINTER(_i64), _int, _i64, ctypes.POINTER(_vp)]),
    "c3mlp_destroy": (None, [_vp]),
    "c3mlp_params": (_int, [_vp, _int, ctypes.POINTER(_vp), ctypes.POINTER(_vp)]),
    "c3mlp_forward": (_int, [_vp, _vp, _vp, _vp]),
    "c3mlp_step": (_int, [_vp, _vp, _vp, _f, ctypes.POINTER(_f), _vp]),
    "c3mlp_warm_up": (_int, [_vp, _vp, _vp, _f, _int, ctypes.POINTER(_int), _vp]),
    "c3mlp_stats": (_int, [_vp, ctypes.POINTER(_i64)]),
    "c3mlp_set_keep_gradients": (_int, [_vp, _int]),
    "c3mlp_tensor": (_int, [_vp, _int, _int, ctypes.POINTER(_vp)]),
    "c3mlp_capture": (_int, [_vp, _vp, _vp, _f, _vp]),
    "c3mlp_replay": (_int, [_vp, _vp]),
}

_core = None


def load() -> ctypes.CDLL:
    global _core
    if _core is None:
        native.load()  # libc3hip.so first (and torch's HIP runtime before it)
        if not CORE_PATH.exists():
            raise RuntimeError(f"{CORE_PATH} is not built: run `python -m c3_amd.build`")
        lib = ctypes.CDLL(str(CORE_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _core = lib
    return _core


class TrainerError(RuntimeError):
    pass


def _check(fn: str, rc: int) -> None:
    if rc != 0:
        raise TrainerError(f"{fn} failed: {load().c3mlp_last_error().decode(errors='replace')}")


STAT_NAMES = ("steps", "region_hits", "single_op_hits", "eager_ops", "backward_hits", "backward_misses",
              "fully_dispatched", "graph_replays")
ACTIVATION, OUTPUT_GRAD, WEIGHT_GRAD, BIAS_GRAD = range(4)


class MlpTrainer:
    """Linear layers dims[0] -> ... -> dims[-1], ReLU between them, batch rows."""

    def __init__(self, dims, batch: int, dtype: int = native.F32):
        L = load()
        arr = (_i64 * len(dims))(*dims)
        h = _vp()
        _check("c3mlp_create", L.c3mlp_create(dtype, arr, len(dims), batch, ctypes.byref(h)))
        self._h = h
        self.dims = list(dims)
        self.batch = batch
        self.dtype = dtype

    def close(self) -> None:
        if self._h:
            load().c3mlp_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def num_layers(self) -> int:
        return len(self.dims) - 1

    def params(self, layer: int) -> tuple[int, int]:
        w, b = _vp(), _vp()
        _check("c3mlp_params", load().c3mlp_params(self._h, layer, ctypes.byref(w), ctypes.byref(b)))
        return w.value, b.value

    def forward(self, X: int, logits_out: int, stream: int = 0) -> None:
        _check("c3mlp_forward", load().c3mlp_forward(self._h, X, logits_out, stream))

    def step(self, X: int, labels: int, lr: float, want_loss: bool = True, stream: int = 0) -> float | None:
        loss = _f()
        _check("c3mlp_step", load().c3mlp_step(self._h, X, labels, lr, ctypes.byref(loss) if want_loss else None,
                                               stream))
        return loss.value if want_loss else None

    def warm_up(self, X: int, labels: int, lr: float, max_steps: int = 16, stream: int = 0) -> int:
        n = _int()
        _check("c3mlp_warm_up", load().c3mlp_warm_up(self._h, X, labels, lr, max_steps, ctypes.byref(n), stream))
        return n.value

    def stats(self) -> dict:
        out = (_i64 * 8)()
        _check("c3mlp_stats", load().c3mlp_stats(self._h, out))
        return dict(zip(STAT_NAMES, list(out)))

    def capture(self, X: int, labels: int, lr: float, stream: int) -> None:
        """Record one train step as a HIP graph on `stream` (not the default
        stream); runs one real step first to size the device pool."""
        _check("c3mlp_capture", load().c3mlp_capture(self._h, X, labels, lr, stream))

    def replay(self, stream: int) -> None:
        _check("c3mlp_replay", load().c3mlp_replay(self._h, stream))

    def keep_gradients(self, keep: bool = True) -> None:
        _check("c3mlp_set_keep_gradients", load().c3mlp_set_keep_gradients(self._h, int(keep)))

    def tensor(self, which: int, layer: int) -> int:
        p = _vp()
        _check("c3mlp_tensor", load().c3mlp_tensor(self._h, which, layer, ctypes.byref(p)))
        return p.value
