"""The C-ABI library without a GPU: it loads, exports every symbol declared in
include/c3hip.h, the code objects hold every kernel the dispatcher can name,
and argument validation answers before any device work."""
import re
import subprocess
from pathlib import Path

import pytest

from c3_amd import native

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "c3hip.h"
LIB = ROOT / "c3_amd" / "lib"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(c3hip_\w+)\s*\(", text)))


def test_header_and_binding_agree():
    assert declared_symbols() == sorted(native.SIGNATURES)


def test_library_exports_every_declared_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", str(native.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\sT\s+(c3hip_\w+)", out))
    missing = set(declared_symbols()) - exported
    assert not missing, missing
    lib = native.load()
    for name in declared_symbols():
        assert hasattr(lib, name)


def test_abi_version():
    assert native.load().c3hip_abi_version() == 1


def _kernel_symbols(hsaco: Path):
    readelf = "/opt/rocm/llvm/bin/llvm-readelf"
    out = subprocess.run([readelf, "--symbols", "--wide", str(hsaco)], capture_output=True, text=True,
                         check=True).stdout
    return set(re.findall(r"FUNC\s+GLOBAL\s+\w+\s+\d+\s+(c3_\w+)$", out, flags=re.M))


def test_code_objects_hold_every_dispatched_kernel():
    gemm = _kernel_symbols(LIB / "gemm_f32.hsaco")
    for kind in ["fwd", "dx", "dx_mask", "dx_mask_dz", "dw", "dw_mask", "tt"]:
        for tile in ["t64x64", "t128x128", "t256x128", "t128x256"]:
            for v in "vs":
                assert f"c3_gemm_f32_{kind}_{tile}_{v}" in gemm
    for kind in ["fwd", "dx", "dw"]:
        for tile in ["t256x128d", "t128x256d", "t64x64d"]:
            assert f"c3_gemm_f32_{kind}_{tile}" in gemm
    assert {"c3_gemm_f32_dx_t256x256d", "c3_gemm_f32_dw_t256x256d"} <= gemm
    for kind in ["fwd", "dx", "dx_mask", "dx_mask_dz", "dw", "dw_mask", "tt"]:  # every k-tile at once (k <= 128)
        assert f"c3_gemm_f32_{kind}_t64x64k_v" in gemm
    for name in ["c3_gemm_f32_bwd_t64x64", "c3_gemm_f32_bwd_mask_t64x64"]:
        assert f"{name}_v" in gemm and f"{name}_s" in gemm
    assert {"c3_gemm_f32_bwd_t64x64k_v", "c3_gemm_f32_bwd_mask_t64x64k_v"} <= gemm
    bf = _kernel_symbols(LIB / "gemm_bf16.hsaco")
    for tile in ["d256w8", "d256rq", "d256pp", "d128w4", "d128w4s4", "d64w4"]:
        for kind in ["fwd", "dx", "dw", "dwb", "tt", "fwdt", "fwdf", "dxf", "ttf"]:
            assert f"c3_gemm_bf16_{kind}_{tile}" in bf
    for tile in ["d256w8", "d128w4", "d64w4", "d64w4_d128w4", "d128w4_d64w4"]:  # layer backward in one launch
        assert f"c3_gemm_bf16_bwd_{tile}" in bf
    assert {"c3_splitk_reduce", "c3_transpose_bf16"} <= bf
    ew = _kernel_symbols(LIB / "elementwise.hsaco")
    for op in list(native.EW_OPS) + list(native.EW_MATH_OPS):
        assert f"c3_ew_{op}_f32_v" in ew and f"c3_ew_{op}_f32_s" in ew
    assert "c3_ew3_div_bwd_b_f32" in ew
    assert {"c3_dz_colsum_f32", "c3_dz_colsum_f32_v", "c3_dz_colsum_bf16"} <= _kernel_symbols(LIB / "reduce.hsaco")
    red = _kernel_symbols(LIB / "reduce.hsaco")
    assert {"c3_colsum_partial_f32", "c3_colsum_final_f32", "c3_rowsum_f32"} <= red
    loss = _kernel_symbols(LIB / "loss.hsaco")
    assert {"c3_softmax_ce_f32", "c3_softmax_ce_bf16", "c3_cast_f32_bf16", "c3_cast_bf16_f32", "c3_sgd_f32",
            "c3_sgd_bf16", "c3_sgd_multi_f32", "c3_sgd_multi_bf16"} <= loss


# Argument validation runs before any HIP call, so it is testable on the CPU.
def _rc(fn, *args):
    return getattr(native.load(), fn)(*args)


def test_elementwise_validation():
    assert _rc("c3hip_elementwise", 99, 0, 16, 16, 0.0, 16, 4, 0, None) == native.ERR_INVALID
    assert "unknown elementwise op" in native.last_error()
    assert _rc("c3hip_elementwise", 0, 7, 16, 16, 0.0, 16, 4, 0, None) == native.ERR_INVALID
    assert _rc("c3hip_elementwise", 0, native.BF16, 16, 16, 0.0, 16, 4, 0, None) == native.ERR_UNSUPPORTED
    assert _rc("c3hip_elementwise", 0, 0, 16, 16, 0.0, 16, -1, 0, None) == native.ERR_INVALID
    assert _rc("c3hip_elementwise", 0, 0, 16, None, 0.0, 16, 4, 0, None) == native.ERR_INVALID
    assert _rc("c3hip_elementwise", 0, 0, None, 16, 0.0, 16, 4, 0, None) == native.ERR_INVALID
    # n == 0 is a successful no-op.
    assert _rc("c3hip_elementwise", 0, 0, None, None, 0.0, None, 0, 0, None) == native.OK
    assert native.last_error() == ""


def test_gemm_validation():
    assert _rc("c3hip_matmul", 3, 16, 16, 16, 4, 4, 4, 0, 0, None) == native.ERR_INVALID
    assert _rc("c3hip_matmul", 0, 16, 16, 16, -1, 4, 4, 0, 0, None) == native.ERR_INVALID
    assert _rc("c3hip_matmul", 0, 16, 16, None, 4, 4, 4, 0, 0, None) == native.ERR_INVALID
    assert _rc("c3hip_matmul", 0, 16, 16, 16, 1 << 20, 1 << 13, 4, 0, 0, None) == native.ERR_TOO_LARGE
    assert _rc("c3hip_matmul", 0, None, None, None, 0, 5, 5, 0, 0, None) == native.OK
    assert _rc("c3hip_linear_fwd", 0, 16, 16, None, 16, 4, 4, 4, 5, None) == native.ERR_INVALID  # act
    assert _rc("c3hip_linear_fwd", 0, None, 16, None, 16, 4, 4, 4, 1, None) == native.ERR_INVALID
    assert _rc("c3hip_linear_bwd", 0, 16, 16, None, 16, 16, None, None, 4, 4, 4, 1, None) == native.ERR_INVALID
    assert "Y" in native.last_error()
    assert _rc("c3hip_linear_bwd", 0, None, None, None, 16, 16, None, None, 4, 4, 4, 0, None) == native.ERR_INVALID
    assert _rc("c3hip_sum_reduce", 16, 16, 4, 4, 2, None) == native.ERR_INVALID
    assert _rc("c3hip_sum_reduce", None, 16, 4, 0, 0, None) == native.OK


def test_elementwise3_and_act_validation():
    assert _rc("c3hip_elementwise3", 5, 0, 16, 16, 16, 16, 4, None) == native.ERR_INVALID
    assert _rc("c3hip_elementwise3", 0, native.BF16, 16, 16, 16, 16, 4, None) == native.ERR_UNSUPPORTED
    assert _rc("c3hip_elementwise3", 0, 0, 16, None, 16, 16, 4, None) == native.ERR_INVALID
    assert _rc("c3hip_elementwise3", 0, 0, None, None, None, None, 0, None) == native.OK
    assert _rc("c3hip_elementwise", 15, 0, 16, 16, 0.0, 16, 4, 0, None) == native.ERR_INVALID
    assert _rc("c3hip_linear_fwd", 0, 16, 16, None, 16, 4, 4, 4, 4, None) == native.ERR_INVALID  # act 4
    assert _rc("c3hip_linear_bwd", 0, 16, 16, None, 16, 16, None, None, 4, 4, 4, 2, None) == native.ERR_INVALID


def test_backward_chain_validation():
    import ctypes

    def arr(t, vals):
        return (t * max(len(vals), 1))(*vals)

    vp, ci = ctypes.c_void_p, ctypes.c_int

    def rc(dtype, grad, xs, nodes, outs, n):
        return native.load().c3hip_backward_chain(dtype, grad, arr(vp, xs), arr(ci, nodes), len(nodes),
                                                  arr(vp, outs), n, None)

    assert rc(native.F32, 16, [16], [native.CHAIN_RELU], [16], -1) == native.ERR_INVALID
    assert rc(native.BF16, 16, [16], [native.CHAIN_RELU], [16], 4) == native.ERR_UNSUPPORTED
    assert rc(native.F32, 16, [], [], [], 4) == native.ERR_INVALID                    # no nodes
    assert rc(native.F32, 16, [16] * 5, [0] * 5, [16] * 5, 4) == native.ERR_INVALID  # beyond the window
    assert rc(native.F32, 16, [16], [6], [16], 4) == native.ERR_INVALID               # unknown node
    assert rc(native.F32, 16, [None], [native.CHAIN_TANH], [16], 4) == native.ERR_INVALID
    assert rc(native.F32, None, [16], [native.CHAIN_RELU], [16], 4) == native.ERR_INVALID
    assert rc(native.F32, None, [None], [native.CHAIN_RELU], [None], 0) == native.OK  # nothing to do


def test_gemm_tile_override_validation():
    assert native.gemm_tile_names(native.F32) == ["t64x64", "t128x128", "t256x128", "t128x256", "t256x128d", "t128x256d",
                                                  "t256x256d", "t64x64d"]
    assert native.gemm_tile_names(native.BF16) == ["t64x64", "t128x128", "t256x128", "t256x256", "d256w8", "d256rq", "d256pp", "d128w4", "d128w4s4", "d64w4"]
    L = native.load()
    assert L.c3hip_set_gemm_tile(native.F32, b"d256w8") == native.ERR_INVALID  # a bf16-only tile
    assert L.c3hip_set_gemm_tile(native.BF16, b"t32x32") == native.ERR_INVALID
    assert L.c3hip_set_gemm_tile(7, b"t64x64") == native.ERR_INVALID
    assert L.c3hip_set_gemm_tile(native.F32, b"t128x128") == native.OK
    assert L.c3hip_set_gemm_tile(native.F32, None) == native.OK
    assert L.c3hip_set_gemm_tile(native.BF16, b"") == native.OK
    import ctypes

    small = ctypes.create_string_buffer(8)
    assert L.c3hip_gemm_tile_names(native.BF16, small, len(small)) == native.ERR_INVALID


def test_train_step_helper_validation():
    assert _rc("c3hip_softmax_ce", 5, 16, 16, 16, 16, 4, 10, None) == native.ERR_INVALID
    assert _rc("c3hip_softmax_ce", 0, 16, 16, 16, 16, 4, 4096, None) == native.ERR_UNSUPPORTED
    assert _rc("c3hip_softmax_ce", 0, 16, 16, 16, 16, 4, 0, None) == native.ERR_INVALID
    assert _rc("c3hip_softmax_ce", 0, None, 16, 16, 16, 4, 10, None) == native.ERR_INVALID
    assert _rc("c3hip_softmax_ce", 0, 16, 16, None, None, 4, 10, None) == native.OK  # nothing asked
    assert _rc("c3hip_cast", 0, 2, 16, 16, 4, None) == native.ERR_INVALID
    assert _rc("c3hip_cast", 0, 1, None, 16, 4, None) == native.ERR_INVALID
    assert _rc("c3hip_cast", 0, 1, None, None, 0, None) == native.OK
    assert _rc("c3hip_sgd_update", 0, None, 16, 0.1, 4, None) == native.ERR_INVALID
    assert _rc("c3hip_sgd_update", 0, 16, 16, 0.1, -1, None) == native.ERR_INVALID
    import ctypes

    P = ctypes.c_void_p * 2
    I = ctypes.c_int64 * 2
    f = ctypes.c_float(0.1)
    assert _rc("c3hip_sgd_update_multi", 0, 17, P(16, 16), P(16, 16), I(4, 4), f, None) == native.ERR_INVALID
    assert _rc("c3hip_sgd_update_multi", 0, -1, P(16, 16), P(16, 16), I(4, 4), f, None) == native.ERR_INVALID
    assert _rc("c3hip_sgd_update_multi", 2, 2, P(16, 16), P(16, 16), I(4, 4), f, None) == native.ERR_INVALID
    assert _rc("c3hip_sgd_update_multi", 0, 2, None, P(16, 16), I(4, 4), f, None) == native.ERR_INVALID
    assert _rc("c3hip_sgd_update_multi", 0, 2, P(16, None), P(16, 16), I(4, 4), f, None) == native.ERR_INVALID
    assert _rc("c3hip_sgd_update_multi", 0, 2, P(16, 16), P(16, 16), I(4, -1), f, None) == native.ERR_INVALID
    assert _rc("c3hip_sgd_update_multi", 0, 0, None, None, None, f, None) == native.OK  # nothing to do
    assert _rc("c3hip_sgd_update_multi", 0, 2, P(None, None), P(None, None), I(0, 0), f, None) == native.OK


def test_python_binding_raises_with_message():
    with pytest.raises(native.C3HipError) as ei:
        native.elementwise(42, native.F32, 16, 16, 0.0, 16, 4)
    assert ei.value.code == native.ERR_INVALID and "unknown elementwise op" in str(ei.value)


def test_trainer_binding_exports_and_fails_cleanly_without_gpu():
    from c3_amd import trainer as T

    lib = T.load()
    for name in T.SIGNATURES:
        assert hasattr(lib, name)
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible: creation would succeed")
    with pytest.raises(T.TrainerError, match="hipGetDevice"):
        T.MlpTrainer([4, 2], 1)
    with pytest.raises(T.TrainerError, match="bad arguments"):
        T.MlpTrainer([4], 1)
